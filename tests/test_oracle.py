"""Pins the CPU oracle (oracle/krk_oracle.c) before anything is checked
against it: the reference's own known-answer tests, closed forms and brute
force, the committed golden vectors written by the reference's own code, and
-- where oracle/_ref was built -- the reference itself, bit for bit."""
import os
import struct

import numpy as np
import pytest

import oracle as O
from conftest import rand_blocks

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz")
FMTS = [O.Q4_0, O.Q8_0, O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K, O.Q6_K, O.IQ4_NL, O.IQ4_XS, O.MXFP4,
        O.Q4_1, O.Q5_0, O.Q5_1, O.F16, O.BF16, *O.CHUNK_FMTS]


def f16bytes(v):
    h = np.float16(v).view(np.uint16)
    return [int(h) & 0xFF, int(h) >> 8]


# ------------------------------------------- reference known-answer tests --
def test_quant_geometry():  # tests/test_kraken.cpp:396-454
    L = O.lib()
    assert L.orc_block_size(O.Q4_0) == 32 and L.orc_block_bytes(O.Q4_0) == 18
    assert L.orc_block_size(O.Q6_K) == 256 and L.orc_block_bytes(O.Q6_K) == 210
    assert L.orc_block_size(O.Q4_K) == 256 and L.orc_block_bytes(O.Q4_K) == 144
    assert L.orc_block_size(O.Q8_0) == 32 and L.orc_block_bytes(O.Q8_0) == 34
    assert O.row_bytes(O.Q8_0, 64) == 68
    assert O.row_bytes(O.Q4_K, 4096) == 2304 and O.row_bytes(O.Q4_K, 14336) == 8064
    assert O.row_bytes(O.Q6_K, 4096) == 3360 and O.row_bytes(O.Q8_0, 4096) == 4352


def test_q4_0_layout():  # tests/test_kraken.cpp:456-469
    blk = np.array(f16bytes(1.0) + [i | (i << 4) for i in range(16)], np.uint8)
    out = O.dequant(O.Q4_0, blk, 1, 32)[0]
    assert np.array_equal(out[:16], np.arange(16) - 8.0)
    assert np.array_equal(out[16:], np.arange(16) - 8.0)


def test_q8_0_layout():  # tests/test_kraken.cpp:563-573
    blk = np.array(f16bytes(0.5) + [(i - 16) & 0xFF for i in range(32)], np.uint8)
    out = O.dequant(O.Q8_0, blk, 1, 32)[0]
    assert np.array_equal(out, 0.5 * (np.arange(32) - 16.0))


def test_kquant_roundtrip_shape():  # tests/test_kraken.cpp:981-1001, made exact
    blk = np.array(f16bytes(0.5) + f16bytes(0.25) + [1] * 12 + [0x88] * 128, np.uint8)
    out = O.dequant(O.Q4_K, blk, 1, 256)[0]
    # sub-blocks 0..3: sc = m = 1 -> 0.5*8 - 0.25 = 3.75; sub-blocks 4..7 take
    # sc from the low nibble of bytes 8..11 (1) and m from their high nibble
    # and byte j's top bits (0) -> 4.0
    assert np.all(out[:128] == 3.75) and np.all(out[128:] == 4.0)
    assert abs(out.sum()) < 256 * 8


def test_q6_k_group_stride():  # tests/test_kraken.cpp:1026-1042
    blk = np.zeros(210, np.uint8)
    blk[208:210] = f16bytes(1.0)
    blk[192:208] = 1
    blk[128 + 32] = 0x03
    out = O.dequant(O.Q6_K, blk, 1, 256)[0]
    assert out[0] == -32 and out[128] == 16 and out[160] == -32


def test_vec_dot_f16_f32():  # tests/test_kraken.cpp:2087-2098
    w = np.arange(1, 65, dtype=np.float32)
    x = np.full(64, 0.5, np.float32)
    assert O.lib().orc_vec_dot(O.F32, O._p(w), O._p(x), 64) == 1040.0
    h = w.astype(np.float16)
    assert O.lib().orc_vec_dot(O.F16, O._p(h), O._p(x), 64) == 1040.0


def test_q8_activation_domain():  # tests/test_kraken.cpp:8143-8163
    mag = np.array([1e30, -1e30, 1e-30, 0.0, 3.5, -0.001], np.float32)
    x = mag[np.arange(512) % 6]
    xq, dx = O.quantize_q8_row(x)
    assert xq.max() == 127 and xq.min() == -127
    assert abs(float(xq[0]) * float(dx[0]) - 1e30) <= 1e30 * 0.02


# ------------------------------------------------- closed forms / brute force
def _pack_q4k(d, dmin, sc, mn, q):
    """Independent Q4_K packer (the inverse of get_scale_min_k4)."""
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    qs = [q[64 * g + l] | (q[64 * g + 32 + l] << 4) for g in range(4) for l in range(32)]
    return np.array(f16bytes(d) + f16bytes(dmin) + s + qs, np.uint8)


def _fma32(a, b, c):
    from fractions import Fraction
    return np.float32(float(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))))


def test_q4_k_closed_form_all_scale_slots():
    rng = np.random.default_rng(7)
    for trial in range(20):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        d, dmin = np.float16(rng.uniform(0.001, 0.05)), np.float16(rng.uniform(0.001, 0.05))
        out = O.dequant(O.Q4_K, _pack_q4k(d, dmin, sc, mn, q), 1, 256)[0]
        for i in range(0, 256, 7):
            j = i // 32
            d1 = np.float32(np.float32(d) * np.float32(sc[j]))
            m1 = np.float32(np.float32(dmin) * np.float32(mn[j]))
            assert out[i] == _fma32(d1, q[i], -m1), (trial, i)


def test_q4_k_contraction_is_immaterial():
    """d1 = d*sc is exact in f32 (11 + 6 significant bits) and so is d1*q
    (+4 bits, 21 <= 24): fused and unfused d1*q - m1 round once, identically.
    So the reference build's vfmsub and a plain multiply-subtract agree on
    every Q4_K block -- checked here over the whole code space of a scale."""
    rng = np.random.default_rng(11)
    for _ in range(3000):
        d, dmin = np.float16(rng.uniform(1e-4, 0.1)), np.float16(rng.uniform(1e-4, 0.1))
        s, m, qv = int(rng.integers(0, 64)), int(rng.integers(0, 64)), int(rng.integers(0, 16))
        d1 = np.float32(np.float32(d) * np.float32(s))
        m1 = np.float32(np.float32(dmin) * np.float32(m))
        assert _fma32(d1, qv, -m1) == np.float32(np.float32(d1 * np.float32(qv)) - m1)
    sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    q = rng.integers(0, 16, 256)
    d, dmin = np.float16(0.0123), np.float16(0.0456)
    out = O.dequant(O.Q4_K, _pack_q4k(d, dmin, sc, mn, q), 1, 256)[0]
    for i in range(256):
        j = i // 32
        d1 = np.float32(np.float32(d) * np.float32(sc[j]))
        m1 = np.float32(np.float32(dmin) * np.float32(mn[j]))
        assert out[i] == np.float32(np.float32(d1 * np.float32(q[i])) - m1)


def test_q6_k_closed_form():
    rng = np.random.default_rng(3)
    blk = rand_blocks(rng, O.Q6_K, 1)
    out = O.dequant(O.Q6_K, blk, 1, 256)[0]
    ql, qh, sc = blk[:128], blk[128:192], blk[192:208].view(np.int8)
    d = np.float32(blk[208:210].view(np.float16)[0])
    for i in range(256):
        h, r = divmod(i, 128)
        qd, l = divmod(r, 32)
        lo = ql[64 * h + l + 32 * (qd & 1)]
        nib = (lo >> 4) if qd >= 2 else (lo & 15)
        q = int(nib) | (((int(qh[32 * h + l]) >> (2 * qd)) & 3) << 4)
        want = np.float32(np.float32(d * np.float32(sc[8 * h + l // 16 + 2 * qd])) * np.float32(q - 32))
        assert out[i] == want, i


def test_vec_dot_is_one_unfused_chain():
    """The strict tier of the block formats: sum += round(w*x), in index
    order (pinned against the reference build, see
    test_oracle_matches_reference_build).  The unquantized types take the
    reference's four fused lanes instead (quant.cpp:5431-5510), pinned by the
    same reference-build test."""
    rng = np.random.default_rng(5)
    for dt in [f for f in FMTS if f not in (O.F16, O.BF16)]:
        bs = O.lib().orc_block_size(dt)
        w = rand_blocks(rng, dt, 1024 // bs)
        x = rng.standard_normal(1024).astype(np.float32)
        v = O.dequant(dt, w, 1, 1024)[0]
        s = np.float32(0)
        for a, b in zip(v, x):
            s = np.float32(s + np.float32(a * b))
        assert O.vec_dot(dt, w, x) == s
        exact = float(np.dot(v.astype(np.float64), x.astype(np.float64)))
        assert abs(float(s) - exact) <= 1e-5 * float(np.abs(v.astype(np.float64) * x).sum())


def test_quantize_q8_row_closed_form():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(4096) * 2).astype(np.float32)
    x[32:64] = 0
    xq, dx = O.quantize_q8_row(x)
    for b in range(128):
        blk = x[32 * b:32 * b + 32]
        amax = np.float32(np.abs(blk).max())
        d = np.float32(amax / np.float32(127)) if amax > 0 else np.float32(0)
        assert dx[b] == d
        if d == 0:
            assert not xq[32 * b:32 * b + 32].any()
            continue
        inv = np.float32(np.float32(1) / d)
        q = np.clip(np.rint(blk * inv), -127, 127).astype(np.int8)
        assert np.array_equal(xq[32 * b:32 * b + 32], q)


def test_dot_q8_0_q8_closed_form():
    rng = np.random.default_rng(13)
    w = rand_blocks(rng, O.Q8_0, 64)
    xq, dx = O.quantize_q8_row(rng.standard_normal(2048).astype(np.float32))
    acc = np.float32(0)
    wb = w.reshape(64, 34)
    for b in range(64):
        d = np.float32(wb[b, :2].view(np.float16)[0])
        s = int(np.dot(wb[b, 2:].view(np.int8).astype(np.int64),
                       xq[32 * b:32 * b + 32].astype(np.int64)))
        acc = _fma32(np.float32(s), np.float32(d * dx[b]), acc)
    assert O.dot_q8_0_q8(w, xq, dx) == acc


def test_router_closed_form():
    rng = np.random.default_rng(17)
    logits = rng.standard_normal((6, 128)).astype(np.float32)
    logits[0, 5] = logits[0, 9] = 9.0  # an exact tie: lower id first
    p = O.router_softmax(logits)
    ref = np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    assert np.allclose(p, ref, rtol=2e-6, atol=1e-9)
    ids, wts = O.router_topk(p, 8)
    assert ids[0, 0] == 5 and ids[0, 1] == 9
    for r in range(6):
        order = sorted(range(128), key=lambda e: (-p[r, e], e))[:8]
        assert list(ids[r]) == order
        sel = p[r, order].astype(np.float32)
        ks = np.float32(0)
        for v in sel:
            ks = np.float32(ks + v)
        assert np.array_equal(wts[r], sel * np.float32(np.float32(1) / ks))


def test_moe_matches_dense_twin(krk):
    """One expert at weight 1.0 is the dense FFN (test_kraken.cpp:15328 idea);
    and the routed sum matches an f64 composition."""
    rng = np.random.default_rng(19)
    ne, E, F, T, k = 4, 256, 512, 3, 2
    mats = {}
    for e in range(ne):
        for nm, (o, i) in (("g", (F, E)), ("u", (F, E)), ("d", (E, F))):
            v = (rng.standard_normal(o * i) * 0.02).astype(np.float32)
            mats[nm, e] = krk.quantize(O.Q4_K, v, o, i)
    x = rng.standard_normal((T, E)).astype(np.float32)
    g = [mats["g", e] for e in range(ne)]
    u = [mats["u", e] for e in range(ne)]
    d = [mats["d", e] for e in range(ne)]
    ids = np.array([[2, 0], [1, 3], [3, 2]], np.int32)
    one = O.moe_ffn(x, g, u, d, O.Q4_K, ids[:, :1], np.ones((T, 1), np.float32), F)
    for t in range(T):
        e = ids[t, 0]
        mid = O.silu_mul(O.gemm(O.Q4_K, g[e], x[t], F), O.gemm(O.Q4_K, u[e], x[t], F))
        assert np.array_equal(one[t], O.gemm(O.Q4_K, d[e], mid, E)[0])
    wts = np.array([[0.7, 0.3], [0.5, 0.5], [0.9, 0.1]], np.float32)
    out = O.moe_ffn(x, g, u, d, O.Q4_K, ids, wts, F)
    deq = {key: O.dequant(O.Q4_K, v, *((F, E) if key[0] != "d" else (E, F))).astype(np.float64)
           for key, v in mats.items()}
    for t in range(T):
        acc = np.zeros(E)
        for s in range(k):
            e = ids[t, s]
            gg, uu = deq["g", e] @ x[t], deq["u", e] @ x[t]
            acc += wts[t, s] * (deq["d", e] @ (gg / (1 + np.exp(-gg)) * uu))
        assert np.linalg.norm(out[t] - acc) <= 1e-5 * np.linalg.norm(acc)


def _f16_expert(gate_row, up_col, down_col, n=4):
    """F16 expert banks of n x n: every gate row is gate_row; up row j is
    [up_col[j], 0, ..]; down row i is [down_col[i], 0, ..] (exact f16 values)."""
    g = np.tile(np.array(gate_row, np.float16), (n, 1))
    u = np.zeros((n, n), np.float16)
    u[:, 0] = up_col
    d = np.zeros((n, n), np.float16)
    d[:, 0] = down_col
    return [m.reshape(-1).view(np.uint8).copy() for m in (g, u, d)]


def test_moe_ffn_f16_slot_order_and_row_scale():
    """The reference GPU's f16 expert FFN (moe_table.hpp:256-305, 418-441,
    536-551) on F16 banks whose dots are exact, so every value below is fixed
    by hand: gate rows [32, 0, 0, 0] against x = e0 give g = 32 and silu(32)
    = 32 in f32; up 2^-5 gives mid = 1; a down entry dd gives v = dd.
      * slot order with an f16 rounding after every add: parts 1, 2^-11,
        2^-11 sum to 1 in that order (1 + 2^-11 ties to even) but to
        1 + 2^-10 in the order 2^-11, 2^-11, 1 -- where the f32 oracle gets
        1 + 2^-10 in either order;
      * the row scale: up 2^11 gives mid = 65536 > 65504, so scale 2, midf =
        32768, and down 2^-15 gives v = 1, part f16(1) * 2 = 2 (no scale: an
        f16 overflow to inf);
      * a dropped slot (id -1) adds nothing."""
    F16 = O.F16
    x = np.array([[1, 0, 0, 0]], np.float32)
    big, small = _f16_expert([32, 0, 0, 0], [2.0 ** -5] * 4, [1.0, 0, 0, 0]), \
        _f16_expert([32, 0, 0, 0], [2.0 ** -5] * 4, [2.0 ** -11, 0, 0, 0])
    scaled = _f16_expert([32, 0, 0, 0], [2.0 ** 11] * 4, [2.0 ** -15, 0, 0, 0])
    banks = [big, small, small, scaled]
    g, u, d = ([b[m] for b in banks] for m in range(3))
    w1 = np.ones((1, 3), np.float32)

    def run(ids):
        return O.moe_ffn_f16(x, g, u, d, F16, np.array([ids], np.int32), w1, 4)[0, 0]

    assert run([0, 1, 2]) == np.float16(1.0)
    assert run([1, 2, 0]) == np.float16(1.0 + 2.0 ** -10)
    assert run([-1, 1, 0]) == np.float16(1.0)           # 2^-11 then 1: ties to even
    for ids in ([0, 1, 2], [1, 2, 0]):
        f32 = O.moe_ffn(x, g, u, d, F16, np.array([ids], np.int32), w1, 4)[0, 0]
        assert f32 == np.float32(1.0 + 2.0 ** -10)
    assert run([3, -1, -1]) == np.float16(2.0)
    assert np.isfinite(run([3, 3, -1]))


def test_moe_ffn_f16_tracks_the_f32_oracle(krk):
    """On quantized banks the f16 form stays within its rounding of the f32
    oracle (a dropped term or a wrong scale would not)."""
    rng = np.random.default_rng(23)
    ne, E, F, T, k = 4, 256, 512, 3, 2
    mats = {}
    for e in range(ne):
        for nm, (o, i) in (("g", (F, E)), ("u", (F, E)), ("d", (E, F))):
            mats[nm, e] = krk.quantize(O.Q4_K, (rng.standard_normal(o * i) * 0.02).astype(np.float32), o, i)
    x = rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)
    g, u, d = ([mats[nm, e] for e in range(ne)] for nm in "gud")
    ids = np.array([[2, 0], [1, 3], [3, 2]], np.int32)
    wts = np.array([[0.7, 0.3], [0.5, 0.5], [0.9, 0.1]], np.float32)
    h = O.moe_ffn_f16(x, g, u, d, O.Q4_K, ids, wts, F).astype(np.float32)
    f = O.moe_ffn(x, g, u, d, O.Q4_K, ids, wts, F)
    e = np.linalg.norm(h - f) / np.linalg.norm(f)
    assert 1e-5 < e < 3e-3


def test_q8_0_fixture_quantizer_matches_python_rule():
    """tools/make_bench_gguf.py:191-202 restated with Python's own float
    semantics (f64, round-half-even, struct '<e')."""
    rng = np.random.default_rng(23)
    v = (rng.standard_normal(32 * 40) * 0.02).astype(np.float32)
    v[32:64] = 0.0
    v[64] = 0.5 * np.float32(1e-3)
    got = O.quantize_q8_0_weights(v)
    want = bytearray()
    for b in range(0, v.size, 32):
        blk = [float(t) for t in v[b:b + 32]]
        amax = max(abs(t) for t in blk) or 1e-8
        d = amax / 127.0
        want += struct.pack("<e", d)
        for t in blk:
            want += struct.pack("<b", max(-127, min(127, int(round(t / d)))))
    assert bytes(got) == bytes(want)


# ------------------------------------------------------------- golden vectors
def test_oracle_matches_golden_vectors():
    g = np.load(GOLDEN)
    for dt, name in ((O.Q4_0, "q4_0"), (O.Q8_0, "q8_0"), (O.Q4_K, "q4_k"), (O.Q5_K, "q5_k"),
                     (O.Q6_K, "q6_k"), (O.IQ4_NL, "iq4_nl"), (O.IQ4_XS, "iq4_xs"), (O.Q2_K, "q2_k"),
                     (O.Q3_K, "q3_k"), (O.MXFP4, "mxfp4"), (O.Q4_1, "q4_1"), (O.Q5_0, "q5_0"),
                     (O.Q5_1, "q5_1"), *((dt, f"chunk{dt}") for dt in O.CHUNK_FMTS)):
        w, x = g[f"{name}_w"], g[f"{name}_x"]
        n = x.size
        deq = O.dequant(dt, w, 1, n)[0]
        assert np.array_equal(deq.view(np.uint32), g[f"{name}_deq"].view(np.uint32)), name
        assert np.array_equal(O.dequant_f16(dt, w, 1, n)[0], g[f"{name}_deq_f16"]), name
        bs = O.lib().orc_block_size(dt)
        for i in range(8):
            m = n * (i + 1) // 8 // bs * bs
            got = np.float32(O.lib().orc_vec_dot(dt, O._p(w), O._p(x), m))
            assert got == g[f"{name}_dot"][i], (name, i)
    xq, dx = O.quantize_q8_row(g["q8act_x"])
    assert np.array_equal(xq, g["q8act_xq"]) and np.array_equal(dx, g["q8act_dx"])
    xq2, dx2 = O.quantize_q8_row(g["q8dot_x"])
    assert np.float32(O.dot_q8_0_q8(g["q8dot_w"], xq2, dx2)) == g["q8dot_out"][0]


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference tree)")
def test_reference_strict_gemv_equals_oracle():
    """The bench's CPU baseline (the reference's own vec_dot per row over
    threads) gives the oracle's GEMV bit for bit, for any thread count."""
    rng = np.random.default_rng(41)
    for dt in (O.Q4_K, O.Q6_K, O.Q8_0, O.Q4_0):
        n_out, n_in = 37, 1024
        w = rand_blocks(rng, dt, n_out * n_in // O.lib().orc_block_size(dt))
        x = rng.standard_normal(n_in).astype(np.float32)
        want = O.gemm(dt, w, x, n_out)[0]
        for th in (1, 3, 8):
            assert np.array_equal(O.ref_gemv(dt, w, x, n_out, nthreads=th).view(np.uint32), want.view(np.uint32))


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference tree)")
def test_oracle_matches_reference_build():
    ref = O.ref()
    rng = np.random.default_rng(29)
    for dt in FMTS:
        bs = O.lib().orc_block_size(dt)
        for trial in range(4):
            nb = 4096 // bs
            w = rand_blocks(rng, dt, nb)
            x = rng.standard_normal(nb * bs).astype(np.float32)
            a = O.dequant(dt, w, 1, nb * bs)[0]
            b = np.empty_like(a)
            ref.ref_dequant_row(dt, O._p(w), O._p(b), nb * bs)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
            assert np.float32(O.vec_dot(dt, w, x)) == np.float32(
                ref.ref_vec_dot(dt, O._p(w), O._p(x), nb * bs))
            h = np.empty(nb * bs, np.uint16)
            ref.ref_dequant_row_f16(dt, O._p(w), O._p(h), nb * bs)
            assert np.array_equal(O.dequant_f16(dt, w, 1, nb * bs)[0], h)
    x = (rng.standard_normal(8192) * 5).astype(np.float32)
    xq, dx = O.quantize_q8_row(x)
    xq2, dx2 = np.empty_like(xq), np.empty_like(dx)
    ref.ref_quantize_q8_row(O._p(x), 8192, O._p(xq2), O._p(dx2))
    assert np.array_equal(xq, xq2) and np.array_equal(dx, dx2)
    w = rand_blocks(rng, O.Q8_0, 256)
    assert np.float32(O.dot_q8_0_q8(w, xq, dx)) == np.float32(
        ref.ref_dot_q8_0_q8_scalar(O._p(w), O._p(xq), O._p(dx), 8192))
    for f in (0.5, 1.0 + 2.0 ** -11, 65504.0, 1e-7, 3.0e-5, -2.5):
        assert O.lib().orc_fp32_to_fp16(f) == ref.ref_fp32_to_fp16(f)


def test_q5_k_closed_form():
    """Q5_K (quant.cpp:462-489) by construction: d = 1, dmin = 0.5, every
    scale slot 1..8 and min slot 2 * j, codes and high bits from known
    patterns, so each value is sc_j * (nibble + 16 * bit) - 0.5 * m_j; then
    the high-bit order (bit 2j low nibble, bit 2j+1 high nibble) with all
    qh bytes a single bit."""
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    sc = list(range(1, 9))
    mn = [2 * j for j in range(8)]
    # get_scale_min_k4 packing: j < 4 in the low 6 bits of bytes j and j + 4;
    # j >= 4 in byte j + 4 (low nibble scale, high nibble min) plus the top
    # two bits of bytes j - 4 and j
    for j in range(4):
        blk[4 + j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        blk[8 + j] = mn[j] | ((mn[j + 4] >> 4) << 6)
        blk[12 + j] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    codes = np.arange(128, dtype=np.uint8)
    blk[48:] = (codes * 7) & 0xFF
    for bit in range(8):
        qh = np.zeros(32, np.uint8)
        qh[:] = 1 << bit
        blk[16:48] = qh
        y = O.dequant(O.Q5_K, blk, 1, 256)[0]
        want = np.empty(256, np.float64)
        for j in range(4):
            q = blk[48 + 32 * j: 48 + 32 * j + 32].astype(np.int64)
            lo = (q & 15) + (16 if bit == 2 * j else 0)
            hi = (q >> 4) + (16 if bit == 2 * j + 1 else 0)
            want[64 * j: 64 * j + 32] = sc[2 * j] * lo - 0.5 * mn[2 * j]
            want[64 * j + 32: 64 * j + 64] = sc[2 * j + 1] * hi - 0.5 * mn[2 * j + 1]
        assert np.array_equal(y, want.astype(np.float32)), bit


def test_iq4_nl_closed_form():
    """IQ4_NL (quant.cpp:566-574): with d = 1 every index 0..15 in both
    nibbles decodes to the grid value itself, low nibbles first."""
    grid = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:] = [(k & 15) | ((15 - k) << 4) for k in range(16)]
    y = O.dequant(O.IQ4_NL, blk, 1, 32)[0]
    assert y[:16].tolist() == grid and y[16:].tolist() == grid[::-1]


def test_iq4_xs_closed_form():
    """IQ4_XS (quant.cpp:641-659): d = 0.5, sub-block ib's 6-bit scale
    ls = 17 + 5 ib split over scales_l (low nibble) and scales_h (2 bits),
    indices k and 15 - k: value 0.5 (ls - 32) grid[q]."""
    grid = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    blk = np.zeros(136, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    ls = [17 + 5 * ib for ib in range(8)]
    sh = sum(((l >> 4) & 3) << (2 * ib) for ib, l in enumerate(ls))
    blk[2], blk[3] = sh & 0xFF, sh >> 8
    for ib in range(8):
        blk[4 + ib // 2] |= (ls[ib] & 15) << (4 * (ib % 2))
        blk[8 + 16 * ib: 24 + 16 * ib] = [(k & 15) | ((15 - k) << 4) for k in range(16)]
    y = O.dequant(O.IQ4_XS, blk, 1, 256)[0]
    for ib in range(8):
        dl = np.float32(0.5) * np.float32(ls[ib] - 32)
        want = [dl * np.float32(g) for g in grid] + [dl * np.float32(g) for g in grid[::-1]]
        assert y[32 * ib: 32 * ib + 32].tolist() == [float(np.float32(w)) for w in want], ib


def test_q2_k_closed_form():
    """Q2_K (quant.cpp:398-423): d = 0.25, dmin = 0.5; scale byte i holds
    scale i % 16 and min 15 - i % 16; qs byte l holds codes (l + k) % 4 in
    its four bit pairs k.  Value index 128g + 32j + 16s + l: code bit pair
    j of qs[32g + 16s + l], scale byte 8g + 2j + s; value d sc q - dmin m."""
    blk = np.zeros(84, np.uint8)
    for i in range(16):
        blk[i] = (i & 15) | ((15 - i) << 4)
    for l in range(64):
        blk[16 + l] = sum(((l + k) % 4) << (2 * k) for k in range(4))
    blk[80:82] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    blk[82:84] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    y = O.dequant(O.Q2_K, blk, 1, 256)[0]
    for g in range(2):
        for j in range(4):
            for s in range(2):
                i = 8 * g + 2 * j + s
                for l in range(16):
                    q = (16 * s + l + j) % 4
                    want = 0.25 * i * q - 0.5 * (15 - i)
                    assert y[128 * g + 32 * j + 16 * s + l] == np.float32(want), (g, j, s, l)


def test_q3_k_closed_form():
    """Q3_K (quant.cpp:514-554): d = 0.5, the sixteen 6-bit scales
    sc_i = 7 + 3i (so sc - 32 crosses zero) packed as the reference packs
    them (low nibbles in bytes 0..7, high 2-bit pairs in bytes 8..11);
    qs byte l holds codes (l + k) % 4; hmask bit 4n + j of byte m is set when
    (m + n + j) is even.  Value (d (sc - 32)) (code - (hbit ? 0 : 4))."""
    sc = [7 + 3 * i for i in range(16)]
    blk = np.zeros(110, np.uint8)
    for m in range(32):
        blk[m] = sum(1 << (4 * n + j) for n in range(2) for j in range(4) if (m + n + j) % 2 == 0)
    for l in range(64):
        blk[32 + l] = sum(((l + k) % 4) << (2 * k) for k in range(4))
    r = [0] * 12
    for i in range(16):
        if i < 8:
            r[i] |= sc[i] & 15
        else:
            r[i - 8] |= (sc[i] & 15) << 4
        r[8 + i % 4] |= ((sc[i] >> 4) & 3) << (2 * (i // 4))
    blk[96:108] = r
    blk[108:110] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    y = O.dequant(O.Q3_K, blk, 1, 256)[0]
    for n in range(2):
        for j in range(4):
            for s in range(2):
                i = 8 * n + 2 * j + s
                for l in range(16):
                    m = 16 * s + l
                    code = (32 * n + m + j) % 4 - (0 if (m + n + j) % 2 == 0 else 4)
                    want = np.float32(0.5 * (sc[i] - 32)) * np.float32(code)
                    assert y[128 * n + 32 * j + 16 * s + l] == want, (n, j, s, l)


def test_mxfp4_closed_form_every_exponent():
    """MXFP4 (quant.cpp:674-686, e8m0_to_fp32_half 319-330): one block per
    exponent byte e = 0..255, codes k and 15 - k in byte k; value
    grid[q] * 2^(e - 128) with the doubled E2M1 grid, exact (ldexp) up to
    overflow to inf."""
    grid = [0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12]
    blk = np.zeros((256, 17), np.uint8)
    blk[:, 0] = np.arange(256)
    blk[:, 1:] = [(k & 15) | ((15 - k) << 4) for k in range(16)]
    y = O.dequant(O.MXFP4, blk.reshape(-1), 256, 32)
    with np.errstate(over="ignore"):
        for e in range(256):
            want = [np.float32(np.ldexp(np.float64(g), e - 128)) for g in grid + grid[::-1]]
            assert y[e].tolist() == [float(w) for w in want], e


@pytest.mark.parametrize("dt,qh,qs", [(O.Q4_1, None, 4), (O.Q5_0, 2, 6), (O.Q5_1, 4, 8)])
def test_legacy_32_closed_form(dt, qh, qs):
    """Q4_1 / Q5_0 / Q5_1 (quant.cpp:341-378): d = 0.5 (and m = -3 where the
    format has a min); code byte k holds k and 15 - k; the high-bit plane
    has bit j set for odd j.  Value d q + m, or d (q - 16) for Q5_0, with
    q the nibble plus 16 times the plane bit."""
    bb = {O.Q4_1: 20, O.Q5_0: 22, O.Q5_1: 24}[dt]
    blk = np.zeros(bb, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    has_m = dt != O.Q5_0
    if has_m:
        blk[2:4] = np.frombuffer(np.float16(-3.0).tobytes(), np.uint8)
    if qh is not None:
        blk[qh:qh + 4] = np.frombuffer(np.uint32(0xAAAAAAAA).tobytes(), np.uint8)
    blk[qs:qs + 16] = [k | ((15 - k) << 4) for k in range(16)]
    y = O.dequant(dt, blk, 1, 32)[0]
    for j in range(32):
        nib = j if j < 16 else 15 - (j - 16)
        q = nib + (16 * (j % 2) if qh is not None else 0)
        want = 0.5 * q - 3.0 if has_m else 0.5 * (q - 16)
        assert y[j] == np.float32(want), j


@pytest.mark.parametrize("dt", [O.Q4_K, O.Q5_K, O.Q6_K])
def test_kquant_int8_fold(dt):
    """The int8 rung's affine fold for the K-quants (gemm_dp4a.hpp:532-552):
    against the exact sum of dequant(w) * xq * dx (the dequant is pinned bit
    for bit) and, where oracle/_ref is built, against the reference's own CPU
    int8 twin (dot_q4_K_q8 / dot_q6_K_q8, quant.cpp:3125, 3193), both to f32
    rounding of the sum of |terms|.  A dropped min term, a sign or a wrong
    sub-block scale moves the result by O(1) of that sum."""
    rng = np.random.default_rng(40 + dt)
    n = 4096
    ref = O.ref() if O.ref_available() else None
    for _ in range(10):
        w = rand_blocks(rng, dt, n // 256)
        x = rng.standard_normal(n).astype(np.float32)
        xq, dx = O.quantize_q8_row(x)
        got = np.float32(O.lib().orc_dot_kq_q8(dt, O._p(w), O._p(xq), O._p(dx), n))
        terms = O.dequant(dt, w, 1, n)[0].astype(np.float64) * xq * np.repeat(dx.astype(np.float64), 32)
        scale = float(np.sum(np.abs(terms)))
        assert abs(float(got) - float(np.sum(terms))) <= 1e-6 * scale
        if ref is not None and dt != O.Q5_K:
            fn = ref.ref_dot_q4_K_q8 if dt == O.Q4_K else ref.ref_dot_q6_K_q8
            r = np.float32(fn(O._p(w), O._p(xq), O._p(dx), n))
            assert abs(float(got) - float(r)) <= 1e-6 * scale


def test_moe_plan_build_closed_form():
    """The plan of router.hpp:241-275 worked by hand: three rows of two slots,
    a dropped id (-1) and an id past n_expert skipped, pairs of one expert in
    (row, slot) order, and the reference's cursor limit of 256 experts."""
    ids = np.array([[3, 1], [1, 0], [3, -1], [3, 9]], np.int32)
    wts = np.array([[0.5, 0.25], [0.125, 1.0], [2.0, 4.0], [8.0, 16.0]], np.float32)
    off, rows, wt = O.moe_plan_build(ids, 4, wts)
    assert off.tolist() == [0, 1, 3, 3, 6]
    assert rows[:6].tolist() == [1, 0, 1, 0, 2, 3]
    assert wt[:6].tolist() == [1.0, 0.25, 0.125, 0.5, 2.0, 8.0]
    assert (rows[6:] == -1).all()
    _, _, wt0 = O.moe_plan_build(ids, 4)
    assert (wt0[:6] == 0.0).all()
    # experts from 256 up are counted but, with the reference's cursors, not placed
    big = np.array([[280, 5], [5, 280]], np.int32)
    off, rows, _ = O.moe_plan_build(big, 300, cursor_experts=256)
    assert off[300] == 4 and off[6] == 2 and off[281] == 4
    assert rows[:2].tolist() == [0, 1] and (rows[2:] == -1).all()
    _, rows_all, _ = O.moe_plan_build(big, 300)
    assert rows_all.tolist() == [0, 1, 0, 1]


def test_scan_accum_closed_form():
    """router.hpp:222-239 by hand: hits count routed pairs per (layer,
    expert), mass adds each expert's probability summed over the rows; both
    accumulate across calls and layers."""
    probs = np.array([[0.5, 0.25, 0.25], [0.125, 0.875, 0.0]], np.float32)
    ids = np.array([[0, 1], [1, -1]], np.int32)
    hits = np.zeros(2 * 3, np.uint32)
    mass = np.zeros(2 * 3, np.float32)
    O.scan_accum(probs, ids, 3, 1, hits, mass)
    O.scan_accum(probs, ids, 3, 1, hits, mass)
    assert hits.tolist() == [0, 0, 0, 2, 4, 0]
    assert mass.tolist() == [0, 0, 0, 1.25, 2.25, 0.5]
