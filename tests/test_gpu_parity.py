"""GPU parity: the HIP library, called through its C ABI, against the CPU
oracle on the same seeded inputs.

Bars: dequantized values bit-exact; GEMV within
1e-5 relative (||gpu - ref||_2 / ||ref||_2 over the output, the reference's
own gate uses a norm for the same cancellation reason,
tools/bench_ops.cpp:255-262); f16-staged MFMA GEMM within 2e-3 relative
Frobenius error."""
import sys

import numpy as np
import pytest

import oracle as O
from conftest import rand_blocks

pytestmark = pytest.mark.gpu

FMTS = [O.Q4_0, O.Q8_0, O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K, O.Q6_K, O.IQ4_NL, O.IQ4_XS, O.MXFP4,
        O.Q4_1, O.Q5_0, O.Q5_1, O.F16, O.BF16]
GEMV_TOL = 1e-5
GEMM_TOL = 2e-3


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def make_weights(krk, dt, n_out, n_in, seed, std=0.02):
    v = krk.synth_normal(n_out * n_in, seed=seed, std=std)
    return krk.quantize(dt, v, n_out, n_in)


# ------------------------------------------------------------------ dequant --
@pytest.mark.parametrize("dt", FMTS)
def test_dequant_bit_exact(torch_cuda, be32, rng, dt):
    torch = torch_cuda
    n_in = 1024
    n_rows = 37
    bs = O.lib().orc_block_size(dt)
    w = rand_blocks(rng, dt, n_rows * n_in // bs)
    say("dequant", dt, n_rows, n_in)
    out = torch.empty((n_rows, n_in), dtype=torch.float32, device="cuda")
    be32.dequant_rows(out, dev(torch, w), dt, n_rows, n_in)
    be32.sync()
    ref = O.dequant(dt, w, n_rows, n_in)
    assert np.array_equal(host(out).view(np.uint32), ref.view(np.uint32))
    out16 = torch.empty((n_rows, n_in), dtype=torch.float16, device="cuda")
    be32.dequant_rows(out16, dev(torch, w), dt, n_rows, n_in, f16=True)
    be32.sync()
    # device rounding is IEEE round-to-nearest-even of the bit-exact f32
    assert np.array_equal(host(out16).view(np.uint16), ref.astype(np.float16).view(np.uint16))


def test_quantize_q8_rows_bit_exact(torch_cuda, be32, rng):
    torch = torch_cuda
    x = (rng.standard_normal((3, 2048)) * 4).astype(np.float32)
    x[0, :6] = [1e30, -1e30, 1e-30, 0.0, 3.5, -0.001]
    x[1, 32:64] = 0.0
    xq = torch.empty((3, 2048), dtype=torch.int8, device="cuda")
    dx = torch.empty((3, 64), dtype=torch.float32, device="cuda")
    be32.quantize_q8_rows(dev(torch, x), 3, 2048, xq, dx)
    be32.sync()
    for r in range(3):
        q, d = O.quantize_q8_row(x[r])
        assert np.array_equal(host(xq)[r], q)
        assert np.array_equal(host(dx)[r].view(np.uint32), d.view(np.uint32))


def test_mxfp4_dequant_every_exponent(torch_cuda, be32):
    """Every E8M0 byte (the f32 denormal scales 2^-128, 2^-127 and the
    overflowing 2^127) and every code, bit for bit against the oracle."""
    torch = torch_cuda
    blk = np.zeros((256, 17), np.uint8)
    blk[:, 0] = np.arange(256)
    blk[:, 1:] = [(k & 15) | ((15 - k) << 4) for k in range(16)]
    w = blk.reshape(-1)
    say("dequant mxfp4 every exponent")
    out = torch.empty((256, 32), dtype=torch.float32, device="cuda")
    be32.dequant_rows(out, dev(torch, w), O.MXFP4, 256, 32)
    be32.sync()
    assert np.array_equal(host(out).view(np.uint32), O.dequant(O.MXFP4, w, 256, 32).view(np.uint32))


# --------------------------------------------------------------------- GEMV --
@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("rows", [1, 2, 3, 5, 8])
def test_gemv_f32_parity(krk, torch_cuda, be32, dt, rows):
    torch = torch_cuda
    n_out, n_in = 300, 2560 if dt in (O.Q4_0, O.Q8_0) else 2304
    w = make_weights(krk, dt, n_out, n_in, seed=100 + dt)
    x = krk.synth_normal(rows * n_in, seed=200 + rows).reshape(rows, n_in)
    say("gemv", dt, rows, n_out, n_in)
    out = torch.full((rows, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), dt, n_out, n_in, rows)
    be32.sync()
    ref = O.gemm(dt, w, x, n_out)
    e = rel(host(out), ref)
    say("  rel", e)
    assert e <= GEMV_TOL


@pytest.mark.parametrize("dt", FMTS)
def test_gemv_f16_activations(krk, torch_cuda, be16, dt):
    torch = torch_cuda
    n_out, n_in = 520, 4096
    w = make_weights(krk, dt, n_out, n_in, seed=300 + dt)
    x = krk.synth_normal(n_in, seed=301).astype(np.float16)
    out = torch.empty((1, n_out), dtype=torch.float16, device="cuda")
    be16.gemm(out, dev(torch, x), dev(torch, w), dt, n_out, n_in, 1)
    be16.sync()
    ref = O.gemm(dt, w, x.astype(np.float32), n_out)
    # only the f16 store rounds: 2^-11 relative per element
    assert rel(host(out).astype(np.float32), ref) <= 6e-4


@pytest.mark.parametrize("dt", [O.Q4_K, O.Q5_K])
def test_gemv_exact_path_many_rows(krk, torch_cuda, be32, dt):
    torch = torch_cuda
    rows, n_out, n_in = 13, 136, 1024
    w = make_weights(krk, dt, n_out, n_in, seed=11)
    x = krk.synth_normal(rows * n_in, seed=12).reshape(rows, n_in)
    be32.set_gemm_path(krk.PATH_EXACT)
    try:
        out = torch.empty((rows, n_out), dtype=torch.float32, device="cuda")
        be32.gemm(out, dev(torch, x), dev(torch, w), dt, n_out, n_in, rows)
        be32.sync()
    finally:
        be32.set_gemm_path(krk.PATH_AUTO)
    assert rel(host(out), O.gemm(dt, w, x, n_out)) <= GEMV_TOL
    # rows > 1 reproduce rows == 1 per row within the GEMV bar
    one = torch.empty((1, n_out), dtype=torch.float32, device="cuda")
    be32.gemm(one, dev(torch, x[4:5]), dev(torch, w), dt, n_out, n_in, 1)
    be32.sync()
    assert rel(host(one)[0], host(out)[4]) <= GEMV_TOL


def test_gemm_accumulate(krk, torch_cuda, be32, be16):
    torch = torch_cuda
    dt, n_out, n_in = O.Q6_K, 264, 2048
    w = make_weights(krk, dt, n_out, n_in, seed=21)
    x = krk.synth_normal(n_in, seed=22)
    base = krk.synth_normal(n_out, seed=23)
    dst = dev(torch, base.reshape(1, -1))
    assert be32.gemm_accumulate(dst, dev(torch, x), dev(torch, w), dt, n_out, n_in, 1)
    be32.sync()
    assert rel(host(dst)[0], base + O.gemm(dt, w, x, n_out)[0]) <= GEMV_TOL
    # rows > 1 declines, as the reference's default does
    assert not be32.gemm_accumulate(dev(torch, np.zeros((2, n_out), np.float32)),
                                    dev(torch, np.zeros((2, n_in), np.float32)),
                                    dev(torch, w), dt, n_out, n_in, 2)
    # f16: product rounded to f16, scaled by 2^-rexp, added, saturated
    rexp = dev(torch, np.array([2], np.int32))
    b16 = base.astype(np.float16)
    dst16 = dev(torch, b16.reshape(1, -1))
    assert be16.gemm_accumulate(dst16, dev(torch, x.astype(np.float16)), dev(torch, w), dt,
                                n_out, n_in, 1, rexp)
    be16.sync()
    prod = O.gemm(dt, w, x.astype(np.float16).astype(np.float32), n_out)[0]
    want = (b16.astype(np.float32) + prod.astype(np.float16).astype(np.float32) * 0.25)
    assert rel(host(dst16)[0].astype(np.float32), want) <= 1e-3


def test_gemm_group_qkv_and_silu(krk, torch_cuda, be32):
    torch = torch_cuda
    dt, n_in = O.Q4_K, 2048
    shapes = [512, 256, 256]
    ws = [make_weights(krk, dt, n, n_in, seed=40 + i) for i, n in enumerate(shapes)]
    x = krk.synth_normal(n_in, seed=44)
    outs = [torch.empty((1, n), dtype=torch.float32, device="cuda") for n in shapes]
    fused, sf = be32.gemm_group(outs, dev(torch, x), [dev(torch, w) for w in ws], dt, shapes,
                                n_in, 1)
    be32.sync()
    assert fused and not sf
    for o, w, n in zip(outs, ws, shapes):
        assert rel(host(o)[0], O.gemm(dt, w, x, n)[0]) <= GEMV_TOL
    # gate/up + silu folded: out[0] = silu(gate) * up
    n_ff = 704
    g, u = make_weights(krk, dt, n_ff, n_in, 50), make_weights(krk, dt, n_ff, n_in, 51)
    o0 = torch.empty((1, n_ff), dtype=torch.float32, device="cuda")
    o1 = torch.empty((1, n_ff), dtype=torch.float32, device="cuda")
    fused, sf = be32.gemm_group([o0, o1], dev(torch, x), [dev(torch, g), dev(torch, u)], dt,
                                [n_ff, n_ff], n_in, 1, silu=True)
    be32.sync()
    assert fused and sf
    want = O.silu_mul(O.gemm(dt, g, x, n_ff)[0], O.gemm(dt, u, x, n_ff)[0])
    assert rel(host(o0)[0], want) <= GEMV_TOL


# --------------------------------------------------------------- MFMA GEMM --
@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("shape", [(300, 520, 1024), (64, 256, 4096), (40, 96, 288)])
def test_gemm_mfma_parity(krk, torch_cuda, be16, be32, dt, shape):
    """f16 MFMA GEMM: whole 64-value K steps, a trailing half step (K = 288
    for the 32-value formats) and edge tiles in M and N."""
    torch = torch_cuda
    M, N, K = shape
    if K % krk.BLOCK_VALUES[dt]:
        pytest.skip("K is not a whole number of this format's blocks")
    w = make_weights(krk, dt, N, K, seed=60 + dt)
    x = krk.synth_normal(M * K, seed=61).reshape(M, K).astype(np.float16)
    say("gemm", dt, M, N, K)
    out = torch.empty((M, N), dtype=torch.float16, device="cuda")
    be16.gemm(out, dev(torch, x), dev(torch, w), dt, N, K, M)
    be16.sync()
    ref = O.gemm(dt, w, x.astype(np.float32), N)
    e16 = rel(host(out).astype(np.float32), ref)
    out32 = torch.empty((M, N), dtype=torch.float32, device="cuda")
    be32.gemm(out32, dev(torch, x.astype(np.float32)), dev(torch, w), dt, N, K, M)
    be32.sync()
    e32 = rel(host(out32), ref)
    say("  rel f16-out", e16, "f32-out", e32)
    assert e16 <= GEMM_TOL and e32 <= GEMM_TOL


@pytest.mark.parametrize("dt", [O.Q4_K, O.Q6_K])
def test_gemm_mfma_parity_many_tiles(krk, torch_cuda, be16, dt):
    """384 tiles (no split-K) with an M edge tile of 8 rows."""
    torch = torch_cuda
    M, N, K = 520, 32768, 256
    w = make_weights(krk, dt, N, K, seed=70 + dt)
    x = krk.synth_normal(M * K, seed=71).reshape(M, K).astype(np.float16)
    say("gemm many tiles", dt, M, N, K)
    out = torch.empty((M, N), dtype=torch.float16, device="cuda")
    be16.gemm(out, dev(torch, x), dev(torch, w), dt, N, K, M)
    be16.sync()
    ref = O.gemm(dt, w, x.astype(np.float32), N)
    assert rel(host(out).astype(np.float32), ref) <= GEMM_TOL


@pytest.mark.parametrize("dt", [O.Q4_K, O.Q6_K, O.Q8_0])
@pytest.mark.parametrize("shape", [(300, 2000, 2304), (700, 1000, 4096), (64, 256, 4096),
                                   (300, 10277, 2048)])
def test_gemm_splits_repeat(krk, torch_cuda, be16, be32, dt, shape):
    """Few tiles over the CUs: split-K in four (700 x 1000, K 4096: the reduce
    kernel), in two (82 tiles, K 2048: the splits summed inside the GEMM by
    the last to arrive, ragged M and N edge tiles) and a single split (K
    2304), each checked against the oracle in both activation types and
    bit-equal on a repeated call (partials and tile counters leave no state
    behind)."""
    torch = torch_cuda
    M, N, K = shape
    w = make_weights(krk, dt, N, K, seed=80 + dt)
    x = krk.synth_normal(M * K, seed=81).reshape(M, K).astype(np.float16)
    say("gemm splits", dt, M, N, K)
    ref = O.gemm(dt, w, x.astype(np.float32), N, nthreads=16)
    wd, xd = dev(torch, w), dev(torch, x)
    outs = []
    for _ in range(2):
        out = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
        be16.gemm(out, xd, wd, dt, N, K, M)
        be16.sync()
        outs.append(host(out))
    assert rel(outs[0].astype(np.float32), ref) <= GEMM_TOL
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))
    out32 = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out32, dev(torch, x.astype(np.float32)), wd, dt, N, K, M)
    be32.sync()
    assert rel(host(out32), ref) <= GEMM_TOL


# ------------------------------------------------------------------ router --
# expert counts: each experts-per-lane instantiation (1, 2, 4, 8, 16 of the
# 64 lanes) at and past its boundary
@pytest.mark.parametrize("ne,k", [(8, 2), (64, 8), (65, 8), (128, 8), (129, 6), (256, 8), (300, 8),
                                  (512, 16), (1000, 8), (1024, 64)])
def test_router_softmax_topk(krk, torch_cuda, be32, ne, k):
    torch = torch_cuda
    rng = np.random.default_rng(ne)
    logits = rng.standard_normal((16, ne)).astype(np.float32)
    logits[3, 1] = logits[3, ne - 1] = 6.0
    probs = torch.empty((16, ne), dtype=torch.float32, device="cuda")
    be32.router_softmax(probs, dev(torch, logits), 16, ne)
    be32.sync()
    ref = O.router_softmax(logits)
    assert np.allclose(host(probs), ref, rtol=2e-6, atol=1e-12)
    # selection on identical probabilities is exact, ties to the lower id
    p = dev(torch, ref)
    ids = torch.empty((16, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((16, k), dtype=torch.float32, device="cuda")
    be32.router_topk(p, 16, ne, k, ids, wts, True, 1.0)
    be32.sync()
    rid, rwt = O.router_topk(ref, k)
    assert np.array_equal(host(ids), rid)
    assert np.array_equal(host(wts).view(np.uint32), rwt.view(np.uint32))
    assert host(ids)[3, 0] == 1 and host(ids)[3, 1] == ne - 1


@pytest.mark.parametrize("ne", [40, 128, 200, 300])
def test_router_topk_edge_rows(krk, torch_cuda, be32, ne):
    """top-k on arbitrary inputs: values at or below -1 and NaN are never
    picked, equal values (-0 and +0 among them) go to the lower id, rows with
    fewer candidates than k fill the rest with id -1 and weight 0."""
    torch = torch_cuda
    k = 8
    rng = np.random.default_rng(7 + ne)
    p = rng.random((6, ne)).astype(np.float32)
    p[0, :] = 0.25                                  # all equal
    p[1, :] = -1.0                                  # no candidate
    p[1, [5, ne - 3]] = [0.5, -0.999]               # two candidates
    p[2, ::3] = np.nan
    p[2, 1::3] = -2.0
    p[3, :] = 0.0
    p[3, 1::2] = -0.0                               # +0 / -0 ties
    p[4, :] = rng.integers(0, 3, ne) * 0.125        # many ties
    p[5, :] = -rng.random(ne).astype(np.float32)    # all in (-1, 0]
    ids = torch.empty((6, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((6, k), dtype=torch.float32, device="cuda")
    for norm, scale in ((True, 1.0), (False, 2.5)):
        be32.router_topk(dev(torch, p), 6, ne, k, ids, wts, norm, scale)
        be32.sync()
        rid, rwt = O.router_topk(p, k, norm, scale)
        assert np.array_equal(host(ids), rid)
        assert np.array_equal(host(wts).view(np.uint32), rwt.view(np.uint32))
    assert list(host(ids)[1, 2:]) == [-1] * (k - 2)


# --------------------------------------------------------------------- MoE --
_TABLES = []   # MoE tables built by the running test


@pytest.fixture(autouse=True)
def _forget_moe_tables(request):
    """A dispatched table is remembered by its handle (validated once); the
    test's tables are freed when it ends, so the handles forget them, and a
    later table at a reused address is validated afresh."""
    yield
    for name in ("be32", "be16"):
        if _TABLES and name in request.fixturenames:
            be = request.getfixturevalue(name)
            for t in _TABLES:
                be.moe_table_forget(t)
    _TABLES.clear()


@pytest.fixture
def exact_path(krk, be32):
    """KRK_PATH_EXACT for the test: f32 batches of 32 tokens and more take
    the GEMV paths (the grouped MFMA GEMM otherwise)."""
    be32.set_gemm_path(krk.PATH_EXACT)
    yield
    be32.set_gemm_path(krk.PATH_AUTO)


def build_moe(krk, torch, dt, ne, n_embd, n_ff, seed):
    mats = {}
    entries = []
    keep = []
    for e in range(ne):
        ent = krk.MoeEntry()
        dte = dt[e % len(dt)] if isinstance(dt, list) else dt   # a list: types per expert
        for m, (o, i) in enumerate(((n_ff, n_embd), (n_ff, n_embd), (n_embd, n_ff))):
            dtm = dte if isinstance(dte, int) else dte[m]
            q = make_weights(krk, dtm, o, i, seed=seed + 3 * e + m)
            mats[m, e] = q
            t = dev(torch, q)
            keep.append(t)
            ent.p[m] = t.data_ptr()
            ent.n_out[m], ent.n_in[m] = o, i
            ent.row_bytes[m] = krk.row_bytes(dtm, i)
            ent.type[m] = dtm
            ent.present[m] = 1
        entries.append(ent)
    table = dev(torch, np.frombuffer(krk.moe_table_bytes(entries), np.uint8).copy())
    _TABLES.append(table)
    return mats, table, keep


@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("n_tok", [1, 5])
def test_moe_dispatch_parity(krk, torch_cuda, be32, n_tok, dt):
    """Expert banks of every served weight type, one and several tokens."""
    torch = torch_cuda
    ne, n_embd, n_ff, k = 8, 512, 768, 3
    mats, table, keep = build_moe(krk, torch, dt, ne, n_embd, n_ff, seed=900)
    logits = krk.synth_normal(n_tok * ne, seed=77).reshape(n_tok, ne)
    ids, wts = O.router_topk(O.router_softmax(logits), k)
    x = krk.synth_normal(n_tok * n_embd, seed=78).reshape(n_tok, n_embd)
    say("moe", dt, n_tok, ids.tolist())
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device="cuda")
    be32.moe_dispatch(table, 0, ne, dev(torch, ids), dev(torch, wts), dev(torch, x), out, n_tok,
                      n_embd, n_ff, k)
    be32.sync()
    ref = O.moe_ffn(x, [mats[0, e] for e in range(ne)], [mats[1, e] for e in range(ne)],
                    [mats[2, e] for e in range(ne)], dt, ids, wts, n_ff)
    e = rel(host(out), ref)
    say("  rel", e)
    assert e <= GEMV_TOL


@pytest.mark.usefixtures("exact_path")
@pytest.mark.parametrize("dt", [(O.Q4_K, O.Q4_K, O.Q6_K), (O.Q6_K, O.Q4_K, O.Q8_0)])
@pytest.mark.parametrize("n_tok", [1, 5, 70])
def test_moe_mixed_roles(krk, torch_cuda, be32, n_tok, dt):
    """A Q4_K_M-style layer (Q4_K gate / up with Q6_K down), and gate and up
    of different types (two row passes per expert): the VALU expert path;
    the matrix-core paths take all-Q4_K layers only."""
    torch = torch_cuda
    ne, n_embd, n_ff, k = 8, 512, 1024, 4
    mats, table, keep = build_moe(krk, torch, dt, ne, n_embd, n_ff, seed=980)
    logits = krk.synth_normal(n_tok * ne, seed=99).reshape(n_tok, ne)
    ids, wts = O.router_topk(O.router_softmax(logits), k)
    x = krk.synth_normal(n_tok * n_embd, seed=100).reshape(n_tok, n_embd)
    say("moe mixed", n_tok)
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device="cuda")
    be32.moe_dispatch(table, 0, ne, dev(torch, ids), dev(torch, wts), dev(torch, x), out, n_tok,
                      n_embd, n_ff, k)
    be32.sync()
    ref = O.moe_ffn(x, [mats[0, e] for e in range(ne)], [mats[1, e] for e in range(ne)],
                    [mats[2, e] for e in range(ne)], dt, ids, wts, n_ff)
    assert rel(host(out), ref) <= GEMV_TOL


@pytest.mark.parametrize("n_tok", [1, 5, 70])
def test_moe_types_vary_across_experts(krk, torch_cuda, be32, n_tok):
    """The table carries a type per expert and matrix (moe_table.hpp:47):
    experts of one layer in different formats, gate = up per expert.  The
    reference: each routed expert's FFN by the oracle's GEMV in that
    expert's types, added per token in ascending expert id."""
    torch = torch_cuda
    types = [(O.Q4_K, O.Q4_K, O.Q6_K), (O.Q8_0, O.Q8_0, O.Q4_0), (O.Q6_K, O.Q6_K, O.Q4_K),
             (O.IQ4_NL, O.IQ4_NL, O.Q8_0), (O.Q5_K, O.Q5_K, O.Q5_K)]
    ne, n_embd, n_ff, k = 8, 512, 768, 3
    mats, table, keep = build_moe(krk, torch, types, ne, n_embd, n_ff, seed=1300)
    logits = krk.synth_normal(n_tok * ne, seed=1301).reshape(n_tok, ne)
    ids, wts = O.router_topk(O.router_softmax(logits), k)
    x = krk.synth_normal(n_tok * n_embd, seed=1302).reshape(n_tok, n_embd)
    say("moe types per expert", n_tok)
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device="cuda")
    be32.moe_dispatch(table, 0, ne, dev(torch, ids), dev(torch, wts), dev(torch, x), out, n_tok,
                      n_embd, n_ff, k)
    be32.sync()
    ref = np.zeros((n_tok, n_embd))
    for t in range(n_tok):
        for e, s in sorted((int(ids[t, s]), s) for s in range(k)):
            tg, tu, td = types[e % len(types)]
            g = O.gemm(tg, mats[0, e], x[t], n_ff)[0]
            u = O.gemm(tu, mats[1, e], x[t], n_ff)[0]
            ref[t] += float(wts[t, s]) * O.gemm(td, mats[2, e], O.silu_mul(g, u), n_embd)[0]
    assert rel(host(out), ref.astype(np.float32)) <= GEMV_TOL


@pytest.mark.parametrize("n_rows,k,ne,drop", [(1, 8, 128, 0), (70, 8, 128, 5), (16, 4, 256, 3),
                                               (300, 6, 300, 0)])
def test_moe_plan_build(krk, torch_cuda, be32, rng, n_rows, k, ne, drop):
    """Backend::moe_plan_build against the oracle: offsets, rows and weights
    in expert-major, then (row, slot) order, bit for bit; dropped pairs (id -1)
    leave the tail unwritten.  300 experts: every expert is placed (the
    reference's cursors stop at 256, router.hpp:263-268)."""
    torch = torch_cuda
    ids = np.stack([rng.choice(ne, size=k, replace=False) for _ in range(n_rows)]).astype(np.int32)
    if drop:
        ids.reshape(-1)[rng.choice(ids.size, size=drop, replace=False)] = -1
    wts = rng.random((n_rows, k), dtype=np.float32)
    want_off, want_rows, want_wt = O.moe_plan_build(ids, ne, wts)
    P = n_rows * k
    off = torch.full((ne + 1,), -7, dtype=torch.int32, device="cuda")
    rows = torch.full((P,), -1, dtype=torch.int32, device="cuda")
    wt = torch.full((P,), float("nan"), dtype=torch.float32, device="cuda")
    be32.moe_plan_build(dev(torch, ids), n_rows, k, ne, off, rows, wt, dev(torch, wts))
    be32.sync()
    n = int(want_off[-1])
    assert np.array_equal(host(off), want_off)
    assert np.array_equal(host(rows)[:n], want_rows[:n]) and (host(rows)[n:] == -1).all()
    assert np.array_equal(host(wt)[:n], want_wt[:n])
    be32.moe_plan_build(dev(torch, ids), n_rows, k, ne, off, rows, wt, None)
    be32.sync()
    assert (host(wt)[:n] == 0.0).all()


def test_scan_accum(krk, torch_cuda, be32, rng):
    """Backend::scan_accum against the oracle: two layers, two calls on one
    (the histograms accumulate), dropped ids skipped; hits exact and mass
    bit-equal (each expert's sum runs in row order, one add per call)."""
    torch = torch_cuda
    ne, k, n_layer = 128, 8, 3
    hits_h = np.zeros(n_layer * ne, np.uint32)
    mass_h = np.zeros(n_layer * ne, np.float32)
    hits = dev(torch, hits_h.view(np.int32))
    mass = dev(torch, mass_h)
    for layer, n_rows, seed in ((1, 16, 1), (1, 5, 2), (2, 70, 3)):
        logits = krk.synth_normal(n_rows * ne, seed=1400 + seed).reshape(n_rows, ne)
        probs = O.router_softmax(logits)
        ids, _ = O.router_topk(probs, k)
        ids[0, 0] = -1
        be32.scan_accum(dev(torch, probs), dev(torch, ids), n_rows, ne, k, layer, hits, mass)
        O.scan_accum(probs, ids, ne, layer, hits_h, mass_h)
    be32.sync()
    assert np.array_equal(host(hits).view(np.uint32), hits_h)
    assert np.array_equal(host(mass), mass_h)


def f16_ulps(a, b):
    """Distance in f16 steps between two float16 arrays (same-sign finite)."""
    ia = a.view(np.int16).astype(np.int32)
    ib = b.view(np.int16).astype(np.int32)
    ia = np.where(ia < 0, -32768 - ia, ia)
    ib = np.where(ib < 0, -32768 - ib, ib)
    return np.abs(ia - ib)


@pytest.mark.parametrize("dt", [O.Q4_K, O.Q6_K, O.Q8_0, O.Q5_K, O.IQ4_XS, O.MXFP4, (O.Q6_K, O.Q4_K, O.Q8_0)])
@pytest.mark.parametrize("n_tok", [1, 5, 70])
def test_moe_dispatch_f16_activations(krk, torch_cuda, be16, n_tok, dt):
    """f16 activations (the reference GPU backend's own act_type) follow its
    rounding points (moe_table.hpp:250-305, 418-441, 536-551): gate and up
    dots rounded to f16 before the activation, each (token, slot) row scaled
    by a power of two and rounded to f16 for the down dot, the partial
    w * (f16(v) * scale), and the slots added in slot order with an f16
    rounding after every add.  The oracle restates exactly that
    (orc_moe_ffn_f16, pinned by closed forms in test_oracle.py).  The row
    dots' own f32 order differs from the oracle's chain by ~1e-7, which moves
    an intermediate f16 rounding by one step now and then, and that step
    propagates; so the bar is: most outputs bit-equal (measured 90-99%), the
    rest within 3e-4 relative over the output (measured 4e-5..2e-4), and at
    most half the distance between the f16 and f32 oracles (~5.4e-4) -- a
    dispatch with the f32 oracle's rounding points would sit at that
    distance and fail."""
    torch = torch_cuda
    ne, n_embd, n_ff, k = 8, 512, 768, 3
    mats, table, keep = build_moe(krk, torch, dt, ne, n_embd, n_ff, seed=1900)
    logits = krk.synth_normal(n_tok * ne, seed=177).reshape(n_tok, ne)
    ids, wts = O.router_topk(O.router_softmax(logits), k)
    x = krk.synth_normal(n_tok * n_embd, seed=178).reshape(n_tok, n_embd).astype(np.float16)
    say("moe f16", dt, n_tok)
    out = torch.empty((n_tok, n_embd), dtype=torch.float16, device="cuda")
    be16.moe_dispatch(table, 0, ne, dev(torch, ids), dev(torch, wts), dev(torch, x), out, n_tok,
                      n_embd, n_ff, k)
    be16.sync()
    ref = O.moe_ffn_f16(x.astype(np.float32), [mats[0, e] for e in range(ne)], [mats[1, e] for e in range(ne)],
                        [mats[2, e] for e in range(ne)], dt, ids, wts, n_ff)
    got = host(out)
    u = f16_ulps(got, ref)
    ref32 = O.moe_ffn(x.astype(np.float32), [mats[0, e] for e in range(ne)], [mats[1, e] for e in range(ne)],
                      [mats[2, e] for e in range(ne)], dt, ids, wts, n_ff)
    e16 = rel(got.astype(np.float32), ref.astype(np.float32))
    gap = rel(ref.astype(np.float32), ref32)
    say("  bit-equal", float((u == 0).mean()), "rel to the f16 oracle", e16, "f16-f32 oracle gap", gap)
    assert (u == 0).mean() >= 0.85
    assert e16 <= 3e-4
    assert e16 <= 0.5 * gap


def test_moe_table_rewritten_in_place(krk, torch_cuda, be32):
    """A dispatched table rewritten in place (same address, another bank
    type) is read and checked again after krk_moe_table_forget."""
    torch = torch_cuda
    ne, n_embd, n_ff, k, n_tok = 8, 512, 768, 2, 2
    logits = krk.synth_normal(n_tok * ne, seed=97).reshape(n_tok, ne)
    ids, wts = O.router_topk(O.router_softmax(logits), k)
    x = krk.synth_normal(n_tok * n_embd, seed=98).reshape(n_tok, n_embd)
    mats_a, table, keep_a = build_moe(krk, torch, O.Q4_K, ne, n_embd, n_ff, seed=960)
    mats_b, table_b, keep_b = build_moe(krk, torch, O.IQ4_NL, ne, n_embd, n_ff, seed=970)
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device="cuda")
    for mats, dt in ((mats_a, O.Q4_K), (mats_b, O.IQ4_NL)):
        if dt == O.IQ4_NL:
            be32.moe_table_forget(table)
            table.copy_(table_b)       # the same address now holds the other layer
        say("moe table", dt)
        be32.moe_dispatch(table, 0, ne, dev(torch, ids), dev(torch, wts), dev(torch, x), out, n_tok,
                          n_embd, n_ff, k)
        be32.sync()
        ref = O.moe_ffn(x, [mats[0, e] for e in range(ne)], [mats[1, e] for e in range(ne)],
                        [mats[2, e] for e in range(ne)], dt, ids, wts, n_ff)
        assert rel(host(out), ref) <= GEMV_TOL


def test_moe_table_row_bytes_checked(krk, torch_cuda, be32):
    """A bank whose row_bytes is not its type's row size (a padded stride)
    is refused before any launch: the kernels step rows by the type's size
    (the reference reads row_bytes per matrix, moe_table.hpp:108-168)."""
    torch = torch_cuda
    ne, n_embd, n_ff, k = 4, 512, 512, 2
    mats, table, keep = build_moe(krk, torch, O.Q4_K, ne, n_embd, n_ff, seed=980)
    ent = np.frombuffer(bytes(host(table)), np.uint8).copy()
    entries = (krk.MoeEntry * ne).from_buffer(ent)
    entries[2].row_bytes[2] += 16
    bad = dev(torch, ent)
    _TABLES.append(bad)
    ids = dev(torch, np.array([[0, 2]], np.int32))
    wts = dev(torch, np.array([[0.5, 0.5]], np.float32))
    x = dev(torch, krk.synth_normal(n_embd, seed=981).reshape(1, n_embd))
    out = torch.full((1, n_embd), 3.0, dtype=torch.float32, device="cuda")
    with pytest.raises(krk.KrkError, match="row_bytes"):
        be32.moe_dispatch(bad, 0, ne, ids, wts, x, out, 1, n_embd, n_ff, k)
    be32.sync()
    assert bool((out == 3.0).all())


def test_moe_table_record_evicts_oldest(krk, torch_cuda):
    """Past 256 remembered (table, layer) keys the oldest is dropped, not the
    newest refused: every layer still dispatches, and re-dispatching the
    first layer (dropped, so read and checked again) gives the same bytes."""
    torch = torch_cuda
    be = krk.Backend(0, krk.ACT_F32)
    try:
        ne, n_embd, n_ff, k, L = 2, 256, 256, 1, 300
        mats, table1, keep = build_moe(krk, torch, O.Q4_K, ne, n_embd, n_ff, seed=985)
        # L layers that all point at the same banks
        one = np.frombuffer(bytes(host(table1)), np.uint8)
        table = dev(torch, np.tile(one, L))
        ids = dev(torch, np.array([[1]], np.int32))
        wts = dev(torch, np.array([[1.0]], np.float32))
        x = dev(torch, krk.synth_normal(n_embd, seed=986).reshape(1, n_embd))
        outs = []
        for layer in (0, *range(1, L), 0):
            out = torch.empty((1, n_embd), dtype=torch.float32, device="cuda")
            be.moe_dispatch(table, layer, ne, ids, wts, x, out, 1, n_embd, n_ff, k)
            outs.append(out)
        be.sync()
        first, last = host(outs[0]), host(outs[-1])
        assert np.array_equal(first.view(np.uint32), last.view(np.uint32))
        ref = O.moe_ffn(host(x), [mats[0, e] for e in range(ne)], [mats[1, e] for e in range(ne)],
                        [mats[2, e] for e in range(ne)], O.Q4_K, np.array([[1]], np.int32),
                        np.array([[1.0]], np.float32), n_ff)
        assert rel(last, ref) <= GEMV_TOL
        be.moe_table_forget(table)
    finally:
        be.close()


@pytest.mark.usefixtures("exact_path")
@pytest.mark.parametrize("n_tok,k,drop", [(1, 2, False), (1, 8, False), (1, 4, True), (3, 4, True),
                                          (16, 8, False), (70, 2, True), (520, 8, True)])
def test_moe_dispatch_whole_units(krk, torch_cuda, be32, n_tok, k, drop):
    """n_ff a multiple of 512: one token runs gate/up and down on the
    register-streaming kernel (down over the concatenated slots, each wave's
    slice inside one slot); 2..64 tokens on the digit-plane kernel, one
    workgroup group per token; 70 and 520 tokens take expert-major items
    (520 x 8 pairs exceed the plan's LDS copy of the ids).  drop: a slot
    with id -1 contributes nothing, as in the host loop."""
    torch = torch_cuda
    dt, ne, n_embd, n_ff = O.Q4_K, 8, 1024, 1024
    mats, table, keep = build_moe(krk, torch, dt, ne, n_embd, n_ff, seed=950)
    logits = krk.synth_normal(n_tok * ne, seed=81 + k).reshape(n_tok, ne)
    ids, wts = O.router_topk(O.router_softmax(logits), k)
    if drop:
        ids[0, 1] = -1
        ids[n_tok - 1, k - 1] = -1
    x = krk.synth_normal(n_tok * n_embd, seed=82).reshape(n_tok, n_embd)
    say("moe whole units", n_tok, k, ids.tolist())
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device="cuda")
    be32.moe_dispatch(table, 0, ne, dev(torch, ids), dev(torch, wts), dev(torch, x), out, n_tok,
                      n_embd, n_ff, k)
    be32.sync()
    ref = O.moe_ffn(x, [mats[0, e] for e in range(ne)], [mats[1, e] for e in range(ne)],
                    [mats[2, e] for e in range(ne)], dt, ids, wts, n_ff)
    e = rel(host(out), ref)
    say("  rel", e)
    assert e <= GEMV_TOL


@pytest.mark.parametrize("rows,n_out,n_in", [(2, 520, 4096), (4, 300, 4096), (7, 200, 4096),
                                          (3, 96, 14336), (8, 64, 11008), (5, 40, 256)])
def test_q4_k_digits_rows(krk, torch_cuda, be32, rows, n_out, n_in):
    """Rows 2..8 on the digit-plane kernel: passes of up to 4 activation rows
    (2 for rows longer than 8192 values) share each weight unit."""
    torch = torch_cuda
    w = make_weights(krk, O.Q4_K, n_out, n_in, seed=800 + rows)
    x = krk.synth_normal(rows * n_in, seed=801 + rows).reshape(rows, n_in)
    say("digits rows", rows, n_out, n_in)
    out = torch.full((rows, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), O.Q4_K, n_out, n_in, rows)
    be32.sync()
    ref = O.gemm(O.Q4_K, w, x, n_out)
    for r in range(rows):
        assert rel(host(out)[r], ref[r]) <= GEMV_TOL, r


def test_q4_k_digits_rows_f16(krk, torch_cuda, be16):
    torch = torch_cuda
    rows, n_out, n_in = 3, 260, 4096
    w = make_weights(krk, O.Q4_K, n_out, n_in, seed=820)
    x = krk.synth_normal(rows * n_in, seed=821).reshape(rows, n_in).astype(np.float16)
    out = torch.empty((rows, n_out), dtype=torch.float16, device="cuda")
    be16.gemm(out, dev(torch, x), dev(torch, w), O.Q4_K, n_out, n_in, rows)
    be16.sync()
    ref = O.gemm(O.Q4_K, w, x.astype(np.float32), n_out)
    assert rel(host(out).astype(np.float32), ref) <= 6e-4


# ------------------------------------------------- digit-plane edge cases --
def digit_edge_x(n_in, seed):
    """Activations whose 32-value sub-blocks put the digit split at its
    limits: a largest magnitude just under a power of two (the top int8 digit
    at its bound), constant sub-blocks, zero, subnormal and wide-range ones."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n_in).astype(np.float32)
    top = np.float32(np.nextafter(np.float32(2.0), np.float32(0.0)))   # 2 - 2^-23
    for sb in range(n_in // 32):
        v = x[32 * sb:32 * sb + 32]
        kind, scale = sb % 6, np.float32(2.0) ** int(rng.integers(-8, 8))
        if kind == 0:
            np.clip(v, -1.9, 1.9, out=v)
            v[int(rng.integers(32))] = top * (1 if sb % 2 else -1)
        elif kind == 1:
            v[:] = top
        elif kind == 2:
            v[:] = -top * rng.uniform(0.999, 1.0, 32).astype(np.float32)
        elif kind == 3:
            v[:] = 0.0
        elif kind == 4:
            v[:] = v * np.float32(1e-41)
        v *= scale
    return x


@pytest.mark.parametrize("n_in", [512, 4096, 14336])
def test_q4_k_digits_extreme_sub_blocks(krk, torch_cuda, be32, n_in):
    torch = torch_cuda
    n_out = 96
    w = make_weights(krk, O.Q4_K, n_out, n_in, seed=700 + n_in)
    x = digit_edge_x(n_in, seed=n_in)
    say("digits edge", n_out, n_in)
    out = torch.empty((1, n_out), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), O.Q4_K, n_out, n_in, 1)
    be32.sync()
    assert rel(host(out)[0], O.gemm(O.Q4_K, w, x, n_out)[0]) <= GEMV_TOL


@pytest.mark.parametrize("rows,n_out,n_in", [(1, 300, 4096), (3, 520, 2048), (1, 64, 16384),
                                          (8, 40, 512), (2, 130, 14336)])
def test_q6_k_digits(krk, torch_cuda, be32, rows, n_out, n_in):
    """Q6_K on the digit-plane kernel: two-block units packed by dword
    LDS-DMA, one MFMA per 16-value scale group, the code offset 32 applied
    through exact integer sums of the activation digits."""
    torch = torch_cuda
    w = make_weights(krk, O.Q6_K, n_out, n_in, seed=840 + rows)
    x = krk.synth_normal(rows * n_in, seed=841 + rows).reshape(rows, n_in)
    say("q6_k digits", rows, n_out, n_in)
    out = torch.full((rows, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), O.Q6_K, n_out, n_in, rows)
    be32.sync()
    ref = O.gemm(O.Q6_K, w, x, n_out)
    for r in range(rows):
        assert rel(host(out)[r], ref[r]) <= GEMV_TOL, r


def test_q6_k_digits_extreme_sub_blocks(krk, torch_cuda, be32, be16):
    torch = torch_cuda
    n_out, n_in = 96, 4096
    w = make_weights(krk, O.Q6_K, n_out, n_in, seed=850)
    x = digit_edge_x(n_in, seed=851)
    out = torch.empty((1, n_out), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), O.Q6_K, n_out, n_in, 1)
    be32.sync()
    assert rel(host(out)[0], O.gemm(O.Q6_K, w, x, n_out)[0]) <= GEMV_TOL
    xh = krk.synth_normal(n_in, seed=852).astype(np.float16)
    out16 = torch.empty((1, n_out), dtype=torch.float16, device="cuda")
    be16.gemm(out16, dev(torch, xh), dev(torch, w), O.Q6_K, n_out, n_in, 1)
    be16.sync()
    assert rel(host(out16).astype(np.float32), O.gemm(O.Q6_K, w, xh.astype(np.float32), n_out)) <= 6e-4


@pytest.mark.parametrize("dt,rows,n_out", [(O.Q4_K, 1, 70001), (O.Q4_K, 2, 70000), (O.Q6_K, 1, 66001),
                                          (O.Q6_K, 3, 66000), (O.Q8_0, 2, 70003), (O.Q4_0, 2, 66002)])
def test_digits_row_split(krk, torch_cuda, be32, dt, rows, n_out):
    """Enough tiles that each wave owns whole tiles (no cross-wave
    reduction), with a partial last tile."""
    torch = torch_cuda
    n_in = 512
    w = make_weights(krk, dt, n_out, n_in, seed=860 + rows)
    x = krk.synth_normal(rows * n_in, seed=861 + rows).reshape(rows, n_in)
    say("row split", dt, rows, n_out, n_in)
    out = torch.full((rows, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), dt, n_out, n_in, rows)
    be32.sync()
    ref = O.gemm(dt, w, x, n_out)
    for r in range(rows):
        assert rel(host(out)[r], ref[r]) <= GEMV_TOL, r


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("rows,n_out,n_in", [(2, 300, 4096), (4, 96, 1024), (3, 50, 16384)])
def test_small_block_digits(krk, torch_cuda, be32, dt, rows, n_out, n_in):
    """Q8_0 and Q4_0 with 2..8 rows on the digit-plane kernel: 32-value
    blocks placed in 16-byte-aligned LDS slots, Q8_0 codes as the int8
    operand, Q4_0 nibbles with the offset 8 applied through exact integer
    digit sums; row 0 carries the extreme sub-blocks."""
    torch = torch_cuda
    w = make_weights(krk, dt, n_out, n_in, seed=870 + rows)
    x = krk.synth_normal(rows * n_in, seed=871 + rows).reshape(rows, n_in)
    x[0] = digit_edge_x(n_in, seed=872)
    say("small-block digits", dt, rows, n_out, n_in)
    out = torch.full((rows, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), dt, n_out, n_in, rows)
    be32.sync()
    ref = O.gemm(dt, w, x, n_out)
    for r in range(rows):
        assert rel(host(out)[r], ref[r]) <= GEMV_TOL, r


# ------------------------------------------------- full-size configurations --
def test_headline_q4_k_gemv_full_size(krk, torch_cuda, be32):
    """BASELINE config 2 headline shape: Q4_K 4096 -> 14336, M = 1."""
    torch = torch_cuda
    n_out, n_in = 14336, 4096
    w = make_weights(krk, O.Q4_K, n_out, n_in, seed=1)
    x = krk.synth_normal(n_in, seed=2)
    out = torch.empty((1, n_out), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), O.Q4_K, n_out, n_in, 1)
    be32.sync()
    assert rel(host(out), O.gemm(O.Q4_K, w, x, n_out)) <= GEMV_TOL


def test_q8_0_config1_gemv(krk, torch_cuda, be32):
    """Q8_0 2048 x 2048, weights N(0, 0.02), x N(0, 1)."""
    torch = torch_cuda
    w = make_weights(krk, O.Q8_0, 2048, 2048, seed=3)
    x = krk.synth_normal(2048, seed=4)
    out = torch.empty((1, 2048), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), O.Q8_0, 2048, 2048, 1)
    be32.sync()
    assert rel(host(out), O.gemm(O.Q8_0, w, x, 2048)) <= GEMV_TOL


# ------------------------------------------------------------- int8 rung --
@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(17, 96, 256), (130, 200, 2048), (256, 384, 4096)])
def test_int8_rung_q8_0_bit_exact(krk, torch_cuda, be16, be32, shape):
    """KRK_PATH_INT8: Q8_0 weights x activations quantized per 32
    (quantize_q8_32_d), integer block dots folded as fma(isum, dw*dx, acc) in
    block order -- bit-identical to dot_q8_0_q8_scalar (quant.cpp:3261-3279)."""
    torch = torch_cuda
    M, N, K = shape
    w = make_weights(krk, krk.Q8_0, N, K, seed=70)
    x = krk.synth_normal(M * K, seed=71).reshape(M, K)
    x[0, :32] = 0.0                      # an all-zero block: d = 0, codes 0
    x[1, 5] = 6.0e4                      # one large value: the rest of its block rounds to 0
    say("int8 rung", M, N, K)
    ref = O.gemm_q8_0_q8(w, x, N)
    for be in (be32, be16):
        be.set_gemm_path(krk.PATH_INT8)
    try:
        out32 = torch.empty((M, N), dtype=torch.float32, device="cuda")
        be32.gemm(out32, dev(torch, x), dev(torch, w), krk.Q8_0, N, K, M)
        be32.sync()
        assert np.array_equal(host(out32).view(np.uint32), ref.view(np.uint32))
        xh = x.astype(np.float16)
        ref16 = O.gemm_q8_0_q8(w, xh.astype(np.float32), N).astype(np.float16)
        out16 = torch.empty((M, N), dtype=torch.float16, device="cuda")
        be16.gemm(out16, dev(torch, xh), dev(torch, w), krk.Q8_0, N, K, M)
        be16.sync()
        assert np.array_equal(host(out16).view(np.uint16), ref16.view(np.uint16))
    finally:
        for be in (be32, be16):
            be.set_gemm_path(krk.PATH_AUTO)


@pytest.mark.parametrize("dt", [O.Q4_K, O.Q5_K, O.Q6_K])
@pytest.mark.parametrize("shape", [(300, 520, 1024), (64, 256, 4096), (17, 40, 256)])
def test_int8_rung_kquants(krk, torch_cuda, be16, be32, dt, shape):
    """KRK_PATH_INT8 for the K-quants: the fold the oracle restates
    (orc_dot_kq_q8: the reference GPU rung's two-term fold for Q4_K / Q5_K,
    gemm_dp4a.hpp:532-552; the CPU twin's I - 32 S for Q6_K), bit for bit,
    with edge tiles in M and N."""
    torch = torch_cuda
    M, N, K = shape
    w = make_weights(krk, dt, N, K, seed=74 + dt)
    x = krk.synth_normal(M * K, seed=75).reshape(M, K)
    x[0, :32] = 0.0
    say("int8 rung", dt, M, N, K)
    ref = O.gemm_int8(dt, w, x, N)
    for be in (be32, be16):
        be.set_gemm_path(krk.PATH_INT8)
    try:
        out32 = torch.empty((M, N), dtype=torch.float32, device="cuda")
        be32.gemm(out32, dev(torch, x), dev(torch, w), dt, N, K, M)
        be32.sync()
        assert np.array_equal(host(out32).view(np.uint32), ref.view(np.uint32))
        xh = x.astype(np.float16)
        ref16 = O.gemm_int8(dt, w, xh.astype(np.float32), N).astype(np.float16)
        out16 = torch.empty((M, N), dtype=torch.float16, device="cuda")
        be16.gemm(out16, dev(torch, xh), dev(torch, w), dt, N, K, M)
        be16.sync()
        assert np.array_equal(host(out16).view(np.uint16), ref16.view(np.uint16))
    finally:
        for be in (be32, be16):
            be.set_gemm_path(krk.PATH_AUTO)


@pytest.mark.gpu
def test_int8_rung_refuses_other_formats(krk, torch_cuda, be32):
    torch = torch_cuda
    be32.set_gemm_path(krk.PATH_INT8)
    try:
        w = make_weights(krk, krk.Q4_0, 32, 256, seed=72)
        x = dev(torch, krk.synth_normal(16 * 256, seed=73).reshape(16, 256))
        out = torch.empty((16, 32), dtype=torch.float32, device="cuda")
        with pytest.raises(krk.KrkError, match="UNSUPPORTED|int8 rung"):
            be32.gemm(out, x, dev(torch, w), krk.Q4_0, 32, 256, 16)
    finally:
        be32.set_gemm_path(krk.PATH_AUTO)


def test_moe_dispatch_graph_replay(krk, torch_cuda, be32):
    """After the first (checking) call a dispatch is asynchronous: it can be
    captured in a HIP graph, and every replay equals the eager result."""
    torch = torch_cuda
    dt, ne, n_embd, n_ff, k, n_tok = O.Q4_K, 8, 512, 512, 2, 3
    mats, table, keep = build_moe(krk, torch, dt, ne, n_embd, n_ff, seed=950)
    logits = krk.synth_normal(n_tok * ne, seed=79).reshape(n_tok, ne)
    ids, wts = O.router_topk(O.router_softmax(logits), k)
    x = dev(torch, krk.synth_normal(n_tok * n_embd, seed=80).reshape(n_tok, n_embd))
    dids, dwts = dev(torch, ids), dev(torch, wts)
    eager = torch.empty((n_tok, n_embd), dtype=torch.float32, device="cuda")
    be32.moe_dispatch(table, 0, ne, dids, dwts, x, eager, n_tok, n_embd, n_ff, k)
    be32.sync()
    out = torch.zeros((n_tok, n_embd), dtype=torch.float32, device="cuda")
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    main = be32.stream
    with torch.cuda.graph(g, stream=side):
        be32.set_stream(side)
        be32.moe_dispatch(table, 0, ne, dids, dwts, x, out, n_tok, n_embd, n_ff, k)
    be32.set_stream(main)
    want = host(eager)
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(out).view(np.uint32), want.view(np.uint32)), rep


@pytest.mark.parametrize("shape", [(300, 10277, 2048), (700, 1000, 4096)])
def test_gemm_graph_replay(krk, torch_cuda, be16, shape):
    """The MFMA GEMM captured in a HIP graph: two splits summed in the GEMM
    through per-tile counters (300 x 10277, K 2048), four splits through the
    reduce kernel (700 x 1000, K 4096).  Every replay, with eager GEMMs of
    the same shape on other operands between the replays, equals the eager
    result bit for bit (the counters are back at zero after every call)."""
    torch = torch_cuda
    M, N, K = shape
    w = dev(torch, make_weights(krk, O.Q4_K, N, K, seed=970))
    w2 = dev(torch, make_weights(krk, O.Q4_K, N, K, seed=971))
    x = dev(torch, krk.synth_normal(M * K, seed=972).reshape(M, K).astype(np.float16))
    eager = torch.empty((M, N), dtype=torch.float16, device="cuda")
    be16.gemm(eager, x, w, O.Q4_K, N, K, M)
    be16.sync()
    want = host(eager)
    other = torch.empty((M, N), dtype=torch.float16, device="cuda")
    out = torch.empty((M, N), dtype=torch.float16, device="cuda")
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    main = be16.stream
    with torch.cuda.graph(g, stream=side):
        be16.set_stream(side)
        be16.gemm(out, x, w, O.Q4_K, N, K, M)
    be16.set_stream(main)
    for rep in range(3):
        out.fill_(float("nan"))
        be16.gemm(other, x, w2, O.Q4_K, N, K, M)
        be16.sync()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(out).view(np.uint16), want.view(np.uint16)), rep


def test_handles_on_host_threads(krk, torch_cuda):
    """Four host threads, each with its own handle and stream, run GEMVs and
    GEMMs of several types and shapes at the same time (the launchers' shape
    caches are per thread; a handle's calls stay on its thread): every result
    equals a one-thread run of the same calls bit for bit."""
    import threading

    torch = torch_cuda
    cases = [(O.Q4_K, 1, 3072, 4096), (O.Q8_0, 1, 2048, 2048), (O.Q6_K, 1, 1536, 4096),
             (O.Q5_K, 3, 1000, 2048), (O.Q4_0, 1, 4096, 1024), (O.Q4_K, 300, 520, 2048)]
    ops = []
    for i, (dt, rows, n_out, n_in) in enumerate(cases):
        w = dev(torch, make_weights(krk, dt, n_out, n_in, seed=1100 + i))
        x = dev(torch, krk.synth_normal(rows * n_in, seed=1110 + i).reshape(rows, n_in))
        ops.append((dt, rows, n_out, n_in, w, x))

    def run(be, stream):
        outs = []
        with torch.cuda.stream(stream):
            for dt, rows, n_out, n_in, w, x in ops:
                o = torch.empty((rows, n_out), dtype=torch.float32, device="cuda")
                be.gemm(o, x, w, dt, n_out, n_in, rows)
                outs.append(o)
        be.sync()
        return [host(o) for o in outs]

    be0 = krk.Backend(0, krk.ACT_F32, stream=torch.cuda.Stream())
    try:
        want = run(be0, be0.stream)
    finally:
        be0.close()
    got, errs = [None] * 4, []

    def worker(k):
        try:
            st = torch.cuda.Stream()
            be = krk.Backend(0, krk.ACT_F32, stream=st)
            try:
                for _ in range(3):
                    got[k] = run(be, st)
            finally:
                be.close()
        except Exception as e:   # reported in the main thread
            errs.append(e)

    ts = [threading.Thread(target=worker, args=(k,)) for k in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errs, errs
    for k in range(4):
        for a, b in zip(got[k], want):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_error_paths_write_nothing(krk, torch_cuda, be32):
    """Arguments the reference aborts on (a K that is not whole blocks,
    backend_hip.hip:3186-3191; geometry moe_dispatch cannot express,
    2500-2524) come back here as status codes, before any launch: the output
    keeps its sentinel and the backend stays usable for the next call."""
    torch = torch_cuda
    n_out, n_in = 64, 4096
    w = dev(torch, make_weights(krk, O.Q4_K, n_out, n_in, seed=990))
    x = dev(torch, krk.synth_normal(2 * n_in, seed=991))
    out = torch.full((2, n_out), float("nan"), dtype=torch.float32, device="cuda")
    cases = [
        ("not whole blocks", lambda: be32.gemm(out, x, w, O.Q4_0, n_out, 100, 1), "shape"),
        ("type not served", lambda: be32.gemm(out, x, w, 24, n_out, n_in, 1), "type"),
        ("zero rows", lambda: be32.gemm(out, x, w, O.Q4_K, n_out, n_in, 0), "argument"),
        ("zero outputs", lambda: be32.gemm(out, x, w, O.Q4_K, 0, n_in, 1), "argument"),
        ("x under-aligned", lambda: be32.gemm(out, x[1:], w, O.Q4_K, n_out, n_in, 1), "argument"),
        ("w under-aligned", lambda: be32.gemm(out, x, w[1:], O.Q4_K, n_out, n_in, 1), "argument"),
        ("k above n_expert", lambda: be32.router_topk(out, 1, 4, 8, out, out), "argument"),
    ]
    for name, call, word in cases:
        say("error path", name)
        with pytest.raises(krk.KrkError, match=f"(?i){word}"):
            call()
    be32.sync()
    assert torch.isnan(out).all()
    be32.gemm(out, x, w, O.Q4_K, n_out, n_in, 2)
    be32.sync()
    ref = O.gemm(O.Q4_K, host(w), host(x).reshape(2, n_in), n_out)
    assert rel(host(out), ref) <= GEMV_TOL
