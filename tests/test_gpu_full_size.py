"""GPU parity at the BASELINE configurations' full shapes.

The other GPU modules pin every kernel against the oracle at reduced sizes;
this one runs each benchmarked configuration at the shape the bench times,
so tile counts, split-K choices, row-split modes and slot counts are the
ones that run there:

* config 2: Llama-2-7B Q4_K decode layer at M = 1 -- q/k/v/o 4096^2,
  gate/up 4096 -> 11008, down 11008 -> 4096 -- one matrix at a time, and as
  the engine issues it (gemm_group q/k/v; gate/up with the SiLU epilogue);
* config 3: Q4_K prefill GEMM, up 4096 -> 14336 and down 14336 -> 4096, at
  M = 512 and 2048, checked on 64 output rows spread over M (the oracle's
  single chain for the whole output would take minutes);
* config 4: Q6_K output head 128256 x 4096 at M = 1 (the row-split mode at
  its real K), and the Q8_0 head with Q8-quantized activations on the int8
  rung (bit-exact against the oracle's fold);
* config 5: qwen3moe MoE layer, 128 experts of Q4_K gate/up 4096 -> 1536 and
  down 1536 -> 4096, router softmax -> top-8 -> normalize, 1 and 16 tokens.

Tolerances are the north_star's: GEMV 1e-5 relative, f16 MFMA GEMM 2e-3
relative Frobenius; int8 rung bit-exact.
"""
import numpy as np
import pytest

import oracle as O
from test_gpu_parity import GEMM_TOL, GEMV_TOL, build_moe, dev, host, make_weights, rel, say  # noqa: F401

pytestmark = pytest.mark.gpu

LLAMA2 = {"q": (4096, 4096), "k": (4096, 4096), "v": (4096, 4096), "o": (4096, 4096),
          "gate": (11008, 4096), "up": (11008, 4096), "down": (4096, 11008)}


@pytest.fixture(scope="module")
def llama2_layer(krk):
    return {nm: make_weights(krk, O.Q4_K, o, i, seed=300 + j)
            for j, (nm, (o, i)) in enumerate(LLAMA2.items())}


@pytest.mark.parametrize("name", list(LLAMA2))
def test_config2_layer_matrix(krk, torch_cuda, be32, llama2_layer, name):
    torch = torch_cuda
    n_out, n_in = LLAMA2[name]
    w = llama2_layer[name]
    x = krk.synth_normal(n_in, seed=310)
    say("config 2", name, n_out, n_in)
    out = torch.full((1, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), O.Q4_K, n_out, n_in, 1)
    be32.sync()
    e = rel(host(out), O.gemm(O.Q4_K, w, x, n_out, nthreads=16))
    say("  rel", e)
    assert e <= GEMV_TOL


def test_config2_layer_grouped(krk, torch_cuda, be32, llama2_layer):
    """q/k/v in one grouped launch, gate/up with the SiLU epilogue, then o and
    down on the grouped results -- the four launches of one decode layer."""
    torch = torch_cuda
    L = {nm: dev(torch, w) for nm, w in llama2_layer.items()}
    x = krk.synth_normal(4096, seed=311)
    xt = dev(torch, x).reshape(1, 4096)
    qkv = [torch.full((1, 4096), float("nan"), device="cuda") for _ in range(3)]
    fused, sf = be32.gemm_group(qkv, xt, [L["q"], L["k"], L["v"]], O.Q4_K, [4096] * 3, 4096, 1)
    assert fused and not sf
    o = torch.full((1, 4096), float("nan"), device="cuda")
    be32.gemm(o, qkv[0], L["o"], O.Q4_K, 4096, 4096, 1)
    ffn = torch.full((1, 11008), float("nan"), device="cuda")
    up = torch.empty((1, 11008), device="cuda")
    fused, sf = be32.gemm_group([ffn, up], xt, [L["gate"], L["up"]], O.Q4_K, [11008, 11008], 4096, 1,
                                silu=True)
    assert fused and sf
    y = torch.full((1, 4096), float("nan"), device="cuda")
    be32.gemm(y, ffn, L["down"], O.Q4_K, 4096, 11008, 1)
    be32.sync()
    W = llama2_layer
    for nm, t in zip("qkv", qkv):
        assert rel(host(t)[0], O.gemm(O.Q4_K, W[nm], x, 4096, 16)[0]) <= GEMV_TOL, nm
    # o and down take the device's own q and SiLU rows as their inputs, so
    # each stage is checked on exactly the activations it consumed
    qd = host(qkv[0])
    assert rel(host(o), O.gemm(O.Q4_K, W["o"], qd, 4096, 16)) <= GEMV_TOL
    g = O.gemm(O.Q4_K, W["gate"], x, 11008, 16)[0]
    u = O.gemm(O.Q4_K, W["up"], x, 11008, 16)[0]
    assert rel(host(ffn)[0], O.silu_mul(g, u)) <= GEMV_TOL
    assert rel(host(y), O.gemm(O.Q4_K, W["down"], host(ffn), 4096, 16)) <= GEMV_TOL


# ---------------------------------------------------------------- config 3 --
@pytest.fixture(scope="module")
def c3_weights(krk):
    return {"up": make_weights(krk, O.Q4_K, 14336, 4096, seed=320),
            "down": make_weights(krk, O.Q4_K, 4096, 14336, seed=321)}


def sample_rows(M, n=64):
    """64 rows spread over M: both ends, every tile row position mod 256."""
    r = np.unique(np.concatenate([[0, 1, M - 2, M - 1], np.linspace(0, M - 1, n - 4).astype(int)]))
    return r


@pytest.mark.parametrize("M", [512, 2048])
@pytest.mark.parametrize("name", ["up", "down"])
def test_config3_prefill_gemm(krk, torch_cuda, be16, c3_weights, name, M):
    torch = torch_cuda
    N, K = (14336, 4096) if name == "up" else (4096, 14336)
    w = c3_weights[name]
    x = krk.synth_normal(M * K, seed=330 + M).reshape(M, K).astype(np.float16)
    say("config 3", name, M, N, K)
    out = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    be16.gemm(out, dev(torch, x), dev(torch, w), O.Q4_K, N, K, M)
    be16.sync()
    got = host(out)
    assert np.isfinite(got).all()
    rows = sample_rows(M)
    ref = O.gemm(O.Q4_K, w, x[rows].astype(np.float32), N, nthreads=16)
    e = rel(got[rows].astype(np.float32), ref)
    say("  rel", e, "rows", len(rows))
    assert e <= GEMM_TOL
    # every row: the same rows' worth of error budget, row by row
    for i, r in enumerate(rows):
        assert rel(got[r].astype(np.float32), ref[i]) <= GEMM_TOL, r


# ---------------------------------------------------------------- config 4 --
def test_config4_q6_k_head(krk, torch_cuda, be32):
    torch = torch_cuda
    n_out, n_in = 128256, 4096
    w = make_weights(krk, O.Q6_K, n_out, n_in, seed=340)
    # prefill final-row-only: the head runs on the last row of a batch
    xb = krk.synth_normal(3 * n_in, seed=341).reshape(3, n_in)
    x = xb[-1]
    say("config 4 q6_k head")
    out = torch.full((1, n_out), float("nan"), dtype=torch.float32, device="cuda")
    xt = dev(torch, xb)
    be32.gemm(out, xt[2:3], dev(torch, w), O.Q6_K, n_out, n_in, 1)
    be32.sync()
    e = rel(host(out), O.gemm(O.Q6_K, w, x, n_out, nthreads=16))
    say("  rel", e)
    assert e <= GEMV_TOL


def test_config4_q8_0_head(krk, torch_cuda, be32, be16):
    """The Q8_0 head at M = 1 (GEMV, f32 tolerance), and with Q8-quantized
    activations on the int8 rung for a 16-row batch, the smallest the rung
    takes (rows <= 8 are GEMV rows on every path), bit-exact."""
    torch = torch_cuda
    n_out, n_in = 128256, 4096
    w = make_weights(krk, O.Q8_0, n_out, n_in, seed=342)
    wt = dev(torch, w)
    x = krk.synth_normal(16 * n_in, seed=343).reshape(16, n_in)
    say("config 4 q8_0 head")
    out = torch.full((1, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x[:1]), wt, O.Q8_0, n_out, n_in, 1)
    be32.sync()
    assert rel(host(out), O.gemm(O.Q8_0, w, x[:1], n_out, nthreads=16)) <= GEMV_TOL
    be32.set_gemm_path(krk.PATH_INT8)
    try:
        o4 = torch.full((16, n_out), float("nan"), dtype=torch.float32, device="cuda")
        be32.gemm(o4, dev(torch, x), wt, O.Q8_0, n_out, n_in, 16)
        be32.sync()
    finally:
        be32.set_gemm_path(krk.PATH_AUTO)
    ref = O.gemm_int8(O.Q8_0, w, x, n_out, nthreads=16)
    assert np.array_equal(host(o4).view(np.uint32), ref.view(np.uint32))


# ---------------------------------------------------------------- config 5 --
@pytest.fixture(scope="module")
def c5_layer(krk, torch_cuda):
    """The C5 banks as the config states them: Q4_K gate/up [1536, 4096] and
    down [4096, 1536] quantized from seeded N(0, 0.02) weights.  Eight
    distinct experts are generated (all 128 would take the host ~40 s) and
    the 128 banks are separate device copies of them."""
    torch = torch_cuda
    ne, n_embd, n_ff, distinct = 128, 4096, 1536, 8
    shapes = ((n_ff, n_embd), (n_ff, n_embd), (n_embd, n_ff))
    proto = [[krk.quantize(O.Q4_K, krk.synth_normal(o * i, seed=350 + 3 * d + m, std=0.02, nthreads=16), o, i, 16)
              for m, (o, i) in enumerate(shapes)] for d in range(distinct)]
    banks = {}
    entries = []
    keep = []
    for e in range(ne):
        ent = krk.MoeEntry()
        for m, (o, i) in enumerate(shapes):
            q = proto[e % distinct][m]
            banks[m, e] = q
            t = dev(torch, q)
            keep.append(t)
            ent.p[m] = t.data_ptr()
            ent.n_out[m], ent.n_in[m] = o, i
            ent.row_bytes[m] = krk.row_bytes(O.Q4_K, i)
            ent.type[m] = O.Q4_K
            ent.present[m] = 1
        entries.append(ent)
    table = dev(torch, np.frombuffer(krk.moe_table_bytes(entries), np.uint8).copy())
    return banks, table, keep


@pytest.mark.parametrize("n_tok", [1, 16])
def test_config5_moe_layer(krk, torch_cuda, be32, c5_layer, n_tok):
    """Router softmax, top-8 with normalization, and the expert dispatch, all
    on the device, against the oracle's routing and expert FFN."""
    torch = torch_cuda
    banks, table, _ = c5_layer
    ne, n_embd, n_ff, k = 128, 4096, 1536, 8
    logits = krk.synth_normal(n_tok * ne, seed=360 + n_tok).reshape(n_tok, ne)
    x = krk.synth_normal(n_tok * n_embd, seed=370 + n_tok).reshape(n_tok, n_embd)
    probs = torch.empty((n_tok, ne), dtype=torch.float32, device="cuda")
    ids = torch.empty((n_tok, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((n_tok, k), dtype=torch.float32, device="cuda")
    out = torch.full((n_tok, n_embd), float("nan"), dtype=torch.float32, device="cuda")
    say("config 5", n_tok)
    try:
        be32.router_softmax(probs, dev(torch, logits), n_tok, ne)
        be32.router_topk(probs, n_tok, ne, k, ids, wts, True, 1.0)
        be32.moe_dispatch(table, 0, ne, ids, wts, dev(torch, x), out, n_tok, n_embd, n_ff, k)
        be32.sync()
    finally:
        be32.moe_table_forget(table)
    # routing: the device softmax is within 2e-6 of the host's (expf
    # differs in the last bit), so the selected ids are the oracle's and the
    # weights agree to that rounding; the expert FFN is then checked on the
    # device's own ids and weights
    rid, rwt = O.router_topk(O.router_softmax(logits), k)
    assert np.array_equal(host(ids), rid)
    assert np.allclose(host(wts), rwt, rtol=4e-6, atol=0)
    rid, rwt = host(ids), host(wts)
    say("  experts", len(set(rid.reshape(-1).tolist())))
    # experts no token routes to are never read; the oracle gets the same
    # (unread) stand-in for them
    used = set(rid.reshape(-1).tolist())
    stand = banks[0, 0]
    g = [banks[0, e] if e in used else stand for e in range(ne)]
    u = [banks[1, e] if e in used else stand for e in range(ne)]
    d = [banks[2, e] if e in used else stand for e in range(ne)]
    ref = O.moe_ffn(x, g, u, d, O.Q4_K, rid, rwt, n_ff, nthreads=16)
    e = rel(host(out), ref)
    say("  rel", e)
    assert e <= GEMV_TOL


@pytest.mark.parametrize("path", ["mfma", "exact"])
def test_config5_moe_prefill_batch(krk, torch_cuda, be32, c5_layer, path):
    """A prefill-sized batch (512 tokens, every expert active, 32 pairs per
    expert on average) at the C5 shape.  Under the default gemm path it takes
    the grouped expert GEMM (f16 products, the MFMA GEMM bar); under
    KRK_PATH_EXACT the expert-major streaming runs (the GEMV bar).  Tokens
    are independent of one another, so the oracle checks a sample of 12 of
    them (first, last and ten spread between) on the device's routing."""
    torch = torch_cuda
    banks, table, _ = c5_layer
    ne, n_embd, n_ff, k, n_tok = 128, 4096, 1536, 8, 512
    logits = krk.synth_normal(n_tok * ne, seed=390).reshape(n_tok, ne)
    x = krk.synth_normal(n_tok * n_embd, seed=391).reshape(n_tok, n_embd)
    probs = torch.empty((n_tok, ne), dtype=torch.float32, device="cuda")
    ids = torch.empty((n_tok, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((n_tok, k), dtype=torch.float32, device="cuda")
    out = torch.full((n_tok, n_embd), float("nan"), dtype=torch.float32, device="cuda")
    say("config 5 prefill", path)
    be32.set_gemm_path(krk.PATH_EXACT if path == "exact" else krk.PATH_AUTO)
    try:
        be32.router_softmax(probs, dev(torch, logits), n_tok, ne)
        be32.router_topk(probs, n_tok, ne, k, ids, wts, True, 1.0)
        be32.moe_dispatch(table, 0, ne, ids, wts, dev(torch, x), out, n_tok, n_embd, n_ff, k)
        be32.sync()
    finally:
        be32.set_gemm_path(krk.PATH_AUTO)
        be32.moe_table_forget(table)
    rid, rwt = host(ids), host(wts)
    assert len(set(rid.reshape(-1).tolist())) == ne
    sel = np.unique(np.r_[0, n_tok - 1, np.linspace(1, n_tok - 2, 10).astype(int)])
    used = set(rid[sel].reshape(-1).tolist())
    stand = banks[0, 0]
    g = [banks[0, e] if e in used else stand for e in range(ne)]
    u = [banks[1, e] if e in used else stand for e in range(ne)]
    d = [banks[2, e] if e in used else stand for e in range(ne)]
    ref = O.moe_ffn(x[sel], g, u, d, O.Q4_K, rid[sel], rwt[sel], n_ff, nthreads=16)
    got = host(out)
    assert np.isfinite(got).all()
    e = rel(got[sel], ref)
    say("  rel", e)
    assert e <= (GEMM_TOL if path == "mfma" else GEMV_TOL)


@pytest.mark.parametrize("n_tok", [1, 16])
def test_config5_q4_k_m_layer(krk, torch_cuda, be32, c5_layer, n_tok):
    """The C5 shape with Q6_K down banks (the Q4_K_M layout): gate/up on the
    streaming kernel's routed modes for Q4_K, down on its Q6_K modes (one
    token: over the concatenated slots; several: expert-major runs), against
    the oracle on the device's routing (the GEMV bar)."""
    torch = torch_cuda
    banks, _, _ = c5_layer
    ne, n_embd, n_ff, k = 128, 4096, 1536, 8
    # Q6_K down banks quantized from N(0, 0.02): eight distinct, 128 copies
    d6 = [krk.quantize(O.Q6_K, krk.synth_normal(n_embd * n_ff, seed=380 + d, std=0.02, nthreads=16), n_embd,
                       n_ff, 16) for d in range(8)]
    down, entries, keep = {}, [], []
    for e in range(ne):
        ent = krk.MoeEntry()
        for m, (o, i) in enumerate(((n_ff, n_embd), (n_ff, n_embd), (n_embd, n_ff))):
            q = banks[m, e] if m < 2 else d6[e % 8]
            if m == 2:
                down[e] = q
            t = dev(torch, q)
            keep.append(t)
            dt = O.Q6_K if m == 2 else O.Q4_K
            ent.p[m] = t.data_ptr()
            ent.n_out[m], ent.n_in[m] = o, i
            ent.row_bytes[m] = krk.row_bytes(dt, i)
            ent.type[m] = dt
            ent.present[m] = 1
        entries.append(ent)
    table = dev(torch, np.frombuffer(krk.moe_table_bytes(entries), np.uint8).copy())
    logits = krk.synth_normal(n_tok * ne, seed=385 + n_tok).reshape(n_tok, ne)
    x = krk.synth_normal(n_tok * n_embd, seed=386 + n_tok).reshape(n_tok, n_embd)
    ids, wts = O.router_topk(O.router_softmax(logits), k)
    out = torch.full((n_tok, n_embd), float("nan"), dtype=torch.float32, device="cuda")
    say("config 5 q4_k_m", n_tok)
    try:
        be32.moe_dispatch(table, 0, ne, dev(torch, ids), dev(torch, wts), dev(torch, x), out, n_tok,
                          n_embd, n_ff, k)
        be32.sync()
    finally:
        be32.moe_table_forget(table)
    used = set(ids.reshape(-1).tolist())
    g = [banks[0, e] if e in used else banks[0, 0] for e in range(ne)]
    u = [banks[1, e] if e in used else banks[0, 0] for e in range(ne)]
    d = [down[e] if e in used else down[0] for e in range(ne)]
    ref = O.moe_ffn(x, g, u, d, (O.Q4_K, O.Q4_K, O.Q6_K), ids, wts, n_ff, nthreads=16)
    e = rel(host(out), ref)
    say("  rel", e)
    assert e <= GEMV_TOL
