"""The grouped expert GEMM (prefill-sized MoE batches under the default gemm
path) against the CPU oracle's expert FFN (orc_moe_ffn, f32 throughout).

The kernel rounds the activations, the decoded weights and the gate/up
output to f16 and accumulates in f32, as the dense MFMA GEMM does, so it is
held to the MFMA GEMM bar (2e-3 relative Frobenius).  Cases cover the three
item heights (32, 64 and 128 pairs: 8, 38 and 260 mean pairs per expert),
experts with several items, dropped slots, a Q4_K_M-style layer (Q4_K
gate/up, Q6_K down) and each bank type the kernel takes.  Below 32 tokens
and under KRK_PATH_EXACT the same layers keep the GEMV bar
(test_gpu_parity.py)."""
import numpy as np
import pytest

import oracle as O
from test_gpu_parity import GEMM_TOL, GEMV_TOL, build_moe, dev, host, make_weights, rel, say

pytestmark = pytest.mark.gpu


def run(krk, torch, be, dt, ne, n_embd, n_ff, k, n_tok, seed, drop=False):
    mats, table, keep = build_moe(krk, torch, dt, ne, n_embd, n_ff, seed=seed)
    logits = krk.synth_normal(n_tok * ne, seed=seed + 1).reshape(n_tok, ne)
    ids, wts = O.router_topk(O.router_softmax(logits), k)
    if drop:
        ids[0, 1] = -1
        ids[n_tok - 1, k - 1] = -1
    x = krk.synth_normal(n_tok * n_embd, seed=seed + 2).reshape(n_tok, n_embd)
    out = torch.full((n_tok, n_embd), float("nan"), dtype=torch.float32, device="cuda")
    be.moe_dispatch(table, 0, ne, dev(torch, ids), dev(torch, wts), dev(torch, x), out, n_tok,
                    n_embd, n_ff, k)
    be.sync()
    ref = O.moe_ffn(x, [mats[0, e] for e in range(ne)], [mats[1, e] for e in range(ne)],
                    [mats[2, e] for e in range(ne)], dt, ids, wts, n_ff, nthreads=16)
    got = host(out)
    assert np.isfinite(got).all()
    return rel(got, ref)


@pytest.mark.parametrize("n_tok,k,drop", [(32, 2, False), (100, 3, True), (260, 8, True)])
def test_moe_gemm_q4_k(krk, torch_cuda, be32, n_tok, k, drop):
    say("moe gemm q4_k", n_tok, k, drop)
    e = run(krk, torch_cuda, be32, O.Q4_K, 8, 512, 768, k, n_tok, seed=2100, drop=drop)
    say("  rel", e)
    assert e <= GEMM_TOL


@pytest.mark.parametrize("dt", [(O.Q4_K, O.Q4_K, O.Q6_K), O.Q5_K, O.Q6_K, O.Q8_0, O.Q4_0, O.MXFP4])
def test_moe_gemm_types(krk, torch_cuda, be32, dt):
    say("moe gemm types", dt)
    e = run(krk, torch_cuda, be32, dt, 6, 768, 1024, 4, 90, seed=2200, drop=True)
    say("  rel", e)
    assert e <= GEMM_TOL


def test_moe_gemm_exact_path_keeps_gemv_bar(krk, torch_cuda, be32):
    """The same batch under KRK_PATH_EXACT: the expert-major GEMV runs."""
    be32.set_gemm_path(krk.PATH_EXACT)
    try:
        e = run(krk, torch_cuda, be32, O.Q4_K, 8, 512, 768, 3, 100, seed=2100, drop=True)
    finally:
        be32.set_gemm_path(krk.PATH_AUTO)
    assert e <= GEMV_TOL


def test_moe_gemm_repeat_smaller(krk, torch_cuda, be32):
    """Two calls in a row, the second smaller (fewer items than the first
    left in the plan's scratch): each against its own oracle."""
    e1 = run(krk, torch_cuda, be32, O.Q4_K, 8, 512, 768, 8, 200, seed=2300)
    e2 = run(krk, torch_cuda, be32, O.Q4_K, 8, 512, 768, 2, 40, seed=2400)
    assert e1 <= GEMM_TOL and e2 <= GEMM_TOL


@pytest.mark.parametrize("rows", [9, 16, 33, 64, 100, 128])
@pytest.mark.parametrize("dt", [O.Q4_K, O.Q6_K, O.Q8_0, O.Q5_K, O.Q4_0, O.MXFP4])
@pytest.mark.parametrize("n_in", [1024, 4096])
def test_dense_streaming_gemm(krk, torch_cuda, be32, be16, rows, dt, n_in):
    """Dense GEMMs of 9..128 rows take the grouped kernel's dense mode (items
    of 32 or 64 rows, K split over whole blocks, f32 partials summed in a
    fixed order): f32 and f16 activations against the oracle, MFMA bar."""
    torch = torch_cuda
    n_out = 520   # a partial 256-row tile
    w = make_weights(krk, dt, n_out, n_in, seed=2500 + rows)
    x = krk.synth_normal(rows * n_in, seed=2600 + rows).reshape(rows, n_in)
    ref = O.gemm(dt, w, x, n_out)
    say("dense streaming gemm", dt, rows, n_in)
    out = torch.full((rows, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), dt, n_out, n_in, rows)
    be32.sync()
    assert rel(host(out), ref) <= GEMM_TOL
    x16 = x.astype(np.float16)
    out16 = torch.full((rows, n_out), float("nan"), dtype=torch.float16, device="cuda")
    be16.gemm(out16, dev(torch, x16), dev(torch, w), dt, n_out, n_in, rows)
    be16.sync()
    assert rel(host(out16).astype(np.float32), O.gemm(dt, w, x16.astype(np.float32), n_out)) <= GEMM_TOL


@pytest.mark.parametrize("rows,n_out", [(9, 1001), (17, 1001), (33, 333)])
def test_dense_streaming_gemm_odd_outputs(krk, torch_cuda, be32, be16, rows, n_out):
    """Split-K partials of an M N that is not a multiple of four (every slice
    after the first starts off 16-byte alignment), and an output that starts
    2 bytes off alignment: the fixed-order reduce sums them value by value."""
    torch = torch_cuda
    n_in = 4096
    w = make_weights(krk, O.Q4_K, n_out, n_in, seed=2700 + rows)
    x = krk.synth_normal(rows * n_in, seed=2800 + rows).reshape(rows, n_in)
    say("dense streaming gemm, odd outputs", rows, n_out)
    out = torch.full((rows, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), O.Q4_K, n_out, n_in, rows)
    be32.sync()
    assert rel(host(out), O.gemm(O.Q4_K, w, x, n_out)) <= GEMM_TOL
    x16 = x.astype(np.float16)
    buf = torch.full((rows * n_out + 1,), float("nan"), dtype=torch.float16, device="cuda")
    out16 = buf[1:].view(rows, n_out)   # 2 bytes past the allocation's alignment
    be16.gemm(out16, dev(torch, x16), dev(torch, w), O.Q4_K, n_out, n_in, rows)
    be16.sync()
    assert rel(host(out16).astype(np.float32), O.gemm(O.Q4_K, w, x16.astype(np.float32), n_out)) <= GEMM_TOL
