"""GPU parity of the formats served through the generic chunk path (Q8_1,
Q8_K, TQ1_0, TQ2_0, NVFP4, ROCmFP4, ROCmFP4_FAST and the three ROCmFPX
formats, Q1_0, Q2_0, Q2_0_64, PQ2_0, PTQ1_0) against the CPU oracle, whose decoders are pinned bit for bit
against the reference build and its golden vectors (test_oracle.py).

Every kernel reads these blocks through dequant_chunk alone (byte loads, any
alignment): dequant must be bit-exact, the GEMV rows 1..8 within 1e-5, the
f16-staged MFMA GEMM within 2e-3 Frobenius, and MoE dispatch over banks of
these types within 1e-5.  Weights are random valid blocks (every code
pattern; f16 / f32 scale fields finite, UE4M3 scale bytes all finite by
construction)."""
import numpy as np
import pytest

import oracle as O
from conftest import rand_blocks
from test_gpu_parity import GEMM_TOL, GEMV_TOL, _TABLES, dev, host, rel, say

pytestmark = pytest.mark.gpu

CHUNK = list(O.CHUNK_FMTS)


def weights(dt, n_out, n_in, seed):
    bs = O.lib().orc_block_size(dt)
    return rand_blocks(np.random.default_rng(seed), dt, n_out * n_in // bs)


@pytest.mark.parametrize("dt", CHUNK)
def test_chunk_dequant_bit_exact(torch_cuda, be32, dt):
    torch = torch_cuda
    n_rows, n_in = 37, 1024
    w = weights(dt, n_rows, n_in, 10 + dt)
    say("dequant chunk fmt", dt)
    out = torch.empty((n_rows, n_in), dtype=torch.float32, device="cuda")
    be32.dequant_rows(out, dev(torch, w), dt, n_rows, n_in)
    be32.sync()
    ref = O.dequant(dt, w, n_rows, n_in)
    assert np.array_equal(host(out).view(np.uint32), ref.view(np.uint32))
    out16 = torch.empty((n_rows, n_in), dtype=torch.float16, device="cuda")
    be32.dequant_rows(out16, dev(torch, w), dt, n_rows, n_in, f16=True)
    be32.sync()
    assert np.array_equal(host(out16).view(np.uint16), ref.astype(np.float16).view(np.uint16))


def test_ue4m3_every_byte(torch_cuda, be32):
    """Every UE4M3 scale byte (0x00 and 0x7F are zero, bit 7 is ignored) with
    every ROCmFP4_FAST code, bit for bit against the oracle."""
    torch = torch_cuda
    blk = np.zeros((256, 17), np.uint8)
    blk[:, :16] = [(k & 15) | ((15 - k) << 4) for k in range(16)]
    blk[:, 16] = np.arange(256)
    w = blk.reshape(-1)
    out = torch.empty((256, 32), dtype=torch.float32, device="cuda")
    be32.dequant_rows(out, dev(torch, w), O.ROCMFP4_FAST, 256, 32)
    be32.sync()
    ref = O.dequant(O.ROCMFP4_FAST, w, 256, 32)
    assert np.array_equal(host(out).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dt", CHUNK)
@pytest.mark.parametrize("rows", [1, 3, 8])
def test_chunk_gemv_parity(torch_cuda, be32, dt, rows):
    torch = torch_cuda
    n_out, n_in = 300, 2048
    w = weights(dt, n_out, n_in, 100 + dt)
    x = np.random.default_rng(rows).standard_normal((rows, n_in)).astype(np.float32)
    say("gemv chunk fmt", dt, rows)
    out = torch.full((rows, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), dt, n_out, n_in, rows)
    be32.sync()
    assert rel(host(out), O.gemm(dt, w, x, n_out)) <= GEMV_TOL


@pytest.mark.parametrize("dt", CHUNK)
def test_chunk_gemv_f16_activations(torch_cuda, be16, dt):
    torch = torch_cuda
    n_out, n_in = 200, 1024
    w = weights(dt, n_out, n_in, 200 + dt)
    # activations scaled so that products of the largest UE4M3 scales stay
    # inside f16's range at the output
    x = (np.random.default_rng(5).standard_normal(n_in) * 0.01).astype(np.float16)
    out = torch.empty((1, n_out), dtype=torch.float16, device="cuda")
    be16.gemm(out, dev(torch, x), dev(torch, w), dt, n_out, n_in, 1)
    be16.sync()
    # only the f16 store rounds: 2^-11 relative per element
    assert rel(host(out).astype(np.float32), O.gemm(dt, w, x.astype(np.float32), n_out)) <= 6e-4


@pytest.mark.parametrize("dt", CHUNK)
@pytest.mark.parametrize("M,N,K", [(40, 300, 1024), (300, 520, 2048)])
def test_chunk_gemm_mfma(torch_cuda, be16, dt, M, N, K):
    torch = torch_cuda
    w = weights(dt, N, K, 300 + dt)
    x = (np.random.default_rng(M).standard_normal((M, K)) * 0.01).astype(np.float16)
    say("gemm chunk fmt", dt, M, N, K)
    out = torch.empty((M, N), dtype=torch.float16, device="cuda")
    be16.gemm(out, dev(torch, x), dev(torch, w), dt, N, K, M)
    be16.sync()
    assert rel(host(out).astype(np.float32), O.gemm(dt, w, x.astype(np.float32), N)) <= GEMM_TOL


@pytest.mark.parametrize("dt", [O.Q8_K, O.TQ2_0, O.NVFP4, O.Q3_0_ROCMFPX])
@pytest.mark.parametrize("n_tok", [1, 5])
def test_chunk_moe_dispatch(krk, torch_cuda, be32, dt, n_tok):
    torch = torch_cuda
    ne, n_embd, n_ff, k = 8, 512, 768, 3
    mats, entries, keep = {}, [], []
    for e in range(ne):
        ent = krk.MoeEntry()
        for m, (o, i) in enumerate(((n_ff, n_embd), (n_ff, n_embd), (n_embd, n_ff))):
            q = weights(dt, o, i, 1000 + 3 * e + m)
            mats[m, e] = q
            t = dev(torch, q)
            keep.append(t)
            ent.p[m] = t.data_ptr()
            ent.n_out[m], ent.n_in[m] = o, i
            ent.row_bytes[m] = krk.row_bytes(dt, i)
            ent.type[m] = dt
            ent.present[m] = 1
        entries.append(ent)
    table = dev(torch, np.frombuffer(krk.moe_table_bytes(entries), np.uint8).copy())
    _TABLES.append(table)
    rng = np.random.default_rng(n_tok)
    logits = rng.standard_normal((n_tok, ne)).astype(np.float32)
    ids, wts = O.router_topk(O.router_softmax(logits), k)
    x = rng.standard_normal((n_tok, n_embd)).astype(np.float32) * 0.01
    say("moe chunk fmt", dt, n_tok)
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device="cuda")
    be32.moe_dispatch(table, 0, ne, dev(torch, ids), dev(torch, wts), dev(torch, x), out, n_tok,
                      n_embd, n_ff, k)
    be32.sync()
    ref = O.moe_ffn(x, [mats[0, e] for e in range(ne)], [mats[1, e] for e in range(ne)],
                    [mats[2, e] for e in range(ne)], dt, ids, wts, n_ff)
    assert rel(host(out), ref) <= GEMV_TOL


@pytest.mark.parametrize("dt", [O.ROCMFP4_FAST, O.Q3_0_ROCMFPX, O.TQ1_0])
def test_chunk_gemv_odd_address(torch_cuda, be32, dt):
    """Byte loads only: a weight matrix starting at an odd address (the
    odd-sized blocks of these formats put rows there anyway)."""
    torch = torch_cuda
    n_out, n_in = 64, 1024
    w = weights(dt, n_out, n_in, 400 + dt)
    buf = torch.zeros(w.size + 1, dtype=torch.uint8, device="cuda")
    buf[1:] = dev(torch, w)
    x = np.random.default_rng(9).standard_normal((2, n_in)).astype(np.float32)
    out = torch.empty((2, n_out), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), buf[1:], dt, n_out, n_in, 2)
    be32.sync()
    assert rel(host(out), O.gemm(dt, w, x, n_out)) <= GEMV_TOL
