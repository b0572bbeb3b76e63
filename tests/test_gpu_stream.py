"""GPU parity of the one-row Q4_K / Q6_K / Q4_0 / Q8_0 GEMV that loads each tile's weights
into registers up front (gemv_stream.hip), against the CPU oracle.

The kernel takes Q4_K, Q6_K, Q4_0 and Q8_0 launches with one activation row (plain,
residual and gate/up segments), so these cases walk its shape rules: K slices of two
to four blocks per wave with a ragged last slice, one to sixteen waves, tile
heights 16..32 with partial last tiles, several segments per launch, f32
and f16 activations, and the digit split's edge activations.  Bars: 1e-5
relative for f32 outputs (north_star); f16 outputs within their rounding.
"""
import numpy as np
import pytest

import oracle as O
from test_gpu_parity import GEMV_TOL, dev, digit_edge_x, host, make_weights, rel, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt", [O.Q4_K, O.Q6_K, O.Q4_0, O.Q8_0])
@pytest.mark.parametrize("n_out,n_in", [(1, 256), (17, 512), (300, 2304), (4096, 4096), (14336, 4096),
                                        (11008, 4096), (4096, 11008), (77, 14336), (1000, 16384),
                                        (33, 8192)])
def test_stream_shapes(krk, torch_cuda, be32, dt, n_out, n_in):
    torch = torch_cuda
    w = make_weights(krk, dt, n_out, n_in, seed=n_out + n_in)
    x = digit_edge_x(n_in, seed=n_in) if n_in % 1024 == 0 else krk.synth_normal(n_in, seed=n_in)
    say("stream", dt, n_out, n_in)
    out = torch.full((1, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), dt, n_out, n_in, 1)
    be32.sync()
    e = rel(host(out), O.gemm(dt, w, x, n_out, nthreads=16))
    say("  rel", e)
    assert e <= GEMV_TOL


@pytest.mark.parametrize("dt", [O.Q4_K, O.Q6_K, O.Q4_0, O.Q8_0])
@pytest.mark.parametrize("n_in", [4096, 11008])
def test_stream_f16(krk, torch_cuda, be16, dt, n_in):
    torch = torch_cuda
    n_out = 1234
    w = make_weights(krk, dt, n_out, n_in, seed=5 + n_in)
    x = krk.synth_normal(n_in, seed=6).astype(np.float16)
    out = torch.full((1, n_out), float("nan"), dtype=torch.float16, device="cuda")
    be16.gemm(out, dev(torch, x), dev(torch, w), dt, n_out, n_in, 1)
    be16.sync()
    ref = O.gemm(dt, w, x.astype(np.float32), n_out)[0]
    got = host(out)[0].astype(np.float32)
    # the f32 result (1e-5 relative over the output) rounded once to f16:
    # the output's f16 rounding adds at most 2^-11 relative
    assert rel(got, ref) <= 2.0 ** -11 + GEMV_TOL


@pytest.mark.parametrize("dt", [O.Q4_K, O.Q6_K, O.Q4_0, O.Q8_0])
def test_stream_groups(krk, torch_cuda, be32, be16, dt):
    """Three plain segments of different heights in one launch; a gate/up
    pair with the SiLU epilogue; the residual epilogue with rexp in f16."""
    torch = torch_cuda
    n_in = 4096
    shapes = [100, 4096, 33]
    ws = [make_weights(krk, dt, n, n_in, seed=70 + i) for i, n in enumerate(shapes)]
    x = krk.synth_normal(n_in, seed=74)
    outs = [torch.full((1, n), float("nan"), dtype=torch.float32, device="cuda") for n in shapes]
    fused, sf = be32.gemm_group(outs, dev(torch, x), [dev(torch, w) for w in ws], dt, shapes, n_in, 1)
    be32.sync()
    assert fused and not sf
    for o, w, n in zip(outs, ws, shapes):
        assert rel(host(o)[0], O.gemm(dt, w, x, n)[0]) <= GEMV_TOL
    n_ff = 1000
    g, u = make_weights(krk, dt, n_ff, n_in, 75), make_weights(krk, dt, n_ff, n_in, 76)
    o0 = torch.full((1, n_ff), float("nan"), dtype=torch.float32, device="cuda")
    o1 = torch.empty((1, n_ff), dtype=torch.float32, device="cuda")
    fused, sf = be32.gemm_group([o0, o1], dev(torch, x), [dev(torch, g), dev(torch, u)], dt,
                                [n_ff, n_ff], n_in, 1, silu=True)
    be32.sync()
    assert fused and sf
    want = O.silu_mul(O.gemm(dt, g, x, n_ff)[0], O.gemm(dt, u, x, n_ff)[0])
    assert rel(host(o0)[0], want) <= GEMV_TOL
    # residual in f16: the product rounded to f16, scaled by 2^-rexp, added
    # in f32 and saturated (gemm.hpp:96-108)
    n_out = 500
    w = make_weights(krk, dt, n_out, n_in, seed=77)
    base = krk.synth_normal(n_out, seed=78).astype(np.float16)
    dst = dev(torch, base.reshape(1, -1))
    rexp = dev(torch, np.array([1], np.int32))
    xh = x.astype(np.float16)
    assert be16.gemm_accumulate(dst, dev(torch, xh), dev(torch, w), dt, n_out, n_in, 1, rexp)
    be16.sync()
    prod = O.gemm(dt, w, xh.astype(np.float32), n_out)[0]
    want = base.astype(np.float32) + prod.astype(np.float16).astype(np.float32) * 0.5
    assert rel(host(dst)[0].astype(np.float32), want) <= 1e-3


@pytest.mark.parametrize("rows", [2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("n_out,n_in", [(17, 512), (300, 2304), (14336, 4096), (4096, 11008), (77, 14336)])
def test_stream_rows(krk, torch_cuda, be32, be16, rows, n_out, n_in):
    """Dense Q4_K launches of 2..8 activation rows on the streaming kernel
    (five and more on two-block slices; wider ones go to the digit kernel):
    one digit table per row, every weight group multiplied against each
    row; f32 rows at the 1e-5 bar, f16 rows within their rounding."""
    torch = torch_cuda
    w = make_weights(krk, O.Q4_K, n_out, n_in, seed=900 + rows)
    x = krk.synth_normal(rows * n_in, seed=901 + n_in).reshape(rows, n_in)
    say("stream rows", rows, n_out, n_in)
    out = torch.full((rows, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), O.Q4_K, n_out, n_in, rows)
    be32.sync()
    ref = O.gemm(O.Q4_K, w, x, n_out, nthreads=16)
    for r in range(rows):
        assert rel(host(out)[r], ref[r]) <= GEMV_TOL, r
    xh = x.astype(np.float16)
    out16 = torch.full((rows, n_out), float("nan"), dtype=torch.float16, device="cuda")
    be16.gemm(out16, dev(torch, xh), dev(torch, w), O.Q4_K, n_out, n_in, rows)
    be16.sync()
    ref16 = O.gemm(O.Q4_K, w, xh.astype(np.float32), n_out, nthreads=16)
    for r in range(rows):
        assert rel(host(out16)[r].astype(np.float32), ref16[r]) <= 2.0 ** -11 + GEMV_TOL, r


def test_stream_q4_k_vocab_head(krk, torch_cuda, be32):
    """A vocabulary-sized Q4_K matrix (128256 x 4096, one row) streams in many
    rounds of load-transpose tiles: every row against the oracle at 1e-5."""
    torch = torch_cuda
    n_out, n_in, rep = 128256, 4096, 16
    part = make_weights(krk, O.Q4_K, n_out // rep, n_in, seed=77)
    w = np.tile(part, rep)
    x = krk.synth_normal(n_in, seed=78)
    say("stream q4_k head", n_out, n_in)
    out = torch.full((1, n_out), float("nan"), dtype=torch.float32, device="cuda")
    be32.gemm(out, dev(torch, x), dev(torch, w), O.Q4_K, n_out, n_in, 1)
    be32.sync()
    ref = O.gemm(O.Q4_K, part, x, n_out // rep, nthreads=16)[0]
    got = host(out)[0]
    assert rel(got, np.tile(ref, rep)) <= GEMV_TOL
