"""The f16 GEMM probe (krk_probe_gemm) computes the product it is timed as.

The bench reports a plain f16 GEMM beside the prefill GEMM as the ceiling
dense f16 matrix-core work reaches on this part; that figure means something
only if the probe is a correct GEMM.  Checked against torch's f32 product of
the same f16 operands, at shapes with partial tiles in M and N and the bench's
own shape, to the north-star GEMM bar (2e-3 relative Frobenius; the f16
output rounding alone is ~3e-4).  loads = 0 (operands staged once) is a
timing skeleton and only has to run.
"""
import pytest

from test_gpu_parity import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K", [(300, 520, 96), (256, 256, 32), (40, 1000, 4096), (2048, 14336, 4096)])
def test_probe_gemm_is_a_gemm(krk, torch_cuda, be16, M, N, K):
    torch = torch_cuda
    say("probe_gemm", M, N, K)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(M + N + K)
    x = torch.randn((M, K), dtype=torch.float16, device="cuda", generator=gen)
    w = torch.randn((N, K), dtype=torch.float16, device="cuda", generator=gen)
    out = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    be16.probe_gemm(x, w, out, M, N, K, True)
    be16.sync()
    ref = x.float() @ w.float().t()
    err = float(torch.linalg.norm(out.float() - ref) / torch.linalg.norm(ref))
    assert err <= 2e-3, err
    be16.probe_gemm(x, w, out, M, N, K, False)
    be16.sync()


def test_probe_gemm_rejects_bad_shapes(krk, torch_cuda, be16):
    torch = torch_cuda
    x = torch.zeros((64, 48), dtype=torch.float16, device="cuda")
    out = torch.zeros((64, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(krk.KrkError):
        be16.probe_gemm(x, x, out, 64, 64, 48, True)   # K not a multiple of 32
