"""krk_gemm_noalloc against krk_gemm, through the C ABI.

The allocation-free entry point runs the same kernels with its scratch in a
fixed per-device array, so its outputs must equal krk_gemm's bit for bit:
GEMV rows, the f16 MFMA GEMM with split-K partials, the int8 rung with its
activation codes.  Two calls in a row, the second smaller, show the array
keeps no state that a later call depends on; a shape whose scratch exceeds
the array is refused before any launch; and a fresh handle's free device
memory does not move across the calls (krk_gemm would grow a workspace)."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from test_gpu_parity import dev, host, make_weights, say

pytestmark = pytest.mark.gpu


def free_bytes():
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(0), C.c_size_t(0)
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


@pytest.mark.parametrize("path,dt,shapes", [
    ("auto", O.Q4_K, [(512, 4096, 14336), (64, 4096, 4096)]),     # split-K 8 (64 MiB of partials), then 4
    ("auto", O.Q6_K, [(300, 2048, 8192), (24, 512, 4096)]),
    ("auto", O.Q4_K, [(512, 14336, 4096), (300, 10277, 2048)]),    # two splits summed in the GEMM
    ("auto", O.Q4_K, [(1, 14336, 4096), (3, 1000, 2048)]),         # GEMV rows
    ("int8", O.Q8_0, [(256, 2048, 4096), (40, 300, 1024)]),
])
def test_noalloc_equals_gemm(krk, torch_cuda, path, dt, shapes):
    torch = torch_cuda
    be = krk.Backend(0, krk.ACT_F16)
    ref_be = krk.Backend(0, krk.ACT_F16)
    try:
        if path == "int8":
            be.set_gemm_path(krk.PATH_INT8)
            ref_be.set_gemm_path(krk.PATH_INT8)
        for i, (M, N, K) in enumerate(shapes):
            say("noalloc", path, dt, M, N, K)
            w = dev(torch, make_weights(krk, dt, N, K, seed=500 + i))
            x = dev(torch, krk.synth_normal(M * K, seed=510 + i).reshape(M, K).astype(np.float16))
            want = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
            got = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
            ref_be.gemm(want, x, w, dt, N, K, M)
            ref_be.sync()
            torch.cuda.synchronize()
            f0 = free_bytes()
            be.gemm_noalloc(got, x, w, dt, N, K, M)
            be.sync()
            assert free_bytes() == f0
            assert np.array_equal(host(got).view(np.uint16), host(want).view(np.uint16)), (M, N, K)
    finally:
        be.close()
        ref_be.close()


def test_noalloc_refuses_past_its_scratch(krk, torch_cuda):
    torch = torch_cuda
    cap = int(krk.lib().krk_gemm_noalloc_scratch_bytes())
    assert cap == 64 << 20
    be = krk.Backend(0, krk.ACT_F16)
    try:
        be.set_gemm_path(krk.PATH_INT8)
        # int8 codes of 8192 x 8192 activations: 128 MiB > 64 MiB
        M, N, K = 8192, 64, 8192
        w = dev(torch, make_weights(krk, O.Q8_0, N, K, seed=520))
        x = torch.zeros((M, K), dtype=torch.float16, device="cuda")
        out = torch.full((M, N), 7.0, dtype=torch.float16, device="cuda")
        with pytest.raises(krk.KrkError, match="NOMEM|scratch"):
            be.gemm_noalloc(out, x, w, O.Q8_0, N, K, M)
        be.sync()
        assert bool((out == 7.0).all())
    finally:
        be.close()
