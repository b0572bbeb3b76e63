"""CPU-side checks of the product library: it loads, it exports every entry
point include/*.h declares, its host-side geometry and synthetic
input generators are right, and it refuses to run without a GPU."""
import os
import re
import struct
import subprocess
import sys

import numpy as np
import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def declared_functions():
    names = set()
    for h in HEADERS:
        txt = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(krk_\w+)\s*\(", txt))
    return sorted(names)


def test_header_declares_the_operator_surface():
    names = declared_functions()
    for need in ("krk_gemm", "krk_gemm_accumulate", "krk_gemm_group", "krk_gemm_k_ok",
                 "krk_moe_dispatch", "krk_router_softmax", "krk_router_topk",
                 "krk_backend_create"):
        assert need in names


def test_library_exports_every_declared_symbol(krk):
    names = declared_functions()
    out = subprocess.run(["nm", "-D", "--defined-only", krk.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(l.split()[-1] for l in out.splitlines() if l.strip())
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    assert set(names) == set(krk.SIGNATURES), set(names) ^ set(krk.SIGNATURES)


def test_geometry_matches_oracle(krk):
    L = krk.lib()
    for dt in (O.Q4_0, O.Q8_0, O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K, O.Q6_K, O.IQ4_NL, O.IQ4_XS, O.MXFP4,
               O.Q4_1, O.Q5_0, O.Q5_1, O.F16, O.BF16):
        assert L.krk_dtype_block_size(dt) == O.lib().orc_block_size(dt)
        assert L.krk_dtype_block_bytes(dt) == O.lib().orc_block_bytes(dt)
        for n in (32, 256, 4096, 11008, 14336):
            if n % L.krk_dtype_block_size(dt) == 0:
                assert L.krk_dtype_row_bytes(dt, n) == O.row_bytes(dt, n)
    assert not L.krk_dtype_row_aligned(O.Q4_K, 100)
    assert L.krk_dtype_row_aligned(O.F16, 100)
    assert L.krk_dtype_block_size(99) == 0
    assert L.krk_gemm_k_ok(None, 4096) and not L.krk_gemm_k_ok(None, 100)
    assert not L.krk_gemm_k_ok(None, 0)


def test_synth_normal_is_seeded_and_thread_independent(krk):
    a = krk.synth_normal(100003, seed=42, nthreads=1)
    b = krk.synth_normal(100003, seed=42, nthreads=7)
    c = krk.synth_normal(100003, seed=43, nthreads=7)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 0.02 and abs(a.std() - 1.0) < 0.02
    s = krk.synth_normal(1000, seed=1, mean=0.0, std=0.02)
    assert abs(s.std() - 0.02) < 0.003


def test_q8_0_quantizer_matches_fixture_generator(krk):
    """The product's Q8_0 quantizer is the reference fixture generator's rule
    (tools/make_bench_gguf.py:191-202), checked against the oracle's
    independent restatement (itself pinned to Python's struct/round)."""
    v = krk.synth_normal(64 * 2048, seed=7, std=0.02)
    v[:32] = 0
    got = krk.quantize(O.Q8_0, v, 64, 2048)
    assert np.array_equal(got, O.quantize_q8_0_weights(v))


def test_q4_0_quantizer_matches_fixture_generator(krk):
    v = krk.synth_normal(32 * 40, seed=8, std=0.02)
    got = krk.quantize(O.Q4_0, v, 1, v.size)
    want = bytearray()
    for b in range(0, v.size, 32):  # tools/make_bench_gguf.py:205-218
        blk = [float(t) for t in v[b:b + 32]]
        amax = max((-min(blk), max(blk)))
        d = amax / -8.0 if amax else 0.0
        id_ = 1.0 / d if d else 0.0
        q = [max(0, min(15, int(round(t * id_ + 8)))) for t in blk]
        want += struct.pack("<e", d)
        for k in range(16):
            want += struct.pack("<B", (q[k] & 0xF) | ((q[k + 16] & 0xF) << 4))
    assert bytes(got) == bytes(want)


@pytest.mark.parametrize("dt,bound", [(O.Q4_K, 0.12), (O.Q5_K, 0.06), (O.Q6_K, 0.03), (O.Q8_0, 0.01),
                                      (O.Q4_0, 0.12), (O.IQ4_NL, 0.12), (O.IQ4_XS, 0.12),
                                      (O.Q2_K, 0.45), (O.Q3_K, 0.25), (O.MXFP4, 0.2),
                                      (O.Q4_1, 0.12), (O.Q5_0, 0.06), (O.Q5_1, 0.06),
                                      (O.F16, 1e-3), (O.BF16, 4e-3)])
def test_weight_quantizers_round_trip(krk, dt, bound):
    """The library's own K-quant quantizers (the reference has none): the
    bytes they write decode, through the pinned oracle, to the input within
    the format's resolution."""
    n_rows, n_in = 16, 4096
    v = krk.synth_normal(n_rows * n_in, seed=dt, std=0.02).reshape(n_rows, n_in)
    q = krk.quantize(dt, v, n_rows, n_in)
    back = O.dequant(dt, q, n_rows, n_in)
    rel = np.linalg.norm(back - v) / np.linalg.norm(v)
    assert rel < bound, rel


def test_quantizer_rejects_bad_shapes(krk):
    v = np.zeros(300, np.float32)
    out = np.zeros(1000, np.uint8)
    L = krk.lib()
    assert L.krk_quantize_weights(O.Q4_K, v.ctypes.data, 1, 300, out.ctypes.data, 1) == -3
    assert L.krk_quantize_weights(99, v.ctypes.data, 1, 256, out.ctypes.data, 1) == -2


def test_no_gpu_no_fallback(krk):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(krk.KrkError):
        krk.Backend()


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_dma_wait_check_catches_a_short_count():
    """kraken_amd/build.py's check of the grouped expert GEMM's DMA publish
    waits (run on every build): a vmcnt(N) before a barrier is accepted only
    after at least N vector loads issued after the last DMA."""
    from kraken_amd.build import check_dma_waits
    ok = "\n".join(["_ZN3krk15moe_gemm_kernelX: ; @k", "\tglobal_load_lds_dwordx4 v[0:1], off",
                    "\tglobal_load_dwordx4 v[2:5], v[6:7], off", "\tglobal_load_dwordx4 v[8:11], v[6:7], off",
                    "\ts_waitcnt vmcnt(2)", "\ts_barrier", "\ts_endpgm"])
    assert check_dma_waits(ok) == (1, [])
    short = ok.replace("vmcnt(2)", "vmcnt(3)")
    sites, bad = check_dma_waits(short)
    assert sites == 1 and bad and bad[0][2:] == (2, 3)
