"""Shared test setup: the `gpu` marker, repo-root imports, seeded inputs."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def krk():
    import kraken_amd
    kraken_amd.lib()  # raises if the library was not built
    return kraken_amd


def rand_blocks(rng, dt, n_blocks):
    """Random block bytes with finite f16 scale fields (every code pattern)."""
    import oracle
    if dt in (oracle.F16, oracle.BF16):   # finite values of a weight's scale
        v = (rng.standard_normal(n_blocks) * 0.02).astype(np.float32)
        if dt == oracle.F16:
            return v.astype(np.float16).view(np.uint8).copy()
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).copy()
    bb = {oracle.Q4_0: 18, oracle.Q8_0: 34, oracle.Q4_K: 144, oracle.Q5_K: 176, oracle.Q6_K: 210,
          oracle.IQ4_NL: 18, oracle.IQ4_XS: 136, oracle.Q2_K: 84, oracle.Q3_K: 110,
          oracle.MXFP4: 17, oracle.Q4_1: 20, oracle.Q5_0: 22, oracle.Q5_1: 24,
          oracle.Q8_1: 36, oracle.Q8_K: 292, oracle.TQ1_0: 54, oracle.TQ2_0: 66, oracle.NVFP4: 36,
          oracle.ROCMFP4: 18, oracle.ROCMFP4_FAST: 17, oracle.Q6_0_ROCMFPX: 26, oracle.Q3_0_ROCMFPX: 14,
          oracle.Q2_0_ROCMFPX: 10, oracle.Q1_0: 18, oracle.Q2_0: 34, oracle.Q2_0_64: 18,
          oracle.PQ2_0: 34, oracle.PTQ1_0: 28}[dt]
    w = rng.integers(0, 256, size=(n_blocks, bb), dtype=np.uint8)

    def setf16(off, scale):
        v = (rng.standard_normal(n_blocks) * scale).astype(np.float16).view(np.uint16)
        w[:, off] = v & 0xFF
        w[:, off + 1] = v >> 8

    if dt in (oracle.Q4_0, oracle.Q8_0, oracle.IQ4_NL, oracle.IQ4_XS, oracle.Q5_0):
        setf16(0, 0.01)
    elif dt in (oracle.Q4_K, oracle.Q5_K, oracle.Q4_1, oracle.Q5_1):
        setf16(0, 0.01)
        setf16(2, 0.01)
    elif dt == oracle.Q2_K:
        setf16(80, 0.01)
        setf16(82, 0.01)
    elif dt == oracle.Q3_K:
        setf16(108, 0.01)
    elif dt == oracle.Q8_1:
        setf16(0, 0.01)
        setf16(2, 0.01)
    elif dt == oracle.Q8_K:
        d = (rng.standard_normal(n_blocks) * 0.01).astype(np.float32).view(np.uint8).reshape(n_blocks, 4)
        w[:, 0:4] = d
    elif dt == oracle.TQ1_0:
        setf16(52, 0.01)
    elif dt == oracle.PTQ1_0:
        setf16(26, 0.01)
    elif dt in (oracle.Q1_0, oracle.Q2_0, oracle.Q2_0_64, oracle.PQ2_0):
        setf16(0, 0.01)
    elif dt == oracle.TQ2_0:
        setf16(64, 0.01)
    elif dt in oracle.CHUNK_FMTS:
        pass   # UE4M3 scale bytes: every byte value is finite
    elif dt == oracle.MXFP4:
        # exponent bytes near 2^-7 scale (finite products and sums); every
        # exponent byte is covered by the dequant tests of their own
        w[:, 0] = rng.integers(110, 128, size=n_blocks)
    else:
        setf16(208, 0.01)
    return w.reshape(-1)


@pytest.fixture
def rng():
    return np.random.default_rng(20261201)


# GPU fixtures: one backend per activation type per test module
@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    return torch


@pytest.fixture(scope="module")
def be32(krk, torch_cuda):
    b = krk.Backend(0, krk.ACT_F32)
    yield b
    b.close()


@pytest.fixture(scope="module")
def be16(krk, torch_cuda):
    b = krk.Backend(0, krk.ACT_F16)
    yield b
    b.close()
