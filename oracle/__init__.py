"""ctypes view of the CPU oracle (oracle/liboracle.so) and, when it was built,
of the reference's own host quant code (oracle/_ref/libkrk_ref.so).

TEST INFRASTRUCTURE. Only tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg import this package, and only as the checker. The product
(kraken_amd/) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libkrk_ref.so")

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS = 0, 1, 2, 8, 12, 13, 14, 20, 23
Q2_K, Q3_K, MXFP4 = 10, 11, 39
Q4_1, Q5_0, Q5_1 = 3, 6, 7
BF16 = 30
# formats served through the generic 32-value chunk path
Q8_1, Q8_K, TQ1_0, TQ2_0, NVFP4 = 9, 15, 34, 35, 40
ROCMFP4, ROCMFP4_FAST, Q6_0_ROCMFPX, Q3_0_ROCMFPX, Q2_0_ROCMFPX = 100, 101, 102, 104, 107
Q1_0, Q2_0, Q2_0_64, PQ2_0, PTQ1_0 = 41, 42, 48, 142, 143
CHUNK_FMTS = (Q8_1, Q8_K, TQ1_0, TQ2_0, NVFP4, ROCMFP4, ROCMFP4_FAST, Q6_0_ROCMFPX, Q3_0_ROCMFPX, Q2_0_ROCMFPX,
              Q1_0, Q2_0, Q2_0_64, PQ2_0, PTQ1_0)

_vp, _i64, _i32, _f32, _u16 = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_uint16


def build(force: bool = False) -> None:
    """Compile liboracle.so (and oracle/_ref when the reference tree exists)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.check_call(["make", "-s", "-C", HERE, "-B" if force else "all"])


def _p(a):
    return None if a is None else a.ctypes.data_as(_vp)


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    sig = {
        "orc_fp16_to_fp32": (_f32, [_u16]),
        "orc_fp32_to_fp16": (_u16, [_f32]),
        "orc_block_size": (_i32, [_i32]),
        "orc_block_bytes": (_i32, [_i32]),
        "orc_row_bytes": (_i64, [_i32, _i64]),
        "orc_dequant_row": (None, [_i32, _vp, _vp, _i64]),
        "orc_dequant_row_f16": (None, [_i32, _vp, _vp, _i64]),
        "orc_vec_dot": (_f32, [_i32, _vp, _vp, _i64]),
        "orc_gemm": (None, [_vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32]),
        "orc_quantize_q8_row": (None, [_vp, _i64, _vp, _vp]),
        "orc_dot_q8_0_q8": (_f32, [_vp, _vp, _vp, _i64]),
        "orc_gemm_q8_0_q8": (None, [_vp, _vp, _vp, _i64, _i64, _i64, _i32]),
        "orc_gemm_int8": (None, [_i32, _vp, _vp, _vp, _i64, _i64, _i64, _i32]),
        "orc_dot_kq_q8": (_f32, [_i32, _vp, _vp, _vp, _i64]),
        "orc_silu_mul": (None, [_vp, _vp, _vp, _i64]),
        "orc_router_softmax": (None, [_vp, _vp, _i64, _i32]),
        "orc_router_topk": (None, [_vp, _i64, _i32, _i32, _vp, _vp, _i32, _f32]),
        "orc_moe_ffn": (None, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp,
                               _vp, _i64, _i64, _i64, _i32, _i32, _i32]),
        "orc_moe_ffn_f16": (None, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp,
                                   _vp, _i64, _i64, _i64, _i32, _i32, _i32]),
        "orc_quantize_q8_0_weights": (None, [_vp, _i64, _vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


_ref = None


def ref():
    """The reference's own quant code, or None when oracle/_ref was not built."""
    global _ref
    if _ref is None and ref_available():
        r = C.CDLL(REF_PATH)
        sig = {
            "ref_row_bytes": (_i64, [_i32, _i64]),
            "ref_block_size": (_i32, [_i32]),
            "ref_block_bytes": (_i32, [_i32]),
            "ref_dequant_row": (None, [_i32, _vp, _vp, _i64]),
            "ref_dequant_row_f16": (None, [_i32, _vp, _vp, _i64]),
            "ref_vec_dot": (_f32, [_i32, _vp, _vp, _i64]),
            "ref_quantize_q8_row": (None, [_vp, _i64, _vp, _vp]),
            "ref_dot_q8_0_q8_scalar": (_f32, [_vp, _vp, _vp, _i64]),
            "ref_dot_q4_K_q8": (_f32, [_vp, _vp, _vp, _i64]),
            "ref_dot_q6_K_q8": (_f32, [_vp, _vp, _vp, _i64]),
            "ref_fp16_to_fp32": (_f32, [_u16]),
            "ref_fp32_to_fp16": (_u16, [_f32]),
            "ref_gemv_strict": (None, [_i32, _vp, _i64, _vp, _i64, _i64, _vp, _i32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(r, name)
            fn.restype, fn.argtypes = res, args
        _ref = r
    return _ref


def ref_gemv(dt: int, w: np.ndarray, x: np.ndarray, n_out: int, nthreads: int = 8) -> np.ndarray:
    """The reference's own strict vec_dot per output row (oracle/_ref),
    rows over nthreads threads; None when oracle/_ref was not built."""
    r = ref()
    if r is None:
        return None
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    rb = int(r.ref_row_bytes(dt, x.size))
    assert w.size >= n_out * rb
    out = np.empty(n_out, np.float32)
    r.ref_gemv_strict(dt, _p(w), rb, _p(x), n_out, x.size, _p(out), nthreads)
    return out


# ---------------------------------------------------------------- numpy API --
def row_bytes(dt: int, n: int) -> int:
    return int(lib().orc_row_bytes(dt, n))


def dequant(dt: int, w: np.ndarray, n_rows: int, n_in: int) -> np.ndarray:
    """f32 [n_rows, n_in] from raw row-major blocks."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    rb = row_bytes(dt, n_in)
    assert w.size >= n_rows * rb
    out = np.empty((n_rows, n_in), np.float32)
    for r in range(n_rows):
        lib().orc_dequant_row(dt, _p(w[r * rb:]), _p(out[r]), n_in)
    return out


def dequant_f16(dt: int, w: np.ndarray, n_rows: int, n_in: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    rb = row_bytes(dt, n_in)
    out = np.empty((n_rows, n_in), np.uint16)
    for r in range(n_rows):
        lib().orc_dequant_row_f16(dt, _p(w[r * rb:]), _p(out[r]), n_in)
    return out


def vec_dot(dt: int, wrow: np.ndarray, x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, dtype=np.float32)
    wrow = np.ascontiguousarray(wrow, dtype=np.uint8)
    return float(lib().orc_vec_dot(dt, _p(wrow), _p(x), x.size))


def gemm(dt: int, w: np.ndarray, x: np.ndarray, n_out: int, nthreads: int = 8
         ) -> np.ndarray:
    """out[rows, n_out] = x[rows, n_in] . W^T, the strict scalar oracle."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    rows, n_in = x.shape
    w = np.ascontiguousarray(w, dtype=np.uint8)
    assert w.size >= n_out * row_bytes(dt, n_in)
    out = np.empty((rows, n_out), np.float32)
    lib().orc_gemm(_p(out), _p(x), _p(w), dt, n_out, n_in, rows, nthreads)
    return out


def quantize_q8_row(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    xq = np.empty(x.size, np.int8)
    dx = np.empty(x.size // 32, np.float32)
    lib().orc_quantize_q8_row(_p(x), x.size, _p(xq), _p(dx))
    return xq, dx


def dot_q8_0_q8(wrow: np.ndarray, xq: np.ndarray, dx: np.ndarray) -> float:
    return float(lib().orc_dot_q8_0_q8(_p(np.ascontiguousarray(wrow)), _p(xq),
                                       _p(dx), xq.size))


def gemm_q8_0_q8(w: np.ndarray, x: np.ndarray, n_out: int, nthreads: int = 8
                 ) -> np.ndarray:
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    rows, n_in = x.shape
    out = np.empty((rows, n_out), np.float32)
    lib().orc_gemm_q8_0_q8(_p(out), _p(x), _p(np.ascontiguousarray(w)), n_out,
                           n_in, rows, nthreads)
    return out


def gemm_int8(dt: int, w: np.ndarray, x: np.ndarray, n_out: int, nthreads: int = 8
              ) -> np.ndarray:
    """The int8 rung for any of its weight types (Q8_0, Q4_K, Q5_K, Q6_K)."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    rows, n_in = x.shape
    out = np.empty((rows, n_out), np.float32)
    lib().orc_gemm_int8(dt, _p(out), _p(x), _p(np.ascontiguousarray(w)), n_out, n_in, rows, nthreads)
    return out


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    out = np.empty_like(g)
    lib().orc_silu_mul(_p(out), _p(g), _p(u), g.size)
    return out


def router_softmax(logits: np.ndarray) -> np.ndarray:
    logits = np.ascontiguousarray(np.atleast_2d(logits), dtype=np.float32)
    out = np.empty_like(logits)
    lib().orc_router_softmax(_p(out), _p(logits), logits.shape[0], logits.shape[1])
    return out


def router_topk(probs: np.ndarray, k: int, normalize: bool = True,
                scale: float = 1.0):
    probs = np.ascontiguousarray(np.atleast_2d(probs), dtype=np.float32)
    n, ne = probs.shape
    ids = np.empty((n, k), np.int32)
    wts = np.empty((n, k), np.float32)
    lib().orc_router_topk(_p(probs), n, ne, k, _p(ids), _p(wts), int(normalize),
                          scale)
    return ids, wts


def moe_plan_build(ids, n_expert: int, wts=None, cursor_experts: int | None = None):
    """Backend::moe_plan_build's plan (router.hpp:241-275): off [n_expert + 1]
    prefix counts of the routed pairs per expert; rows / wt [n * k] in
    expert-major order, each expert's pairs in (row, slot) order, row = pair
    index // k, wt = the pair's weight (0 without wts).  Entries past
    off[n_expert] are left as -1 / NaN here (the reference leaves them
    unwritten).  cursor_experts: the reference's fill keeps cursors for
    experts below 256 only (router.hpp:263-268); pass 256 to restate that,
    None to fill every expert.  Pure integer work: numpy loops."""
    ids = np.ascontiguousarray(np.atleast_2d(ids), dtype=np.int32)
    n, k = ids.shape
    flat = ids.reshape(-1)
    off = np.zeros(n_expert + 1, np.int32)
    for e in flat:
        if 0 <= e < n_expert:
            off[e + 1] += 1
    off = np.cumsum(off).astype(np.int32)
    rows = np.full(n * k, -1, np.int32)
    wt = np.full(n * k, np.nan, np.float32)
    cursor = off[:-1].copy()
    w = None if wts is None else np.ascontiguousarray(wts, dtype=np.float32).reshape(-1)
    for i, e in enumerate(flat):
        if not (0 <= e < n_expert) or (cursor_experts is not None and e >= cursor_experts):
            continue
        at = cursor[e]
        cursor[e] += 1
        rows[at] = i // k
        wt[at] = 0.0 if w is None else w[i]
    return off, rows, wt


def scan_accum(probs, ids, n_expert: int, layer: int, hits, mass):
    """Backend::scan_accum (router.hpp:222-239), in place on host copies:
    hits[layer * n_expert + id] += 1 per routed pair; mass[layer * n_expert + e]
    += the f32 sum over rows, in row order, of probs[row, e] (skipped when
    that sum is 0)."""
    probs = np.ascontiguousarray(np.atleast_2d(probs), dtype=np.float32)
    base = layer * n_expert
    s = np.zeros(n_expert, np.float32)
    for t in range(probs.shape[0]):
        s = (s + probs[t]).astype(np.float32)
    for e in range(n_expert):
        if s[e] != 0.0:
            mass[base + e] = np.float32(mass[base + e] + s[e])
    for e in np.ascontiguousarray(ids, dtype=np.int32).reshape(-1):
        if 0 <= e < n_expert:
            hits[base + e] += 1


def moe_ffn(x, gate, up, down, wt, ids, wts, n_ff, nthreads: int = 8):
    """x f32 [n_tok, n_embd]; gate/up/down: lists of per-expert uint8 arrays;
    wt one weight type or a (gate, up, down) triple."""
    wg, wu, wd = (wt, wt, wt) if isinstance(wt, int) else wt
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    n_tok, n_embd = x.shape
    ne = len(gate)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    wts = np.ascontiguousarray(wts, dtype=np.float32)
    k = ids.shape[-1]
    keep = [np.ascontiguousarray(a) for a in (*gate, *up, *down)]
    arr = (_vp * ne)
    g = arr(*[a.ctypes.data for a in keep[:ne]])
    u = arr(*[a.ctypes.data for a in keep[ne:2 * ne]])
    d = arr(*[a.ctypes.data for a in keep[2 * ne:]])
    out = np.empty((n_tok, n_embd), np.float32)
    lib().orc_moe_ffn(_p(out), _p(x), C.cast(g, _vp), C.cast(u, _vp),
                      C.cast(d, _vp), wg, wu, wd, _p(ids), _p(wts), n_tok,
                      n_embd, n_ff, ne, k, nthreads)
    return out


def moe_ffn_f16(x, gate, up, down, wt, ids, wts, n_ff, nthreads: int = 8):
    """The reference GPU backend's f16 expert FFN (orc_moe_ffn_f16); x holds
    f16 values; returns float16 [n_tok, n_embd]."""
    wg, wu, wd = (wt, wt, wt) if isinstance(wt, int) else wt
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    n_tok, n_embd = x.shape
    ne = len(gate)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    wts = np.ascontiguousarray(wts, dtype=np.float32)
    k = ids.shape[-1]
    keep = [np.ascontiguousarray(a) for a in (*gate, *up, *down)]
    arr = (_vp * ne)
    g = arr(*[a.ctypes.data for a in keep[:ne]])
    u = arr(*[a.ctypes.data for a in keep[ne:2 * ne]])
    d = arr(*[a.ctypes.data for a in keep[2 * ne:]])
    out = np.empty((n_tok, n_embd), np.uint16)
    lib().orc_moe_ffn_f16(_p(out), _p(x), C.cast(g, _vp), C.cast(u, _vp), C.cast(d, _vp), wg, wu,
                          wd, _p(ids), _p(wts), n_tok, n_embd, n_ff, ne, k, nthreads)
    return out.view(np.float16)


def quantize_q8_0_weights(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
    out = np.empty(v.size // 32 * 34, np.uint8)
    lib().orc_quantize_q8_0_weights(_p(v), v.size, _p(out))
    return out
