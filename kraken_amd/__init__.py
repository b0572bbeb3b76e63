"""kraken_amd -- MI355X (gfx950) quantized weight-math backend.

Python mirror of Kraken's ``Backend`` hot-path operators
(include/krk/backend.hpp:337-1876 in the reference) over the C ABI in
include/krk_mi355x.h, implemented by the in-tree HIP library
``kraken_amd/libkrk_mi355x.so``.  Tensors are torch tensors on the GPU; torch
is only the allocator and stream provider here, every operator runs in the
library's own kernels.  There is no fallback: if the library or a GPU is
missing the operators raise.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkrk_mi355x.so")

# GGUF type ids (include/krk/quant.hpp:16-34) and the ABI's enums.
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS = 0, 1, 2, 8, 12, 13, 14, 20, 23
Q2_K, Q3_K, MXFP4 = 10, 11, 39
Q4_1, Q5_0, Q5_1 = 3, 6, 7
BF16 = 30
# served through the generic 32-value chunk path
Q8_1, Q8_K, TQ1_0, TQ2_0, NVFP4 = 9, 15, 34, 35, 40
ROCMFP4, ROCMFP4_FAST, Q6_0_ROCMFPX, Q3_0_ROCMFPX, Q2_0_ROCMFPX = 100, 101, 102, 104, 107
Q1_0, Q2_0, Q2_0_64, PQ2_0, PTQ1_0 = 41, 42, 48, 142, 143
CHUNK_FMTS = (Q8_1, Q8_K, TQ1_0, TQ2_0, NVFP4, ROCMFP4, ROCMFP4_FAST, Q6_0_ROCMFPX, Q3_0_ROCMFPX, Q2_0_ROCMFPX,
              Q1_0, Q2_0, Q2_0_64, PQ2_0, PTQ1_0)
ACT_F32, ACT_F16 = 0, 1
PATH_AUTO, PATH_EXACT, PATH_MFMA, PATH_INT8 = 0, 1, 2, 3
DTYPE_NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K",
               IQ4_NL: "IQ4_NL", IQ4_XS: "IQ4_XS", Q2_K: "Q2_K", Q3_K: "Q3_K", MXFP4: "MXFP4",
               Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1", BF16: "BF16", Q8_1: "Q8_1", Q8_K: "Q8_K",
               TQ1_0: "TQ1_0", TQ2_0: "TQ2_0", NVFP4: "NVFP4", ROCMFP4: "ROCMFP4",
               ROCMFP4_FAST: "ROCMFP4_FAST", Q6_0_ROCMFPX: "Q6_0_ROCMFPX", Q3_0_ROCMFPX: "Q3_0_ROCMFPX",
               Q2_0_ROCMFPX: "Q2_0_ROCMFPX", Q1_0: "Q1_0", Q2_0: "Q2_0", Q2_0_64: "Q2_0_64", PQ2_0: "PQ2_0",
               PTQ1_0: "PTQ1_0"}
BLOCK_VALUES = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, IQ4_NL: 32, IQ4_XS: 256,
                Q2_K: 256, Q3_K: 256, MXFP4: 32, Q4_1: 32, Q5_0: 32, Q5_1: 32, F16: 1, BF16: 1,
                Q8_1: 32, Q8_K: 256, TQ1_0: 256, TQ2_0: 256, NVFP4: 64, ROCMFP4: 32, ROCMFP4_FAST: 32,
                Q6_0_ROCMFPX: 32, Q3_0_ROCMFPX: 32, Q2_0_ROCMFPX: 32, Q1_0: 128, Q2_0: 128, Q2_0_64: 64,
                PQ2_0: 128, PTQ1_0: 128}
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ4_NL: 18, IQ4_XS: 136,
               Q2_K: 84, Q3_K: 110, MXFP4: 17, Q4_1: 20, Q5_0: 22, Q5_1: 24, F16: 2, BF16: 2,
               Q8_1: 36, Q8_K: 292, TQ1_0: 54, TQ2_0: 66, NVFP4: 36, ROCMFP4: 18, ROCMFP4_FAST: 17,
               Q6_0_ROCMFPX: 26, Q3_0_ROCMFPX: 14, Q2_0_ROCMFPX: 10, Q1_0: 18, Q2_0: 34, Q2_0_64: 18,
               PQ2_0: 34, PTQ1_0: 28}

_vp, _i64, _i32, _f32, _u64 = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_uint64
_P = C.POINTER

# name -> (restype, argtypes); the complete exported surface of the header.
SIGNATURES = {
    "krk_backend_create": (_i32, [_i32, _i32, _P(_vp)]),
    "krk_backend_destroy": (_i32, [_vp]),
    "krk_set_stream": (_i32, [_vp, _vp]),
    "krk_set_gemm_path": (_i32, [_vp, _i32]),
    "krk_act_type": (_i32, [_vp]),
    "krk_sync": (_i32, [_vp]),
    "krk_last_error": (C.c_char_p, [_vp]),
    "krk_status_string": (C.c_char_p, [_i32]),
    "krk_dtype_block_size": (_i32, [_i32]),
    "krk_dtype_block_bytes": (_i32, [_i32]),
    "krk_dtype_row_bytes": (_i64, [_i32, _i64]),
    "krk_dtype_row_aligned": (_i32, [_i32, _i64]),
    "krk_gemm": (_i32, [_vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64]),
    "krk_gemm_noalloc": (_i32, [_vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64]),
    "krk_gemm_noalloc_scratch_bytes": (C.c_size_t, []),
    "krk_gemm_k_ok": (_i32, [_vp, _i64]),
    "krk_gemm_accumulate": (_i32, [_vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp,
                                   _P(_i32)]),
    "krk_gemm_group": (_i32, [_vp, _P(_vp), _vp, _P(_vp), _i32, _P(_i64), _i64, _i32,
                              _i64, _i32, _P(_i32), _i32, _P(_i32), _P(_vp), _P(_i32)]),
    "krk_router_softmax_supported": (_i32, [_vp]),
    "krk_router_softmax": (_i32, [_vp, _vp, _vp, _i64, _i32]),
    "krk_router_topk_supported": (_i32, [_vp]),
    "krk_router_topk": (_i32, [_vp, _vp, _i64, _i32, _i32, _vp, _vp, _i32, _f32]),
    "krk_scan_accum_supported": (_i32, [_vp]),
    "krk_scan_accum": (_i32, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp, _vp]),
    "krk_moe_plan_build": (_i32, [_vp, _vp, _i64, _i32, _i32, _vp, _vp, _vp, _vp]),
    "krk_moe_dispatch_supported": (_i32, [_vp]),
    "krk_moe_table_forget": (_i32, [_vp, _vp]),
    "krk_moe_dispatch": (_i32, [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64,
                                _i64, _i32]),
    "krk_dequant_rows_f32": (_i32, [_vp, _vp, _vp, _i32, _i64, _i64]),
    "krk_dequant_rows_f16": (_i32, [_vp, _vp, _vp, _i32, _i64, _i64]),
    "krk_quantize_q8_rows": (_i32, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "krk_synth_normal": (None, [_vp, _i64, _u64, _f32, _f32, _i32]),
    "krk_quantize_weights": (_i32, [_i32, _vp, _i64, _i64, _vp, _i32]),
    # include/krk_gguf.h
    "krk_gguf_open": (_i32, [C.c_char_p, _P(_vp), C.c_char_p, C.c_size_t]),
    "krk_gguf_close": (None, [_vp]),
    "krk_gguf_version": (C.c_uint32, [_vp]),
    "krk_gguf_alignment": (_u64, [_vp]),
    "krk_gguf_data_offset": (_u64, [_vp]),
    "krk_gguf_tensor_count": (_i64, [_vp]),
    "krk_gguf_tensor": (_i32, [_vp, _i64, _vp]),
    "krk_gguf_find_tensor": (_i64, [_vp, C.c_char_p]),
    "krk_gguf_kv_count": (_i64, [_vp]),
    "krk_gguf_kv_key": (C.c_char_p, [_vp, _i64]),
    "krk_gguf_kv_type": (_i32, [_vp, _i64, _P(C.c_uint32), _P(C.c_uint32), _P(_u64)]),
    "krk_gguf_find_kv": (_i64, [_vp, C.c_char_p]),
    "krk_gguf_get_i64": (_i32, [_vp, C.c_char_p, _P(_i64)]),
    "krk_gguf_get_f64": (_i32, [_vp, C.c_char_p, _P(C.c_double)]),
    "krk_gguf_get_bool": (_i32, [_vp, C.c_char_p, _P(_i32)]),
    "krk_gguf_get_str": (_i32, [_vp, C.c_char_p, _P(C.c_char_p)]),
    "krk_gguf_array_i64": (_i32, [_vp, C.c_char_p, _u64, _P(_i64)]),
    "krk_gguf_array_f64": (_i32, [_vp, C.c_char_p, _u64, _P(C.c_double)]),
    "krk_gguf_array_str": (_i32, [_vp, C.c_char_p, _u64, _P(C.c_char_p)]),
    "krk_gguf_upload": (_i32, [_vp, _vp, _i64, _vp]),
}


class GgufTensorInfo(C.Structure):
    """krk_gguf_tensor_info (include/krk_gguf.h)."""
    _fields_ = [("name", C.c_char_p), ("type_id", C.c_uint32), ("dtype_known", C.c_int),
                ("n_dims", C.c_int), ("ne", C.c_uint64 * 4), ("offset", C.c_uint64),
                ("n_elements", C.c_int64), ("n_bytes", C.c_uint64), ("data", C.c_void_p)]


class KrkError(RuntimeError):
    pass


_lib = None


def lib():
    """The loaded HIP library; raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise KrkError(f"{LIB_PATH} is missing: run kraken_amd/build.py "
                           "(or __graft_entry__.build()) first")
        # torch ships its own copy of the HIP runtime (soname libamdhip64.so.7,
        # file name libamdhip64.so).  Loading torch first makes this library
        # bind to that same copy, so the process holds ONE runtime and torch's
        # streams and allocations are valid here; the other order would load
        # two runtimes side by side.
        import torch  # noqa: F401
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def row_bytes(wt: int, n: int) -> int:
    return int(lib().krk_dtype_row_bytes(wt, n))


# ------------------------------------------------------------ host helpers --
def synth_normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0,
                 nthreads: int = 8):
    """numpy f32[n] from the library's seeded generator."""
    import numpy as np
    v = np.empty(n, np.float32)
    lib().krk_synth_normal(v.ctypes.data, n, seed, mean, std, nthreads)
    return v


def quantize(wt: int, v, n_rows: int, n_in: int, nthreads: int = 8):
    """GGUF bytes (numpy uint8) of an f32 [n_rows, n_in] matrix."""
    import numpy as np
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
    assert v.size == n_rows * n_in
    out = np.empty(n_rows * row_bytes(wt, n_in), np.uint8)
    st = lib().krk_quantize_weights(wt, v.ctypes.data, n_rows, n_in, out.ctypes.data,
                                    nthreads)
    if st != 0:
        raise KrkError(lib().krk_status_string(st).decode())
    return out


# ------------------------------------------------------------------ backend --
def _ptr(t):
    return None if t is None else t.data_ptr()


class Backend:
    """The MI355X backend: the reference's Backend hot-path surface.

    ``act`` is the activation type (``ACT_F32`` to compare against the f32 CPU
    oracle, ``ACT_F16`` like the reference's GPU backend).  All tensors are
    torch CUDA tensors; results are asynchronous on ``stream`` (torch's
    current stream by default) until :meth:`sync`.
    """

    def __init__(self, device: int = 0, act: int = ACT_F32, stream=None):
        import torch
        if not torch.cuda.is_available():
            raise KrkError("no GPU visible: the MI355X backend has no CPU fallback")
        h = _vp()
        st = lib().krk_backend_create(device, act, C.byref(h))
        if st != 0:
            raise KrkError(f"krk_backend_create: {lib().krk_status_string(st).decode()}")
        self._h = h
        # bound now: module globals may already be gone when __del__ runs at exit
        self._destroy = lib().krk_backend_destroy
        self.device = device
        self.act = act
        self.set_stream(stream if stream is not None else torch.cuda.current_stream(device))

    # context
    def close(self):
        if getattr(self, "_h", None):
            self._destroy(self._h)
            self._h = None

    __del__ = close

    def _check(self, st: int, what: str):
        if st != 0:
            msg = lib().krk_last_error(self._h).decode()
            raise KrkError(f"{what}: {lib().krk_status_string(st).decode()}: {msg}")

    def set_stream(self, stream):
        self.stream = stream
        self._check(lib().krk_set_stream(self._h, stream.cuda_stream), "set_stream")

    def set_gemm_path(self, path: int):
        self._check(lib().krk_set_gemm_path(self._h, path), "set_gemm_path")

    def act_type(self) -> int:
        return int(lib().krk_act_type(self._h))

    def sync(self):
        self._check(lib().krk_sync(self._h), "sync")

    # hot operators (backend.hpp:859-1054)
    def gemm(self, out, x, w, wt: int, n_out: int, n_in: int, rows: int):
        self._check(lib().krk_gemm(self._h, _ptr(out), _ptr(x), _ptr(w), wt, n_out, n_in,
                                   rows), "gemm")

    def gemm_noalloc(self, out, x, w, wt: int, n_out: int, n_in: int, rows: int):
        """gemm with its scratch in the library's fixed per-device array
        (krk_gemm_noalloc): never allocates; KRK_ERR_NOMEM past its size."""
        self._check(lib().krk_gemm_noalloc(self._h, _ptr(out), _ptr(x), _ptr(w), wt, n_out, n_in,
                                           rows), "gemm_noalloc")

    def gemm_k_ok(self, k: int) -> bool:
        return bool(lib().krk_gemm_k_ok(self._h, k))

    def gemm_accumulate(self, dst, x, w, wt: int, n_out: int, n_in: int, rows: int,
                        rexp=None) -> bool:
        fused = _i32(0)
        self._check(lib().krk_gemm_accumulate(self._h, _ptr(dst), _ptr(x), _ptr(w), wt,
                                              n_out, n_in, rows, _ptr(rexp),
                                              C.byref(fused)), "gemm_accumulate")
        return bool(fused.value)

    def gemm_group(self, outs, x, ws, wt: int, n_outs, n_in: int, rows: int,
                   silu: bool = False, row_parallel_only: bool = False, wts=None,
                   xs=None):
        """Returns (fused, silu_fused)."""
        n = len(ws)
        arr_o = (_vp * n)(*[_ptr(o) for o in outs])
        arr_w = (_vp * n)(*[_ptr(w) for w in ws])
        arr_n = (_i64 * n)(*n_outs)
        arr_t = (_i32 * n)(*wts) if wts is not None else None
        arr_x = (_vp * n)(*[_ptr(t) for t in xs]) if xs is not None else None
        sf, fu = _i32(0), _i32(0)
        self._check(lib().krk_gemm_group(self._h, arr_o, _ptr(x), arr_w, wt, arr_n, n_in, n,
                                         rows, int(silu), C.byref(sf),
                                         int(row_parallel_only), arr_t, arr_x,
                                         C.byref(fu)), "gemm_group")
        return bool(fu.value), bool(sf.value)

    def router_softmax(self, probs, logits, n_rows: int, n_expert: int):
        self._check(lib().krk_router_softmax(self._h, _ptr(probs), _ptr(logits), n_rows,
                                             n_expert), "router_softmax")

    def router_topk(self, probs, n_rows: int, n_expert: int, k: int, ids, wts,
                    normalize: bool = True, scale: float = 1.0):
        self._check(lib().krk_router_topk(self._h, _ptr(probs), n_rows, n_expert, k,
                                          _ptr(ids), _ptr(wts), int(normalize), scale),
                    "router_topk")

    def scan_accum(self, probs, ids, n_rows: int, n_expert: int, k: int, layer: int, hits, mass):
        """Fold one layer's routing into the device histograms hits (u32) and
        mass (f32), both [n_layer, n_expert] (Backend::scan_accum)."""
        self._check(lib().krk_scan_accum(self._h, _ptr(probs), _ptr(ids), n_rows, n_expert, k, layer,
                                         _ptr(hits), _ptr(mass)), "scan_accum")

    def moe_plan_build(self, ids, n_rows: int, k: int, n_expert: int, off, rows, wt, wts=None):
        """The expert-major plan of the routed pairs (Backend::moe_plan_build)."""
        self._check(lib().krk_moe_plan_build(self._h, _ptr(ids), n_rows, k, n_expert, _ptr(off),
                                             _ptr(rows), _ptr(wt), _ptr(wts) if wts is not None else None),
                    "moe_plan_build")

    def moe_dispatch(self, table, layer: int, n_expert: int, ids, wts, xn, out,
                     n_tok: int, n_embd: int, n_ff: int, k: int):
        self._check(lib().krk_moe_dispatch(self._h, _ptr(table), layer, n_expert, _ptr(ids),
                                           _ptr(wts), _ptr(xn), _ptr(out), n_tok, n_embd,
                                           n_ff, k), "moe_dispatch")

    def moe_table_forget(self, table):
        """Drop the remembered validation of every layer of `table` (before
        the table is rewritten or freed)."""
        self._check(lib().krk_moe_table_forget(self._h, _ptr(table)), "moe_table_forget")

    # exactness surface
    def dequant_rows(self, out, w, wt: int, n_rows: int, n_in: int, f16: bool = False):
        fn = lib().krk_dequant_rows_f16 if f16 else lib().krk_dequant_rows_f32
        self._check(fn(self._h, _ptr(out), _ptr(w), wt, n_rows, n_in), "dequant_rows")

    def quantize_q8_rows(self, x, rows: int, n: int, xq, dx):
        self._check(lib().krk_quantize_q8_rows(self._h, _ptr(x), rows, n, _ptr(xq), _ptr(dx)),
                    "quantize_q8_rows")


# MoE device table: krk_moe_entry (include/krk_mi355x.h), the reference's
# MoeDispatchEntry layout (include/krk/moe_table.hpp:42-50).
class MoeEntry(C.Structure):
    _fields_ = [("p", _vp * 3), ("n_out", _i64 * 3), ("n_in", _i64 * 3),
                ("row_bytes", _i64 * 3), ("type", _i32 * 3), ("present", _i32 * 3),
                ("_pad", _i32)]


def moe_table_bytes(entries) -> bytes:
    """Pack a list of MoeEntry into the byte image the device table holds."""
    arr = (MoeEntry * len(entries))(*entries)
    return bytes(C.string_at(C.addressof(arr), C.sizeof(arr)))


# ------------------------------------------------------------------ GGUF --
class Gguf:
    """A memory-mapped GGUF file: krk::Gguf (include/krk/gguf.hpp:86-160) over
    include/krk_gguf.h.  ``tensors()`` gives the descriptors in file order,
    ``data(name)`` a zero-copy numpy view of a tensor's bytes (valid while the
    object lives), ``upload(backend, name, dst)`` copies them verbatim into a
    device tensor."""

    def __init__(self, path: str):
        h = _vp()
        err = C.create_string_buffer(512)
        st = lib().krk_gguf_open(os.fsencode(path), C.byref(h), err, 512)
        if st != 0:
            raise KrkError(f"gguf_open: {lib().krk_status_string(st).decode()}: "
                           f"{err.value.decode(errors='replace')}")
        self._h = h
        self._close = lib().krk_gguf_close

    def close(self):
        if getattr(self, "_h", None):
            self._close(self._h)
            self._h = None

    __del__ = close

    @property
    def version(self) -> int:
        return int(lib().krk_gguf_version(self._h))

    @property
    def alignment(self) -> int:
        return int(lib().krk_gguf_alignment(self._h))

    @property
    def data_offset(self) -> int:
        return int(lib().krk_gguf_data_offset(self._h))

    def tensor_count(self) -> int:
        return int(lib().krk_gguf_tensor_count(self._h))

    def tensor(self, i) -> GgufTensorInfo:
        if isinstance(i, str):
            j = int(lib().krk_gguf_find_tensor(self._h, i.encode()))
            if j < 0:
                raise KeyError(i)
            i = j
        t = GgufTensorInfo()
        if lib().krk_gguf_tensor(self._h, i, C.byref(t)) != 0:
            raise IndexError(i)
        return t

    def tensors(self):
        return [self.tensor(i) for i in range(self.tensor_count())]

    def data(self, name):
        """Zero-copy numpy uint8 view of a served-type tensor's bytes."""
        import numpy as np
        t = self.tensor(name)
        if not t.dtype_known:
            raise KrkError(f"tensor {t.name.decode()} has type {t.type_id}, not served")
        buf = (C.c_uint8 * t.n_bytes).from_address(t.data)
        return np.ctypeslib.as_array(buf)

    def keys(self):
        return [lib().krk_gguf_kv_key(self._h, i).decode(errors="replace")
                for i in range(int(lib().krk_gguf_kv_count(self._h)))]

    def kv_type(self, i: int):
        t, e, n = C.c_uint32(), C.c_uint32(), _u64()
        lib().krk_gguf_kv_type(self._h, i, C.byref(t), C.byref(e), C.byref(n))
        return t.value, e.value, n.value

    def get_i64(self, key: str, default: int = 0) -> int:
        v = _i64(default)
        lib().krk_gguf_get_i64(self._h, key.encode(), C.byref(v))
        return v.value

    def get_f64(self, key: str, default: float = 0.0) -> float:
        v = C.c_double(default)
        lib().krk_gguf_get_f64(self._h, key.encode(), C.byref(v))
        return v.value

    def get_bool(self, key: str, default: bool = False) -> bool:
        v = _i32(int(default))
        lib().krk_gguf_get_bool(self._h, key.encode(), C.byref(v))
        return bool(v.value)

    def get_str(self, key: str, default: str = "") -> str:
        v = C.c_char_p()
        if lib().krk_gguf_get_str(self._h, key.encode(), C.byref(v)) != 0:
            return default
        return v.value.decode(errors="replace")

    def upload(self, backend: "Backend", name, dst) -> None:
        """Copy tensor ``name`` verbatim into device tensor ``dst``."""
        t = self.tensor(name)
        if dst.numel() * dst.element_size() < t.n_bytes:
            raise KrkError("gguf upload: destination smaller than the tensor")
        j = int(lib().krk_gguf_find_tensor(self._h, t.name))
        backend._check(lib().krk_gguf_upload(backend._h, self._h, j, _ptr(dst)), "gguf_upload")
