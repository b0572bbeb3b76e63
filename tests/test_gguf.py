"""The GGUF reader (include/krk_gguf.h, kraken_amd/csrc/gguf.cpp).

CPU: against the reference's own reader (krk::Gguf, src/gguf.cpp, built in
place into oracle/_ref) on the reference's three GGUF checkpoints; on files
written here from the specification (every metadata type, a non-default
alignment, a type id the library does not serve); and its refusals.
GPU: real Q8_0 and IQ4_NL blocks of the reference checkpoints (tests/golden fixture),
written into a GGUF, read, uploaded verbatim and decoded on the device
bit-for-bit against the oracle."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import oracle as O
from gguf_writer import (ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64,
                         encode_kv, write_gguf)

REF_DIR = "/root/reference"
REF_FILES = ["TinyLLama-v0.Q8_0.gguf", "tinystories-gpt-0.1-3m.Q2_K.gguf",
             "tiny-llama3-test-Q3_K_M.gguf"]
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gguf_q8_0_blocks.npz")
SERVED = {0, 1, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 20, 23, 30, 39}


def _ref_reader():
    ref = O.ref()
    if ref is None or not os.path.isdir(REF_DIR):
        pytest.skip("reference tree or oracle/_ref not present")
    ref.ref_gguf_open.restype = C.c_void_p
    ref.ref_gguf_open.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
    for n in ("ref_gguf_close",):
        getattr(ref, n).argtypes = [C.c_void_p]
    for n, r in (("ref_gguf_tensor_count", C.c_int64), ("ref_gguf_kv_count", C.c_int64),
                 ("ref_gguf_alignment", C.c_uint64), ("ref_gguf_data_offset", C.c_uint64),
                 ("ref_gguf_version", C.c_uint32)):
        getattr(ref, n).restype = r
        getattr(ref, n).argtypes = [C.c_void_p]
    ref.ref_gguf_tensor.argtypes = [C.c_void_p, C.c_int64, C.c_char_p, C.c_size_t] + [C.c_void_p] * 7
    ref.ref_gguf_kv.argtypes = [C.c_void_p, C.c_int64, C.c_char_p, C.c_size_t] + [C.c_void_p] * 5 + \
        [C.c_char_p, C.c_size_t]
    return ref


@pytest.mark.parametrize("fname", REF_FILES)
def test_reader_matches_reference_reader(krk, fname):
    ref = _ref_reader()
    path = os.path.join(REF_DIR, fname)
    g = krk.Gguf(path)
    err = C.create_string_buffer(256)
    r = ref.ref_gguf_open(path.encode(), err, 256)
    assert r, err.value
    try:
        assert g.version == ref.ref_gguf_version(r)
        assert g.alignment == ref.ref_gguf_alignment(r)
        assert g.data_offset == ref.ref_gguf_data_offset(r)
        n = ref.ref_gguf_tensor_count(r)
        assert g.tensor_count() == n
        name = C.create_string_buffer(256)
        tid, known, nd = C.c_uint32(), C.c_int(), C.c_int()
        ne = (C.c_uint64 * 4)()
        off, nel, nb = C.c_uint64(), C.c_int64(), C.c_uint64()
        for i in range(n):
            ref.ref_gguf_tensor(r, i, name, 256, C.byref(tid), C.byref(known), C.byref(nd), ne,
                                C.byref(off), C.byref(nel), C.byref(nb))
            t = g.tensor(i)
            assert t.name == name.value
            assert (t.type_id, t.n_dims, t.offset, t.n_elements) == (tid.value, nd.value, off.value, nel.value)
            assert list(t.ne) == list(ne)
            # types this library serves are sized as the reference sizes them;
            # the others are reported unknown (the reference knows them)
            if tid.value in SERVED:
                assert t.dtype_known and t.n_bytes == nb.value
            else:
                assert not t.dtype_known and t.n_bytes == 0
        keys = g.keys()
        assert len(keys) == ref.ref_gguf_kv_count(r)
        key, s = C.create_string_buffer(512), C.create_string_buffer(4096)
        ty, el, cnt = C.c_uint32(), C.c_uint32(), C.c_uint64()
        ai, af = C.c_int64(), C.c_double()
        for i, k in enumerate(keys):
            ref.ref_gguf_kv(r, i, key, 512, C.byref(ty), C.byref(el), C.byref(cnt), C.byref(ai),
                            C.byref(af), s, 4096)
            assert k.encode() == key.value
            t, e, c = g.kv_type(i)
            assert t == ty.value and c == cnt.value, k
            if t == ARRAY:
                assert e == el.value, k
            elif t == STRING:
                assert g.get_str(k) == s.value.decode(errors="replace"), k
            else:
                assert g.get_i64(k) == ai.value and g.get_f64(k) == af.value, k
    finally:
        ref.ref_gguf_close(r)


def test_reader_reads_every_metadata_type(krk, tmp_path):
    rng = np.random.default_rng(5)
    q8 = bytes(rng.integers(0, 256, 2 * 34 * 3, dtype=np.uint8))
    q4k = bytes(rng.integers(0, 256, 144 * 2, dtype=np.uint8))
    f32 = np.arange(5, dtype=np.float32).tobytes()
    unknown = bytes(range(50))   # type 24 (I8), not served
    kvs = [("general.architecture", STRING, "llama"), ("general.alignment", U32, 64),
           ("a.u8", U8, 250), ("a.i8", I8, -5), ("a.u16", U16, 65000), ("a.i16", I16, -300),
           ("a.i32", I32, -70000), ("a.f32", F32, 1.5), ("a.bool", BOOL, 1), ("a.u64", U64, 2 ** 40),
           ("a.i64", I64, -(2 ** 40)), ("a.f64", F64, -2.25),
           ("a.arr_i32", ARRAY, [1, -2, 3], I32), ("a.arr_f32", ARRAY, [0.5, 0.25], F32),
           ("a.arr_str", ARRAY, ["x", "yz"], STRING), ("a.arr_u64", ARRAY, [7, 2 ** 33], U64)]
    tensors = [("w.q8", 8, [64, 3], q8), ("w.q4k", 12, [256, 2], q4k), ("v.f32", 0, [5], f32),
               ("u.i8", 24, [50], unknown)]
    path = str(tmp_path / "m.gguf")
    data_off = write_gguf(path, kvs, tensors, alignment=64)
    g = krk.Gguf(path)
    assert g.version == 3 and g.alignment == 64 and g.data_offset == data_off
    assert g.keys() == [k[0] for k in kvs]
    assert g.get_str("general.architecture") == "llama"
    assert g.get_i64("a.u8") == 250 and g.get_i64("a.i8") == -5 and g.get_i64("a.u16") == 65000
    assert g.get_i64("a.i16") == -300 and g.get_i64("a.i32") == -70000 and g.get_i64("a.u64") == 2 ** 40
    assert g.get_i64("a.i64") == -(2 ** 40) and g.get_f64("a.f32") == 1.5 and g.get_f64("a.f64") == -2.25
    assert g.get_i64("a.f32") == 1 and g.get_bool("a.bool") and g.get_str("absent", "d") == "d"
    assert g.get_i64("absent", 7) == 7
    L, h = krk.lib(), g._h
    v, d, sp = C.c_int64(), C.c_double(), C.c_char_p()
    assert L.krk_gguf_array_i64(h, b"a.arr_i32", 1, C.byref(v)) == 0 and v.value == -2
    assert L.krk_gguf_array_i64(h, b"a.arr_u64", 1, C.byref(v)) == 0 and v.value == 2 ** 33
    assert L.krk_gguf_array_f64(h, b"a.arr_f32", 1, C.byref(d)) == 0 and d.value == 0.25
    assert L.krk_gguf_array_str(h, b"a.arr_str", 1, C.byref(sp)) == 0 and sp.value == b"yz"
    assert L.krk_gguf_array_i64(h, b"a.arr_i32", 3, C.byref(v)) != 0
    assert L.krk_gguf_array_str(h, b"a.arr_i32", 0, C.byref(sp)) != 0
    assert g.kv_type(g.keys().index("a.arr_str")) == (ARRAY, STRING, 2)
    for name, tid, ne, data in tensors:
        t = g.tensor(name)
        assert t.type_id == tid and list(t.ne)[: len(ne)] == ne
        if tid == 24:
            assert not t.dtype_known and t.n_bytes == 0
            with pytest.raises(krk.KrkError):
                g.data(name)
        else:
            assert t.n_bytes == len(data) and g.data(name).tobytes() == data
    assert g.tensor("w.q4k").offset % 64 == 0
    with pytest.raises(KeyError):
        g.tensor("absent")


def test_reader_refuses_bad_files(krk, tmp_path):
    good = str(tmp_path / "g.gguf")
    data_off = write_gguf(good, [("k", U32, 1)], [("w", 8, [32, 1], bytes(34))])
    raw = open(good, "rb").read()
    krk.Gguf(good)
    cases = {
        "magic": b"GGUX" + raw[4:],
        "version": raw[:4] + struct.pack("<I", 1) + raw[8:],
        "truncated": raw[:30],
        "data past end": raw[:data_off + 20],   # the 34 bytes of w cut at 20
        "nested array": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) +
        struct.pack("<Q", 1) + b"k" + struct.pack("<IIQ", ARRAY, ARRAY, 1),
    }
    split = str(tmp_path / "s.gguf")
    write_gguf(split, [("split.count", U16, 2), ("split.no", U16, 0)], [])
    cases["split"] = open(split, "rb").read()
    for name, blob in cases.items():
        p = str(tmp_path / f"bad_{name.replace(' ', '_')}.gguf")
        open(p, "wb").write(blob)
        with pytest.raises(krk.KrkError):
            krk.Gguf(p)
    with pytest.raises(krk.KrkError):
        krk.Gguf(str(tmp_path / "absent.gguf"))


@pytest.mark.gpu
def test_gguf_upload_real_blocks(krk, torch_cuda, be32, tmp_path):
    """Real ggml blocks (Q8_0, IQ4_NL and Q3_K tensors of the reference's
    checkpoints) through a GGUF file, the reader, the verbatim upload and the
    device decoder, bit for bit against the oracle; and one GEMV on each."""
    torch = torch_cuda
    f = np.load(GOLD)
    n = len([k for k in f.files if k.startswith("name")])
    # names are unique per source file; two files share "blk.0.attn_q.weight"
    tensors = [(f"t{i}." + f[f"name{i}"].tobytes().decode(), int(f[f"type{i}"][0]),
                [int(x) for x in f[f"ne{i}"]], f[f"bytes{i}"].tobytes()) for i in range(n)]
    path = str(tmp_path / "real.gguf")
    write_gguf(path, [("general.architecture", STRING, "llama")], tensors)
    g = krk.Gguf(path)
    for name, dt, ne, data in tensors:
        n_in, n_rows = ne[0], ne[1]
        dev = torch.empty(len(data), dtype=torch.uint8, device="cuda")
        g.upload(be32, name, dev)
        assert bytes(dev.cpu().numpy()) == data
        out = torch.empty((n_rows, n_in), dtype=torch.float32, device="cuda")
        be32.dequant_rows(out, dev, dt, n_rows, n_in)
        be32.sync()
        want = O.dequant(dt, np.frombuffer(data, np.uint8), n_rows, n_in)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)), name
        x = krk.synth_normal(n_in, seed=3)
        y = torch.empty((1, n_rows), dtype=torch.float32, device="cuda")
        be32.gemm(y, torch.from_numpy(x).cuda(), dev, dt, n_rows, n_in, 1)
        be32.sync()
        ref = O.gemm(dt, np.frombuffer(data, np.uint8), x.reshape(1, n_in), n_rows)
        assert np.linalg.norm(y.cpu().numpy() - ref) <= 1e-5 * np.linalg.norm(ref), name
