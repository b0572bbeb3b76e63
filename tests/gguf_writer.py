"""A minimal GGUF v2/v3 writer for the reader's tests (test infrastructure,
written from the GGUF specification): header, metadata, tensor
descriptors, the data section at the alignment boundary, each tensor's
bytes padded to the alignment."""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _scalar(t, v):
    return _str(v) if t == STRING else struct.pack(_FMT[t], v)


def encode_kv(key, t, v, elem=None):
    out = _str(key) + struct.pack("<I", t)
    if t == ARRAY:
        out += struct.pack("<IQ", elem, len(v)) + b"".join(_scalar(elem, x) for x in v)
    else:
        out += _scalar(t, v)
    return out


def write_gguf(path, kvs, tensors, alignment=32, version=3, raw_kv=b""):
    """kvs: [(key, type, value[, elem])]; tensors: [(name, type_id, ne, data bytes)]."""
    blob = b"".join(encode_kv(*kv) for kv in kvs) + raw_kv
    n_kv = len(kvs) + (1 if raw_kv else 0)
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), n_kv) + blob
    infos, off, datas = b"", 0, []
    for name, tid, ne, data in tensors:
        infos += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        infos += struct.pack("<IQ", tid, off)
        pad = (-len(data)) % alignment
        datas.append(bytes(data) + b"\0" * pad)
        off += len(data) + pad
    body = head + infos
    body += b"\0" * ((-len(body)) % alignment)
    with open(path, "wb") as f:
        f.write(body + b"".join(datas))
    return len(body)
