"""Writes tests/golden/gguf_q8_0_blocks.npz: the raw bytes of real Q8_0
tensors from the reference's own test checkpoint TinyLLama-v0.Q8_0.gguf
(data the reference's tests read), taken with this library's GGUF reader,
which tests/test_gguf.py checks against the reference's reader.  The GPU
tests use them as real ggml blocks (the reference tree is not on the GPU
box).  Run:  python tests/golden/make_gguf_fixture.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import kraken_amd as K  # noqa: E402

SRC = "/root/reference/TinyLLama-v0.Q8_0.gguf"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gguf_q8_0_blocks.npz")
NAMES = ["blk.0.attn_q.weight", "blk.0.ffn_down.weight", "blk.7.ffn_gate.weight"]


def main():
    g = K.Gguf(SRC)
    out = {}
    for i, name in enumerate(NAMES):
        t = g.tensor(name)
        assert t.type_id == K.Q8_0, (name, t.type_id)
        out[f"name{i}"] = np.frombuffer(name.encode(), np.uint8)
        out[f"ne{i}"] = np.array(list(t.ne)[: t.n_dims], np.int64)
        out[f"bytes{i}"] = g.data(name).copy()
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
