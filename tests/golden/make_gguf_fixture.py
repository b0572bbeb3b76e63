"""Writes tests/golden/gguf_q8_0_blocks.npz: the raw bytes of real Q8_0,
IQ4_NL and Q3_K tensors from the reference's own test checkpoints (TinyLLama-v0
Q8_0, tinystories-gpt Q2_K mix, tiny-llama3 Q3_K_M: data the reference's
tests read), taken with this library's GGUF reader,
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

REF = "/root/reference/"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gguf_q8_0_blocks.npz")
PICK = [("TinyLLama-v0.Q8_0.gguf", "blk.0.attn_q.weight", K.Q8_0),
        ("TinyLLama-v0.Q8_0.gguf", "blk.0.ffn_down.weight", K.Q8_0),
        ("TinyLLama-v0.Q8_0.gguf", "blk.7.ffn_gate.weight", K.Q8_0),
        ("tinystories-gpt-0.1-3m.Q2_K.gguf", "blk.0.attn_qkv.weight", K.IQ4_NL),
        ("tinystories-gpt-0.1-3m.Q2_K.gguf", "blk.0.ffn_up.weight", K.IQ4_NL),
        ("tiny-llama3-test-Q3_K_M.gguf", "blk.0.attn_q.weight", K.IQ4_NL),
        ("tinystories-gpt-0.1-3m.Q2_K.gguf", "blk.0.ffn_down.weight", K.Q3_K),
        ("tinystories-gpt-0.1-3m.Q2_K.gguf", "blk.7.ffn_down.weight", K.Q3_K)]


def main():
    out = {}
    for i, (fname, name, want) in enumerate(PICK):
        g = K.Gguf(REF + fname)
        t = g.tensor(name)
        assert t.type_id == want, (fname, name, t.type_id)
        out[f"name{i}"] = np.frombuffer(name.encode(), np.uint8)
        out[f"type{i}"] = np.array([t.type_id], np.int64)
        out[f"ne{i}"] = np.array(list(t.ne)[: t.n_dims], np.int64)
        out[f"bytes{i}"] = g.data(name).copy()
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
