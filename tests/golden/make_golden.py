"""Writes tests/golden/quant_golden.npz from the REFERENCE's own host quant
code (oracle/_ref/libkrk_ref.so, compiled by oracle/Makefile from
/root/reference/src/quant.cpp + src/common.cpp).

The fixture is data only: seeded block bytes and activations (inputs) and
the reference's outputs for them (Q4_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS, MXFP4, Q4_1, Q5_0, Q5_1:
dequant_row f32, dequant_row_f16,
vec_dot in the strict scalar tier, quantize_q8_row, dot_q8_0_q8_scalar; and the generic-chunk formats Q8_1, Q8_K, TQ1_0, TQ2_0,
NVFP4, ROCmFP4, ROCmFP4_FAST and the three ROCmFPX formats).
It lets the oracle be checked bit for bit where the reference tree is absent
(the GPU box).  Run:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import oracle  # noqa: E402
from conftest import rand_blocks  # noqa: E402

# the formats served through the generic 32-value chunk path, each from a
# stream of its own
CHUNK_GOLDEN = tuple((dt, f"chunk{dt}", 0x5EE000 + dt) for dt in oracle.CHUNK_FMTS)

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quant_golden.npz")


def main():
    oracle.build()
    ref = oracle.ref()
    if ref is None:
        raise SystemExit("oracle/_ref/libkrk_ref.so is not built (needs /root/reference)")
    p = oracle._p
    rng = np.random.default_rng(0x5EED)
    data = {}
    for dt, name in ((oracle.Q4_0, "q4_0"), (oracle.Q8_0, "q8_0"), (oracle.Q4_K, "q4_k"),
                     (oracle.Q6_K, "q6_k")):
        bs = ref.ref_block_size(dt)
        nb = 2048 // bs
        n = nb * bs
        w = rand_blocks(rng, dt, nb)
        x = rng.standard_normal(n).astype(np.float32)
        deq = np.empty(n, np.float32)
        ref.ref_dequant_row(dt, p(w), p(deq), n)
        h = np.empty(n, np.uint16)
        ref.ref_dequant_row_f16(dt, p(w), p(h), n)
        dots = np.empty(8, np.float32)
        for i in range(8):  # prefixes of growing length pin the chain order
            m = n * (i + 1) // 8 // bs * bs
            dots[i] = ref.ref_vec_dot(dt, p(w), p(x), m)
        data[f"{name}_w"] = w
        data[f"{name}_x"] = x
        data[f"{name}_deq"] = deq
        data[f"{name}_deq_f16"] = h
        data[f"{name}_dot"] = dots
    # int8 activation path
    x = (rng.standard_normal(2048) * 3).astype(np.float32)
    x[:6] = [1e30, -1e30, 1e-30, 0.0, 3.5, -0.001]
    x[64:96] = 0.0  # an all-zero block
    xq = np.empty(2048, np.int8)
    dx = np.empty(64, np.float32)
    ref.ref_quantize_q8_row(p(x), 2048, p(xq), p(dx))
    w = rand_blocks(rng, oracle.Q8_0, 64)
    x2 = rng.standard_normal(2048).astype(np.float32)
    xq2 = np.empty(2048, np.int8)
    dx2 = np.empty(64, np.float32)
    ref.ref_quantize_q8_row(p(x2), 2048, p(xq2), p(dx2))
    d8 = np.float32(ref.ref_dot_q8_0_q8_scalar(p(w), p(xq2), p(dx2), 2048))
    data.update(q8act_x=x, q8act_xq=xq, q8act_dx=dx, q8dot_w=w, q8dot_x=x2,
                q8dot_out=np.array([d8], np.float32))
    # Q5_K, from a stream of its own so the vectors above stay as they were
    rng5 = np.random.default_rng(0x5EED5)
    dt, bs = oracle.Q5_K, 256
    n = 2048
    w = rand_blocks(rng5, dt, n // bs)
    x = rng5.standard_normal(n).astype(np.float32)
    deq = np.empty(n, np.float32)
    ref.ref_dequant_row(dt, p(w), p(deq), n)
    h = np.empty(n, np.uint16)
    ref.ref_dequant_row_f16(dt, p(w), p(h), n)
    dots = np.empty(8, np.float32)
    for i in range(8):
        m = n * (i + 1) // 8 // bs * bs
        dots[i] = ref.ref_vec_dot(dt, p(w), p(x), m)
    data.update(q5_k_w=w, q5_k_x=x, q5_k_deq=deq, q5_k_deq_f16=h, q5_k_dot=dots)
    # IQ4_NL, also from a stream of its own
    rng4 = np.random.default_rng(0x5EED4)
    dt, bs = oracle.IQ4_NL, 32
    w = rand_blocks(rng4, dt, n // bs)
    x = rng4.standard_normal(n).astype(np.float32)
    deq = np.empty(n, np.float32)
    ref.ref_dequant_row(dt, p(w), p(deq), n)
    h = np.empty(n, np.uint16)
    ref.ref_dequant_row_f16(dt, p(w), p(h), n)
    dots = np.empty(8, np.float32)
    for i in range(8):
        m = n * (i + 1) // 8 // bs * bs
        dots[i] = ref.ref_vec_dot(dt, p(w), p(x), m)
    data.update(iq4_nl_w=w, iq4_nl_x=x, iq4_nl_deq=deq, iq4_nl_deq_f16=h, iq4_nl_dot=dots)
    # IQ4_XS, also from a stream of its own
    rngx = np.random.default_rng(0x5EEDB)
    dt, bs = oracle.IQ4_XS, 256
    w = rand_blocks(rngx, dt, n // bs)
    x = rngx.standard_normal(n).astype(np.float32)
    deq = np.empty(n, np.float32)
    ref.ref_dequant_row(dt, p(w), p(deq), n)
    h = np.empty(n, np.uint16)
    ref.ref_dequant_row_f16(dt, p(w), p(h), n)
    dots = np.empty(8, np.float32)
    for i in range(8):
        m = n * (i + 1) // 8 // bs * bs
        dots[i] = ref.ref_vec_dot(dt, p(w), p(x), m)
    data.update(iq4_xs_w=w, iq4_xs_x=x, iq4_xs_deq=deq, iq4_xs_deq_f16=h, iq4_xs_dot=dots)
    # Q2_K and Q3_K, each from a stream of its own
    for dt, name, seed in ((oracle.Q2_K, "q2_k", 0x5EED2), (oracle.Q3_K, "q3_k", 0x5EED3),
                           (oracle.MXFP4, "mxfp4", 0x5EEDF), (oracle.Q4_1, "q4_1", 0x5EED1),
                           (oracle.Q5_0, "q5_0", 0x5EED6), (oracle.Q5_1, "q5_1", 0x5EED7),
                           *CHUNK_GOLDEN):
        r = np.random.default_rng(seed)
        bs = ref.ref_block_size(dt)
        w = rand_blocks(r, dt, n // bs)
        x = r.standard_normal(n).astype(np.float32)
        deq = np.empty(n, np.float32)
        ref.ref_dequant_row(dt, p(w), p(deq), n)
        h = np.empty(n, np.uint16)
        ref.ref_dequant_row_f16(dt, p(w), p(h), n)
        dots = np.empty(8, np.float32)
        for i in range(8):
            m = n * (i + 1) // 8 // bs * bs
            dots[i] = ref.ref_vec_dot(dt, p(w), p(x), m)
        data.update({f"{name}_w": w, f"{name}_x": x, f"{name}_deq": deq, f"{name}_deq_f16": h,
                     f"{name}_dot": dots})
    np.savez_compressed(OUT, **data)
    print("wrote", OUT, sum(v.nbytes for v in data.values()), "bytes")


if __name__ == "__main__":
    main()
