#!/usr/bin/env python3
"""Benchmark of the quantized weight-math hot path on one MI355X.

Headline (BASELINE.json metric): Q4_K decode GEMV, 4096 -> 14336, M = 1,
f32 activations, GB/s and fraction of the 8 TB/s HBM roofline.  A "step" is
one GEMV over one weight matrix; the matrix rotates through >= 1 GiB of
distinct copies so every call streams from HBM rather than the 256 MB MALL.
The same run reports the Q4_K prefill GEMM (M = 2048, Llama-3-8B FFN up and
down) in TFLOP/s against the dense FP16 MFMA peak, and the scalar CPU oracle
timed on this host's cores.  ``--all`` adds the other BASELINE configs.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0
ROTATE_BYTES = 2 << 30   # distinct weight copies per GEMV configuration: 8x the MALL


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="", help="comma list of sections: gemm,rows,int8,layer,formats,head,moe "
                    "(the headline GEMV always runs); default all")
    ap.add_argument("--rotate-gib", type=float, default=2.0,
                    help="GiB of distinct weight copies each GEMV configuration rotates through")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--soak-seconds", type=float, default=3.0,
                    help="untimed back-to-back headline GEMVs before its timed steps")
    ap.add_argument("--moe-tokens", default="1,16,512", help="comma list of MoE batch sizes to time")
    ap.add_argument("--moe-q4km-tokens", default="16,512",
                    help="comma list of MoE batch sizes also timed with Q6_K down banks (Q4_K_M)")
    ap.add_argument("--moe-exact-tokens", default="512",
                    help="comma list of MoE batch sizes also timed under KRK_PATH_EXACT")
    ap.add_argument("--pmc-rows", default="", metavar="ROWS",
                    help="run the rows GEMV (comma list of row counts) for a counter pass and exit")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="counter run: 5 plain copies of 256 MiB, then 20 headline GEMVs")
    ap.add_argument("--summarize-trace", metavar="KERNEL_TRACE_CSV",
                    help="turn a rocprofv3 --kernel-trace csv into per-(kernel, grid, block) "
                         "duration rows (markdown, printed)")
    ap.add_argument("--summarize-counters", metavar="COUNTER_CSV",
                    help="turn a rocprofv3 --pmc counter_collection.csv into per-(kernel, grid) "
                         "medians and derived rates (markdown, printed)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="turn two rocprofv3 --pmc counter_collection.csv files of a "
                         "--pmc-pass run into the traffic summary (printed)")
    return ap.parse_args()


class Timer:
    """HIP events on the stream the kernels are launched on, marginal time
    per call as the reference's kraken-bench measures it
    (tools/bench_ops.cpp:269-285: (t_many - t_one) / (iters - 1)).

    A Python call through ctypes costs ~13 us of host time, longer than a
    decode GEMV kernel, so timing a loop of eager calls measures the host.
    ``run`` therefore captures the calls into HIP graphs (on a side stream,
    with the backends switched to it): graphs of ``iters`` back-to-back
    calls and graphs of a single call, each replay timed alone.  The median
    single-call replay is subtracted from the median ``iters``-call replay,
    so the graph's launch latency and the first call's ramp cancel and what
    remains is the steady-state time per call, independent of ``iters``.

    ``distinct``: fn(i) reads weight copy i % distinct.  The calls are then
    split over windows of ``iters`` consecutive copies, one graph each, and
    the windows (and the single-call graphs, one per copy) are replayed in
    turn, so successive replays read distinct copies and no replay finds
    its weights in the 256 MB MALL left there by the one before.

    Each timed batch keeps the GPU busy for at least ``min_batch_ms``:
    replays enqueued back to back, one event pair each, one synchronisation
    at the end.  Short bursts separated by host synchronisations let the
    clocks recover between replays and read several percent faster than
    sustained load (the headline: 6.9-7.1 us per call in 20-call windows
    with a synchronisation after each replay, 7.5 us in 400-call windows);
    with sustained batches the two agree within 2%.
    """

    min_batch_ms = 60.0

    def __init__(self, torch, stream, backends, warm_replays=2, reps=3):
        self.t, self.s, self.backends = torch, stream, backends
        self.warm_replays, self.reps = warm_replays, reps

    def _capture(self, fn, first, count):
        torch = self.t
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        with torch.cuda.graph(g, stream=side):
            for be in self.backends:
                be.set_stream(side)
            for i in range(first, first + count):
                fn(i)
        for be in self.backends:
            be.set_stream(self.s)
        return g

    def _time(self, graphs, reps):
        """Median replay time over rounds of the graphs taken in turn, at
        least reps rounds and enough for min_batch_ms of back-to-back work
        (one untimed-for-the-result round sizes the batch)."""
        import math
        torch = self.t
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(self.s)
        for g in graphs:
            g.replay()
        e1.record(self.s)
        torch.cuda.synchronize()
        rounds = max(reps, math.ceil(self.min_batch_ms / max(e0.elapsed_time(e1), 1e-3)))
        pairs = []
        for _ in range(rounds):
            for g in graphs:
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(self.s)
                g.replay()
                b.record(self.s)
                pairs.append((a, b))
        torch.cuda.synchronize()
        ts = sorted(a.elapsed_time(b) for a, b in pairs)
        return ts[len(ts) // 2]

    def run(self, fn, iters, warmup, soak_s=0.0, distinct=1):
        """Marginal ms per call of fn over `iters` back-to-back calls;
        soak_s: untimed replays for that many seconds first (the headline,
        so the GPU is busy long enough for an outside sampler to see it)."""
        torch = self.t
        iters = max(1, iters)
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        nwin = max(1, -(-distinct // iters))
        many = [self._capture(fn, j * iters, iters) for j in range(nwin)]
        ones = [self._capture(fn, j, 1) for j in range(max(1, distinct))] if iters > 1 else []
        # untimed replays until the clocks and caches settle: the first
        # replays of a fresh graph run up to ~7% slower than later ones
        for _ in range(self.warm_replays):
            for g in many + ones:
                g.replay()
        torch.cuda.synchronize()
        t_end = time.perf_counter() + soak_s
        while time.perf_counter() < t_end:
            for g in many:
                g.replay()
            torch.cuda.synchronize()
        t_many = self._time(many, max(self.reps, -(-5 // nwin)))
        if not ones:
            return t_many
        t_one = self._time(ones, max(1, -(-5 // len(ones))))
        return (t_many - t_one) / (iters - 1)


def rotation(torch, w_host, min_bytes=None):
    """Distinct copies of a weight matrix filling >= min_bytes, carved out of
    one allocation (as a model's weights sit in one arena), so every call
    streams its matrix from HBM rather than from the 256 MB MALL."""
    min_bytes = ROTATE_BYTES if min_bytes is None else min_bytes
    base = torch.from_numpy(w_host).cuda()
    n = max(2, -(-min_bytes // base.numel()))
    stride = -(-base.numel() // 256) * 256
    arena = torch.empty(n * stride, dtype=base.dtype, device=base.device)
    copies = []
    for i in range(n):
        c = arena[i * stride:i * stride + base.numel()]
        c.copy_(base)
        copies.append(c)
    return copies


def bench_gemv(K, torch, be, timer, args, dt, n_out, n_in, seed, act_f16=False, tile=1, soak_s=0.0):
    """tile > 1: n_out / tile seeded rows quantized and repeated, for the
    vocabulary-sized heads (the host generator would take ~20 s for 525 M
    values; the bytes stream from HBM either way)."""
    import numpy as np
    part = n_out // tile
    assert part * tile == n_out
    w = K.quantize(dt, K.synth_normal(part * n_in, seed=seed, std=0.02), part, n_in, 16)
    if tile > 1:
        w = np.tile(w, tile)
    ws = rotation(torch, w)
    x = K.synth_normal(n_in, seed=seed + 1)
    xt = torch.from_numpy(x.astype(np.float16) if act_f16 else x).cuda()
    out = torch.empty((1, n_out), dtype=torch.float16 if act_f16 else torch.float32,
                      device="cuda")
    ms = timer.run(lambda i: be.gemm(out, xt, ws[i % len(ws)], dt, n_out, n_in, 1),
                   args.steps, args.warmup, soak_s=soak_s, distinct=len(ws))
    nbytes = K.row_bytes(dt, n_in) * n_out
    act_bytes = (n_in + n_out) * (2 if act_f16 else 4)
    return {"ms": ms, "weight_bytes": nbytes, "bytes": nbytes + act_bytes,
            "GBps": (nbytes + act_bytes) / ms / 1e6, "copies": len(ws), "w": w, "x": x, "ws": ws}


def bench_gemm(K, torch, be, timer, dt, M, n_out, n_in, seed, iters=20, warmup=3):
    import numpy as np
    w = K.quantize(dt, K.synth_normal(n_out * n_in, seed=seed, std=0.02), n_out, n_in, 16)
    wt = torch.from_numpy(w).cuda()
    x = torch.from_numpy(K.synth_normal(M * n_in, seed=seed + 1).astype(np.float16)).cuda()
    out = torch.empty((M, n_out), dtype=torch.float16, device="cuda")
    ms = timer.run(lambda i: be.gemm(out, x, wt, dt, n_out, n_in, M), iters, warmup)
    flops = 2.0 * M * n_out * n_in
    return {"ms": ms, "TFLOPs": flops / ms / 1e9, "frac": flops / ms / 1e9 / FP16_PEAK_TFLOPS,
            "M": M, "N": n_out, "K": n_in}


def moe_banks(K, torch, down, n_expert=128, n_embd=4096, n_ff=1536, distinct=8):
    """BASELINE config 5's expert banks: Q4_K gate/up [1536, 4096] and down
    [4096, 1536] (down = K.Q6_K: the Q4_K_M layout), quantized by the
    library's quantizer from seeded N(0, 0.02) weights.  `distinct` experts
    are generated (2.4 G values for all 128 would take the host ~40 s) and
    the 128 banks are separate device copies of them: every bank is its own
    memory, so the bytes a call streams are those of 128 distinct experts."""
    import numpy as np
    shapes = ((n_ff, n_embd), (n_ff, n_embd), (n_embd, n_ff))
    proto = []
    for d in range(distinct):
        mats = []
        for m, (o, i) in enumerate(shapes):
            dt = down if m == 2 else K.Q4_K
            v = K.synth_normal(o * i, seed=500 + 3 * d + m, std=0.02, nthreads=16)
            mats.append(K.quantize(dt, v, o, i, 16))
        proto.append(mats)
    keep, entries = [], []
    for e in range(n_expert):
        ent = K.MoeEntry()
        for m, (o, i) in enumerate(shapes):
            dt = down if m == 2 else K.Q4_K
            t = torch.from_numpy(proto[e % distinct][m]).cuda()
            keep.append(t)
            ent.p[m] = t.data_ptr()
            ent.n_out[m], ent.n_in[m] = o, i
            ent.row_bytes[m] = K.row_bytes(dt, i)
            ent.type[m] = dt
            ent.present[m] = 1
        entries.append(ent)
    table = torch.from_numpy(np.frombuffer(K.moe_table_bytes(entries), np.uint8).copy()).cuda()
    return keep, table


def bench_moe(K, torch, be, timer, n_tok, banks, n_expert=128, n_embd=4096, n_ff=1536, k=8, calls=64, down=None):
    """qwen3moe-shaped experts (moe_banks), router softmax
    -> top-8 -> normalize -> dispatch.  Each timed call routes a different
    seeded logits block, so the experts read vary and the 1.36 GB of banks
    stream from HBM."""
    down = K.Q4_K if down is None else down
    import numpy as np
    _, table = banks
    logits = torch.from_numpy(K.synth_normal(calls * n_tok * n_expert, seed=31)).cuda()
    logits = logits.reshape(calls, n_tok, n_expert)
    x = torch.from_numpy(K.synth_normal(n_tok * n_embd, seed=32)).cuda().reshape(n_tok, n_embd)
    probs = torch.empty((n_tok, n_expert), dtype=torch.float32, device="cuda")
    ids = torch.empty((n_tok, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((n_tok, k), dtype=torch.float32, device="cuda")
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device="cuda")

    def step(i):
        be.router_softmax(probs, logits[i % calls], n_tok, n_expert)
        be.router_topk(probs, n_tok, n_expert, k, ids, wts, True, 1.0)
        be.moe_dispatch(table, 0, n_expert, ids, wts, x, out, n_tok, n_embd, n_ff, k)

    ms = timer.run(step, calls, 4, distinct=calls)
    # distinct experts per call, from the same routing on the host
    import oracle as O
    distinct = []
    lg = logits.cpu().numpy()
    for i in range(calls):
        rid, _ = O.router_topk(O.router_softmax(lg[i]), k)
        distinct.append(len(set(rid.reshape(-1).tolist())))
    per_expert = 2 * n_ff * K.row_bytes(K.Q4_K, n_embd) + n_embd * K.row_bytes(down, n_ff)
    nbytes = float(np.mean(distinct)) * per_expert + 4 * (2 * n_tok * n_embd + n_tok * n_expert)
    flops = 2.0 * 3 * n_tok * k * n_embd * n_ff   # gate, up and down of every (token, slot) pair
    return {"us": ms * 1e3, "GBps": nbytes / ms / 1e6, "distinct_experts": float(np.mean(distinct)),
            "bytes_per_call": nbytes, "TFLOPs": flops / ms / 1e9}


def bench_layer_grouped(K, torch, be, timer, copies=None):
    """One Llama-2-7B decode layer's weight math the way the engine issues it:
    gemm_group(q, k, v), gemm(o), gemm_group(gate, up, silu), gemm(down).
    The layer's 113.8 MB rotate through `copies` distinct layers (default:
    as many as fill the rotation bytes)."""
    import numpy as np
    copies = copies or -(-ROTATE_BYTES // 113_836_032)
    shapes = {"q": (4096, 4096), "k": (4096, 4096), "v": (4096, 4096), "o": (4096, 4096),
              "gate": (11008, 4096), "up": (11008, 4096), "down": (4096, 11008)}
    # one layer quantized from seeded N(0, 0.02), `copies` device copies of it
    host = {nm: K.quantize(K.Q4_K, K.synth_normal(o * i, seed=40 + j, std=0.02, nthreads=16), o, i, 16)
            for j, (nm, (o, i)) in enumerate(shapes.items())}
    layers = [{nm: torch.from_numpy(h).cuda() for nm, h in host.items()} for _ in range(copies)]
    x = torch.from_numpy(K.synth_normal(4096, seed=40)).cuda().reshape(1, 4096)
    q, kk, v, o = (torch.empty((1, 4096), device="cuda") for _ in range(4))
    ffn = torch.empty((1, 11008), device="cuda")
    up = torch.empty((1, 11008), device="cuda")
    y = torch.empty((1, 4096), device="cuda")

    def step(i):
        L = layers[i % copies]
        be.gemm_group([q, kk, v], x, [L["q"], L["k"], L["v"]], K.Q4_K, [4096] * 3, 4096, 1)
        be.gemm(o, q, L["o"], K.Q4_K, 4096, 4096, 1)
        be.gemm_group([ffn, up], x, [L["gate"], L["up"]], K.Q4_K, [11008, 11008], 4096, 1, silu=True)
        be.gemm(y, ffn, L["down"], K.Q4_K, 4096, 11008, 1)

    ms = timer.run(step, 64, 4, distinct=copies)
    nbytes = sum(K.row_bytes(K.Q4_K, i) * o for o, i in shapes.values())
    nbytes += 4 * (4 * 4096 + 4 * 4096 + 11008 * 2 + 4096)
    return {"us": ms * 1e3, "GBps": nbytes / ms / 1e6, "bytes": nbytes, "launches": 4}


def cpu_baseline(O, w, x, n_out, n_in, seconds):
    """The reference's strict scalar CPU path (one f32 vec_dot chain per
    output row, rows split over threads) on this host's cores, on a bounded
    sample of the same GEMV: the reference's own quant code built from its
    sources (oracle/_ref, kind "reference") where that build travelled with
    the tree, else the C restatement (kind "port"), which equals it bit for
    bit."""
    # the GPU box gives one GPU's job 16 host threads (its CPU share), whatever
    # nproc shows; the thread count used and nproc are both reported
    nproc = os.cpu_count() or 1
    cores = min(16, nproc)
    kind = "reference" if O.ref_available() else "port"

    def run(wb, rows, threads):
        if kind == "reference":
            O.ref_gemv(O.Q4_K, wb, x, rows, nthreads=threads)
        else:
            O.gemm(O.Q4_K, wb, x, rows, nthreads=threads)

    t0 = time.perf_counter()
    reps = 0
    while True:
        run(w, n_out, cores)
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt_all = (time.perf_counter() - t0) / reps
    # one core: a 1/16 slice of the rows, scaled
    rows1 = max(1, n_out // 16)
    rb = O.row_bytes(O.Q4_K, n_in)
    t1 = time.perf_counter()
    run(w[:rows1 * rb], rows1, 1)
    dt_one = (time.perf_counter() - t1) * n_out / rows1
    nbytes = rb * n_out + (n_in + n_out) * 4
    return {"value": nbytes / dt_all / 1e9, "unit": "GB/s", "cores": cores, "nproc": nproc, "kind": kind,
            "sample": f"Q4_K GEMV {n_in}->{n_out} M=1, {reps} calls over {dt_all * reps:.1f} s",
            "one_core_GBps": nbytes / dt_one / 1e9}


COPY_BYTES = 256 << 20


def pmc_pass():
    """The program the HBM-traffic counters are read on: a plain copy of known
    size (the calibration) and the headline GEMV, eagerly, on one stream."""
    import torch

    import kraken_amd as K
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    be = K.Backend(0, K.ACT_F32)
    n_out, n_in = 14336, 4096
    w = K.quantize(K.Q4_K, K.synth_normal(n_out * n_in, seed=1, std=0.02), n_out, n_in, 16)
    ws = rotation(torch, w)
    x = torch.from_numpy(K.synth_normal(n_in, seed=2)).cuda()
    out = torch.empty((1, n_out), dtype=torch.float32, device="cuda")
    for i in range(20):
        be.gemm(out, x, ws[i % len(ws)], K.Q4_K, n_out, n_in, 1)
    torch.cuda.synchronize()
    be.close()


def pmc_rows(rows):
    """The program the rows counters are read on: the Q4_K GEMV of each
    activation-row count (4096 -> 14336, f16 activations, as the bench's
    rows section), ten eager calls each."""
    import torch

    import kraken_amd as K
    be = K.Backend(0, K.ACT_F16)
    n_out, n_in = 14336, 4096
    w = torch.from_numpy(K.quantize(K.Q4_K, K.synth_normal(n_out * n_in, seed=1, std=0.02, nthreads=16),
                                    n_out, n_in, 16)).cuda()
    for m in rows:
        x = torch.from_numpy(K.synth_normal(m * n_in, seed=2)).cuda().reshape(m, n_in).half()
        out = torch.empty((m, n_out), dtype=torch.float16, device="cuda")
        for _ in range(10):
            be.gemm(out, x, w, K.Q4_K, n_out, n_in, m)
    torch.cuda.synchronize()
    be.close()


def summarize_pmc(fetch_csv, write_csv):
    """Per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) of the copy and the GEMV,
    the copy's counter/true-bytes factor, and the GEMV's HBM bytes."""
    import csv
    import statistics

    def per_kernel(path, counter):
        # per dispatch: the calibration copies are the largest copy dispatches
        # (the 256 MiB ones; the weight clones are smaller), the GEMV is ours
        copies, gemv = [], []
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] != counter:
                continue
            v = float(r["Counter_Value"])
            if "krk::" in r["Kernel_Name"]:
                gemv.append(v)
            elif "copyBuffer" in r["Kernel_Name"]:
                copies.append(v)
        top = max(copies)
        cal = [v for v in copies if v > 0.9 * top]
        return {"copy": statistics.median(cal), "gemv": statistics.median(gemv),
                "n_copy": len(cal), "n_gemv": len(gemv)}

    f, w = per_kernel(fetch_csv, "FETCH_SIZE"), per_kernel(write_csv, "WRITE_SIZE")
    kib = COPY_BYTES / 1024.0
    rf, rw = f["copy"] / kib, w["copy"] / kib
    gf, gw = f["gemv"] / rf * 1024.0, w["gemv"] / rw * 1024.0
    return {"copy_dispatches": f["n_copy"], "gemv_dispatches": f["n_gemv"],
            "copy_fetch_kib": f["copy"], "copy_write_kib": w["copy"], "copy_true_kib": kib,
            "fetch_factor": rf, "write_factor": rw, "gemv_fetch_kib": f["gemv"],
            "gemv_write_kib": w["gemv"], "gemv_fetch_bytes": gf, "gemv_write_bytes": gw,
            "hbm_bytes_per_launch": gf + gw}


# Labels of the default bench's launches for the trace summary: (substring
# of the kernel name, grid size, configuration, work per launch, unit of the
# work: "B" algorithmic bytes, "f16" / "int8" 2 M N K operations, or None).
_Q4K_ROW, _Q6K_ROW, _Q8_ROW = 2304, 3360, 4352
_HEAD_BYTES = 14336 * _Q4K_ROW + 4 * (4096 + 14336)
TRACE_LABELS = [
    ("gemv_stream_kernel<12, float, float, 2, 28, 8, true, 0, 8", "262144",
     "headline: Q4_K GEMV 4096->14336, M=1, f32 activations", _HEAD_BYTES, "B"),
    ("gemv_stream_kernelILi12EDF16_DF16_Li2ELi28", "262144", "headline shape, f16 activations",
     14336 * _Q4K_ROW + 2 * (4096 + 14336), "B"),
    ("gemv_stream_kernel<2, float, float, 2, 28", "262144", "Q4_0 GEMV 4096->14336, M=1", _HEAD_BYTES, "B"),
    ("gemv_stream_kernel<8, float, float, 2, 28", "262144", "Q8_0 GEMV 4096->14336, M=1",
     14336 * _Q8_ROW + 4 * (4096 + 14336), "B"),
    ("gemv_stream_kernel<14, float, float, 2, 16, 8, true, 0, 8", "458752", "Q6_K GEMV 4096->14336, M=1 (16-row tiles)",
     14336 * _Q6K_ROW + 4 * (4096 + 14336), "B"),
    ("gemv_stream_kernel<12, float, float, 2, 16, 8, true, 0, 8", "131072",
     "C2 layer: q, k, v, o (Q4_K 4096->4096)", 4096 * _Q4K_ROW + 4 * 8192, "B"),
    ("gemv_stream_kernel<12, float, float, 2, 24, 8, true, 0, 8", "235008",
     "C2 layer: gate, up (Q4_K 4096->11008)", 11008 * _Q4K_ROW + 4 * (4096 + 11008), "B"),
    ("gemv_stream_kernel<12, float, float, 3, 16, 16, false, 0, 8", "245760",
     "C2 layer: down (Q4_K 11008->4096)", 4096 * 6192 + 4 * (4096 + 11008), "B"),
    ("gemv_stream_kernel<12, float, float, 2, 28, 8, true, 0, 8", "75264",
     "C2 grouped: q/k/v in one launch (3 segments)", None, None),
    ("gemv_stream_kernel<12, float, float, 2, 32, 8, true, 0, 8", "352256",
     "C2 grouped: gate+up with the SiLU epilogue", None, None),
    ("gemv_digits_kernel<14, float, float, 16", "131072", "C4 head: Q6_K 128256x4096, row split",
     128256 * _Q6K_ROW + 4 * (4096 + 128256), "B"),
    ("gemv_valu_kernel<8, float, float, 2, 2, true>", "131072", "C4 head: Q8_0 128256x4096, VALU stream kernel",
     128256 * _Q8_ROW + 4 * (4096 + 128256), "B"),
    ("gemv_stream_kernel<12, float, float, 2, 32, 8, true, 1, 8", "49152", "C5 x1: routed gate/up, 8 slots",
     None, None),
    ("gemv_stream_kernel<12, float, float, 3, 16, 16, true, 2, 8", "262144", "C5 x1: routed down over the 8 slots",
     None, None),
    ("gemv_stream_kernel<12, float, float, 2, 32, 8, true, 3, 8", "49152",
     "C5 x16: expert-major gate/up (about 83 experts x 7.08 MB)", None, None),
    ("gemv_stream_kernel<12, float, float, 2, 16, 8, false, 4, 8", "49152",
     "C5 x16: expert-major down (about 83 experts x 3.54 MB)", None, None),
    ("gemv_stream_kernel<14, float, float, 2, 16, 8, false, 4, 8", "49152",
     "C5 x16, Q6_K down banks: expert-major down", None, None),
    ("gemv_stream_kernel<14, float, float, 2, 16, 16, true, 2, 8", "262144",
     "C5 x1, Q6_K down banks: routed down over the 8 slots", None, None),
    ("moe_gemm_kernel<12, true, 2>", "1179648", "C5 x512: grouped expert GEMM, gate/up (64-row items)",
     2 * 4096 * 4096 * 3072, "f16"),
    ("moe_gemm_kernel<12, false, 2>", "1572864", "C5 x512: grouped expert GEMM, down (Q4_K)",
     2 * 4096 * 1536 * 4096, "f16"),
    ("moe_gemm_kernel<14, false, 2>", "1572864", "C5 x512: grouped expert GEMM, down (Q6_K banks)",
     2 * 4096 * 1536 * 4096, "f16"),
    ("moe_gather_f16_kernel", "131072", "C5 x512: the tokens' activation rows to f16, once per token", None, None),
    ("stream_xtab_kernelIDF16", "512", "rows 4, 5 and 8: the rows' digit tables, built once per call (rows in grid y)",
     None, None),
    ("router_softmax_kernel<float, 2>", "64", "C5 x1: router softmax (128 experts)", None, None),
    ("router_topk_rank_kernel<2>", "128", "C5 x1: router top-8 (rank per expert)", None, None),
    ("router_softmax_kernel<float, 2>", "1024", "C5 x16: router softmax", None, None),
    ("router_topk_rank_kernel<2>", "2048", "C5 x16: router top-8", None, None),
    ("router_softmax_kernel<float, 2>", "32768", "C5 x512: router softmax", None, None),
    ("router_topk_rank_kernel<2>", "65536", "C5 x512: router top-8", None, None),
    ("gemv_stream_kernelILi12EDF16_DF16_Li2ELi28ELi8ELb1ELi0ELi8ELi4ELb0E", "262144",
     "rows 4: Q4_K 4096->14336, f16 activations, one pass (weights only in the rate)", 14336 * _Q4K_ROW, "B"),
    ("gemv_stream_kernelILi12EDF16_DF16_Li2ELi28ELi8ELb1ELi0ELi8ELi5ELb0E", "262144",
     "rows 5: the same, one pass", 14336 * _Q4K_ROW, "B"),
    ("gemv_stream_kernelILi12EDF16_DF16_Li2ELi16ELi8ELb1ELi0ELi8ELi8ELb0E", "458752",
     "rows 8: the same, one pass, two passes of four rows' tables", 14336 * _Q4K_ROW, "B"),
    ("moe_gemm_kernel<12, false, 1>", "114688", "rows 16 and 32: Q4_K 4096->14336, streaming dense mode (split-K 4)",
     None, None),
    ("moe_gemm_kernel<12, false, 2>", "114688", "rows 64 and 128: Q4_K 4096->14336, streaming dense mode", None, None),
    ("moe_plan_kernel", "256", "C5 x16 and x512: plan", None, None),
    ("moe_reduce_kernel<float>", "4096", "C5 x16 and x512: ordered reduce", None, None),
    ("gemm_f16_kernelILi12EDF16", "229376", "C3 prefill up, M=2048 (448 tiles)", 2 * 2048 * 14336 * 4096, "f16"),
    ("gemm_f16_kernelILi12EDF16", "65536", "C3 prefill down, M=2048 (128 tiles x split 2, summed in the kernel)",
     2 * 2048 * 14336 * 4096, "f16"),
    ("gemm_f16_kernelILi12EDF16", "57344", "C3 prefill up, M=512 (112 tiles x split 2, summed in the kernel)",
     2 * 512 * 14336 * 4096, "f16"),
    ("gemm_f16_kernelILi12EDF16", "16384", "C3 prefill down, M=512 (32 tiles x split 8)",
     2 * 512 * 14336 * 4096, "f16"),
    ("splitk_reduce_kernelIDF16", "262144", "C3 prefill down, M=512: split-K reduce", None, None),
    ("gemm_i8_kernelILi8EDF16", "458752", "int8 rung: Q8_0 4096->14336, M=2048", 2 * 2048 * 14336 * 4096, "int8"),
    ("quantize_q8_kernelIDF16", "262144", "int8 rung, M=2048: activation quantizer", None, None),
    ("gemm_i8_kernelILi8EDF16", "114688", "int8 rung: Q8_0 4096->14336, M=512", 2 * 512 * 14336 * 4096, "int8"),
    ("quantize_q8_kernelIDF16", "65536", "int8 rung, M=512: activation quantizer", None, None),
]


def summarize_trace(path):
    """Average device duration per (kernel, grid, workgroup), one row per
    launch of the default bench (each configuration launches its kernel with
    its own grid), labelled from TRACE_LABELS with the rate its work implies;
    this library's launches no label names follow unlabelled.  The last line names the
    headline's kernel (read back by the bench's roofline)."""
    import csv
    import statistics
    rows, seq = {}, []
    for r in csv.DictReader(open(path)):
        key = (r["Kernel_Name"], r.get("Grid_Size", r.get("Grid_Size_X", "")),
               r.get("Workgroup_Size", r.get("Workgroup_Size_X", "")))
        t0, t1 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        rows.setdefault(key, []).append((t1 - t0) / 1e3)
        seq.append((t1, key))
    # end-to-end spacing: the interval between the ends of two consecutive
    # dispatches of the same launch with nothing between them (back to back
    # in a graph replay): the time per call the bench's marginal method
    # measures.  A dispatch's own start stamp can precede the end of the one
    # before it, so its duration overstates back-to-back launches.
    seq.sort()
    spacing = {}
    for (ta, ka), (tb, kb) in zip(seq, seq[1:]):
        if ka == kb:
            spacing.setdefault(kb, []).append((tb - ta) / 1e3)
    peaks = {"f16": (2500.0, "TFLOP/s", "f16 peak"), "int8": (5000.0, "TOP/s", "int8 peak")}
    print("| configuration | kernel | grid | block | calls | average (us) | median (us) | median spacing (us) | rate from the spacing |")
    print("|---|---|---|---|---|---|---|---|---|")
    used, headline = set(), None
    order = [(lab, [k for k in rows if lab[0] in k[0] and k[1] == lab[1]]) for lab in TRACE_LABELS]
    for (sub, grid, label, work, unit), hits in order + [((None, None, "", None, None), [k for k in rows if "krk" in k[0]])]:
        for k in hits:
            if k in used:
                continue
            used.add(k)
            d = rows[k]
            avg, med = statistics.mean(d), statistics.median(d)
            sp = statistics.median(spacing[k]) if len(spacing.get(k, [])) >= 3 else None
            per = sp if sp is not None else avg
            rate = ""
            if unit == "B":
                g = work / per / 1e3
                rate = f"{g:.0f} GB/s ({100 * g / HBM_PEAK_GBS:.1f}% of HBM)"
            elif unit in peaks:
                peak, u, what = peaks[unit]
                t = work / per / 1e6
                rate = f"{t:.0f} {u} ({100 * t / peak:.1f}% of {what})"
            name = k[0].replace("|", "\\|")
            sps = f"{sp:.2f}" if sp is not None else "-"
            print(f"| {label} | `{name}` | {k[1]} | {k[2]} | {len(d)} | {avg:.2f} | {med:.2f} | {sps} | {rate} |")
            if headline is None and sub is not None:
                headline = k[0]
            if sub is not None:
                break
    print()
    print(f"headline_kernel: {headline}")


def summarize_counters(path, cus=256, xcds=8):
    """Median per dispatch of every counter, per (kernel, grid), plus:
    clock = GRBM_GUI_ACTIVE / xcds / duration; MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES
    over (4 SIMDs x cus) x the per-XCD active cycles; wait = SQ_WAIT_ANY /
    SQ_WAVE_CYCLES."""
    import csv
    import statistics
    groups = {}
    for r in csv.DictReader(open(path)):
        key = (r["Kernel_Name"], r["Grid_Size"])
        g = groups.setdefault(key, {"dur": {}, "c": {}})
        g["c"].setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
        g["dur"][r["Dispatch_Id"]] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    for (name, grid), g in groups.items():
        med = {c: statistics.median(v) for c, v in g["c"].items()}
        dur = statistics.median(g["dur"].values())
        print(f"### `{name}` grid {grid}")
        print(f"dispatches: {len(g['dur'])}, median duration under counters: {dur:.1f} us")
        for c in sorted(med):
            print(f"- {c}: {med[c]:.0f}")
        if "GRBM_GUI_ACTIVE" in med:
            cyc = med["GRBM_GUI_ACTIVE"] / xcds
            print(f"- clock: {cyc / dur / 1e3:.2f} GHz")
            if "SQ_VALU_MFMA_BUSY_CYCLES" in med:
                print(f"- MFMA busy: {100 * med['SQ_VALU_MFMA_BUSY_CYCLES'] / (4 * cus * cyc):.1f}% of SIMD cycles")
        if "SQ_WAIT_ANY" in med and "SQ_WAVE_CYCLES" in med:
            print(f"- waiting: {100 * med['SQ_WAIT_ANY'] / med['SQ_WAVE_CYCLES']:.1f}% of wave cycles")
        print()


def read_profile_field(fname, key):
    p = os.path.join(ROOT, "profiles", fname)
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith(key + ":"):
            return line.split(":", 1)[1].strip()
    return None


def read_traffic():
    p = os.path.join(ROOT, "profiles", "q4k_gemv_4096x14336_traffic.txt")
    if not os.path.exists(p):
        return None
    vals = {}
    for line in open(p):
        if ":" in line:
            k, v = line.split(":", 1)
            vals[k.strip()] = v.strip()
    try:
        return float(vals["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def main():
    args = parse()
    if args.summarize_counters:
        summarize_counters(args.summarize_counters)
        return
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.summarize_pmc:
        for k, v in summarize_pmc(*args.summarize_pmc).items():
            print(f"{k}: {v:.1f}" if isinstance(v, float) else f"{k}: {v}")
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (no sharding, no collectives); "
              "run it with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.pmc_rows:
        pmc_rows([int(v) for v in args.pmc_rows.split(",")])
        return
    if args.pmc_pass:
        pmc_pass()
        return
    import numpy as np
    import torch

    import kraken_amd as K

    global ROTATE_BYTES
    ROTATE_BYTES = int(args.rotate_gib * (1 << 30))
    only = set(filter(None, args.only.split(",")))
    want = (lambda k: k in only) if only else (lambda k: True)
    stream = torch.cuda.current_stream()
    be32 = K.Backend(0, K.ACT_F32, stream)
    be16 = K.Backend(0, K.ACT_F16, stream)
    timer = Timer(torch, stream, (be32, be16))
    extras = {}

    # ---- headline: Q4_K GEMV 4096 -> 14336, M = 1 ---------------------------
    log("gemv q4_k 4096->14336 ...")
    n_out, n_in = 14336, 4096
    g = bench_gemv(K, torch, be32, timer, args, K.Q4_K, n_out, n_in, seed=1, soak_s=args.soak_seconds)
    log(f"  {g['ms'] * 1e3:.2f} us/call  {g['GBps']:.0f} GB/s  ({g['copies']} copies)")
    # the same call with f16 activations (the reference GPU's activation type)
    g16 = bench_gemv(K, torch, be16, timer, args, K.Q4_K, n_out, n_in, seed=1, act_f16=True)
    extras["gemv_q4k_f16act"] = {"us": g16["ms"] * 1e3, "GBps": g16["GBps"]}

    if want("gemm"):
        for name, (N_, K_) in (("up", (14336, 4096)), ("down", (4096, 14336))):
            for M in (512, 2048):
                log(f"gemm q4_k {name} M={M} ...")
                r = bench_gemm(K, torch, be16, timer, K.Q4_K, M, N_, K_, seed=10)
                log(f"  {r['ms'] * 1e3:.1f} us  {r['TFLOPs']:.1f} TFLOP/s  ({100 * r['frac']:.1f}%)")
                extras[f"prefill_q4k_{name}_m{M}"] = {"us": r["ms"] * 1e3, "TFLOPs": r["TFLOPs"],
                                                      "frac_fp16_peak": r["frac"]}

    if want("rows"):
        # batched rows between the decode GEMV (<= 8) and prefill: 16..128
        # activation rows of the C3 up shape on the MFMA path
        for M in (4, 5, 8, 16, 32, 64, 128):
            log(f"gemm q4_k up M={M} ...")
            r = bench_gemm(K, torch, be16, timer, K.Q4_K, M, 14336, 4096, seed=11)
            gbs = 14336 * K.row_bytes(K.Q4_K, 4096) / r["ms"] / 1e6
            log(f"  {r['ms'] * 1e3:.1f} us  {r['TFLOPs']:.1f} TFLOP/s  {gbs:.0f} GB/s of weights")
            extras[f"gemm_q4k_up_m{M}"] = {"us": r["ms"] * 1e3, "TFLOPs": r["TFLOPs"], "weight_GBps": gbs}

    if want("int8"):
        # the Q8_0 x Q8 int8 rung at the C3 up shape (KRK_PATH_INT8)
        be16.set_gemm_path(K.PATH_INT8)
        for M in (512, 2048):
            log(f"gemm q8_0 int8 rung up M={M} ...")
            r = bench_gemm(K, torch, be16, timer, K.Q8_0, M, 14336, 4096, seed=12)
            extras[f"prefill_q8_0_int8_up_m{M}"] = {
                "us": r["ms"] * 1e3, "TOPs": r["TFLOPs"], "frac_int8_peak": r["TFLOPs"] / INT8_PEAK_TOPS}
            log(f"  {r['ms'] * 1e3:.1f} us  {r['TFLOPs']:.1f} TOP/s  ({100 * r['TFLOPs'] / INT8_PEAK_TOPS:.1f}% of int8 peak)")
        be16.set_gemm_path(K.PATH_AUTO)

    if want("layer"):
        # config 2: Llama-2-7B Q4_K decode layer, M = 1 -- per matrix, and as
        # the reference's decode issues it (fused.hpp:48-275): q/k/v in one
        # grouped launch, gate/up with the SiLU folded in, then o and down
        tot_b, tot_ms = 0, 0.0
        for nm, (o, i) in (("q", (4096, 4096)), ("k", (4096, 4096)), ("v", (4096, 4096)),
                           ("o", (4096, 4096)), ("gate", (11008, 4096)), ("up", (11008, 4096)),
                           ("down", (4096, 11008))):
            r = bench_gemv(K, torch, be32, timer, args, K.Q4_K, o, i, seed=20)
            extras[f"layer_{nm}"] = {"us": r["ms"] * 1e3, "GBps": r["GBps"], "frac_hbm": r["GBps"] / HBM_PEAK_GBS}
            tot_b += r["bytes"]
            tot_ms += r["ms"]
        extras["layer_total"] = {"us": tot_ms * 1e3, "GBps": tot_b / tot_ms / 1e6,
                                 "frac_hbm": tot_b / tot_ms / 1e6 / HBM_PEAK_GBS}
        log(f"  layer, 7 launches: {tot_ms * 1e3:.1f} us {tot_b / tot_ms / 1e6:.0f} GB/s")
        r = bench_layer_grouped(K, torch, be32, timer)
        r["frac_hbm"] = r["GBps"] / HBM_PEAK_GBS
        extras["layer_grouped"] = r
        log(f"  layer, 4 grouped launches: {r['us']:.1f} us {r['GBps']:.0f} GB/s")
    if want("formats"):
        # the other north-star formats at the headline's shape and M = 1
        for dt, nm in ((K.Q6_K, "q6_k"), (K.Q4_0, "q4_0"), (K.Q8_0, "q8_0")):
            r = bench_gemv(K, torch, be32, timer, args, dt, n_out, n_in, seed=3)
            extras[f"gemv_{nm}_4096x14336"] = {"us": r["ms"] * 1e3, "GBps": r["GBps"],
                                                "frac_hbm": r["GBps"] / HBM_PEAK_GBS}
            log(f"  gemv {nm} 4096->14336: {r['ms'] * 1e3:.2f} us {r['GBps']:.0f} GB/s")
    if want("head"):
        for dt, nm in ((K.Q6_K, "q6_k"), (K.Q8_0, "q8_0")):
            r = bench_gemv(K, torch, be32, timer, args, dt, 128256, 4096, seed=30, tile=16)
            extras[f"head_{nm}"] = {"us": r["ms"] * 1e3, "GBps": r["GBps"],
                                    "frac_hbm": r["GBps"] / HBM_PEAK_GBS}
            log(f"  head {nm} {r['ms'] * 1e3:.1f} us {r['GBps']:.0f} GB/s")

    if want("moe"):
        log("moe banks ...")
        banks = moe_banks(K, torch, K.Q4_K)
        for T in (int(v) for v in args.moe_tokens.split(",") if v):
            log(f"moe C5 n_tok={T} ...")
            r = bench_moe(K, torch, be32, timer, T, banks)
            r["frac_hbm"] = r["GBps"] / HBM_PEAK_GBS
            extras[f"moe_c5_t{T}"] = r
            log(f"  {r['us']:.1f} us  {r['GBps']:.0f} GB/s  {r['TFLOPs']:.1f} TFLOP/s  "
                f"({r['distinct_experts']:.1f} experts)")
        banks6 = None
        for T in (int(v) for v in args.moe_q4km_tokens.split(",") if v):
            log(f"moe C5 n_tok={T}, Q6_K down banks ...")
            banks6 = banks6 or moe_banks(K, torch, K.Q6_K)
            r = bench_moe(K, torch, be32, timer, T, banks6, down=K.Q6_K)
            r["frac_hbm"] = r["GBps"] / HBM_PEAK_GBS
            extras[f"moe_c5_q4km_t{T}"] = r
            log(f"  {r['us']:.1f} us  {r['GBps']:.0f} GB/s  {r['TFLOPs']:.1f} TFLOP/s")
        for T in (int(v) for v in args.moe_exact_tokens.split(",") if v):
            log(f"moe C5 n_tok={T}, KRK_PATH_EXACT ...")
            be32.set_gemm_path(K.PATH_EXACT)
            try:
                r = bench_moe(K, torch, be32, timer, T, banks)
            finally:
                be32.set_gemm_path(K.PATH_AUTO)
            r["frac_hbm"] = r["GBps"] / HBM_PEAK_GBS
            extras[f"moe_c5_t{T}_exact"] = r
            log(f"  {r['us']:.1f} us  {r['GBps']:.0f} GB/s  {r['TFLOPs']:.1f} TFLOP/s")
        # the handle remembers a dispatched table by its address, which a
        # later allocation may reuse
        be32.moe_table_forget(banks[1])
        if banks6 is not None:
            be32.moe_table_forget(banks6[1])

    # ---- CPU baseline (rank 0, N = 1) ----------------------------------------
    cpu = None
    if not args.no_cpu:
        import oracle as O
        log("cpu baseline ...")
        cpu = cpu_baseline(O, g["w"], g["x"], n_out, n_in, args.cpu_seconds)
        log(f"  {cpu['value']:.2f} GB/s on {cpu['cores']} cores")

    achieved = g["bytes"] / (g["ms"] * 1e-3) / 1e9
    line = {
        "metric": "decode GEMV GB/s & %HBM peak (Q4_K 4096x14336); prefill GEMM TFLOPS",
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": g["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights quantized to Q4_K, x ~ N(0,1))",
        "config": {"workload": "q4_k_gemv_4096x14336_m1", "n_in": n_in, "n_out": n_out,
                   "rows": 1, "activations": "f32", "weight_copies": g["copies"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(), "kernel": read_profile_field("bench_all_configs_kernel_trace.md", "headline_kernel"),
                     "algorithmic_bytes_per_launch": g["bytes"]},
        "cpu_baseline": cpu and {k: v for k, v in cpu.items()},
        "extras": extras,
    }
    print(json.dumps(line), flush=True)
    be32.close()
    be16.close()


if __name__ == "__main__":
    main()
