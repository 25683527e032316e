#!/usr/bin/env python3
"""Benchmark of the quantized `tgc batch` path on one MI355X.

Workload ("config 2"): a single int4 linear layer,
W 4096 x 4096 ~ N(0, 0.02) quantized per output channel (round to nearest
with the reference's clip search), run over batches of {1, 16, 256, 4096}
rows of f32[4096] ~ N(0, 1). One step = one pass over each of the four
batches (4369 rows), inputs already resident in device memory, outputs left
there. value = rows / second over the K timed steps (whole job, one GPU).

roofline: the dominant kernel is the int8-MFMA GEMM at batch 4096; its
average duration comes from HIP events on the backend's stream (a separate
program built with TG_HIP_TIMING), and achieved = 2*4096^3 algorithmic int8
ops (one multiply-add = 2 ops, counted once whatever the limb count) /
duration, against 5000 TOP/s dense int8. The "sweep" field repeats this per
batch. Every timed call there follows a pass, on the same stream, that
streams 1 GiB through HBM, so neither the 8 MiB weight nor the rows can be
served from the 256 MB Infinity Cache, and the device is never idle while
the host queues the next call (HIP events then time kernels, not launch
latency).

cpu_baseline: the reference's own interpreter (oracle/_ref/tgc_ref, compiled
from the reference sources) on this host's cores over a sample of rows of the
same layer; falls back to the oracle restatement when the reference build is
absent.
"""
import argparse
import json
import os
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

BATCHES = (1, 16, 256, 4096)
K = 4096
C = 4096
METRIC = "quantized rows/sec via tgc batch at 1 GPU; % of HBM / int8-MFMA roofline"
HBM_PEAK_GBS = 8000.0
MFMA_I8_PEAK_TOPS = 5000.0


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def flush_program(hip):
    """x * 2 over 2048 rows of 64 Ki floats: 512 MiB read + 512 MiB written."""
    text = ("(tgir 1\n  (model flush)\n  (param c (f32)\n    (data 2))\n  (input x (f32 65536))\n  (block\n"
            "    (%0 (f32 65536) (mul x c))\n  )\n  (output %0))\n")
    p = hip.Program(text, max_rows=2048)
    buf_in = hip.DeviceBuffer(2048 * 65536 * 4)
    buf_out = hip.DeviceBuffer(2048 * 65536 * 4)
    return p, buf_in, buf_out


def cpu_baseline(text, X, sample_rows, threads):
    from oracle import oracle as O
    tmp = tempfile.mkdtemp(prefix="tgbench")
    x = X[:sample_rows]
    if O.have_ref():
        mpath = os.path.join(tmp, "linear4096.tgir")
        with open(mpath, "w") as f:
            f.write(text)
        _, _, ms = O.ref_batch(mpath, x, K, C, 0, tmp, threads=threads)
        kind = "reference"
    else:
        m = O.Model(text)
        t0 = time.perf_counter()
        m.batch(x, threads=threads)
        ms = (time.perf_counter() - t0) * 1e3
        kind = "port"
    return {"value": sample_rows / (ms / 1e3), "unit": "rows/s", "cores": threads, "kind": kind,
            "sample": "%d rows of config 2 (int4 4096x4096) through the %s interpreter, -j %d, compute time only" % (
                sample_rows, "reference's" if kind == "reference" else "oracle's", threads)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-rows", type=int, default=96)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--reps", type=int, default=10, help="kernel-timing repetitions per batch")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this backend runs on one GPU per process and this build measures one GPU only; "
              "rows shard across GPUs with no collective (see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    from technograd_amd import hip, synth

    hip.init(0)
    log("building config 2 (int4 4096x4096)")
    W = synth.config2_weight()
    text = synth.linear_tgir("linear4096", W, 4)
    X = synth.normal(2, 1.0, 4096 * K).reshape(4096, K)
    log("loading programs")
    prog = hip.Program(text, max_rows=4096)
    tprog = hip.Program(text, flags=hip.TIMING, max_rows=4096)
    d_x = hip.DeviceBuffer.from_array(X)
    d_y = hip.DeviceBuffer(4096 * C * 4)

    # ---- whole-job throughput ----
    for _ in range(args.warmup):
        for b in BATCHES:
            prog.batch_device(d_x.ptr, b, d_y.ptr)
    prog.sync()
    log("timing %d steps" % args.steps)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        for b in BATCHES:
            prog.batch_device(d_x.ptr, b, d_y.ptr)
    prog.sync()
    elapsed = time.perf_counter() - t0
    rows_per_step = sum(BATCHES)
    value = rows_per_step * args.steps / elapsed
    y = d_y.to_array(np.float32, (4096, C))
    assert np.isfinite(y).all()

    # ---- kernel durations per batch (HIP events on the backend's stream) ----
    fprog, fin, fout = flush_program(hip)
    fprog.set_stream(tprog.stream())  # flush passes and timed calls in one queue
    wbytes = C * K / 2 + 4 * C
    sweep = []
    for b in BATCHES:
        tprog.batch_device(d_x.ptr, b, d_y.ptr)  # warm-up call (code, scratch)
        tprog.sync()
        tprog.reset_stats()
        for _ in range(args.reps):
            fprog.batch_device(fin.ptr, 2048, fout.ptr)
            tprog.batch_device(d_x.ptr, b, d_y.ptr)
        tprog.sync()
        st = tprog.stats()
        mfma_us = st.qgemm_ms / st.qgemm_calls * 1e3
        dig_us = st.digits_ms / max(st.qgemm_calls, 1) * 1e3
        ops = 2.0 * b * C * K
        byts = wbytes + 4.0 * b * (K + C)
        sweep.append({
            "batch": b, "mfma_kernel_us": round(mfma_us, 3), "digits_kernel_us": round(dig_us, 3),
            "alg_ops": ops, "alg_bytes": byts,
            "hbm_GBs": round(byts / (mfma_us + dig_us) / 1e3, 1),
            "hbm_frac": round(byts / (mfma_us + dig_us) / 1e3 / HBM_PEAK_GBS, 4),
            "mfma_TOPs": round(ops / mfma_us / 1e6, 2),
            "mfma_frac": round(ops / mfma_us / 1e6 / MFMA_I8_PEAK_TOPS, 4),
            "cold_infinity_cache": True,
        })
        log("batch %4d: mfma %.2f us, digits %.2f us" % (b, mfma_us, dig_us))
    big = sweep[-1]
    roofline = {"bound": "mfma", "achieved": big["mfma_TOPs"], "peak": MFMA_I8_PEAK_TOPS, "unit": "TOP/s",
                "frac": big["mfma_frac"], "traffic": None,
                "kernel": "qgemm_k<4> (int8 MFMA, 3 activation digits) at batch 4096",
                "alg_ops_per_launch": big["alg_ops"], "avg_kernel_us": big["mfma_kernel_us"]}

    cpu = None
    if not args.no_cpu:
        log("cpu baseline: %d rows, %d threads" % (args.cpu_rows, args.cpu_threads))
        cpu = cpu_baseline(text, X, args.cpu_rows, args.cpu_threads)

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "rows/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(elapsed / args.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) rows)",
        "config": {"workload": "config 2: int4 4096x4096 linear, one pass at each batch of {1,16,256,4096} rows per step",
                   "rows_per_step": rows_per_step, "parallelism": "1 GPU"},
        "roofline": roofline, "cpu_baseline": cpu, "sweep": sweep,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
