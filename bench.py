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
duration, against 5000 TOP/s dense int8; hw_mfma_frac = 3 x frac (three
int8 MFMAs per multiply-add). traffic = HBM bytes per launch of that kernel
from two rocprofv3 --pmc runs of this script's --profile-child mode
(FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by what the
counter reads for the 1 GiB flush pass (512 MiB read + 512 MiB written, an
elementwise kernel of known traffic) in the same run. roofline.matvec: the
int4 matvec at B = 1 and 16 against HBM, from a rocprofv3 kernel trace of
the same child (cold calls, each after a flush pass) and the same traffic
counters.

The "sweep" field repeats the kernel timings per batch: HIP events around
each kernel, and the kernel-trace durations. Every timed call follows a
pass, on the same stream, that reads 512 MiB of other data (a row sum: it
writes next to nothing, so no dirty lines are left to write back), so
neither the 8 MiB weight nor the rows can be served from the 256 MB
Infinity Cache, and the device is never idle while the host queues the next
call.

cpu_baseline: the reference's own interpreter (oracle/_ref/tgc_ref, compiled
from the reference sources) on this host's cores, -j auto (one thread per
CPU the process may run on), median of three runs over a sample of rows of
the same layer; value = compute time, wall_value = input load to last write;
falls back to the oracle restatement when the reference build is absent.

legs: config 1 (int8 MLP, 65,536 rows), config 4 (Q16.16 latent
reasoner, 1,048,576 rows), config 5 (selective SSM, 4096 sequences) and
config 3 (Qwen3-shaped decoder: 64 prompts of 512 tokens, 128 generated
tokens each), each with its own roofline (config 1: calibrated HBM traffic
of its GEMMs from rocprofv3 FETCH_SIZE and WRITE_SIZE; config 4: VALU
instructions from SQ_INSTS_VALU) and CPU baseline; a leg that fails is
reported as {"error": ...} in its place.
"""
import argparse
import csv
import glob
import json
import os
import shutil
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
FLUSH_ROWS, FLUSH_COLS = 2048, 65536  # the flush pass: x * c over 512 MiB in, 512 MiB out
FLOOR_BYTES = (C * K // 2 + 4 * C) // 16 * 16  # config 2's packed weight and scales, the matvec's main read


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def evict_program(hip):
    """sum over 2048 rows of 64 Ki floats: 512 MiB read, 8 KiB written. Run before each timed call of the
    sweep, it leaves the Infinity Cache holding clean lines of other data, so the timed kernel reads its
    operands from HBM without also paying for the write-back of another kernel's dirty lines."""
    text = ("(tgir 1\n  (model evict)\n  (input x (f32 %d))\n  (block\n"
            "    (%%0 (f32) (sum x))\n  )\n  (output %%0))\n" % FLUSH_COLS)
    p = hip.Program(text, max_rows=FLUSH_ROWS)
    buf_in = hip.DeviceBuffer(FLUSH_ROWS * FLUSH_COLS * 4)
    buf_out = hip.DeviceBuffer(FLUSH_ROWS * 4)
    return p, buf_in, buf_out


def flush_program(hip):
    """x * 2 over 2048 rows of 64 Ki floats: 512 MiB read + 512 MiB written."""
    text = ("(tgir 1\n  (model flush)\n  (param c (f32)\n    (data 2))\n  (input x (f32 %d))\n  (block\n"
            "    (%%0 (f32 %d) (mul x c))\n  )\n  (output %%0))\n" % (FLUSH_COLS, FLUSH_COLS))
    p = hip.Program(text, max_rows=FLUSH_ROWS)
    buf_in = hip.DeviceBuffer(FLUSH_ROWS * FLUSH_COLS * 4)
    buf_out = hip.DeviceBuffer(FLUSH_ROWS * FLUSH_COLS * 4)
    return p, buf_in, buf_out


def cpu_info():
    """The host's CPU count, the CPUs this process may run on and the CPU model."""
    model = None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpus_usable": len(os.sched_getaffinity(0)), "cpu_model": model}


def auto_threads():
    """`-j auto`: one thread per CPU this process may run on (the reference's
    par_init(0), src/par.c:84-92, takes the online CPUs; under a CPU set the
    usable ones are the ones that count)."""
    return len(os.sched_getaffinity(0))


def ref_unit_cpu(text, rows_q16, y_dev, steps_dev, nout, nthink, what, runs=3):
    """Q16.16: the reference's own `tgc c --fixed` unit (src/cgen.c, built
    into oracle/_ref/tgc_ref; the unit compiled cc -std=c99 -O2) over
    `rows_q16` on one thread, `runs` times: median rate from input read to last
    write. Its outputs and think steps are compared with the device's for the
    same rows (`matches_device`). Without the reference build: the threaded
    oracle restatement (ref_cpu)."""
    import numpy as np
    from oracle import oracle as O
    if not O.have_ref():
        return ref_cpu(text, rows_q16, rows_q16.shape[1], nout, nthink, auto_threads(), True, what, runs)
    tmp = tempfile.mkdtemp(prefix="tgbench")
    wall = []
    try:
        mpath = os.path.join(tmp, "model.tgir")
        with open(mpath, "w") as f:
            f.write(text)
        exe = O.ref_unit_build(mpath, tmp)
        d = os.path.dirname(exe)
        inp, outp, stp = (os.path.join(d, n) for n in ("in.bin", "out.bin", "steps.bin"))
        np.ascontiguousarray(rows_q16, dtype="<i4").tofile(inp)
        for _ in range(runs):
            t0 = time.perf_counter()
            subprocess.run([exe, inp, outp, stp], check=True, capture_output=True)
            wall.append((time.perf_counter() - t0) * 1e3)
        out = np.fromfile(outp, dtype="<i4").reshape(-1, nout)
        stq = np.fromfile(stp, dtype="<i4").reshape(-1, max(nthink, 1))
        same = bool(np.array_equal(out, y_dev) and np.array_equal(stq[:, 0], steps_dev))
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    wm = sorted(wall)[len(wall) // 2]
    out = {"value": round(len(rows_q16) / (wm / 1e3), 1), "unit": "rows/s", "cores": 1, "kind": "reference",
           "runs": runs, "wall_ms": [round(v, 2) for v in wall], "matches_device": same,
           "sample": "%d rows of %s through the reference's own `tgc c --fixed` unit (emitted by src/cgen.c, compiled "
                     "cc -std=c99 -O2; the unit is single-threaded), median of %d runs from input read to last write"
                     % (len(rows_q16), what, runs)}
    out.update(cpu_info())
    return out


def ref_cpu(text, rows, per, nout, nthink, threads, fixed, what, runs=3):
    """The reference interpreter (oracle/_ref/tgc_ref, built from the
    reference's sources; the oracle restatement if that build is absent) over
    `rows`, `runs` times: median compute and wall (input load to last write)
    rates."""
    from oracle import oracle as O
    tmp = tempfile.mkdtemp(prefix="tgbench")
    comp, wall = [], []
    try:
        if O.have_ref():
            mpath = os.path.join(tmp, "model.tgir")
            with open(mpath, "w") as f:
                f.write(text)
            for _ in range(runs):
                _, _, ms, wms = O.ref_batch(mpath, rows, per, nout, nthink, tmp, threads=threads, fixed=fixed, wall=True)
                comp.append(ms)
                wall.append(wms)
            kind = "reference"
        else:
            m = O.Model(text)
            for _ in range(runs):
                t0 = time.perf_counter()
                (m.batch_fixed if fixed else m.batch)(rows, threads=threads)
                comp.append((time.perf_counter() - t0) * 1e3)
                wall.append(comp[-1])
            kind = "port"
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    cm, wm = sorted(comp)[len(comp) // 2], sorted(wall)[len(wall) // 2]
    out = {"value": round(len(rows) / (cm / 1e3), 1), "unit": "rows/s", "cores": threads, "kind": kind,
           "wall_value": round(len(rows) / (wm / 1e3), 1), "runs": runs,
           "compute_ms": [round(v, 2) for v in comp], "wall_ms": [round(v, 2) for v in wall],
           "sample": "%d rows of %s through the %s interpreter, -j auto (%d threads), median of %d runs; value = "
                     "compute time, wall_value = input load to last write" % (
                         len(rows), what, "reference's" if kind == "reference" else "oracle's", threads, runs)}
    out.update(cpu_info())
    return out


def cli_batch_wall(text, rows, what, runs=3):
    """`bin/tgc-hip batch MODEL rows.bin -o out.bin -v` as a user runs it, on
    `rows` written to a raw f32 file: the driver's own timer (input load to
    last write, the reference's `batch` timer, src/main.c:413-443) and the
    process wall time (start to exit, model load and device set-up
    included), medians of `runs` runs."""
    import re
    import numpy as np
    cli = os.path.join(ROOT, "technograd_amd", "bin", "tgc-hip")
    if not os.path.exists(cli):
        return None
    tmp = tempfile.mkdtemp(prefix="tge2e")
    try:
        mpath, rpath, opath = (os.path.join(tmp, n) for n in ("model.tgir", "rows.bin", "out.bin"))
        with open(mpath, "w") as f:
            f.write(text)
        np.ascontiguousarray(rows, np.float32).tofile(rpath)
        timer, wall = [], []
        for _ in range(runs):
            t0 = time.perf_counter()
            r = subprocess.run([cli, "batch", mpath, rpath, "-o", opath, "-v", "--rows", str(len(rows))],
                               capture_output=True, text=True, timeout=300)
            wall.append((time.perf_counter() - t0) * 1e3)
            m = re.search(r"row\(s\) in ([0-9.]+) ms", r.stderr)
            if r.returncode or not m:
                log("tgc-hip batch failed (rc %d): %s" % (r.returncode, r.stderr[-300:]))
                return None
            timer.append(float(m.group(1)))
        tm, wm = sorted(timer)[len(timer) // 2], sorted(wall)[len(wall) // 2]
        n = len(rows)
        log("tgc-hip batch, %s: %.2f ms input load to last write (%.0f rows/s), %.0f ms process wall" % (what, tm, n / tm * 1e3, wm))
        return {"rows": n, "ms": round(tm, 2), "rows_per_s": round(n / tm * 1e3, 1), "process_wall_ms": round(wm, 1),
                "runs": runs, "files": "raw f32 rows in, raw f32 outputs out (%d MiB + %d MiB), in %s" % (
                    rows.nbytes >> 20, os.path.getsize(opath) >> 20, tempfile.gettempdir()),
                "note": "bin/tgc-hip batch MODEL rows.bin -o out.bin -v --rows N: ms = the driver's timer from before "
                        "the input load to after the last write (the reference's batch timer); rows_per_s from it, "
                        "the measure of cpu_baseline.wall_value"}
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def setup(synth):
    W = synth.config2_weight()
    text = synth.linear_tgir("linear4096", W, 4)
    X = synth.normal(2, 1.0, 4096 * K).reshape(4096, K)
    return text, X


def profile_child(mode):
    """What the profiled runs see. c2: each batch of BATCHES called twice,
    every call after a flush pass (512 MiB read and written) on the same
    stream, so each call reads its weight from HBM and the flush kernels
    split the dispatches into one segment per call. c4: two passes of
    config 4, each after a flush pass."""
    from technograd_amd import hip, synth
    hip.init(0)
    fprog, fin, fout = None, None, None
    if mode == "c1":
        text, X = synth.config1(65536)
        prog = hip.Program(text, max_rows=65536)
        d_x = hip.DeviceBuffer.from_array(X)
        d_y = hip.DeviceBuffer(65536 * 512 * 4)
        calls = [(65536, lambda: prog.batch_device(d_x.ptr, 65536, d_y.ptr))] * 2
    elif mode == "c5":
        import numpy as np
        seqs, T = C5_PROFILE_SEQS, 512
        prog = hip.Program(synth.ssm_tgir("ssm"), max_rows=seqs)
        d_x = hip.DeviceBuffer.from_array(synth.config5_rows(seqs, T, 256))
        d_y = hip.DeviceBuffer(seqs * 8 * 4)
        calls = [(seqs, lambda: prog.batch_device(d_x.ptr, seqs, d_y.ptr))] * 2
    elif mode == "c2":
        text, X = setup(synth)
        prog = hip.Program(text, max_rows=4096)
        d_x = hip.DeviceBuffer.from_array(X)
        d_y = hip.DeviceBuffer(4096 * C * 4)
        calls = [(b, lambda b=b: prog.batch_device(d_x.ptr, b, d_y.ptr)) for b in BATCHES] * 2
        # the read floor: a plain read of a span the size of the packed weight, cold like the calls
        span = hip.DeviceBuffer(FLOOR_BYTES)
        calls += [("floor", lambda: hip.read_pass(span.ptr, FLOOR_BYTES, 2048, prog.stream()))] * 2
        # and at the single-row kernel's launch shape (256 workgroups of 256 threads)
        calls += [("floor256", lambda: hip.read_pass(span.ptr, FLOOR_BYTES, 256, prog.stream()))] * 2
    else:
        import numpy as np
        rows = 1048576
        prog = hip.Program(synth.latent_reasoner_tgir(), flags=hip.FIXED, max_rows=rows)
        d_x = hip.DeviceBuffer.from_array((synth.config4_rows(rows) * 65536.0).astype(np.int32))
        d_y, d_s = hip.DeviceBuffer(rows * 16), hip.DeviceBuffer(rows * 4)
        calls = [(rows, lambda: prog.batch_device(d_x.ptr, rows, d_y.ptr, d_s.ptr))] * 2
    fprog, fin, fout = flush_program(hip)
    fprog.set_stream(prog.stream())
    warmed = set()
    for lab, call in calls:  # each kind of call once before the profiled ones (before the first flush: not
        if lab not in warmed:  # counted), so first-launch costs stay out of the cold calls
            warmed.add(lab)
            call()
    for _, call in calls:
        fprog.batch_device(fin.ptr, FLUSH_ROWS, fout.ptr)
        call()
    prog.sync()


def _short(name):
    return name.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]


def _is_flush(name, grid):
    return "binary" in name and grid >= FLUSH_ROWS * FLUSH_COLS // 16


def profiled(tool_args, mode, outdir, tag):
    """Dispatches of a profiled --profile-child run, in order, split at each
    flush kernel: [[(kernel, grid, {field: value})...] per call], and the
    flush kernels' records. None if the run failed."""
    d = os.path.join(outdir, tag)
    cmd = ["rocprofv3"] + tool_args + ["--output-format", "csv", "-d", d, "-o", "p", "--",
                                       sys.executable, os.path.abspath(__file__), "--profile-child", mode]
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=170, env=env, cwd=ROOT)
    pmc = "--pmc" in tool_args
    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv" if pmc else "*kernel_trace.csv"), recursive=True)
    if not files:
        log("rocprofv3 %s failed (rc %d): %s" % (" ".join(tool_args), r.returncode, r.stdout.decode(errors="replace")[-400:]))
        return None
    disp = {}
    for f in files:
        with open(f) as fh:
            for row in csv.DictReader(fh):
                did = int(row.get("Dispatch_Id") or row.get("Correlation_Id") or len(disp))
                e = disp.setdefault(did, {"name": row["Kernel_Name"],
                                          "grid": int(row.get("Grid_Size") or row.get("Grid_Size_X") or 0), "v": {}})
                if pmc:
                    e["v"][row["Counter_Name"]] = e["v"].get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
                else:
                    e["v"]["us"] = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3
    segs, flushes = [], []
    for did in sorted(disp):
        e = disp[did]
        if _is_flush(e["name"], e["grid"]):
            flushes.append(e)
            segs.append([])
        elif segs:
            segs[-1].append((_short(e["name"]), e["grid"], e["v"]))
    return segs, flushes


def calibrated_traffic(fetch, write):
    """Per-call HBM bytes from a FETCH_SIZE and a WRITE_SIZE run (KiB per
    dispatch), each scaled by what the counter reads for the flush pass
    (512 MiB read and 512 MiB written): [(bytes per call, per-kernel bytes)]
    and the two factors."""
    half = FLUSH_ROWS * FLUSH_COLS * 4
    rf = half / (sum(e["v"]["FETCH_SIZE"] for e in fetch[1]) / len(fetch[1]) * 1024.0)
    rw = half / (sum(e["v"]["WRITE_SIZE"] for e in write[1]) / len(write[1]) * 1024.0)
    out = []
    for sf, sw in zip(fetch[0], write[0]):
        per = {}
        for (n, _, vf), (_, _, vw) in zip(sf, sw):
            per[n] = per.get(n, 0.0) + vf["FETCH_SIZE"] * 1024.0 * rf + vw["WRITE_SIZE"] * 1024.0 * rw
        out.append((sum(per.values()), per))
    return out, rf, rw


def profile_c2(alg_bytes):
    """Cold kernel durations (kernel trace) and calibrated HBM traffic per
    batch of config 2: {batch: {"kernels_us": {...}, "us": total, "traffic":
    bytes, "traffic_kernels": {...}}}, and a note."""
    if not shutil.which("rocprofv3"):
        return None, "rocprofv3 not found"
    out = tempfile.mkdtemp(prefix="tgprof")
    try:
        kt = profiled(["--kernel-trace"], "c2", out, "kt")
        fe = profiled(["--pmc", "FETCH_SIZE"], "c2", out, "fetch") if kt else None
        wr = profiled(["--pmc", "WRITE_SIZE"], "c2", out, "write") if fe else None
    except subprocess.TimeoutExpired:
        return None, "rocprofv3 timed out"
    finally:
        shutil.rmtree(out, ignore_errors=True)
    nb = 2 * len(BATCHES)
    if not kt or len(kt[0]) != nb + 4:
        return None, "kernel trace: %s segments" % (None if not kt else len(kt[0]))
    res = {b: {"kernels_us": {}} for b in BATCHES}
    for key, segs in (("floor", kt[0][nb:nb + 2]), ("floor256", kt[0][nb + 2:])):
        fl = [v["us"] for seg in segs for _, _, v in seg]
        res[key] = {"us": round(sum(fl) / max(len(fl), 1), 3), "bytes": FLOOR_BYTES}
    for i, seg in enumerate(kt[0][:nb]):  # two calls per batch: averages
        r = res[BATCHES[i % len(BATCHES)]]
        for n, _, v in seg:
            r["kernels_us"][n] = r["kernels_us"].get(n, 0.0) + v["us"] / 2
    for b in BATCHES:
        r = res[b]
        r["kernels_us"] = {k: round(v, 3) for k, v in r["kernels_us"].items()}
        r["us"] = round(sum(r["kernels_us"].values()), 3)
    note = "kernel trace of two cold calls per batch"
    if fe and wr and len(fe[0]) == len(wr[0]) == nb + 4:
        tr, rf, rw = calibrated_traffic(fe, wr)
        res["floor"]["traffic"] = round(sum(t for t, _ in tr[nb:nb + 2]) / 2)
        res["floor256"]["traffic"] = round(sum(t for t, _ in tr[nb + 2:]) / 2)
        for i, (tot, per) in enumerate(tr[:nb]):
            r = res[BATCHES[i % len(BATCHES)]]
            r["traffic"] = r.get("traffic", 0.0) + tot / 2
            tk = r.setdefault("traffic_kernels", {})
            for k, v in per.items():
                tk[k] = tk.get(k, 0.0) + v / 2
        note += "; traffic = FETCH_SIZE x %.4f + WRITE_SIZE x %.4f (factors: 512 MiB / the flush pass's reading)" % (rf, rw)
    else:
        note += "; traffic counters gave no data"
    return res, note


def profile_pass(mode):
    """Calibrated HBM traffic of one pass of a --profile-child mode that runs
    two passes, each after a flush pass (FETCH_SIZE and WRITE_SIZE of every
    dispatch, averaged over the two): {kernel: bytes per pass}, or None."""
    if not shutil.which("rocprofv3"):
        return None
    out = tempfile.mkdtemp(prefix="tgprof")
    try:
        fe = profiled(["--pmc", "FETCH_SIZE"], mode, out, "fetch")
        wr = profiled(["--pmc", "WRITE_SIZE"], mode, out, "write") if fe else None
    except subprocess.TimeoutExpired:
        return None
    finally:
        shutil.rmtree(out, ignore_errors=True)
    if not fe or not wr or len(fe[0]) != 2 or len(wr[0]) != 2:
        return None
    tr, _, _ = calibrated_traffic(fe, wr)
    per = {}
    for _, kern in tr:
        for k, v in kern.items():
            per[k] = per.get(k, 0.0) + v / 2
    return per


# config 1's algorithmic bytes per pass (the measure of the reference's
# metric): rows in, rows out, the int8 weights and their scales once
C1_ALG_BYTES = 4 * 65536 * (512 + 512) + (2048 * 512 + 2048 * 2048 + 512 * 2048) + 4 * (2048 + 2048 + 512)


def config1_leg(args, steps=None, profile=True):
    """Config 1: int8 MLP 512 -> 2048 -> 2048 -> 512 (tanh, tanh, rmsnorm), 65,536
    rows in one device pass. roofline: the three quantized GEMMs, 12.58 M
    algorithmic ops per row, against 5000 TOP/s dense int8."""
    import numpy as np
    from technograd_amd import hip, synth
    rows = 65536
    hip.init(0)
    log("building config 1 (int8 MLP, %d rows)" % rows)
    text, X = synth.config1(rows)
    prog = hip.Program(text, max_rows=rows)
    tprog = hip.Program(text, flags=hip.TIMING, max_rows=rows)
    d_x = hip.DeviceBuffer.from_array(X)
    d_y = hip.DeviceBuffer(rows * 512 * 4)
    for _ in range(args.warmup):
        prog.batch_device(d_x.ptr, rows, d_y.ptr)
    prog.sync()
    steps = steps or max(1, min(args.steps, 10))
    t0 = time.perf_counter()
    for _ in range(steps):
        prog.batch_device(d_x.ptr, rows, d_y.ptr)
    prog.sync()
    elapsed = time.perf_counter() - t0
    y = d_y.to_array(np.float32, (rows, 512))
    assert np.isfinite(y).all()
    tprog.batch_device(d_x.ptr, rows, d_y.ptr)
    tprog.sync()
    tprog.reset_stats()
    for _ in range(3):
        tprog.batch_device(d_x.ptr, rows, d_y.ptr)
    tprog.sync()
    st = tprog.stats()
    mfma_us, dig_us, oth_us = (v / 3 * 1e3 for v in (st.qgemm_ms, st.digits_ms, st.other_ms))
    ops = 2.0 * (2048 * 512 + 2048 * 2048 + 512 * 2048) * rows
    alg_bytes = C1_ALG_BYTES  # rows in + rows out + weights once: 274.7 MB per pass
    log("config 1: %.2f ms per pass: GEMMs %.0f us, digits %.0f us, other %.0f us" % (
        elapsed / steps * 1e3, mfma_us, dig_us, oth_us))
    cpu = None if args.no_cpu else ref_cpu(text, X[:2048], 512, 512, 0, auto_threads(), False,
                                           "config 1 (int8 MLP 512-2048-2048-512)")
    frac = ops / mfma_us / 1e6 / MFMA_I8_PEAK_TOPS
    e2e = None if getattr(args, "no_e2e", False) else cli_batch_wall(text, X, "config 1 (int8 MLP, 65,536 rows)")
    per = profile_pass("c1") if profile else None
    traffic = None if per is None else sum(v for k, v in per.items() if k.startswith("qgemm_k"))
    traffic_pass = None if per is None else sum(per.values())
    pass_us = elapsed / steps * 1e6
    return {
        "metric": "config 1 int8 MLP rows/sec at 1 GPU; % of int8-MFMA roofline", "value": round(rows * steps / elapsed, 1),
        "unit": "rows/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(elapsed / steps * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "W8A32", "data": "synthetic (rand(1, 0.05) weights quantized int8 RTN, N(0,1) rows seed 0)",
        "config": {"workload": "config 1: int8 MLP 512-2048-2048-512, tanh, rmsnorm; 65,536 rows per step"},
        "roofline": {"bound": "mfma", "achieved": round(ops / mfma_us / 1e6, 2), "peak": MFMA_I8_PEAK_TOPS,
                     "unit": "TOP/s", "frac": round(frac, 4), "traffic": None if traffic is None else round(traffic),
                     "traffic_note": "calibrated FETCH_SIZE + WRITE_SIZE of the pass's qgemm_k dispatches (rocprofv3); "
                                     "traffic_pass: of every dispatch of the pass" if traffic is not None else
                                     ("not profiled (--no-traffic)" if not profile else "rocprofv3 gave no data"),
                     "alg_bytes_per_pass": alg_bytes,
                     "alg_bytes_note": "rows in + rows out + int8 weights and scales once (65,536 x 512 f32 each way)",
                     "traffic_pass": None if traffic_pass is None else round(traffic_pass),
                     "traffic_ratio": None if traffic is None else round(traffic / alg_bytes, 2),
                     "traffic_pass_ratio": None if traffic_pass is None else round(traffic_pass / alg_bytes, 2),
                     "traffic_kernels": None if per is None else {k: round(v) for k, v in sorted(per.items())},
                     "hbm_view": {"achieved": round(alg_bytes / pass_us / 1e3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": round(alg_bytes / pass_us / 1e3 / HBM_PEAK_GBS, 4),
                                  "note": "algorithmic bytes over the whole pass's time"},
                     "limb_factor": 3, "hw_mfma_frac": round(3 * frac, 4),
                     "kernel": "the three quantized GEMMs of a pass (qgemm_k<8>), summed",
                     "alg_ops_per_launch": ops, "avg_kernel_us": round(mfma_us, 1)},
        "cpu_baseline": cpu,
        "breakdown_us": {"gemm": round(mfma_us, 1), "digits": round(dig_us, 1), "other": round(oth_us, 1)},
        "end_to_end": e2e,
    }


def bench_config1(args):
    print(json.dumps(config1_leg(args, profile=not args.no_traffic)), flush=True)


VALU_PEAK_GINST = 256 * 2.4  # wave64 VALU instructions per ns: one per CU per clock (4 SIMDs, 4 clocks each), 2.4 GHz


# config 4's row kernel: compiled for the model at load time, or the interpreter
C4_KERNELS = ("tg_rowprog_model", "rowprog_k")


def profile_c4():
    """config 4's row kernel under rocprofv3: cold kernel duration (kernel
    trace) and VALU instructions per dispatch (SQ_INSTS_VALU), averaged over
    two passes; (us, insts) or (None, None)."""
    if not shutil.which("rocprofv3"):
        return None, None
    out = tempfile.mkdtemp(prefix="tgprof")
    try:
        kt = profiled(["--kernel-trace"], "c4", out, "kt")
        pm = profiled(["--pmc", "SQ_INSTS_VALU", "SQ_BUSY_CYCLES"], "c4", out, "valu") if kt else None
    except subprocess.TimeoutExpired:
        return None, None
    finally:
        shutil.rmtree(out, ignore_errors=True)
    if not kt or not pm:
        return None, None
    us = [v["us"] for seg in kt[0] for n, _, v in seg if n.startswith(C4_KERNELS)]
    ins = [v.get("SQ_INSTS_VALU", 0.0) for seg in pm[0] for n, _, v in seg if n.startswith(C4_KERNELS)]
    return (sum(us) / len(us) if us else None), (sum(ins) / len(ins) if ins else None)


def config4_leg(args, steps=None, profile=True):
    """Config 4: the Q16.16 latent reasoner (think <= 32 steps, halting at
    d <= 7) over 1,048,576 rows of {0, 1}^8, one device pass. Integer VALU
    work: the roofline is VALU instruction issue (rocprofv3 SQ_INSTS_VALU
    over the kernel's duration) against one wave64 instruction per CU per
    clock; the HBM fraction is shown beside it."""
    import numpy as np
    from technograd_amd import hip, synth
    rows = 1048576
    hip.init(0)
    log("building config 4 (Q16.16 latent reasoner, %d rows)" % rows)
    text = synth.latent_reasoner_tgir()
    X = synth.config4_rows(rows)
    xq = (X * 65536.0).astype(np.int32)  # inputs are 0 or 1: exact in Q16.16
    prog = hip.Program(text, flags=hip.FIXED, max_rows=rows)
    pst = prog.stats()
    kname = "tg_rowprog_model (the row program compiled for the model, %d instructions hoisted out of the think loop)" % \
        pst.rowprog_hoisted if pst.rowprog_jit else "rowprog_k<true> (the row-program interpreter)"
    d_x = hip.DeviceBuffer.from_array(xq)
    d_y = hip.DeviceBuffer(rows * 4 * 4)
    d_s = hip.DeviceBuffer(rows * 4)
    for _ in range(args.warmup):
        prog.batch_device(d_x.ptr, rows, d_y.ptr, d_s.ptr)
    prog.sync()
    steps = steps or max(1, min(args.steps, 10))
    t0 = time.perf_counter()
    for _ in range(steps):
        prog.batch_device(d_x.ptr, rows, d_y.ptr, d_s.ptr)
    prog.sync()
    elapsed = time.perf_counter() - t0
    st = d_s.to_array(np.int32, (rows,))
    byts = rows * (8 * 4 + 4 * 4 + 4)
    t = elapsed / steps
    log("config 4: %.2f ms per pass, mean think steps %.2f" % (t * 1e3, st.mean()))
    kus, ins = profile_c4() if profile else (None, None)
    if kus and ins:
        roof = {"bound": "valu", "achieved": round(ins / kus / 1e3, 2), "peak": VALU_PEAK_GINST, "unit": "Ginst/s",
                "frac": round(ins / kus / 1e3 / VALU_PEAK_GINST, 4), "traffic": None,
                "valu_insts_per_launch": ins, "avg_kernel_us": round(kus, 1),
                "hbm_frac": round(byts / (kus * 1e-6) / 1e9 / HBM_PEAK_GBS, 5),
                "kernel": kname + "; one lane per row; wave64 VALU instructions per second from rocprofv3 "
                          "SQ_INSTS_VALU over the kernel-trace duration, peak one per CU per clock at 2.4 GHz"}
    else:
        roof = {"bound": "valu", "achieved": None, "peak": VALU_PEAK_GINST, "unit": "Ginst/s", "frac": None,
                "traffic": None, "hbm_frac": round(byts / t / 1e9 / HBM_PEAK_GBS, 5),
                "kernel": kname + (": rocprofv3 gave no data" if profile else ": not profiled (--no-traffic)")}
    cpu = None
    if not args.no_cpu:
        y = d_y.to_array(np.int32, (rows, 4))
        cpu = ref_unit_cpu(text, xq[:131072], y[:131072], st[:131072], 4, 1, "config 4 (Q16.16 latent reasoner)")
    return {
        "metric": "config 4 Q16.16 latent reasoner rows/sec at 1 GPU", "value": round(rows / t, 1), "unit": "rows/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup, "ms_per_step": round(t * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q16.16 (int32, int64 products)",
        "data": "synthetic (rows uniform in {0,1}^8, seed 4)",
        "config": {"workload": "config 4: latent reasoner, think <= 32 steps, 1,048,576 rows per step",
                   "mean_think_steps": round(float(st.mean()), 3)},
        "roofline": roof,
        "cpu_baseline": cpu,
    }


def bench_config4(args):
    print(json.dumps(config4_leg(args)), flush=True)


def q3_macs_per_token(L=28, D=1024, NQ=16, NKV=8, HD=128, FF=3072, T=512):
    """Quantized-projection MACs per prompt token of config 3 (all layers):
    q, k, v, o, gate, up, down and the RoPE rotations (x @ Rot per q and k
    head); the attention products and the LM head are counted apart."""
    per_layer = D * NQ * HD + 2 * D * NKV * HD + NQ * HD * D + 3 * D * FF + (NQ + NKV) * HD * HD
    return L * per_layer


def bench_config3(args):
    print(json.dumps(config3_leg(args)), flush=True)


def config3_leg(args):
    """Config 3, prefill: the Qwen3-0.6B-shaped int4 decoder at fixed T = 512
    over 64 prompts of uniform token ids, one device pass; each sequence's
    output is its last position's 151,936 logits (the importer's graph,
    examples/qwen3/import.py:129-130). Throughput = prompt tokens per second.
    roofline: the int4 projections (q3_macs_per_token x 2 ops per token)
    against 5000 TOP/s dense int8 MFMA. cpu_baseline: the reference at 1 and
    2 layers (full widths, T = 512, a 2048-token vocabulary), extrapolated to
    28 layers and the full LM head (the full model is hours of CPU time)."""
    import numpy as np
    from technograd_amd import hip, synth
    seqs, T, V, GEN = 64, 512, 151936, 128
    hip.init(0)
    tmp = tempfile.mkdtemp(prefix="tgq3")
    try:
        log("building config 3 (Qwen3-0.6B-shaped int4 decoder, %d prompts x %d tokens)" % (seqs, T))
        t0 = time.perf_counter()
        text = synth.qwen3_tgir("qwen3", T=T, files=tmp, quantizer=hip.quantize_rtn, rope_len=T + GEN)
        X = synth.config3_prompts(seqs, T, V)
        log("config 3: weights written in %.0f s; loading" % (time.perf_counter() - t0))
        t0 = time.perf_counter()
        prog = hip.Program(text, max_rows=seqs)
        log("config 3: loaded in %.0f s, %.1f MiB of arena per sequence" % (time.perf_counter() - t0,
                                                                          prog.stats().arena_bytes / seqs / 2**20))
        d_x = hip.DeviceBuffer.from_array(X)
        d_y = hip.DeviceBuffer(seqs * V * 4)
        prog.batch_device(d_x.ptr, seqs, d_y.ptr)
        prog.sync()
        steps = max(1, min(args.steps, 3))
        t0 = time.perf_counter()
        for _ in range(steps):
            prog.batch_device(d_x.ptr, seqs, d_y.ptr)
        prog.sync()
        t = (time.perf_counter() - t0) / steps
        y = d_y.to_array(np.float32, (seqs, V))
        assert np.isfinite(y).all()
        log("config 3: %.1f ms per pass of %d x %d tokens; first sequences' next tokens %s"
            % (t * 1e3, seqs, T, y[:4].argmax(axis=1).tolist()))
        # generation: prefill, then GEN greedy tokens per sequence with the KV cache
        dec = hip.Decoder(prog, seqs, T, T + GEN)
        d_tok = hip.DeviceBuffer(seqs * GEN * 4)
        dec.generate_device(d_x, seqs, T, 2, d_tok)
        prog.sync()
        t0 = time.perf_counter()
        dec.generate_device(d_x, seqs, T, 1, d_tok)
        prog.sync()
        t_pre = time.perf_counter() - t0
        t0 = time.perf_counter()
        dec.generate_device(d_x, seqs, T, GEN, d_tok)
        prog.sync()
        t_gen = time.perf_counter() - t0
        tok = d_tok.to_array(np.int32, (seqs, GEN))
        # every sequence's first generated token is the fixed-length forward's 151,936-way argmax (the same logits,
        # bit for bit, through the decoder's own kernels: the KV-cache prefill)
        first_same = int((tok[:, 0] == y.argmax(axis=1)).sum())
        assert first_same == seqs, (first_same, seqs)
        distinct = float(np.mean([len(set(r.tolist())) for r in tok]))
        log("config 3: generation %.1f ms (prefill %.1f ms, %d decode steps %.1f ms); sequence 0 starts %s"
            % (t_gen * 1e3, t_pre * 1e3, GEN - 1, (t_gen - t_pre) * 1e3, tok[0, :8].tolist()))
        dec.close()
        prog.close()
        tprog = hip.Program(text, flags=hip.TIMING, max_rows=seqs)
        tprog.batch_device(d_x.ptr, seqs, d_y.ptr)
        tprog.sync()
        st = tprog.stats()
        tprog.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    mfma_us, dig_us, oth_us = (v * 1e3 for v in (st.qgemm_ms, st.digits_ms, st.other_ms))
    ops = 2.0 * q3_macs_per_token() * seqs * T
    log("config 3: projections %.0f us, digits %.0f us, other (attention, norms, elementwise) %.0f us"
        % (mfma_us, dig_us, oth_us))
    # decode steps read every packed weight once (int4 codes + scales) and the K and V cache up to their position
    layer_params = 1024 * 16 * 128 + 2 * 1024 * 8 * 128 + 16 * 128 * 1024 + 3 * 1024 * 3072
    wbytes = (28 * layer_params + 128 * 128 + 1024 * V) / 2.0 + 4.0 * (28 * (4096 + 16 * 1024 + 6144 + 1024) + 128 + V)
    kv = sum(seqs * (T + s) * 28 * 2 * 8 * 128 * 4.0 for s in range(1, GEN))
    dec_bytes = (GEN - 1) * wbytes + kv
    dec_s = t_gen - t_pre
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        if O.have_ref():
            cs = 16
            Xs = synth.config3_prompts(cs, T, 2048, seed=33)
            secs = []
            for L in (1, 2):
                log("config 3: cpu baseline, the reference at %d layer(s)" % L)
                tx = synth.qwen3_tgir("q3cpu", L=L, V=2048, T=T)
                r = ref_cpu(tx, Xs, T, 2048, 0, auto_threads(), False, "", runs=1)
                secs.append(cs / r["value"])
            layer = secs[1] - secs[0]
            rest = secs[0] - layer  # embedding and the 2048-column LM head
            full = 28 * layer + rest * V / 2048.0
            cpu = {"value": round(cs * T / full, 2), "unit": "prompt tokens/s", "cores": auto_threads(),
                   "kind": "reference",
                   "sample": "%d prompts x %d tokens through the reference's interpreter at 1 and 2 layers (full widths, "
                             "vocabulary 2048, -j %d): %.1f s per added layer, %.1f s for the rest; extrapolated to 28 "
                             "layers and the 151,936-column LM head: %.0f s for the %d prompts"
                             % (cs, T, auto_threads(), layer, rest, full, cs)}
            cpu.update(cpu_info())
    out = {
        "metric": "config 3 generated tokens/sec at 1 GPU (64 sequences: 512-token prompt, 128 greedy tokens)",
        "value": round(seqs * GEN / t_gen, 1), "unit": "generated tokens/s", "n_gpus": 1, "steps": 1, "warmup": 1,
        "ms_per_step": round(t_gen * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int4 projections, f32 attention and KV cache",
        "data": "synthetic (N(0,0.02) weights seed 3 quantized int4 RTN per channel, token ids uniform seed 3)",
        "config": {"workload": "config 3: Qwen3-0.6B-shaped decoder (28 layers, hidden 1024, 16/8 heads of 128, SwiGLU "
                               "3072, vocab 151,936); one step = prefill of 64 prompts x 512 tokens + 127 KV-cache "
                               "decode steps (128 greedy tokens per sequence)",
                   "prefill_ms": round(t_pre * 1e3, 2), "decode_ms": round(dec_s * 1e3, 2),
                   "prefill_prompt_tokens_per_s": round(seqs * T / t_pre, 1),
                   "fixed_length_forward_ms": round(t * 1e3, 3),
                   "first_token_equals_forward_argmax": "%d of %d sequences" % (first_same, seqs),
                   "distinct_tokens_per_sequence_mean": round(distinct, 1)},
        "roofline": {"bound": "hbm", "achieved": round(dec_bytes / dec_s / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(dec_bytes / dec_s / 8e12, 4), "traffic": None,
                     "kernel": "the decode steps, summed: every packed weight once per step plus the K and V cache up to "
                               "the step's position (%.1f GB in all)" % (dec_bytes / 1e9),
                     "prefill_projections": {"bound": "mfma", "achieved_TOPs": round(ops / mfma_us / 1e6, 2),
                                             "frac": round(ops / mfma_us / 1e6 / MFMA_I8_PEAK_TOPS, 4)}},
        "cpu_baseline": cpu,
        "breakdown_us": {"projections": round(mfma_us, 1), "digits": round(dig_us, 1), "other": round(oth_us, 1)},
    }
    d_x.free()
    d_y.free()
    return out


C5_PROFILE_SEQS = 256  # sequences of the profiled config 5 pass
# the dispatches that make config 5's projections: digit kernels and the resolves after them, quantized GEMMs
# and matvecs, and the short products (16 inputs: the dt projection) on the reference's loop; the timers count all
# of them as projections or their digits
C5_PROJ_KERNELS = ("qgemm_k", "qgemv_k", "qtiny_k", "digits_", "resolve_k")


def c5_alg_bytes(seqs, T=512, dm=256, di=512, ns=16, dtr=16, blocks=4):
    """Config 5's projection bytes: per block and time step the inputs read
    once (x, u, the dt-rank vector, the gated SSM output) and the outputs
    written once (xi, z, the dt-rank vector, B, C, dt, the block output), f32;
    the int8 weights and their scales once."""
    per_step = 4 * ((dm + di + dtr + di) + (di + di + dtr + ns + ns + di + dm))
    weights = blocks * (2 * dm * di + 2 * di * dtr + 2 * di * ns + di * dm) + 4 * blocks * (2 * di + dtr + 2 * ns + di + dm)
    return blocks * seqs * T * per_step + weights


def bench_config5(args):
    print(json.dumps(config5_leg(args)), flush=True)


def config5_leg(args):
    """Config 5: int8 selective-SSM classifier (4 blocks, d_model 256, state 16,
    expand 2, T = 512) over 4096 sequences in device passes of `pass_rows`
    sequences. roofline: the int8 projections, 2 x 426 K MACs per step per
    block, against 5000 TOP/s (the f32 scan runs on the VALU)."""
    import numpy as np
    from technograd_amd import hip, synth
    rows, T, dm = 4096, 512, 256
    per = T * dm
    hip.init(0)
    log("building config 5 (selective SSM, %d sequences of %d x %d)" % (rows, T, dm))
    text = synth.ssm_tgir("ssm")
    X = synth.config5_rows(rows, T, dm)
    probe = hip.Program(text, max_rows=8)
    arena_row = probe.stats().arena_bytes / 8
    probe.close()
    pass_rows = int(max(8, min(4096, (32 << 30) // max(arena_row, 1))))
    pass_rows = 1 << (pass_rows.bit_length() - 1)
    log("config 5: %.1f MiB of arena per sequence, passes of %d sequences" % (arena_row / 2**20, pass_rows))
    prog = hip.Program(text, max_rows=pass_rows)
    tprog = hip.Program(text, flags=hip.TIMING, max_rows=pass_rows)
    d_x = hip.DeviceBuffer.from_array(X)
    d_y = hip.DeviceBuffer(rows * 8 * 4)

    def run(p):
        for r0 in range(0, rows, pass_rows):
            n = min(pass_rows, rows - r0)
            p.batch_device(d_x.ptr + r0 * per * 4, n, d_y.ptr + r0 * 8 * 4)

    run(prog)
    prog.sync()
    steps = max(1, min(args.steps, 3))
    t0 = time.perf_counter()
    for _ in range(steps):
        run(prog)
    prog.sync()
    t = (time.perf_counter() - t0) / steps
    y = d_y.to_array(np.float32, (rows, 8))
    assert np.isfinite(y).all()
    tprog.reset_stats()
    tprog.batch_device(d_x.ptr, pass_rows, d_y.ptr)
    tprog.sync()
    st = tprog.stats()
    scale = rows / pass_rows
    mfma_us, dig_us, oth_us = (v * scale * 1e3 for v in (st.qgemm_ms, st.digits_ms, st.other_ms))
    macs = 4 * T * (2 * dm * 512 + 3 * 512 * 16 + 16 * 512 + 512 * dm) + dm * 8
    ops = 2.0 * macs * rows
    alg_bytes = c5_alg_bytes(rows, T)
    proj_us = mfma_us + dig_us
    per = None if args.no_traffic else profile_pass("c5")
    traffic = None if per is None else sum(v for k, v in per.items() if k.startswith(C5_PROJ_KERNELS)) * rows / C5_PROFILE_SEQS
    log("config 5: %.1f ms per 4096 sequences: projections %.0f us, digits %.0f us, other (scan, elementwise) %.0f us"
        % (t * 1e3, mfma_us, dig_us, oth_us))
    cpu = None if args.no_cpu else ref_cpu(text, X[:32], per, 8, 0, auto_threads(), False,
                                           "config 5 (selective SSM, 4 blocks, T 512)")
    out = {
        "metric": "config 5 selective-SSM sequences/sec at 1 GPU", "value": round(rows / t, 1), "unit": "sequences/s",
        "n_gpus": 1, "steps": steps, "warmup": 1, "ms_per_step": round(t * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8 projections, f32 scan",
        "data": "synthetic (N(0,0.02) weights seed 105 quantized int8 per channel, N(0,1) inputs seed 5)",
        "config": {"workload": "config 5: 4 Mamba-style blocks d_model 256, state 16, expand 2, T 512; 4096 sequences "
                               "per step", "pass_rows": pass_rows},
        "roofline": {"bound": "hbm", "achieved": round(alg_bytes / proj_us / 1e3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(alg_bytes / proj_us / 1e3 / HBM_PEAK_GBS, 4),
                     "traffic": None if traffic is None else round(traffic),
                     "traffic_ratio": None if traffic is None else round(traffic / alg_bytes, 2),
                     "alg_bytes_per_pass": alg_bytes,
                     "alg_bytes_note": "per block and time step: the projections' inputs read once (x 1 KiB, u 2 KiB, "
                                       "the dt-rank vector 64 B, the gated SSM output 2 KiB) and their outputs written "
                                       "once (xi, z, dt 2 KiB each, the dt-rank vector, B and C 64 B each, the block's "
                                       "output 1 KiB): 12,544 B; the int8 weights and scales once",
                     "traffic_note": ("calibrated FETCH_SIZE + WRITE_SIZE of the projections' dispatches (%s) of a pass "
                                      "of %d sequences (rocprofv3), scaled to %d"
                                      % (", ".join(C5_PROJ_KERNELS), C5_PROFILE_SEQS, rows))
                                     if traffic is not None else "not profiled",
                     "traffic_kernels": None if per is None else {k: round(v * rows / C5_PROFILE_SEQS)
                                                                  for k, v in sorted(per.items())},
                     "kernel": "the projections of a pass: digit kernels, quantized GEMMs and the short products on "
                               "the reference's loop (qtiny_k, the dt projection), their epilogues included, summed; "
                               "output-bound (the f32 scan is VALU work)",
                     "avg_kernel_us": round(proj_us, 1),
                     "mfma_view": {"achieved": round(ops / mfma_us / 1e6, 2), "peak": MFMA_I8_PEAK_TOPS, "unit": "TOP/s",
                                   "frac": round(ops / mfma_us / 1e6 / MFMA_I8_PEAK_TOPS, 4)}},
        "cpu_baseline": cpu,
        "breakdown_us": {"projections": round(mfma_us, 1), "digits": round(dig_us, 1), "other": round(oth_us, 1)},
    }
    for o in (prog, tprog):
        o.close()
    for b in (d_x, d_y):
        b.free()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-rows", type=int, default=2048, help="config 2 rows of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 runs (kernel trace and counters)")
    ap.add_argument("--no-legs", action="store_true", help="skip the config 1, 4, 5 and 3 legs")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end `tgc-hip batch` runs")
    ap.add_argument("--reps", type=int, default=10, help="kernel-timing repetitions per batch")
    ap.add_argument("--config", type=int, default=2, choices=(1, 2, 3, 4, 5),
                    help="BASELINE configuration: 2 (default, the headline metric), 1 (int8 MLP), 3 (Qwen3-shaped "
                         "decoder, prefill), 4 (Q16.16 reasoner), 5 (selective-SSM classifier)")
    ap.add_argument("--profile-child", choices=("c1", "c2", "c4", "c5"), help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.profile_child:
        profile_child(args.profile_child)
        return
    if args.gpus != 1:
        print("bench.py: this backend runs on one GPU per process and this build measures one GPU only; "
              "rows shard across GPUs with no collective. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.config != 2:
        {1: bench_config1, 3: bench_config3, 4: bench_config4, 5: bench_config5}[args.config](args)
        return

    import numpy as np
    from technograd_amd import hip, synth

    hip.init(0)
    log("building config 2 (int4 4096x4096)")
    text, X = setup(synth)
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
    fprog, fin, fout = evict_program(hip)
    fprog.set_stream(tprog.stream())  # eviction passes and timed calls in one queue
    wbytes = C * K / 2 + 4 * C
    sweep = []
    for b in BATCHES:
        tprog.batch_device(d_x.ptr, b, d_y.ptr)  # warm-up call (code, scratch)
        tprog.sync()
        tprog.reset_stats()
        for _ in range(args.reps):
            fprog.batch_device(fin.ptr, FLUSH_ROWS, fout.ptr)
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
            "cold_infinity_cache": True, "timing": "HIP events around each kernel (dispatch latency included)",
        })
        log("batch %4d: events: product %.2f us, digits %.2f us" % (b, mfma_us, dig_us))
    big = sweep[-1]
    fprog.set_stream(None)

    # ---- host buffers (PCIe included): reported beside value, never as value ----
    xh = np.ascontiguousarray(X, np.float32)
    prog.batch(xh)
    t0 = time.perf_counter()
    for _ in range(3):
        prog.batch(xh)
    pageable_rps = 3 * 4096 / (time.perf_counter() - t0)
    hin, hout = hip.HostBuffer(xh.nbytes), hip.HostBuffer(4096 * C * 4)
    xp, yp = hin.array(np.float32, xh.shape), hout.array(np.float32, (4096, C))
    xp[:] = xh
    sp = np.zeros((4096, 1), np.int32)
    prog.batch(xp, yp, sp)
    t0 = time.perf_counter()
    for _ in range(3):
        prog.batch(xp, yp, sp)
    pcie_rps = 3 * 4096 / (time.perf_counter() - t0)
    log("host-buffer batch 4096: %.0f rows/s from pinned buffers, %.0f from pageable ones (PCIe in and out included)"
        % (pcie_rps, pageable_rps))
    hin.free()
    hout.free()
    e2e = None if args.no_e2e else cli_batch_wall(text, xh, "config 2 (int4 4096 x 4096, 4096 rows)")

    # ---- rocprofv3: cold kernel durations and HBM traffic per batch ----
    prof, pnote = None, "skipped (--no-traffic)"
    if not args.no_traffic:
        log("rocprofv3: kernel trace, FETCH_SIZE, WRITE_SIZE of the profiling child")
        prof, pnote = profile_c2(big["alg_bytes"])
        log("rocprofv3: %s" % pnote)
    if prof:
        for e in sweep:
            p = prof[e["batch"]]
            e["trace_kernels_us"] = p["kernels_us"]
            e["trace_us"] = p["us"]
            e["trace_hbm_frac"] = round(e["alg_bytes"] / p["us"] / 1e3 / HBM_PEAK_GBS, 4)
            if "traffic" in p:
                e["traffic"] = round(p["traffic"])
    def qgemm_of(d):  # the large-batch GEMM's entry (qgemm_k<4, epilogue variant>)
        return next((v for k, v in (d or {}).items() if k.startswith("qgemm_k<4")), None)

    big_traffic = qgemm_of(prof[4096].get("traffic_kernels")) if prof else None
    roofline = {"bound": "mfma", "achieved": big["mfma_TOPs"], "peak": MFMA_I8_PEAK_TOPS, "unit": "TOP/s",
                "frac": big["mfma_frac"], "traffic": None if big_traffic is None else round(big_traffic),
                "traffic_note": pnote,
                "limb_factor": 3, "hw_mfma_frac": round(3 * big["mfma_frac"], 4),
                "hw_note": "each multiply-add runs as three exact int8 MFMAs (the activation's 24-bit digits): the matrix "
                           "cores execute 3 x alg_ops; hw_mfma_frac = 3 x frac",
                "kernel": "qgemm_k<4> (int8 MFMA, 3 activation digits) at batch 4096",
                "alg_ops_per_launch": big["alg_ops"], "avg_kernel_us": big["mfma_kernel_us"],
                "trace_kernel_us": None if not prof else qgemm_of(prof[4096]["kernels_us"])}
    if prof:
        mv = {}
        for b in (1, 16):
            p, e = prof[b], sweep[BATCHES.index(b)]
            mv["b%d" % b] = {"kernels": sorted(p["kernels_us"]), "us": p["us"],
                             "achieved": round(e["alg_bytes"] / p["us"] / 1e3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(e["alg_bytes"] / p["us"] / 1e3 / HBM_PEAK_GBS, 4), "alg_bytes": e["alg_bytes"],
                             "traffic": None if "traffic" not in p else round(p["traffic"])}
        fl = prof.get("floor", {})
        if fl.get("us"):
            mv["read_floor"] = {"us": fl["us"], "bytes": fl["bytes"], "GBs": round(fl["bytes"] / fl["us"] / 1e3, 1),
                                "traffic": fl.get("traffic"),
                                "note": "a plain read of the packed weight's size (tg_hip_read_pass, 2048 x 256 "
                                        "threads) after the same flush pass: what a cold read of these bytes takes "
                                        "on this device"}
            for b in (1, 16):
                mv["b%d" % b]["of_read_floor"] = round(fl["us"] / mv["b%d" % b]["us"], 4)
        f2 = prof.get("floor256", {})
        if f2.get("us"):
            mv["read_floor_256wg"] = {"us": f2["us"], "bytes": f2["bytes"], "traffic": f2.get("traffic"),
                                      "note": "the same read in 256 workgroups of 256 threads, the B=1 kernel's "
                                              "launch shape: a cold read spread over fewer workgroups takes longer"}
            mv["b1"]["of_read_floor_256wg"] = round(f2["us"] / mv["b1"]["us"], 4)
        mv["note"] = ("int4 matvec: algorithmic bytes (weights, scales, rows in and out) over the summed kernel-trace "
                      "durations of the call's kernels (one kernel at B=1: its digits are made inside it), each call "
                      "after a 512 MiB flush pass; traffic: calibrated FETCH_SIZE + WRITE_SIZE of the same kernels; "
                      "of_read_floor: the read floor's time over the call's")
        roofline["matvec"] = mv

    cpu = None
    if not args.no_cpu:
        log("cpu baseline: %d rows, -j auto (%d threads), 3 runs" % (args.cpu_rows, auto_threads()))
        cpu = ref_cpu(text, X[:args.cpu_rows], K, C, 0, auto_threads(), False, "config 2 (int4 4096x4096)")

    legs = None
    if not args.no_legs:
        def leg(f, *a, **k):  # a failing leg is reported in its place, the headline line still printed
            try:
                return f(*a, **k)
            except Exception as e:  # noqa: BLE001
                log("leg %s failed: %r" % (f.__name__, e))
                return {"error": repr(e)}
        legs = {"config1": leg(config1_leg, args, steps=3, profile=not args.no_traffic),
                "config4": leg(config4_leg, args, steps=3, profile=not args.no_traffic),
                "config5": leg(config5_leg, args), "config3": leg(config3_leg, args)}

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "rows/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(elapsed / args.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "W4A32",
        "dtype_note": "int4 weights x f32 activations, computed exactly as three int8 digit planes of each row's 24-bit "
                      "fixed-point form on the int8 matrix cores (int32 sums, combined in int64/f64, one f32 rounding)",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) rows)",
        "config": {"workload": "config 2: int4 4096x4096 linear, one pass at each batch of {1,16,256,4096} rows per step",
                   "rows_per_step": rows_per_step, "parallelism": "1 GPU"},
        "roofline": roofline, "cpu_baseline": cpu, "sweep": sweep,
        "pcie_inclusive": {"rows_per_s": round(pcie_rps, 1), "batch": 4096, "pageable_rows_per_s": round(pageable_rps, 1),
                           "note": "tg_hip_batch with host buffers: 64 MiB in and 64 MiB out over PCIe per call; rows_per_s "
                                   "with rows and outputs in pinned memory from tg_hip_host_alloc (moved directly), "
                                   "pageable_rows_per_s from ordinary numpy arrays (copied through the library's pinned "
                                   "staging slots)"},
        "end_to_end": e2e,
        "legs": legs,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
