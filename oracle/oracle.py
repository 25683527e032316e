"""TEST INFRASTRUCTURE ONLY: ctypes access to the CPU parity oracle.

`liboracle.so` (built by oracle/Makefile from oracle/*.c) is a C restatement
of the reference's quantized `tgc batch` semantics; `_ref/tgc_ref` is the
reference's own path sources compiled from /root/reference. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use this module, and
only to check or time the CPU side; the product never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_BIN = os.path.join(HERE, "_ref", "tgc_ref")

_lib = None


def build(ref=None):
    """Compile liboracle.so (and _ref/tgc_ref when the reference tree exists)."""
    targets = ["all"]
    if ref is None:
        ref = os.path.isdir("/root/reference/src")
    if ref:
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", HERE, "-j8"] + targets, check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("oracle/liboracle.so is not built (run make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        vp, cp, ip = ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int
        L.tgo_load.restype = vp
        L.tgo_load.argtypes = [cp, cp, ip]
        L.tgo_free.argtypes = [vp]
        L.tgo_info.argtypes = [vp, ctypes.POINTER(ip), ctypes.POINTER(ip), ctypes.POINTER(ip), ctypes.POINTER(ctypes.c_long)]
        L.tgo_batch.argtypes = [vp, vp, ctypes.c_long, vp, vp, ip]
        L.tgo_batch_fixed.argtypes = [vp, vp, ctypes.c_long, vp, vp, ip]
        L.tgo_batch64.argtypes = [vp, vp, ctypes.c_long, vp, vp, ip]
        L.tgo_write.restype = ctypes.c_void_p
        L.tgo_write.argtypes = [vp]
        L.tgo_str_free.argtypes = [vp]
        L.tgo_rand.argtypes = [ctypes.c_uint32, ctypes.c_float, vp, ctypes.c_long]
        L.tgo_to_fixed_rows.argtypes = [vp, vp, ctypes.c_long]
        L.tgo_to_fixed.restype = ctypes.c_int32
        L.tgo_to_fixed.argtypes = [ctypes.c_double, ip]
        L.tgo_fx_format.restype = cp
        L.tgo_fx_format.argtypes = [ctypes.c_int32, cp]
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


class Model:
    """A TGIR model held by the oracle."""

    def __init__(self, text):
        if isinstance(text, str):
            text = text.encode()
        err = ctypes.create_string_buffer(512)
        self.h = lib().tgo_load(text, err, 512)
        if not self.h:
            raise ValueError("oracle: " + err.value.decode())
        per, nout, nthink = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        arena = ctypes.c_long()
        self.nupd = lib().tgo_info(self.h, ctypes.byref(per), ctypes.byref(nout), ctypes.byref(nthink), ctypes.byref(arena))
        self.per, self.nout, self.nthink, self.arena = per.value, nout.value, nthink.value, arena.value

    def __del__(self):
        if getattr(self, "h", None):
            lib().tgo_free(self.h)
            self.h = None

    def batch(self, rows, threads=8):
        rows = np.ascontiguousarray(rows, dtype=np.float32).reshape(-1, self.per)
        out = np.empty((rows.shape[0], self.nout), np.float32)
        steps = np.zeros((rows.shape[0], max(self.nthink, 1)), np.int32)
        rc = lib().tgo_batch(self.h, _ptr(rows), rows.shape[0], _ptr(out), _ptr(steps), threads)
        if rc:
            raise RuntimeError("oracle batch failed (%d)" % rc)
        return out, steps

    def batch64(self, rows, threads=8):
        """The same interpreter in double precision (vm64.c): a high-precision
        truth for tests, not the reference's arithmetic."""
        rows = np.ascontiguousarray(rows, dtype=np.float32).astype(np.float64).reshape(-1, self.per)
        out = np.empty((rows.shape[0], self.nout), np.float64)
        steps = np.zeros((rows.shape[0], max(self.nthink, 1)), np.int32)
        rc = lib().tgo_batch64(self.h, _ptr(rows), rows.shape[0], _ptr(out), _ptr(steps), threads)
        if rc:
            raise RuntimeError("oracle f64 batch failed (%d)" % rc)
        return out, steps

    def batch_fixed(self, rows_q16, threads=8):
        rows = np.ascontiguousarray(rows_q16, dtype=np.int32).reshape(-1, self.per)
        out = np.empty((rows.shape[0], self.nout), np.int32)
        steps = np.zeros((rows.shape[0], max(self.nthink, 1)), np.int32)
        rc = lib().tgo_batch_fixed(self.h, _ptr(rows), rows.shape[0], _ptr(out), _ptr(steps), threads)
        if rc:
            raise RuntimeError("oracle fixed batch failed (%d)" % rc)
        return out, steps

    def write(self):
        p = lib().tgo_write(self.h)
        s = ctypes.string_at(p).decode()
        lib().tgo_str_free(p)
        return s


def rand(seed, scale, n):
    out = np.empty(n, np.float32)
    lib().tgo_rand(seed, scale, _ptr(out), n)
    return out


def to_fixed_rows(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.int32)
    lib().tgo_to_fixed_rows(_ptr(x), _ptr(out), x.size)
    return out


def to_fixed(v, frac=16):
    return lib().tgo_to_fixed(float(v), frac)


def fx_format(v):
    buf = ctypes.create_string_buffer(32)
    return lib().tgo_fx_format(int(v), buf).decode()


# ---- the reference build (oracle/_ref) ----

def have_ref():
    return os.path.exists(REF_BIN)


def ref_run(args, **kw):
    return subprocess.run([REF_BIN] + list(args), check=True, capture_output=True, **kw)


def ref_ir(model_path):
    return ref_run(["ir", model_path]).stdout.decode()


def ref_batch(model_path, rows, per, nout, nthink, workdir, threads=1, fixed=False, wall=False):
    """Run the reference VM (or its Q16.16 kernels with fixed=True) over rows.
    Returns (out, steps, compute ms), and the wall ms as a fourth item with
    wall=True (from before the input load to after the last write)."""
    dt = np.int32 if fixed else np.float32
    inp, outp, stp = (os.path.join(workdir, n) for n in ("ref_in.bin", "ref_out.bin", "ref_steps.bin"))
    np.ascontiguousarray(rows, dtype=dt).astype("<" + dt().dtype.str[1:]).tofile(inp)
    args = ["batch", model_path, inp, "-o", outp, "--steps", stp, "-j", str(threads)]
    if fixed:
        args.append("--fixed")
    r = ref_run(args)
    out = np.fromfile(outp, dtype=dt).reshape(-1, nout)
    steps = np.fromfile(stp, dtype=np.int32).reshape(-1, max(nthink, 1))
    ms = wall_ms = None
    for line in r.stderr.decode().splitlines():
        if line.startswith("ref-batch"):
            f = line.split()
            ms = float(f[f.index("ms") + 1])
            wall_ms = float(f[f.index("wall_ms") + 1])
    return (out, steps, ms, wall_ms) if wall else (out, steps, ms)


def ref_unit_build(model_path, workdir):
    """Emit the reference's `tgc c --fixed` unit for the model with the
    raw-row driver and compile it (cc -std=c99 -O2, as tests/run.sh:309 of the
    reference compiles units). Returns the executable's path (`exe ROWS OUT
    STEPS`)."""
    d = os.path.join(workdir, "unit_" + os.path.basename(model_path).replace(".", "_"))
    os.makedirs(d, exist_ok=True)
    unit, main, exe = (os.path.join(d, n) for n in ("unit.c", "main.c", "unit"))
    ref_run(["c", model_path, "-o", unit, "--fixed", "--harness", main])
    subprocess.run([os.environ.get("CC", "cc"), "-std=c99", "-O2", "-o", exe, main], check=True, capture_output=True)
    return exe


def ref_unit(model_path, rows_q16, nout, nthink, workdir):
    """Run the reference's own `tgc c --fixed` unit over Q16.16 rows.

    src/cgen.c (compiled into _ref/tgc_ref) emits the freestanding unit for the
    model, as `tgc c MODEL --fixed` does; it is compiled the way the
    reference's tests compile such units (tests/run.sh:309, cc -std=c99 -O2),
    with the raw-row driver tgc_ref writes beside it instead of the unit's own
    decimal driver. Returns (int32 outputs [rows, nout], int32 steps [rows,
    max(nthink, 1)])."""
    exe = ref_unit_build(model_path, workdir)
    d = os.path.dirname(exe)
    inp, outp, stp = (os.path.join(d, n) for n in ("in.bin", "out.bin", "steps.bin"))
    np.ascontiguousarray(rows_q16, dtype="<i4").tofile(inp)
    subprocess.run([exe, inp, outp, stp], check=True, capture_output=True)
    out = np.fromfile(outp, dtype="<i4").reshape(-1, nout)
    steps = np.fromfile(stp, dtype="<i4").reshape(-1, max(nthink, 1))
    return out, steps
