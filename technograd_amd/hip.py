"""ctypes binding of the MI355X batch backend's C ABI (include/tg_hip.h).

The library is built in-tree (technograd_amd/lib/libtg_hip.so, see
technograd_amd/Makefile). There is no CPU fallback: if the library is missing
or a call fails, these functions raise.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# TG_HIP_LIB names another build of the library (the host sanitizer build runs the CPU tests that way)
LIB_PATH = os.environ.get("TG_HIP_LIB") or os.path.join(HERE, "lib", "libtg_hip.so")

FIXED, EXACT, ROWPROG, TIMING, INTERP = 1, 2, 4, 8, 16


class Stats(ctypes.Structure):
    _fields_ = [
        ("executor", ctypes.c_int), ("rows", ctypes.c_int), ("batch_ms", ctypes.c_double), ("qgemm_ms", ctypes.c_double),
        ("qgemm_calls", ctypes.c_long), ("digits_ms", ctypes.c_double), ("other_ms", ctypes.c_double),
        ("weight_bytes", ctypes.c_double), ("macs", ctypes.c_double), ("arena_bytes", ctypes.c_long),
        ("rowprog_jit", ctypes.c_int), ("rowprog_hoisted", ctypes.c_long), ("epilogue_ins", ctypes.c_int),
        ("scan_folded_ins", ctypes.c_int),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("technograd_amd: %s is not built; run technograd_amd.build.build()" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        vp, ip, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        L.tg_hip_init.argtypes = [ip]
        L.tg_hip_load.restype = vp
        L.tg_hip_load.argtypes = [ctypes.c_char_p, sz, ip, ip]
        L.tg_hip_info.argtypes = [vp, ctypes.POINTER(ip), ctypes.POINTER(ip), ctypes.POINTER(ip)]
        L.tg_hip_batch.argtypes = [vp, vp, ctypes.c_long, vp, vp]
        L.tg_hip_batch_fixed.argtypes = [vp, vp, ctypes.c_long, vp, vp]
        L.tg_hip_batch_device.argtypes = [vp, vp, ctypes.c_long, vp, vp]
        L.tg_hip_sync.argtypes = [vp]
        L.tg_hip_matmul_q.argtypes = [vp, vp, ip, vp, vp, ip, ip, ip, ip, ip]
        L.tg_hip_matmul_qa.argtypes = [vp, vp, ip, vp, vp, ip, ip, ip]
        L.tg_hip_read_pass.argtypes = [vp, ctypes.c_size_t, ip, vp]
        L.tg_hip_matmul_qb.argtypes = [vp, vp, vp, ip, vp, ip, ip, ip]
        L.tg_hip_matmul_q_noalloc.argtypes = [vp, vp, ip, vp, vp, ip, ip, ip, ip, vp]
        L.tg_hip_quantize_rtn.argtypes = [vp, ip, ip, ip, ip, vp, vp, ip]
        L.tg_hip_dec_create.restype = vp
        L.tg_hip_dec_create.argtypes = [vp, ip, ip, ip]
        L.tg_hip_dec_generate.argtypes = [vp, vp, ip, ip, ip, vp, vp]
        L.tg_hip_dec_info.argtypes = [vp, ctypes.POINTER(ip), ctypes.POINTER(ip)]
        L.tg_hip_dec_free.argtypes = [vp]
        L.tg_hip_free.argtypes = [vp]
        L.tg_hip_emit_unit.restype = vp
        L.tg_hip_emit_unit.argtypes = [ctypes.c_char_p, sz, ip, ctypes.c_char_p]
        L.tg_hip_str_free.argtypes = [vp]
        L.tg_hip_surface_to_tgir.restype = vp
        L.tg_hip_surface_to_tgir.argtypes = [ctypes.c_char_p]
        L.tg_hip_quantize_model.restype = vp
        L.tg_hip_quantize_model.argtypes = [ctypes.c_char_p, ctypes.c_size_t, ip, ip, vp, ctypes.c_long, ip, ip, vp, vp,
                                            ctypes.c_size_t]
        L.tg_hip_error.restype = ctypes.c_char_p
        L.tg_hip_stats.argtypes = [vp, ctypes.POINTER(Stats)]
        L.tg_hip_reset_stats.argtypes = [vp]
        L.tg_hip_set_stream.argtypes = [vp, vp]
        L.tg_hip_get_stream.restype = vp
        L.tg_hip_get_stream.argtypes = [vp]
        L.tg_hip_dev_alloc.restype = vp
        L.tg_hip_dev_alloc.argtypes = [sz]
        L.tg_hip_dev_free.argtypes = [vp]
        L.tg_hip_host_alloc.restype = vp
        L.tg_hip_host_alloc.argtypes = [sz]
        L.tg_hip_host_free.argtypes = [vp]
        L.tg_hip_h2d.argtypes = [vp, vp, sz]
        L.tg_hip_d2h.argtypes = [vp, vp, sz]
        _lib = L
    return _lib


def _check(rc, what):
    if rc != 0:
        raise RuntimeError("%s: %s" % (what, lib().tg_hip_error().decode()))


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def init(device=0):
    _check(lib().tg_hip_init(device), "tg_hip_init")


class DeviceBuffer:
    """Device memory from tg_hip_dev_alloc."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = lib().tg_hip_dev_alloc(self.nbytes)
        if not self.ptr:
            raise RuntimeError("tg_hip_dev_alloc: " + lib().tg_hip_error().decode())

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        _check(lib().tg_hip_h2d(b.ptr, _p(a), a.nbytes), "tg_hip_h2d")
        return b

    def to_array(self, dtype, shape):
        out = np.empty(shape, dtype)
        _check(lib().tg_hip_d2h(_p(out), self.ptr, out.nbytes), "tg_hip_d2h")
        return out

    def free(self):
        if self.ptr:
            lib().tg_hip_dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        self.free()


class HostBuffer:
    """Pinned host memory from tg_hip_host_alloc: rows and outputs inside it
    travel to and from the device without tg_hip_batch's staging copy."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = lib().tg_hip_host_alloc(self.nbytes)
        if not self.ptr:
            raise RuntimeError("tg_hip_host_alloc: " + lib().tg_hip_error().decode())

    def array(self, dtype, shape):
        """a numpy view of the buffer (valid until free)"""
        dtype = np.dtype(dtype)
        n = int(np.prod(shape)) * dtype.itemsize
        if n > self.nbytes:
            raise ValueError("view of %d bytes in a %d-byte buffer" % (n, self.nbytes))
        return np.frombuffer((ctypes.c_char * n).from_address(self.ptr), dtype).reshape(shape)

    def free(self):
        if self.ptr:
            lib().tg_hip_host_free(self.ptr)
            self.ptr = None

    def __del__(self):
        self.free()


class Program:
    """A model loaded on the device (tg_hip_load)."""

    def __init__(self, tgir, flags=0, max_rows=4096):
        if isinstance(tgir, str):
            tgir = tgir.encode()
        self.flags = flags
        self.h = lib().tg_hip_load(tgir, len(tgir), flags, max_rows)
        if not self.h:
            raise RuntimeError("tg_hip_load: " + lib().tg_hip_error().decode())
        per, nout, nthink = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        _check(lib().tg_hip_info(self.h, ctypes.byref(per), ctypes.byref(nout), ctypes.byref(nthink)), "tg_hip_info")
        self.per, self.nout, self.nthink = per.value, nout.value, nthink.value
        self.max_rows = max_rows

    def close(self):
        if getattr(self, "h", None):
            lib().tg_hip_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def batch(self, rows, out=None, steps=None):
        """rows [n, per] -> (out [n, nout], steps [n, max(nthink, 1)]); out and
        steps may be given (C-contiguous f32 / int32 arrays, e.g. views of a
        HostBuffer)"""
        rows = np.ascontiguousarray(rows, dtype=np.float32).reshape(-1, self.per)
        if out is None:
            out = np.empty((rows.shape[0], self.nout), np.float32)
        if steps is None:
            steps = np.zeros((rows.shape[0], max(self.nthink, 1)), np.int32)
        assert out.dtype == np.float32 and out.flags.c_contiguous and out.size == rows.shape[0] * self.nout
        assert steps.dtype == np.int32 and steps.flags.c_contiguous and steps.size == rows.shape[0] * max(self.nthink, 1)
        _check(lib().tg_hip_batch(self.h, _p(rows), rows.shape[0], _p(out), _p(steps)), "tg_hip_batch")
        return out, steps

    def batch_fixed(self, rows_q16):
        rows = np.ascontiguousarray(rows_q16, dtype=np.int32).reshape(-1, self.per)
        out = np.empty((rows.shape[0], self.nout), np.int32)
        steps = np.zeros((rows.shape[0], max(self.nthink, 1)), np.int32)
        _check(lib().tg_hip_batch_fixed(self.h, _p(rows), rows.shape[0], _p(out), _p(steps)), "tg_hip_batch_fixed")
        return out, steps

    def batch_device(self, d_rows, nrows, d_out, d_steps=None):
        _check(lib().tg_hip_batch_device(self.h, d_rows, nrows, d_out, d_steps), "tg_hip_batch_device")

    def sync(self):
        _check(lib().tg_hip_sync(self.h), "tg_hip_sync")

    def stats(self):
        s = Stats()
        _check(lib().tg_hip_stats(self.h, ctypes.byref(s)), "tg_hip_stats")
        return s

    def reset_stats(self):
        _check(lib().tg_hip_reset_stats(self.h), "tg_hip_reset_stats")

    def stream(self):
        """The hipStream_t (as an int) this program launches on."""
        return lib().tg_hip_get_stream(self.h)

    def set_stream(self, stream):
        """Launch on another hipStream_t (an int handle, e.g. another
        program's stream() or torch.cuda.current_stream().cuda_stream);
        None restores the program's own stream."""
        _check(lib().tg_hip_set_stream(self.h, stream), "tg_hip_set_stream")


def matmul_q(q, bits, s, b, m, k, n, axis, flags=0):
    """tg_matmul_qa (axis 0) / tg_matmul_qb (axis 1) on the device, host arrays."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    o = np.empty((m, n), np.float32)
    _check(lib().tg_hip_matmul_q(_p(o), _p(q), bits, _p(s), _p(b), m, k, n, axis, flags), "tg_hip_matmul_q")
    return o


def matmul_qa(q, bits, s, b, m, k, n):
    """tg_hip_matmul_qa: tg_matmul_qa's argument list (o = diag(s) Q @ b)."""
    q, s, b = (np.ascontiguousarray(v, dtype=t) for v, t in ((q, np.int8), (s, np.float32), (b, np.float32)))
    o = np.empty((m, n), np.float32)
    _check(lib().tg_hip_matmul_qa(_p(o), _p(q), bits, _p(s), _p(b), m, k, n), "tg_hip_matmul_qa")
    return o


def matmul_qb(a, q, bits, s, m, k, n):
    """tg_hip_matmul_qb: tg_matmul_qb's argument list (o = a @ Q diag(s))."""
    a, q, s = (np.ascontiguousarray(v, dtype=t) for v, t in ((a, np.float32), (q, np.int8), (s, np.float32)))
    o = np.empty((m, n), np.float32)
    _check(lib().tg_hip_matmul_qb(_p(o), _p(a), _p(q), bits, _p(s), m, k, n), "tg_hip_matmul_qb")
    return o


def read_pass(ptr, nbytes, blocks=2048, stream=None):
    """tg_hip_read_pass: read nbytes of device memory at ptr (16-byte aligned),
    writing nothing, asynchronous on `stream` (a measurement floor)."""
    _check(lib().tg_hip_read_pass(ptr, nbytes, blocks, stream), "tg_hip_read_pass")


def matmul_q_noalloc(d_o, d_q, bits, d_s, d_b, m, k, n, axis, stream=None):
    """tg_hip_matmul_q_noalloc: device pointers (ints), asynchronous on
    `stream` (None: the null stream). Returns the C status (0, or -2 when the
    call is larger than the library's fixed scratch; the message is in
    error())."""
    return lib().tg_hip_matmul_q_noalloc(d_o, d_q, bits, d_s, d_b, m, k, n, axis, stream)


def emit_unit(tgir, flags=0, kernel=None):
    """The model's row program as a freestanding HIP unit (tg_hip_emit_unit); no GPU needed."""
    t = tgir.encode() if isinstance(tgir, str) else tgir
    p = lib().tg_hip_emit_unit(t, len(t), flags, kernel.encode() if kernel else None)
    if not p:
        raise RuntimeError("emit_unit: %s" % lib().tg_hip_error().decode())
    try:
        return ctypes.string_at(p).decode()
    finally:
        lib().tg_hip_str_free(p)


def surface_to_tgir(path):
    """A .tg model file lowered to canonical TGIR text (tg_hip_surface_to_tgir); no GPU needed."""
    p = lib().tg_hip_surface_to_tgir(os.fsencode(path))
    if not p:
        raise RuntimeError(lib().tg_hip_error().decode())
    try:
        return ctypes.string_at(p).decode()
    finally:
        lib().tg_hip_str_free(p)


def quantize_model(tgir, bits=8, method="rtn", calib=None, min_size=256, max_k=2048):
    """`tgc quantize` (tg_hip_quantize_model): the model's eligible params
    quantized to int`bits`. method "gptq" needs calib, an [n, per] f32 array
    of calibration rows, and a GPU (the calibration run and the Hessians are
    on the device); RTN without calib runs on the host. max_k = 2048 is the
    reference's Hessian width limit, 0 none. Returns (TGIR text, report
    lines, (param bytes before, after))."""
    if method not in ("rtn", "gptq"):
        raise ValueError("method is rtn or gptq")
    t = tgir.encode() if isinstance(tgir, str) else bytes(tgir)
    rows, n = None, 0
    if calib is not None:
        rows = np.ascontiguousarray(calib, dtype=np.float32)
        n = rows.shape[0]
        init()
    log = ctypes.create_string_buffer(1 << 16)
    nbytes = (ctypes.c_long * 2)()
    p = lib().tg_hip_quantize_model(t, len(t), bits, method == "gptq", None if rows is None else _p(rows), n, min_size,
                                    max_k, nbytes, log, len(log))
    if not p:
        raise RuntimeError(lib().tg_hip_error().decode())
    try:
        return ctypes.string_at(p).decode(), log.value.decode(), (nbytes[0], nbytes[1])
    finally:
        lib().tg_hip_str_free(p)


def error():
    return lib().tg_hip_error().decode()


def quantize_rtn(w, bits, axis, threads=None):
    """tg_hip_quantize_rtn on the host (no device): (codes int8 in w's
    layout, scales f32 per channel), as `tgc quantize --method rtn` writes
    them."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    codes = np.empty((rows, cols), np.int8)
    scales = np.empty(rows if axis == 0 else cols, np.float32)
    t = threads or min(16, os.cpu_count() or 1)
    _check(lib().tg_hip_quantize_rtn(_p(w), rows, cols, bits, axis, _p(codes), _p(scales), t), "tg_hip_quantize_rtn")
    return codes, scales


class Decoder:
    """tg_hip_dec_*: KV-cache greedy decoding of a loaded program in the
    Qwen3 importer's layout (the program must outlive the decoder)."""

    def __init__(self, prog, max_seqs, max_prompt, max_len):
        self.prog = prog
        self.h = lib().tg_hip_dec_create(prog.h, max_seqs, max_prompt, max_len)
        if not self.h:
            raise RuntimeError("tg_hip_dec_create: " + lib().tg_hip_error().decode())
        layers, vocab = ctypes.c_int(), ctypes.c_int()
        lib().tg_hip_dec_info(self.h, ctypes.byref(layers), ctypes.byref(vocab))
        self.layers, self.vocab = layers.value, vocab.value

    def generate_device(self, d_prompt, seqs, prompt_len, steps, d_tokens=None, d_logits=None):
        """Asynchronous, device buffers (DeviceBuffer or raw pointers)."""
        ptr = lambda b: None if b is None else (b.ptr if hasattr(b, "ptr") else b)
        _check(lib().tg_hip_dec_generate(self.h, ptr(d_prompt), seqs, prompt_len, steps, ptr(d_tokens), ptr(d_logits)),
               "tg_hip_dec_generate")

    def generate(self, prompts, steps, logits=False):
        """Host arrays: prompts [seqs][prompt_len] token ids -> tokens
        [seqs][steps] (int32), and logits [steps][seqs][vocab] if asked."""
        prompts = np.ascontiguousarray(prompts, np.float32)
        seqs, plen = prompts.shape
        dp = DeviceBuffer.from_array(prompts)
        dt = DeviceBuffer(seqs * steps * 4)
        dl = DeviceBuffer(steps * seqs * self.vocab * 4) if logits else None
        self.generate_device(dp, seqs, plen, steps, dt, dl)
        self.prog.sync()
        tokens = dt.to_array(np.int32, (seqs, steps))
        return (tokens, dl.to_array(np.float32, (steps, seqs, self.vocab))) if logits else tokens

    def close(self):
        if self.h:
            lib().tg_hip_dec_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
