"""Parity predicates shared by the GPU tests.

Integer, byte, index and Q16.16 results must be bit-exact (np.array_equal).

f32 results: an element passes when
    |gpu - ref| <= max(1e-5 * |ref|, 4 ulp(ref))            (the north-star bound)
or, for a quantized matmul whose reference sum cancels, when the difference
is inside the reference's own provable rounding-error bound plus the GPU's:
    |gpu - ref| <= u * |s| * sum_p |S_p|  +  2^-23 * |s| * max|x| * sum_p |code_p|  + 2 ulp(ref)
with u = 2^-24 and S_p the exact running sums of the reference's sequential
loop (runtime/tg_rt.h:132-151): the reference's result is within the first
term of the exact value, the GPU's within the second (24-bit activation grid).
Elements passing only by the second clause are counted and reported.
"""
import numpy as np

U = 2.0 ** -24


def ulp(x):
    return np.spacing(np.abs(np.asarray(x, np.float32))).astype(np.float64)


def strict_ok(gpu, ref):
    g = np.asarray(gpu, np.float64)
    r = np.asarray(ref, np.float64)
    return (np.abs(g - r) <= np.maximum(1e-5 * np.abs(r), 4 * ulp(ref))) | (np.isnan(g) & np.isnan(r)) | (g == r)


def qmatmul_bound(codes_ck, scale_c, x_mk):
    """Per-output bound (M, C) for o[m, c] = s[c] * sum_k code[c, k] x[m, k]."""
    codes = np.asarray(codes_ck, np.float64)
    x = np.asarray(x_mk, np.float64)
    s = np.abs(np.asarray(scale_c, np.float64))
    terms = x[:, None, :] * codes[None, :, :]               # (M, C, K) exact products
    partial = np.abs(np.cumsum(terms, axis=2)).sum(axis=2)  # sum_p |S_p|
    grid = np.abs(x).max(axis=1)[:, None] * np.abs(codes).sum(axis=1)[None, :]
    return U * s[None, :] * partial + 2.0 ** -23 * s[None, :] * grid


def check_qmatmul(gpu, ref, codes_ck, scale_c, x_mk):
    """Returns the fraction of elements that pass only by the bound clause."""
    ok = strict_ok(gpu, ref)
    if ok.all():
        return 0.0
    bound = qmatmul_bound(codes_ck, scale_c, x_mk) + 2 * ulp(ref)
    diff = np.abs(np.asarray(gpu, np.float64) - np.asarray(ref, np.float64))
    bad = ~ok & (diff > bound)
    assert not bad.any(), "quantized matmul outside the parity bound at %s" % (np.argwhere(bad)[:5].tolist(),)
    return float((~ok).mean())


def check_model(gpu, ref, row_atol=2e-6):
    """Whole-model f32 outputs: the strict bound per element, with an absolute
    floor of row_atol * max|ref| over the row for elements that sit near zero
    after cancellation in an earlier layer."""
    g = np.asarray(gpu, np.float64)
    r = np.asarray(ref, np.float64)
    floor = row_atol * np.abs(r).max(axis=-1, keepdims=True)
    ok = strict_ok(gpu, ref) | (np.abs(g - r) <= floor)
    assert ok.all(), "f32 outputs outside tolerance: worst %g at %s" % (
        np.nanmax(np.abs(g - r)), np.argwhere(~ok)[:5].tolist())


def digit_path_matmul(x_mk, codes_kc, scale_c):
    """The matrix-core path's arithmetic, restated on the host (not the
    reference's order): per row, E from max |x| (frexp; raised by one when
    rint(max |x| 2^(23-E)) > 8355328), q = rint(x 2^(23-E)) exactly, the exact
    integer sum t = sum_k code[k, c] q[m, k], then f32(t 2^(E-23)) * s[c] in
    f32. Rows with a NaN or max |x| above 2^100 (inf included) are special:
    the device runs the reference's loop for them; they are returned masked.
    Returns (f32 [M, C], special [M])."""
    x = np.asarray(x_mk, np.float32)
    amax = np.abs(x).max(axis=1)
    special = np.isnan(x).any(axis=1) | (amax > np.float32(2.0 ** 100))
    _, E = np.frexp(np.where(special, 0, amax).astype(np.float64))
    E = np.where(amax > 0, E, 0).astype(np.int64)
    top = np.rint(np.ldexp(np.where(special, 0, amax).astype(np.float64), 23 - E))
    E = np.where((top > 8355328) & ~special, E + 1, E)
    xs = np.where(special[:, None], 0, x).astype(np.float64)
    q = np.rint(np.ldexp(xs, (23 - E)[:, None]))                        # exact integers, |q| < 2^23
    t = q @ np.asarray(codes_kc, np.float64)                              # exact: every partial sum < 2^53
    v = np.ldexp(t, (E - 23)[:, None]).astype(np.float32)                 # one rounding to f32
    return (v * np.asarray(scale_c, np.float32)[None, :]).astype(np.float32), special
