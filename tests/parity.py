"""Parity predicates shared by the GPU tests.

Integer, byte, index and Q16.16 results must be bit-exact (np.array_equal).

f32 results: an element passes when it is within the north-star bound of
the reference's result,
    |gpu - ref| <= max(1e-5 * |ref|, 4 ulp(ref)),
or, where that cannot hold because the reference's own sequential f32 sums
cancel (at K = 4096 the reference misses 1e-5 relative of the exact value on
a few percent of outputs), when the GPU result is accurate against a truth:

- a single quantized product: within N0 = 4 units of the scale at which any
  f32 evaluation of the sum rounds, of the exact product (f64):
      |gpu - truth| <= 4 * 2^-24 * sum_k |s w_k x_k| + ulp(truth).
  This is the normalized error of the sum's forward error analysis; the
  reference's sequential sum is guaranteed only within K such units and
  typically lands within 1.
- a whole model: truth = the oracle's interpreter in double precision
  (oracle/vm64.c: every op of the model in the same order, rounded to
  double); the GPU's largest error on an output row may be at most twice the
  reference's largest error on that row, plus 2 ulp:
      |gpu - truth| <= 2 * max_row |ref - truth| + 2 ulp(truth).
  No absolute floor: a row the reference computes to the last ulp must be
  computed as well by the GPU.
Every check reports how many elements needed the second clause.
"""
import numpy as np

U = 2.0 ** -24
N0 = 4


def ulp(x):
    return np.spacing(np.abs(np.asarray(x, np.float32))).astype(np.float64)


def strict_ok(gpu, ref):
    g = np.asarray(gpu, np.float64)
    r = np.asarray(ref, np.float64)
    return (np.abs(g - r) <= np.maximum(1e-5 * np.abs(r), 4 * ulp(ref))) | (np.isnan(g) & np.isnan(r)) | (g == r)


def qmatmul_truth(codes_ck, scale_c, x_mk):
    """(truth [M, C], sum |s w x| [M, C]) of o[m, c] = s[c] sum_k code[c, k] x[m, k], in f64."""
    codes = np.asarray(codes_ck, np.float64)
    x = np.asarray(x_mk, np.float64)
    s = np.asarray(scale_c, np.float64)
    return (x @ codes.T) * s[None, :], (np.abs(x) @ np.abs(codes).T) * np.abs(s)[None, :]


def normalized_error(val, codes_ck, scale_c, x_mk):
    """|val - exact| / (2^-24 sum |s w x|) per element (0 where the sum is 0)."""
    truth, mag = qmatmul_truth(codes_ck, scale_c, x_mk)
    with np.errstate(invalid="ignore", divide="ignore"):
        n = np.abs(np.asarray(val, np.float64) - truth) / (U * mag)
    return np.where(mag > 0, n, 0.0)


def check_qmatmul(gpu, ref, codes_ck, scale_c, x_mk, max_fallback=None):
    """A quantized product against the reference's result (strict, or within
    N0 normalized units of the exact product). Returns (fraction of elements
    that needed the second clause, largest normalized error of the GPU
    result, largest normalized error of the reference's result)."""
    truth, mag = qmatmul_truth(codes_ck, scale_c, x_mk)
    g = np.asarray(gpu, np.float64)
    ok = strict_ok(gpu, ref)
    with np.errstate(invalid="ignore"):
        near = np.abs(g - truth) <= N0 * U * mag + ulp(truth)
    rescued = ~ok & near
    bad = ~ok & ~rescued
    assert not bad.any(), "quantized matmul: %d elements fail both clauses, e.g. %s" % (
        bad.sum(), [(tuple(int(v) for v in i), float(g[tuple(i)]), float(np.asarray(ref)[tuple(i)]), float(truth[tuple(i)]),
                     float(U * mag[tuple(i)])) for i in np.argwhere(bad)[:3]])
    frac = float(rescued.mean())
    if max_fallback is not None:
        assert frac <= max_fallback, "%.4f of outputs needed the second clause (limit %.4f)" % (frac, max_fallback)
    ng = normalized_error(gpu, codes_ck, scale_c, x_mk)
    nr = normalized_error(ref, codes_ck, scale_c, x_mk)
    return frac, float(np.nanmax(ng)) if ng.size else 0.0, float(np.nanmax(nr)) if nr.size else 0.0


def check_model(gpu, ref, truth=None, steps_same=None):
    """Whole-model f32 outputs [rows, n]: strict per element, or (given the
    f64 truth) within twice the reference's own largest error on the row.
    Rows whose think loops halted at a different step in double precision
    (steps_same[row] False) take the strict clause only. Returns the number
    of elements that needed the second clause."""
    g = np.asarray(gpu, np.float64)
    r = np.asarray(ref, np.float64)
    g2, r2 = g.reshape(g.shape[0], -1), r.reshape(r.shape[0], -1)
    ok = strict_ok(g2, r2)
    rescued = np.zeros_like(ok)
    if truth is not None:
        t2 = np.asarray(truth, np.float64).reshape(g2.shape)
        with np.errstate(invalid="ignore"):
            rerr = np.where(np.isnan(r2 - t2), 0.0, np.abs(r2 - t2)).max(axis=1, keepdims=True)
            rescued = ~ok & (np.abs(g2 - t2) <= 2 * rerr + 2 * ulp(t2))
        if steps_same is not None:
            rescued &= np.asarray(steps_same, bool).reshape(-1, 1)
    bad = ~ok & ~rescued
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError("f32 outputs outside tolerance: %d elements, first %s gpu %r ref %r truth %r" % (
            bad.sum(), i, float(g2[i]), float(r2[i]), None if truth is None else float(np.asarray(truth).reshape(g2.shape)[i])))
    return int(rescued.sum())


def grid_bound(codes_ck, scale_c, x_mk):
    """The digit path's own error bound against the exact product, for rows
    that are not special: the 24-bit activation grid, 2^-23 max|x| per
    element (tests of the host restatement only; not a parity predicate)."""
    codes = np.asarray(codes_ck, np.float64)
    x = np.asarray(x_mk, np.float64)
    s = np.abs(np.asarray(scale_c, np.float64))
    return 2.0 ** -23 * s[None, :] * np.abs(x).max(axis=1)[:, None] * np.abs(codes).sum(axis=1)[None, :]


def peaked_rows(x_mk):
    """Rows the digit kernels flag as peaked (technograd_amd/csrc/tg_qdigits.h):
    some nonzero entry below the band |x| >= max|x| / 4, and at most
    8 (max(1, K / 4) for K < 32) entries in the band."""
    x = np.asarray(x_mk, np.float32)
    a = np.abs(x)
    with np.errstate(invalid="ignore"):
        amax = np.where(np.isnan(x).any(axis=1), np.float32(0), a.max(axis=1)).astype(np.float32)
        band = np.ldexp(amax, np.int32(-2)).astype(np.float32)
        nz = a != 0
        inb = ((a >= band[:, None]) & nz).sum(axis=1)
        below = ((a < band[:, None]) & nz).sum(axis=1)
    K = x.shape[1]
    return (below > 0) & (inb <= (8 if K >= 32 else max(1, K >> 2)))


def digit_path_matmul(x_mk, codes_kc, scale_c, peak=True, f64=False):
    """The matrix-core path's arithmetic, restated on the host (not the
    reference's order): per row, E from max |x| (frexp; raised by one when
    rint(max |x| 2^(23-E)) > 8355328), q = rint(x 2^(23-E)) exactly, the exact
    integer sum t = sum_k code[k, c] q[m, k], then f32(t 2^(E-23)) * s[c] in
    f32. Rows with a NaN or max |x| above 2^100 (inf included), and peaked
    rows (peaked_rows), are special: the device runs the reference's loop for
    them (reference_loop); they are returned masked. peak=False leaves peaked
    rows on the grid (the path before the peak test; tests plant it).
    f64: return the grid sums t 2^(E-23) unrounded (scale_c not applied).
    Returns (f32 [M, C], special [M])."""
    x = np.asarray(x_mk, np.float32)
    amax = np.abs(x).max(axis=1)
    special = np.isnan(x).any(axis=1) | (amax > np.float32(2.0 ** 100))
    if peak:
        special |= peaked_rows(x) & ~special
    _, E = np.frexp(np.where(special, 0, amax).astype(np.float64))
    E = np.where(amax > 0, E, 0).astype(np.int64)
    top = np.rint(np.ldexp(np.where(special, 0, amax).astype(np.float64), 23 - E))
    E = np.where((top > 8355328) & ~special, E + 1, E)
    xs = np.where(special[:, None], 0, x).astype(np.float64)
    q = np.rint(np.ldexp(xs, (23 - E)[:, None]))                        # exact integers, |q| < 2^23
    t = q @ np.asarray(codes_kc, np.float64)                              # exact: every partial sum < 2^53
    if f64:
        return np.ldexp(t, (E - 23)[:, None]), special
    v = np.ldexp(t, (E - 23)[:, None]).astype(np.float32)                 # one rounding to f32
    return (v * np.asarray(scale_c, np.float32)[None, :]).astype(np.float32), special


def reference_loop(x_mk, codes_kc, scale_c):
    """The reference's quantized product (runtime/tg_rt.h:132-151) for a few
    rows, vectorised over channels: acc = acc + (float)code * x in k order,
    each product and each sum rounded to f32 (no FMA), then s * acc in f32."""
    x = np.asarray(x_mk, np.float32)
    codes = np.asarray(codes_kc, np.float32)
    acc = np.zeros((x.shape[0], codes.shape[1]), np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        for k in range(x.shape[1]):
            acc = acc + codes[k][None, :] * x[:, k:k + 1]
        return acc * np.asarray(scale_c, np.float32)[None, :]


def split_rows_matmul(x_mk, codes_kc, scale_c):
    """Split rows (technograd_amd/csrc/kern_qgemm.hip: split_k, batches of
    TGK_SPLIT_ROWS rows or more): a peaked row's band entries (|x| >=
    max|x| / 4, nonzero) are outliers; the other entries are put on a grid of
    their own (E from their largest magnitude, as digit_path_matmul); each
    output is f32(g + o) * s[c] with g = t 2^(E-23) the grid sum and
    o = sum over the outliers in increasing k of code[k, c] x_k, both in f64
    (every product exact, o summed from 0.0 in k order)."""
    x = np.asarray(x_mk, np.float32)
    codes = np.asarray(codes_kc, np.float64)
    a = np.abs(x)
    amax = a.max(axis=1)
    band = np.ldexp(amax, np.int32(-2)).astype(np.float32)
    inb = (a >= band[:, None]) & (a != 0)
    rest = np.where(inb, np.float32(0), x)
    g, _ = digit_path_matmul(rest, codes_kc, np.ones(codes.shape[1], np.float32), peak=False, f64=True)
    out = np.empty((x.shape[0], codes.shape[1]), np.float32)
    for m in range(x.shape[0]):
        o = np.zeros(codes.shape[1])
        for k in np.flatnonzero(inb[m]):
            o = o + codes[k] * np.float64(x[m, k])
        out[m] = (g[m] + o).astype(np.float32) * np.asarray(scale_c, np.float32)
    return out


def device_path_matmul(x_mk, codes_kc, scale_c, peak=True, split=False):
    """What the device computes for x @ W: the digit path, and the reference's
    loop for special rows; with split (batches of TGK_SPLIT_ROWS rows or
    more) peaked rows that are finite and at most 2^100 are split rows
    instead (split_rows_matmul). Returns (f32 [M, C], special [M]): special
    marks the rows off the plain grid."""
    got, special = digit_path_matmul(x_mk, codes_kc, scale_c, peak)
    if special.any():
        x = np.asarray(x_mk, np.float32)
        ref = special.copy()
        if split:
            amax = np.abs(x).max(axis=1)
            sp = special & ~np.isnan(x).any(axis=1) & (amax <= np.float32(2.0 ** 100))
            if sp.any():
                got[sp] = split_rows_matmul(x[sp], codes_kc, scale_c)
            ref &= ~sp
        if ref.any():
            got[ref] = reference_loop(x[ref], codes_kc, scale_c)
    return got, special


def outlier_rows(K, codes_kc, seed=0):
    """Rows with outliers where the per-row grid would be too coarse, and
    rows that stay on the grid: one outlier 1e2, 1e3, 1e4, 1e6 times the rest
    on a column whose codes are all zero; two opposite outliers of 1e3 and
    1e5 on two columns with equal codes (their terms cancel); a single 14
    sigma entry; and three dense rows: nine entries at 30 sigma, a row
    scaled by 1e4 as a whole, a plain N(0, 1) row. codes_kc is modified:
    column z0 becomes all zero, column c1 a copy of c0. Returns (x [10, K],
    expected special flags [10])."""
    rng = np.random.default_rng(seed)
    z0, c0, c1 = 3, 10, K - 7
    codes_kc[z0] = 0
    codes_kc[c1] = codes_kc[c0]
    x = rng.normal(size=(10, K)).astype(np.float32)
    for i, f in enumerate((1e2, 1e3, 1e4, 1e6)):
        x[i, z0] = f
    x[4, c0], x[4, c1] = 1e3, -1e3
    x[5, c0], x[5, c1] = -1e5, 1e5
    x[6, K // 2] = 14.0
    x[7, rng.choice(K, 9, replace=False)] = 30.0
    x[8] *= 1e4
    return x, np.array([True] * 7 + [False] * 3)
