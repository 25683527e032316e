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
import math

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
    on their grid: the 24-bit activation grid, 2^-23 max|x| per element
    (tests of the host restatement only; not a parity predicate)."""
    codes = np.asarray(codes_ck, np.float64)
    x = np.asarray(x_mk, np.float64)
    s = np.abs(np.asarray(scale_c, np.float64))
    return 2.0 ** -23 * s[None, :] * np.abs(x).max(axis=1)[:, None] * np.abs(codes).sum(axis=1)[None, :]


# Row classes (technograd_amd/csrc/tg_qdigits.h), restated: which rows keep
# their 24-bit grid, which are split (outliers as exact terms, the rest on a
# grid of its own), which take the reference's loop. Integer arithmetic
# only, as on the device.
MAX_OUT = 64     # outliers of a split row, at most (TGQ_MAX_OUT)
MASS_SHIFT = 44  # the histogram's mass unit 2^(E-44) (TGQ_MASS_SHIFT)


def jcap(n):
    """J(n): how many of a row's largest entries may be outliers."""
    return 1 if n < 32 else MAX_OUT if n >= 16 * MAX_OUT else n >> 4


def acoef(n):
    """A(n) = ceil(3 isqrt(n) / 4): grid steps the rest must hold."""
    return (3 * math.isqrt(int(n)) + 3) >> 2


def grid_rows(x_mk):
    """(special [M], E [M]): special rows have a NaN, or max |x| above 2^100
    (inf included); E from max |x| (frexp), raised by one when
    rint(max |x| 2^(23-E)) > 8355328; 0 for special and all-zero rows."""
    x = np.asarray(x_mk, np.float32)
    a = np.abs(x)
    nan = np.isnan(x).any(axis=1)
    with np.errstate(invalid="ignore"):
        amax = np.where(nan, np.float32(0), a.max(axis=1)).astype(np.float32)
    special = nan | (amax > np.float32(2.0 ** 100))
    _, E = np.frexp(np.where(special, 0, amax).astype(np.float64))
    E = np.where(amax > 0, E, 0).astype(np.int64)
    top = np.rint(np.ldexp(np.where(special, 0, amax).astype(np.float64), 23 - E))
    E = np.where((top > 8355328) & ~special, E + 1, E)
    return special, np.where(special, 0, E)


def candidates(x_mk):
    """The producers' test (tgq_candidate): (candidate [M], n [M]) with n the
    entries inexact on the row's grid; a candidate has n > 0 and
    sum |q| < (J(n) + A(n)) 2^23."""
    x = np.asarray(x_mk, np.float32)
    special, E = grid_rows(x)
    xs = np.where(special[:, None], 0, x).astype(np.float64)
    v = np.ldexp(xs, (23 - E)[:, None])
    q = np.rint(v)
    n = (q != v).sum(axis=1)
    mass = np.abs(q).sum(axis=1)
    thr = np.array([(jcap(int(k)) + acoef(int(k))) << 23 for k in n], np.float64)
    return ~special & (n > 0) & (mass < thr), n


def _bins(a, E):
    """bin of each |x| > 0: E - (frexp exponent), at most 63"""
    _, e = np.frexp(a)
    return np.minimum(E - e, 63)


def resolve_row(x_k, E, n):
    """tgq_decide on one candidate row: the peel level (0 the grid, L > 0 a
    split at level L, -1 the reference's loop)."""
    a = np.abs(np.asarray(x_k, np.float32).astype(np.float64))
    a = a[a != 0]
    d = _bins(a, E)
    mass = np.floor(np.ldexp(a, MASS_SHIFT - E)).astype(np.int64)
    cnt = np.bincount(d, minlength=64)
    ms = np.zeros(64, np.int64)
    np.add.at(ms, d, mass)
    J, A = jcap(n), acoef(n)
    P = np.concatenate([[0], np.cumsum(cnt)])
    for L in range(64):
        if P[L] > J:
            continue
        nz = np.flatnonzero(cnt[L:])
        if len(nz) == 0:
            return L
        r = L + int(nz[0])
        if r > MASS_SHIFT:
            continue
        left, top = J, 0
        for dd in range(r, 64):  # the rest's J largest, bin by bin from its top
            take = min(int(cnt[dd]), left)
            top += int(ms[dd]) if take == cnt[dd] else (take << (MASS_SHIFT - dd) if dd <= MASS_SHIFT else 0)
            left -= take
            if left == 0:
                break
        if int(ms[L:].sum()) - top >= A << (MASS_SHIFT - r):
            return L
    return -1


def coarse_groups(x_k, E):
    """the coarse test's integers (tgq_coarse16 summed over the row): counts
    of |q| >= 2^22, of 2^21 <= |q| < 2^22 and of nonzero entries; the first
    two groups' sums of |q|; the row's sum of |q|"""
    x = np.asarray(x_k, np.float32).astype(np.float64)
    aq = np.abs(np.rint(np.ldexp(x, 23 - E))).astype(np.int64)
    g0, g1 = aq >= 2 ** 22, (aq >= 2 ** 21) & (aq < 2 ** 22)
    return (int(g0.sum()), int(g1.sum()), int((x != 0).sum()), int(aq[g0].sum()), int(aq[g1].sum()), int(aq.sum()))


def coarse_grid(x_k, E, n):
    """tgq_coarse_grid on one candidate row (grid exponent E, n inexact
    entries): tgq_decide's level-0 test on three groups of q (|q| >= 2^22,
    2^21 <= |q| < 2^22, the other nonzero entries), a whole group counting
    (|q| + 1/2) 2^21 per entry, a group taken in part 2^44, 2^43 or 2^42 per
    taken entry, the row's mass counted as sum (|q| - 1/2) 2^21 over its
    nonzero entries. Passing it implies resolve_row(...) == 0."""
    c0, c1, nz, s0, s1, aq = coarse_groups(x_k, E)
    cnt, sq = [c0, c1, nz - c0 - c1], [s0, s1, aq - s0 - s1]
    nzs = [d for d in range(3) if cnt[d]]
    if not nzs:
        return False
    r = nzs[0]
    left, top = jcap(n), 0
    for d in range(r, 3):
        if left == 0:
            break
        take = min(cnt[d], left)
        top += (sq[d] << 21) + (cnt[d] << 20) if take == cnt[d] else take << (MASS_SHIFT - d)
        left -= take
    return (aq << 21) - (nz << 20) - top >= acoef(n) << (MASS_SHIFT - r)


def row_classes(x_mk):
    """(cls [M], level [M], E [M]) as the device decides them: cls 0 a row on
    its grid, 1 the reference's loop (special rows, and candidates no level
    resolves), 2 a split row at peel level `level` (outliers: nonzero
    entries with |x| >= 2^(E - level))."""
    x = np.asarray(x_mk, np.float32)
    special, E = grid_rows(x)
    cand, n = candidates(x)
    cls = np.where(special, 1, 0)
    level = np.zeros(x.shape[0], np.int64)
    for m in np.flatnonzero(cand):
        L = resolve_row(x[m], int(E[m]), int(n[m]))
        cls[m] = 1 if L < 0 else 2 if L > 0 else 0
        level[m] = max(L, 0)
    return cls, level, E


def outlier_mask(x_mk, E, level):
    """the outliers of split rows at their levels (nonzero, bin below level)"""
    a = np.abs(np.asarray(x_mk, np.float32).astype(np.float64))
    with np.errstate(divide="ignore"):
        d = _bins(np.where(a == 0, 1.0, a), np.asarray(E)[:, None])
    return (a != 0) & (d < np.asarray(level)[:, None])


def digit_path_matmul(x_mk, codes_kc, scale_c, f64=False):
    """The matrix-core path's arithmetic for rows on their grid, restated on
    the host (not the reference's order): per row, E from max |x|
    (grid_rows), q = rint(x 2^(23-E)) exactly, the exact integer sum
    t = sum_k code[k, c] q[m, k], then f32(t 2^(E-23)) * s[c] in f32. Rows
    with a NaN or max |x| above 2^100 (inf included) are special: the device
    runs the reference's loop for them; they are returned masked.
    f64: return the grid sums t 2^(E-23) unrounded (scale_c not applied).
    Returns (f32 [M, C], special [M])."""
    x = np.asarray(x_mk, np.float32)
    special, E = grid_rows(x)
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


def split_rows_matmul(x_mk, codes_kc, scale_c, omask):
    """Split rows (kern_qgemm.hip: resolve_k and the epilogue): the outliers
    (omask) are exact terms, the other entries are put on a grid of their
    own (E from their largest magnitude, as digit_path_matmul); each output
    is f32(g + o) * s[c] with g = t 2^(E-23) the grid sum and o = sum over
    the outliers in increasing k of code[k, c] x_k, both in f64 (every
    product exact, o summed from 0.0 in k order)."""
    x = np.asarray(x_mk, np.float32)
    codes = np.asarray(codes_kc, np.float64)
    rest = np.where(omask, np.float32(0), x)
    g, _ = digit_path_matmul(rest, codes_kc, np.ones(codes.shape[1], np.float32), f64=True)
    out = np.empty((x.shape[0], codes.shape[1]), np.float32)
    for m in range(x.shape[0]):
        o = np.zeros(codes.shape[1])
        for k in np.flatnonzero(omask[m]):
            o = o + codes[k] * np.float64(x[m, k])
        out[m] = (g[m] + o).astype(np.float32) * np.asarray(scale_c, np.float32)
    return out


REFLOOP_K = 32  # kern_qgemm.hip (tg_kern.h: TGK_REFLOOP_K)


def device_path_matmul(x_mk, codes_kc, scale_c):
    """What the device computes for x @ W, at any batch size: rows on their
    grid (digit_path_matmul), split rows (split_rows_matmul) and the
    reference's loop, by row_classes; products over at most REFLOOP_K inputs
    take the reference's loop for every row. Returns (f32 [M, C], cls [M])."""
    x = np.asarray(x_mk, np.float32)
    if x.shape[1] <= REFLOOP_K:
        return reference_loop(x, codes_kc, scale_c), np.ones(x.shape[0], np.int64)
    got, _ = digit_path_matmul(x, codes_kc, scale_c)
    cls, level, E = row_classes(x)
    sp = cls == 2
    if sp.any():
        got[sp] = split_rows_matmul(x[sp], codes_kc, scale_c, outlier_mask(x[sp], E[sp], level[sp]))
    if (cls == 1).any():
        got[cls == 1] = reference_loop(x[cls == 1], codes_kc, scale_c)
    return got, cls


def outlier_rows(K, codes_kc, seed=0):
    """Rows with outliers where one grid for the row would be too coarse,
    and rows that stay on their grid. codes_kc is modified: its first
    64 + 3 columns of a seeded permutation become all-zero codes (z0 and the
    zero-code outlier columns) and column c1 a copy of c0. Rows:
      0-3  one outlier 1e2, 1e3, 1e4, 1e6 times the rest on an all-zero column;
      4-5  two opposite outliers (1e3, 1e5) on two columns with equal codes
           (their terms cancel);
      6    a single 14 sigma entry;
      7-8  nine entries at 30 sigma, a row scaled by 1e4 as a whole;
      9    a plain N(0, 1) row;
      10-33 n = 9, 16, 32, 64 outliers of 1e2, 1e3, 1e4 (random signs), on
           all-zero columns (even rows) and on columns with codes (odd rows).
    Returns (x [34, K], planted [34]: rows 0-5 and 10-33, whose outliers
    must not leave them on one grid)."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(K)
    z0, c0, c1 = int(perm[0]), int(perm[1]), int(perm[2])
    zcols = perm[3:3 + min(64, K - 3)]
    codes_kc[z0] = 0
    codes_kc[zcols] = 0
    codes_kc[c1] = codes_kc[c0]
    live = perm[3 + len(zcols):]
    x = rng.normal(size=(34, K)).astype(np.float32)
    for i, f in enumerate((1e2, 1e3, 1e4, 1e6)):
        x[i, z0] = f
    x[4, c0], x[4, c1] = 1e3, -1e3
    x[5, c0], x[5, c1] = -1e5, 1e5
    x[6, K // 2] = 14.0
    x[7, rng.choice(K, 9, replace=False)] = 30.0
    x[8] *= 1e4
    i = 10
    for n in (9, 16, 32, 64):
        for f in (1e2, 1e3, 1e4):
            for cols in (zcols, live):
                sel = rng.choice(cols, min(n, len(cols)), replace=False)
                x[i, sel] = (f * rng.choice([-1.0, 1.0], len(sel))).astype(np.float32)
                i += 1
    planted = np.zeros(34, bool)
    planted[:6] = True
    planted[10:] = True
    return x, planted
