"""The host restatement of the matrix-core path's arithmetic
(parity.digit_path_matmul, parity.device_path_matmul), which the GPU tests
compare against bit for bit, pinned on the CPU: to the exact real product
within the 24-bit activation grid's bound, to the reference's sequential
order (the oracle) under the parity predicate, on rows with outliers (the
row classes split them or send them to the reference's loop; with one grid
per row the predicate fails), and on cases whose answer is fixed by hand."""
import numpy as np
import pytest

from oracle import oracle as O
from technograd_amd import synth
from parity import acoef, coarse_groups, jcap
from parity import (candidates, check_qmatmul, coarse_grid, device_path_matmul, digit_path_matmul, grid_bound, grid_rows,
                    outlier_mask, outlier_rows, qmatmul_truth, reference_loop, resolve_row, row_classes, ulp)


def _case(seed, M=7, K=96, C=40, lim=7):
    rng = np.random.default_rng(seed)
    codes = rng.integers(-lim, lim + 1, size=(K, C)).astype(np.int8)
    scales = rng.uniform(0.001, 0.1, size=C).astype(np.float32)
    x = rng.normal(size=(M, K)).astype(np.float32)
    x[1] *= 1e6
    x[2] *= 1e-20
    return x, codes, scales


def test_within_the_grid_bound_of_the_exact_product():
    for seed in range(5):
        x, codes, scales = _case(seed)
        got, special = digit_path_matmul(x, codes, scales)
        truth = (x.astype(np.float64) @ codes.astype(np.float64)) * scales.astype(np.float64)
        assert not special.any()
        assert (np.abs(got - truth) <= grid_bound(codes.T, scales, x) + 2 * ulp(truth)).all()


def test_within_the_parity_predicate_of_the_reference_order():
    for seed in range(3):
        x, codes, scales = _case(seed + 10)
        got, _ = digit_path_matmul(x, codes, scales)
        ref = reference_loop(x, codes, scales)
        check_qmatmul(got, ref, codes.T, scales, x)


def test_reference_loop_is_the_oracle():
    """parity.reference_loop (used for special rows below) equals the oracle's
    quantized product bit for bit, both axes' layout as x @ W."""
    rng = np.random.default_rng(4)
    codes = rng.integers(-7, 8, size=(300, 20)).astype(np.int8)
    scales = rng.uniform(0.001, 0.1, size=20).astype(np.float32)
    x = rng.normal(size=(5, 300)).astype(np.float32)
    x[1, 9] = 1e5
    text = synth.linear_tgir_codes("lq", codes, scales, 4, axis=1)
    want, _ = O.Model(text).batch(x)
    assert np.array_equal(reference_loop(x, codes, scales).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", [4, 8])
def test_outlier_rows_against_the_oracle(bits):
    """K = 4096: rows with 1 to 64 outliers of 1e2 to 1e6 (on all-zero code
    columns and on columns with codes), cancelling outliers, a 14 sigma
    entry, and dense rows. Every planted row leaves its single grid (split,
    or the reference's loop) and the dense rows keep it; what the device
    computes passes the parity predicate against the oracle, rows of the
    reference's loop bit for bit, and each split row is within its own
    grid's bound of the exact product (the grid of the entries other than
    its outliers) plus one f32 rounding. With one grid per row (no classes)
    the predicate fails."""
    K, C = 4096, 256
    lim = 7 if bits == 4 else 127
    rng = np.random.default_rng(bits)
    codes = rng.integers(-lim, lim + 1, size=(K, C)).astype(np.int8)
    scales = rng.uniform(0.001, 0.1, size=C).astype(np.float32)
    x, planted = outlier_rows(K, codes)
    cls, level, E = row_classes(x)
    assert (cls[planted] != 0).all() and (cls[7:10] == 0).all(), cls
    text = synth.linear_tgir_codes("lq", codes, scales, bits, axis=1)
    ref, _ = O.Model(text).batch(x)
    got, cls2 = device_path_matmul(x, codes, scales)
    assert np.array_equal(cls, cls2)
    assert np.array_equal(got[cls == 1].view(np.uint32), ref[cls == 1].view(np.uint32))
    check_qmatmul(got, ref, codes.T, scales, x)
    sp = cls == 2
    truth, _ = qmatmul_truth(codes.T, scales, x)
    rest = np.where(outlier_mask(x[sp], E[sp], level[sp]), 0, x[sp])
    bound = grid_bound(codes.T, scales, rest) + np.abs(truth[sp]) * 2.0 ** -23
    assert (np.abs(got[sp] - truth[sp]) <= bound).all()
    coarse, _ = digit_path_matmul(x, codes, scales)
    with pytest.raises(AssertionError):
        check_qmatmul(coarse, ref, codes.T, scales, x)


@pytest.mark.parametrize("kind", ["gauss", "laplace", "t3", "silu_up", "sparse"])
def test_dense_and_heavy_tailed_rows(kind):
    """Rows without planted outliers, at the configs' widths: Gaussian,
    Laplace, Student t(3), products silu(g) * u (config 3's and 5's gated
    activations) and 95 %-sparse Gaussian rows. The device path passes the
    parity predicate against the oracle; Gaussian and Laplace rows of 1024
    or more inputs all keep their grid."""
    rng = np.random.default_rng(len(kind))
    for K in (64, 512, 1024, 3072):
        C, M = 64, 48
        codes = rng.integers(-7, 8, size=(K, C)).astype(np.int8)
        scales = rng.uniform(0.001, 0.1, size=C).astype(np.float32)
        if kind == "gauss":
            x = rng.normal(size=(M, K))
        elif kind == "laplace":
            x = rng.laplace(size=(M, K))
        elif kind == "t3":
            x = rng.standard_t(3, size=(M, K))
        elif kind == "silu_up":
            g = rng.normal(size=(M, K))
            x = g / (1 + np.exp(-g)) * rng.normal(size=(M, K))
        else:
            x = rng.normal(size=(M, K)) * (rng.random((M, K)) < 0.05)
        x = x.astype(np.float32)
        text = synth.linear_tgir_codes("lq", codes, scales, 4, axis=1)
        ref, _ = O.Model(text).batch(x)
        got, cls = device_path_matmul(x, codes, scales)
        check_qmatmul(got, ref, codes.T, scales, x)
        if kind in ("gauss", "laplace") and K >= 1024:
            assert (cls == 0).all()


def _coarse_rows():
    """(kind, K, x [M, K]) of Gaussian, Student t(3), gated (silu x up, config
    3's and 5's activations), 90 %-sparse and planted-outlier rows"""
    rng = np.random.default_rng(11)
    for K in (16, 64, 512, 3072):
        M = 200
        g = rng.normal(size=(M, K))
        sets = {"gauss": rng.normal(size=(M, K)), "t3": rng.standard_t(3, size=(M, K)),
                "silu_up": g / (1 + np.exp(-g)) * rng.normal(size=(M, K)),
                "sparse": rng.normal(size=(M, K)) * (rng.random((M, K)) < 0.1)}
        if K >= 512:
            codes = rng.integers(-7, 8, size=(K, 8)).astype(np.int8)
            sets["outliers"] = outlier_rows(K, codes, seed=K)[0]
        for kind, x in sets.items():
            yield kind, K, x.astype(np.float32)


def _coarse_check(test):
    """per (kind, K): [rows the test settles, candidates the full resolve keeps on the grid,
    settled rows the full resolve does not keep on the grid]"""
    out = {}
    for kind, K, x in _coarse_rows():
        special, E = grid_rows(x)
        cand, n = candidates(x)
        st = out.setdefault((kind, K), [0, 0, 0])
        for m in np.flatnonzero(cand):
            c = test(x[m], int(E[m]), int(n[m]))
            grid = resolve_row(x[m], int(E[m]), int(n[m])) == 0
            st[0] += c
            st[1] += grid
            st[2] += c and not grid
    return out


def test_coarse_test_implies_the_grid():
    """The producers' coarse test (tgq_coarse_grid) settles a candidate as a
    grid row only where the full resolve keeps its grid too: every row it
    passes resolves to level 0. Of the gated rows' candidates of 512 and more
    inputs that the full resolve keeps on the grid, it settles most (the
    point of it)."""
    st = _coarse_check(coarse_grid)
    print("coarse test (settled, grid candidates, wrong):", st)
    assert sum(v[2] for v in st.values()) == 0
    gated = [st[("silu_up", K)] for K in (512, 3072)] + [st[("t3", K)] for K in (512, 3072)]
    assert sum(v[0] for v in gated) > 0.8 * sum(v[1] for v in gated)


def test_coarse_check_catches_a_slip():
    """The implication check has teeth: the same test asking the rest for A
    units of 2^(E-2) whatever its first nonempty group (a plausible slip:
    the merged group's index in place of the rest's top bin) settles rows
    that the full resolve splits."""
    def slipped(x_k, E, n):
        c0, c1, nz, s0, s1, aq = coarse_groups(x_k, E)
        cnt, sq = [c0, c1, nz - c0 - c1], [s0, s1, aq - s0 - s1]
        r = next(d for d in range(3) if cnt[d])
        left, top = jcap(n), 0
        for d in range(r, 3):
            if left == 0:
                break
            take = min(cnt[d], left)
            top += (sq[d] << 21) + (cnt[d] << 20) if take == cnt[d] else take << (44 - d)
            left -= take
        return (aq << 21) - (nz << 20) - top >= acoef(n) << (44 - 2)
    st = _coarse_check(slipped)
    assert sum(v[2] for v in st.values()) > 0, st


def test_row_classes_hand_cases():
    """Integers on the row's grid are exact whatever their spread: no
    candidate, the exact product rounded once. The same spread with the
    small entries off the full grid (multiples of 2^-20 next to 1000) is
    split at the first level: the rest's own grid holds it exactly and the
    outlier term is exact, so the output is again the exact product rounded
    once, where one grid would lose the small entries."""
    codes = (np.arange(40 * 3).reshape(40, 3) % 5 - 2).astype(np.int8)
    one = np.ones(3, np.float32)
    x = np.zeros((2, 40), np.float32)
    x[:, :39] = np.arange(1, 40) % 7 - 3
    x[:, 39] = 1000.0
    x[1, :39] *= np.float32(2.0 ** -20)
    cls, level, _ = row_classes(x)
    assert cls.tolist() == [0, 2] and level[1] == 1
    got, _ = device_path_matmul(x, codes, one)
    want = (x.astype(np.float64) @ codes.astype(np.float64)).astype(np.float32)
    assert np.array_equal(got, want)
    coarse, _ = digit_path_matmul(x[1:], codes, one)
    assert not np.array_equal(coarse, want[1:])


def test_hand_cases():
    # small integers: every q is x * 2^(23 - E) exactly and the sum is exact, so the
    # result is the exact product, rounded once
    x = np.array([[1, 2, 3, -4], [0, 0, 0, 0], [0.5, 0, 0, 0]], np.float32)
    codes = np.array([[1], [1], [1], [1]], np.int8)
    got, special = digit_path_matmul(x, codes, np.ones(1, np.float32))
    assert got[:, 0].tolist() == [2.0, 0.0, 0.5] and not special.any()
    # the top digit bump: x = 1 - 2^-24 has E = 0, but rint(x 2^23) = 2^23 (a tie, to
    # even) leaves the top digit's range, so E = 1 and q = rint(x 2^22) = 2^22: the
    # 24-bit grid gives exactly 1.0 (an error of 2^-24 = 2^-23 max |x| / 2)
    x = np.array([[np.float32(1) - np.float32(2.0 ** -24)]], np.float32)
    got, _ = digit_path_matmul(x, np.array([[1]], np.int8), np.ones(1, np.float32))
    assert got[0, 0] == np.float32(1.0)
    # just inside the range: 0.99 2^23 rounds to 8304722 < 8355328, no bump, exact to 2^-24
    x = np.array([[0.99]], np.float32)
    got, _ = digit_path_matmul(x, np.array([[1]], np.int8), np.ones(1, np.float32))
    assert got[0, 0] == np.float32(np.rint(np.float64(np.float32(0.99)) * 2 ** 23) / 2 ** 23)
    # special rows: a NaN, an infinity, or max |x| above 2^100
    x = np.array([[np.nan, 1], [np.inf, 1], [2.0 ** 101, 1], [1, 1]], np.float32)
    _, special = digit_path_matmul(x, np.ones((2, 1), np.int8), np.ones(1, np.float32))
    assert special.tolist() == [True, True, True, False]
