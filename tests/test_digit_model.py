"""The host restatement of the matrix-core path's arithmetic
(parity.digit_path_matmul), which the GPU launch-shape tests compare against
bit for bit, pinned on the CPU: to the exact real product within the 24-bit
activation grid's bound, to the reference's sequential order (the oracle)
under the parity predicate, on rows with outliers (the peak test sends them
to the reference's loop, and without it the predicate fails), and on cases
whose answer is fixed by hand."""
import numpy as np
import pytest

from oracle import oracle as O
from technograd_amd import synth
from parity import (check_qmatmul, device_path_matmul, digit_path_matmul, grid_bound, outlier_rows, peaked_rows,
                    qmatmul_truth, reference_loop, ulp)


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
    """K = 4096: rows with one outlier of 1e2 to 1e6 on a zero-code column,
    cancelling outliers, a 14 sigma entry, and dense rows. What the device
    computes (the digit path, the reference's loop for special rows) against
    the oracle: peaked rows are special and bit-identical with the oracle; the
    rest pass the parity predicate. With the peak test taken out (the per-row
    grid for every row), the predicate fails."""
    K, C = 4096, 256
    lim = 7 if bits == 4 else 127
    rng = np.random.default_rng(bits)
    codes = rng.integers(-lim, lim + 1, size=(K, C)).astype(np.int8)
    scales = rng.uniform(0.001, 0.1, size=C).astype(np.float32)
    x, want_special = outlier_rows(K, codes)
    assert np.array_equal(peaked_rows(x), want_special)
    text = synth.linear_tgir_codes("lq", codes, scales, bits, axis=1)
    ref, _ = O.Model(text).batch(x)
    got, special = device_path_matmul(x, codes, scales)
    assert np.array_equal(special, want_special)
    assert np.array_equal(got[special].view(np.uint32), ref[special].view(np.uint32))
    check_qmatmul(got, ref, codes.T, scales, x)
    coarse, _ = device_path_matmul(x, codes, scales, peak=False)
    with pytest.raises(AssertionError):
        check_qmatmul(coarse, ref, codes.T, scales, x)


@pytest.mark.parametrize("bits", [4, 8])
def test_split_rows_against_the_oracle(bits):
    """The split of peaked rows (large batches): the same outlier rows through
    split_rows_matmul pass the parity predicate against the oracle, and each
    split row is within its own grid's bound of the exact product (the grid
    set by the entries below the band, not by the outlier), plus one f32
    rounding."""
    K, C = 4096, 256
    lim = 7 if bits == 4 else 127
    rng = np.random.default_rng(bits + 10)
    codes = rng.integers(-lim, lim + 1, size=(K, C)).astype(np.int8)
    scales = rng.uniform(0.001, 0.1, size=C).astype(np.float32)
    x, want_special = outlier_rows(K, codes)
    text = synth.linear_tgir_codes("lq", codes, scales, bits, axis=1)
    ref, _ = O.Model(text).batch(x)
    got, special = device_path_matmul(x, codes, scales, split=True)
    assert np.array_equal(special, want_special)
    check_qmatmul(got, ref, codes.T, scales, x)
    truth, _ = qmatmul_truth(codes.T, scales, x)
    rest = np.where(np.abs(x) >= np.ldexp(np.abs(x).max(axis=1), -2)[:, None], 0, x)
    bound = grid_bound(codes.T, scales, rest) + np.abs(truth) * 2.0 ** -23
    assert (np.abs(got[special] - truth[special]) <= bound[special]).all()


def test_split_hand_case():
    """integers: the rest's grid holds them exactly and the outlier term is
    exact, so a split row's output is the exact product rounded once"""
    x = np.zeros((1, 40), np.float32)
    x[0, :39] = np.arange(1, 40) % 7 - 3
    x[0, 39] = 1000.0
    codes = (np.arange(40 * 3).reshape(40, 3) % 5 - 2).astype(np.int8)
    assert peaked_rows(x).all()
    got, special = device_path_matmul(x, codes, np.ones(3, np.float32), split=True)
    want = (x.astype(np.float64) @ codes.astype(np.float64)).astype(np.float32)
    assert special.all() and np.array_equal(got, want)
    # without the split the same row takes the reference's loop
    got0, _ = device_path_matmul(x, codes, np.ones(3, np.float32))
    assert np.array_equal(got0, reference_loop(x, codes, np.ones(3, np.float32)))


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
