"""The host restatement of the matrix-core path's arithmetic
(parity.digit_path_matmul), which the GPU launch-shape tests compare against
bit for bit, pinned on the CPU: to the exact real product within the 24-bit
activation grid's bound, to the reference's sequential order (the oracle)
within the parity bound, and on cases whose answer is fixed by hand."""
import numpy as np

from parity import digit_path_matmul, qmatmul_bound, ulp


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
        grid = 2.0 ** -23 * np.abs(x).max(axis=1)[:, None].astype(np.float64) * np.abs(codes).sum(axis=0)[None, :] * scales
        assert not special.any()
        assert (np.abs(got - truth) <= grid + 2 * ulp(truth)).all()


def test_within_the_parity_bound_of_the_reference_order():
    for seed in range(3):
        x, codes, scales = _case(seed + 10)
        got, _ = digit_path_matmul(x, codes, scales)
        ref = np.zeros_like(got)  # the reference's loop: f32 adds in k order, then the scale
        for m in range(x.shape[0]):
            for c in range(codes.shape[1]):
                acc = np.float32(0)
                for k in range(x.shape[1]):
                    acc = np.float32(acc + np.float32(codes[k, c]) * x[m, k])
                ref[m, c] = np.float32(scales[c] * acc)
        bound = qmatmul_bound(codes.T, scales, x) + 2 * ulp(ref)
        assert (np.abs(got.astype(np.float64) - ref) <= bound).all()


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
