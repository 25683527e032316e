"""Every launch shape of the matrix-core path (technograd_amd/csrc/kern_qgemm.hip,
launch_gemm): the large-batch LDS kernel, each (NB column blocks, W waves)
instantiation of the small-batch kernel and the kernel for rows of at most
32 inputs, int4 and int8 weights, checked bit
for bit against the path's own arithmetic restated on the host
(tests/parity.py: device_path_matmul: the digit path, a split row for an
outlier, and the reference's loop for special rows). The reference-order parity of the same
entry point is in test_gpu_parity.py."""
import numpy as np
import pytest

from parity import device_path_matmul

pytestmark = pytest.mark.gpu

# (bits, M rows, K inputs, C channels): the comment names the kernel launch_gemm picks
SHAPES = [
    (4, 1024, 256, 4096),  # qgemm_k: 128 x 256 tiles, 128 of them
    (8, 1024, 320, 4096),  # qgemm_k, int8 weights, K not a multiple of 64
    (4, 4000, 300, 1000),  # qgemm_k, int4 channel pairs: rows, K and channels not multiples of 128, 64 and 64
    (4, 2100, 512, 4000),  # qgemm_k, int4: the last pair's second block all padding
    (4, 256, 4096, 4096),  # qgemv_k NB=4 W=4
    (4, 256, 2048, 4096),  # NB=4 W=2
    (8, 256, 512, 4096),   # NB=4 W=1
    (8, 256, 4096, 4096),  # NB=4 W=4, int8 weights
    (8, 256, 2048, 4096),  # NB=4 W=2, int8
    (8, 250, 2048, 2016),  # NB=2 W=2, int8, rows and channels not multiples of 32
    (4, 128, 4096, 4096),  # NB=2 W=4
    (8, 128, 2048, 4096),  # NB=2 W=2
    (4, 100, 256, 4096),   # NB=2 W=1, rows not a multiple of 32
    (4, 20, 8192, 4096),   # NB=1 W=8
    (8, 40, 1024, 4096),   # NB=1 W=4
    (4, 33, 640, 4096),    # NB=1 W=2
    (4, 50, 256, 4096),    # NB=1 W=1
    (8, 60, 8192, 2048),   # NB=1 W=8, int8
    (4, 64, 1024, 1000),   # NB=1, channels not a multiple of 32
    (4, 16, 8192, 4096),   # gemv16_k NS=8 W=16 (at most 16 rows)
    (4, 1, 4096, 4096),    # gemv1_k fused (one int4 row, digits made in the kernel): config 2 at B=1
    (4, 1, 8192, 2048),    # gemv1_k fused, NL=16
    (4, 1, 1000, 4096),    # gemv1_k on the digit kernel's digits (K not a multiple of 16)
    (8, 1, 4096, 4096),    # one int8 row: gemv16_k NS=8 W=8
    (4, 16, 4096, 4096),   # NS=8 W=8: config 2 at B=16
    (8, 5, 2048, 4096),    # NS=4 W=8, int8
    (4, 12, 3000, 4096),   # NS=8 W=8, int4, K not a multiple of 64
    (8, 7, 4096, 4096),    # NS=8 W=8, int8
    (8, 16, 1792, 2048),   # NS=4 W=8, int8
    (4, 5, 1000, 4096),    # NS=2 W=8, K not a multiple of 16 (the digit kernel's element loads)
    (8, 16, 1024, 4096),   # NS=2 W=8, int8
    (4, 3, 640, 4096),     # NS=2 W=8, K not a multiple of 64
    (4, 4, 448, 1000),     # NS=2 W=4, channels not a multiple of 16
    (4, 9, 384, 4096),     # NS=2 W=4
    (4, 2, 128, 1000),     # NS=1 W=4
    (4, 1, 256, 4096),     # gemv1_k fused, NL=1
    (8, 1, 256, 4096),     # gemv16_k NS=1 W=4
    (8, 2, 8192, 2048),    # int8 beyond 4096 inputs: qgemv_k NB=1 W=8
    (8, 2048, 16, 512),    # qtiny_k (at most 32 inputs, at least 1024 rows): one 16-input group
    (4, 1500, 30, 1000),   # qtiny_k, two groups, int4, channels not a multiple of 256
    (8, 1024, 1, 300),     # qtiny_k, one input
]


@pytest.mark.parametrize("bits_,M,K,C", SHAPES)
def test_launch_shape_bit_exact(bits_, M, K, C):
    from technograd_amd import hip
    print("case launch shape", bits_, M, K, C, flush=True)
    rng = np.random.default_rng(M * 131 + K * 7 + C + bits_)
    lim = 127 if bits_ == 8 else 7
    codes = rng.integers(-lim, lim + 1, size=(K, C)).astype(np.int8)  # x @ W: W [K][C], axis 1
    scales = rng.uniform(0.001, 0.1, size=C).astype(np.float32)
    if bits_ == 4:
        flat = codes.ravel().astype(np.int64)
        if flat.size % 2:
            flat = np.concatenate([flat, [0]])
        packed = ((flat[0::2] & 15) | ((flat[1::2] & 15) << 4)).astype(np.uint8).view(np.int8)
    else:
        packed = codes.ravel()
    x = rng.normal(size=(M, K)).astype(np.float32)
    x[0] *= 1e3  # rows of different magnitudes: different exponents per row
    if M > 2:
        x[2] *= 1e-30
    if M > 3:
        x[3, K // 3] = 1e4  # an outlier: its row leaves its grid (split)
    got = hip.matmul_q(packed, bits_, scales, x, M, K, C, 1)
    want, cls = device_path_matmul(x, codes, scales)
    assert M <= 3 or K < 16 or cls[3] != 0  # (one input: a lone large entry is the whole row, on its grid)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), np.argwhere(got != want)[:5].tolist()


@pytest.mark.parametrize("K", [4096, 1000])
def test_single_row_kinds(K):
    """One row at a time (the single-row kernel, fused at K = 4096, fed by
    the digit kernel at K = 1000): an outlier row (split), rows with inf,
    nan or an entry above 2^100 (special), a row of zeros, a tiny row and a
    plain row, each bit for bit against the path restated on the host."""
    from technograd_amd import hip
    print("case single rows", K, flush=True)
    rng = np.random.default_rng(K)
    C = 2048
    codes = rng.integers(-7, 8, size=(K, C)).astype(np.int8)
    scales = rng.uniform(0.001, 0.1, size=C).astype(np.float32)
    flat = codes.ravel().astype(np.int64)
    packed = ((flat[0::2] & 15) | ((flat[1::2] & 15) << 4)).astype(np.uint8).view(np.int8)
    rows = rng.normal(size=(7, K)).astype(np.float32)
    rows[0, K // 2] = 1e4
    rows[1, 5] = np.inf
    rows[2, 7] = np.nan
    rows[3, 9] = 2e30
    rows[4] = 0
    rows[5] *= 1e-30
    want, cls = device_path_matmul(rows, codes, scales)
    assert cls.tolist() == [2, 1, 1, 1, 0, 0, 0]
    for i in range(len(rows)):
        got = hip.matmul_q(packed, 4, scales, rows[i:i + 1], 1, K, C, 1)
        assert np.array_equal(np.isnan(got[0]), np.isnan(want[i]))
        ok = ~np.isnan(want[i])
        assert np.array_equal(got[0][ok].view(np.uint32), want[i][ok].view(np.uint32)), i

