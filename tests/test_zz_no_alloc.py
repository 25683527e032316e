"""tg_hip_matmul_q_noalloc (include/tg_hip.h): the matrix-core quantized
product with no device allocation, its packed weights and digits in the
library's fixed scratch array. Called through the C ABI on device buffers
and checked bit for bit against tg_hip_matmul_q (the same kernels, with
scratch it allocates per call), twice in a row with the second call
smaller (the array keeps the first call's contents), then a call too large
for the array, which must be refused."""
import ctypes

import numpy as np
import pytest

from technograd_amd import hip

pytestmark = pytest.mark.gpu


def _pack(codes, bits):
    if bits == 8:
        return codes.ravel()
    flat = codes.ravel().astype(np.int64)
    if flat.size % 2:
        flat = np.concatenate([flat, [0]])
    return ((flat[0::2] & 15) | ((flat[1::2] & 15) << 4)).astype(np.uint8).view(np.int8)


def _case(seed, bits, axis, m, k, n):
    rng = np.random.default_rng(seed)
    lim = 127 if bits == 8 else 7
    codes = rng.integers(-lim, lim + 1, size=(m, k) if axis == 0 else (k, n)).astype(np.int8)
    scales = rng.uniform(0.001, 0.1, size=m if axis == 0 else n).astype(np.float32)
    b = rng.normal(size=(k, n) if axis == 0 else (m, k)).astype(np.float32)
    if axis == 1 and m > 3:
        b[3, k // 2] = 1e4  # an outlier: a split row (its outlier terms read the caller's codes)
    return _pack(codes, bits), scales, b


def _noalloc(q, bits, s, b, m, k, n, axis):
    dq, ds, db = (hip.DeviceBuffer.from_array(a) for a in (q, s, b))
    do = hip.DeviceBuffer(m * n * 4)
    rc = hip.matmul_q_noalloc(do.ptr, dq.ptr, bits, ds.ptr, db.ptr, m, k, n, axis)
    assert rc == 0, hip.error()
    return do.to_array(np.float32, (m, n))  # a blocking copy on the null stream: after the product


def test_no_alloc_equals_matmul_q_twice_then_refuses():
    print("case no-alloc entry point", flush=True)
    hip.init(0)
    # first: config 2's layer at 2048 rows (x @ W^T as axis 0: 4096 x 4096 int4, b [4096][2048]);
    # second, smaller: int8 weights on axis 1 with an outlier row, odd sizes
    for seed, (bits, axis, m, k, n) in enumerate([(4, 0, 4096, 4096, 2048), (8, 1, 300, 500, 17)]):
        q, s, b = _case(seed, bits, axis, m, k, n)
        got = _noalloc(q, bits, s, b, m, k, n, axis)
        want = hip.matmul_q(q, bits, s, b, m, k, n, axis)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (bits, axis, m, k, n)
    # the documented limit (include/tg_hip.h): config 2's layer fits at 6528 rows, not at 6529
    rc = hip.matmul_q_noalloc(1, 1, 4, 1, 1, 4096, 4096, 6529, 0)
    assert rc == -2 and "scratch" in hip.error()
    # 8192 x 16384 int8 weights alone need 128 MiB: refused before any launch
    rc = hip.matmul_q_noalloc(1, 1, 8, 1, 1, 8192, 16384, 1, 0)
    assert rc == -2 and "scratch" in hip.error()


def test_no_alloc_at_its_documented_limit():
    """Config 2's 4096 x 4096 int4 layer at 6528 activation rows (axis 0,
    the largest call the header promises), after a call of 4096 rows: both
    equal tg_hip_matmul_q bit for bit."""
    print("case no-alloc at the limit", flush=True)
    hip.init(0)
    for seed, n in ((7, 6528), (8, 4096)):
        q, s, b = _case(seed, 4, 0, 4096, 4096, n)
        got = _noalloc(q, 4, s, b, 4096, 4096, n, 0)
        want = hip.matmul_q(q, 4, s, b, 4096, 4096, n, 0)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), n
