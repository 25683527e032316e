"""Host checks of the row programs' Q16.16 element functions
(technograd_amd/csrc/tg_rowdev.h: the one header that both the row-program
interpreter and the per-model compiled row programs include), built with the
host clang++ and compared with the oracle's restatement of runtime/tg_rtq.h:30-145 on edge
values and dense random samples. The oracle's primitives are pinned by the
reference's emitted fixed-point units (test_oracle.py)."""
import ctypes
import math
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
I32 = (-(1 << 31), (1 << 31) - 1)
CLANG = "/opt/rocm/llvm/bin/clang++"  # the header uses clang's saturating builtins


@pytest.fixture(scope="module")
def lib(tmp_path_factory):
    if not os.path.exists(O.LIB_PATH):
        O.build(ref=False)
    so = tmp_path_factory.mktemp("rowdev") / "rowdev.so"
    subprocess.run([CLANG, "-O2", "-std=c++17", "-shared", "-fPIC", "-ffp-contract=off", "-I",
                    os.path.join(ROOT, "technograd_amd", "csrc"), "-o", str(so),
                    os.path.join(ROOT, "tests", "cpp", "rowdev_check.cpp")], check=True)
    d = ctypes.CDLL(str(so))
    d.rowdev_prim.restype = ctypes.c_long
    d.rowdev_prim.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_long]
    d.rowdev_prim_n.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long]
    d.rowdev_const.restype = ctypes.c_long
    d.rowdev_const.argtypes = [ctypes.c_int]
    o = O.lib().tgo_fx_prim
    o.restype = ctypes.c_int64
    o.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64]
    return d, o


def edge_values():
    v = [0, 1, -1, 2, -2, 32767, 32768, -32768, 65535, 65536, -65536, 65537, I32[0], I32[0] + 1, I32[1], I32[1] - 1]
    for k in range(-20, 20):  # around multiples of ln 2 and the exp cut-offs
        v += [45426 * k + d for d in (-1, 0, 1)]
    v += [681389, 681390, 681391, -786431, -786432, -786433, 9 * 65536, 9 * 65536 + 1, -9 * 65536 - 1]
    v += [205887 * k + d for k in range(-4, 5) for d in (-1, 0, 1)]
    return [x for x in v if I32[0] <= x <= I32[1]]


@pytest.mark.parametrize("op,name", [(2, "expq"), (3, "logq"), (5, "sinq"), (6, "tanhq"), (7, "sigmoidq")])
def test_unary_primitives_equal_the_oracle(lib, op, name):
    d, o = lib
    rng = np.random.default_rng(op)
    xs = edge_values() + [int(v) for v in rng.integers(I32[0], I32[1], 20000)]
    xs += [int(v) for v in rng.integers(-13 * 65536, 11 * 65536, 20000)]  # exp's working range
    for x in xs:
        assert d.rowdev_prim(op, x, 0) == o(op, x, 0), (name, x)


@pytest.mark.parametrize("op,name", [(6, "tanhq"), (7, "sigmoidq")])
def test_tanh_and_sigmoid_exhaustive(lib, op, name):
    """Every input where the result is not yet saturated (|x| <= 12 in Q16),
    against the oracle: pins the f64 quotient that replaces the int64 division."""
    d, o = lib
    xs = np.arange(-12 * 65536 - 2, 12 * 65536 + 3, dtype=np.int64)
    got = np.empty_like(xs)
    d.rowdev_prim_n(op, xs.ctypes.data, got.ctypes.data, xs.size)
    want = np.fromiter((o(op, int(x), 0) for x in xs), np.int64, xs.size)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (name, xs[bad[:5]], got[bad[:5]], want[bad[:5]])


@pytest.mark.parametrize("op,name", [(0, "fmulq"), (1, "fdivq")])
def test_binary_primitives_equal_the_oracle(lib, op, name):
    d, o = lib
    rng = np.random.default_rng(10 + op)
    e = edge_values()
    pairs = [(a, b) for a in e[:40] for b in e[:40]]
    pairs += [tuple(int(v) for v in p) for p in rng.integers(I32[0], I32[1], (20000, 2))]
    pairs += [tuple(int(v) for v in p) for p in rng.integers(-4 * 65536, 4 * 65536, (20000, 2))]
    for a, b in pairs:
        assert d.rowdev_prim(op, a, b) == o(op, a, b), (name, a, b)


def test_isqrt64_and_coefficients(lib):
    d, o = lib
    rng = np.random.default_rng(20)
    for v in [0, 1, 3, 4, (1 << 32) - 1, 1 << 32, (1 << 62), (1 << 63) - 1] + [int(x) for x in rng.integers(0, 1 << 63, 5000)]:
        assert d.rowdev_prim(4, v, 0) == math.isqrt(v), v
    for j in range(9):
        assert d.rowdev_prim(8, j, 0) == o(8, j, 0) == round((1 << 30) / math.factorial(j)), j


def test_constants_are_the_rounded_definitions(lib):
    d, _ = lib
    want = [round(math.log(2) * 65536), round(math.pi * 65536), round(math.pi / 2 * 65536), round(2 * math.pi * 65536),
            round(0.044715 * 65536), round(0.7978845608 * 65536), round(1e-6 * 2 ** 32), round(math.log(32768) * 65536),
            -12 * 65536]
    assert [d.rowdev_const(i) for i in range(9)] == want


def test_softmax_and_rmsnorm_steps(lib):
    """softq and rmsq against exact integer arithmetic in Python: the rounded
    quotient (y * 2^16 + floor(s / 2)) // s for s > 0, and the integer square
    root of ss // cols + round(1e-6 * 2^32), never 0."""
    d, _ = lib
    rng = np.random.default_rng(21)
    for _ in range(5000):
        s = int(rng.integers(65536, 64 * 65536))
        y = int(rng.integers(0, 65537))
        assert d.rowdev_prim(9, y, s) == (y * 65536 + s // 2) // s
        cols = int(rng.integers(1, 4096))
        ss = int(rng.integers(0, 1 << 62))
        assert d.rowdev_prim(11, ss, cols) == max(math.isqrt(ss // cols + 4295), 1)


def test_exp_of_nonpositive_arguments_exhaustive(lib):
    """expq_neg (32-bit arithmetic) equals the oracle's expq on every input
    in [-12 ONE - 2, 0]."""
    d, o = lib
    xs = np.arange(-12 * 65536 - 2, 1, dtype=np.int64)
    got = np.empty_like(xs)
    d.rowdev_prim_n(12, xs.ctypes.data, got.ctypes.data, xs.size)
    want = np.fromiter((o(2, int(x), 0) for x in xs), np.int64, xs.size)
    assert np.array_equal(got, want)


def test_unit_quotient_every_divisor(lib):
    """fdivq_unit(a, b) equals fdivq for every b in [ONE, 2 ONE] at a = 0,
    ONE, and 64 random numerators each."""
    d, o = lib
    rng = np.random.default_rng(22)
    for b in range(65536, 131073):
        for a in [0, 65536, 2 * 65536 - b] + [int(v) for v in rng.integers(0, 65537, 4 if b % 64 else 64)]:
            assert d.rowdev_prim(13, a, b) == o(1, a, b), (a, b)


def test_saturating_add_sub_abs(lib):
    d, _ = lib
    rng = np.random.default_rng(23)
    e = edge_values()
    pairs = [(a, b) for a in e[:30] for b in e[:30]] + [tuple(int(v) for v in p) for p in rng.integers(I32[0], I32[1], (5000, 2))]
    clamp = lambda v: max(I32[0], min(I32[1], v))
    for a, b in pairs:
        assert d.rowdev_prim(14, a, b) == clamp(a + b) and d.rowdev_prim(15, a, b) == clamp(a - b), (a, b)
        assert d.rowdev_prim(16, a, 0) == clamp(abs(a))
