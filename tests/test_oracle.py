"""The CPU oracle against the reference's golden vectors, known answers and
closed forms (CPU only). The fixtures in tests/golden were written by the
reference's own code (tests/golden/make_golden.py); the oracle must reproduce
them bit for bit before any GPU result is compared with it."""
import ctypes
import glob
import math
import os

import numpy as np
import pytest

from oracle import oracle as O
from technograd_amd import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "*.npz")))


@pytest.fixture(scope="module", autouse=True)
def _built():
    if not os.path.exists(O.LIB_PATH):
        O.build(ref=False)


def load(name):
    with open(os.path.join(GOLDEN, name + ".tgir")) as f:
        text = f.read()
    return text, np.load(os.path.join(GOLDEN, name + ".npz"))


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("name", NAMES)
def test_f32_matches_reference_bit_for_bit(name):
    text, d = load(name)
    m = O.Model(text)
    y, steps = m.batch(d["x"], threads=4)
    assert np.array_equal(bits(y), bits(d["y"])), "f32 outputs differ from the reference VM"
    assert np.array_equal(steps, d["steps"])


@pytest.mark.parametrize("name", [n for n in NAMES if "xq" in np.load(os.path.join(GOLDEN, n + ".npz")).files])
def test_fixed_matches_reference_bit_for_bit(name):
    """xq/yq/stepsq come from the reference's emitted `tgc c --fixed` unit."""
    text, d = load(name)
    m = O.Model(text)
    assert np.array_equal(O.to_fixed_rows(d["x"]), d["xq"])
    yq, sq = m.batch_fixed(d["xq"], threads=4)
    assert np.array_equal(yq, d["yq"]), "Q16.16 outputs differ from the reference kernels"
    assert np.array_equal(sq, d["stepsq"])


@pytest.mark.parametrize("plant", [1, 2])
def test_planted_halting_mistake_is_caught(plant):
    """The Q16.16 goldens (outputs and steps of the reference's emitted
    `tgc c --fixed` unit) catch a slip in the think loop's halting test: `<`
    for `<=` (plant 1) or a threshold one below to_fixed(1e-4, 16) = 7
    (plant 2), each planted in the oracle."""
    text, d = load("latent_f32")
    m = O.Model(text)
    knob = ctypes.c_int.in_dll(O.lib(), "tgo_plant")
    knob.value = plant
    try:
        yq, sq = m.batch_fixed(d["xq"], threads=4)
    finally:
        knob.value = 0
    assert not np.array_equal(sq, d["stepsq"]) and not np.array_equal(yq, d["yq"])
    yq, sq = m.batch_fixed(d["xq"], threads=4)
    assert np.array_equal(sq, d["stepsq"]) and np.array_equal(yq, d["yq"])


@pytest.mark.skipif(not O.have_ref(), reason="needs the reference build (oracle/_ref, made from /root/reference)")
def test_fixed_oracle_matches_emitted_unit_on_fresh_rows(tmp_path):
    """Config 4's model through the reference's own emitted Q16.16 unit
    (src/cgen.c, compiled with cc as tests/run.sh:309 does) on rows that are
    not in the goldens: the whole {0,1}^8 domain again, 4096 N(0,1) rows and
    4096 rows uniform in [-3, 3]. Outputs and steps bit for bit."""
    import itertools
    text, _ = load("latent_f32")
    m = O.Model(text)
    rng = np.random.default_rng(5)
    dom = np.array(list(itertools.product([0, 1], repeat=8)), np.float32)
    x = np.concatenate([dom, rng.normal(size=(4096, 8)).astype(np.float32),
                        rng.uniform(-3, 3, size=(4096, 8)).astype(np.float32)])
    xq = O.to_fixed_rows(x)
    yu, su = O.ref_unit(os.path.join(GOLDEN, "latent_f32.tgir"), xq, m.nout, m.nthink, str(tmp_path))
    yo, so = m.batch_fixed(xq, threads=4)
    assert np.array_equal(so, su) and np.array_equal(yo, yu)
    assert len(np.unique(su)) >= 3  # rows halt at different steps


@pytest.mark.skipif(not O.have_ref(), reason="needs the reference build (oracle/_ref, made from /root/reference)")
@pytest.mark.parametrize("name", [n for n in NAMES if "xq" in np.load(os.path.join(GOLDEN, n + ".npz")).files])
def test_fixed_goldens_are_the_emitted_units(name, tmp_path):
    """Every Q16.16 golden is what the reference's emitted unit computes, and
    the reference's kernels walked over its Module (tgc_ref --fixed) agree."""
    text, d = load(name)
    m = O.Model(text)
    path = os.path.join(GOLDEN, name + ".tgir")
    yu, su = O.ref_unit(path, d["xq"], m.nout, m.nthink, str(tmp_path))
    assert np.array_equal(yu, d["yq"]) and np.array_equal(su, d["stepsq"])
    yw, sw, _ = O.ref_batch(path, d["xq"], m.per, m.nout, m.nthink, str(tmp_path), threads=2, fixed=True)
    assert np.array_equal(yw, yu) and np.array_equal(sw, su)


def test_writer_is_a_fixed_point():
    for name in NAMES:
        text, _ = load(name)
        assert O.Model(text).write() == text, name


def test_latent_reasoner_known_answer():
    """README.md:49-51 of the reference: `tgc run examples/latent_reasoner.tg
    1,0,0,1,0,1,1,0` prints 0.225605994 0.24476327 0.162138939 0.367491812,
    steps 0 9."""
    text, _ = load("latent_f32")
    y, s = O.Model(text).batch(np.array([[1, 0, 0, 1, 0, 1, 1, 0]], np.float32))
    assert ["%.9g" % v for v in y[0]] == ["0.225605994", "0.24476327", "0.162138939", "0.367491812"]
    assert s[0, 0] == 9


def test_rand_initializer_reproduces_lowered_params():
    """rand(seed, scale) (src/lower.c:661-775): the lowered w_emb/w_core/
    w_inj/w_out of the latent model are rand(11, .35), rand(23, .12),
    rand(37, .10), rand(41, .5)."""
    text, _ = load("latent_f32")
    for name, seed, scale, n in [("w_emb", 11, 0.35, 128), ("w_core", 23, 0.12, 256), ("w_inj", 37, 0.10, 256), ("w_out", 41, 0.5, 64)]:
        i = text.index("(param %s " % name)
        body = text[text.index("(data", i) + 5:text.index("))", i)]
        vals = np.array([float(t) for t in body.split()], np.float32)
        assert np.array_equal(bits(vals), bits(O.rand(seed, scale, n))), name


def test_fixed_vs_float_bound():
    """tests/run.sh:306-322: a fixed-point unit stays within 5e-4 of the float VM."""
    for name in ("latent_f32", "latent_q4g", "qmlp_q4g", "qmlp_q8", "ssm_small_q8"):
        text, d = load(name)
        m = O.Model(text)
        x = d["x"][3:64]  # rows 0-2 are the zero / tiny / x50 edge rows
        y, _ = m.batch(x)
        yq, _ = m.batch_fixed(O.to_fixed_rows(x))
        err = np.abs(yq / 65536.0 - y.astype(np.float64))
        assert err.max() < 5e-4, (name, err.max())


def test_thread_invariance():
    """tests/run.sh:114-127: -j 1 and -j N are byte-identical."""
    text, d = load("mlp3s_q8")
    m = O.Model(text)
    y1, _ = m.batch(d["x"], threads=1)
    y8, _ = m.batch(d["x"], threads=8)
    assert np.array_equal(bits(y1), bits(y8))


def test_int4_nibble_rule():
    """tg_qget (runtime/tg_rt.h:124-129): element i in byte i/2, low nibble
    first, sign-extended; checked against the codes the reference wrote."""
    text, _ = load("odd_q4")
    i = text.index("(param W ")
    codes = np.array(text[text.index("(codes", i) + 6:text.index(")", text.index("(codes", i))].split(), int)
    assert codes.size == 33 * 513 and codes.size % 2 == 1
    assert codes.min() >= -7 and codes.max() <= 7


# ---- Q16.16 primitives against their mathematical definitions ----

def prim(op, a, b=0):
    f = O.lib().tgo_fx_prim
    f.restype = ctypes.c_int64
    f.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64]
    return f(op, a, b)


def test_exp_coefficients_are_inverse_factorials():
    for j in range(9):
        assert prim(8, j) == int(round((1 << 30) / math.factorial(j) + 1e-12)), j


def test_isqrt64_is_floor_sqrt():
    rng = np.random.default_rng(3)
    vals = [0, 1, 2, 3, 4, 15, 16, 17, (1 << 32) - 1, 1 << 32, (1 << 62) - 1, (1 << 62), (1 << 63) - 1]
    vals += [int(v) for v in rng.integers(0, 1 << 62, size=2000, dtype=np.int64)]
    for v in vals:
        assert prim(4, v) == math.isqrt(v), v


def test_fdiv_rounding():
    """tg_fdiv (runtime/tg_rtq.h:32-37): with a positive divisor the quotient
    a * 2^16 / b is rounded half away from zero. With a negative divisor the
    reference adds the half-divisor on the wrong side, so the magnitude is
    floor((|n| - h) / |b|), one below the rounded value for most inputs (e.g.
    1 / -2 gives -32767, not -32768). The oracle keeps that behaviour because
    the reference's kernels (golden vectors) do."""
    rng = np.random.default_rng(4)
    for _ in range(5000):
        a, b = (int(v) for v in rng.integers(-(1 << 31), 1 << 31, size=2))
        if b == 0:
            continue
        n, h = a * 65536, abs(b) // 2
        if b > 0:
            mag = (abs(n) * 2 + b) // (2 * b)
        else:
            mag = max(abs(n) - h, 0) // abs(b)
            exact = abs(n) / abs(b)
            assert mag in (round(exact) - 1, round(exact), math.floor(exact)) or abs(mag - exact) <= 1
        q = mag if (n >= 0) == (b > 0) else -mag
        q = max(-(1 << 31), min((1 << 31) - 1, q))
        assert prim(1, a, b) == q, (a, b)
    assert prim(1, 1, -2) == -32767 and prim(1, 1, 2) == 32768
    assert prim(1, 5, 0) == (1 << 31) - 1 and prim(1, -5, 0) == -(1 << 31) and prim(1, 0, 0) == 0


def test_fmul_rounds_half_up():
    rng = np.random.default_rng(5)
    for _ in range(5000):
        a, b = (int(v) for v in rng.integers(-(1 << 31), 1 << 31, size=2))
        q = (a * b + 32768) >> 16
        assert prim(0, a, b) == max(-(1 << 31), min((1 << 31) - 1, q))


def test_expq_tracks_exp():
    for x in np.linspace(-12, 10.39, 4001):
        q = int(round(x * 65536))
        got = prim(2, q) / 65536.0
        want = math.exp(q / 65536.0)
        assert abs(got - want) <= 3e-5 * max(1.0, want), x  # degree-8 polynomial in Q30
    assert prim(2, 11 * 65536) == (1 << 31) - 1 and prim(2, -13 * 65536) == 0


def test_tanhq_and_sigmoidq_track_float():
    for x in np.linspace(-10, 10, 2001):
        q = int(round(x * 65536))
        assert abs(prim(6, q) / 65536.0 - math.tanh(q / 65536.0)) < 4e-5
        assert abs(prim(7, q) / 65536.0 - 1 / (1 + math.exp(-q / 65536.0))) < 4e-5


def test_planted_mistake_is_caught():
    """A plausible oracle mistake (a transposed quantized operand) must fail the
    golden comparison: swap W's axis on a copy of the model and re-run."""
    text, d = load("qmlp_q8")
    broken = text.replace("(quant 8 0", "(quant 8 1", 1)
    with pytest.raises(ValueError):
        O.Model(broken)  # the channel count no longer matches: the reader refuses it
    text4, d4 = load("odd_q4")
    m = O.Model(text4)
    y, _ = m.batch(d4["x"])
    assert np.array_equal(bits(y), bits(d4["y"]))
    y_bad, _ = m.batch(d4["x"][:, ::-1].copy())  # a reversed input order changes the sums
    assert not np.array_equal(bits(y_bad), bits(d4["y"]))


# ---- the f64 interpreter (oracle/vm64.c), the truth of the whole-model
# predicate (tests/parity.py: check_model): pinned by closed forms ----

def _exact_qproduct(codes_kc, scales, x):
    """o[m, c] = s[c] * sum_k code[k, c] x[m, k], each sum exactly rounded
    (math.fsum over exact f64 products), then the scale in f64; and
    sum_k |s code x| (the scale of the rounding bound)."""
    t = np.empty((x.shape[0], codes_kc.shape[1]))
    mag = np.empty_like(t)
    cf, xf = codes_kc.astype(np.float64), x.astype(np.float64)
    for m in range(x.shape[0]):
        prods = xf[m][:, None] * cf  # exact: an int8 times an f32
        for c in range(cf.shape[1]):
            t[m, c] = math.fsum(prods[:, c])
        mag[m] = np.abs(prods).sum(axis=0)
    return t * scales.astype(np.float64)[None, :], mag * np.abs(scales.astype(np.float64))[None, :]


def _qlinear_case(bits, axis, K, C, seed):
    rng = np.random.default_rng(seed)
    lim = 7 if bits == 4 else 127
    codes = rng.integers(-lim, lim + 1, size=(K, C)).astype(np.int8)  # as x @ W
    scales = rng.uniform(0.001, 0.1, size=C).astype(np.float32)
    x = rng.normal(size=(6, K)).astype(np.float32)
    x[1] *= 1e4
    x[2, K // 2] = 3e3  # an outlier
    stored = codes if axis == 1 else np.ascontiguousarray(codes.T)
    return O.Model(synth.linear_tgir_codes("q", stored, scales, bits, axis)), codes, scales, x


@pytest.mark.parametrize("bits,axis,K", [(4, 1, 7), (8, 1, 513), (4, 0, 513), (8, 0, 4096)])
def test_f64_quantized_product_is_the_exact_product(bits, axis, K):
    """A one-matmul quantized model through batch64 equals the exact product
    (exactly rounded sums, tests/parity.py's truth) to f64 rounding: within
    (K + 2) 2^-53 sum |s w x|. A dropped term, a wrong sign, index or
    operand order, or a sum left in f32 is orders of magnitude outside."""
    m, codes, scales, x = _qlinear_case(bits, axis, K, 40, K + bits + axis)
    got, _ = m.batch64(x)
    want, mag = _exact_qproduct(codes, scales, x)
    assert (np.abs(got - want) <= (K + 2) * 2.0 ** -53 * mag + 1e-300).all()
    y32, _ = m.batch(x)
    assert (y32.astype(np.float64) != got).any()  # an f64 result, not the f32 one widened


def test_f64_planted_f32_sums_are_caught():
    """tgo_plant64 = 1 leaves the quantized products' running sums in f32
    inside the f64 interpreter; the closed form above rejects it."""
    m, codes, scales, x = _qlinear_case(8, 1, 513, 40, 7)
    want, mag = _exact_qproduct(codes, scales, x)
    knob = ctypes.c_int.in_dll(O.lib(), "tgo_plant64")
    knob.value = 1
    try:
        bad, _ = m.batch64(x)
    finally:
        knob.value = 0
    assert not (np.abs(bad - want) <= 515 * 2.0 ** -53 * mag).all()
    good, _ = m.batch64(x)
    assert (np.abs(good - want) <= 515 * 2.0 ** -53 * mag).all()


def _row_model(op, n):
    return "(tgir 1\n  (model r)\n  (input x (f32 %d))\n  (block\n    (%%0 (f32 %d) (%s x))\n  )\n  (output %%0))\n" % (n, n, op)


@pytest.mark.parametrize("op", ["rmsnorm", "softmax", "tanh", "exp", "sigmoid"])
def test_f64_row_ops_are_numpy_f64(op):
    """rmsnorm (sum of squares, 1 / sqrt(s / n + 1e-6), no gain:
    runtime/tg_rt.h:165-175), softmax (max, exp(x - max), sum, divide:
    :154-164) and the elementwise functions through batch64 equal numpy's
    double-precision evaluation of the same formulas within a few f64 ulps."""
    rng = np.random.default_rng(len(op))
    n = 257
    x = (rng.normal(size=(16, n)) * np.array([1, 10, 0.01, 30] * 4)[:, None]).astype(np.float32)
    got, _ = O.Model(_row_model(op, n)).batch64(x)
    xd = x.astype(np.float64)
    if op == "rmsnorm":
        want = xd / np.sqrt((xd * xd).sum(axis=1, keepdims=True) / n + float(np.float32(1e-6)))
    elif op == "softmax":
        e = np.exp(xd - xd.max(axis=1, keepdims=True))
        want = e / e.sum(axis=1, keepdims=True)
    elif op == "tanh":
        want = np.tanh(xd)
    elif op == "exp":
        want = np.exp(xd)
    else:
        want = 1.0 / (1.0 + np.exp(-xd))
    assert np.allclose(got, want, rtol=64 * 2.0 ** -53, atol=1e-300), np.abs(got / want - 1).max()


@pytest.mark.parametrize("name", NAMES)
def test_goldens_within_reach_of_the_f64_truth(name):
    """Every golden's f32 output (the reference's own) lies within 1e-4 of
    its row's largest magnitude from the f64 interpreter, on rows whose think
    loops halt at the same step in both (the largest such distance over the
    goldens is 6.5e-6). A truth missing a term, with a wrong sign or operand,
    or a wrong op order on whole-model scale would be outside."""
    text, d = load(name)
    t, st = O.Model(text).batch64(d["x"])
    y = d["y"].astype(np.float64).reshape(t.shape)
    same = (st == d["steps"]).all(axis=1)
    assert same.mean() > 0.9
    scale = np.abs(t[same]).max(axis=1, keepdims=True)
    assert (np.abs(y[same] - t[same]) <= 1e-4 * scale).all()


def test_file_backed_params_equal_the_text_forms(tmp_path):
    """The oracle's test-only file forms (data-file, scale-file, codes-file,
    used for models too large to write as text) give the values of the text
    forms: a small Qwen3-shaped model written both ways computes the same
    bits, and a second length T written through the weight cache reuses the
    first one's weight files."""
    dims = dict(L=1, D=32, NQ=2, NKV=1, HD=16, FF=48, V=64)
    ids = np.random.default_rng(1).integers(0, 64, size=(3, 6)).astype(np.float32)
    want, _ = O.Model(synth.qwen3_tgir("q", T=6, **dims)).batch(ids)
    cache = {}
    got, _ = O.Model(synth.qwen3_tgir("q", T=6, files=str(tmp_path), cache=cache, **dims)).batch(ids)
    assert np.array_equal(bits(got), bits(want))
    stamp = os.path.getmtime(tmp_path / "LM.codes")
    text4 = synth.qwen3_tgir("q", T=4, files=str(tmp_path), cache=cache, **dims)
    assert os.path.getmtime(tmp_path / "LM.codes") == stamp and "mask.T4.f32" in text4
    want4, _ = O.Model(synth.qwen3_tgir("q", T=4, **dims)).batch(ids[:, :4])
    got4, _ = O.Model(text4).batch(ids[:, :4])
    assert np.array_equal(bits(got4), bits(want4))
    with pytest.raises(ValueError):
        synth.qwen3_tgir("q", T=4, files=str(tmp_path), cache=cache, **dict(dims, FF=64))
    short = tmp_path / "short.f32"
    np.zeros(3, np.float32).tofile(short)
    for path in (short, tmp_path / "absent.f32"):  # a file of the wrong size, and none
        with pytest.raises(ValueError, match="short.f32|absent.f32"):
            O.Model("(tgir 1 (model m) (param w (f32 4) (data-file %s)) (input x (f32 4)) (block) (output x))" % path)
