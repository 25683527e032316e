"""Row programs compiled for the model (hipRTC, tg_rpgen.cpp) against the
row-program interpreter (TG_HIP_INTERP) and the oracle, on the GPU. Both
executors run the same element functions in the same order, so outputs and
steps agree bit for bit, f32 included."""
import glob
import os

import numpy as np
import pytest

from oracle import oracle as O
from technograd_amd import hip, synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "*.npz")))


@pytest.fixture(scope="module", autouse=True)
def device():
    print("gpu rowprog: tg_hip_init(0)", flush=True)
    hip.init(0)


def text_of(name):
    with open(os.path.join(GOLDEN, name + ".tgir")) as f:
        return f.read()


def compiled(text, flags):
    try:
        hip.emit_unit(text, flags)
        return True
    except RuntimeError:
        return False


def run(text, flags, x):
    p = hip.Program(text, flags=flags, max_rows=4096)
    st = p.stats()
    if flags & hip.FIXED:
        y, s = p.batch_fixed(x)
    else:
        y, s = p.batch(x)
    p.close()
    return y, s, st


CASES = [(n, f) for n in NAMES for f in (hip.FIXED, hip.ROWPROG) if compiled(text_of(n), f & hip.FIXED)]


@pytest.mark.parametrize("name,flags", CASES)
def test_compiled_equals_interpreter(name, flags):
    print("case", name, flags, flush=True)
    text = text_of(name)
    d = np.load(os.path.join(GOLDEN, name + ".npz"))
    x = d["xq"] if flags & hip.FIXED and "xq" in d.files else d["x"]
    if flags & hip.FIXED and x.dtype != np.int32:
        x = O.to_fixed_rows(x)
    y1, s1, st1 = run(text, flags, x)
    y0, s0, st0 = run(text, flags | hip.INTERP, x)
    assert st1.rowprog_jit == 1 and st0.rowprog_jit == 0
    assert st1.arena_bytes == 0 < st0.arena_bytes
    assert np.array_equal(np.asarray(y1).view(np.uint32), np.asarray(y0).view(np.uint32))
    assert np.array_equal(s1, s0)


@pytest.mark.parametrize("flags", [hip.FIXED, hip.ROWPROG])
def test_latent_reasoner_compiled_against_oracle(flags):
    """Config 4's model on 65,536 rows (all 256 inputs, shuffled, repeated):
    Q16.16 bit for bit with the oracle; f32 bit for bit with the interpreter
    and steps equal to the oracle's."""
    print("case latent reasoner", flags, flush=True)
    text = synth.latent_reasoner_tgir()
    rng = np.random.default_rng(7)
    x = synth.config4_rows(256)[rng.integers(0, 256, 65536)]
    m = O.Model(text)
    if flags & hip.FIXED:
        xq = O.to_fixed_rows(x)
        want, wsteps = m.batch_fixed(xq)
        got, steps, st = run(text, flags, xq)
        assert np.array_equal(got, want)
    else:
        _, wsteps = m.batch(x)
        got, steps, st = run(text, flags, x)
        y0, _, _ = run(text, flags | hip.INTERP, x)
        assert np.array_equal(got.view(np.uint32), y0.view(np.uint32))
    assert st.rowprog_jit == 1 and st.rowprog_hoisted >= 1
    assert np.array_equal(steps, wsteps)


@pytest.mark.parametrize("name", ["ssm_small_f32", "opsmix_f32"])
def test_interpreter_keeps_what_the_compiler_refuses(name):
    """Scans and gathers stay in the interpreter, and still match the oracle's steps."""
    print("case", name, flush=True)
    text = text_of(name)
    d = np.load(os.path.join(GOLDEN, name + ".npz"))
    y, s, st = run(text, hip.ROWPROG, d["x"])
    assert st.rowprog_jit == 0
    assert np.array_equal(s, d["steps"])
