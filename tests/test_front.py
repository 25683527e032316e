"""The surface-language front end (technograd_amd/csrc/tg_front.c) on the CPU:
.tg models lowered through the C ABI (tg_hip_surface_to_tgir) must give the
reference's `tgc ir` bytes, and rejected sources the reference's diagnostic.

Fixtures: tests/golden/*_f32.tgir are `tgc ir` of tests/golden/models/*.tg;
tests/golden/front/NAME.tgir are `tgc ir` of this repository's front-end
models front/NAME.tg (imports, every initializer, states and updates, rope,
attention, take_along, the losses, nested loops, scans, syntax forms), and
front/errors.json holds the reference's message for each rejected source,
all written by the reference built from its sources
(tests/golden/make_golden.py)."""
import glob
import json
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O
from technograd_amd import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
FRONT = os.path.join(GOLDEN, "front")
FRONT_ENV = {"TGF_FRONT_VALUES": "1.5, -2 3e-1,4"}  # as make_golden.py sets it for the reference
CLI = os.environ.get("TGC_HIP") or os.path.join(ROOT, "technograd_amd", "bin", "tgc-hip")

MODELS = sorted(os.path.basename(p)[:-3] for p in glob.glob(os.path.join(GOLDEN, "models", "*.tg"))
                if os.path.exists(os.path.join(GOLDEN, os.path.basename(p)[:-3] + "_f32.tgir")))
FRONT_MODELS = sorted(os.path.basename(p)[:-3] for p in glob.glob(os.path.join(FRONT, "*.tg")))
with open(os.path.join(FRONT, "errors.json")) as fh:
    ERRORS = json.load(fh)


def lower_in(directory, name, monkeypatch):
    """Lower NAME.tg from its own directory, as the reference was run."""
    monkeypatch.chdir(directory)
    for k, v in FRONT_ENV.items():
        monkeypatch.setenv(k, v)
    monkeypatch.delenv("TGF_FRONT_UNSET", raising=False)
    return hip.surface_to_tgir(name + ".tg")


@pytest.mark.parametrize("name", MODELS)
def test_golden_models_lower_to_the_reference_bytes(name, monkeypatch):
    got = lower_in(os.path.join(GOLDEN, "models"), name, monkeypatch)
    with open(os.path.join(GOLDEN, name + "_f32.tgir")) as fh:
        assert got == fh.read()


@pytest.mark.parametrize("name", FRONT_MODELS)
def test_front_models_lower_to_the_reference_bytes(name, monkeypatch):
    got = lower_in(FRONT, name, monkeypatch)
    with open(os.path.join(FRONT, name + ".tgir")) as fh:
        want = fh.read()
    if got != want:  # name the first differing line
        g, w = got.splitlines(), want.splitlines()
        i = next((k for k in range(min(len(g), len(w))) if g[k] != w[k]), min(len(g), len(w)))
        raise AssertionError("line %d: %r != %r" % (i + 1, g[i] if i < len(g) else None, w[i] if i < len(w) else None))


def test_quantized_golden_from_the_surface(monkeypatch):
    """mlp3s.tg lowered here, then quantized by the backend's host quantizer
    (`tgc quantize --bits 8`, no device): the reference's mlp3s_q8.tgir byte
    for byte."""
    text = lower_in(os.path.join(GOLDEN, "models"), "mlp3s", monkeypatch)
    q, _, _ = hip.quantize_model(text, bits=8)
    with open(os.path.join(GOLDEN, "mlp3s_q8.tgir")) as fh:
        assert q == fh.read()


@pytest.mark.parametrize("case", sorted(ERRORS))
def test_rejected_sources_give_the_reference_diagnostic(case, tmp_path, monkeypatch):
    for fn, body in ERRORS[case]["files"].items():
        p = tmp_path / fn
        p.parent.mkdir(parents=True, exist_ok=True)
        if isinstance(body, list):
            p.write_bytes(bytes(body))
        else:
            p.write_text(body)
    monkeypatch.chdir(tmp_path)
    monkeypatch.delenv("TGF_FRONT_NEVER_SET", raising=False)
    with pytest.raises(RuntimeError) as e:
        hip.surface_to_tgir("err.tg")
    assert str(e.value) == ERRORS[case]["message"]


def test_operations_outside_the_batch_path_are_refused(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    cases = {"grad(sum(x), x)": "grad", "topk(x, 1)": "topk", "spmm(s, w)": "spmm"}
    for expr, word in cases.items():
        (tmp_path / "m.tg").write_text("model m\nparam w : f32[4, 2] = zeros\nparam s : f32[3, 2] = zeros\n"
                                       "def forward(x: f32[2]) -> f32[2]:\n    y = %s\n    return x\n" % expr)
        with pytest.raises(RuntimeError, match=word):
            hip.surface_to_tgir("m.tg")


def test_lowered_model_runs_like_its_golden(monkeypatch):
    """The lowered text is the golden's, so the oracle's run of it is the
    reference's: a check that nothing but bytes is compared above."""
    if not os.path.exists(O.LIB_PATH):
        O.build(ref=False)
    text = lower_in(os.path.join(GOLDEN, "models"), "latent", monkeypatch)
    d = np.load(os.path.join(GOLDEN, "latent_f32.npz"))
    y, steps = O.Model(text).batch(d["x"])
    assert np.array_equal(y.view(np.uint32), d["y"].view(np.uint32)) and np.array_equal(steps, d["steps"])


def test_cli_ir(tmp_path):
    r = subprocess.run([CLI, "ir", os.path.join(GOLDEN, "models", "haltm.tg")], capture_output=True, text=True)
    assert r.returncode == 0
    with open(os.path.join(GOLDEN, "haltm_f32.tgir")) as fh:
        assert r.stdout == fh.read()
    (tmp_path / "err.tg").write_text(ERRORS["undefined_name"]["files"]["err.tg"])
    r = subprocess.run([CLI, "ir", "err.tg"], capture_output=True, text=True, cwd=tmp_path)
    assert r.returncode == 1 and r.stderr.strip() == "tgc-hip: error: " + ERRORS["undefined_name"]["message"]
