"""`tgc quantize` on the backend's host side: RTN (no calibration rows, no
device) through tg_hip_quantize_model and `tgc-hip quantize`. The goldens are
the reference's own `tgc quantize` outputs (tests/golden/make_golden.py runs
src/quant.c:318-384 on the same f32 models), so every quantized model must
come back byte for byte: the eligible params (src/quant.c:42-89), the
MSE-clipped per-channel scales, the codes, the dequantized data and the
canonical TGIR writer (src/ir.c:150-202, %.9g floats, codes 24 per line)."""
import os
import subprocess

import pytest

from technograd_amd import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
CLI = os.environ.get("TGC_HIP") or os.path.join(ROOT, "technograd_amd", "bin", "tgc-hip")

# golden: (f32 source, bits, min-size); mlp3s is lowered from its .tg model
RTN = {
    "qmlp_q8": ("qmlp_f32.tgir", 8, 256),
    "qmlp_q4": ("qmlp_f32.tgir", 4, 256),
    "mlp3s_q8": ("models/mlp3s.tg", 8, 256),
    "mlp3s_q4": ("models/mlp3s.tg", 4, 256),
    "odd_q4": ("odd_f32.tgir", 4, 1),
    "odd_q8": ("odd_f32.tgir", 8, 1),
    "ssm_small_q8": ("ssm_small_f32.tgir", 8, 1),
}


def source_text(src):
    path = os.path.join(GOLDEN, src)
    return hip.surface_to_tgir(path) if src.endswith(".tg") else open(path).read()


def golden_text(name):
    with open(os.path.join(GOLDEN, name + ".tgir")) as fh:
        return fh.read()


@pytest.mark.parametrize("name", sorted(RTN))
def test_rtn_byte_identical(name):
    src, bits, min_size = RTN[name]
    text, log, (before, after) = hip.quantize_model(source_text(src), bits=bits, min_size=min_size)
    assert text == golden_text(name)
    lines = log.splitlines()
    assert lines[0].startswith("quantize: ") and " param(s) of " in lines[0]
    assert all(", rtn, relative weight error " in ln for ln in lines[1:])
    assert len(lines) - 1 == int(lines[0].split()[1])
    assert after < before


@pytest.mark.parametrize("name", ["qmlp_q4", "mlp3s_q8", "odd_q4"])
def test_cli_rtn(tmp_path, name):
    """the reference's command line: default output name MODEL.qBITS.tgir,
    the report on stderr ending with the size line."""
    src, bits, min_size = RTN[name]
    model = tmp_path / os.path.basename(src)
    model.write_text(open(os.path.join(GOLDEN, src)).read())
    r = subprocess.run([CLI, "quantize", str(model), "--bits", str(bits), "--min-size", str(min_size)],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    out = tmp_path / (model.stem + ".q%d.tgir" % bits)
    assert out.read_text() == golden_text(name)
    last = r.stderr.splitlines()[-1]
    assert last.startswith("quantize: params ") and last.endswith("; wrote " + str(out))


def test_size_report():
    """params 4 bytes per f32 value before; codes (one byte, or a nibble
    each rounded up per param) plus 4 bytes per channel scale after
    (src/quant.c:352-360)."""
    _, _, (before, after) = hip.quantize_model(golden_text("qmlp_f32"), bits=4)
    # W1 48x40 (48 row scales), W2 48x24 (24 column scales), b 24 stays f32
    assert before == 4 * (48 * 40 + 48 * 24 + 24)
    assert after == (48 * 40 + 1) // 2 + 4 * 48 + (48 * 24 + 1) // 2 + 4 * 24 + 4 * 24


def test_quantizing_twice_changes_nothing_more():
    """a quantized param is no longer eligible (src/quant.c:73): quantizing
    the q8 model again leaves no param to quantize"""
    with pytest.raises(RuntimeError, match="no param is eligible"):
        hip.quantize_model(golden_text("qmlp_q8"), bits=8)


@pytest.mark.parametrize("args,msg", [
    (["--bits", "5"], "--bits is 8 or 4"),
    (["--method", "awq"], "--method is rtn or gptq"),
    (["--method", "gptq"], "--method gptq needs --calib DATA"),
    (["--min-size", "100000"], "no param is eligible"),
])
def test_cli_errors(tmp_path, args, msg):
    model = tmp_path / "qmlp.tgir"
    model.write_text(golden_text("qmlp_f32"))
    r = subprocess.run([CLI, "quantize", str(model)] + args, capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and msg in r.stderr
    assert not (tmp_path / "qmlp.q8.tgir").exists()


def test_binding_errors():
    with pytest.raises(ValueError):
        hip.quantize_model(golden_text("qmlp_f32"), method="awq")
    with pytest.raises(RuntimeError, match="bits is 8 or 4"):
        hip.quantize_model(golden_text("qmlp_f32"), bits=2)
    with pytest.raises(RuntimeError, match="GPTQ needs calibration rows"):
        hip.quantize_model(golden_text("qmlp_f32"), method="gptq")
