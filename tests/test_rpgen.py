"""The row-program compiler (technograd_amd/csrc/tg_rpgen.cpp) on the CPU:
emitted units compile for gfx950, and the same units built as host code
(tests/cpp/unit_host.cpp) reproduce the reference's golden vectors and the
oracle bit for bit. The GPU runs of the compiled programs are in
test_gpu_rowprog.py."""
import glob
import os
import re
import subprocess

import numpy as np
import pytest

from oracle import oracle as O
from technograd_amd import hip, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
CSRC = os.path.join(ROOT, "technograd_amd", "csrc")
HIPFLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def golden(name):
    with open(os.path.join(GOLDEN, name + ".tgir")) as f:
        return f.read(), np.load(os.path.join(GOLDEN, name + ".npz"))


def host_unit(tmp, text, fixed):
    """Emit the unit, build it as host code (clang++: the element functions use
    its saturating builtins); returns a runner rows -> (out, steps)."""
    src = hip.emit_unit(text, hip.FIXED if fixed else 0, kernel="tgu")
    unit = tmp / ("u%d.hip" % fixed)
    unit.write_text(src)
    exe = tmp / ("u%d" % fixed)
    subprocess.run(["/opt/rocm/llvm/bin/clang++", "-O1", "-std=c++17", "-ffp-contract=off", "-I", CSRC, "-DTG_UNIT_FILE=\"%s\"" % unit,
                    "-DTG_KERNEL=tgu", "-DTG_T=%s" % ("int" if fixed else "float"), "-o", str(exe),
                    os.path.join(ROOT, "tests", "cpp", "unit_host.cpp"), "-lm"], check=True)
    m = O.Model(text)

    def run(rows):
        rows = np.ascontiguousarray(rows, np.int32 if fixed else np.float32)
        n = rows.shape[0]
        rows.tofile(tmp / "in.bin")
        nt = max(m.nthink, 1)
        subprocess.run([str(exe), str(tmp / "in.bin"), str(tmp / "out.bin"), str(tmp / "st.bin"), str(n), str(m.per),
                        str(m.nout), str(nt)], check=True)
        out = np.fromfile(tmp / "out.bin", np.int32 if fixed else np.float32).reshape(n, m.nout)
        return out, np.fromfile(tmp / "st.bin", np.int32).reshape(n, nt)
    return run


@pytest.fixture(scope="module", autouse=True)
def _built():
    if not os.path.exists(O.LIB_PATH):
        O.build(ref=False)


FIXED_GOLDENS = [n for n in sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "*.npz")))
                 if "xq" in np.load(os.path.join(GOLDEN, n + ".npz")).files]


def compiled(name):
    try:
        hip.emit_unit(golden(name)[0], hip.FIXED)
        return True
    except RuntimeError:
        return False


@pytest.mark.parametrize("name", [n for n in FIXED_GOLDENS if compiled(n)])
def test_fixed_unit_reproduces_reference_goldens(tmp_path, name):
    """Q16.16 units run on the host: outputs and steps equal the reference's
    emitted `tgc c --fixed` units bit for bit."""
    text, d = golden(name)
    run = host_unit(tmp_path, text, True)
    yq, sq = run(d["xq"])
    assert np.array_equal(yq, d["yq"]) and np.array_equal(sq, d["stepsq"])


def test_latent_reasoner_unit_over_all_inputs(tmp_path):
    """Config 4's model over its whole {0,1}^8 input domain, against the oracle."""
    text = synth.latent_reasoner_tgir()
    xq = O.to_fixed_rows(synth.config4_rows(256))
    want, wsteps = O.Model(text).batch_fixed(xq)
    got, steps = host_unit(tmp_path, text, True)(xq)
    assert np.array_equal(got, want) and np.array_equal(steps, wsteps)
    assert len(set(steps[:, 0].tolist())) >= 3  # divergent halting (8, 9 and 10 steps)


@pytest.mark.parametrize("name", ["latent_f32", "haltm_f32", "qmlp_q8", "qmlp_q4", "qmlp_f32"])
def test_f32_unit_reproduces_reference_goldens(tmp_path, name):
    """f32 units run on the host with the reference's libm (glibc): the VM's
    operation order, so outputs and steps equal the reference's bit for bit."""
    text, d = golden(name)
    y, st = host_unit(tmp_path, text, False)(d["x"])
    assert np.array_equal(y.view(np.uint32), d["y"].view(np.uint32)) and np.array_equal(st, d["steps"])


def test_think_body_hoists_the_injection_product():
    """The latent reasoner's think body keeps w_core @ h (16 sums) and loses
    w_inj @ e (16 sums): the loop holds 16 multiply-add blocks; the embedding,
    injection and readout products (16 + 16 + 4) run outside it."""
    src = hip.emit_unit(synth.latent_reasoner_tgir(), hip.FIXED)
    i = src.index("for (;;) {")
    depth, j = 0, i
    while True:
        c = src[j]
        depth += c == "{"
        depth -= c == "}"
        j += 1
        if depth == 0 and c == "}":
            break
    loop = src[i:j]
    inside = loop.count("{ long s = 0;")
    assert inside == 16, inside
    assert src.count("{ long s = 0;") - inside == 16 + 16 + 4


@pytest.mark.parametrize("name,why", [("ssm_small_f32", "scan"), ("opsmix_f32", "take"), ("qwen3_tiny", "arena")])
def test_units_refuse_what_the_interpreter_keeps(name, why):
    text, _ = golden(name)
    with pytest.raises(RuntimeError, match=why):
        hip.emit_unit(text)


@pytest.mark.parametrize("fixed", [1, 0])
def test_unit_compiles_for_gfx950(tmp_path, fixed):
    """The latent reasoner's unit, launcher included, builds with hipcc as a
    standalone translation unit."""
    src = hip.emit_unit(synth.latent_reasoner_tgir(), hip.FIXED if fixed else 0)
    assert re.search(r'extern "C" __global__ __launch_bounds__\(256\) void tg_\w+_rows\(const %s ' % ("int" if fixed else "float"), src)
    unit = tmp_path / "u.hip"
    unit.write_text(src)
    subprocess.run(["/opt/rocm/bin/hipcc"] + HIPFLAGS + ["-fPIC", "-c", "-o", str(tmp_path / "u.o"), str(unit)], check=True,
                   capture_output=True)


def test_cli_writes_the_unit(tmp_path):
    out = tmp_path / "unit.hip"
    subprocess.run([os.path.join(ROOT, "technograd_amd", "bin", "tgc-hip"), "c", os.path.join(GOLDEN, "latent_f32.tgir"),
                    "--fixed", "-o", str(out), "--kernel", "lat"], check=True)
    assert 'void lat(const int *__restrict__ in' in out.read_text()
    r = subprocess.run([os.path.join(ROOT, "technograd_amd", "bin", "tgc-hip"), "c", os.path.join(GOLDEN, "ssm_small_f32.tgir")],
                       capture_output=True, text=True)
    assert r.returncode == 1 and "scan" in r.stderr
