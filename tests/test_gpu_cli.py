"""`tgc batch` end to end on the GPU: technograd_amd/bin/tgc-hip over the
golden models (written by the reference's own code), with the reference's
I/O contract (src/main.c:400-444, src/io.c:43-93): binary rows in and out,
text rows in and out with the steps of every think loop appended, Q16.16
text and binary rows, the stop after the current block on SIGTERM (exit
128 + 15), the `batch` trace event (--log), and validation before output."""
import json
import os
import subprocess
import sys
from decimal import Decimal, getcontext

import numpy as np
import pytest

from oracle import oracle as O

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import parity  # noqa: E402

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.environ.get("TGC_HIP") or os.path.join(ROOT, "technograd_amd", "bin", "tgc-hip")
GOLDEN = os.path.join(ROOT, "tests", "golden")


def golden(name):
    return os.path.join(GOLDEN, name + ".tgir"), np.load(os.path.join(GOLDEN, name + ".npz"))


def cli(args, env=None):
    print("case cli", " ".join(os.path.basename(str(a)) for a in args), flush=True)
    return subprocess.run([CLI, "batch"] + [str(a) for a in args], capture_output=True, text=True, timeout=120,
                          env=dict(os.environ, **(env or {})))


def text_rows(path):
    return [line.split(",") for line in open(path).read().splitlines() if line]


def test_binary_rows_exact_path_byte_identical(tmp_path):
    """odd_q4 (int4 weights, no transcendental) on the exact path: the output
    file is the reference's output, byte for byte."""
    model, d = golden("odd_q4")
    inp, out = tmp_path / "x.bin", tmp_path / "y.bin"
    d["x"].astype("<f4").tofile(inp)
    r = cli([model, inp, "-o", out, "--exact"])
    assert r.returncode == 0, r.stderr
    assert out.read_bytes() == d["y"].astype("<f4").tobytes()


def test_text_rows_with_steps(tmp_path):
    """latent_f32 (a think loop): text rows in, %.9g values and the steps
    column out; values under the parity predicate, steps exact."""
    model, d = golden("latent_f32")
    inp, out = tmp_path / "x.txt", tmp_path / "y.txt"
    with open(inp, "w") as fh:
        fh.write("# rows of the golden fixture\n")
        for row in d["x"]:
            fh.write(", ".join("%.9g" % v for v in row) + "\n")
    r = cli([model, inp, "-o", out])
    assert r.returncode == 0, r.stderr
    rows = text_rows(out)
    assert len(rows) == len(d["x"]) and all(len(t) == d["y"].shape[1] + 1 for t in rows)
    y = np.array([[np.float32(v) for v in t[:-1]] for t in rows], np.float32)
    steps = np.array([[int(t[-1])] for t in rows], np.int32)
    assert np.array_equal(steps, d["steps"])
    t64, st64 = O.Model(open(model).read()).batch64(d["x"])
    parity.check_model(y, d["y"], t64, (st64 == d["steps"]).all(axis=1))


def _exact_decimal(q):
    getcontext().prec = 40
    return str(Decimal(int(q)) / Decimal(65536))


def test_fixed_text_and_binary(tmp_path):
    """latent_f32 in Q16.16 (--fixed): text rows of exact decimals in, the
    6-decimal text of the reference unit's outputs and its steps out; binary
    f32 rows in, q / 65536 out. Both equal the reference's bit for bit."""
    model, d = golden("latent_f32")
    inp, out = tmp_path / "xq.txt", tmp_path / "yq.txt"
    with open(inp, "w") as fh:
        for row in d["xq"]:
            fh.write(",".join(_exact_decimal(q) for q in row) + "\n")
    r = cli([model, inp, "-o", out, "--fixed"])
    assert r.returncode == 0, r.stderr
    rows = text_rows(out)
    assert [t[:-1] for t in rows] == [[O.fx_format(v) for v in row] for row in d["yq"]]
    assert [int(t[-1]) for t in rows] == d["stepsq"][:, 0].tolist()
    binp, bout = tmp_path / "x.bin", tmp_path / "y.bin"
    d["x"].astype("<f4").tofile(binp)  # f32 rows: x * 2^16 rounded half away from zero, as the goldens' xq
    r = cli([model, binp, "-o", bout, "--fixed"])
    assert r.returncode == 0, r.stderr
    got = np.fromfile(bout, "<f4").reshape(d["yq"].shape)
    assert np.array_equal(got, (d["yq"].astype(np.float64) / 65536.0).astype(np.float32))


def test_stop_after_current_block(tmp_path):
    """SIGTERM after the second block of 16 rows: the batch stops there, the
    output holds exactly the first 32 rows (as a full run writes them), and
    the exit status is 128 + 15."""
    model, d = golden("qmlp_q8")
    inp, full, part = tmp_path / "x.bin", tmp_path / "full.bin", tmp_path / "part.bin"
    d["x"].astype("<f4").tofile(inp)
    assert cli([model, inp, "-o", full, "--rows", 16]).returncode == 0
    r = cli([model, inp, "-o", part, "--rows", 16], env={"TGC_HIP_TEST_SIGTERM_AFTER_BLOCKS": "2"})
    assert r.returncode == 128 + 15, (r.returncode, r.stderr)
    nout = d["y"].shape[1]
    assert part.read_bytes() == full.read_bytes()[:32 * nout * 4]


def test_log_events(tmp_path):
    """--log appends the reference's `batch` and `think` events as JSON Lines."""
    model, d = golden("latent_f32")
    inp, out, log = tmp_path / "x.bin", tmp_path / "y.bin", tmp_path / "log.jsonl"
    d["x"].astype("<f4").tofile(inp)
    r = cli([model, inp, "-o", out, "--log", log])
    assert r.returncode == 0, r.stderr
    ev = [json.loads(line) for line in open(log)]
    assert [e["stage"] for e in ev] == ["batch", "think"]
    assert ev[0]["rows"] == len(d["x"]) and ev[0]["level"] == "info" and ev[0]["ms"] > 0
    st = d["steps"][:, 0]
    assert (ev[1]["steps_min"], ev[1]["steps_max"]) == (int(st.min()), int(st.max()))
    assert abs(ev[1]["steps_mean"] - st.mean()) < 1e-6


def test_rows_are_validated_before_output(tmp_path):
    """A bad number on line 3: an error naming the line, no output file."""
    model, d = golden("qmlp_q8")
    inp, out = tmp_path / "x.txt", tmp_path / "y.txt"
    per = d["x"].shape[1]
    with open(inp, "w") as fh:
        fh.write(",".join(["1"] * per) + "\n" + ",".join(["2"] * per) + "\n" + ",".join(["3x"] * per) + "\n")
    r = cli([model, inp, "-o", out])
    assert r.returncode == 1 and ":3: bad number" in r.stderr and not out.exists()


def test_surface_model_runs_like_its_tgir(tmp_path):
    """A .tg model given to `batch` is lowered first (the reference's
    load_module rule): the output file equals the one for its TGIR golden,
    byte for byte, in f32 and in Q16.16."""
    model, d = golden("latent_f32")
    surface = os.path.join(GOLDEN, "models", "latent.tg")
    inp = tmp_path / "x.bin"
    d["x"].astype("<f4").tofile(inp)
    for flags in ([], ["--fixed"]):
        a, b = tmp_path / "a.bin", tmp_path / "b.bin"
        ra = cli([model, inp, "-o", a] + flags)
        rb = cli([surface, inp, "-o", b] + flags)
        assert ra.returncode == 0 and rb.returncode == 0, ra.stderr + rb.stderr
        assert a.read_bytes() == b.read_bytes()
