"""The `tgc batch` driver (technograd_amd/bin/tgc-hip) on the CPU: its
Q16.16 text rule against the reference's tg_fx_parse (runtime/tg_rtq.h:
375-401), pinned by tests/golden/fx_parse.json (written through the
reference's own `tgc c --fixed` unit, tests/golden/make_golden.py)."""
import json
import os
import subprocess
from fractions import Fraction

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.environ.get("TGC_HIP") or os.path.join(ROOT, "technograd_amd", "bin", "tgc-hip")
FX = os.path.join(ROOT, "tests", "golden", "fx_parse.json")

pytestmark = pytest.mark.skipif(not os.path.exists(CLI), reason="bin/tgc-hip is not built")


def fxparse(tokens):
    out = subprocess.run([CLI, "fxparse"] + list(tokens), check=True, capture_output=True, text=True).stdout.split()
    return [None if v == "error" else int(v) for v in out]


def test_fixed_text_rule_matches_reference():
    d = json.load(open(FX))
    assert fxparse(d["tokens"]) == d["q16"]
    assert fxparse(d["refused"]) == [None] * len(d["refused"])


def test_fixture_pins_rounding():
    """The fixture tells the rule from plausible slips: rounding the token's
    exact decimal to 1/65536 half away from zero, without the reference's
    quirks (the 100000 integer cut, 12 fraction digits), or truncating it,
    each disagree with the reference on some tokens."""
    d = json.load(open(FX))

    def exact(t, trunc):
        neg = t.startswith("-")
        body = t.lstrip("+-")
        mant, _, ex = body.partition("e") if "e" in body else body.partition("E")
        v = Fraction(mant if mant not in (".", "") else "0") * Fraction(10) ** int(ex or 0) * 65536
        q = int(v) if trunc else int(v + Fraction(1, 2))
        q = -q if neg else q
        return max(-2 ** 31, min(2 ** 31 - 1, q))

    def plain(t):  # an exponent of a few digits (the wrapped ones have their own rule)
        return not t.endswith(("e", "E")) and len(t.lower().partition("e")[2].lstrip("+-")) <= 3

    toks = [t for t in d["tokens"] if plain(t)]
    want = [q for t, q in zip(d["tokens"], d["q16"]) if plain(t)]
    assert [exact(t, False) for t in toks] != want
    assert [exact(t, True) for t in toks] != want


def test_refuses_bad_usage():
    r = subprocess.run([CLI, "batch"], capture_output=True, text=True)
    assert r.returncode == 1 and "usage" in r.stderr
