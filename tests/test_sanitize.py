"""The host parsers under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU only): tests/cpp/sanitize.mk builds tests/cpp/host_fuzz.c with the
library's host C sources (TGIR reader and writer, quantizers, the .tg front
end) and the driver's row, Q16.16 and HTTP parsers, every report fatal, and
runs a short seeded fuzz of each (mutated TGIR and .tg text, GPTQ with
random and rank-deficient Hessians, row text, HTTP requests over a socket
pair). Longer runs: `make -f tests/cpp/sanitize.mk check ITERS=20000`."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _has_asan():
    cc = shutil.which("gcc") or shutil.which("cc")
    if not cc:
        return False
    lib = subprocess.run([cc, "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    return os.path.isabs(lib) and os.path.exists(lib)


@pytest.mark.skipif(not _has_asan(), reason="no gcc with AddressSanitizer")
def test_host_parsers_fuzz_clean_under_sanitizers():
    r = subprocess.run(["make", "-s", "-f", "tests/cpp/sanitize.mk", "check", "ITERS=400", "SEED=7"], cwd=ROOT,
                       capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-4000:])
    for mode in ("tgir:", "front:", "gptq:", "rows:", "http:"):
        assert mode in r.stdout, r.stdout
    assert "runtime error" not in r.stderr and "ERROR: AddressSanitizer" not in r.stderr, r.stderr[-4000:]
