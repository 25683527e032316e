"""`tgc-hip stream` and `tgc-hip serve` on the GPU against the reference's
own `tgc serve` (src/serve.c), whose conversations over the row protocol and
HTTP were recorded byte for byte (tests/golden/front/serve.json, written by
tests/golden/make_golden.py from the reference built from its sources):
health, signature, POST /run, 404, a malformed request line, and rows with
blank, comment, malformed and short lines. odd_q4 (no transcendental) on the
exact path must answer with the reference's bytes; latent_f32 (a think loop,
device libm) with its bytes except the output values, which are held to the
parity predicate. Many concurrent clients must get their own rows' outputs,
gathered into fewer device batches than rows."""
import json
import os
import re
import signal
import socket
import subprocess
import sys
import threading
from contextlib import contextmanager

import numpy as np
import pytest

from oracle import oracle as O

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import parity  # noqa: E402

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.environ.get("TGC_HIP") or os.path.join(ROOT, "technograd_amd", "bin", "tgc-hip")
GOLDEN = os.path.join(ROOT, "tests", "golden")
with open(os.path.join(GOLDEN, "front", "serve.json")) as fh:
    SERVE = json.load(fh)


@contextmanager
def server(name, *flags):
    print("case serve", name, *flags, flush=True)
    p = subprocess.Popen([CLI, "serve", os.path.join(GOLDEN, name + ".tgir"), "--listen", "127.0.0.1:0"] + list(flags),
                         stderr=subprocess.PIPE, text=True)
    line = p.stderr.readline()
    m = re.search(r" on [^ ]*:(\d+) ", line)
    if not m:
        p.kill()
        raise AssertionError("server did not start: %r %s" % (line, p.stderr.read()))
    try:
        yield p, int(m.group(1))
    finally:
        if p.poll() is None:
            p.send_signal(signal.SIGTERM)
            p.wait(timeout=60)


# lines to wait for on conversations that stay open (the row protocol; a
# request line without a method and path is taken as a row)
OPEN_LINES = {"rows": 5, "bad": 1}


def converse(port, data, expect_lines=None, timeout=60):
    s = socket.create_connection(("127.0.0.1", port), timeout=timeout)
    s.sendall(data.encode())
    got = b""
    while expect_lines is None or got.count(b"\n") < expect_lines:
        k = s.recv(1 << 16)
        if not k:
            break
        got += k
    s.close()
    return got.decode()


def test_exact_path_answers_with_the_reference_bytes():
    with server("odd_q4", "--exact") as (_, port):
        for tag, c in sorted(SERVE["odd_q4"].items()):
            got = converse(port, c["send"], OPEN_LINES.get(tag))
            assert got == c["recv"], tag


def values(text):
    rows = [l for l in text.splitlines() if l and not l.startswith("error:")]
    return np.array([[float(v) for v in r.split(",")] for r in rows])


def split_http(s):
    """(header lines without Content-Length, body) of a response; ([], s) for the row protocol."""
    if not s.startswith("HTTP/"):
        return [], s
    h, b = s.split("\r\n\r\n", 1)
    return [l for l in h.split("\r\n") if not l.startswith("Content-Length")], b


def test_think_model_answers_like_the_reference():
    """Protocol bytes equal (headers, error lines and their places, steps);
    output values under the parity predicate against the reference's, with
    the f64 interpreter as truth."""
    conv = SERVE["latent_f32"]
    x = np.load(os.path.join(GOLDEN, "latent_f32.npz"))["x"][:3]
    text = open(os.path.join(GOLDEN, "latent_f32.tgir")).read()
    t, st = O.Model(text).batch64(x)
    with server("latent_f32") as (_, port):
        for tag, c in sorted(conv.items()):
            got = converse(port, c["send"], OPEN_LINES.get(tag))
            if tag not in ("rows", "run"):
                assert got == c["recv"], tag
                continue
            (gh, gb), (rh, rb) = split_http(got), split_http(c["recv"])
            assert gh == rh, tag
            gl, rl = gb.splitlines(), rb.splitlines()
            assert [l for l in gl if l.startswith("error:")] == [l for l in rl if l.startswith("error:")], tag
            assert [l.startswith("error:") for l in gl] == [l.startswith("error:") for l in rl], tag
            g, r = values(gb), values(rb)
            assert np.array_equal(g[:, -1], r[:, -1]), tag  # steps
            parity.check_model(g[:, :-1], r[:, :-1], t, (st == g[:, -1:].astype(int)).all(axis=1))


def batch_text(name, rows, tmp_path, *flags):
    inp, out = tmp_path / "in.txt", tmp_path / "out.txt"
    inp.write_text("".join(",".join("%.9g" % v for v in r) + "\n" for r in rows))
    r = subprocess.run([CLI, "batch", os.path.join(GOLDEN, name + ".tgir"), str(inp), "-o", str(out)] + list(flags),
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return out.read_text()


def test_concurrent_clients_get_their_own_rows_in_shared_batches(tmp_path):
    """16 clients, 64 rows each, sent at once over the row protocol: every
    client's outputs equal `tgc-hip batch` on its rows (the same compiled
    kernel per row), and the server ran them in fewer device batches than
    clients."""
    from technograd_amd import synth
    rng = np.random.default_rng(11)
    text = open(os.path.join(GOLDEN, "latent_f32.tgir")).read()
    per = O.Model(text).per
    xs = [rng.uniform(-1, 1, size=(64, per)).astype(np.float32) for _ in range(16)]
    want = [batch_text("latent_f32", x, tmp_path) for x in xs]
    got = [None] * len(xs)
    with server("latent_f32", "--window-us", "2000") as (p, port):
        def client(i):
            body = "".join(",".join("%.9g" % v for v in r) + "\n" for r in xs[i])
            got[i] = converse(port, body, expect_lines=len(xs[i]))
        th = [threading.Thread(target=client, args=(i,)) for i in range(len(xs))]
        for t in th:
            t.start()
        for t in th:
            t.join(timeout=120)
        p.send_signal(signal.SIGTERM)
        rc = p.wait(timeout=60)
        tail = p.stderr.read()
    assert rc == 128 + signal.SIGTERM
    for i in range(len(xs)):
        assert got[i] == want[i], i
    m = re.search(r"(\d+) row\(s\) in (\d+) device batch", tail)
    assert m and int(m.group(1)) == 16 * 64, tail
    print("serve: %s rows in %s device batches" % (m.group(1), m.group(2)), flush=True)
    assert int(m.group(2)) < 16, tail


def test_stream_file_and_pipe(tmp_path):
    """stream over a file and over stdin/stdout: the reference's row-protocol
    answer (odd_q4, exact path), byte for byte."""
    c = SERVE["odd_q4"]["rows"]
    src, out = tmp_path / "rows.txt", tmp_path / "out.txt"
    src.write_text(c["send"])
    model = os.path.join(GOLDEN, "odd_q4.tgir")
    print("case stream file", flush=True)
    r = subprocess.run([CLI, "stream", model, str(src), "-o", str(out), "--exact"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert out.read_text() == c["recv"]
    print("case stream pipe", flush=True)
    r = subprocess.run([CLI, "stream", model, "--exact"], input=c["send"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout == c["recv"], r.stderr


def test_overlong_lines_and_a_stop_with_a_connection_open():
    """A row line and an HTTP header line longer than 64 MiB end their
    connection with an error (the server does not grow its buffer past
    that), while other connections are served; SIGTERM with a client still
    connected stops the server cleanly (the batcher drained and joined) with
    status 128 + SIGTERM."""
    big = b"1," * (33 << 20) + b"1"  # 66 MiB, no line end
    with server("odd_q4", "--exact") as (p, port):
        s = socket.create_connection(("127.0.0.1", port), timeout=60)
        try:
            s.sendall(big)
        except OSError:
            pass  # the server may close the connection while we still send
        got = b""
        try:
            while True:
                k = s.recv(1 << 16)
                if not k:
                    break
                got += k
        except OSError:
            pass
        s.close()
        assert got.startswith(b"error: line longer than"), got[:200]
        h = socket.create_connection(("127.0.0.1", port), timeout=60)
        try:
            h.sendall(b"GET /health HTTP/1.1\r\nX-Big: " + big + b"\r\n\r\n")
        except OSError:
            pass
        reply = b""
        try:
            while True:
                k = h.recv(1 << 16)
                if not k:
                    break
                reply += k
        except OSError:
            pass
        h.close()
        assert reply.startswith(b"HTTP/1.1 431 "), reply[:200]
        assert converse(port, SERVE["odd_q4"]["health"]["send"]) == SERVE["odd_q4"]["health"]["recv"]
        idle = socket.create_connection(("127.0.0.1", port), timeout=60)  # stays open through the stop
        p.send_signal(signal.SIGTERM)
        rc = p.wait(timeout=60)
        idle.close()
    assert rc == 128 + signal.SIGTERM
