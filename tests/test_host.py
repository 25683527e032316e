"""Host-side checks that need no GPU: the C-ABI library loads and exports every
entry point of include/tg_hip.h, the CLI is built, and the benchmark's host
preparation (seeded initializers, quantizer, TGIR text) reproduces the
reference's algorithms as pinned through the oracle."""
import os
import re
import subprocess

import numpy as np
import pytest

from oracle import oracle as O
from technograd_amd import hip, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def header_functions():
    text = open(os.path.join(ROOT, "include", "tg_hip.h")).read()
    return sorted(set(re.findall(r"\b(tg_hip_\w+)\s*\(", text)))


def test_library_exports_every_declared_entry_point():
    L = hip.lib()
    names = header_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(L, n), n


def test_symbols_are_c_abi():
    out = subprocess.run(["nm", "-D", "--defined-only", hip.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (tg_hip_\w+)", out))
    assert set(header_functions()) <= exported  # plain C names, no C++ mangling


def test_cli_is_built_and_refuses_bad_usage():
    exe = os.environ.get("TGC_HIP") or os.path.join(ROOT, "technograd_amd", "bin", "tgc-hip")
    assert os.access(exe, os.X_OK)
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode != 0 and "usage" in r.stderr


def test_rand_matches_reference_initializer():
    for seed, scale, n in [(0, 1.0, 5000), (1, 0.05, 70000), (11, 0.35, 128), (0x7FFFFFFF, 2.0, 9999)]:
        a, b = synth.rand(seed, scale, n), O.rand(seed, scale, n)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), seed


def test_latent_reasoner_text_is_the_reference_lowering():
    assert synth.latent_reasoner_tgir() == open(os.path.join(GOLDEN, "latent_f32.tgir")).read()


@pytest.mark.parametrize("bits,axis,shape", [(8, 0, (48, 40)), (4, 0, (33, 513)), (4, 1, (48, 24)), (8, 1, (16, 300))])
def test_rtn_quantizer_matches_the_backend_quantizer(bits, axis, shape):
    """synth.quantize_rtn == the backend's `tgc quantize` (tg_hip_quantize_model
    on the host, byte-identical with the reference's quantizer on the goldens:
    tests/test_quantize.py)."""
    w = synth.normal(bits * 10 + axis, 0.3, shape[0] * shape[1]).reshape(shape)
    w[0] = 0  # an all-zero row
    codes, scales = synth.quantize_rtn(w, bits, axis)
    nm_in = "x" if axis == 0 else "h"
    if axis == 0:
        text = "(tgir 1\n  (model q)\n" + synth.param_f32("W", w) + "  (input x (f32 %d))\n  (block\n    (%%0 (f32 %d) (matmul W x))\n  )\n  (output %%0))\n" % (shape[1], shape[0])
    else:
        text = "(tgir 1\n  (model q)\n" + synth.param_f32("W", w) + "  (input h (f32 %d))\n  (block\n    (%%0 (f32 %d) (matmul h W))\n  )\n  (output %%0))\n" % (shape[0], shape[1])
    del nm_in
    want, _, _ = hip.quantize_model(text, bits=bits, min_size=1)
    got = "(tgir 1\n  (model q)\n" + synth.param_quant("W", codes, scales, bits, axis)
    # compare codes and scales token by token (the code layout is not canonical)
    def qtokens(s):
        q = s[s.index("(quant"):]
        sc = q[q.index("(scale") + 6:q.index(")", q.index("(scale"))].split()
        cd = q[q.index("(codes") + 6:q.index(")", q.index("(codes"))].split()
        return [float(v) for v in sc], [int(v) for v in cd]
    ws, wc = qtokens(want)
    gs, gc = qtokens(got)
    assert np.array_equal(np.float32(ws), np.float32(gs))
    assert wc == gc


def test_config2_model_text_round_trips_through_the_oracle():
    W = synth.normal(5, 0.02, 64 * 96).reshape(64, 96)
    text = synth.linear_tgir("lin", W, 4)
    m = O.Model(text)
    x = synth.normal(6, 1.0, 3 * 96).reshape(3, 96)
    y, _ = m.batch(x)
    c, s = synth.quantize_rtn(W, 4, 0)
    dq = c.astype(np.float32) * s[:, None]
    assert np.allclose(y, x @ dq.T, rtol=1e-4, atol=1e-5)


def test_xorshift_lanes_equal_sequential_stream():
    """The jump-ahead stream (used for large inputs) is the same stream."""
    import numpy as np
    from technograd_amd import synth
    n = 2 * 4096 * 64 + 4096 * 3 + 11
    lanes = synth._stream_lanes(np.uint32(5), n, L=4096, B=64)
    assert np.array_equal(lanes, synth.xorshift_stream(5, n))


def test_normal_is_chunk_invariant():
    """normal() of a prefix equals the prefix of a longer normal()."""
    import numpy as np
    from technograd_amd import synth
    a = synth.normal(3, 1.0, 1001)
    b = synth.normal(3, 1.0, 5000)
    assert np.array_equal(a, b[:1001])


@pytest.mark.parametrize("bits,axis,shape", [(4, 0, (70, 130)), (4, 1, (130, 70)), (8, 0, (33, 257)), (8, 1, (257, 200)),
                                             (4, 1, (64, 1000))])
def test_native_rtn_quantizer_matches_python(bits, axis, shape):
    """tg_hip_quantize_rtn (the library's host quantizer, used for models too
    large for numpy) writes the same codes and scales as synth.quantize_rtn,
    itself pinned to the reference's quantizer; all-zero and constant
    channels included."""
    from technograd_amd import hip
    rng = np.random.default_rng(sum(shape) + bits)
    w = rng.normal(0, 0.02, size=shape).astype(np.float32)
    if axis == 0:
        w[3] = 0.0
        w[5] = 0.25
    else:
        w[:, 3] = 0.0
        w[:, 5] = -0.5
    c1, s1 = synth.quantize_rtn(w, bits, axis)
    c2, s2 = hip.quantize_rtn(w, bits, axis, threads=3)
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))
    assert np.array_equal(c1, c2)
