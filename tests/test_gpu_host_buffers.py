"""tg_hip_batch with rows, outputs and steps in pinned memory from
tg_hip_host_alloc (moved over PCIe directly, in smaller chunks) against the
same call on ordinary numpy arrays (copied through the library's staging
slots): the same bits, for a quantized model over several chunks and for a
think model's outputs and steps, with buffers at an offset inside their
allocations."""
import os

import numpy as np
import pytest

from technograd_amd import hip, synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def device():
    print("host buffers: tg_hip_init(0)", flush=True)
    hip.init(0)


def pinned_like(a, offset=64):
    """a copy of a in a HostBuffer, `offset` bytes into the allocation"""
    hb = hip.HostBuffer(a.nbytes + offset)
    v = hb.array(np.uint8, (a.nbytes + offset,))[offset:].view(a.dtype).reshape(a.shape)
    v[:] = a
    return hb, v


@pytest.mark.parametrize("case", ["config2_4096", "latent_f32"])
def test_pinned_buffers_equal_pageable(case):
    print("case host buffers", case, flush=True)
    if case == "config2_4096":
        text = synth.linear_tgir("linear4096", synth.config2_weight(), 4)
        x = synth.normal(2, 1.0, 4096 * 4096).reshape(4096, 4096)
    else:
        with open(os.path.join(GOLDEN, case + ".tgir")) as f:
            text = f.read()
        x = np.load(os.path.join(GOLDEN, case + ".npz"))["x"]
    prog = hip.Program(text, max_rows=len(x))
    want, wsteps = prog.batch(x)
    bx, px = pinned_like(np.ascontiguousarray(x, np.float32))
    by, py = pinned_like(np.zeros_like(want))
    bs, ps = pinned_like(np.zeros_like(wsteps))
    got, gsteps = prog.batch(px, py, ps)
    assert got is py and gsteps is ps
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(gsteps, wsteps)
    # rows pinned, outputs not (and the other way round)
    o1, _ = prog.batch(px)
    o2, _ = prog.batch(x, py, ps)
    assert np.array_equal(o1.view(np.uint32), want.view(np.uint32)) and np.array_equal(o2.view(np.uint32), want.view(np.uint32))
    for b in (bx, by, bs):
        b.free()
    prog.close()


def test_host_free_refuses_foreign_pointers():
    a = np.zeros(16, np.float32)
    assert hip.lib().tg_hip_host_free(a.ctypes.data) == -1
    hb = hip.HostBuffer(64)
    assert hip.lib().tg_hip_host_free(hb.ptr + 16) == -1  # inside, but not the start
    hb.free()
