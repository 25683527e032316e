"""A quantized product read only by the tanh after it runs as one GEMM with
tanhf in its epilogue (technograd_amd/csrc/tg_hip.cpp: layer_block). Its
values must be those of the two instructions run apart: the same GEMM's
output, then the elementwise tanh kernel over it, bit for bit."""
import numpy as np
import pytest

from technograd_amd import synth

pytestmark = pytest.mark.gpu


def _model(body, K, C, W, bits):
    c, s = synth.quantize_rtn(W, bits, 0)
    return ("(tgir 1\n  (model m)\n" + synth.param_quant("W", c, s, bits, 0) +
            "  (input x (f32 %d))\n  (block\n%s  )\n  (output %%1))\n" % (K, body))


@pytest.mark.parametrize("bits_,rows,K,C", [(8, 700, 512, 2048), (4, 5, 1024, 96), (8, 64, 2048, 512)])
def test_fused_tanh_equals_product_then_tanh(bits_, rows, K, C):
    from technograd_amd import hip
    print("case fused tanh", bits_, rows, K, C, flush=True)
    W = synth.normal(7, 0.05, C * K).reshape(C, K)
    x = synth.normal(8, 1.0, rows * K).reshape(rows, K)
    fused = _model("    (%%0 (f32 %d) (matmul W x))\n    (%%1 (f32 %d) (tanh %%0))\n" % (C, C), K, C, W, bits_)
    prod = _model("    (%%0 (f32 %d) (matmul W x))\n    (%%1 (f32 %d) (mul %%0 %%0))\n" % (C, C), K, C, W, bits_)
    # the product alone: read it back through an output that is the product itself
    prod = prod.replace("(output %1)", "(output %0)")
    tanh_only = "(tgir 1\n  (model t)\n  (input y (f32 %d))\n  (block\n    (%%0 (f32 %d) (tanh y))\n  )\n  (output %%0))\n" % (C, C)
    got, _ = hip.Program(fused, max_rows=rows).batch(x)
    y, _ = hip.Program(prod, max_rows=rows).batch(x)
    want, _ = hip.Program(tanh_only, max_rows=rows).batch(y)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
