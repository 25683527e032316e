"""GEMM epilogue chains (technograd_amd/csrc/tg_hip.cpp: epi_chain,
kern_qgemm.hip: staged_epilogue): the instructions right after a
quantized product that only read its results (bias and residual adds,
scalings, activations, then a softmax or rmsnorm over the channels) run in
the product's own kernel. The values must be those of the same instructions
run one launch at a time, bit for bit: each model is also run with one more
instruction reading the product, which keeps the layer builder from fusing,
and the two outputs are compared. The row op runs inside the large-batch GEMM
when a tile holds whole lines (C <= 256, channel stride 1) and after it
otherwise; the cases cover both, every other GEMM kernel (one row, up to 16
rows, the small-batch tiles, the kernel for rows of at most 32 inputs), int4
and int8 weights, both operand orders,
all three operand forms, rows the reference's loop takes (inf, nan), and a
line with an outlier (a split row)."""
import numpy as np
import pytest

from technograd_amd import synth

pytestmark = pytest.mark.gpu


def _weight(name, seed, C, K, bits, axis):
    """name: [C][K] (axis 0, W @ x) or [K][C] (axis 1, x @ W) int-`bits` param"""
    W = synth.normal(seed, 0.05, C * K).reshape(C, K)
    if axis == 1:
        W = np.ascontiguousarray(W.T)
    c, s = synth.quantize_rtn(W, bits, axis)
    return synth.param_quant(name, c, s, bits, axis)


def _f32(name, a):
    return synth.param_f32(name, np.asarray(a, np.float32))


def _model(params, inputs, body, out, extra=None):
    """extra: one more instruction reading the product (no fusion)"""
    text = "(tgir 1\n  (model e)\n" + "".join(params)
    text += "".join("  (input %s (f32 %s))\n" % (n, s) for n, s in inputs)
    text += "  (block\n" + body + (extra or "") + "  )\n  (output %s))\n" % out
    return text


def _run(text, x):
    from technograd_amd import hip
    prog = hip.Program(text, max_rows=len(x))
    y, _ = prog.batch(x)
    return y, prog.stats().epilogue_ins


def _same(a, b):
    na, nb = np.isnan(a), np.isnan(b)
    assert np.array_equal(na, nb)
    assert np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def _case(params, inputs, body, out, shape_of_product, x, fused_ins):
    n = int(body.strip().splitlines()[-1].split()[0].lstrip("(%")) + 1  # next temporary
    extra = "    (%%%d (f32 %s) (mul %%0 %%0))\n" % (n, shape_of_product)
    got, ins = _run(_model(params, inputs, body, out), x)
    want, ins0 = _run(_model(params, inputs, body, out, extra), x)
    assert ins == fused_ins and ins0 == 0
    _same(got, want)
    return got


def _rows(seed, rows, per, specials=False):
    x = synth.normal(seed, 1.0, rows * per).reshape(rows, per)
    if specials and rows > 4:
        x[1, 5] = np.inf
        x[2, 7] = np.nan
        x[3, :] *= 1e-30
        x[4, 10] = 1e4  # an outlier: its line is a split row
    return x


@pytest.mark.parametrize("bits,rows,K,C", [(4, 1, 1024, 96), (4, 5, 1024, 96), (8, 40, 512, 300), (8, 700, 512, 2048),
                                           (4, 2100, 512, 2048), (8, 1200, 16, 600)])
def test_bias_tanh_vector(bits, rows, K, C):
    """W @ x + b, then tanh: every GEMM kernel, one output line per row"""
    print("case bias tanh", bits, rows, K, C, flush=True)
    params = [_weight("W", 11, C, K, bits, 0), _f32("b", synth.normal(12, 0.1, C))]
    body = ("    (%%0 (f32 %d) (matmul W x))\n    (%%1 (f32 %d) (add %%0 b))\n    (%%2 (f32 %d) (tanh %%1))\n" % (C, C, C))
    _case(params, [("x", str(K))], body, "%2", str(C), _rows(13, rows, K, specials=True), 2)


@pytest.mark.parametrize("bits,rows,T,K,C", [(4, 300, 64, 256, 256), (8, 3, 64, 256, 256), (8, 200, 96, 384, 200),
                                             (4, 40, 64, 512, 512), (4, 20, 64, 30, 64)])
def test_residual_rmsnorm(bits, rows, T, K, C):
    """rmsnorm(r + x @ W) over the C channels: inside the large-batch GEMM
    for C <= 256 at >= 16384 lines, after it otherwise"""
    print("case residual rmsnorm", bits, rows, T, K, C, flush=True)
    params = [_weight("W", 21, C, K, bits, 1)]
    body = ("    (%%0 (f32 %d %d) (matmul x W))\n    (%%1 (f32 %d %d) (add r %%0))\n    (%%2 (f32 %d %d) (rmsnorm %%1))\n" %
            (T, C, T, C, T, C))
    x = np.concatenate([_rows(22, rows, T * K, specials=True), _rows(23, rows, T * C)], axis=1)
    _case(params, [("x", "%d %d" % (T, K)), ("r", "%d %d" % (T, C))], body, "%2", "%d %d" % (T, C), x, 2)


@pytest.mark.parametrize("bits,rows,T,K,C", [(8, 200, 96, 384, 200), (4, 300, 64, 256, 24), (4, 7, 64, 256, 24),
                                             (8, 40, 64, 16, 24)])
def test_scale_bias_softmax(bits, rows, T, K, C):
    """softmax(s * (x @ W) - b): a scalar, a per-channel operand on the left
    of a subtraction, then the softmax"""
    print("case scale bias softmax", bits, rows, T, K, C, flush=True)
    params = [_weight("W", 31, C, K, bits, 1), _f32("s", [0.75]), _f32("b", synth.normal(32, 0.5, C))]
    body = ("    (%%0 (f32 %d %d) (matmul x W))\n    (%%1 (f32 %d %d) (mul s %%0))\n    (%%2 (f32 %d %d) (sub b %%1))\n"
            "    (%%3 (f32 %d %d) (softmax %%2))\n" % (T, C, T, C, T, C, T, C))
    _case(params, [("x", "%d %d" % (T, K))], body, "%3", "%d %d" % (T, C), _rows(33, rows, T * K, specials=True), 3)


def test_chain_stops_where_a_value_is_read_twice():
    """tanh's result is read three times after it: the chain (bias, tanh)
    ends there and the GEMM stores tanh's result for the later reads"""
    C, K, rows = 128, 256, 64
    params = [_weight("W", 41, C, K, 8, 0), _f32("b", synth.normal(42, 0.1, C))]
    body = ("    (%%0 (f32 %d) (matmul W x))\n    (%%1 (f32 %d) (add %%0 b))\n    (%%2 (f32 %d) (tanh %%1))\n"
            "    (%%3 (f32 %d) (mul %%2 %%2))\n    (%%4 (f32 %d) (add %%3 %%2))\n" % (C, C, C, C, C))
    _case(params, [("x", str(K))], body, "%4", str(C), _rows(43, rows, K), 2)


def test_operand_made_by_an_elementwise_run():
    """the residual is an elementwise result that only the epilogue reads:
    the fused elementwise run must still store it (a run keeps only the
    results read outside it)"""
    T, K, C, rows = 64, 256, 128, 40
    params = [_weight("W", 51, C, K, 8, 1), _f32("g", [1.5])]
    body = ("    (%%0 (f32 %d %d) (mul r g))\n    (%%1 (f32 %d %d) (tanh %%0))\n    (%%2 (f32 %d %d) (matmul x W))\n"
            "    (%%3 (f32 %d %d) (add %%1 %%2))\n    (%%4 (f32 %d %d) (rmsnorm %%3))\n" % (T, C, T, C, T, C, T, C, T, C))
    x = np.concatenate([_rows(52, rows, T * K), _rows(53, rows, T * C)], axis=1)
    n = 5
    extra = "    (%%%d (f32 %d %d) (mul %%2 %%2))\n" % (n, T, C)
    inputs = [("x", "%d %d" % (T, K)), ("r", "%d %d" % (T, C))]
    got, ins = _run(_model(params, inputs, body, "%4"), x)
    want, ins0 = _run(_model(params, inputs, body, "%4", extra), x)
    assert ins == 2 and ins0 == 0
    _same(got, want)


@pytest.mark.parametrize("bits,rows,T,K,C", [(8, 64, 512, 16, 512), (4, 40, 512, 64, 768)])
def test_bias_rows_of_several_channel_tiles(bits, rows, T, K, C):
    """x @ W + b, then softplus, over more than one channel tile of the
    large-batch GEMM (config 5's dt projection: 16 inputs, 512 channels)"""
    print("case bias tiles", bits, rows, T, K, C, flush=True)
    params = [_weight("W", 61, C, K, bits, 1), _f32("b", synth.normal(62, 0.5, C))]
    body = ("    (%%0 (f32 %d %d) (matmul x W))\n    (%%1 (f32 %d %d) (add %%0 b))\n    (%%2 (f32 %d %d) (softplus %%1))\n" %
            (T, C, T, C, T, C))
    _case(params, [("x", "%d %d" % (T, K))], body, "%2", "%d %d" % (T, C), _rows(63, rows, T * K, specials=True), 2)


def test_chain_that_saves_nothing_is_not_taken():
    """four instructions fill a chain and a fifth elementwise instruction
    reads its value, which nothing else reads: without the chain the five
    would be one fused elementwise run reading the product, so the chain
    would only slow the GEMM down; the builder keeps the product alone"""
    C, K, rows = 128, 256, 64
    params = [_weight("W", 71, C, K, 8, 0), _f32("b", synth.normal(72, 0.1, C)), _f32("s", [0.5])]
    body = ("    (%%0 (f32 %d) (matmul W x))\n    (%%1 (f32 %d) (add %%0 b))\n    (%%2 (f32 %d) (tanh %%1))\n"
            "    (%%3 (f32 %d) (mul %%2 s))\n    (%%4 (f32 %d) (sub %%3 b))\n    (%%5 (f32 %d) (relu %%4))\n" % ((C,) * 6))
    _case(params, [("x", str(K))], body, "%5", str(C), _rows(73, rows, K), 0)


def test_scan_neighbours_folded():
    """A selective scan's du product (mul dt x) and Mamba's gate after it
    ((y + x * D) * silu(z)) run inside the fused scan's kernel: 5
    instructions per block of the config 5 model; and over 16384 rows or
    more the in-projection's silu, its only reader but not the next
    instruction, runs in that projection's stores (it then does not merge
    with the z projection). The same model with one more reader of each
    scan's du and stacked output and of each silu's input (which keeps the
    builder from folding anything) gives the same bits, on 520 sequences of
    32 steps (16,640 rows, every block)."""
    import re
    from technograd_amd import hip
    print("case scan neighbours folded", flush=True)
    T, seqs = 32, 520
    text = synth.ssm_tgir("ssm", T=T)
    x = synth.config5_rows(seqs, T)
    prog = hip.Program(text, max_rows=seqs)
    got, _ = prog.batch(x)
    st = prog.stats()
    emits = re.findall(r"\(emit (%\d+) \((f32 [\d ]+)\)", text)
    dus = re.findall(r"\(carry [^\n]*\n\s+\(in %\d+ \(f32 \d+\) (%\d+)\)\n\s+\(in %\d+ \(f32 \d+\) (%\d+)\)", text)
    silus = re.findall(r"\(%\d+ \((f32 [\d ]+)\) \(silu (%\d+)\)\)", text)
    assert len(emits) == 4 and len(dus) == 4 and st.scan_folded_ins == 5 * len(emits), (st.scan_folded_ins, len(emits), len(dus))
    extra, nid = "", 90000
    for (ys, shape), (_, du) in zip(emits, dus):
        for v in (ys, du):
            extra += "    (%%%d (%s) (mul %s %s))\n" % (nid, shape, v, v)
            nid += 1
    for shape, v in silus:
        extra += "    (%%%d (%s) (mul %s %s))\n" % (nid, shape, v, v)
        nid += 1
    cut = text.rindex("  )\n  (output")
    prog2 = hip.Program(text[:cut] + extra + text[cut:], max_rows=seqs)
    want, _ = prog2.batch(x)
    st2 = prog2.stats()
    assert st2.scan_folded_ins == 0 and st.epilogue_ins - st2.epilogue_ins == len(emits), (st.epilogue_ins, st2.epilogue_ins)
    _same(got, want)
