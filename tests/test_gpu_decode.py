"""KV-cache decoding (tg_hip_dec_*) against the fixed-length forward.

The reference runs a Qwen3-shaped model at one sequence length and has no
cache. Its fixed-length forward (the layer executor, pinned to the
reference's own outputs by the qwen3_* goldens) fed the prompt plus the tokens
generated so far gives the logits the decoder must produce at each step: bit
for bit, since every kernel keeps the reference's operations and order and the
masked keys contribute exact zeros."""
import numpy as np
import pytest

from technograd_amd import hip, synth

pytestmark = pytest.mark.gpu

DIMS = dict(L=2, D=64, NQ=4, NKV=2, HD=16, FF=96, V=320)


@pytest.fixture(scope="module", autouse=True)
def device():
    hip.init(0)


def fixed_forward(T, ids, dims=DIMS):
    """Last-position logits of the fixed-length graph at length T."""
    text = synth.qwen3_tgir("q", T=T, **dims)
    return hip.Program(text, max_rows=len(ids)).batch(np.asarray(ids, np.float32))[0]


def check_decode(seqs, T0, steps, dims):
    text = synth.qwen3_tgir("q", T=T0, rope_len=T0 + steps, **dims)
    prog = hip.Program(text, max_rows=seqs)
    dec = hip.Decoder(prog, seqs, T0, T0 + steps)
    assert dec.layers == dims["L"] and dec.vocab == dims["V"]
    prompts = np.random.default_rng(T0 + seqs).integers(0, dims["V"], size=(seqs, T0)).astype(np.float32)
    prompts[0, 0] = dims["V"] - 1
    tokens, logits = dec.generate(prompts, steps, logits=True)
    ids = prompts
    for s in range(steps):
        want = fixed_forward(T0 + s, ids, dims)
        assert np.array_equal(logits[s].view(np.uint32), want.view(np.uint32)), "step %d" % s
        assert np.array_equal(tokens[:, s], want.argmax(axis=1)), "step %d" % s
        ids = np.concatenate([ids, tokens[:, s:s + 1].astype(np.float32)], axis=1)
    dec.close()


# (32, 72, 2): a prompt of 2304 token rows takes the many-lines norm kernels
@pytest.mark.parametrize("seqs,T0,steps", [(5, 8, 6), (3, 1, 4), (2, 70, 3), (32, 72, 2)])
def test_decode_equals_fixed_length_forward(seqs, T0, steps):
    print("case decode", seqs, T0, steps, flush=True)
    check_decode(seqs, T0, steps, DIMS)


def test_decode_prompt_attention_tiles():
    """Head size 64 and a 130-token prompt: the prompt's causal products run
    tiled, score tiles above the diagonal skipped and each 64-row tile of the
    probability-times-V product summing keys up to its last row only."""
    print("case decode tiles", flush=True)
    check_decode(4, 130, 2, dict(L=1, D=128, NQ=2, NKV=1, HD=64, FF=96, V=320))
