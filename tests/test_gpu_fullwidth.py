"""Configs 3 and 5 at their real widths on the GPU, against the CPU oracle.

Config 3 (examples/qwen3/import.py:110-130): hidden 1024, 16 query and 8 KV
heads of 128, SwiGLU 3072, vocabulary 151,936, two of its layers, int4
weights quantized per output channel. The weights go to raw files next to
the TGIR text (the text forms would take several GB; the product's reader
and the oracle's both take the file forms). The fixed-length forward is
checked against the oracle interpreter (the reference's arithmetic) under
the whole-model predicate with the f64 interpreter as truth, its
151,936-way argmax against the oracle's wherever the two top logits are not
within that tolerance of each other, and the KV-cache decoder's logits
against that forward bit for bit at every step.

Config 5 (the selective-SSM classifier): d_model 256, 16 states, expand 2,
four blocks, T = 32, 520 sequences, so every projection runs on 16,640 rows
(past the 16,384-row block the launchers split at)."""
import os
import sys

import numpy as np
import pytest

from oracle import oracle as O
from technograd_amd import hip, synth

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import parity  # noqa: E402

pytestmark = pytest.mark.gpu

C3 = dict(L=2, D=1024, NQ=16, NKV=8, HD=128, FF=3072, V=151936)


@pytest.fixture(scope="module", autouse=True)
def device():
    print("full width: tg_hip_init(0)", flush=True)
    hip.init(0)


@pytest.fixture(scope="module")
def c3_files(tmp_path_factory):
    """One set of config 3 weight files for every sequence length here."""
    return str(tmp_path_factory.mktemp("qwen3")), {}


def c3_text(files, T, rope_len=None):
    path, cache = files
    return synth.qwen3_tgir("q", T=T, files=path, cache=cache, rope_len=rope_len,
                            quantizer=hip.quantize_rtn, **C3)


def prompts(seqs, T, seed):
    ids = np.random.default_rng(seed).integers(0, C3["V"], size=(seqs, T)).astype(np.float32)
    ids[0, 0] = C3["V"] - 1  # the last embedding row
    return ids


def check_argmax(name, y, ref, t):
    """Device argmax equals the oracle's on every row, or the two logits are
    within the row's tolerance of each other in the truth (a tie)."""
    tol = 2 * np.abs(ref.astype(np.float64) - t).max(axis=1) + 2 * parity.ulp(np.abs(t).max(axis=1))
    for r in range(len(y)):
        g, o = int(y[r].argmax()), int(ref[r].argmax())
        if g != o:
            assert abs(t[r, g] - t[r, o]) <= 2 * tol[r], (name, r, g, o, t[r, g], t[r, o])
    print("%s argmax: %d of %d rows as the oracle's" % (name, int((y.argmax(1) == ref.argmax(1)).sum()), len(y)),
          flush=True)


def test_config3_forward_against_oracle(c3_files):
    print("case config3 full width: forward T=16, 3 sequences", flush=True)
    text = c3_text(c3_files, 16)
    ids = prompts(3, 16, 7)
    y, _ = hip.Program(text, max_rows=3).batch(ids)
    assert y.shape == (3, C3["V"]) and np.isfinite(y).all()
    m = O.Model(text)
    ref, _ = m.batch(ids)
    t, _ = m.batch64(ids)
    ng = parity.check_model(y, ref, t)
    print("config3: %d of %d logits needed the row-error clause" % (ng, y.size), flush=True)
    check_argmax("config3", y, ref, t)


def test_config3_decoder_against_forward(c3_files):
    """Prompt of 12 tokens, 3 steps: every step's logits equal the
    fixed-length forward over the prompt plus the tokens so far, bit for
    bit, and every token is that forward's argmax."""
    seqs, T0, steps = 2, 12, 3
    print("case config3 full width: decoder", seqs, T0, steps, flush=True)
    prog = hip.Program(c3_text(c3_files, T0, rope_len=T0 + steps), max_rows=seqs)
    dec = hip.Decoder(prog, seqs, T0, T0 + steps)
    assert dec.layers == C3["L"] and dec.vocab == C3["V"]
    ids = prompts(seqs, T0, 11)
    tokens, logits = dec.generate(ids, steps, logits=True)
    dec.close()
    for s in range(steps):
        want = hip.Program(c3_text(c3_files, T0 + s), max_rows=seqs).batch(ids)[0]
        assert np.array_equal(logits[s].view(np.uint32), want.view(np.uint32)), "step %d" % s
        assert np.array_equal(tokens[:, s], want.argmax(axis=1)), "step %d" % s
        print("config3 decoder step %d: tokens %s" % (s, tokens[:, s].tolist()), flush=True)
        ids = np.concatenate([ids, tokens[:, s:s + 1].astype(np.float32)], axis=1)


def test_config5_past_one_row_block():
    seqs, T = 520, 32
    print("case config5 full width: %d sequences of %d steps" % (seqs, T), flush=True)
    text = synth.ssm_tgir("ssm", T=T)
    x = synth.config5_rows(seqs, T)
    y, _ = hip.Program(text, max_rows=seqs).batch(x)
    assert y.shape == (seqs, 8) and np.isfinite(y).all()
    m = O.Model(text)
    ref, _ = m.batch(x)
    t, _ = m.batch64(x)
    ng = parity.check_model(y, ref, t)
    print("config5: %d of %d outputs needed the row-error clause" % (ng, y.size), flush=True)
    check_argmax("config5", y, ref, t)
