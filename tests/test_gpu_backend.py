"""The HIP backend (include/hq_backend.h) driven through the reference's backend_t vtable: config 1
(tiny Llama, Q8_0, every projection through hq_gemm) against the reference CPU path's committed
golden logits, the snapshot / restore and single-token paths against the full prefill, last_hidden
against the readout, and hip_selftest (src/cuda_backend.cu:1392-1466) on the same model.

The HIP path rounds each GEMM input to fp16, so logits agree with the fp32 CPU path to the
north-star bar (max-abs <= 1e-2), not bit for bit; two HIP paths over the same tokens agree to 1e-3.
"""
import numpy as np
import pytest

import synth
from conftest import max_abs

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu]", *a, flush=True)


@pytest.fixture(scope="module")
def view(hqlib):
    return hqlib.RefModelView(synth.tiny_llama(1))


def test_backend_vtable_config1(hqlib, oracle, view):
    from test_oracle import load_golden
    g = load_golden("tiny_llama.npz")
    tokens, ids = g["tokens"], g["ids"]
    say("hip_backend_create: tiny Llama, max_seq 256")
    be = hqlib.HipBackend(view, 256)
    assert be.pos == 0
    full = be.forward(tokens, ids)
    say(f"full prefill logits {full} golden {g['logits']} max_abs {max_abs(full, g['logits']):.2e}")
    assert be.pos == len(tokens)
    assert max_abs(full, g["logits"]) <= 1e-2 and np.argmax(full) == np.argmax(g["logits"])
    # prefix, snapshot, suffix, restore, suffix again
    be.reset()
    be.forward(tokens[:64])
    be.snapshot()
    s1 = be.forward(tokens[64:], ids)
    be.restore()
    assert be.pos == 64
    s2 = be.forward(tokens[64:], ids)
    say(f"prefix+suffix {s1} after restore {s2}")
    assert np.array_equal(s1, s2)
    assert max_abs(s1, full) <= 1e-3
    # prefill of 127 tokens, then the last token alone (the fused T = 1 gate/up+SwiGLU path)
    be.reset()
    be.forward(tokens[:-1])
    step = be.forward(tokens[-1:], ids)
    say(f"one-token step {step}")
    assert max_abs(step, full) <= 1e-3
    # last_hidden is the final-normalised readout input: its dots with the lm_head rows are the logits
    h = be.last_hidden()
    head = synth.tiny_llama(1)["lm_head"]
    w = oracle.dequantize(np.ascontiguousarray(head[ids]), synth.Q8_0, len(ids), h.size)
    assert max_abs(w.astype(np.float64) @ h.astype(np.float64), step) <= 1e-4
    # errors, as the reference's forward reports them
    with pytest.raises(hqlib.HQError, match="out of range"):
        be.forward(np.array([32000], np.uint32))
    with pytest.raises(hqlib.HQError, match="exceed context"):
        be.forward(np.zeros(300, np.uint32))
    be.destroy()


def test_backend_chunks_and_gqa(hqlib, oracle):
    """A prompt longer than one layer-loop chunk (1024 tokens) and grouped-query attention (8 query
    heads over 2 kv heads) against the oracle's CPU forward of the same model."""
    cfg = dict(synth.TINY_LLAMA, n_layers=2, n_kv_heads=2, vocab=4096)
    model = synth.tiny_llama(3, cfg)
    tokens, ids = synth.tiny_llama_prompt(4, T=1100, vocab=cfg["vocab"], n_ids=8)
    v = hqlib.RefModelView(model)
    be = hqlib.HipBackend(v, 1200)
    say("chunked forward T=1100, GQA 8/2")
    got = be.forward(tokens, ids)
    be.destroy()
    ref = oracle.llama_forward(model, tokens, ids)
    say(f"hip {got} cpu {ref} max_abs {max_abs(got, ref):.2e}")
    assert max_abs(got, ref) <= 1e-2 and np.argmax(got) == np.argmax(ref)


def test_hip_selftest(hqlib, view):
    say("hip_selftest on the tiny Llama, 96 tokens")
    assert hqlib.hip_selftest(view, 0, 96, 1) == 0, hqlib.last_error()
