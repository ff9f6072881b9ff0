"""Config 1: the tiny Llama forward of the reference CPU path with every linear layer (q, k, v, o,
gate, up, down; 28 matmuls) and the option readout routed through the HIP path (hq_llama_forward),
against the oracle's pure-CPU forward, which is bit-exact with the reference build (test_oracle.py)
and with the committed golden logits.

The HIP path rounds each matmul input to fp16 (the GEMM operand type); the logits therefore agree to
within the north-star bar (max-abs <= 1e-2), not bit for bit.
"""
import numpy as np
import pytest

import synth
from conftest import max_abs, rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    return synth.tiny_llama(1)


def test_tiny_llama_logits(hqlib, oracle, model):
    from test_oracle import load_golden
    g = load_golden("tiny_llama.npz")
    tokens, ids = g["tokens"], g["ids"]
    print("[gpu] config 1: upload tiny Llama (4 layers, Q8_0)", flush=True)
    m = hqlib.LlamaModel(model)
    print("[gpu] config 1: forward T=128", flush=True)
    got = m.forward(tokens, ids)
    ref = oracle.llama_forward(model, tokens, ids)
    assert np.array_equal(ref.view(np.uint32), g["logits"].view(np.uint32))
    print(f"[gpu] logits hip {got} cpu {ref} max_abs {max_abs(got, ref):.2e} rel_l2 {rel_l2(got, ref):.2e}",
          flush=True)
    assert max_abs(got, ref) <= 1e-2
    assert rel_l2(got, ref) <= 1e-2
    # a second prompt: short, with repeated ids
    t2, i2 = tokens[:9], np.array([3, 3, 31999, 0], np.uint32)
    got2, ref2 = m.forward(t2, i2), oracle.llama_forward(model, t2, i2)
    assert max_abs(got2, ref2) <= 1e-2
    assert got2[0] == got2[1]
    with pytest.raises(hqlib.HQError, match="out of range"):
        m.forward(np.array([32000], np.uint32), i2)
    with pytest.raises(hqlib.HQError, match="out of range"):
        m.forward(t2, np.array([32000], np.uint32))
    m.free()


def test_tiny_llama_rope_table(hqlib, oracle, model):
    """A caller's RoPE table (model_t.rope_inv_freq; here the theta powers over per-frequency
    divisors 1 .. 8, the Llama 3.1 scaling a GGUF file carries, the table test_oracle.py pins
    bit-exact against the reference's model_load) reaches the HIP path's forward: it matches the
    oracle under that table, whose logits differ from the unscaled table's."""
    import synth as s
    tokens, ids = s.tiny_llama_prompt(T=96)
    c = model["cfg"]
    half = c["rot_dim"] // 2
    div = np.ones(half, np.float32)
    div[half // 2:] = 8.0
    div[half // 2 - 4:half // 2] = np.float32([1.5, 2.5, 4.0, 6.0])
    inv = (hqlib.rope_inv_freq(c["rope_theta"], c["rot_dim"]) / div).astype(np.float32)
    plain = oracle.llama_forward(model, tokens, ids)
    scaled_model = dict(model, rope_inv_freq=inv)
    m = hqlib.LlamaModel(scaled_model)
    got = m.forward(tokens, ids)
    m.free()
    ref = oracle.llama_forward(scaled_model, tokens, ids)
    print(f"[gpu] llama3 RoPE: max_abs {max_abs(got, ref):.2e} rel_l2 {rel_l2(got, ref):.2e}; "
          f"vs unscaled {max_abs(ref, plain):.2e}", flush=True)
    assert max_abs(got, ref) <= 1e-2 and rel_l2(got, ref) <= 1e-2
    assert max_abs(ref, plain) > 1e-4
