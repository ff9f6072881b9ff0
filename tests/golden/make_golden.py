"""Writes the golden fixtures in tests/golden/ from the reference's own CPU code.

Run in the build container (needs oracle/_ref/libref.so, compiled from /root/reference by
oracle/Makefile):  python tests/golden/make_golden.py
Every expected output below comes from the reference build (Reference), never from the oracle.
Inputs are synthetic (hilbert-pruned-8b_amd/synth.py), so only inputs and outputs are stored.

  dequant_q8_0.npz / dequant_q4_k.npz / dequant_q6_k.npz
                                       blocks (random + special scales) -> fp32 rows (wmat_row_f32)
  matmul_q8_0.npz / matmul_q4_k.npz / matmul_q6_k.npz
                                       blocks, x, y0 -> y = matmul(W, x, accumulate) (cpu_backend.c:39)
  tiny_llama.npz                       config-1 prompt -> logits (model_load + cpu backend forward),
                                       with the sha256 of synth.tiny_llama(1) to catch generator drift
  dequant_q{2,3,5}_k.npz / matmul_q{2,3,5}_k.npz
                                       the same two fixtures for Q2_K, Q3_K and Q5_K

`python tests/golden/make_golden.py kquants` writes only the Q2_K / Q3_K / Q5_K fixtures.
"""
import hashlib
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "hilbert-pruned-8b_amd"), os.path.join(ROOT, "oracle"), HERE,
                os.path.join(ROOT, "tests")]

import gguf_writer  # noqa: E402
import oracle  # noqa: E402
import synth  # noqa: E402
from test_oracle import (special_kquant_blocks, special_q4_k_blocks, special_q6_k_blocks,  # noqa: E402
                         special_q8_0_blocks)


def digest(model):
    h = hashlib.sha256()
    for key in ("embed", "lm_head", "final_norm"):
        h.update(np.ascontiguousarray(model[key]).tobytes())
    for L in model["layers"]:
        for key in sorted(L):
            h.update(np.ascontiguousarray(L[key]).tobytes())
    return h.hexdigest()


def main():
    ref = oracle.Reference()
    rng = synth.Rng(777)

    # dequant: 8 random rows + the special-scale rows, one matrix per type (perm_heads on Q8_0)
    sp = special_q8_0_blocks()  # 1 row x 512 values
    rnd = synth.q8_0_blocks(rng, 7, 512)
    blocks = np.ascontiguousarray(np.concatenate([sp, rnd]))
    vals = ref.dequantize(blocks, synth.Q8_0, 8, 512, perm_heads=2)
    np.savez_compressed(os.path.join(HERE, "dequant_q8_0.npz"), blocks=blocks, values=vals, gtype=synth.Q8_0, rows=8,
                        cols=512, perm_heads=2)

    sp = special_q4_k_blocks()  # 2 rows x 1024 values
    rnd = synth.q4_k_blocks(rng, 6, 1024)
    blocks = np.ascontiguousarray(np.concatenate([sp, rnd]))
    vals = ref.dequantize(blocks, synth.Q4_K, 8, 1024)
    np.savez_compressed(os.path.join(HERE, "dequant_q4_k.npz"), blocks=blocks, values=vals, gtype=synth.Q4_K, rows=8,
                        cols=1024, perm_heads=0)

    # matmul (reference selftest quant shape N=40, K=512, M=5; accumulate into y0)
    for name, gtype in (("matmul_q8_0.npz", synth.Q8_0), ("matmul_q4_k.npz", synth.Q4_K)):
        blocks = gen(rng, 40, 512)
        x = synth.activations_f16(rng, 5, 512).view(np.float16).astype(np.float32)
        y0 = rng.normal(5 * 40).astype(np.float32).reshape(5, 40)
        y = ref.matmul(blocks, gtype, 40, 512, x, y0.copy(), True)
        np.savez_compressed(os.path.join(HERE, name), blocks=blocks, x=x, y0=y0, y=y, gtype=gtype, rows=40, cols=512,
                            accumulate=True)

    # config 1: tiny Llama prompt logits
    model = synth.tiny_llama(1)
    tokens, ids = synth.tiny_llama_prompt(2)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.gguf")
        gguf_writer.write_tiny_llama(path, model)
        logits = ref.logits(path, tokens, ids)
    np.savez_compressed(os.path.join(HERE, "tiny_llama.npz"), tokens=tokens, ids=ids, logits=logits,
                        model_sha256=digest(model))
    # Q6_K (its own generator, so the fixtures above do not change): dequant of random + special
    # blocks with perm_heads, and a matmul with accumulate
    rng6 = synth.Rng(6666)
    sp = special_q6_k_blocks()  # 2 rows x 1024 values
    blocks = np.ascontiguousarray(np.concatenate([sp, synth.q6_k_blocks(rng6, 6, 1024)]))
    vals = ref.dequantize(blocks, synth.Q6_K, 8, 1024, perm_heads=2)
    np.savez_compressed(os.path.join(HERE, "dequant_q6_k.npz"), blocks=blocks, values=vals, gtype=synth.Q6_K, rows=8,
                        cols=1024, perm_heads=2)
    blocks = synth.q6_k_blocks(rng6, 40, 512)
    x = synth.activations_f16(rng6, 5, 512).view(np.float16).astype(np.float32)
    y0 = rng6.normal(5 * 40).astype(np.float32).reshape(5, 40)
    y = ref.matmul(blocks, synth.Q6_K, 40, 512, x, y0.copy(), True)
    np.savez_compressed(os.path.join(HERE, "matmul_q6_k.npz"), blocks=blocks, x=x, y0=y0, y=y, gtype=synth.Q6_K, rows=40,
                        cols=512, accumulate=True)
    print("golden fixtures written:", logits)


def kquants():
    """Q2_K, Q3_K, Q5_K: dequant of special + random blocks (perm_heads 2) and a matmul with
    accumulate (N = 40, K = 512, M = 5, the reference selftest's quant shape)."""
    ref = oracle.Reference()
    for gtype in (synth.Q2_K, synth.Q3_K, synth.Q5_K):
        name = synth.TYPE_NAMES[gtype].lower()
        rng = synth.Rng(7000 + gtype)
        sp = special_kquant_blocks(gtype)  # 2 rows x 1024 values
        gen = (lambda r, n, k: synth.q2_k_blocks(r, n, k, scale=1e-2)) if gtype == synth.Q2_K else \
            (lambda r, n, k: synth.random_blocks(gtype, r, n, k))  # (the scale these fixtures were written with)
        blocks = np.ascontiguousarray(np.concatenate([sp, gen(rng, 6, 1024)]))
        vals = ref.dequantize(blocks, gtype, 8, 1024, perm_heads=2)
        np.savez_compressed(os.path.join(HERE, f"dequant_{name}.npz"), blocks=blocks, values=vals, gtype=gtype, rows=8,
                            cols=1024, perm_heads=2)
        blocks = gen(rng, 40, 512)
        x = synth.activations_f16(rng, 5, 512).view(np.float16).astype(np.float32)
        y0 = rng.normal(5 * 40).astype(np.float32).reshape(5, 40)
        y = ref.matmul(blocks, gtype, 40, 512, x, y0.copy(), True)
        np.savez_compressed(os.path.join(HERE, f"matmul_{name}.npz"), blocks=blocks, x=x, y0=y0, y=y, gtype=gtype,
                            rows=40, cols=512, accumulate=True)
    print("k-quant fixtures written")


if __name__ == "__main__":
    if sys.argv[1:] == ["kquants"]:
        kquants()
    else:
        main()
        kquants()
