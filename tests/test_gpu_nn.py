"""GPU parity of the skinny Q4_K kernel (k_gemm_q4_k_nn: N <= 32 output columns, M of several
thousand rows; config 4's b / a projections), through the C ABI, against the CPU oracle.

Shapes: M = 4133 (64 whole 64-row workgroups and a ragged one of 37 rows), N = 32 (two 16-column
blocks), 20 (a ragged second block) and 9 (one block), K = 256 (one super-block), 2560 (an even
super-block count) and 2816 (odd: the last super-block in the first register set). Weights: random
blocks and the special-scale blocks of test_gpu_parity (d = 0, dmin = 0, negative, subnormal and 30x
scales, all-zero rows). Bars as in test_gpu_parity.py: rel-L2 <= 1e-3 and max-abs <= 2e-3 (Q4_K; 1e-2
for the special scales, as test_gemm_special_scales), and within 2^-13 |W| @ |a| of the float64 product; the kernel carries each weight as an exact fp16
hi / lo pair, so it meets the exact kernels' bound. The accumulate mode adds into fp32 and fp16 C.
"""
import numpy as np
import pytest

import synth
from conftest import max_abs, rel_l2
from test_gpu_parity import f64_reference, special_q4_k_weights

pytestmark = pytest.mark.gpu

M_NN = 4133


def say(*a):
    print("[gpu]", *a, flush=True)


@pytest.mark.parametrize("N,K", [(32, 2560), (20, 2816), (9, 256)])
@pytest.mark.parametrize("special", [False, True])
def test_nn_parity(hqlib, oracle, N, K, special):
    blocks = special_q4_k_weights(300 + N, N, K) if special else synth.q4_k_blocks(synth.Rng(301 + N), N, K)
    a = synth.activations_f16(synth.Rng(302 + K), M_NN, K)
    name = hqlib.gemm_kernel(synth.Q4_K, M_NN, N, K)
    say(f"nn M={M_NN} N={N} K={K} special={special} kernel={name}")
    assert name.startswith("k_gemm_q4_k_nn<")
    W = hqlib.Mat(blocks, synth.Q4_K, N, K)
    got = hqlib.gemm_np(W, a, c_f32=True)
    c0b = synth.activations_f16(synth.Rng(303), M_NN, N)
    c0 = c0b.view(np.float16).astype(np.float32)
    acc32 = hqlib.gemm_np(W, a, c_f32=True, c_init=c0)
    acc16 = hqlib.gemm_np(W, a, c_f32=False, c_init=c0b).view(np.float16).astype(np.float32)
    W.free()
    ref = oracle.matmul(blocks, synth.Q4_K, N, K, oracle.f16_to_f32(a))
    r, m = rel_l2(got, ref), max_abs(got, ref)
    say(f"rel_l2 {r:.2e} max_abs {m:.2e} max|ref| {np.abs(ref).max():.2f}")
    bar = 1e-2 if special else 2e-3  # (special scales: outputs up to ~1e3, the bar of test_gemm_special_scales)
    assert r <= 1e-3 and m <= bar
    f64, bound = f64_reference(oracle, blocks, synth.Q4_K, N, K, a)
    assert np.all(np.abs(got - f64) <= 2.0 ** -13 * bound + 1e-30)
    if special:
        assert np.all(got[:, N // 7] == 0.0)  # the row with d = dmin = 0 everywhere
    assert max_abs(acc32, ref + c0) <= bar
    # fp16 C: the sum rounded once to fp16 (half an ulp of |y| on top of the bar)
    y = ref + c0
    assert np.all(np.abs(acc16 - y) <= bar + np.abs(y) * 2.0 ** -11)
