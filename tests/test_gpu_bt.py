"""GPU parity of the large-M Q4_K tile kernel (k_gemm_q4_k_bt: 256 x 256 tiles over the whole of K,
chosen where the Stream-K kernel ran before, from M of a few thousand up), through the C ABI,
against the CPU oracle on sampled rows.

Shapes: M = 4196 (16 whole 256-row tiles and a ragged one of 100 rows), N = 9672 (37 whole
256-column tiles and a ragged one of 200) or 9674 (N not a multiple of 4: the scalar store path),
K = 256 (one super-block: no rescale between units), 512, 1024 and 4096. Sampling: 8 rows of every
256-row tile plus the first and last row, every column. Bars as in test_gpu_parity.py: rel-L2 <=
1e-3 and max-abs <= 1e-2 (2e-3 for Q4_K); against the float64 product, 2^-13 |W| @ |a| per output.
"""
import numpy as np
import pytest

import synth
from conftest import max_abs, rel_l2
from test_gpu_configs import sample_cols, sample_rows
from test_gpu_parity import f64_reference, special_q4_k_weights

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS, Q4K_MAX_ABS = 1e-3, 1e-2, 2e-3
M_BT = 4196


def say(*a):
    print("[gpu]", *a, flush=True)


def check(got, ref, what):
    r, m = rel_l2(got, ref), max_abs(got, ref)
    say(f"{what}: rel_l2 {r:.2e} max_abs {m:.2e}")
    assert r <= REL_L2 and m <= Q4K_MAX_ABS, what


def run(hqlib, oracle, blocks, a, N, K, what, c_f32=True, c_init=None):
    M = a.shape[0]
    name = hqlib.gemm_kernel(synth.Q4_K, M, N, K)
    say(f"{what}: M={M} N={N} K={K} kernel={name}")
    assert name == "k_gemm_q4_k_bt"
    W = hqlib.Mat(blocks, synth.Q4_K, N, K)
    got = hqlib.gemm_np(W, a, c_f32=c_f32, c_init=c_init)
    W.free()
    return got


@pytest.mark.parametrize("N,K", [(9672, 512), (9674, 256)])
def test_bt_special_scales_ragged(hqlib, oracle, N, K):
    """Weights with zero, negative, subnormal and widely varying super-block scales (and one all-zero
    row, one min-term-only row), ragged last row and column tiles."""
    blocks = special_q4_k_weights(71 + N, N, K)
    a = synth.activations_f16(synth.Rng(72 + N), M_BT, K)
    got = run(hqlib, oracle, blocks, a, N, K, "bt special scales")
    rows = sample_rows(M_BT, tile=256)
    ref = oracle.matmul(blocks, synth.Q4_K, N, K, oracle.f16_to_f32(a[rows]))
    check(got[rows], ref, f"bt special scales ({len(rows)} rows)")
    r64, bound = f64_reference(oracle, blocks, synth.Q4_K, N, K, a[rows])
    assert np.all(np.abs(got[rows] - r64) <= 2.0 ** -13 * bound)
    assert np.all(got[:, N // 7] == 0.0)
    assert np.all(np.isfinite(got))


def test_bt_accumulate_and_fp16_output(hqlib, oracle):
    N, K = 9672, 1024
    blocks = synth.random_blocks(synth.Q4_K, synth.Rng(81), N, K)
    rng = synth.Rng(82)
    a = synth.activations_f16(rng, M_BT, K)
    c0 = rng.normal(M_BT * N).astype(np.float32).reshape(M_BT, N)
    rows = sample_rows(M_BT, tile=256)
    a_rows = oracle.f16_to_f32(a[rows])
    plain = oracle.matmul(blocks, synth.Q4_K, N, K, a_rows)
    got = run(hqlib, oracle, blocks, a, N, K, "bt accumulate fp32", c_init=c0)
    check(got[rows], plain + c0[rows], "bt accumulate fp32")
    got16 = run(hqlib, oracle, blocks, a, N, K, "bt fp16 out", c_f32=False).view(np.float16).astype(np.float32)
    assert np.all(np.abs(got16[rows] - plain) <= 1e-2 + np.abs(plain) * 2.0 ** -11)
    c16 = synth.f16_bits(c0)
    acc16 = run(hqlib, oracle, blocks, a, N, K, "bt accumulate fp16", c_f32=False, c_init=c16)
    acc16 = acc16.view(np.float16).astype(np.float32)
    want = plain + c16.view(np.float16).astype(np.float32)[rows]
    assert np.all(np.abs(acc16[rows] - want) <= 1e-2 + np.abs(want) * 2.0 ** -11)


def test_bt_positive_activations(hqlib, oracle):
    """Non-negative activations up to ~16: the min term no longer cancels within a sub-block, so the
    bf16 hi/lo split of the sub-block sums carries its largest error; scaling the activations by
    2^6 scales every output by 2^6 bit for bit."""
    N, K = 9672, 1024
    blocks = synth.random_blocks(synth.Q4_K, synth.Rng(91), N, K)
    rng = synth.Rng(92)
    a = synth.f16_bits(np.abs(rng.normal(M_BT * K)) * 4).reshape(M_BT, K)
    got = run(hqlib, oracle, blocks, a, N, K, "bt positive activations")
    a64 = synth.f16_bits(oracle.f16_to_f32(a) * 64).reshape(M_BT, K)
    got64 = run(hqlib, oracle, blocks, a64, N, K, "bt positive activations x 2^6")
    assert np.array_equal(got64, got * 64)
    rows = sample_rows(M_BT, tile=256)
    ref = oracle.matmul(blocks, synth.Q4_K, N, K, oracle.f16_to_f32(a[rows]))
    r = rel_l2(got[rows], ref)
    say(f"bt positive activations: rel_l2 {r:.2e} max_abs {max_abs(got[rows], ref):.2e}")
    assert r <= REL_L2
    r64, bound = f64_reference(oracle, blocks, synth.Q4_K, N, K, a[rows])
    assert np.all(np.abs(got[rows] - r64) <= 2.0 ** -13 * bound)


def test_bt_long_k_repeatable(hqlib, oracle):
    """K = 4096 (16 super-blocks, 64 stages through the triple-buffered LDS rings and the per-super-
    block tables written while the previous super-block is read): sampled parity, and three calls
    give the same bits (each output is one workgroup's fixed sequence of MFMAs, so any difference
    would come from a race between the waves' LDS writes and reads)."""
    N, K = 9672, 4096
    blocks = synth.random_blocks(synth.Q4_K, synth.Rng(101), N, K)
    a = synth.activations_f16(synth.Rng(102), M_BT, K)
    name = hqlib.gemm_kernel(synth.Q4_K, M_BT, N, K)
    say(f"bt long K: M={M_BT} N={N} K={K} kernel={name}")
    assert name == "k_gemm_q4_k_bt"
    W = hqlib.Mat(blocks, synth.Q4_K, N, K)
    got = [hqlib.gemm_np(W, a) for _ in range(3)]
    W.free()
    assert np.array_equal(got[0], got[1]) and np.array_equal(got[0], got[2])
    rows = sample_rows(M_BT, per_tile=4, tile=256)
    cols = sample_cols(N)
    ref = oracle.matmul(np.ascontiguousarray(blocks[cols]), synth.Q4_K, len(cols), K, oracle.f16_to_f32(a[rows]))
    check(got[0][np.ix_(rows, cols)], ref, f"bt long K ({len(rows)} rows x {len(cols)} columns)")
