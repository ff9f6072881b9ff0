"""GPU parity of the one-round Q4_K tile kernels with loader waves, through the C ABI, against the
CPU oracle: k_gemm_q4_k_wr160 (128 x 160 tiles; the headline shape M = 512, N = 9728, K = 2560: 244
tiles) and k_gemm_q4_k_wr<3> (128 x 192 tiles, where 160-column tiles would not fit one round:
M = 300 .. 384 at N ~ 13000), both with 4 MFMA waves and 4 loader waves.

Shapes: M = 256, 300, 350 (two whole 128-row tiles and a ragged one of 94 rows), 384 and 512;
N = 9672 (60 whole 160-column tiles and a ragged one of 72: wave 0's and wave 1's full blocks whole,
wave 2's first half valid, the rest and both half blocks past N) or 9674 (N not a multiple of 4: the
element-wise store path); N = 13000 / 12996 for the 192-column kernel (67 whole tiles and a ragged one
of 136 / 132 columns); K = 256 (one super-block: no rescale between super-blocks), 512, 1024, 2560
and 4096 (the record ring of three slots wraps); more tiles than one round as launches of one round
each, or one launch of two rounds (test_wr_launches). The per-super-block column tables come from the
upload (k_q4k_tables), so every test also checks them. Bars as in test_gpu_parity.py: rel-L2 <= 1e-3
and max-abs <= 2e-3 (Q4_K); against the float64 product, 2^-13 |W| @ |a| per output.
"""
import numpy as np
import pytest

import synth
from conftest import max_abs, rel_l2
from test_gpu_configs import sample_cols, sample_rows
from test_gpu_parity import f64_reference, special_q4_k_weights

pytestmark = pytest.mark.gpu

REL_L2, Q4K_MAX_ABS = 1e-3, 2e-3
KERNELS = ("k_gemm_q4_k_wr160", "k_gemm_q4_k_wr<3>")


def say(*a):
    print("[gpu]", *a, flush=True)


def check(got, ref, what):
    r, m = rel_l2(got, ref), max_abs(got, ref)
    say(f"{what}: rel_l2 {r:.2e} max_abs {m:.2e}")
    assert r <= REL_L2 and m <= Q4K_MAX_ABS, what


def run(hqlib, blocks, a, N, K, what, c_f32=True, c_init=None):
    M = a.shape[0]
    name = hqlib.gemm_kernel(synth.Q4_K, M, N, K)
    say(f"{what}: M={M} N={N} K={K} kernel={name}")
    assert name in KERNELS
    W = hqlib.Mat(blocks, synth.Q4_K, N, K)
    got = hqlib.gemm_np(W, a, c_f32=c_f32, c_init=c_init)
    W.free()
    return got


@pytest.mark.parametrize("M,N,K", [(350, 9672, 512), (350, 9674, 256), (350, 9674, 2560), (300, 13000, 512),
                                   (300, 12996, 2560)])
def test_wr_special_scales_ragged(hqlib, oracle, M, N, K):
    """Weights with zero, negative, subnormal and widely varying super-block scales (and one all-zero
    row, one min-term-only row); ragged last row and column tiles; N % 4 != 0 at N = 9674; both tile
    widths."""
    blocks = special_q4_k_weights(171 + N, N, K)
    a = synth.activations_f16(synth.Rng(172 + N), M, K)
    got = run(hqlib, blocks, a, N, K, "wr special scales")
    rows = sample_rows(M)
    ref = oracle.matmul(blocks, synth.Q4_K, N, K, oracle.f16_to_f32(a[rows]))
    check(got[rows], ref, f"wr special scales ({len(rows)} rows)")
    r64, bound = f64_reference(oracle, blocks, synth.Q4_K, N, K, a[rows])
    assert np.all(np.abs(got[rows] - r64) <= 2.0 ** -13 * bound)
    assert np.all(got[:, N // 7] == 0.0)
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("M,N,K", [(512, 9728, 1024), (512, 9674, 1024), (512, 9728, 2560), (512, 9674, 2560),
                                   (384, 13000, 1024)])
def test_wr_accumulate_and_fp16_output(hqlib, oracle, M, N, K):
    blocks = synth.random_blocks(synth.Q4_K, synth.Rng(181 + N), N, K)
    rng = synth.Rng(182)
    a = synth.activations_f16(rng, M, K)
    c0 = rng.normal(M * N).astype(np.float32).reshape(M, N)
    rows = sample_rows(M)
    plain = oracle.matmul(blocks, synth.Q4_K, N, K, oracle.f16_to_f32(a[rows]))
    got = run(hqlib, blocks, a, N, K, "wr accumulate fp32", c_init=c0)
    check(got[rows], plain + c0[rows], "wr accumulate fp32")
    got16 = run(hqlib, blocks, a, N, K, "wr fp16 out", c_f32=False).view(np.float16).astype(np.float32)
    assert np.all(np.abs(got16[rows] - plain) <= 1e-2 + np.abs(plain) * 2.0 ** -11)
    c16 = synth.f16_bits(c0)
    acc16 = run(hqlib, blocks, a, N, K, "wr accumulate fp16", c_f32=False, c_init=c16)
    acc16 = acc16.view(np.float16).astype(np.float32)
    want = plain + c16.view(np.float16).astype(np.float32)[rows]
    assert np.all(np.abs(acc16[rows] - want) <= 1e-2 + np.abs(want) * 2.0 ** -11)


# more tiles than one round (wr4_plan): M = 1100 at N = 9672 as three launches of 4 row tiles (the
# last 76 rows) x 61 column tiles (the last ragged); M = 512, N = 19448 as one launch of two rounds
# (4 x 122 tiles, the last column tile ragged); M = 4096, N = 2560 as two launches of 16 x 16 tiles.
# Rows sampled for the oracle; fp32 output, then fp16 through the same launches.
@pytest.mark.parametrize("M,N,K", [(1100, 9672, 1024), (512, 19448, 1024), (4096, 2560, 1024)])
def test_wr_launches(hqlib, oracle, M, N, K):
    blocks = synth.random_blocks(synth.Q4_K, synth.Rng(201 + M), N, K)
    a = synth.activations_f16(synth.Rng(202 + N), M, K)
    rows = sample_rows(M)
    ref = oracle.matmul(blocks, synth.Q4_K, N, K, oracle.f16_to_f32(a[rows]))
    got = run(hqlib, blocks, a, N, K, "wr launches")
    check(got[rows], ref, f"wr launches M={M} N={N}")
    assert np.all(np.isfinite(got))
    got16 = run(hqlib, blocks, a, N, K, "wr launches fp16 out", c_f32=False).view(np.float16).astype(np.float32)
    assert np.all(np.abs(got16[rows] - ref) <= 1e-2 + np.abs(ref) * 2.0 ** -11)


def test_wr_positive_activations(hqlib, oracle):
    """Non-negative activations up to ~16: the min term no longer cancels within a sub-block, so the
    bf16 hi/lo split of the sub-block sums carries its largest error; scaling the activations by
    2^6 scales every output by 2^6 bit for bit."""
    M, N, K = 512, 9728, 1024
    blocks = synth.random_blocks(synth.Q4_K, synth.Rng(191), N, K)
    rng = synth.Rng(192)
    a = synth.f16_bits(np.abs(rng.normal(M * K)) * 4).reshape(M, K)
    got = run(hqlib, blocks, a, N, K, "wr positive activations")
    a64 = synth.f16_bits(oracle.f16_to_f32(a) * 64).reshape(M, K)
    got64 = run(hqlib, blocks, a64, N, K, "wr positive activations x 2^6")
    assert np.array_equal(got64, got * 64)
    rows = sample_rows(M)
    ref = oracle.matmul(blocks, synth.Q4_K, N, K, oracle.f16_to_f32(a[rows]))
    r = rel_l2(got[rows], ref)
    say(f"wr positive activations: rel_l2 {r:.2e} max_abs {max_abs(got[rows], ref):.2e}")
    assert r <= REL_L2
    r64, bound = f64_reference(oracle, blocks, synth.Q4_K, N, K, a[rows])
    assert np.all(np.abs(got[rows] - r64) <= 2.0 ** -13 * bound)


@pytest.mark.parametrize("M,N", [(350, 9672), (300, 13000)])
def test_wr_long_k_repeatable(hqlib, oracle, M, N):
    """K = 4096 (16 super-blocks, 64 stages through the 4-slot LDS ring and the double-buffered table
    records): sampled parity, and three calls give the same bits (each output is one workgroup's
    fixed sequence of MFMAs, so any difference would come from a race between the loader waves'
    DMA and the MFMA waves' reads); both tile widths."""
    K = 4096
    blocks = synth.random_blocks(synth.Q4_K, synth.Rng(201), N, K)
    a = synth.activations_f16(synth.Rng(202), M, K)
    name = hqlib.gemm_kernel(synth.Q4_K, M, N, K)
    say(f"wr long K: M={M} N={N} K={K} kernel={name}")
    assert name in KERNELS
    W = hqlib.Mat(blocks, synth.Q4_K, N, K)
    got = [hqlib.gemm_np(W, a) for _ in range(3)]
    W.free()
    assert np.array_equal(got[0], got[1]) and np.array_equal(got[0], got[2])
    rows = sample_rows(M, per_tile=4)
    cols = sample_cols(N)
    ref = oracle.matmul(np.ascontiguousarray(blocks[cols]), synth.Q4_K, len(cols), K, oracle.f16_to_f32(a[rows]))
    check(got[0][np.ix_(rows, cols)], ref, f"wr long K ({len(rows)} rows x {len(cols)} columns)")


def test_wr_two_row_tiles(hqlib, oracle):
    """M = 256 (two row tiles per column tile, no ragged rows), K = 2560: sampled parity; the
    workspace query reports none (the loader waves form the sub-block sums)."""
    M, N, K = 256, 9728, 2560
    assert hqlib.gemm_workspace_bytes(synth.Q4_K, M, N, K) == (0, 0, 0, True)
    blocks = synth.random_blocks(synth.Q4_K, synth.Rng(221), N, K)
    a = synth.activations_f16(synth.Rng(222), M, K)
    got = run(hqlib, blocks, a, N, K, "wr two row tiles")
    rows = sample_rows(M, per_tile=4)
    ref = oracle.matmul(blocks, synth.Q4_K, N, K, oracle.f16_to_f32(a[rows]))
    check(got[rows], ref, f"wr two row tiles ({len(rows)} rows)")


def test_wr_download_round_trip(hqlib):
    """The column tables sit after the blocks in the matrix's allocation: a download returns the
    GGUF blocks alone, and the device bytes count both."""
    N, K = 200, 512
    blocks = synth.random_blocks(synth.Q4_K, synth.Rng(211), N, K)
    W = hqlib.Mat(blocks, synth.Q4_K, N, K)
    assert np.array_equal(W.download(), blocks)
    assert W.device_bytes >= N * (K // 256) * (144 + 48)
    W.free()
