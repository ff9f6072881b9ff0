"""GPU parity of the one-round Q8_0 tile kernel with loader waves (k_gemm_q8_0_wr: 128 x 192 tiles,
4 MFMA waves and 4 loader waves; config 2's M = 512, N = 9728, K = 2560), through the C ABI, against
the CPU oracle.

Shapes: M = 500 (three whole 128-row tiles and a ragged one of 116 rows) and 512; N = 9672 (50 whole
192-column tiles and a ragged one of 72: one MFMA wave's columns whole, the next one's half, two waves
with none) or 9674 (N not a multiple of 4: the element-wise store path); K = 256 (one super-stage of
scales), 512, 1024, 2560 and 4096 (64 stages through the 4-slot LDS ring). Bars as in
test_gpu_parity.py: rel-L2 <= 1e-3 and max-abs <= 1e-2; the weight operand is fp16(q * d), one
rounding of the exact weight, so against the float64 product every output is within
2^-11 |W| @ |a| (the operand rounding) plus the fp32 accumulation's 2^-13 |W| @ |a|.
"""
import numpy as np
import pytest

import synth
from conftest import max_abs, rel_l2
from test_gpu_configs import sample_cols, sample_rows
from test_gpu_parity import f64_reference

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS = 1e-3, 1e-2
KERNEL = "k_gemm_q8_0_wr"
OPERAND_BOUND = 2.0 ** -11 + 2.0 ** -13


def say(*a):
    print("[gpu]", *a, flush=True)


def check(got, ref, what):
    r, m = rel_l2(got, ref), max_abs(got, ref)
    say(f"{what}: rel_l2 {r:.2e} max_abs {m:.2e}")
    assert r <= REL_L2 and m <= MAX_ABS, what


def run(hqlib, blocks, a, N, K, what, c_f32=True, c_init=None):
    M = a.shape[0]
    name = hqlib.gemm_kernel(synth.Q8_0, M, N, K)
    say(f"{what}: M={M} N={N} K={K} kernel={name}")
    assert name == KERNEL
    W = hqlib.Mat(blocks, synth.Q8_0, N, K)
    got = hqlib.gemm_np(W, a, c_f32=c_f32, c_init=c_init)
    W.free()
    return got


def special_q8_0_weights(seed, rows, cols):
    """Q8_0 weights whose block scales span the fp16 range the tile kernel supports: zero and -0,
    negative, subnormal (down to 2^-24), the smallest normal, and |N(0,1)| x 10^e for e = -5.5 .. 1.5
    (|q d| stays below fp16's 65504), each block's scale drawn independently; plus one
    row of zero scales (exact zeros) and q = -128 and 127 in every block."""
    rng = synth.Rng(seed)
    blk = synth.q8_0_blocks(rng, rows, cols)
    nb = rows * (cols // 32)
    v = blk.reshape(nb, 34)
    d = v[:, 0:2].copy().view(np.uint16).ravel()
    kind = rng.bytes(nb) % 8
    sub = (rng.bytes(nb * 2).view(np.uint16) & 0x3FF) | 1
    wide = synth.f16_bits(np.abs(rng.normal(nb)) * 10.0 ** (rng.bytes(nb) % 8 - 5.5))
    d = np.where(kind == 0, 0, d)
    d = np.where(kind == 1, 0x8000, d)
    d = np.where(kind == 2, d | 0x8000, d)
    d = np.where(kind == 3, sub, d)
    d = np.where(kind == 4, 0x0400, d)
    d = np.where(kind >= 5, wide, d).astype(np.uint16)
    d.reshape(rows, cols // 32)[rows // 7] = 0
    v[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    v[:, 2] = 0x80  # q = -128
    v[:, 3] = 0x7F  # q = 127
    return blk


@pytest.mark.parametrize("N,K", [(9672, 512), (9674, 256), (9674, 2560)])
def test_wr8_special_scales_ragged(hqlib, oracle, N, K):
    """Zero, negative, subnormal and widely varying block scales (one all-zero row); ragged last row
    and column tiles; N % 4 != 0 at N = 9674. Against the float64 product the error stays within the
    operand rounding's bound; the zero row is exactly zero."""
    M = 500
    blocks = special_q8_0_weights(231 + N, N, K)
    a = synth.activations_f16(synth.Rng(232 + N), M, K)
    got = run(hqlib, blocks, a, N, K, "wr8 special scales")
    rows = sample_rows(M)
    ref = oracle.matmul(blocks, synth.Q8_0, N, K, oracle.f16_to_f32(a[rows]))
    assert rel_l2(got[rows], ref) <= REL_L2
    r64, bound = f64_reference(oracle, blocks, synth.Q8_0, N, K, a[rows])
    err = np.abs(got[rows] - r64)
    say(f"wr8 special scales: rel_l2 {rel_l2(got[rows], ref):.2e}, max err / bound {np.max(err / np.maximum(bound, 1e-30)):.2e}")
    assert np.all(err <= OPERAND_BOUND * bound)
    assert np.all(got[:, N // 7] == 0.0)
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("N,K", [(9728, 1024), (9674, 1024), (9728, 2560), (9674, 2560)])
def test_wr8_accumulate_and_fp16_output(hqlib, oracle, N, K):
    M = 512
    blocks = synth.random_blocks(synth.Q8_0, synth.Rng(241 + N), N, K)
    rng = synth.Rng(242)
    a = synth.activations_f16(rng, M, K)
    c0 = rng.normal(M * N).astype(np.float32).reshape(M, N)
    rows = sample_rows(M)
    plain = oracle.matmul(blocks, synth.Q8_0, N, K, oracle.f16_to_f32(a[rows]))
    got = run(hqlib, blocks, a, N, K, "wr8 accumulate fp32", c_init=c0)
    check(got[rows], plain + c0[rows], "wr8 accumulate fp32")
    got16 = run(hqlib, blocks, a, N, K, "wr8 fp16 out", c_f32=False).view(np.float16).astype(np.float32)
    assert np.all(np.abs(got16[rows] - plain) <= 1e-2 + np.abs(plain) * 2.0 ** -11)
    c16 = synth.f16_bits(c0)
    acc16 = run(hqlib, blocks, a, N, K, "wr8 accumulate fp16", c_f32=False, c_init=c16)
    acc16 = acc16.view(np.float16).astype(np.float32)
    want = plain + c16.view(np.float16).astype(np.float32)[rows]
    assert np.all(np.abs(acc16[rows] - want) <= 1e-2 + np.abs(want) * 2.0 ** -11)


def test_wr8_positive_activations(hqlib, oracle):
    """Non-negative activations up to ~16 (no cancellation in the dot products); scaling the
    activations by 2^6 scales every output by 2^6 bit for bit."""
    M, N, K = 512, 9728, 1024
    blocks = synth.random_blocks(synth.Q8_0, synth.Rng(251), N, K)
    rng = synth.Rng(252)
    a = synth.f16_bits(np.abs(rng.normal(M * K)) * 4).reshape(M, K)
    got = run(hqlib, blocks, a, N, K, "wr8 positive activations")
    a64 = synth.f16_bits(f16_values(a) * 64).reshape(M, K)
    got64 = run(hqlib, blocks, a64, N, K, "wr8 positive activations x 2^6")
    assert np.array_equal(got64, got * 64)
    rows = sample_rows(M)
    ref = oracle.matmul(blocks, synth.Q8_0, N, K, oracle.f16_to_f32(a[rows]))
    check(got[rows], ref, "wr8 positive activations")
    r64, bound = f64_reference(oracle, blocks, synth.Q8_0, N, K, a[rows])
    assert np.all(np.abs(got[rows] - r64) <= OPERAND_BOUND * bound)


def f16_values(a16):
    return np.asarray(a16, dtype=np.uint16).view(np.float16).astype(np.float32)


def test_wr8_long_k_repeatable(hqlib, oracle):
    """K = 4096 (64 stages through the 4-slot LDS ring, 16 super-stages of scales through their two
    parities): sampled parity, and three calls give the same bits (each output is one workgroup's
    fixed sequence of MFMAs, so any difference would come from a race between the loader waves' DMA
    and the MFMA waves' reads)."""
    M, N, K = 500, 9672, 4096
    blocks = synth.random_blocks(synth.Q8_0, synth.Rng(261), N, K)
    a = synth.activations_f16(synth.Rng(262), M, K)
    name = hqlib.gemm_kernel(synth.Q8_0, M, N, K)
    say(f"wr8 long K: M={M} N={N} K={K} kernel={name}")
    assert name == KERNEL
    W = hqlib.Mat(blocks, synth.Q8_0, N, K)
    got = [hqlib.gemm_np(W, a) for _ in range(3)]
    W.free()
    assert np.array_equal(got[0], got[1]) and np.array_equal(got[0], got[2])
    rows = sample_rows(M, per_tile=4)
    cols = sample_cols(N)
    ref = oracle.matmul(np.ascontiguousarray(blocks[cols]), synth.Q8_0, len(cols), K, oracle.f16_to_f32(a[rows]))
    check(got[0][np.ix_(rows, cols)], ref, f"wr8 long K ({len(rows)} rows x {len(cols)} columns)")


def test_wr8_workspace_none(hqlib):
    """The kernel needs no workspace (its loads go straight to LDS, its output straight to C)."""
    assert hqlib.gemm_workspace_bytes(synth.Q8_0, 512, 9728, 2560) == (0, 0, 0, True)
    assert hqlib.gemm_tiles(synth.Q8_0, 512, 9728) == (128, 192)


@pytest.mark.parametrize("M,N,K", [(1000, 9672, 512), (2048, 2560, 1024)])
def test_wr8_several_launches(hqlib, oracle, M, N, K):
    """Many tiles: the GEMM as launches of at most one round of tiles per XCD (M = 1000: two launches
    of 512 and 488 rows, the second's last row tile ragged, x 51 column tiles; M = 2048 at N = 2560:
    one launch of 16 x 14 tiles, 32 on each of the XCDs that get two column tiles)."""
    blocks = synth.random_blocks(synth.Q8_0, synth.Rng(271 + M), N, K)
    a = synth.activations_f16(synth.Rng(272 + M), M, K)
    got = run(hqlib, blocks, a, N, K, "wr8 launches")
    rows = sample_rows(M, per_tile=4)
    ref = oracle.matmul(blocks, synth.Q8_0, N, K, oracle.f16_to_f32(a[rows]))
    check(got[rows], ref, f"wr8 launches ({len(rows)} rows)")
