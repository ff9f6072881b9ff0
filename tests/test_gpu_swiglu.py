"""The SwiGLU FFN input (src/cuda_backend.cu:845-849 gate + up + k_swiglu :413-416) as one GEMM over a
gate/up pair matrix (hq_mat_upload_pair + hq_gemm_swiglu), through the C ABI, against the oracle's
gate and up matmuls: silu(g) * u in float64, the GPU's fp16 output within half an ulp of |y| on top
of the 1e-2 bar. M > 64 runs the fused epilogue of the full-K tile kernels (the product never
leaves the tile: the register-decode kernels k_gemm_q4_k_wr / k_gemm_q4_k_wr160 / k_gemm_q8_0_wr where
their 128 x 192 or 128 x 160 tiles fill the CUs, e.g. M = 512 at I = 9728, else the LDS-decode
kernels); other M run one GEMM for both halves and a separate epilogue pass."""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu]", *a, flush=True)


CASES = [(synth.Q4_K, 9728, 2560, M) for M in (1, 16, 64, 65, 512)] + \
        [(synth.Q8_0, 9728, 2560, M) for M in (1, 33, 128, 512)] + \
        [(synth.Q4_K, 1000, 512, 200), (synth.Q8_0, 1000, 512, 131), (synth.Q6_K, 1024, 512, 100),
         (synth.Q4_K, 2560, 9728, 300)] + \
        [(synth.Q4_K, 9728, 1024, 448), (synth.Q8_0, 9728, 1024, 500), (synth.Q4_K, 9720, 512, 512),
         (synth.Q8_0, 9720, 512, 512)]
# (the last four: the register-decode tile kernels' epilogue over two launches, with a ragged last row
# tile, and with a ragged last column tile: 2 x 9720 = 101 x 192 + 48 = 121 x 160 + 80)


@pytest.mark.parametrize("gtype,I,K,M", CASES)
def test_gemm_swiglu_parity(hqlib, oracle, gtype, I, K, M):
    gb = synth.random_blocks(gtype, synth.Rng(90 + I), I, K)
    ub = synth.random_blocks(gtype, synth.Rng(91 + I), I, K)
    a = synth.activations_f16(synth.Rng(92 + M), M, K)
    P = hqlib.PairMat(gb, ub, gtype, I, K)
    say(f"gemm_swiglu type={gtype} M={M} I={I} K={K}")
    got = hqlib.gemm_swiglu_np(P, a).view(np.float16).astype(np.float64)
    P.free()
    x = oracle.f16_to_f32(a)
    g = oracle.matmul(gb, gtype, I, K, x).astype(np.float64)
    u = oracle.matmul(ub, gtype, I, K, x).astype(np.float64)
    want = g / (1.0 + np.exp(-g)) * u
    err = np.abs(got - want)
    say(f"max err {err.max():.2e} max|y| {np.abs(want).max():.2f}")
    assert np.all(err <= 1e-2 + np.abs(want) * 2.0 ** -11)


def test_pair_refusals(hqlib):
    import ctypes as C
    gb = synth.q4_k_blocks(synth.Rng(1), 24, 256)
    ub = synth.q8_0_blocks(synth.Rng(2), 24, 256)
    wg = hqlib.WMat(3, 24, 256, gb.ctypes.data, synth.Q4_K, 0)
    wu = hqlib.WMat(3, 24, 256, ub.ctypes.data, synth.Q8_0, 0)
    h = C.c_void_p()
    assert hqlib.load().hq_mat_upload_pair(C.byref(wg), C.byref(wu), 0, C.byref(h)) == -1
    assert "differ" in hqlib.last_error() and h.value is None
    with pytest.raises(hqlib.HQError, match="multiple of 8"):
        hqlib.PairMat(synth.q4_k_blocks(synth.Rng(3), 12, 256), synth.q4_k_blocks(synth.Rng(4), 12, 256), synth.Q4_K,
                      12, 256)
    W = hqlib.Mat(gb, synth.Q4_K, 24, 256)
    with pytest.raises(hqlib.HQError, match="pair"):
        hqlib.gemm_swiglu_np(W, synth.activations_f16(synth.Rng(5), 2, 256))
    W.free()
