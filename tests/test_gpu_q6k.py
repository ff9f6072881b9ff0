"""GGUF Q6_K on the GPU (src/ggml_quant.h:151-169), through the C ABI, against the CPU oracle
(pinned bit-exact to the reference build and to tests/golden/*q6_k.npz): upload round trip, bit-exact
decode, GEMV / GEMM / gather parity at the north-star bar, and the fused single-token gate/up+SwiGLU
with a Q4_K gate and a Q6_K up as Q4_K_M files pair them (src/cuda_backend.cu:1256)."""
import numpy as np
import pytest

import synth
from conftest import max_abs, rel_l2, same_bits_nan_aware

pytestmark = pytest.mark.gpu
Q6 = synth.Q6_K


def say(*a):
    print("[gpu]", *a, flush=True)


def test_q6k_upload_round_trip_and_dequant(hqlib, oracle):
    import ctypes as C
    import oracle as o
    from test_oracle import load_golden, special_q6_k_blocks
    N, K = 64, 1024
    blocks = synth.q6_k_blocks(synth.Rng(61), N, K)
    W = hqlib.Mat(blocks, Q6, N, K, 4)
    wm = o.WMat(3, N, K, blocks.ctypes.data, Q6, 4)
    src = [oracle.lib.or_src_row(C.byref(wm), r) for r in range(N)]
    say("Q6_K upload round trip, perm_heads 4")
    assert np.array_equal(W.download(), blocks[src])
    assert same_bits_nan_aware(hqlib.dequant(W), oracle.dequantize(blocks, Q6, N, K, 4))
    assert same_bits_nan_aware(hqlib.dequant(W, 5, 11), oracle.dequantize(blocks, Q6, N, K, 4)[5:16])
    W.free()
    sp = special_q6_k_blocks()
    W = hqlib.Mat(sp, Q6, 2, 1024)
    say("Q6_K special scales")
    assert same_bits_nan_aware(hqlib.dequant(W), oracle.dequantize(sp, Q6, 2, 1024))
    W.free()
    g = load_golden("dequant_q6_k.npz")
    W = hqlib.Mat(g["blocks"], Q6, int(g["rows"]), int(g["cols"]), int(g["perm_heads"]))
    assert same_bits_nan_aware(hqlib.dequant(W), g["values"])
    W.free()


# GEMV, the Stream-K GEMM at each row-block count, the tile kernel (M = 128, 512), ragged M / N, long K
CASES = [(9728, 2560, M) for M in (1, 2, 16, 33, 64, 128, 512)] + \
        [(100, 512, M) for M in (1, 5, 17, 65, 200)] + [(2560, 9728, 1), (2560, 9728, 64), (1000, 256, 3)] + \
        [(2560, 9728, 512), (9728, 2560, 300), (200, 20480, 1)] + \
        [(9728, 2560, 96), (4000, 4096, 100), (100, 33024, 1)]
# (the last six: the tile kernel with K split in 4, ragged M; a GEMV over a long K; the tile kernel
# with K split in 2 parts of 10 stages, ragged M, and in 4 parts of 8 stages, ragged M and N; a GEMV
# whose activation vector (K > 32768) stays in global memory)


@pytest.mark.parametrize("N,K,M", CASES)
def test_q6k_gemm_parity(hqlib, oracle, N, K, M):
    blocks = synth.q6_k_blocks(synth.Rng(62 + N), N, K)
    a = synth.activations_f16(synth.Rng(63 + M), M, K)
    W = hqlib.Mat(blocks, Q6, N, K)
    say(f"Q6_K gemm M={M} N={N} K={K} kernel={hqlib.gemm_kernel(Q6, M, N, K)}")
    got = hqlib.gemm_np(W, a)
    c0 = synth.activations_f16(synth.Rng(64), M, N).view(np.float16).astype(np.float32)
    acc = hqlib.gemm_np(W, a, c_f32=True, c_init=c0)
    W.free()
    ref = oracle.matmul(blocks, Q6, N, K, oracle.f16_to_f32(a))
    r, m = rel_l2(got, ref), max_abs(got, ref)
    say(f"rel_l2 {r:.2e} max_abs {m:.2e} max|ref| {np.abs(ref).max():.2f}")
    assert r <= 1e-3 and m <= 1e-2
    assert max_abs(acc, ref + c0) <= 1e-2


def test_q6k_gather(hqlib, oracle):
    V, K, B, k = 4096, 2560, 64, 8
    blocks = synth.q6_k_blocks(synth.Rng(65), V, K)
    rng = synth.Rng(66)
    H = synth.activations_f16(rng, B, K)
    ids = np.stack([rng.choice_without_replacement(V, k) for _ in range(B)]).astype(np.uint32)
    W = hqlib.Mat(blocks, Q6, V, K)
    say("Q6_K gather")
    got = hqlib.gather_dot_np(W, H, ids)
    W.free()
    ref = oracle.gather_dot(blocks, Q6, V, K, oracle.f16_to_f32(H), ids)
    assert rel_l2(got, ref) <= 1e-3 and max_abs(got, ref) <= 1e-2


@pytest.mark.parametrize("gate_type,up_type", [(synth.Q4_K, Q6), (synth.Q8_0, synth.Q8_0), (Q6, Q6)])
def test_gemv_swiglu_mixed_types(hqlib, oracle, gate_type, up_type):
    """hq_gemv_swiglu against silu(oracle gate . a) * (oracle up . a), rounded to fp16 (half an ulp
    of |y| on top of the 1e-2 bar)."""
    N, K = 9728, 2560
    gb = synth.random_blocks(gate_type, synth.Rng(67), N, K)
    ub = synth.random_blocks(up_type, synth.Rng(68), N, K)
    a = synth.activations_f16(synth.Rng(69), 1, K)
    G, U = hqlib.Mat(gb, gate_type, N, K), hqlib.Mat(ub, up_type, N, K)
    say(f"gemv_swiglu gate={gate_type} up={up_type}")
    got = hqlib.gemv_swiglu_np(G, U, a[0]).view(np.float16).astype(np.float32)
    G.free(), U.free()
    x = oracle.f16_to_f32(a)
    g = oracle.matmul(gb, gate_type, N, K, x)[0].astype(np.float64)
    u = oracle.matmul(ub, up_type, N, K, x)[0].astype(np.float64)
    want = g / (1.0 + np.exp(-g)) * u
    err = np.abs(got - want)
    say(f"max err {err.max():.2e} max|y| {np.abs(want).max():.2f}")
    assert np.all(err <= 1e-2 + np.abs(want) * 2.0 ** -11)
