"""GGUF Q2_K, Q3_K and Q5_K on the GPU (src/ggml_quant.h:100-150), through the C ABI, against the CPU
oracle (pinned bit-exact to the reference build, to closed forms and to tests/golden/*q{2,3,5}_k.npz):
upload round trip with perm_heads, bit-exact decode (random, special scales, golden), GEMV / GEMM /
gather parity at the north-star bar (rel-L2 <= 1e-3, max-abs <= 1e-2) at 9728 x 2560 with M in
{1, 64, 512} and at ragged and long-K shapes, the accumulate mode, and the fused single-token
gate/up + SwiGLU with a k-quant on either side."""
import ctypes as C

import numpy as np
import pytest

import synth
from conftest import max_abs, rel_l2, same_bits_nan_aware

pytestmark = pytest.mark.gpu
TYPES = [synth.Q2_K, synth.Q3_K, synth.Q5_K]


def say(*a):
    print("[gpu]", *a, flush=True)


@pytest.mark.parametrize("gtype", TYPES)
def test_upload_round_trip_and_dequant(hqlib, oracle, gtype):
    import oracle as o
    from test_oracle import load_golden, special_kquant_blocks
    name = synth.TYPE_NAMES[gtype]
    N, K = 64, 1024
    blocks = synth.random_blocks(gtype, synth.Rng(71 + gtype), N, K)
    say(f"{name} upload round trip, perm_heads 4")
    W = hqlib.Mat(blocks, gtype, N, K, 4)
    wm = o.WMat(3, N, K, blocks.ctypes.data, gtype, 4)
    src = [oracle.lib.or_src_row(C.byref(wm), r) for r in range(N)]
    assert np.array_equal(W.download(), blocks[src])
    assert same_bits_nan_aware(hqlib.dequant(W), oracle.dequantize(blocks, gtype, N, K, 4))
    assert same_bits_nan_aware(hqlib.dequant(W, 5, 11), oracle.dequantize(blocks, gtype, N, K, 4)[5:16])
    W.free()
    sp = special_kquant_blocks(gtype)
    say(f"{name} special scales")
    W = hqlib.Mat(sp, gtype, 2, 1024)
    assert same_bits_nan_aware(hqlib.dequant(W), oracle.dequantize(sp, gtype, 2, 1024))
    W.free()
    g = load_golden(f"dequant_{name.lower()}.npz")
    W = hqlib.Mat(g["blocks"], gtype, int(g["rows"]), int(g["cols"]), int(g["perm_heads"]))
    assert same_bits_nan_aware(hqlib.dequant(W), g["values"])
    W.free()


# GEMV, the Stream-K GEMM at each row-block count, ragged M / N, long K
CASES = [(9728, 2560, M) for M in (1, 2, 16, 33, 64, 512)] + \
        [(100, 512, M) for M in (1, 5, 17, 65)] + [(2560, 9728, 1), (2560, 9728, 64), (1000, 256, 3)] + \
        [(2560, 9728, 512), (9728, 2560, 300), (200, 20480, 1)] + \
        [(9728, 2560, 96), (4000, 4096, 100), (100, 33024, 1)]
# (the last six: the tile kernel with K split in 4, ragged M; a GEMV over a long K; the tile kernel
# with K split in 2 parts of 10 stages, ragged M, and in 4 parts of 8 stages, ragged M and N; a GEMV
# whose activation vector (K > 32768) stays in global memory)


@pytest.mark.parametrize("gtype", TYPES)
@pytest.mark.parametrize("N,K,M", CASES)
def test_gemm_parity(hqlib, oracle, gtype, N, K, M):
    blocks = synth.random_blocks(gtype, synth.Rng(72 + N + gtype), N, K)
    a = synth.activations_f16(synth.Rng(73 + M), M, K)
    W = hqlib.Mat(blocks, gtype, N, K)
    say(f"{synth.TYPE_NAMES[gtype]} gemm M={M} N={N} K={K} kernel={hqlib.gemm_kernel(gtype, M, N, K)}")
    got = hqlib.gemm_np(W, a)
    c0 = synth.activations_f16(synth.Rng(74), M, N).view(np.float16).astype(np.float32)
    acc = hqlib.gemm_np(W, a, c_f32=True, c_init=c0)
    W.free()
    ref = oracle.matmul(blocks, gtype, N, K, oracle.f16_to_f32(a))
    r, m = rel_l2(got, ref), max_abs(got, ref)
    say(f"rel_l2 {r:.2e} max_abs {m:.2e} max|ref| {np.abs(ref).max():.2f}")
    assert r <= 1e-3 and m <= 1e-2
    assert max_abs(acc, ref + c0) <= 1e-2


@pytest.mark.parametrize("gtype", TYPES)
def test_gemm_special_scales(hqlib, oracle, gtype):
    """Zero, subnormal and large d / dmin and all-zero / all-0xFF codes (the finite ones of the special
    blocks): GEMV and GEMM at the bar, and within 2^-13 |W| @ |a| of the float64 product."""
    from test_oracle import special_kquant_blocks
    sp = special_kquant_blocks(gtype).reshape(8, -1)  # 8 super-blocks
    bb = synth.BLOCK_BYTES[gtype]
    fin = []
    for i in range(8):
        w = oracle.dequantize(np.ascontiguousarray(sp[i:i + 1]), gtype, 1, 256)
        if np.all(np.isfinite(w)) and np.abs(w).max() < 1e4:
            fin.append(i)
    rows = np.stack([np.concatenate([sp[fin[(r + c) % len(fin)]] for c in range(10)]) for r in range(48)])
    N, K = rows.shape[0], 10 * 256
    assert rows.shape[1] == 10 * bb
    W = hqlib.Mat(np.ascontiguousarray(rows), gtype, N, K)
    wf = oracle.dequantize(np.ascontiguousarray(rows), gtype, N, K).astype(np.float64)
    for M in (1, 7, 40):
        a = synth.activations_f16(synth.Rng(75 + M), M, K)
        say(f"{synth.TYPE_NAMES[gtype]} special M={M}")
        got = hqlib.gemm_np(W, a)
        x = oracle.f16_to_f32(a).astype(np.float64)
        ref = oracle.matmul(np.ascontiguousarray(rows), gtype, N, K, oracle.f16_to_f32(a))
        assert rel_l2(got, ref) <= 1e-3 and max_abs(got, ref) <= 1e-2
        assert np.all(np.abs(got - x @ wf.T) <= 2.0 ** -13 * (np.abs(x) @ np.abs(wf.T)) + 1e-30)
    W.free()


@pytest.mark.parametrize("gtype,rel", [(synth.Q3_K, 2.0 ** -10), (synth.Q6_K, 2.0 ** -10), (synth.Q2_K, 2.0 ** -10),
                                       (synth.Q5_K, 2.0 ** -13)])
def test_tile_kernel_special_scales(hqlib, oracle, gtype, rel):
    """The LDS-decode tile kernels (M > 64) on the finite special blocks: rel-L2 at the bar, and within
    rel |W| @ |a| of the float64 product plus 2^-24 sum |a|. Q3_K / Q6_K (k_gemm_kq_ws: B =
    fp16(q * fp16(d * s)), two roundings of at most 2^-11 each, and the fp16 subnormal spacing of d * s
    and of the weights) and Q2_K (k_gemm_kq_ws: B = fp16 of the fp32 weight): rel = 2^-10. Q5_K (k_gemm_q5_k_ws: B the exact integer s * q in units of d, the
    min term through bf16 hi / lo parts): rel = 2^-13, as for the exact kernels. (d = 1 with extreme
    scales gives outputs of ~2e5, where fp32 sums alone differ by more than the absolute 1e-2 of the
    bar; the float64 bound is the element-wise check here.)"""
    from test_oracle import SPECIAL_BLOCKS
    sp = SPECIAL_BLOCKS[gtype]().reshape(8, -1)
    fin = []
    for i in range(8):
        w = oracle.dequantize(np.ascontiguousarray(sp[i:i + 1]), gtype, 1, 256)
        if np.all(np.isfinite(w)) and np.abs(w).max() < 1e4:
            fin.append(i)
    N, K, M = 5120, 10 * 256, 512
    rows = np.stack([np.concatenate([sp[fin[(r + c) % len(fin)]] for c in range(10)]) for r in range(N)])
    W = hqlib.Mat(np.ascontiguousarray(rows), gtype, N, K)
    name = hqlib.gemm_kernel(gtype, M, N, K)
    say(f"{synth.TYPE_NAMES[gtype]} special tile M={M} kernel={name}")
    assert name.startswith("k_gemm_q5_k_ws<" if gtype == synth.Q5_K else "k_gemm_kq_ws<")
    a = synth.activations_f16(synth.Rng(79), M, K)
    got = hqlib.gemm_np(W, a)
    W.free()
    wf = oracle.dequantize(np.ascontiguousarray(rows), gtype, N, K).astype(np.float64)
    x = oracle.f16_to_f32(a).astype(np.float64)
    ref = oracle.matmul(np.ascontiguousarray(rows), gtype, N, K, oracle.f16_to_f32(a))
    r, m = rel_l2(got, ref), max_abs(got, ref)
    say(f"rel_l2 {r:.2e} max_abs {m:.2e} max|ref| {np.abs(ref).max():.2f}")
    assert r <= 1e-3
    bound = rel * (np.abs(x) @ np.abs(wf.T)) + 2.0 ** -24 * np.abs(x).sum(axis=1, keepdims=True)
    assert np.all(np.abs(got - x @ wf.T) <= bound)


@pytest.mark.parametrize("gtype", TYPES)
def test_gather(hqlib, oracle, gtype):
    V, K, B, k = 4096, 2560, 64, 8
    blocks = synth.random_blocks(gtype, synth.Rng(76 + gtype), V, K)
    rng = synth.Rng(77)
    H = synth.activations_f16(rng, B, K)
    ids = np.stack([rng.choice_without_replacement(V, k) for _ in range(B)]).astype(np.uint32)
    W = hqlib.Mat(blocks, gtype, V, K)
    say(f"{synth.TYPE_NAMES[gtype]} gather")
    got = hqlib.gather_dot_np(W, H, ids)
    W.free()
    ref = oracle.gather_dot(blocks, gtype, V, K, oracle.f16_to_f32(H), ids)
    assert rel_l2(got, ref) <= 1e-3 and max_abs(got, ref) <= 1e-2


@pytest.mark.parametrize("gate_type,up_type", [(synth.Q5_K, synth.Q6_K), (synth.Q2_K, synth.Q3_K), (synth.Q4_K, synth.Q5_K)])
def test_gemv_swiglu_kquants(hqlib, oracle, gate_type, up_type):
    """hq_gemv_swiglu against silu(oracle gate . a) * (oracle up . a), rounded to fp16 (half an ulp
    of |y| on top of the 1e-2 bar)."""
    N, K = 2048, 2560
    gb = synth.random_blocks(gate_type, synth.Rng(78), N, K)
    ub = synth.random_blocks(up_type, synth.Rng(79), N, K)
    a = synth.activations_f16(synth.Rng(80), 1, K)
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
