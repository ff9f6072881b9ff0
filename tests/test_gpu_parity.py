"""GPU parity of the HIP path against the CPU oracle, through the C ABI (libhq.so).

Bars: dequantised weights bit-exact; GEMM/GEMV/gather outputs fp32 with
relative L2 <= 1e-3 and max-abs <= 1e-2 against the oracle matmul on identical inputs (fp16
activations widened exactly to fp32 on the CPU side). The Q4_K kernels never round a weight to
16 bits, so they are also held to a tighter internal bar (max-abs 2e-3) that a fp16-rounded-weight
regression would break (its tail error is ~2e-2 at K = 2560).
"""
import numpy as np
import pytest

import synth
from conftest import max_abs, rel_l2, same_bits_nan_aware

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS = 1e-3, 1e-2
Q4K_MAX_ABS = 2e-3


def say(*a):
    print("[gpu]", *a, flush=True)


def check(got, ref, gtype, what):
    r, m = rel_l2(got, ref), max_abs(got, ref)
    say(f"{what}: rel_l2 {r:.2e} max_abs {m:.2e}")
    assert r <= REL_L2 and m <= MAX_ABS, what
    if gtype == synth.Q4_K:
        assert m <= Q4K_MAX_ABS, what


_cache = {}


def weights(gtype, N, K, seed):
    key = (gtype, N, K, seed)
    if key not in _cache:
        _cache.clear()
        _cache[key] = synth.random_blocks(gtype, synth.Rng(seed), N, K)
    return _cache[key]


# ------------------------------------------------------------------ residency
@pytest.mark.parametrize("gtype,N,K,perm", [(synth.Q8_0, 64, 1408, 0), (synth.Q8_0, 512, 512, 8),
                                            (synth.Q4_K, 96, 2560, 0), (synth.Q4_K, 512, 512, 4)])
def test_upload_round_trip(hqlib, oracle, gtype, N, K, perm):
    say(f"upload round trip type={gtype} {N}x{K} perm={perm}")
    blocks = synth.random_blocks(gtype, synth.Rng(N + K), N, K)
    W = hqlib.Mat(blocks, gtype, N, K, perm)
    back = W.download()
    import oracle as o
    import ctypes as C
    wm = o.WMat(3, N, K, blocks.ctypes.data, gtype, perm)
    src = [oracle.lib.or_src_row(C.byref(wm), r) for r in range(N)]
    assert np.array_equal(back, blocks[src])
    W.free()


# ------------------------------------------------------------------ dequant (bit-exact)
@pytest.mark.parametrize("gtype,N,K,perm", [(synth.Q8_0, 37, 2560, 0), (synth.Q8_0, 64, 1408, 8),
                                            (synth.Q4_K, 37, 2560, 0), (synth.Q4_K, 64, 512, 2)])
def test_dequant_bit_exact(hqlib, oracle, gtype, N, K, perm):
    say(f"dequant type={gtype} {N}x{K} perm={perm}")
    blocks = synth.random_blocks(gtype, synth.Rng(5 * N + K), N, K)
    W = hqlib.Mat(blocks, gtype, N, K, perm)
    got = hqlib.dequant(W)
    assert same_bits_nan_aware(got, oracle.dequantize(blocks, gtype, N, K, perm))
    part = hqlib.dequant(W, 5, 11)
    assert same_bits_nan_aware(part, got[5:16])
    W.free()


def test_dequant_special_scales_bit_exact(hqlib, oracle):
    from test_oracle import special_q4_k_blocks, special_q8_0_blocks
    for gtype, sp in ((synth.Q8_0, special_q8_0_blocks()), (synth.Q4_K, special_q4_k_blocks())):
        r = sp.shape[0]
        c = sp.shape[1] // synth.BLOCK_BYTES[gtype] * synth.BLOCK_VALUES[gtype]
        say(f"dequant specials type={gtype} {r}x{c}")
        W = hqlib.Mat(np.ascontiguousarray(sp), gtype, r, c)
        assert same_bits_nan_aware(hqlib.dequant(W), oracle.dequantize(sp, gtype, r, c))
        W.free()


@pytest.mark.parametrize("name", ["dequant_q8_0.npz", "dequant_q4_k.npz"])
def test_dequant_golden(hqlib, name):
    from test_oracle import load_golden
    g = load_golden(name)
    say(f"dequant golden {name}")
    W = hqlib.Mat(g["blocks"], int(g["gtype"]), int(g["rows"]), int(g["cols"]), int(g["perm_heads"]))
    assert same_bits_nan_aware(hqlib.dequant(W), g["values"])
    W.free()


def test_embed_rows_bit_exact(hqlib, oracle):
    blocks = synth.q8_0_blocks(synth.Rng(8), 300, 512)
    W = hqlib.Mat(blocks, synth.Q8_0, 300, 512)
    ids = np.array([0, 299, 17, 17, 150], np.uint32)
    say("embed rows")
    got = hqlib.embed(W, ids)
    assert same_bits_nan_aware(got, oracle.dequantize(blocks, synth.Q8_0, 300, 512)[ids])
    with pytest.raises(hqlib.HQError, match="out of range"):
        hqlib.embed(W, np.array([300], np.uint32))
    W.free()


# ------------------------------------------------------------------ GEMV / GEMM parity
# configs 2 and 3 at full shape, every M of their sweeps up to 512, plus ragged shapes
FULL = [(synth.Q8_0, 9728, 2560, M) for M in (1, 16, 128, 512)] + \
       [(synth.Q4_K, 9728, 2560, M) for M in (1, 64, 512)] + \
       [(synth.Q4_K, 2560, 9728, M) for M in (1, 64, 512)]
RAGGED = [(synth.Q8_0, 100, 512, M) for M in (1, 2, 5, 17, 33, 65, 200)] + \
         [(synth.Q4_K, 100, 512, M) for M in (1, 2, 5, 17, 33, 65, 200)] + \
         [(synth.Q8_0, 40, 512, 5), (synth.Q8_0, 40, 512, 40), (synth.Q4_K, 40, 512, 5), (synth.Q4_K, 40, 512, 40),
          (synth.Q8_0, 1408, 512, 128), (synth.Q8_0, 512, 1408, 128), (synth.Q8_0, 72, 96, 3), (synth.Q8_0, 72, 96, 40),
          (synth.Q4_K, 130, 2560, 31), (synth.Q4_K, 33, 256, 1), (synth.Q4_K, 33, 256, 20)] + \
         [(synth.Q4_K, 9500, 768, 500), (synth.Q4_K, 9728, 512, 350), (synth.Q4_K, 9728, 256, 350),
          (synth.Q4_K, 9000, 768, 1000)] + \
         [(synth.Q4_K, 8200, 1536, 1), (synth.Q4_K, 9728, 512, 1), (synth.Q4_K, 8192, 1024, 1)] + \
         [(synth.Q8_0, 9500, 768, 500), (synth.Q8_0, 9728, 384, 512)] + \
         [(synth.Q4_K, 2560, 9728, 300), (synth.Q4_K, 2500, 4096, 300)] + \
         [(synth.Q8_0, 2560, 9728, 512), (synth.Q8_0, 2500, 8192, 300)] + \
         [(synth.Q4_K, 8200, 1536, 40), (synth.Q4_K, 8192, 512, 33)] + \
         [(synth.Q8_0, 8200, 1024, 5), (synth.Q8_0, 9728, 512, 40), (synth.Q8_0, 8192, 256, 30)] + \
         [(synth.Q4_K, 2500, 4096, 40), (synth.Q4_K, 4096, 2560, 48)] + \
         [(synth.Q8_0, 2560, 9728, 16), (synth.Q8_0, 2500, 4096, 40)] + \
         [(synth.Q8_0, 9728, 2560, 96), (synth.Q8_0, 4000, 4096, 100)] + \
         [(synth.Q4_K, 9728, 2560, 100), (synth.Q4_K, 4000, 4096, 96), (synth.Q4_K, 9728, 2560, 200),
          (synth.Q4_K, 10996, 5120, 100)]
# (the last: full-K tiles; Stream-K with more tiles than CUs; the streamed GEMV with a ragged last
# row group and an odd K split, with one wave per row group, and with an even split; the Q8_0 tile
# kernel with ragged M and N, and with an odd number of 128-wide stages; the Q4_K tile kernel with
# each tile's K split over 4 workgroups of 9 or 10 super-blocks, ragged M, and over 2 workgroups
# with ragged M and N; the Q8_0 tile kernel with K split over 4 workgroups, also with ragged M, N;
# the mid-M Q4_K kernel with a ragged last column tile and ragged M, and at M = 33 with K = 512; the
# mid-M Q8_0 kernel with ragged N and M at each of its row-block counts, and with one stage per
# pipeline; the mid-M Q4_K kernel with each tile's K split over 4 (ragged N, M) and 2 workgroups; the
# mid-M Q8_0 kernel with K splits over 6 and (ragged N, M) 4 workgroups; the Q8_0 tile kernel with K
# split over 2 workgroups of 10 stages (ragged M) and over 4 of 8 stages (ragged N, M); the Q4_K tile
# kernel with K split over 2 workgroups of 5 super-blocks (ragged M) and over 4 of 4 (ragged N, M); the
# register-decode kernel with K split over 2 workgroups of 5 super-blocks, ragged M, with 128 x 160
# tiles and, where those would not fit one round, 128 x 192 ones (4 workgroups of 5 super-blocks,
# ragged M and a ragged last column tile))


@pytest.mark.parametrize("gtype,N,K,M", FULL + RAGGED)
def test_gemm_parity(hqlib, oracle, gtype, N, K, M):
    say(f"gemm type={gtype} M={M} N={N} K={K} tiles={hqlib.gemm_tiles(gtype, M, N)}")
    blocks = weights(gtype, N, K, 100 + gtype)
    rng = synth.Rng(1000 + M + N + K)
    a = synth.activations_f16(rng, M, K)
    W = hqlib.Mat(blocks, gtype, N, K)
    got = hqlib.gemm_np(W, a)
    ref = oracle.matmul(blocks, gtype, N, K, oracle.f16_to_f32(a))
    check(got, ref, gtype, f"type={gtype} M={M} N={N} K={K}")
    W.free()


@pytest.mark.parametrize("gtype,M,N,K", [(synth.Q8_0, 1, 320, 1024), (synth.Q8_0, 48, 320, 1024),
                                         (synth.Q4_K, 1, 320, 1024), (synth.Q4_K, 48, 320, 1024),
                                         (synth.Q4_K, 350, 9728, 256), (synth.Q4_K, 1, 8192, 1024),
                                         (synth.Q8_0, 512, 9728, 640), (synth.Q4_K, 512, 9728, 2560),
                                         (synth.Q8_0, 512, 9500, 2560), (synth.Q4_K, 512, 2560, 9728),
                                         (synth.Q8_0, 512, 2560, 9728), (synth.Q4_K, 64, 9728, 2560),
                                         (synth.Q8_0, 16, 9728, 2560), (synth.Q4_K, 64, 2560, 9728)])
def test_gemm_accumulate_and_fp16_output(hqlib, oracle, gtype, M, N, K):
    blocks = weights(gtype, N, K, 7)
    rng = synth.Rng(77 + M)
    a = synth.activations_f16(rng, M, K)
    c0 = rng.normal(M * N).astype(np.float32).reshape(M, N)
    W = hqlib.Mat(blocks, gtype, N, K)
    ref = oracle.matmul(blocks, gtype, N, K, oracle.f16_to_f32(a), c0.copy(), True)
    say(f"gemm accumulate fp32 type={gtype} M={M} N={N} K={K} tiles={hqlib.gemm_tiles(gtype, M, N)}")
    check(hqlib.gemm_np(W, a, c_f32=True, c_init=c0), ref, gtype, "accumulate fp32")
    say(f"gemm fp16 out type={gtype} M={M}")
    got16 = hqlib.gemm_np(W, a, c_f32=False).view(np.float16).astype(np.float32)
    plain = oracle.matmul(blocks, gtype, N, K, oracle.f16_to_f32(a))
    # fp16 output: half an ulp of |y| on top of the fp32 bar
    assert np.all(np.abs(got16 - plain) <= 1e-2 + np.abs(plain) * 2.0 ** -11)
    c16 = synth.f16_bits(c0)
    say(f"gemm accumulate fp16 type={gtype} M={M}")
    acc16 = hqlib.gemm_np(W, a, c_f32=False, c_init=c16).view(np.float16).astype(np.float32)
    want = plain + c16.view(np.float16).astype(np.float32)
    assert np.all(np.abs(acc16 - want) <= 1e-2 + np.abs(want) * 2.0 ** -11)
    W.free()


def test_gemm_large_m_row_sample(hqlib, oracle):
    """M = 2048 (Q8_0) and 4096 (Q4_K), full K and N on the GPU; the oracle checks 768 sampled
    output columns (weight rows) at every M, which covers every tile position in N."""
    for gtype, M in ((synth.Q8_0, 2048), (synth.Q4_K, 4096)):
        N, K = 9728, 2560
        blocks = weights(gtype, N, K, 100 + gtype)
        a = synth.activations_f16(synth.Rng(M), M, K)
        W = hqlib.Mat(blocks, gtype, N, K)
        say(f"gemm large type={gtype} M={M} tiles={hqlib.gemm_tiles(gtype, M, N)}")
        got = hqlib.gemm_np(W, a)
        cols = np.unique(np.concatenate([np.arange(0, 256), np.arange(N - 256, N),
                                         synth.Rng(3).choice_without_replacement(N, 256)])).astype(np.int64)
        sub = np.ascontiguousarray(blocks[cols])
        ref = oracle.matmul(sub, gtype, len(cols), K, oracle.f16_to_f32(a))
        check(got[:, cols], ref, gtype, f"large M={M}")
        W.free()


def special_q4_k_weights(seed, rows, cols):
    """Q4_K weights whose super-block scales take the values the kernels treat specially: d = 0
    with dmin kept (the tile kernel then works in units of 1 and zeroes that super-block's
    quants), dmin = 0, negative d or dmin, subnormal d or dmin, and d 30x larger than its
    neighbours (so consecutive super-blocks differ in scale by up to ~2^30); plus one row with
    d = dmin = 0 everywhere (exact zeros) and one with d = 0 everywhere (min term only)."""
    rng = synth.Rng(seed)
    blk = synth.q4_k_blocks(rng, rows, cols)
    nb = rows * (cols // 256)
    v = blk.reshape(nb, 144)
    d = v[:, 0:2].copy().view(np.uint16).ravel()
    dm = v[:, 2:4].copy().view(np.uint16).ravel()
    kind = rng.bytes(nb) % 16
    sub = (rng.bytes(nb * 2).view(np.uint16) & 0x3FF) | 1
    big = synth.f16_bits(np.abs(rng.normal(nb)) * 3e-2)
    d = np.where(kind < 2, 0, d)
    dm = np.where(kind == 2, 0, dm)
    d = np.where(kind == 3, d | 0x8000, d)
    dm = np.where(kind == 4, dm | 0x8000, dm)
    d = np.where(kind == 5, sub, d)
    dm = np.where(kind == 6, sub, dm)
    d = np.where(kind == 7, big, d).astype(np.uint16)
    dm = dm.astype(np.uint16)
    spb = cols // 256
    d.reshape(rows, spb)[rows // 7] = 0
    dm.reshape(rows, spb)[rows // 7] = 0
    d.reshape(rows, spb)[2 * (rows // 7)] = 0
    v[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    v[:, 2:4] = dm.view(np.uint8).reshape(nb, 2)
    return blk


def f64_reference(oracle, blocks, gtype, N, K, a16):
    """float64 product of the oracle's (bit-exact) dequantised weights and the fp16 activations,
    and the row-wise |W| @ |a| that bounds any fp32 summation order's error."""
    a = oracle.f16_to_f32(a16).astype(np.float64)
    w = oracle.dequantize(blocks, gtype, N, K).astype(np.float64)
    return a @ w.T, np.abs(a) @ np.abs(w).T


# the loader-wave tile kernel k_gemm_q4_k_wr (M = 350, 512 at N = 9728), the full-K tile kernel
# k_gemm_q4_k_ws (M = 512 at N = 2560: each tile's K split over 4 workgroups), the mid-M kernel
# k_gemm_q4_k_rb (M = 48 at N = 9728: one workgroup per tile; M = 64 at N = 2560, K = 9728: each
# tile's K split over 6, so every part restarts its accumulator units), the narrow kernel
# k_gemm_q4_k (M = 16) and the GEMVs (M = 1); test_abi.py pins these kernel names
SPECIAL = [(9728, 512, 350), (9728, 2560, 512), (2560, 9728, 512), (9728, 2560, 48), (2560, 9728, 64),
           (9728, 2560, 16), (9728, 2560, 1), (2560, 9728, 1)]


@pytest.mark.parametrize("N,K,M", SPECIAL)
def test_gemm_special_scales(hqlib, oracle, N, K, M):
    """Q4_K GEMM/GEMV on weights with zero, negative, subnormal and widely varying super-block
    scales, at the north-star bar against the oracle; the float64 product bounds the error by
    2^-13 |W| @ |a| per output (the oracle's own fp32 error stays below 1e-6 of it)."""
    blocks = special_q4_k_weights(31 + M, N, K)
    a = synth.activations_f16(synth.Rng(400 + M), M, K)
    W = hqlib.Mat(blocks, synth.Q4_K, N, K)
    say(f"gemm special scales M={M} N={N} K={K} tiles={hqlib.gemm_tiles(synth.Q4_K, M, N)}")
    got = hqlib.gemm_np(W, a)
    W.free()
    ref = oracle.matmul(blocks, synth.Q4_K, N, K, oracle.f16_to_f32(a))
    r, m = rel_l2(got, ref), max_abs(got, ref)
    say(f"special scales: rel_l2 {r:.2e} max_abs {m:.2e} max|ref| {np.abs(ref).max():.1f}")
    assert r <= REL_L2 and m <= MAX_ABS
    r64, bound = f64_reference(oracle, blocks, synth.Q4_K, N, K, a)
    assert np.all(np.abs(got - r64) <= 2.0 ** -13 * bound)
    assert np.all(got[:, N // 7] == 0.0)


@pytest.mark.parametrize("gtype,N,K,M", [(synth.Q4_K, n, k, m) for n, k, m in SPECIAL] +
                         [(synth.Q8_0, 9728, 2560, 1), (synth.Q8_0, 9728, 2560, 128)])
def test_gemm_positive_activations(hqlib, oracle, gtype, N, K, M):
    """Non-negative activations of magnitude up to ~16 (|N(0,1)| * 4): the Q4_K min term no longer
    cancels across a sub-block, so the kernels' reassociated bias terms (the GEMV's 1024 + q
    decode, the tile kernel's bf16 hi/lo sub-block sums) carry their largest error here. Outputs
    reach ~3e4, where the oracle's own fp32 summation is off by ~5e-3, so the bar is rel-L2 <= 1e-3
    against the oracle and 2^-13 |W| @ |a| against the float64 product. The same call with the
    activations scaled by 2^6 must give the outputs scaled by 2^6 bit for bit (every step is exact
    under a power-of-two scale)."""
    blocks = weights(gtype, N, K, 100 + gtype)
    rng = synth.Rng(500 + M + N)
    a = synth.f16_bits(np.abs(rng.normal(M * K)) * 4).reshape(M, K)
    W = hqlib.Mat(blocks, gtype, N, K)
    say(f"gemm positive activations type={gtype} M={M} N={N} K={K} tiles={hqlib.gemm_tiles(gtype, M, N)}")
    got = hqlib.gemm_np(W, a)
    a64 = synth.f16_bits(oracle.f16_to_f32(a) * 64).reshape(M, K)
    say("scaled by 2^6")
    got64 = hqlib.gemm_np(W, a64)
    W.free()
    ref = oracle.matmul(blocks, gtype, N, K, oracle.f16_to_f32(a))
    r = rel_l2(got, ref)
    say(f"positive activations: rel_l2 {r:.2e} max_abs {max_abs(got, ref):.2e} max|ref| {np.abs(ref).max():.1f}")
    assert r <= REL_L2
    r64, bound = f64_reference(oracle, blocks, gtype, N, K, a)
    assert np.all(np.abs(got - r64) <= 2.0 ** -13 * bound)
    assert np.array_equal(got64, got * 64)



@pytest.mark.parametrize("gtype,M", [(synth.Q4_K, 512), (synth.Q8_0, 512), (synth.Q4_K, 64), (synth.Q8_0, 16)])
def test_gemm_k_split_repeatable(hqlib, gtype, M):
    """The K-split tile kernels (N = 2560, K = 9728: M = 512, each tile's K over 4 workgroups; the
    mid-M Q4_K kernel at M = 64 over 6) give the same bits on every call: the last part to arrive
    adds the parts in part order, and the per-tile counters return to zero after each call."""
    N, K = 2560, 9728
    blocks = weights(gtype, N, K, 31 + gtype)
    a = synth.activations_f16(synth.Rng(4242), M, K)
    W = hqlib.Mat(blocks, gtype, N, K)
    say(f"k-split repeat type={gtype} kernel={hqlib.gemm_kernel(gtype, M, N, K)}")
    first = hqlib.gemm_np(W, a)
    for _ in range(4):
        assert np.array_equal(hqlib.gemm_np(W, a), first)
    W.free()
    assert np.all(np.isfinite(first))


def test_gather_special_scales(hqlib, oracle):
    V, K, B, k = 4096, 2560, 64, 5
    blocks = special_q4_k_weights(61, V, K)
    rng = synth.Rng(62)
    H = synth.activations_f16(rng, B, K)
    ids = np.stack([rng.choice_without_replacement(V, k) for _ in range(B)]).astype(np.uint32)
    ids[0, 0], ids[1, 0] = V // 7, 2 * (V // 7)
    W = hqlib.Mat(blocks, synth.Q4_K, V, K)
    say("gather special scales")
    got = hqlib.gather_dot_np(W, H, ids)
    W.free()
    ref = oracle.gather_dot(blocks, synth.Q4_K, V, K, oracle.f16_to_f32(H), ids)
    assert rel_l2(got, ref) <= REL_L2 and max_abs(got, ref) <= MAX_ABS
    assert got[0, 0] == 0.0


def test_matmul_host_drop_in(hqlib, oracle):
    """hq_matmul_host: fp32 host x in, fp32 host y out, accumulate, as cpu_backend.c's matmul; x is
    rounded to fp16 on the device, so it matches the oracle on fp16-rounded x."""
    N, K, T = 1408, 512, 33
    blocks = weights(synth.Q8_0, N, K, 9)
    rng = synth.Rng(91)
    x = rng.normal(T * K).astype(np.float32).reshape(T, K)
    y0 = rng.normal(T * N).astype(np.float32).reshape(T, N)
    W = hqlib.Mat(blocks, synth.Q8_0, N, K)
    say("matmul_host")
    got = hqlib.matmul_host(W, x, y0.copy(), True)
    xr = x.astype(np.float16).astype(np.float32)
    ref = oracle.matmul(blocks, synth.Q8_0, N, K, xr, y0.copy(), True)
    check(got, ref, synth.Q8_0, "matmul_host")
    W.free()


# ------------------------------------------------------------------ option-row gather (config 5)
@pytest.mark.parametrize("gtype,V,k", [(synth.Q8_0, 32000, 2), (synth.Q8_0, 32000, 8), (synth.Q8_0, 32000, 32),
                                       (synth.Q4_K, 4096, 5)])
def test_gather_parity(hqlib, oracle, gtype, V, k):
    K, B = 2560, 256
    blocks = weights(gtype, V, K, 200 + gtype)
    rng = synth.Rng(300 + k)
    H = synth.activations_f16(rng, B, K)
    ids = np.stack([rng.choice_without_replacement(V, k) for _ in range(B)]).astype(np.uint32)
    W = hqlib.Mat(blocks, gtype, V, K)
    say(f"gather type={gtype} V={V} B={B} k={k}")
    got = hqlib.gather_dot_np(W, H, ids)
    ref = oracle.gather_dot(blocks, gtype, V, K, oracle.f16_to_f32(H), ids)
    check(got, ref, gtype, f"gather k={k}")
    say("gather with device ids")
    got2 = hqlib.gather_dot_np(W, H, ids, device_ids=True)
    assert np.array_equal(got, got2)
    W.free()


def test_gather_bad_ids(hqlib):
    blocks = synth.q8_0_blocks(synth.Rng(4), 64, 256)
    W = hqlib.Mat(blocks, synth.Q8_0, 64, 256)
    H = synth.activations_f16(synth.Rng(5), 2, 256)
    say("gather bad ids")
    with pytest.raises(hqlib.HQError, match="out of range"):
        hqlib.gather_dot_np(W, H, np.array([[1, 64]], np.uint32))
    got = hqlib.gather_dot_np(W, H, np.array([[1, 64], [2**32 - 1, 3]], np.uint32), device_ids=True)
    assert np.isnan(got[0, 1]) and np.isnan(got[1, 0]) and np.isfinite(got[0, 0]) and np.isfinite(got[1, 1])
    W.free()


def test_gather_equals_gemm_columns(hqlib):
    """Size-independent property at the full config-5 vocabulary: the gather of ids equals the
    full-vocabulary logits at those ids (as SPEC.md defines the readout), here GEMM vs gather."""
    V, K, B, k = 151936, 2560, 16, 32
    blocks = synth.q8_0_blocks(synth.Rng(55), V, K)
    W = hqlib.Mat(blocks, synth.Q8_0, V, K)
    rng = synth.Rng(56)
    H = synth.activations_f16(rng, B, K)
    ids = np.stack([rng.choice_without_replacement(V, k) for _ in range(B)]).astype(np.uint32)
    say("gather vs full-vocab gemm, V=151936")
    full = hqlib.gemm_np(W, H)
    got = hqlib.gather_dot_np(W, H, ids)
    sel = np.take_along_axis(full, ids.astype(np.int64), axis=1)
    assert max_abs(got, sel) <= 1e-2 and rel_l2(got, sel) <= 1e-3
    W.free()


def test_errors_are_reported(hqlib):
    blocks = synth.q8_0_blocks(synth.Rng(4), 64, 256)
    W = hqlib.Mat(blocks, synth.Q8_0, 64, 256)
    with pytest.raises(hqlib.HQError, match="rows"):
        hqlib.dequant(W, 60, 10)
    with pytest.raises(hqlib.HQError, match="M = 0"):
        hqlib.gemm(W, hqlib.DevBuf(1024), 0, hqlib.DevBuf(1024))
    W.free()
