"""GPU parity at the BASELINE configs' full sizes, through the C ABI (libhq.so), against the CPU
oracle on sampled outputs.

  config 4  the hybrid 4B decoder's five Q4_K projection shapes at M = 16384 (64 sequences of 256
            tokens): N x K = 4096 x 2560, 1024 x 2560, 9216 x 2560, 2560 x 4096, 2560 x 9216;
  config 3  the Q4_K down projection 2560 x 9728 at M = 4096;
  config 5  the 151936 x 2560 Q8_0 lm_head, 256 states x k in {2, 8, 32} option ids;
  plus GEMMs whose activations exceed 4 GiB (the library cuts M into launches of < 2^32 bytes of A)
  and K-split GEMMs running concurrently on two streams (each stream has its own workspace).

Sampling: the GPU computes the whole M x N output; the oracle computes the outputs of 8 rows of
every 128-row tile and of 24 columns of every 256-column block (plus the first and last 64
columns), so every output tile of every kernel (tiles are at most 128 x 256) is checked. Bars as in
test_gpu_parity.py: fp32 outputs, rel-L2 <= 1e-3 and max-abs <= 1e-2 (Q4_K also max-abs <= 2e-3).
"""
import numpy as np
import pytest

import synth
from conftest import max_abs, rel_l2

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS, Q4K_MAX_ABS = 1e-3, 1e-2, 2e-3


def say(*a):
    print("[gpu]", *a, flush=True)


def check(got, ref, gtype, what):
    r, m = rel_l2(got, ref), max_abs(got, ref)
    say(f"{what}: rel_l2 {r:.2e} max_abs {m:.2e}")
    assert r <= REL_L2 and m <= MAX_ABS, what
    if gtype == synth.Q4_K:
        assert m <= Q4K_MAX_ABS, what


def big_activations(seed, M, K, base_rows=2048):
    """fp16 N(0,1) activations [M, K] built from `base_rows` random rows: row r is base row
    r % base_rows, circularly shifted by 7 * (r // base_rows) columns and negated for odd blocks, so
    every row differs from every other (a row-index mistake in any kernel changes the output) while
    only base_rows * K normals are drawn."""
    base = synth.activations_f16(synth.Rng(seed), min(M, base_rows), K)
    out = np.empty((M, K), np.uint16)
    for b0 in range(0, M, base_rows):
        blk = b0 // base_rows
        n = min(base_rows, M - b0)
        rows = np.roll(base[:n], 7 * blk, axis=1)
        out[b0:b0 + n] = rows ^ np.uint16(0x8000) if blk % 2 else rows
    return out


def sample_rows(M, per_tile=8, tile=128, seed=1):
    rng = synth.Rng(seed)
    rows = [t + (rng.draw(per_tile) % np.uint64(min(tile, M - t))).astype(np.int64) for t in range(0, M, tile)]
    return np.unique(np.concatenate(rows + [np.array([0, M - 1])]))


def sample_cols(N, per_block=24, block=256, seed=2):
    rng = synth.Rng(seed)
    cols = [b + (rng.draw(per_block) % np.uint64(min(block, N - b))).astype(np.int64) for b in range(0, N, block)]
    return np.unique(np.concatenate(cols + [np.arange(0, min(64, N)), np.arange(max(0, N - 64), N)]))


def sampled_check(hqlib, oracle, gtype, N, K, M, seed, what):
    blocks = synth.random_blocks(gtype, synth.Rng(seed), N, K)
    a = big_activations(seed + 1, M, K)
    W = hqlib.Mat(blocks, gtype, N, K)
    say(f"{what}: type={gtype} M={M} N={N} K={K} kernel={hqlib.gemm_kernel(gtype, M, N, K)}")
    got = hqlib.gemm_np(W, a)
    W.free()
    rows, cols = sample_rows(M), sample_cols(N)
    ref = oracle.matmul(np.ascontiguousarray(blocks[cols]), gtype, len(cols), K, oracle.f16_to_f32(a[rows]))
    check(got[np.ix_(rows, cols)], ref, gtype, f"{what} ({len(rows)} rows x {len(cols)} columns)")
    assert np.all(np.isfinite(got))


# config 4: the distinct Q4_K projection shapes of the 32-layer hybrid at M = 16384, in
# BASELINE's literal reading and in the reference's layer_weights() reading (src/shapes.c:12-39),
# which adds the 8192-wide q_proj / in_proj_qkv and the 32-row b / a projections
CONFIG4 = sorted({(n, k) for reading in ("baseline", "layer_weights")
                  for layer in synth.hybrid_4b_projections(reading) for _, n, k in layer})


@pytest.mark.parametrize("N,K", CONFIG4)
def test_config4_projection_m16384(hqlib, oracle, N, K):
    sampled_check(hqlib, oracle, synth.Q4_K, N, K, 16384, 4000 + N + K, "config 4")


def test_config3_down_m4096(hqlib, oracle):
    sampled_check(hqlib, oracle, synth.Q4_K, 2560, 9728, 4096, 3003, "config 3 down")


@pytest.fixture(scope="module")
def lm_head(hqlib):
    V, K = 151936, 2560
    blocks = synth.q8_0_blocks(synth.Rng(5151), V, K)
    say(f"config 5 lm_head {V}x{K} Q8_0 ({blocks.nbytes / 1e6:.0f} MB)")
    W = hqlib.Mat(blocks, synth.Q8_0, V, K)
    yield blocks, W
    W.free()


@pytest.mark.parametrize("k", [2, 8, 32])
def test_config5_option_readout(hqlib, oracle, lm_head, k):
    """256 states x k option ids against the oracle's gather (which equals the full-vocab logits at
    those ids: it runs the reference matmul's dot on the decoded rows)."""
    blocks, W = lm_head
    V, K, B = W.rows, W.cols, 256
    rng = synth.Rng(600 + k)
    H = synth.activations_f16(rng, B, K)
    ids = np.stack([rng.choice_without_replacement(V, k) for _ in range(B)]).astype(np.uint32)
    say(f"config 5 readout V={V} B={B} k={k}")
    got = hqlib.gather_dot_np(W, H, ids)
    ref = oracle.gather_dot(blocks, synth.Q8_0, V, K, oracle.f16_to_f32(H), ids)
    check(got, ref, synth.Q8_0, f"config 5 k={k}")


@pytest.mark.parametrize("gtype", [synth.Q4_K, synth.Q8_0])
def test_gemm_activations_over_4gib(hqlib, oracle, gtype):
    """M = 838956 rows of K = 2560 (4.2955e9 bytes of fp16 A, above 2^32): hq_gemm cuts M into
    launches of 838656 rows (the largest multiple of 128 with (rows + 128) * K < 2^31) and 300 rows. A is zero
    except for random rows at the start, on both sides of the cut and at the end; those rows'
    outputs match the oracle, and the zero rows give exact zeros."""
    N, K, M = 64, 2560, 838956
    cut = 838656
    blocks = synth.random_blocks(gtype, synth.Rng(77 + gtype), N, K)
    W = hqlib.Mat(blocks, gtype, N, K)
    A = hqlib.DevBuf(M * K * 2)
    C = hqlib.DevBuf(M * N * 4)
    A.zero()
    picks = [(0, 40), (cut - 40, 80), (M - 40, 40)]
    rng = synth.Rng(78)
    rows, vals = [], []
    for r0, n in picks:
        a = synth.activations_f16(rng, n, K)
        A.upload(a, offset=r0 * K * 2)
        rows.append(np.arange(r0, r0 + n))
        vals.append(a)
    say(f"gemm over 4 GiB of activations: type={gtype} M={M} N={N} K={K}")
    hqlib.gemm(W, A, M, C, True, False)
    hqlib.synchronize()
    got = np.concatenate([C.download((n, N), np.float32, offset=r0 * N * 4) for r0, n in picks])
    zero_rows = [1000, cut - 100, cut + 100, M - 100]
    zeros = np.concatenate([C.download((1, N), np.float32, offset=r * N * 4) for r in zero_rows])
    A.free(), C.free(), W.free()
    ref = oracle.matmul(blocks, gtype, N, K, oracle.f16_to_f32(np.concatenate(vals)))
    check(got, ref, gtype, "over 4 GiB")
    assert np.all(zeros == 0.0)


def test_two_streams_have_separate_workspaces(hqlib):
    """Two K-split GEMMs (each keeps partial tiles and per-tile counters in its workspace) issued
    alternately on two created streams with no synchronisation between them give the same bits as
    the same GEMMs run alone."""
    N, K = 2560, 9728
    jobs = []
    for gtype, M, seed in ((synth.Q8_0, 16, 11), (synth.Q4_K, 64, 12)):
        blocks = synth.random_blocks(gtype, synth.Rng(seed), N, K)
        W = hqlib.Mat(blocks, gtype, N, K)
        A = hqlib.DevBuf.from_array(synth.activations_f16(synth.Rng(seed + 1), M, K))
        say(f"stream job type={gtype} M={M} kernel={hqlib.gemm_kernel(gtype, M, N, K)}")
        alone = hqlib.gemm_np(W, A.download((M, K), np.uint16))
        jobs.append((W, A, M, alone))
    streams = [hqlib.Stream(), hqlib.Stream()]
    outs = [[hqlib.DevBuf(M * N * 4) for _ in range(4)] for (_, _, M, _) in jobs]
    say("two streams, 4 launches each, no synchronisation between them")
    for i in range(4):
        for s, (W, A, M, _) in enumerate(jobs):
            hqlib.gemm(W, A, M, outs[s][i], True, False, streams[s].ptr)
    for st in streams:
        st.sync()
    for s, (W, A, M, alone) in enumerate(jobs):
        for i in range(4):
            assert np.array_equal(outs[s][i].download((M, N), np.float32), alone), (s, i)
    for st in streams:
        st.destroy()
    for s, (W, A, M, _) in enumerate(jobs):
        W.free(), A.free()
        for b in outs[s]:
            b.free()
