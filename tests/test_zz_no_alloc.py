"""hq_gemm_noalloc (the GEMM entry point that allocates nothing: its workspace is the library's
preallocated per-GPU scratch array) gives the same bits as hq_gemm, call after call, and refuses a
launch whose workspace does not fit the scratch before queuing anything."""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu]", *a, flush=True)


# each case uses the scratch differently: a K-split tile GEMM (partial tiles, counters, sums), then a
# smaller mid-M K split (partials, counters), a Stream-K GEMM (64 MiB of partial tiles, counters,
# sums), then a smaller mid-M GEMM (sums only) and a tile GEMM with no workspace at all; then the
# k-quant tile kernel with K split over 4 (Q6_K), the Q5_K tile kernel (sums only) and the Q8_0 tile
# kernel with K split over 2 workgroups (partials, counters)
CASES = [(synth.Q4_K, 512, 2560, 9728), (synth.Q8_0, 16, 2560, 9728), (synth.Q4_K, 4096, 9728, 2560),
         (synth.Q4_K, 64, 9728, 2560), (synth.Q8_0, 512, 9728, 2560), (synth.Q6_K, 512, 2560, 9728),
         (synth.Q5_K, 512, 9728, 2560), (synth.Q8_0, 96, 9728, 2560)]


def test_noalloc_matches_hq_gemm_call_after_call(hqlib):
    for gtype, M, N, K in CASES:
        pb, cb, sb, fits = hqlib.gemm_workspace_bytes(gtype, M, N, K)
        say(f"noalloc type={gtype} M={M} N={N} K={K} kernel={hqlib.gemm_kernel(gtype, M, N, K)} "
            f"workspace partials={pb} counters={cb} sums={sb}")
        assert fits
        blocks = synth.random_blocks(gtype, synth.Rng(900 + M + gtype), N, K)
        W = hqlib.Mat(blocks, gtype, N, K)
        A = hqlib.DevBuf.from_array(synth.activations_f16(synth.Rng(901 + M), M, K))
        C1, C2 = hqlib.DevBuf(M * N * 4), hqlib.DevBuf(M * N * 4)
        hqlib.gemm(W, A, M, C1, True, False)
        hqlib.gemm_noalloc(W, A, M, C2, True, False)
        hqlib.synchronize()
        want = C1.download((M, N), np.float32)
        assert np.array_equal(C2.download((M, N), np.float32), want)
        # fp16 output with accumulate: the same bits again
        C1.upload(np.full((M, N), 0x3c00, np.uint16))
        C2.upload(np.full((M, N), 0x3c00, np.uint16))
        hqlib.gemm(W, A, M, C1, False, True)
        hqlib.gemm_noalloc(W, A, M, C2, False, True)
        hqlib.synchronize()
        assert np.array_equal(C2.download((M, N), np.uint16), C1.download((M, N), np.uint16))
        A.free(), C1.free(), C2.free(), W.free()


def test_noalloc_refuses_oversize_workspace(hqlib):
    # the large-M tile kernel needs only the activation sub-block sums: 151 MB of them here
    gtype, M, N, K = synth.Q4_K, 131072, 256, 9216
    assert not hqlib.gemm_workspace_bytes(gtype, M, N, K)[3]
    blocks = synth.random_blocks(gtype, synth.Rng(5), N, K)
    W = hqlib.Mat(blocks, gtype, N, K)
    A, C = hqlib.DevBuf(M * K * 2), hqlib.DevBuf(M * N * 4)
    say(f"noalloc refusal M={M} N={N} K={K}")
    with pytest.raises(hqlib.HQError, match="use hq_gemm"):
        hqlib.gemm_noalloc(W, A, M, C)
    hqlib.synchronize()
    A.free(), C.free(), W.free()
