"""Benchmark of the gfx950 quantized matmul path (one GPU).

Headline workload (the BASELINE north-star target): Q4_K GEMM, M = 512, K = 2560, N = 9728
(config 3, up/gate shape), fp16 activations, fp32 accumulation, fp16 output. A "step" is one GEMM
launch over one batch; weights rotate over enough distinct device copies (> 512 MB) that every
launch streams its weights from HBM, not from the 256 MB Infinity Cache. The timed steps are HIP-graph
replays of exactly `steps` launches, timed with HIP events on the launch stream, after `warmup`
eager launches, 0.3 s of untimed launches and one untimed replay: five such replays, each graph
continuing the weight rotation, a HIP event between replays; `ms_per_step` and `value` come from the
median of the five per-launch times (`us_first_replay` is the first replay alone). `us_median` and
the roofline's `kernel_us` are medians over five replays of 20-launch graphs of whole calls and of
the main kernel alone; the three kinds of replay are interleaved (one of each per round), so clock
drift during the measurement moves them alike. The headline is also timed with fp32 C
(`headline_fp32_c`), the output mode the parity bar covers and the reference's output type.

Also reported (key "sweep"): the config 2 / 3 M sweeps and the config 5 option readout, each as
achieved TFLOP/s and GB/s of algorithmic bytes (W blocks once + A + C) and their roofline fractions,
and config 4 (the 4B-class hybrid's 32-layer projection sequence at M = 16384, BASELINE's literal
widths: each distinct projection shape timed, weighted by its count in the sequence).

roofline: the headline GEMM's main kernel (k_gemm_q4_k_wr160: full-K 128 x 160 tiles), timed alone
(hq_time_gemm_kernel; a pre-pass, where the plan has one, runs once outside the timed graphs) with HIP
events on its stream, median of five replays of 20 launches; `traffic` is its HBM bytes per launch from the committed rocprofv3
FETCH_SIZE / WRITE_SIZE summary (calibrated against a device copy of known size), null when that
summary was taken for a different kernel.

cpu_baseline: the CPU oracle (a restatement of the reference's cpu_backend.c matmul, compiled with
the reference's flags, OpenMP with OMP_PROC_BIND=close and the box's OMP_NUM_THREADS) on the
headline GEMM and on the three M = 1 GEMV shapes of the sweep, timed on this host's cores (median
of 3 after 1 warm-up); `cores` is the physical cores of the process's CPU set.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "hilbert-pruned-8b_amd"), os.path.join(ROOT, "oracle")]

import numpy as np  # noqa: E402

METRIC = "Q4_K/Q8_0 GEMM TFLOP/s @M=512 and GEMV GB/s @M=1; % of MI355X roofline"
PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA
PEAK_GBS = 8000.0     # MI355X HBM3E
ROTATE_BYTES = 560 << 20


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def gemm_bytes(gtype, M, N, K, c_bytes):
    import synth
    return N * synth.row_bytes(gtype, K) + M * K * 2 + M * N * c_bytes


def read_traffic(name, kernel):
    """HBM bytes per launch of the headline kernel from the committed rocprofv3 counter summary
    (line `traffic_bytes_per_launch <workload> <kernel> <bytes>`), or None when the summary is for
    another kernel."""
    path = os.path.join(ROOT, "profiles", "q4k_gemm_m512_k2560_n9728_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        f = line.split()
        if len(f) == 4 and f[0] == "traffic_bytes_per_launch" and f[1] == name and f[2] == kernel:
            try:
                return float(f[3])
            except ValueError:
                return None
    return None


MEDIAN_ITERS, MEDIAN_REPS = 20, 5  # the median figures: 5 graph replays of 20 launches
SETTLE_S = 0.2  # untimed GPU work before a timed measurement that has no warm-up of its own


def main_kernel_name(hq, gtype, M, N, K):
    """Name of the kernel hq_gemm dispatches for this shape (the main kernel where a pre-pass runs
    first), as rocprofv3 lists it."""
    return hq.gemm_kernel(gtype, M, N, K)


def bench_gemm(hq, synth, gtype, N, K, M, c_f32, steps, warmup, stream, eager_warmup=True, kernel_time=False,
               rotate=True, settle_s=0.0, reps=1):
    rb = synth.row_bytes(gtype, K)
    blocks = synth.random_blocks(gtype, synth.Rng(4242 + gtype + N), N, K)
    copies = max(2, -(-ROTATE_BYTES // (N * rb))) if rotate else 2
    mats = [hq.Mat(blocks, gtype, N, K) for _ in range(copies)]
    A = hq.DevBuf.from_array(synth.activations_f16(synth.Rng(99 + M), M, K))
    C = hq.DevBuf(M * N * (4 if c_f32 else 2))
    if eager_warmup:
        for i in range(warmup):
            hq.gemm(mats[i % copies], A, M, C, c_f32, False, stream.ptr)
        stream.sync()
        # untimed: keep the GPU busy for settle_s so its clocks are at their loaded level
        t_end, i = time.perf_counter() + settle_s, 0
        while time.perf_counter() < t_end:
            for _ in range(20):
                hq.gemm(mats[i % copies], A, M, C, c_f32, False, stream.ptr)
                i += 1
            stream.sync()
    t0 = time.perf_counter()
    ms_first = ms_med = ms_kernel = None
    if kernel_time and M > 1:
        # whole calls and the main kernel alone, replays interleaved (each rep: one graph of `steps`
        # calls, one of MEDIAN_ITERS calls, one of MEDIAN_ITERS main-kernel launches), so that clock
        # drift during the measurement moves all three alike; medians over the reps
        calls, meds, kerns = [], [], []
        for _ in range(max(reps, 1)):
            calls.append(hq.time_gemm(mats, A, M, C, c_f32, steps, 1, stream))
            meds.append(hq.time_gemm(mats, A, M, C, c_f32, MEDIAN_ITERS, 1, stream))
            kerns.append(hq.time_gemm_kernel(mats, A, M, C, c_f32, MEDIAN_ITERS, 1, stream))
        ms, ms_first = statistics.median(calls), calls[0]
        ms_med, ms_kernel = statistics.median(meds), statistics.median(kerns)
    else:
        ms = hq.time_gemm(mats, A, M, C, c_f32, steps, reps, stream)
    wall = time.perf_counter() - t0
    for m in mats:
        m.free()
    A.free(), C.free()
    flop = 2.0 * M * N * K
    nbytes = gemm_bytes(gtype, M, N, K, 4 if c_f32 else 2)
    r = dict(type=synth.TYPE_NAMES[gtype].lower(), M=M, N=N, K=K, us=ms * 1e3,
             tflops=flop / (ms * 1e-3) / 1e12, gbs=nbytes / (ms * 1e-3) / 1e9, copies=copies, wall_s=wall)
    if ms_med is not None:
        r["us_median"] = ms_med * 1e3
    if ms_first is not None:
        r["us_first_replay"] = ms_first * 1e3
    if ms_kernel is not None:
        r["kernel_us"] = ms_kernel * 1e3
        r["kernel_tflops"] = flop / (ms_kernel * 1e-3) / 1e12
    return r


def bench_config4(hq, synth, stream, M=16384, reading="baseline"):
    """Config 4: the hybrid 4B projection sequence (32 layers) at M = 16384; each distinct shape timed
    as the median of MEDIAN_REPS graph replays of 3 launches after SETTLE_S of untimed calls, total =
    sum over the sequence. reading: BASELINE's literal widths or the reference's layer_weights() list
    (synth.hybrid_4b_projections)."""
    counts = {}
    for layer in synth.hybrid_4b_projections(reading):
        for _, n, k in layer:
            counts[(n, k)] = counts.get((n, k), 0) + 1
    total_us, flop, shapes = 0.0, 0.0, []
    for (n, k), cnt in sorted(counts.items()):
        r = bench_gemm(hq, synth, synth.Q4_K, n, k, M, False, 3, 1, stream, rotate=False, settle_s=SETTLE_S,
                       reps=MEDIAN_REPS)
        total_us += cnt * r["us"]
        flop += cnt * 2.0 * M * n * k
        shapes.append({"N": n, "K": k, "count": cnt, "us": round(r["us"], 2), "tflops": round(r["tflops"], 1),
                       "kernel": hq.gemm_kernel(synth.Q4_K, M, n, k)})
    return dict(type="config4_hybrid_4b_q4_k", reading=reading, M=M, projections=sum(counts.values()),
                total_ms=round(total_us / 1e3, 3),
                tflop=round(flop / 1e12, 2), tflops=round(flop / (total_us * 1e-6) / 1e12, 1),
                frac=round(flop / (total_us * 1e-6) / 1e12 / PEAK_TFLOPS, 4), bound="mfma", shapes=shapes)


def bench_gather(hq, synth, k, stream, reps=3):
    V, K, B = 151936, 2560, 256
    blocks = synth.q8_0_blocks(synth.Rng(5151), V, K)
    W = hq.Mat(blocks, synth.Q8_0, V, K)
    del blocks
    rng = synth.Rng(600 + k)
    n_sets = max(1, V // (B * k))
    perm = np.argsort(rng.uniform(V))[: n_sets * B * k].astype(np.uint32)  # distinct rows across sets
    ids = hq.DevBuf.from_array(perm.reshape(n_sets, B, k))
    H = hq.DevBuf.from_array(synth.activations_f16(rng, B, K))
    out = hq.DevBuf(B * k * 4)
    iters = max(n_sets, 32)
    ms = hq.time_gather([W], H, ids, n_sets, B, k, out, iters, reps, stream)
    W.free(), ids.free(), H.free(), out.free()
    nbytes = B * k * synth.row_bytes(synth.Q8_0, K) + B * K * 2 + B * k * 4
    return dict(type="q8_0_gather", B=B, k=k, V=V, K=K, us=ms * 1e3, gbs=nbytes / (ms * 1e-3) / 1e9,
                tflops=2.0 * B * k * K / (ms * 1e-3) / 1e12, id_sets=n_sets)


def bench_swiglu(hq, synth, gtype, stream, M=512, I=9728, K=2560):
    """The SwiGLU FFN input silu(A gate^T) * (A up^T) of config 3's up/gate shape as one pair GEMM
    (hq_gemm_swiglu; the epilogue in the tile kernel) against the unfused sequence's two GEMMs alone
    (hq_gemm on gate and on up, fp16 outputs; the reference adds a k_swiglu pass on top); both as
    the median per-launch time of HIP-graph replays (MEDIAN_REPS graphs of MEDIAN_ITERS calls)."""
    gb = synth.random_blocks(gtype, synth.Rng(4242 + gtype + I), I, K)
    rb = synth.row_bytes(gtype, K)
    copies = max(2, -(-ROTATE_BYTES // (2 * I * rb)))
    pairs = [hq.PairMat(gb, gb, gtype, I, K) for _ in range(copies)]
    A = hq.DevBuf.from_array(synth.activations_f16(synth.Rng(99 + M), M, K))
    out = hq.DevBuf(M * I * 2)

    def settled(run):  # untimed replays for SETTLE_S first, so the clocks are at their loaded level
        t_end = time.perf_counter() + SETTLE_S
        while time.perf_counter() < t_end:
            run(1)
        return run(MEDIAN_REPS)

    ms = settled(lambda reps: hq.time_gemm_swiglu(pairs, A, M, out, MEDIAN_ITERS, reps, stream))
    for p in pairs:
        p.free()
    mats = [hq.Mat(gb, gtype, I, K) for _ in range(2 * copies)]
    C = hq.DevBuf(M * I * 2)
    ms2 = settled(lambda reps: hq.time_gemm(mats, A, M, C, False, MEDIAN_ITERS, reps, stream)) * 2
    for m in mats:
        m.free()
    A.free(), out.free(), C.free()
    flop = 2.0 * 2 * M * I * K
    r = dict(type=synth.TYPE_NAMES[gtype].lower() + "_gate_up_swiglu", M=M, I=I, K=K,
             us=round(ms * 1e3, 2), tflops=round(flop / (ms * 1e-3) / 1e12, 1),
             unfused_two_gemms_us=round(ms2 * 1e3, 2), copies=copies)
    if M == 1:  # HBM-bound: bytes of both matrices once, the activation row and the fp16 output
        nbytes = 2 * I * rb + K * 2 + I * 2
        r["gbs"], r["frac"], r["bound"] = round(nbytes / (ms * 1e-3) / 1e9, 1), round(nbytes / (ms * 1e-3) / 1e9 / PEAK_GBS, 4), "hbm"
    return r


def bench_prefill(hq, synth, T=2048, reps=5):
    """Config 1 (the tiny Llama, Q8_0) through the backend_t vtable (hip_backend_create), as the
    reference's selftest times it (src/cuda_backend.cu:1447-1457): a T-token prefill with two readout
    ids, median of `reps` timed passes after one warm-up (each pass resets the position; forward is
    synchronous), and one-token decode steps after a 128-token prompt. Every projection runs through
    hq_gemm / hq_gemm_swiglu; host wall-clock per forward call."""
    view = hq.RefModelView(synth.tiny_llama(1))
    be = hq.HipBackend(view, T)
    tokens, ids = synth.tiny_llama_prompt(2, T=T)
    ids2 = ids[:2]
    be.forward(tokens, ids2)
    times = []
    for _ in range(reps):
        be.reset()
        t0 = time.perf_counter()
        be.forward(tokens, ids2)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    be.reset()
    be.forward(tokens[:128])
    steps = []
    for i in range(32):
        t0 = time.perf_counter()
        be.forward(tokens[128 + i:129 + i], ids2)
        steps.append(time.perf_counter() - t0)
    be.destroy()
    ts = statistics.median(steps)
    return dict(type="config1_tiny_llama_vtable", T=T, prefill_ms=round(t * 1e3, 3), prefill_tokens_s=round(T / t, 1),
                decode_step_ms=round(ts * 1e3, 4), decode_tokens_s=round(1.0 / ts, 1),
                timing=f"prefill: median of {reps} after a warm-up; decode: median of 32 steps after 128 tokens")


def bench_read_floor(hq, synth, stream, iters=20):
    """The floor of one HBM-bound dispatch: a pure streaming read (hq_time_read) of the GEMVs' weight
    bytes (Q4_K 9728 x 2560: 14,008,320 B; Q8_0: 26,460,160 B), over rotated buffers (> 512 MB in all,
    as the GEMV timings), for several grid sizes; median of MEDIAN_REPS graph replays."""
    out = []
    for nbytes in (14008320, 26460160):
        copies = max(2, -(-ROTATE_BYTES // nbytes))
        bufs = [hq.DevBuf(nbytes) for _ in range(copies)]
        for grid in (1024, 2048, 4096):
            ms = hq.time_read(bufs, nbytes, grid, iters, MEDIAN_REPS, stream)
            out.append(dict(type="stream_read", bytes=nbytes, grid=grid, us=round(ms * 1e3, 3),
                            gbs=round(nbytes / (ms * 1e-3) / 1e9, 1), frac=round(nbytes / (ms * 1e-3) / 1e9 / PEAK_GBS, 4)))
        for b in bufs:
            b.free()
    return out


def bench_upload(hq, synth, reps=3):
    """hq_mat_upload of the config-5 lm_head (151936 x 2560 Q8_0, 413 MB of GGUF blocks) from host
    memory: rows through the pinned staging buffers, asynchronous copies, device-side plane repack.
    GB/s of GGUF bytes, median of `reps` after one warm-up."""
    V, K = 151936, 2560
    blocks = synth.q8_0_blocks(synth.Rng(5151), V, K)
    times = []
    for i in range(reps + 1):
        t0 = time.perf_counter()
        W = hq.Mat(blocks, synth.Q8_0, V, K)
        dt = time.perf_counter() - t0
        W.free()
        if i:
            times.append(dt)
    t = statistics.median(times)
    return dict(type="upload_q8_0", rows=V, cols=K, bytes=int(blocks.nbytes), ms=round(t * 1e3, 2),
                gbs=round(blocks.nbytes / t / 1e9, 2))


def cpu_topology():
    """(physical cores, logical CPUs) of the CPUs this process may run on, from /proc/cpuinfo's
    (physical id, core id) per processor; the physical count is None where the host does not
    expose distinct core ids."""
    allowed = os.sched_getaffinity(0)
    seen, proc, phys, core = set(), None, None, None
    try:
        for line in list(open("/proc/cpuinfo")) + [""]:
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "processor":
                proc = int(v)
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
            elif not k:
                if proc is not None and proc in allowed and core is not None:
                    seen.add((phys, core))
                proc, phys, core = None, None, None
    except OSError:
        pass
    n = len(seen)
    return (n if n > 1 or len(allowed) == 1 else None), len(allowed)


def cpu_time(O, blocks, gtype, N, K, x, reps=3):
    """Median of `reps` timings after one warm-up of the oracle matmul (seconds)."""
    y = np.zeros((x.shape[0], N), np.float32)
    O.matmul(blocks, gtype, N, K, x, y)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        O.matmul(blocks, gtype, N, K, x, y)
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_baseline(synth, gtype, N, K, M):
    phys, logical = cpu_topology()  # before OpenMP binds this thread to one CPU
    os.environ.setdefault("OMP_PROC_BIND", "close")  # read when the oracle's OpenMP runtime loads
    import oracle
    O = oracle.Oracle()
    blocks = synth.random_blocks(gtype, synth.Rng(4242 + gtype + N), N, K)
    x = O.f16_to_f32(synth.activations_f16(synth.Rng(99 + M), M, K))
    t = cpu_time(O, blocks, gtype, N, K, x)
    gemv = []
    for g, n, k in [(synth.Q8_0, 9728, 2560), (synth.Q4_K, 9728, 2560), (synth.Q4_K, 2560, 9728)]:
        b = synth.random_blocks(g, synth.Rng(4242 + g + n), n, k)
        x1 = O.f16_to_f32(synth.activations_f16(synth.Rng(100), 1, k))
        t1 = cpu_time(O, b, g, n, k, x1)
        gemv.append(dict(type="q8_0" if g == synth.Q8_0 else "q4_k", M=1, N=n, K=k, us=round(t1 * 1e6, 1),
                         gbs=round(gemm_bytes(g, 1, n, k, 4) / t1 / 1e9, 3)))
    threads = int(os.environ.get("OMP_NUM_THREADS") or logical)
    cores = min(threads, phys) if phys else threads
    return dict(value=round(2.0 * M * N * K / t / 1e12, 6), unit="TFLOP/s", cores=cores, kind="port",
                threads=threads, omp_proc_bind=os.environ.get("OMP_PROC_BIND"), cpu=cpu_model(),
                sample=f"full headline GEMM (Q4_K M={M} N={N} K={K}), oracle restatement of cpu_backend.c "
                       f"matmul (-O2 -std=c11 -fopenmp), median of 3 after 1 warm-up: {t:.3f} s; "
                       f"{threads} OpenMP threads (OMP_PROC_BIND={os.environ.get('OMP_PROC_BIND')}); the "
                       f"process may run on {logical} logical CPUs, "
                       + (f"{phys} physical cores" if phys else "physical cores not exposed by the host")
                       + f"; CPU {cpu_model()}",
                gemv=gemv)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run 20 device-to-device copies of BYTES bytes (the known-size kernel the "
                         "FETCH_SIZE / WRITE_SIZE counters are scaled by) and exit")
    ap.add_argument("--config4-only", action="store_true",
                    help="only time config 4 (both readings of its shape list) and exit")
    ap.add_argument("--swiglu-only", action="store_true",
                    help="only time the fused gate/up+SwiGLU pair GEMM against two GEMMs and exit")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only time config 1's prefill and decode steps through the backend vtable and exit")
    ap.add_argument("--upload-only", action="store_true",
                    help="only time the upload of the 413 MB config-5 head and exit")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only time the three M = 1 GEMV shapes of the sweep and the streaming-read floor of "
                         "their byte counts (for profiling) and exit")
    ap.add_argument("--gather-only", action="store_true",
                    help="only time the config-5 option readout at k = 2, 8, 32 (for profiling) and exit")
    ap.add_argument("--shape", default="", metavar="TYPE:M:N:K[,TYPE:M:N:K...]",
                    help="only time these GEMM shapes (TYPE q8_0, q2_k .. q6_k; for profiling) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (--gpus {args.gpus} requested); the quantized matmul "
              "path has no multi-GPU mode here (see DESIGN.md, 'How the path would shard').", file=sys.stderr)
        sys.exit(2)
    import hq
    import synth
    hq.load()
    hq.device_init(0)
    if args.calibrate_copy:
        n = args.calibrate_copy
        src, dst = hq.DevBuf(n), hq.DevBuf(n)
        hq._check(hq.load().hq_memset(src.ptr, 1, n, None))
        for _ in range(20):
            hq._check(hq.load().hq_memcpy_d2d(dst.ptr, src.ptr, n, None))
        hq.synchronize()
        log(f"calibration: 20 device copies of {n} bytes")
        return
    name, arch = hq.device_name(0)
    log("device", name, arch)
    stream = hq.Stream()
    if args.shape:
        for shape in args.shape.split(","):
            t, m, n, k = shape.split(":")
            g = {v.lower(): k for k, v in synth.TYPE_NAMES.items()}[t]
            r = bench_gemm(hq, synth, g, int(n), int(k), int(m), False, args.steps, args.warmup, stream, settle_s=0.2)
            log("shape", main_kernel_name(hq, g, int(m), int(n), int(k)), r)
        return
    if args.gather_only:
        for k in (2, 8, 32):
            r = bench_gather(hq, synth, k, stream)
            r["frac"] = round(r["gbs"] / PEAK_GBS, 4)
            log("gather", r)
        return
    if args.config4_only:
        for reading in ("baseline", "layer_weights"):
            log("config4", bench_config4(hq, synth, stream, reading=reading))
        return
    if args.swiglu_only:
        for g in (synth.Q4_K, synth.Q8_0):
            for m in (512, 1):
                log("swiglu", bench_swiglu(hq, synth, g, stream, M=m))
        return
    if args.upload_only:
        log("upload", bench_upload(hq, synth))
        return
    if args.prefill_only:
        log("prefill", bench_prefill(hq, synth))
        return
    if args.gemv_only:
        for g, n, k in [(synth.Q8_0, 9728, 2560), (synth.Q4_K, 9728, 2560), (synth.Q4_K, 2560, 9728)]:
            r = bench_gemm(hq, synth, g, n, k, 1, False, args.steps, args.warmup, stream, settle_s=0.2)
            r["frac_hbm"] = round(r["gbs"] / PEAK_GBS, 4)
            log("gemv", r)
        for r in bench_read_floor(hq, synth, stream, args.steps):
            log("read floor", r)
        return

    gtype, N, K, M = synth.Q4_K, 9728, 2560, 512
    head = bench_gemm(hq, synth, gtype, N, K, M, False, args.steps, args.warmup, stream, kernel_time=True,
                      settle_s=0.3, reps=MEDIAN_REPS)
    log("headline", head)
    value = head["tflops"]
    head32 = bench_gemm(hq, synth, gtype, N, K, M, True, args.steps, args.warmup, stream, kernel_time=True,
                        settle_s=0.3, reps=MEDIAN_REPS)
    log("headline fp32 C", head32)

    sweep = []
    if not args.no_sweep:
        shapes = [(synth.Q8_0, 9728, 2560, m) for m in (1, 16, 128, 512, 2048)] + \
                 [(synth.Q4_K, 9728, 2560, m) for m in (1, 64, 512, 4096)] + \
                 [(synth.Q4_K, 2560, 9728, m) for m in (1, 64, 512, 4096)] + \
                 [(g, 9728, 2560, m) for g in (synth.Q2_K, synth.Q3_K, synth.Q5_K, synth.Q6_K) for m in (1, 64, 512)]
        # each shape: 0.1 s of untimed calls (clocks at their loaded level), then the median of
        # MEDIAN_REPS graph replays of 20 calls (a single replay ran up to a third slow at M = 2048)
        for g, n, k, m in shapes:
            r = bench_gemm(hq, synth, g, n, k, m, False, 20, 2, stream, settle_s=0.1, reps=MEDIAN_REPS)
            bound = "hbm" if (2.0 * m * n * k) / gemm_bytes(g, m, n, k, 2) < 312.5 else "mfma"
            r["bound"] = bound
            r["frac"] = round(r["gbs"] / PEAK_GBS if bound == "hbm" else r["tflops"] / PEAK_TFLOPS, 4)
            log("sweep", r)
            sweep.append({key: (round(v, 4) if isinstance(v, float) else v) for key, v in r.items() if key != "wall_s"})
        for k in (2, 8, 32):
            r = bench_gather(hq, synth, k, stream)
            r["bound"], r["frac"] = "hbm", round(r["gbs"] / PEAK_GBS, 4)
            log("sweep", r)
            sweep.append({key: (round(v, 4) if isinstance(v, float) else v) for key, v in r.items()})
        for reading in ("baseline", "layer_weights"):
            r = bench_config4(hq, synth, stream, reading=reading)
            log("sweep", r)
            sweep.append(r)
        for g in (synth.Q4_K, synth.Q8_0):
            for m in (512, 1):
                r = bench_swiglu(hq, synth, g, stream, M=m)
                log("sweep", r)
                sweep.append(r)
        r = bench_prefill(hq, synth)
        log("sweep", r)
        sweep.append(r)
        r = bench_upload(hq, synth)
        log("sweep", r)
        sweep.append(r)

    kt = head["kernel_tflops"]
    kname = main_kernel_name(hq, gtype, M, N, K)
    roofline = dict(bound="mfma", achieved=round(kt, 3), peak=PEAK_TFLOPS, unit="TFLOP/s",
                    frac=round(kt / PEAK_TFLOPS, 4), traffic=read_traffic("q4_k_gemm_m512_k2560_n9728", kname),
                    kernel=kname, kernel_us=round(head["kernel_us"], 3),
                    kernel_timing=f"median of {MEDIAN_REPS} HIP-graph replays of {MEDIAN_ITERS} launches")
    cpu = None if args.no_cpu else cpu_baseline(synth, gtype, N, K, M)
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(head["us"] / 1e3, 6),
        "us_median": round(head["us_median"], 3), "us_first_replay": round(head["us_first_replay"], 3),
        "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "q4_k_gemm_m512_k2560_n9728", "gtype": "Q4_K", "M": M, "N": N, "K": K,
                   "A": "fp16 N(0,1)", "C": "fp16 (fp32 accumulate)", "weight_copies": head["copies"],
                   "device": f"{name} ({arch})"},
        "roofline": roofline,
        "headline_fp32_c": {"C": "fp32", "us": round(head32["us"], 3), "tflops": round(head32["tflops"], 3),
                            "frac": round(head32["tflops"] / PEAK_TFLOPS, 4), "kernel_us": round(head32["kernel_us"], 3),
                            "kernel_tflops": round(head32["kernel_tflops"], 3),
                            "timing": f"median of {MEDIAN_REPS} HIP-graph replays of {args.steps} launches"},
        "cpu_baseline": cpu,
        "sweep": sweep,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
