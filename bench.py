"""Benchmark of the gfx950 quantized matmul path (one GPU).

Headline workload (the BASELINE north-star target): Q4_K GEMM, M = 512, K = 2560, N = 9728
(config 3, up/gate shape), fp16 activations, fp32 accumulation, fp16 output. A "step" is one GEMM
launch over one batch; weights rotate over enough distinct device copies (> 512 MB) that every
launch streams its weights from HBM, not from the 256 MB Infinity Cache. The timed steps are one
HIP-graph replay of exactly `steps` launches, timed with HIP events on the launch stream, after
`warmup` eager launches and one untimed replay of the same graph.

Also reported (key "sweep"): the config 2 / 3 M sweeps and the config 5 option readout, each as
achieved TFLOP/s and GB/s of algorithmic bytes (W blocks once + A + C) and their roofline fractions.

cpu_baseline: the CPU oracle (a restatement of the reference's cpu_backend.c matmul, compiled with
the reference's flags, OpenMP) on the headline GEMM, timed on this host's cores.
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


def read_traffic(name):
    """HBM bytes per launch of the headline kernel from the committed PMC summary, or None."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith(name + " "):
            try:
                return float(line.split()[1])
            except (IndexError, ValueError):
                return None
    return None


def bench_gemm(hq, synth, gtype, N, K, M, c_f32, steps, warmup, stream, eager_warmup=True):
    rb = synth.row_bytes(gtype, K)
    blocks = synth.random_blocks(gtype, synth.Rng(4242 + gtype + N), N, K)
    copies = max(2, -(-ROTATE_BYTES // (N * rb)))
    mats = [hq.Mat(blocks, gtype, N, K) for _ in range(copies)]
    A = hq.DevBuf.from_array(synth.activations_f16(synth.Rng(99 + M), M, K))
    C = hq.DevBuf(M * N * (4 if c_f32 else 2))
    if eager_warmup:
        for i in range(warmup):
            hq.gemm(mats[i % copies], A, M, C, c_f32, False, stream.ptr)
        stream.sync()
    t0 = time.perf_counter()
    ms = hq.time_gemm(mats, A, M, C, c_f32, steps, 1, stream)
    wall = time.perf_counter() - t0
    for m in mats:
        m.free()
    A.free(), C.free()
    flop = 2.0 * M * N * K
    nbytes = gemm_bytes(gtype, M, N, K, 4 if c_f32 else 2)
    return dict(type="q8_0" if gtype == synth.Q8_0 else "q4_k", M=M, N=N, K=K, us=ms * 1e3,
                tflops=flop / (ms * 1e-3) / 1e12, gbs=nbytes / (ms * 1e-3) / 1e9, copies=copies,
                wall_s=wall)


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


def cpu_baseline(synth, gtype, N, K, M):
    import oracle
    O = oracle.Oracle()
    blocks = synth.random_blocks(gtype, synth.Rng(4242 + gtype + N), N, K)
    x = O.f16_to_f32(synth.activations_f16(synth.Rng(99 + M), M, K))
    y = np.zeros((M, N), np.float32)
    O.matmul(blocks, gtype, N, K, x, y)  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        O.matmul(blocks, gtype, N, K, x, y)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    cores = int(os.environ.get("OMP_NUM_THREADS") or len(os.sched_getaffinity(0)))
    return dict(value=round(2.0 * M * N * K / t / 1e12, 6), unit="TFLOP/s", cores=cores, kind="port",
                sample=f"full headline GEMM (Q4_K M={M} N={N} K={K}), oracle restatement of cpu_backend.c "
                       f"matmul (-O2 -std=c11 -fopenmp), median of 3 after 1 warm-up: {t:.3f} s; "
                       f"host CPU: {cpu_model()}")


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

    gtype, N, K, M = synth.Q4_K, 9728, 2560, 512
    head = bench_gemm(hq, synth, gtype, N, K, M, False, args.steps, args.warmup, stream)
    log("headline", head)
    value = head["tflops"]

    sweep = []
    if not args.no_sweep:
        shapes = [(synth.Q8_0, 9728, 2560, m) for m in (1, 16, 128, 512, 2048)] + \
                 [(synth.Q4_K, 9728, 2560, m) for m in (1, 64, 512, 4096)] + \
                 [(synth.Q4_K, 2560, 9728, m) for m in (1, 64, 512, 4096)]
        for g, n, k, m in shapes:
            r = bench_gemm(hq, synth, g, n, k, m, False, 20, 2, stream)
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

    roofline = dict(bound="mfma", achieved=round(value, 3), peak=PEAK_TFLOPS, unit="TFLOP/s",
                    frac=round(value / PEAK_TFLOPS, 4), traffic=read_traffic("q4_k_gemm_m512_k2560_n9728"))
    cpu = None if args.no_cpu else cpu_baseline(synth, gtype, N, K, M)
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(head["us"] / 1e3, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "q4_k_gemm_m512_k2560_n9728", "gtype": "Q4_K", "M": M, "N": N, "K": K,
                   "A": "fp16 N(0,1)", "C": "fp16 (fp32 accumulate)", "weight_copies": head["copies"],
                   "device": f"{name} ({arch})"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "sweep": sweep,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
