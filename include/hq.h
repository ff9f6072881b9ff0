/* hq.h - C ABI of the MI355X (gfx950) quantized matmul path for GGUF Q8_0 / Q4_K weights.
 *
 * Drop-in boundary for the cleanroom-transformer runtime's quantized matmul path. Plain C types
 * only; streams are opaque `void *` (NULL = the default stream); device pointers are plain
 * pointers into HIP device memory. Conventions follow the reference (paths relative to
 * cleanroom-transformer/):
 *   - W is [rows = N = outputs, cols = K = inputs], GGUF-block-packed along K
 *     (src/transformer.h:245, :293-300, :331-332);
 *   - A is [M, K] row-major, C is [M, N] row-major, C[m][n] (+)= sum_k A[m][k] * W[n][k]
 *     (src/cpu_backend.c:38-54, src/cuda_backend.cu:701-715);
 *   - every fallible call returns 0, or -1 after recording a message for hq_last_error()
 *     (the reference's set_error/last_error convention, src/transformer.h:17-21, src/base.c:11-21).
 * Supported block types: Q8_0 (ggml type 8) and the k-quants Q2_K (10), Q3_K (11), Q4_K (12), Q5_K (13)
 * and Q6_K (14) (src/ggml_quant.h:16-19); K must be a multiple of the block (32 for Q8_0, 256 for the
 * k-quants), as src/gguf.c:331-335 enforces for GGUF tensors.
 * Not thread-safe across concurrent calls that share a matrix's device (as the reference engine,
 * which is single threaded: src/transformer.h:18-19).
 */
#ifndef HQ_H
#define HQ_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { HQ_DT_GGML = 3 };                     /* dtype_t DT_GGML (src/transformer.h:214) */
enum { HQ_GGML_Q8_0 = 8, HQ_GGML_Q2_K = 10, HQ_GGML_Q3_K = 11, HQ_GGML_Q4_K = 12, HQ_GGML_Q5_K = 13,
       HQ_GGML_Q6_K = 14 }; /* src/ggml_quant.h:16-19 */

/* Host matrix descriptor, field for field the reference wmat_t (src/transformer.h:293-300):
 * data points at GGUF blocks (typically into the model's mmap), rows in storage order;
 * perm_heads > 0 marks llama.cpp-interleaved q/k rows in that many heads (src/model.c:283-289). */
typedef struct {
    int dtype;
    uint32_t rows, cols;
    const void *data;
    int ggml_type;
    uint32_t perm_heads;
} hq_wmat_t;

/* A weight matrix resident in one GPU's HBM (opaque), rows in Hugging Face order. */
typedef struct hq_mat hq_mat;

/* Last error message of the calling thread (src/transformer.h:21 last_error). */
const char *hq_last_error(void);

/* Selects `device` for the calling thread and checks it is a gfx950 (MI355X-class) GPU.
 * Replaces the device checks of cu_init (src/cuda_backend.cu:915-924). */
int hq_device_init(int device);
int hq_device_count(int *count);
/* Marketing name and gfx arch of a device, for reports. */
int hq_device_name(int device, char *name, size_t name_len, char *arch, size_t arch_len);

/* Weight residency. Replaces upload_mat (src/cuda_backend.cu:677-699) for GGUF-quantized
 * matrices: the blocks are copied to `device` with rows reordered into Hugging Face order
 * (perm_heads, as src/cuda_backend.cu:689-696). Q4_K blocks are kept byte-identical; Q8_0 is
 * repacked losslessly into a quant plane and a scale plane, Q2_K / Q3_K / Q6_K into 96- / 112- /
 * 224-byte aligned slots (Q5_K keeps its bytes)
 * (hq_mat_download restores the bytes).
 * There is no bf16 fallback: non-GGML dtypes and other block types are rejected. */
int hq_mat_upload(const hq_wmat_t *w, int device, hq_mat **out);
void hq_mat_free(hq_mat *m);
int hq_mat_shape(const hq_mat *m, uint32_t *rows, uint32_t *cols, int *ggml_type);
size_t hq_mat_device_bytes(const hq_mat *m);
/* The matrix as GGUF blocks, rows in Hugging Face order (rows * row_bytes bytes); round-trip check. */
int hq_mat_download(const hq_mat *m, void *out, size_t nbytes);

/* Test hook: rows [row0, row0 + nrows) dequantised to fp32 into device memory `out` [nrows, cols],
 * bit-identical to the reference decoder ggml_dequantize_row (src/gguf.c:59-73). */
int hq_dequant_f32(const hq_mat *W, uint32_t row0, uint32_t nrows, float *out, void *stream);

/* C[M,N] (+)= A[M,K] . W^T with A fp16 [M, K] (device, 16-byte aligned), fp32 accumulation, C fp32
 * (c_is_f32 != 0) or fp16. Replaces gemm_w (src/cuda_backend.cu:701-715) and its kernels
 * k_gemv_q (:445-481), k_dequant_bf16 (:433-443) and k_gemm_wmma (:87-135). M = 1 runs the GEMV.
 * Asynchronous on `stream`. */
int hq_gemm(const hq_mat *W, const uint16_t *A, int M, void *C, int c_is_f32, int accumulate, void *stream);
/* M = 1: c[N] (+)= W . a, the HBM-bound wavefront-reduction GEMV (k_gemv_q at M = 1, :445-481). */
int hq_gemv(const hq_mat *W, const uint16_t *a, void *c, int c_is_f32, int accumulate, void *stream);

/* hq_gemm that allocates nothing: no hipMalloc, hipFree or allocating library call on any path.
 * No counterpart in the reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation). The GEMM workspace
 * (partial tiles, per-tile counters, activation sums) lives in one preallocated device array of
 * HQ_NOALLOC_SCRATCH_BYTES per GPU, held from the library's first use of that GPU until the
 * process ends; a call whose launches need more (see hq_gemm_workspace_bytes) fails with -1 before
 * anything is queued. Same kernels and results as hq_gemm, bit for bit. Every call on one GPU
 * shares that GPU's array: calls that overlap in time on one GPU (other streams, other threads)
 * race and must be serialised by the caller. The first call on a device also waits for a small
 * clearing kernel on `stream` (not capturable); later calls only queue the GEMM's kernels. */
#define HQ_NOALLOC_SCRATCH_BYTES (96 << 20)
#define HQ_NOALLOC_COUNTER_BYTES (1 << 20)
int hq_gemm_noalloc(const hq_mat *W, const uint16_t *A, int M, void *C, int c_is_f32, int accumulate, void *stream);
/* Workspace of one M-row GEMM launch (2 <= M <= rows per launch) of an N x K matrix of the given
 * ggml type on a GPU with n_cu CUs: fp32 partial-tile bytes, counter bytes, activation-sum bytes,
 * and whether it fits hq_gemm_noalloc's scratch (diagnostics; no device is touched). */
int hq_gemm_workspace_bytes(int ggml_type, int M, uint32_t N, uint32_t K, int n_cu, size_t *partial_bytes,
                            size_t *counter_bytes, size_t *sums_bytes, int *fits_noalloc);

/* Single-token FFN input: out[i] = fp16(silu(gate_i . a) * (up_i . a)) for i < rows, with a fp16
 * [cols] and out fp16 [rows] in device memory, fp32 dots of the exactly decoded weights. gate and up
 * share a shape and a device; their block types may differ (Q4_K_M files pair a Q4_K gate with a
 * Q6_K up). Replaces k_gateup_swiglu (src/cuda_backend.cu:548-559); one pass over both matrices. */
int hq_gemv_swiglu(const hq_mat *gate, const hq_mat *up, const uint16_t *a, uint16_t *out, void *stream);

/* Gate/up pair for the SwiGLU FFN input: one resident matrix of 2 * rows rows, rows 16k .. 16k + 7 of
 * gate interleaved with rows 16k + 8 .. 16k + 15 of up (gate and up: same type and shape, rows a
 * multiple of 8), so that one GEMM tile covers matching gate and up columns and the activations are
 * read once for both. */
int hq_mat_upload_pair(const hq_wmat_t *gate, const hq_wmat_t *up, int device, hq_mat **out);
/* out[M, rows] fp16 = silu(A . gate^T) * (A . up^T) for a pair matrix, A fp16 [M, K]; out 16-byte
 * aligned. Replaces gemm_w(gate) + gemm_w(up) + k_swiglu (src/cuda_backend.cu:845-849, :413-416):
 * for M > 64 the product never leaves the GEMM's tile (the epilogue of the full-K tile kernels
 * applies silu(g) * u), other shapes run one GEMM for both halves and a separate epilogue pass. */
int hq_gemm_swiglu(const hq_mat *pair, const uint16_t *A, int M, uint16_t *out, void *stream);

/* Option-row readout: out[b*k + j] = dot(H[b], head[ids[b*k + j]]) for b < B, j < k, fp32.
 * H fp16 [B, K] and out on the device; ids on the HOST (checked against rows, then staged).
 * Replaces the quantized readout of k_readout_q / k_norm_readout (src/cuda_backend.cu:490-502,
 * :561-592) and the CPU readout (src/cpu_backend.c:253-259), batched over states. */
int hq_gather_dot(const hq_mat *head, const uint16_t *H, const uint32_t *ids, int B, int k, float *out, void *stream);
/* Same with ids already in device memory; an id >= rows yields NaN for that pair (never a fault). */
int hq_gather_dot_dev(const hq_mat *head, const uint16_t *H, const uint32_t *ids_dev, int B, int k, float *out,
                      void *stream);

/* Host-pointer drop-in for the CPU backend's matmul (src/cpu_backend.c:39):
 * y[t*rows + r] (+)= dot(x[t*cols ..], W[r]) for t < T, x and y fp32 on the host. x is rounded to
 * fp16 on the device; the call is synchronous. */
int hq_matmul_host(const hq_mat *W, const float *x, size_t T, float *y, bool accumulate);

/* ---- device memory, streams and timing, for callers without their own HIP runtime */
int hq_malloc(void **p, size_t n);
int hq_free(void *p);
int hq_memcpy_h2d(void *dst, const void *src, size_t n, void *stream);
int hq_memcpy_d2h(void *dst, const void *src, size_t n, void *stream);
/* device to device, asynchronous on `stream` (also the copy kernel the HBM-traffic counters are
 * calibrated against) */
int hq_memcpy_d2d(void *dst, const void *src, size_t n, void *stream);
int hq_memset(void *dst, int value, size_t n, void *stream);
int hq_stream_create(void **stream);
int hq_stream_destroy(void *stream);
int hq_stream_synchronize(void *stream);
int hq_device_synchronize(void);

/* Benchmark helpers: `iters` launches of hq_gemm (resp. hq_gather_dot_dev), launch i using
 * Ws[i % n_w] (and, for the gather, id set i % n_sets of n_sets consecutive [B*k] arrays at
 * ids_dev), captured on `stream` in `reps` HIP graphs of `iters` launches each (graph r: launches
 * r * iters .. r * iters + iters - 1; reps <= 64) and replayed in order after one warm-up replay of
 * the last, a HIP event on `stream` between consecutive replays; *ms = the median over the replays
 * of the replay's milliseconds per launch. */
int hq_time_gemm(hq_mat *const *Ws, int n_w, const uint16_t *A, int M, void *C, int c_is_f32, int iters, int reps,
                 void *stream, float *ms);
/* As hq_time_gemm, timing only the GEMM's main kernel (M >= 2): an activation pre-pass the
 * kernel needs (it depends on A alone) runs once before the capture. */
int hq_time_gemm_kernel(hq_mat *const *Ws, int n_w, const uint16_t *A, int M, void *C, int c_is_f32, int iters,
                        int reps, void *stream, float *ms);
/* As hq_time_gemm for hq_gemm_swiglu over pair matrices. */
int hq_time_gemm_swiglu(hq_mat *const *pairs, int n_w, const uint16_t *A, int M, uint16_t *out, int iters, int reps,
                        void *stream, float *ms);
int hq_time_gather(hq_mat *const *Ws, int n_w, const uint16_t *H, const uint32_t *ids_dev, int n_sets, int B, int k,
                   float *out, int iters, int reps, void *stream, float *ms);
/* Diagnostic floor for the HBM-bound kernels: a pure streaming read of `bytes` (a multiple of 16)
 * from bufs[i % n_bufs] by `grid` workgroups of 256 threads, timed as hq_time_gemm times its calls. */
int hq_time_read(void *const *bufs, int n_bufs, size_t bytes, int grid, int iters, int reps, void *stream, float *ms);

/* The output tile hq_gemm uses for an M x N problem of the given ggml type on a 256-CU MI355X
 * (diagnostics; the launch itself sizes for the device's CU count). */
void hq_gemm_tiles(int ggml_type, int M, int N, int *rows_per_tile, int *cols_per_tile);

/* Name of the kernel that does the work of an M x N x K hq_gemm call on a 256-CU MI355X (the main
 * kernel where a pre-pass runs first), as rocprofv3 lists it; NUL-terminated, truncated to
 * name_bytes (diagnostics for profiling). */
void hq_gemm_kernel(int ggml_type, int M, int N, int K, char *name, int name_bytes);

#ifdef __cplusplus
}
#endif
#endif
