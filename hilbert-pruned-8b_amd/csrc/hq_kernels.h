// hq_kernels.h - internal interface between the C-ABI layer (hq_api.hip) and the gfx950 kernels.
#ifndef HQ_KERNELS_H
#define HQ_KERNELS_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

enum { HQ_TYPE_Q8_0 = 8, HQ_TYPE_Q2_K = 10, HQ_TYPE_Q3_K = 11, HQ_TYPE_Q4_K = 12, HQ_TYPE_Q5_K = 13, HQ_TYPE_Q6_K = 14 };

// A weight matrix resident in HBM, rows in Hugging Face order (see hq_kernels.hip for layouts).
typedef struct {
    int type;
    uint32_t rows, cols;
    const uint8_t *qs;   // Q8_0: biased quant plane [rows][cols]; k-quants: super-blocks [rows][row_bytes]
    const uint16_t *d;   // Q8_0: fp16 scale plane [rows][ldd]; Q4_K: unused
    int ldd;             // Q8_0 scale-plane row stride in halves (cols/32 rounded up to 8)
    size_t row_bytes;    // Q8_0 / Q4_K / Q5_K: GGUF bytes per row; Q2_K / Q3_K / Q6_K: device bytes per row
                         // (96 / 112 / 224 per super-block)
    const uint8_t *tab;  // Q4_K: per-super-block column tables of the GEMM kernels (hq_launch_q4k_tables)
} hq_dev_mat;

// Q4_K column tables: HQ_Q4K_TAB_BYTES per row and super-block (Bmin hi / lo, scale words, R, CL)
#define HQ_Q4K_TAB_BYTES 48u
// zero bytes after a matrix's tables: the GEMM's table loads for the columns of its last tile past N
#define HQ_Q4K_TAB_PAD 8192u
hipError_t hq_launch_q4k_tables(const hq_dev_mat *W, uint8_t *tab, hipStream_t st);

// The device view and device of a resident matrix (hq_api.hip), for the library's own host code.
struct hq_mat;
const hq_dev_mat *hq_mat_dev(const struct hq_mat *m);
int hq_mat_device(const struct hq_mat *m);

// rows row0 .. row0 + nrows - 1, or rows ids[0 .. nrows - 1] when ids (device) is not null
hipError_t hq_launch_dequant(const hq_dev_mat *W, uint32_t row0, const uint32_t *ids, uint32_t nrows, float *out,
                             hipStream_t st);
hipError_t hq_launch_gemv(const hq_dev_mat *W, const uint16_t *a, void *C, int c_f32, int accumulate, hipStream_t st);
// Stream-K workspace: fp32 partial tiles and per-tile counters (zero when idle; each launch leaves
// them zero), the activation sub-block sums of the wide Q4_K kernel, and the number of CUs the
// persistent grid is sized for.
struct HqGemmWork {
    float *partials;
    int *counters;
    uint16_t *sums;
    int n_cu;
};
void hq_gemm_work_bytes(const hq_dev_mat *W, int M, int n_cu, size_t *partial_bytes, size_t *counter_bytes,
                        size_t *sums_bytes);
// M >= 2: hq_launch_gemm = hq_launch_gemm_pre (activation pre-pass, if the kernel needs one) then
// hq_launch_gemm_main.
hipError_t hq_launch_gemm_pre(const hq_dev_mat *W, const uint16_t *A, int M, const HqGemmWork &wk, hipStream_t st);
hipError_t hq_launch_gemm_main(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                               const HqGemmWork &wk, hipStream_t st);
hipError_t hq_launch_gemm(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                          const HqGemmWork &wk, hipStream_t st);
hipError_t hq_launch_gather(const hq_dev_mat *W, const uint16_t *H, const uint32_t *ids, int B, int k, float *out,
                            hipStream_t st);
hipError_t hq_launch_f32_to_f16(const float *in, uint16_t *out, size_t n, hipStream_t st);
// diagnostic streaming read of `bytes` (a multiple of 16) by `grid` workgroups; out[4 * grid] words
hipError_t hq_launch_stream_read(const void *p, size_t bytes, uint32_t *out, unsigned grid, hipStream_t st);
// gate/up pair matrices (rows 16k .. 16k + 7 of gate, 16k + 8 .. + 15 of up): the GEMM with the SwiGLU
// epilogue fused into the tile kernels (*fused = 0 when the shape does not run them), and the
// epilogue as a separate pass over an fp32 [M, 2I] product (n_out = M * I)
hipError_t hq_launch_gemm_swiglu(const hq_dev_mat *W, const uint16_t *A, int M, uint16_t *out, const HqGemmWork &wk,
                                 hipStream_t st, int *fused);
hipError_t hq_launch_swiglu_pairs(const float *C, uint16_t *out, size_t n_out, hipStream_t st);
// rows x columns of one GEMM output tile (M >= 2) on a device with n_cu CUs
void hq_gemm_tile_shape(int type, int M, int N, int K, int n_cu, int *rows, int *cols);
void hq_gemm_kernel_name(int type, int M, int N, int K, int n_cu, char *buf, size_t n);
// Full-K tile Q4_K / Q5_K GEMM (hq_gemm_ws.hip): the tile width (32 * nb columns) for an M x N problem
// on n_cu CUs and the fraction of CU time its tiles fill; the launch (S: Q5_K, the k_asums output for
// A; Q4_K forms its activation sums in the kernel and takes none; each tile's K split into `parts`
// workgroups when parts > 1, with fp32 partial tiles and per-tile counters as for Stream-K).
int hq_ws_choose(int M, int N, int n_cu, float *eff);
hipError_t hq_launch_gemm_ws(const hq_dev_mat *W, const uint16_t *A, const uint16_t *S, int M, void *C, int c_f32,
                             int accumulate, int nb, int parts, float *partials, int *counters, hipStream_t st);
// Large-M Q4_K GEMM (hq_gemm_bt.hip): 256 x 256 tiles over the whole of K, one workgroup each (S =
// k_asums<true> output for A); whether a shape's byte offsets suit it, and the launch.
int hq_bt_fits(const hq_dev_mat *W, int M);
hipError_t hq_launch_gemm_bt(const hq_dev_mat *W, const uint16_t *A, const uint16_t *S, int M, void *C, int c_f32,
                             int accumulate, hipStream_t st);
// Prefill Q4_K GEMM of one tile round (hq_gemm_wr.hip): 128 x 192 tiles over the whole of K, 4 waves
// that each decode their own 48 columns and 4 loader waves (which also form the activation sub-block
// sums: no pre-pass, no workspace); whether a shape's byte offsets suit it, and the launch (c_f32:
// 1 fp32 C, 0 fp16 C, HQ_OUT_SWIGLU fp16 silu(gate) * up of a gate/up pair matrix) of the column
// tiles nt0 .. nt1 - 1 (nt1 < 0: to the last); the Q4_K one also with each tile's K split over
// `parts` workgroups (partials / counters as for the other K splits).
int hq_wr_fits(const hq_dev_mat *W, int M);
// The sum of a K split's part tiles (128-row tiles of bn = 160 or 192 columns in tile_finish's layout,
// stored by every part of a kernel launched with no counters), added in part order and stored to C.
hipError_t hq_launch_tile_reduce(const float *partials, int parts, int ntiles, int mt, int bn, int M, int N, void *C, int c_f32,
                                 int accumulate, hipStream_t st);
hipError_t hq_launch_gemm_wr(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                             int nt0, int nt1, int parts, float *partials, int *counters, hipStream_t st, int tw = 192);
// The same tile shape for Q8_0 (hq_gemm_wr8.hip; K a multiple of 256, no workspace).
int hq_wr8_fits(const hq_dev_mat *W, int M);
hipError_t hq_launch_gemm_wr8(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                              int nt0, int nt1, hipStream_t st);
// Mid-M Q4_K GEMM (hq_gemm_rb.hip): whether M, K suit it (33 <= M <= 64, K a multiple of 512,
// 32-bit offsets), its workgroups per tile for a shape, and the launch (no pre-pass: the kernel forms
// the activation sub-block sums; partials / counters as for the other K splits when parts > 1).
int hq_rb_fits(int M, int K);
int hq_rb_parts(int M, int N, int K, int n_cu);  // 0: not this kernel; else workgroups per tile
hipError_t hq_launch_gemm_rb(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32,
                             int accumulate, int parts, float *partials, int *counters, hipStream_t st);
// Mid-M Q8_0 GEMM (hq_gemm_rb.hip): workgroups per tile for a shape (0: not this kernel), and the
// launch (no pre-pass; partials / counters as for the other K splits when parts > 1).
int hq_rb8_parts(int M, int N, int K, int n_cu);
hipError_t hq_launch_gemm_rb8(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                              int parts, float *partials, int *counters, hipStream_t st);
hipError_t hq_launch_gemm_ws8(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                              int nb, int parts, float *partials, int *counters, hipStream_t st);
// Q4_K GEMM with at most 32 output columns (hq_gemm_nn.hip: 64-row workgroups streaming A once, the
// weights decoded per workgroup into LDS as exact fp16 hi / lo pairs); whether a shape suits it.
int hq_nn_fits(const hq_dev_mat *W, int M);
hipError_t hq_launch_gemm_nn(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                             hipStream_t st);
// Q6_K, Q3_K and Q2_K full-K tile GEMM (hq_gemm_ws.hip: producers decode into an fp16 B tile in LDS;
// K split as for the Q8_0 kernel, in whole super-blocks), and whether its byte offsets fit 32 bits.
hipError_t hq_launch_gemm_kqws(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                               int nb, int parts, float *partials, int *counters, hipStream_t st);
int hq_kqws_fits(const hq_dev_mat *W, int M);

// Q6_K (hq_q6k.hip)
struct GemmArgs;
hipError_t hq_launch_dequant_q6k(const hq_dev_mat *W, uint32_t row0, const uint32_t *ids, uint32_t nrows, float *out,
                                 hipStream_t st);
hipError_t hq_launch_gemm_q6k(const GemmArgs &g, int mb, hipStream_t st);

// Q2_K, Q3_K, Q5_K (hq_kquant.hip); the GEMV and gather launchers also take Q6_K
hipError_t hq_launch_dequant_kq(const hq_dev_mat *W, uint32_t row0, const uint32_t *ids, uint32_t nrows, float *out,
                                hipStream_t st);
hipError_t hq_launch_gemv_kq(const hq_dev_mat *W, const uint16_t *a, void *C, int c_f32, int accumulate, hipStream_t st);
int hq_sb_rows(int n_out);       // rows per wave of that GEMV and gather for n_out rows
int hq_sb_lds(int type, int K);  // whether that GEMV copies its activation vector into LDS
hipError_t hq_launch_gather_kq(const hq_dev_mat *W, const uint16_t *H, const uint32_t *ids, int B, int k, float *out,
                               hipStream_t st);
hipError_t hq_launch_gemm_kq(int type, const GemmArgs &g, int mb, hipStream_t st);
constexpr bool hq_is_kq(int type) { return type == HQ_TYPE_Q2_K || type == HQ_TYPE_Q3_K || type == HQ_TYPE_Q5_K; }

#endif
