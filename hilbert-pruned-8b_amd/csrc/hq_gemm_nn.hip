// hq_gemm_nn.hip - Q4_K GEMM for few output columns and many rows (N <= 32, M in the thousands: the
// 32-row b / a projections of the reference's Qwen3.5-4B layer list at prefill, src/shapes.c:12-39) on
// gfx950.
//
// C[M,N] (+)= A[M,K] . W^T with A fp16 and W GGUF Q4_K super-blocks (reference arithmetic:
// cleanroom-transformer/src/ggml_quant.h:51-59, :135-150; matmul src/cpu_backend.c:38-54).
//
// Why a kernel of its own. At N = 32 the work is reading A once (M = 16384, K = 2560: 84 MB against
// 46 KB of weights and 1 MB of C): HBM-bound on the activations, where the general kernels tile N
// 128-256 wide and spend their time on empty columns. Here a workgroup of four waves takes 64 rows,
// each wave 16 of them, and streams its activation fragments straight from HBM into MFMA operands
// (one 16-byte load per lane and k-step, two super-blocks ahead); the whole weight matrix is decoded once
// per workgroup and super-block into LDS. MFMA time is not the bound, so each weight is carried exactly:
// the fp32 weight w = (d * s) * q - dmin * m (the reference decoder's value, one rounding) as two fp16
// terms hi = fp16(w), lo = fp16(w - hi) (w to about 2^-22 relative), one MFMA each.
//
// LDS: two buffers x {hi, lo} x [32 columns][256 k] fp16 (64 KB); 16-byte slot p of column c at
// p ^ (c & 15), so the 16 lanes of an operand read hit 16 distinct slots.
#include "hq_device.h"
#include "hq_kernels.h"

namespace {
constexpr int NN_BM = 64, NN_NT = 256, NN_COLS = 32;

struct NnArgs {
    const uint8_t *W;  // Q4_K super-blocks, row n at n * row_bytes
    uint32_t row_bytes;
    const uint16_t *A;  // fp16 [M][K]
    int M, N, K;
    void *C;
    int c_f32, accumulate;
};

template <int NB>  // 16-column blocks of output (N <= 16 NB)
__global__ void __launch_bounds__(NN_NT) k_gemm_q4_k_nn(NnArgs g) {
    constexpr int TILE = NN_COLS * 256;  // fp16 values of one {hi or lo} tile
    __shared__ __attribute__((aligned(256))) _Float16 sb[2][2][TILE];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, ln = lane & 15, lg = lane >> 4;
    const int M = g.M, N = g.N, K = g.K, U = K / 256;
    const int m0 = blockIdx.x * NN_BM, row = m0 + 16 * wave + ln;
    // rows past M and weight rows past N read zeros (the row index is in the range-checked VGPR offset)
    const rsrc_t ra = make_rsrc(g.A, (uint32_t)((size_t)M * K * 2));
    const rsrc_t rw = make_rsrc(g.W, (uint32_t)((size_t)N * g.row_bytes));
    // activation operand of k-step f of super-block u: row `row`, k = 256 u + 32 f + 8 lg .. + 7
    const uint32_t a_voff = (uint32_t)row * (uint32_t)K * 2u + 16u * (uint32_t)lg;
    auto load_a = [&](u4v (&a)[8], int u) {
#pragma unroll
        for (int f = 0; f < 8; f++) a[f] = buf_load16(ra, a_voff, __builtin_amdgcn_readfirstlane((uint32_t)(u * 512 + f * 64)));
    };
    // weight decode: thread (column c = tid / 8, sub-block j = tid % 8) decodes the 32 values of
    // sub-block j of column c (quant group j / 2, nibble j % 2)
    const int c = tid >> 3, j = tid & 7;
    const uint32_t w_voff = (uint32_t)c * g.row_bytes;
    auto load_w = [&](u4v (&w)[3], int u) {
        // (u is wave-uniform: the scalar offset, so the loads need no per-lane offset loop)
        const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)u * 144u);
        w[0] = buf_load16(rw, w_voff, so);                                    // d, dmin, scales
        w[1] = buf_load16(rw, w_voff + 16u + 32u * (uint32_t)(j >> 1), so);   // quant group j / 2
        w[2] = buf_load16(rw, w_voff + 32u + 32u * (uint32_t)(j >> 1), so);
    };
    auto decode = [&](const u4v (&w)[3], int buf) {
        uint32_t sw0, sw1, mw0, mw1;
        q4k_scale_words(w[0].y, w[0].z, w[0].w, sw0, sw1, mw0, mw1);
        const float d1 = h2f((uint16_t)w[0].x) * (float)byte_of(j < 4 ? sw0 : sw1, j & 3);
        const float m1 = h2f((uint16_t)(w[0].x >> 16)) * (float)byte_of(j < 4 ? mw0 : mw1, j & 3);
        const int sh = 4 * (j & 1);
        const uint32_t qw[8] = {w[1].x, w[1].y, w[1].z, w[1].w, w[2].x, w[2].y, w[2].z, w[2].w};
#pragma unroll
        for (int s = 0; s < 4; s++) {  // 8 values = slot 4 j + s
            h8 hi, lo;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t q = (qw[2 * s + (e >> 2)] >> (8 * (e & 3) + sh)) & 15u;
                const float v = __builtin_fmaf(d1, (float)q, -m1);
                const _Float16 h = (_Float16)v;
                hi[e] = h;
                lo[e] = (_Float16)(v - (float)h);
            }
            const int slot = (4 * j + s) ^ (c & 15);
            *(h8 *)&sb[buf][0][c * 256 + 8 * slot] = hi;
            *(h8 *)&sb[buf][1][c * 256 + 8 * slot] = lo;
        }
    };
    f4 acc[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] = f4{0.f, 0.f, 0.f, 0.f};
    // super-block u: decode its weights into buffer u % 2 (last read by super-block u - 2, whose MFMAs
    // every wave finished before the barrier of u - 1), barrier, multiply; the activations and weight
    // bytes of u + 1 are in flight meanwhile
    auto step = [&](const u4v (&a)[8], const u4v (&w)[3], int u) {
        const int buf = u & 1;
        decode(w, buf);
        // this wave's LDS writes done, then the barrier; no fence: __syncthreads() would also wait
        // for every outstanding load, the prefetched super-blocks included
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
        for (int f = 0; f < 8; f++)
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const int off = (16 * b + ln) * 256 + 8 * ((4 * f + lg) ^ ln);
                const h8 bh = *(const h8 *)&sb[buf][0][off], bl = *(const h8 *)&sb[buf][1][off];
                const h8 av = __builtin_bit_cast(h8, a[f]);
                acc[b] = mfma(bh, av, acc[b]);
                acc[b] = mfma(bl, av, acc[b]);
            }
    };
    // three register sets: the loads of super-block u + 2 are issued as u's step starts (into the set
    // that u - 1 used), so two super-blocks of activations are in flight behind the one multiplied
    // (every step issues its loads, of super-block min(u + 2, U - 1): a loop body without conditional
    // loads lets the compiler's wait counts see the two super-blocks in flight)
    u4v a0[8], a1[8], a2[8], w0[3], w1[3], w2[3];
    const int ul = U - 1;
    load_a(a0, 0), load_w(w0, 0);
    load_a(a1, min(1, ul)), load_w(w1, min(1, ul));
    int u = 0;
    for (; u + 3 <= U; u += 3) {
        load_a(a2, min(u + 2, ul)), load_w(w2, min(u + 2, ul));
        step(a0, w0, u);
        load_a(a0, min(u + 3, ul)), load_w(w0, min(u + 3, ul));
        step(a1, w1, u + 1);
        load_a(a1, min(u + 4, ul)), load_w(w1, min(u + 4, ul));
        step(a2, w2, u + 2);
    }
    if (u < U) step(a0, w0, u);
    if (u + 1 < U) step(a1, w1, u + 1);
    // lane (ln, lg) of block b: row `row`, columns 16 b + 4 lg .. + 3
    if (row >= M) return;
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int n = 16 * b + 4 * lg + e;
            if (n < N) store_out(g.C, (size_t)row * N + n, acc[b][e], g.c_f32, g.accumulate);
        }
}
}  // namespace

int hq_nn_fits(const hq_dev_mat *W, int M) {
    const size_t lim = (size_t)1 << 32;
    return W->type == HQ_TYPE_Q4_K && W->rows >= 1 && W->rows <= NN_COLS && W->cols % 256 == 0 && M >= 1 &&
           ((size_t)M + NN_BM) * W->cols * 2 < lim;
}

hipError_t hq_launch_gemm_nn(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                             hipStream_t st) {
    if (!hq_nn_fits(W, M) || (c_f32 != 0 && c_f32 != 1)) return hipErrorInvalidValue;
    NnArgs g;
    g.W = W->qs, g.row_bytes = (uint32_t)W->row_bytes, g.A = A;
    g.M = M, g.N = (int)W->rows, g.K = (int)W->cols, g.C = C, g.c_f32 = c_f32, g.accumulate = accumulate;
    const unsigned grid = (unsigned)((M + NN_BM - 1) / NN_BM);
    if (g.N <= 16) k_gemm_q4_k_nn<1><<<grid, NN_NT, 0, st>>>(g);
    else k_gemm_q4_k_nn<2><<<grid, NN_NT, 0, st>>>(g);
    return hipGetLastError();
}
