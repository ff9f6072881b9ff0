// hq_kernels.hip - gfx950 (CDNA4) kernels for GGUF Q8_0 / Q4_K matrices resident in HBM.
//
// Device residency (written by hq_api.hip at upload, rows in Hugging Face order):
//   Q8_0  two planes: qs[N][K] bytes holding q ^ 0x80 (biased: u = q + 128), then, at a
//         256-byte aligned offset, d[N][ldd] fp16 with ldd = K/32 rounded up to 8 (zero padded).
//         Lossless: hq_mat_download restores the 34-byte GGUF blocks bit for bit.
//   Q4_K  the 144-byte GGUF super-blocks unchanged: {fp16 d, fp16 dmin, u8 scales[12], u8 qs[128]}.
//
// Arithmetic (reference: cleanroom-transformer/src/ggml_quant.h:95-99 Q8_0, :51-59 and :135-150 Q4_K):
//   Q8_0 w = q*d;  Q4_K w = (d*s)*q - dmin*m with 6-bit (s, m) per 32-value sub-block.
//
// Kernels
//   k_dequant_*   rows -> fp32, bit-identical to the CPU decoder (the products are exact in fp32
//                 and the one rounding, the Q4_K subtraction, is the same fused or not).
//   k_gemv_*      M = 1: 16 lanes per weight row, fp32 VALU, one pass over the blocks (HBM-bound).
//   k_gather_*    option-row readout: the GEMV loop over (state, id) pairs.
//   k_gemm<>      M >= 2: MFMA v_mfma_f32_16x16x32_f16. Each wave decodes its own weight columns
//                 straight from global memory into B fragments (no LDS round trip for weights);
//                 the activation tile is staged once per workgroup in LDS and shared by 4 waves.
//     Q8_0 B operand: fp16(q*d), one rounding of the exact product.
//     Q4_K B operand: the integer s*q (<= 945, exact in fp16); the fp32 accumulator of each
//       256-value super-block is scaled by d once, and the min term -dmin*sum_sub(m*S_sub) (S =
//       fp32 sum of 32 activations) is one extra MFMA with hi/lo fp16 splits of dmin*m and S, so
//       no weight value is ever rounded to 16 bits.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <cstdio>

#include <algorithm>

#include "hq_device.h"
#include "hq_kernels.h"


// ============================================================================ dequantize
// Output row r is matrix row ids[r] when ids is given (embedding gather), else row0 + r.
__global__ void __launch_bounds__(256) k_dequant_q8_0(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ d,
                                                      int K, int ldd, uint32_t row0, const uint32_t *__restrict__ ids,
                                                      uint32_t nrows, float *__restrict__ out) {
    const size_t per_row = (size_t)K / 4, total = (size_t)nrows * per_row;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / per_row, c = (i % per_row) * 4, row = ids ? (size_t)ids[r] : row0 + r;
        const uint32_t w = *(const uint32_t *)(qs + row * (size_t)K + c) ^ 0x80808080u;
        const float dv = h2f(d[row * (size_t)ldd + c / 32]);
        float4 y;
        y.x = (float)(int8_t)byte_of(w, 0) * dv;
        y.y = (float)(int8_t)byte_of(w, 1) * dv;
        y.z = (float)(int8_t)byte_of(w, 2) * dv;
        y.w = (float)(int8_t)byte_of(w, 3) * dv;
        *(float4 *)(out + r * (size_t)K + c) = y;
    }
}

__global__ void __launch_bounds__(256) k_dequant_q4_k(const uint8_t *__restrict__ W, size_t row_bytes, int K,
                                                      uint32_t row0, const uint32_t *__restrict__ ids, uint32_t nrows,
                                                      float *__restrict__ out) {
    // one thread per (row, sub-block of 32, group of 8 values)
    const size_t per_row = (size_t)K / 8, total = (size_t)nrows * per_row;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / per_row, v0 = (i % per_row) * 8;
        const size_t row = ids ? (size_t)ids[r] : row0 + r;
        const uint8_t *b = W + row * row_bytes + (v0 / 256) * 144;
        const int sub = (int)((v0 % 256) / 32), l0 = (int)(v0 % 32);
        const u4v hdr = *(const u4v *)b;
        uint32_t sw0, sw1, mw0, mw1;
        q4k_scale_words(hdr.y, hdr.z, hdr.w, sw0, sw1, mw0, mw1);
        const uint32_t s = byte_of(sub < 4 ? sw0 : sw1, sub & 3), m = byte_of(sub < 4 ? mw0 : mw1, sub & 3);
        const float ds = h2f((uint16_t)hdr.x) * (float)s, dm = h2f((uint16_t)(hdr.x >> 16)) * (float)m;
        const u2v q = *(const u2v *)(b + 16 + 32 * (sub >> 1) + l0);
        const int shift = (sub & 1) ? 4 : 0;
        float y[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t qq = (((j < 4 ? q.x : q.y) >> (8 * (j & 3))) >> shift) & 0xfu;
            y[j] = ds * (float)qq - dm;
        }
        float4 *o = (float4 *)(out + r * (size_t)K + v0);
        o[0] = float4{y[0], y[1], y[2], y[3]};
        o[1] = float4{y[4], y[5], y[6], y[7]};
    }
}

// ============================================================================ GEMV (M = 1) / gather
// LPR lanes per weight row (16, 32 or 64: chosen so the grid covers every CU), 256 / LPR rows per
// workgroup. Lane j of a row walks 16-byte chunks j, j + LPR, ... of the row's quant bytes, four
// chunks per batch with all loads issued before any use (memory-level parallelism), and keeps an
// fp32 partial; an LPR-lane butterfly reduces it. Quants become exact fp16 integers (v_perm_b32 under
// 0x64, then subtract the 1024 / 1152 bias) and meet the fp16 activations in v_dot2_f32_f16, so
// every product is exact and every sum is fp32.
template <int LPR>
DEV float row_sum(float v) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, LPR);
    return v;
}

DEV u4v load16(const void *p) { return *(const u4v *)p; }

// Q8_0 row dot: chunk c = 16 values of block c/2 (biased bytes u = q + 128, d plane).
template <int LPR>
DEV float dot_row_q8_0(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ d, const uint16_t *__restrict__ a,
                       int K, int j) {
    const int nch = K / 16;
    const h2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    float acc = 0.f;
    for (int c0 = j; c0 < nch; c0 += 4 * LPR) {
        u4v q[4], a0[4], a1[4];
        float dv[4];
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int c = c0 + b * LPR, cc = c < nch ? c : nch - 1;
            q[b] = load16(qs + 16 * cc);
            a0[b] = load16(a + 16 * cc);
            a1[b] = load16(a + 16 * cc + 8);
            dv[b] = c < nch ? h2f(d[cc >> 1]) : 0.f;
        }
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t w[4] = {q[b].x, q[b].y, q[b].z, q[b].w};
            h2 lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                lo[2 * i] = as_h2(perm_lo(w[i])) + bias;
                lo[2 * i + 1] = as_h2(perm_hi(w[i])) + bias;
                hi[2 * i] = as_h2(perm_lo(w[2 + i])) + bias;
                hi[2 * i + 1] = as_h2(perm_hi(w[2 + i])) + bias;
            }
            const float s = dot8(hi, a1[b], dot8(lo, a0[b], 0.f));
            acc += s * dv[b];
        }
    }
    return acc;
}

// Q4_K row dot. Chunk c = 16 bytes of qs of super-block c/8: part t = c%8 -> p = t/2, h = t%2;
// low nibbles are values 64p+16h+i (sub 2p), high nibbles 64p+32+16h+i (sub 2p+1).
template <int LPR>
DEV float dot_row_q4_k(const uint8_t *__restrict__ row, const uint16_t *__restrict__ a, int K, int j) {
    const int nch = K / 32;
    const h2 k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const h2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f}, k64 = {(_Float16)-64.0f, (_Float16)-64.0f};
    float acc = 0.f;
    for (int c0 = j; c0 < nch; c0 += 4 * LPR) {
        u4v hd[4], q[4], al0[4], al1[4], ah0[4], ah1[4];
        bool ok[4];
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int c = c0 + b * LPR, cc = c < nch ? c : nch - 1;
            ok[b] = c < nch;
            const uint8_t *blk = row + (size_t)(cc >> 3) * 144;
            const int t = cc & 7;
            hd[b] = load16(blk);
            q[b] = load16(blk + 16 + 16 * t);
            const int kb = (cc >> 3) * 256 + 64 * (t >> 1) + 16 * (t & 1);
            al0[b] = load16(a + kb);
            al1[b] = load16(a + kb + 8);
            ah0[b] = load16(a + kb + 32);
            ah1[b] = load16(a + kb + 40);
        }
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int t = ((c0 + b * LPR) & 7), p = t >> 1;
            uint32_t sw0, sw1, mw0, mw1;
            q4k_scale_words(hd[b].y, hd[b].z, hd[b].w, sw0, sw1, mw0, mw1);
            const int s0 = 2 * p, s1 = 2 * p + 1;
            const float d = h2f((uint16_t)hd[b].x), dmin = h2f((uint16_t)(hd[b].x >> 16));
            const float ds0 = d * (float)byte_of(s0 < 4 ? sw0 : sw1, s0 & 3);
            const float ds1 = d * (float)byte_of(s1 < 4 ? sw0 : sw1, s1 & 3);
            const float dm0 = dmin * (float)byte_of(s0 < 4 ? mw0 : mw1, s0 & 3);
            const float dm1 = dmin * (float)byte_of(s1 < 4 ? mw0 : mw1, s1 & 3);
            const uint32_t w[4] = {q[b].x, q[b].y, q[b].z, q[b].w};
            h2 l0[4], l1[4], g0[4], g1[4];  // low nibbles of bytes 0-7 / 8-15, high nibbles of bytes 0-7 / 8-15
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t x = (i & 1) ? perm_hi(w[i >> 1]) : perm_lo(w[i >> 1]);
                const uint32_t y = (i & 1) ? perm_hi(w[2 + (i >> 1)]) : perm_lo(w[2 + (i >> 1)]);
                l0[i] = as_h2(x & 0xff0fff0fu) + k1024;
                l1[i] = as_h2(y & 0xff0fff0fu) + k1024;
                g0[i] = __builtin_elementwise_fma(as_h2(x & 0xfff0fff0u), s16, k64);
                g1[i] = __builtin_elementwise_fma(as_h2(y & 0xfff0fff0u), s16, k64);
            }
            const float ql = dot8(l1, al1[b], dot8(l0, al0[b], 0.f));
            const float qh = dot8(g1, ah1[b], dot8(g0, ah0[b], 0.f));
            const float sl = sum8(al1[b], sum8(al0[b], 0.f)), sh = sum8(ah1[b], sum8(ah0[b], 0.f));
            const float v = (ds0 * ql - dm0 * sl) + (ds1 * qh - dm1 * sh);
            acc += ok[b] ? v : 0.f;
        }
    }
    return acc;
}


// ---- row-group GEMV: one wave per R weight rows (64 lanes per row), activations loaded once per
// slice into registers and reused by the R rows, all R x TS weight loads of a slice in flight together.
constexpr int GV_TS = 2;  // 16-byte chunks per lane per K slice

// Q8_0: R rows n0 .. n0+R-1 (clamped) against activation vector a; returns the lane's partials.
template <int R>
DEV void rows_q8_0(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ d, int ldd,
                   const uint16_t *__restrict__ a, int K, const int (&n)[R], int j, float (&acc)[R]) {
    const int nch = K / 16;
    const h2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    for (int c0 = j; c0 < nch; c0 += 64 * GV_TS) {
        u4v a0[GV_TS], a1[GV_TS], q[R][GV_TS];
        float dv[R][GV_TS];
#pragma unroll
        for (int t = 0; t < GV_TS; t++) {
            const int c = c0 + 64 * t, cc = c < nch ? c : nch - 1;
            a0[t] = load16(a + 16 * cc);
            a1[t] = load16(a + 16 * cc + 8);
#pragma unroll
            for (int r = 0; r < R; r++) {
                q[r][t] = load16(qs + (size_t)n[r] * K + 16 * cc);
                dv[r][t] = c < nch ? h2f(d[(size_t)n[r] * ldd + (cc >> 1)]) : 0.f;
            }
        }
#pragma unroll
        for (int t = 0; t < GV_TS; t++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t w[4] = {q[r][t].x, q[r][t].y, q[r][t].z, q[r][t].w};
                h2 lo[4], hi[4];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    lo[2 * i] = as_h2(perm_lo(w[i])) + bias;
                    lo[2 * i + 1] = as_h2(perm_hi(w[i])) + bias;
                    hi[2 * i] = as_h2(perm_lo(w[2 + i])) + bias;
                    hi[2 * i + 1] = as_h2(perm_hi(w[2 + i])) + bias;
                }
                acc[r] += dot8(hi, a1[t], dot8(lo, a0[t], 0.f)) * dv[r][t];
            }
    }
}

// Q4_K: chunk c = 16 bytes of qs of super-block c/8 (32 values, see dot_row_q4_k).
template <int R>
DEV void rows_q4_k(const uint8_t *__restrict__ W, size_t row_bytes, const uint16_t *__restrict__ a, int K,
                   const int (&n)[R], int j, float (&acc)[R]) {
    const int nch = K / 32;
    const h2 k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const h2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f}, k64 = {(_Float16)-64.0f, (_Float16)-64.0f};
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    for (int c0 = j; c0 < nch; c0 += 64 * GV_TS) {
        u4v al0[GV_TS], al1[GV_TS], ah0[GV_TS], ah1[GV_TS], hd[R][GV_TS], q[R][GV_TS];
#pragma unroll
        for (int t = 0; t < GV_TS; t++) {
            const int c = c0 + 64 * t, cc = c < nch ? c : nch - 1, tt = cc & 7;
            const int kb = (cc >> 3) * 256 + 64 * (tt >> 1) + 16 * (tt & 1);
            al0[t] = load16(a + kb);
            al1[t] = load16(a + kb + 8);
            ah0[t] = load16(a + kb + 32);
            ah1[t] = load16(a + kb + 40);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint8_t *blk = W + (size_t)n[r] * row_bytes + (size_t)(cc >> 3) * 144;
                hd[r][t] = load16(blk);
                q[r][t] = load16(blk + 16 + 16 * tt);
            }
        }
#pragma unroll
        for (int t = 0; t < GV_TS; t++) {
            const int c = c0 + 64 * t, tt = c & 7, p = tt >> 1;
            const float sl = sum8(al1[t], sum8(al0[t], 0.f)), sh = sum8(ah1[t], sum8(ah0[t], 0.f));
#pragma unroll
            for (int r = 0; r < R; r++) {
                uint32_t sw0, sw1, mw0, mw1;
                q4k_scale_words(hd[r][t].y, hd[r][t].z, hd[r][t].w, sw0, sw1, mw0, mw1);
                const int s0 = 2 * p, s1 = 2 * p + 1;
                const float dd = h2f((uint16_t)hd[r][t].x), dmin = h2f((uint16_t)(hd[r][t].x >> 16));
                const float ds0 = dd * (float)byte_of(s0 < 4 ? sw0 : sw1, s0 & 3);
                const float ds1 = dd * (float)byte_of(s1 < 4 ? sw0 : sw1, s1 & 3);
                const float dm0 = dmin * (float)byte_of(s0 < 4 ? mw0 : mw1, s0 & 3);
                const float dm1 = dmin * (float)byte_of(s1 < 4 ? mw0 : mw1, s1 & 3);
                const uint32_t w[4] = {q[r][t].x, q[r][t].y, q[r][t].z, q[r][t].w};
                h2 l0[4], l1[4], g0[4], g1[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t x = (i & 1) ? perm_hi(w[i >> 1]) : perm_lo(w[i >> 1]);
                    const uint32_t y = (i & 1) ? perm_hi(w[2 + (i >> 1)]) : perm_lo(w[2 + (i >> 1)]);
                    l0[i] = as_h2(x & 0xff0fff0fu) + k1024;
                    l1[i] = as_h2(y & 0xff0fff0fu) + k1024;
                    g0[i] = __builtin_elementwise_fma(as_h2(x & 0xfff0fff0u), s16, k64);
                    g1[i] = __builtin_elementwise_fma(as_h2(y & 0xfff0fff0u), s16, k64);
                }
                const float ql = dot8(l1, al1[t], dot8(l0, al0[t], 0.f));
                const float qh = dot8(g1, ah1[t], dot8(g0, ah0[t], 0.f));
                const float v = (ds0 * ql - dm0 * sl) + (ds1 * qh - dm1 * sh);
                acc[r] += c < nch ? v : 0.f;
            }
        }
    }
}

// ---- Q4_K GEMV (M = 1) through LDS: a workgroup owns R consecutive weight rows, which are one
// contiguous byte range of W. It copies that slab and the activation vector into LDS with 16-byte
// LDS DMAs (1 KB per wave instruction, fully coalesced, no registers), forms the 32-value sub-block
// sums of the activations, then every lane dots units of 64 values (one 32-byte quant group p of a
// super-block: low nibbles = sub-block 2p, high nibbles = sub-block 2p + 1) from LDS. Lane tid
// always works on row tid % R (R divides 256), so its partial sums stay in one register; the R
// row totals are reduced across lanes and waves in a fixed order. Units: gemv_unit_q4_k (one
// super-block header read and one scale decode per 64 values).
template <int R>
__global__ void __launch_bounds__(256) k_gemv_q4_k_s(const uint8_t *__restrict__ W, uint32_t row_bytes,
                                                     const uint16_t *__restrict__ a, int N, int K, void *C, int c_f32,
                                                     int accumulate) {
    extern __shared__ __attribute__((aligned(16))) char gs_lds[];
    const uint32_t slab_bytes = (uint32_t)R * row_bytes, act_bytes = 2u * (uint32_t)K;
    char *const slab = gs_lds;
    char *const sa = gs_lds + slab_bytes;
    float *const ss = (float *)(sa + act_bytes);  // K / 32 sub-block sums
    float *const red = ss + K / 32;               // [4 waves][R] row partials
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const rsrc_t ra = make_rsrc(a, act_bytes);
    const rsrc_t rw = make_rsrc(W, (uint32_t)N * row_bytes);  // rows >= N read as zero
    for (uint32_t o = 1024u * wave; o < act_bytes; o += 4096u)
        if (o + 16u * lane < act_bytes) dma16(ra, sa + o, o + 16u * lane, 0);
    const uint32_t base = (uint32_t)blockIdx.x * slab_bytes;
    for (uint32_t o = 1024u * wave; o < slab_bytes; o += 4096u)
        if (o + 16u * lane < slab_bytes) dma16(rw, slab + o, base + o + 16u * lane, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int i = tid; i < K / 32; i += 256) {
        const u4v *p = (const u4v *)(sa + 64 * i);
        ss[i] = sum8(p[3], sum8(p[2], sum8(p[1], sum8(p[0], 0.f))));
    }
    __syncthreads();
    const int r = tid % R, units = R * (K / 64);
    const char *const row = slab + r * row_bytes;
    float acc = 0.f;
    for (int u = tid; u < units; u += 256) {
        const int ku = u / R;
        acc += gemv_unit_q4_k(row + (ku >> 2) * 144, ku & 3, sa, ss, ku);
    }
#pragma unroll
    for (int o = R; o < 64; o <<= 1) acc += __shfl_xor(acc, o, 64);
    if (lane < R) red[wave * R + lane] = acc;
    __syncthreads();
    const int n = blockIdx.x * R + tid;
    if (tid < R && n < N) store_out(C, n, ((red[tid] + red[R + tid]) + red[2 * R + tid]) + red[3 * R + tid], c_f32, accumulate);
}

// ---- Q4_K GEMV (M = 1), streamed: a workgroup owns 8 weight rows; its S waves split the row's
// super-block pairs into S contiguous ranges. A wave streams its range through a ring of NS LDS
// slots, one stage = one super-block pair of the 8 rows (8 x 288 bytes, three 1 KB LDS DMAs whose
// lanes gather the 8 row pieces), NS stages in flight: it waits for the oldest stage with
// s_waitcnt vmcnt, decodes it while the younger stages land, then refills the slot. In a stage,
// lane (row = lane / 8, j = lane % 8) takes the unit j = 32-byte quant group j % 4 of super-block
// j / 4 (64 values: low nibbles sub-block 2p, high nibbles 2p + 1), dotted by gemv_unit_q4_k.
// The activations and their 32-value sub-block sums are staged once per workgroup. Row totals:
// 8-lane butterfly, then the S wave partials in wave order. Needs an even number of super-blocks
// per row.
constexpr int GVR_SLOT = 8 * 288;

template <int NS>
__global__ void __launch_bounds__(256) k_gemv_q4_k_r(const uint8_t *__restrict__ W, uint32_t row_bytes,
                                                     const uint16_t *__restrict__ a, int N, int K, void *C, int c_f32,
                                                     int accumulate) {
    extern __shared__ __attribute__((aligned(16))) char gr_lds[];
    const int tid = threadIdx.x, lane = tid & 63, S = (int)blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar control flow
    const uint32_t act_bytes = 2u * (uint32_t)K;
    char *const sa = gr_lds;
    float *const ss = (float *)(gr_lds + act_bytes);  // K / 32 sub-block sums
    float *const red = ss + K / 32;                   // [S][8] wave partials
    char *const ring = (char *)(red + 8 * S) + (size_t)wave * NS * GVR_SLOT;
    const uint32_t lds0 = (uint32_t)(uintptr_t)gr_lds;
    const rsrc_t ra = make_rsrc(a, act_bytes);
    const rsrc_t rw = make_rsrc(W, (uint32_t)N * row_bytes);  // rows >= N read as zero
    const int n0 = blockIdx.x * 8, pairs = K / 512;
    const int pr0 = wave * pairs / S, nst = (wave + 1) * pairs / S - pr0;
    // this lane's gather offsets for the three DMA instructions of a stage (lane l = 64 q + lane of
    // the stage: row l / 18, 16-byte piece l % 18)
    uint32_t dvo[3];
#pragma unroll
    for (int q = 0; q < 3; q++) {
        const int l = 64 * q + lane, row = l / 18, piece = l % 18;
        dvo[q] = (uint32_t)(n0 + row) * row_bytes + 16u * (uint32_t)piece;
    }
    const uint32_t ring_addr = (uint32_t)(uintptr_t)ring;
    auto issue = [&](int st) {
        const uint32_t slot = ring_addr + (uint32_t)(st % NS) * GVR_SLOT, off = (uint32_t)(pr0 + st) * 288u;
        dma16_untracked(rw, slot, dvo[0] + off);
        dma16_untracked(rw, slot + 1024u, dvo[1] + off);
        if (lane < 16) dma16_untracked(rw, slot + 2048u, dvo[2] + off);
    };
    // activations (this wave's share of the 1 KB pieces), then the first NS stages
    int nact = 0;
    for (uint32_t o = 1024u * wave; o < act_bytes; o += 1024u * S, nact++)
        if (o + 16u * lane < act_bytes) dma16_untracked(ra, lds0 + o, o + 16u * lane);
    const int pre = nst < NS ? nst : NS;
    for (int st = 0; st < pre; st++) issue(st);
    wait_vmcnt(3 * pre);
    __syncthreads();
    for (int i = tid; i < K / 32; i += 64 * S) {
        const u4v *p = (const u4v *)(sa + 64 * i);
        ss[i] = sum8(p[3], sum8(p[2], sum8(p[1], sum8(p[0], 0.f))));
    }
    __syncthreads();
    const int row = lane >> 3, j = lane & 7, p = j & 3;
    const uint32_t unit_off = (uint32_t)row * 288u + (uint32_t)(j >> 2) * 144u;
    float acc = 0.f;
    for (int st = 0; st < nst; st++) {
        const int ahead = (nst - st - 1 < NS - 1) ? nst - st - 1 : NS - 1;
        wait_vmcnt(3 * ahead);  // stage st has landed
        acc += gemv_unit_q4_k(ring + (st % NS) * GVR_SLOT + unit_off, p, sa, ss, 4 * (2 * (pr0 + st) + (j >> 2)) + p);
        if (st + NS < nst) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this slot's reads are done
            issue(st + NS);
        }
    }
    acc += __shfl_xor(acc, 1, 64);
    acc += __shfl_xor(acc, 2, 64);
    acc += __shfl_xor(acc, 4, 64);
    if (S == 1) {
        if (j == 0 && n0 + row < N) store_out(C, n0 + row, acc, c_f32, accumulate);
        return;
    }
    if (j == 0) red[wave * 8 + row] = acc;
    __syncthreads();
    if (tid < 8 && n0 + tid < N) {
        float v = red[tid];
        for (int w = 1; w < S; w++) v += red[w * 8 + tid];
        store_out(C, n0 + tid, v, c_f32, accumulate);
    }
}

// out row n (wave-uniform) of the R rows of this wave.
template <int R>
__global__ void __launch_bounds__(256) k_gemv_q8_0(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ d,
                                                   int ldd, const uint16_t *__restrict__ a, int N, int K, void *C,
                                                   int c_f32, int accumulate) {
    const int j = threadIdx.x & 63, n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    int n[R];
#pragma unroll
    for (int r = 0; r < R; r++) n[r] = n0 + r < N ? n0 + r : N - 1;
    float acc[R];
    rows_q8_0<R>(qs, d, ldd, a, K, n, j, acc);
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = row_sum<64>(acc[r]);
        if (j == 0 && n0 + r < N) store_out(C, n0 + r, v, c_f32, accumulate);
    }
}

template <int R>
__global__ void __launch_bounds__(256) k_gemv_q4_k(const uint8_t *__restrict__ W, size_t row_bytes,
                                                   const uint16_t *__restrict__ a, int N, int K, void *C, int c_f32,
                                                   int accumulate) {
    const int j = threadIdx.x & 63, n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    int n[R];
#pragma unroll
    for (int r = 0; r < R; r++) n[r] = n0 + r < N ? n0 + r : N - 1;
    float acc[R];
    rows_q4_k<R>(W, row_bytes, a, K, n, j, acc);
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = row_sum<64>(acc[r]);
        if (j == 0 && n0 + r < N) store_out(C, n0 + r, v, c_f32, accumulate);
    }
}

// out[i] = dot(H[i / k], W[ids[i]]) for i < pairs. An id >= rows reads row 0 and stores NaN, so a
// bad id can never move a load outside the matrix.
template <int LPR>
__global__ void __launch_bounds__(256) k_gather_q8_0(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ d,
                                                     int ldd, const uint16_t *__restrict__ H,
                                                     const uint32_t *__restrict__ ids, int pairs, int k, int K,
                                                     uint32_t rows, float *__restrict__ out) {
    const int i = blockIdx.x * (256 / LPR) + (int)threadIdx.x / LPR, j = threadIdx.x % LPR;
    const int ic = i < pairs ? i : pairs - 1;
    const uint32_t id = ids[ic];
    const size_t r = id < rows ? id : 0;
    const float v = row_sum<LPR>(dot_row_q8_0<LPR>(qs + r * K, d + r * ldd, H + (size_t)(ic / k) * K, K, j));
    if (j == 0 && i < pairs) out[i] = id < rows ? v : __builtin_nanf("");
}

template <int LPR>
__global__ void __launch_bounds__(256) k_gather_q4_k(const uint8_t *__restrict__ W, size_t row_bytes,
                                                     const uint16_t *__restrict__ H, const uint32_t *__restrict__ ids,
                                                     int pairs, int k, int K, uint32_t rows, float *__restrict__ out) {
    const int i = blockIdx.x * (256 / LPR) + (int)threadIdx.x / LPR, j = threadIdx.x % LPR;
    const int ic = i < pairs ? i : pairs - 1;
    const uint32_t id = ids[ic];
    const size_t r = id < rows ? id : 0;
    const float v = row_sum<LPR>(dot_row_q4_k<LPR>(W + r * row_bytes, H + (size_t)(ic / k) * K, K, j));
    if (j == 0 && i < pairs) out[i] = id < rows ? v : __builtin_nanf("");
}

#include "hq_sk.h"

template <int MB, int NB>
__global__ void __launch_bounds__(256) k_gemm_q8_0(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) _Float16 sa[2][16 * MB * KC];
    __shared__ int s_flag;
    const SkPlan &p = g.plan;
    const int w = sk_worker(p.G), u0 = sk_start(p, w), u1 = sk_start(p, w + 1);
    const rsrc_t rpart = make_rsrc(g.partials, g.partial_bytes);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ln = lane & 15, lg = lane >> 4;
    const int M = g.M, N = g.N, K = g.K;
    const rsrc_t ra = make_rsrc(g.A, (uint32_t)((size_t)M * K * 2));
    const rsrc_t rq = make_rsrc(g.qs, (uint32_t)((size_t)N * K));
    const rsrc_t rd = make_rsrc(g.d, (uint32_t)((size_t)N * g.ldd * 2));
    // per-tile lane offsets: rows beyond N read zero weights
    ADma adma;
    uint32_t vq[NB], vd[NB];
    auto tile_setup = [&](int tile) {
        const int m0 = (tile % p.tm) * 16 * MB, nw = (tile / p.tm) * 64 * NB + wave * 16 * NB;
        adma = adma_setup<MB>(K, m0);
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const uint32_t n = (uint32_t)(nw + 16 * j + ln);
            vq[j] = n * (uint32_t)K + 16u * lg;
            vd[j] = n * (uint32_t)g.ldd * 2u;
        }
    };
    // lane (ln, lg) holds weights [64s + 16lg, +16) of the unit for s = 0..3 and its 8 block scales
    auto load_w = [&](int k0, u4v (&q)[NB][4], u4v (&d)[NB]) {
#pragma unroll
        for (int j = 0; j < NB; j++) {
            d[j] = buf_load16(rd, vd[j], (uint32_t)(k0 / 16));
#pragma unroll
            for (int s = 0; s < 4; s++) q[j][s] = buf_load16(rq, vq[j] + 64u * s, (uint32_t)k0);
        }
    };
    f4 acc[MB][NB];
    u4v qc[NB][4], dc[NB];
    int cur_tile = u0 / p.upt;
    tile_setup(cur_tile);
    dma_a<MB>(sa[0], ra, adma, K, (u0 % p.upt) * KC);
    load_w((u0 % p.upt) * KC, qc, dc);
    for (int u = u0; u < u1; u++) {
        const int cb = (u - u0) & 1, tile = u / p.upt, ku = u % p.upt;
        const int m0 = (tile % p.tm) * 16 * MB, nw = (tile / p.tm) * 64 * NB + wave * 16 * NB;
        const int k0 = ku * KC, kc = K - k0 < KC ? K - k0 : KC;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        u4v qn[NB][4], dn[NB];
        if (u + 1 < u1) {
            const int t1 = (u + 1) / p.upt;
            if (t1 != cur_tile) {
                cur_tile = t1;
                tile_setup(t1);
            }
            const int k1 = ((u + 1) % p.upt) * KC;
            dma_a<MB>(sa[cb ^ 1], ra, adma, K, k1);
            load_w(k1, qn, dn);
        }
        if (u == u0 || ku == 0) {
#pragma unroll
            for (int i = 0; i < MB; i++)
#pragma unroll
                for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
        }
        // decode: bf[j][2s + t] covers activations 64s + 16lg + 8t .. +8 (chunk index 8s + 2lg + t);
        // pieces past the end of K (last unit of a row only) get a zero scale
        h8 bf[NB][8];
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const uint32_t dw[4] = {dc[j].x, dc[j].y, dc[j].z, dc[j].w};
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const int blk = 2 * s + (lg >> 1);  // block of this lane's 16 weights
                const uint32_t dd = dw[blk >> 1] >> (16 * (blk & 1));
                const int valid = 64 * s + 16 * lg < kc;
                const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)(valid ? dd : 0u));
                const h2 d2 = {dh, dh};
                bf[j][2 * s] = frag_q8_0(qc[j][s].x, qc[j][s].y, d2);
                bf[j][2 * s + 1] = frag_q8_0(qc[j][s].z, qc[j][s].w, d2);
            }
        }
        const _Float16 *buf = sa[cb];
#pragma unroll
        for (int i = 0; i < MB; i++) {
            const int r = 16 * i + ln;
#pragma unroll
            for (int f = 0; f < 8; f++) {
                const h8 af = a_frag(buf, r, 8 * (f >> 1) + 2 * lg + (f & 1));
#pragma unroll
                for (int j = 0; j < NB; j++) acc[i][j] = mfma(af, bf[j][f], acc[i][j]);
            }
        }
        if (ku == p.upt - 1 || u == u1 - 1)
            finish_tile<MB, NB, 256>(acc, p, w, u0, u1, tile, &s_flag, rpart, g.counters, g.C, M, N, m0, nw, ln, lg,
                                g.c_f32, g.accumulate);
        if (u + 1 < u1) {
#pragma unroll
            for (int j = 0; j < NB; j++) {
                dc[j] = dn[j];
#pragma unroll
                for (int s = 0; s < 4; s++) qc[j][s] = qn[j][s];
            }
        }
    }
}

template <int MB, int NB>
__global__ void __launch_bounds__(256) k_gemm_q4_k(GemmArgs g) {
    constexpr int BM = 16 * MB;
    __shared__ __attribute__((aligned(16))) _Float16 sa[2][BM * KC];
    __shared__ __attribute__((aligned(16))) _Float16 ss[2][BM * 16];  // per row: sums hi[8], lo[8]
    __shared__ int s_flag;
    const SkPlan &p = g.plan;
    const int w = sk_worker(p.G), u0 = sk_start(p, w), u1 = sk_start(p, w + 1);
    const rsrc_t rpart = make_rsrc(g.partials, g.partial_bytes);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
    const int M = g.M, N = g.N, K = g.K;
    const rsrc_t ra = make_rsrc(g.A, (uint32_t)((size_t)M * K * 2));
    const rsrc_t rw = make_rsrc(g.qs, (uint32_t)((size_t)N * g.row_bytes));
    ADma adma;
    uint32_t vh[NB], vq[NB];
    // Lane (ln, lg) loads chunk c = 4L + lg (L = 0, 1) of the 128 quant bytes: p = 2L + lg/2,
    // h = lg%2. MFMA 4L + t: t = 0/1 low nibbles of bytes 0-7 / 8-15, t = 2/3 high nibbles; its
    // activations start at k = 64p + 16h + 8(t&1) + 32(t>>1) (chunk k/8); sub-block 2p + (t>>1).
    auto tile_setup = [&](int tile) {
        const int m0 = (tile % p.tm) * BM, nw = (tile / p.tm) * 64 * NB + wave * 16 * NB;
        adma = adma_setup<MB>(K, m0);
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const uint32_t n = (uint32_t)(nw + 16 * j + ln);
            vh[j] = n * (uint32_t)g.row_bytes;
            vq[j] = vh[j] + 16u + 16u * lg;
        }
    };
    auto load_w = [&](int sb, u4v (&h)[NB], u4v (&q0)[NB], u4v (&q1)[NB]) {
        const uint32_t so = (uint32_t)sb * 144u;
#pragma unroll
        for (int j = 0; j < NB; j++) {
            h[j] = buf_load16(rw, vh[j], so);
            q0[j] = buf_load16(rw, vq[j], so);
            q1[j] = buf_load16(rw, vq[j] + 64u, so);
        }
    };
    const int pA = lg >> 1, hA = lg & 1;
    f4 acc[MB][NB];
    u4v hc[NB], q0c[NB], q1c[NB];
    // min term deferred from the previous unit: integer m operand and -dmin per column block
    h8 bm_prev[NB];
    float ndmin_prev[NB];
    bool min_pending = false;
    int cur_tile = u0 / p.upt;
    tile_setup(cur_tile);
    dma_a<MB>(sa[0], ra, adma, K, (u0 % p.upt) * KC);
    load_w(u0 % p.upt, hc, q0c, q1c);
    auto apply_min = [&](const _Float16 *sbuf) {
#pragma unroll
        for (int i = 0; i < MB; i++) {
            // lanes lg even: sums hi, odd: lo (lanes lg >= 2 meet a zero B operand)
            const h8 as = *(const h8 *)(sbuf + (16 * i + ln) * 16 + 8 * (lg & 1));
#pragma unroll
            for (int j = 0; j < NB; j++) {
                const f4 mp = mfma(as, bm_prev[j], f4{0.f, 0.f, 0.f, 0.f});
                acc[i][j] += mp * ndmin_prev[j];
            }
        }
    };
    for (int u = u0; u < u1; u++) {
        const int cb = (u - u0) & 1, tile = u / p.upt, sb = u % p.upt;
        const int m0 = (tile % p.tm) * BM, nw = (tile / p.tm) * 64 * NB + wave * 16 * NB;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (min_pending) {  // the previous unit of this tile: its sums are complete now
            apply_min(ss[cb ^ 1]);
            min_pending = false;
        }
        u4v hn[NB], q0n[NB], q1n[NB];
        if (u + 1 < u1) {
            const int t1 = (u + 1) / p.upt;
            if (t1 != cur_tile) {
                cur_tile = t1;
                tile_setup(t1);
            }
            const int sb1 = (u + 1) % p.upt;
            dma_a<MB>(sa[cb ^ 1], ra, adma, K, sb1 * KC);
            load_w(sb1, hn, q0n, q1n);
        }
        if (u == u0 || sb == 0) {
#pragma unroll
            for (int i = 0; i < MB; i++)
#pragma unroll
                for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
        }
        const _Float16 *buf = sa[cb];
        // sub-block sums of this unit: thread -> (row, sub) pairs, rows fastest (conflict-free reads)
        {
            const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
            for (int q = 0; q < (BM * 8 + 255) / 256; q++) {
                const int pr = tid + 256 * q;
                if ((BM * 8) % 256 == 0 || pr < BM * 8) {
                    const int r = pr % BM, sub = pr / BM;
                    float s = 0.f;
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const u4v x = *(const u4v *)(buf + r * KC + 8 * ((4 * sub + v) ^ (r & 15)));
                        s = __builtin_amdgcn_fdot2(as_h2(x.x), one, s, false);
                        s = __builtin_amdgcn_fdot2(as_h2(x.y), one, s, false);
                        s = __builtin_amdgcn_fdot2(as_h2(x.z), one, s, false);
                        s = __builtin_amdgcn_fdot2(as_h2(x.w), one, s, false);
                    }
                    const _Float16 hi = (_Float16)s;
                    ss[cb][r * 16 + sub] = hi;
                    ss[cb][r * 16 + 8 + sub] = (_Float16)(s - (float)hi);
                }
            }
        }
        h8 bf[NB][8];
        float dsc[NB];
#pragma unroll
        for (int j = 0; j < NB; j++) {
            uint32_t sw0, sw1, mw0, mw1;
            q4k_scale_words(hc[j].y, hc[j].z, hc[j].w, sw0, sw1, mw0, mw1);
            h2 mulL[2][2], addL[2][2];
#pragma unroll
            for (int L = 0; L < 2; L++) {
                const uint32_t sw = L ? sw1 : sw0;
#pragma unroll
                for (int hi = 0; hi < 2; hi++) {
                    const float s = (float)byte_of(sw, 2 * pA + hi);
                    const _Float16 mul = (_Float16)(hi ? s * 0.0625f : s);
                    const _Float16 add = (_Float16)(hi ? -64.0f * s : -1024.0f * s);
                    mulL[L][hi] = h2{mul, mul};
                    addL[L][hi] = h2{add, add};
                }
            }
            bf[j][0] = frag_q4_k<false>(q0c[j].x, q0c[j].y, mulL[0][0], addL[0][0]);
            bf[j][1] = frag_q4_k<false>(q0c[j].z, q0c[j].w, mulL[0][0], addL[0][0]);
            bf[j][2] = frag_q4_k<true>(q0c[j].x, q0c[j].y, mulL[0][1], addL[0][1]);
            bf[j][3] = frag_q4_k<true>(q0c[j].z, q0c[j].w, mulL[0][1], addL[0][1]);
            bf[j][4] = frag_q4_k<false>(q1c[j].x, q1c[j].y, mulL[1][0], addL[1][0]);
            bf[j][5] = frag_q4_k<false>(q1c[j].z, q1c[j].w, mulL[1][0], addL[1][0]);
            bf[j][6] = frag_q4_k<true>(q1c[j].x, q1c[j].y, mulL[1][1], addL[1][1]);
            bf[j][7] = frag_q4_k<true>(q1c[j].z, q1c[j].w, mulL[1][1], addL[1][1]);
            // min operand for the next barrier: lanes lg 0, 1 carry m_0..m_7 (k-slot e = sub-block e)
            const h2 m01 = bytes_f16(mw0, false), m23 = bytes_f16(mw0, true);
            const h2 m45 = bytes_f16(mw1, false), m67 = bytes_f16(mw1, true);
            const h8 mv = {m01.x, m01.y, m23.x, m23.y, m45.x, m45.y, m67.x, m67.y};
            bm_prev[j] = lg < 2 ? mv : h8{0, 0, 0, 0, 0, 0, 0, 0};
            ndmin_prev[j] = -h2f((uint16_t)(hc[j].x >> 16));
            dsc[j] = h2f((uint16_t)hc[j].x);
        }
#pragma unroll
        for (int i = 0; i < MB; i++) {
            const int r = 16 * i + ln;
            f4 part[NB];
#pragma unroll
            for (int j = 0; j < NB; j++) part[j] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int L = 0; L < 2; L++)
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const h8 af = a_frag(buf, r, 8 * (2 * L + pA) + 2 * hA + (t & 1) + 4 * (t >> 1));
#pragma unroll
                    for (int j = 0; j < NB; j++) part[j] = mfma(af, bf[j][4 * L + t], part[j]);
                }
#pragma unroll
            for (int j = 0; j < NB; j++) acc[i][j] += part[j] * dsc[j];
        }
        min_pending = true;
        if (sb == p.upt - 1 || u == u1 - 1) {
            __syncthreads();  // this unit's sums, written by other waves
            apply_min(ss[cb]);
            min_pending = false;
            finish_tile<MB, NB, 256>(acc, p, w, u0, u1, tile, &s_flag, rpart, g.counters, g.C, M, N, m0, nw, ln, lg,
                                g.c_f32, g.accumulate);
        }
        if (u + 1 < u1) {
#pragma unroll
            for (int j = 0; j < NB; j++) hc[j] = hn[j], q0c[j] = q0n[j], q1c[j] = q1n[j];
        }
    }
}

// ---------------------------------------------------------------------------- wide Q4_K GEMM (M > 64)
// 8 waves, two per SIMD (one wave's LDS and memory waits are covered by the other's MFMAs); tile
// 128 (M) x 256 (N): wave w owns columns [32w, 32w + 32) and all 128 rows, decoded as in
// k_gemm_q4_k. The activation sub-block sums come from k_asums (one pass over A per GEMM instead of
// one per N tile): plane S[m][u][16] fp16 = {hi(S_0..S_7), lo(S_0..S_7)} of unit u, staged in LDS
// next to the activation tile. The min term is one MFMA per (16-row block, 16-column block, unit)
// accumulating straight into the output: A operand lanes lg = 0..3 hold S_hi, S_lo, S_hi, S_lo of
// sub-blocks 0..7, B operand lanes hold Bh, Bh, Bl, Bl with Bh = fp16(-dmin*m) and
// Bl = fp16(-dmin*m - Bh), exact because -dmin*m has at most 17 significant bits; the four products
// sum to S*(-dmin*m) to about 2^-22 relative, so no fp32 fold is needed for it.
constexpr int WNW = 8;  // waves per workgroup

// A tile DMA: instruction q = w + 8qq (rows 2q, 2q + 1) of wave w; r & 15 = (2w + (lane >> 5)) & 15
// is the same for every qq, so one per-lane base serves all of them. The row step and k0 go into the
// VGPR offset (the one a buffer load range-checks), so rows past M read zeros.
DEV uint32_t adma_w_base(int K, int m0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, p = lane & 31;
    const int r0 = 2 * wave + (lane >> 5);
    return (uint32_t)((m0 + r0) * K + 8 * (p ^ (r0 & 15))) * 2u;
}

template <int MB>
DEV void dma_a_w(_Float16 *buf, rsrc_t ra, uint32_t base, int K, int k0) {
    constexpr int PER_WAVE = 16 * MB / 2 / WNW;
    static_assert(PER_WAVE * WNW * 2 == 16 * MB, "tile rows must split evenly over the waves");
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int qq = 0; qq < PER_WAVE; qq++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, lds_ptr(buf + (wave + WNW * qq) * 512), 16,
                                                 base + (uint32_t)(qq * 16 * K * 2 + 2 * k0), 0, 0, 0);
}

// Instruction qq of dma_a_w alone (the wide kernel spreads them over a unit's k-steps).
DEV void dma_a_w1(_Float16 *buf, rsrc_t ra, uint32_t base, int K, int k0, int qq) {
    const int wave = threadIdx.x >> 6;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, lds_ptr(buf + (wave + WNW * qq) * 512), 16,
                                             base + (uint32_t)(qq * 16 * K * 2 + 2 * k0), 0, 0, 0);
}

// S tile of unit u: 16*MB rows x 32 bytes, one 1 KB instruction (32 rows) per wave w < 16*MB/32.
// Per-lane base: row 32w + lane/2, half lane % 2.
template <int MB>
DEV void dma_s_w(uint16_t *buf, rsrc_t rs, uint32_t base, int u) {
    constexpr int INSTR = 16 * MB / 32;
    const int wave = threadIdx.x >> 6;
    if (wave < INSTR)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, lds_ptr(buf + wave * 512), 16, base, (uint32_t)(u * 32), 0, 0);
}

template <int MB>
__global__ void __launch_bounds__(512) k_gemm_q4_k_w(GemmArgs g) {
    constexpr int BM = 16 * MB, NB = 2, NT = 64 * WNW, BN = 16 * NB * WNW;
    static_assert(BM / 32 <= WNW, "S tile DMA needs one wave per 32 rows");
    __shared__ __attribute__((aligned(16))) _Float16 sa[2][BM * KC];
    __shared__ __attribute__((aligned(16))) uint16_t ssum[2][BM * 16];
    __shared__ uint32_t s_sink[64];  // target of the L2 warm-up loads (never read)
    __shared__ int s_flag;
    const SkPlan &p = g.plan;
    const int w = sk_worker(p.G), u0 = sk_start(p, w), u1 = sk_start(p, w + 1);
    const rsrc_t rpart = make_rsrc(g.partials, g.partial_bytes);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
    const int M = g.M, N = g.N, K = g.K, U = K / KC;
    const uint32_t rb = (uint32_t)g.row_bytes;
    const rsrc_t ra = make_rsrc(g.A, (uint32_t)((size_t)M * K * 2));
    const rsrc_t rw = make_rsrc(g.qs, (uint32_t)((size_t)N * g.row_bytes));
    const rsrc_t rs = make_rsrc(g.sums, (uint32_t)((size_t)M * U * 32));
    uint32_t abase = 0, sbase = 0, vh[NB];
    const uint32_t vqo = 16u + 16u * lg;  // quant chunk lg of this lane, after the 16-byte header
    auto tile_setup = [&](int tile) {
        const int m0 = (tile % p.tm) * BM, nw = (tile / p.tm) * BN + wave * 16 * NB;
        abase = adma_w_base(K, m0);
        sbase = (uint32_t)((m0 + 32 * wave + (lane >> 1)) * U * 32 + 16 * (lane & 1));
#pragma unroll
        for (int j = 0; j < NB; j++) vh[j] = (uint32_t)(nw + 16 * j + ln) * rb;
    };
    // Pull unit u's weight lines (BN columns x 144 bytes) into L2 ahead of the register loads:
    // thread pair (2c, 2c + 1) touches bytes {0, 143} and {72} of column c's super-block, which
    // covers every 128-byte line it spans. The bytes land in a scratch LDS word, not in registers.
    auto touch_w = [&](int u) {
        const int t = u / p.upt, sb = u % p.upt;
        const uint32_t off = (uint32_t)((t / p.tm) * BN + (tid >> 1)) * rb + (uint32_t)sb * 144u;
        const uint32_t o2 = (tid & 1) ? 72u : 0u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, lds_ptr(s_sink), 4, off + o2, 0, 0, 0);
        if (!(tid & 1)) __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, lds_ptr(s_sink), 4, off + 140u, 0, 0, 0);
    };
    const int pA = lg >> 1, hA = lg & 1;
    const uint32_t ssel = pA ? 0x04030402u : 0x04010400u;  // scale bytes (2pA, 2pA + 1) as fp16 1024 + s
    // A fragment (L, t) of this lane in row block 0 of a tile buffer: row ln, chunk
    // c = 8(2L + pA) + 2hA + (t & 1) + 4(t >> 1) at slot c ^ ln. The step bits (bits 0, 2, 4 of c)
    // are disjoint from the lane bits (8pA + 2hA), so slot = (8pA + 2hA) ^ ln ^ step bits and the
    // byte offset is arow + (xs ^ 16 * step bits); row block i adds 16*KC*2*i.
    const uint32_t arow = (uint32_t)(ln * KC * 2), xs = (uint32_t)(((8 * pA + 2 * hA) ^ ln) * 16);
    const uint32_t soff = (uint32_t)(ln * 16 + 8 * (lg & 1)) * 2u;
    f4 acc[MB][NB];
    // one register set of weights: the header, quant half 0 and quant half 1 of the next unit are
    // loaded into it as soon as the current unit has consumed each part
    u4v hc[NB], q0c[NB], q1c[NB];
    int cur_tile = u0 / p.upt;
    tile_setup(cur_tile);
    {
        const int sb = u0 % p.upt;
        dma_a_w<MB>(sa[0], ra, abase, K, sb * KC);
        dma_s_w<MB>(ssum[0], rs, sbase, sb);
#pragma unroll
        for (int j = 0; j < NB; j++) {
            hc[j] = buf_load16(rw, vh[j], (uint32_t)sb * 144u);
            q0c[j] = buf_load16(rw, vh[j] + vqo, (uint32_t)sb * 144u);
            q1c[j] = buf_load16(rw, vh[j] + vqo + 64u, (uint32_t)sb * 144u);
        }
        if (u0 + 1 < u1) touch_w(u0 + 1);
    }
    for (int u = u0; u < u1; u++) {
        const int cb = (u - u0) & 1, tile = u / p.upt, sb = u % p.upt;
        const int m0 = (tile % p.tm) * BM, nw = (tile / p.tm) * BN + wave * 16 * NB;
        // everything but the last NB loads (quant half 1 of this unit, waited for where it is
        // used) has arrived: this unit's activation and sum tiles are in LDS for all waves after
        // the barrier
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NB) : "memory");
        __syncthreads();
        const bool more = u + 1 < u1;
        const int sb1 = (u + 1) % p.upt;
        const uint32_t so1 = (uint32_t)sb1 * 144u;
        if (more) {
            const int t1 = (u + 1) / p.upt;
            if (t1 != cur_tile) {
                cur_tile = t1;
                tile_setup(t1);
            }
            dma_s_w<MB>(ssum[cb ^ 1], rs, sbase, sb1);
        }
        if (u == u0 || sb == 0) {
#pragma unroll
            for (int i = 0; i < MB; i++)
#pragma unroll
                for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
        }
        // per-unit constants. (x, y) = (low-nibble sub-block 4L + 2pA, high-nibble sub-block
        // 4L + 2pA + 1): the B fragment is fma(fp16(1024 + q), mul, add) with mul = (s, s/16) and
        // add = (-1024 s, -64 s); bmin is the min operand (k-slot e = sub-block e); dsc = d.
        h2 mulL[NB][2], addL[NB][2];
        h8 bmin[NB];
        float dsc[NB];
        const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
        const h2 kmul = {(_Float16)1.0f, (_Float16)0.0625f}, kadd = {(_Float16)-1024.0f, (_Float16)-64.0f};
#pragma unroll
        for (int j = 0; j < NB; j++) {
            uint32_t sw0, sw1, mw0, mw1;
            q4k_scale_words(hc[j].y, hc[j].z, hc[j].w, sw0, sw1, mw0, mw1);
#pragma unroll
            for (int L = 0; L < 2; L++) {
                const h2 sp = as_h2(__builtin_amdgcn_perm(0x64646464u, L ? sw1 : sw0, ssel)) - k1024;
                mulL[j][L] = sp * kmul;
                addL[j][L] = sp * kadd;
            }
            const _Float16 ndm = -__builtin_bit_cast(_Float16, (uint16_t)(hc[j].x >> 16));
            const h2 nd2 = {ndm, ndm};
            const h2 mv[4] = {bytes_f16(mw0, false), bytes_f16(mw0, true), bytes_f16(mw1, false),
                              bytes_f16(mw1, true)};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const h2 bh = mv[q] * nd2;
                const h2 bl = __builtin_elementwise_fma(mv[q], nd2, -bh);
                const h2 v = lg < 2 ? bh : bl;
                bmin[j][2 * q] = v.x;
                bmin[j][2 * q + 1] = v.y;
            }
            dsc[j] = h2f((uint16_t)hc[j].x);
        }
        // Loads for the unit after this one are issued unconditionally (no branch inside the
        // unit): past the workgroup's last unit they read in-bounds rows (or out-of-range zeros)
        // into registers and an LDS buffer that nothing reads again.
#pragma unroll
        for (int j = 0; j < NB; j++) hc[j] = buf_load16(rw, vh[j], so1);
        const uint32_t abuf = (uint32_t)(uintptr_t)sa[cb];
        const char *sbuf = (const char *)ssum[cb] + soff;
        // k-step outermost: step f's A fragments are read together, its two B fragments decoded,
        // then its 2*MB MFMAs issued
        f4 part[MB][NB];
#pragma unroll
        for (int f = 0; f < 8; f++) {
            const int L = f >> 2, t = f & 3;
            const uint32_t ad = abuf + arow + (xs ^ (uint32_t)(16 * ((t & 1) + 4 * (t >> 1) + 16 * L)));
            h8 af[MB];
#pragma unroll
            for (int i = 0; i < MB; i++) af[i] = *(const h8 *)(lds_void *)(uintptr_t)(ad + i * 16 * KC * 2);
            h8 bf[NB];
#pragma unroll
            for (int j = 0; j < NB; j++) {
                const u4v &q = L ? q1c[j] : q0c[j];
                const uint32_t w0 = (t & 1) ? q.z : q.x, w1 = (t & 1) ? q.w : q.y;
                const h2 mu = mulL[j][L], ad2 = addL[j][L];
                bf[j] = (t >> 1) ? frag_q4_k<true>(w0, w1, h2{mu.y, mu.y}, h2{ad2.y, ad2.y})
                                 : frag_q4_k<false>(w0, w1, h2{mu.x, mu.x}, h2{ad2.x, ad2.x});
            }
#pragma unroll
            for (int i = 0; i < MB; i++)
#pragma unroll
                for (int j = 0; j < NB; j++)
                    part[i][j] = mfma(af[i], bf[j], f == 0 ? f4{0.f, 0.f, 0.f, 0.f} : part[i][j]);
            // the next unit's activation tile streams in one instruction per step, so the memory
            // pipeline is not flooded right after the barrier
            static_assert(16 * MB / 2 / WNW == 8, "one DMA instruction per k-step");
            dma_a_w1(sa[cb ^ 1], ra, abase, K, sb1 * KC, f);
            if (f == 4) touch_w(u + 2);
            if (f == 3) {  // quant half 0 consumed: load the next unit's
#pragma unroll
                for (int j = 0; j < NB; j++) q0c[j] = buf_load16(rw, vh[j] + vqo, so1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < NB; j++) q1c[j] = buf_load16(rw, vh[j] + vqo + 64u, so1);
#pragma unroll
        for (int i = 0; i < MB; i++) {
            const h8 as = *(const h8 *)(sbuf + i * 16 * 32);
#pragma unroll
            for (int j = 0; j < NB; j++) acc[i][j] = mfma(as, bmin[j], acc[i][j]);
        }
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) acc[i][j] += part[i][j] * dsc[j];
        if (sb == p.upt - 1 || u == u1 - 1)
            finish_tile<MB, NB, NT>(acc, p, w, u0, u1, tile, &s_flag, rpart, g.counters, g.C, M, N, m0, nw, ln, lg,
                                    g.c_f32, g.accumulate);
    }
}

// Activation sub-block sums for the wide Q4_K GEMMs: S[m][u][s] = hi and S[m][u][8 + s] = lo of the
// fp32 sum of activations 256u + 32s .. +32 of row m, in fp16 (BF16 = false: the Stream-K kernel)
// or bf16 (the full-K tile kernel). One thread per sub-block (four 16-byte loads, 32-bit index math;
// M * K / 32 < 2^31 is checked by the launcher).
template <bool BF16>
__global__ void __launch_bounds__(256) k_asums(const uint16_t *__restrict__ A, int M, int K,
                                               uint16_t *__restrict__ S) {
    const uint32_t kb = (uint32_t)K / 32u, n = (uint32_t)M * kb;
    for (uint32_t t = blockIdx.x * 256u + threadIdx.x; t < n; t += gridDim.x * 256u) {
        const uint16_t *src = A + (size_t)t * 32;
        const u4v x0 = load16(src), x1 = load16(src + 8), x2 = load16(src + 16), x3 = load16(src + 24);
        const float v = sum8(x3, sum8(x2, sum8(x1, sum8(x0, 0.f))));
        const uint32_t m = t / kb, s = t - m * kb;
        uint16_t hb, lb;
        if constexpr (BF16) {
            const __bf16 hi = (__bf16)v;
            hb = __builtin_bit_cast(uint16_t, hi);
            lb = __builtin_bit_cast(uint16_t, (__bf16)(v - (float)hi));
        } else {
            const _Float16 hi = (_Float16)v;
            hb = __builtin_bit_cast(uint16_t, hi);
            lb = __builtin_bit_cast(uint16_t, (_Float16)(v - (float)hi));
        }
        // [M][K/256][hi x 8, lo x 8]
        uint16_t *dst = S + ((size_t)m * (kb / 8) + s / 8) * 16 + (s % 8);
        dst[0] = hb;
        dst[8] = lb;
    }
}

// ============================================================================ misc
__global__ void __launch_bounds__(256) k_f32_to_f16(const float *__restrict__ in, uint16_t *__restrict__ out,
                                                    size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = __builtin_bit_cast(uint16_t, (_Float16)in[i]);
}

// Diagnostic: a pure streaming read of n16 16-byte words (grid-stride, four loads in flight per lane),
// folded into one word per wave so nothing is dead: the floor one dispatch of that many bytes
// reaches, measured beside the HBM-bound GEMVs.
__global__ void __launch_bounds__(256) k_stream_read(const u4v *__restrict__ p, size_t n16, uint32_t *__restrict__ out) {
    const size_t stride = (size_t)gridDim.x * 256;
    uint32_t acc = 0;
    size_t i = blockIdx.x * (size_t)256 + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u4v a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
        acc ^= (a.x ^ a.y ^ a.z ^ a.w) ^ (b.x ^ b.y ^ b.z ^ b.w) ^ (c.x ^ c.y ^ c.z ^ c.w) ^ (d.x ^ d.y ^ d.z ^ d.w);
    }
    for (; i < n16; i += stride) {
        const u4v a = p[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, 64);
    if ((threadIdx.x & 63) == 0) out[blockIdx.x * 4 + (threadIdx.x >> 6)] = acc;
}

hipError_t hq_launch_stream_read(const void *p, size_t bytes, uint32_t *out, unsigned grid, hipStream_t st) {
    k_stream_read<<<grid, 256, 0, st>>>((const u4v *)p, bytes / 16, out);
    return hipGetLastError();
}

// ============================================================================ launchers
static unsigned grid_for(size_t n, unsigned per, unsigned cap) {
    size_t g = (n + per - 1) / per;
    return (unsigned)(g < cap ? (g ? g : 1) : cap);
}

hipError_t hq_launch_dequant(const hq_dev_mat *W, uint32_t row0, const uint32_t *ids, uint32_t nrows, float *out,
                             hipStream_t st) {
    if (W->type == HQ_TYPE_Q6_K) return hq_launch_dequant_q6k(W, row0, ids, nrows, out, st);
    if (hq_is_kq(W->type)) return hq_launch_dequant_kq(W, row0, ids, nrows, out, st);
    if (W->type == HQ_TYPE_Q8_0) {
        const size_t n = (size_t)nrows * W->cols / 4;
        k_dequant_q8_0<<<grid_for(n, 256, 65536), 256, 0, st>>>(W->qs, W->d, W->cols, W->ldd, row0, ids, nrows, out);
    } else {
        const size_t n = (size_t)nrows * W->cols / 8;
        k_dequant_q4_k<<<grid_for(n, 256, 65536), 256, 0, st>>>(W->qs, W->row_bytes, W->cols, row0, ids, nrows, out);
    }
    return hipGetLastError();
}

// Lanes per row. HBM latency is hidden by the number of loads in flight, so rows are spread over
// a whole wave (one load round per lane at K = 2560) unless there are rows enough for several
// waves per SIMD at fewer lanes.
static int lanes_per_row(long rows) { return rows >= 65536 ? 16 : rows >= 32768 ? 32 : 64; }

template <int R>
static void launch_gemv_t(const hq_dev_mat *W, const uint16_t *a, void *C, int c_f32, int accumulate, hipStream_t st) {
    const int N = (int)W->rows, K = (int)W->cols;
    const unsigned g = (unsigned)((N + 4 * R - 1) / (4 * R));
    if (W->type == HQ_TYPE_Q8_0)
        k_gemv_q8_0<R><<<g, 256, 0, st>>>(W->qs, W->d, W->ldd, a, N, K, C, c_f32, accumulate);
    else
        k_gemv_q4_k<R><<<g, 256, 0, st>>>(W->qs, W->row_bytes, a, N, K, C, c_f32, accumulate);
}

// Rows per wave: 2 (activations reused twice; measured best of 1, 2, 4 at N = 9728), 1 when that
// would leave the grid short of about two workgroups per CU.
// GEMV kernel choice for a matrix (shared by the launcher and the diagnostics name).
//   streamed Q4_K kernel when there are at least 1024 groups of 8 rows: two waves per group, each
//   half of K (measured at N = 9728, K = 2560: 6.55 us against 6.8 for the slab kernel and 7.1 with
//   one wave per group); fewer rows go to the slab kernel, whose 4-wave workgroups fill the CUs
//   better there (N = 2560, K = 9728: 7.5 us against 8.3). Slab: the most rows per workgroup (up to
//   32) that still give at least 512 workgroups (two per CU) and fit the slab, activations and sums
//   in 64 KB of LDS. Byte offsets are 32-bit up to the end of the last, possibly partial, group.
struct GemvPlan {
    enum Kind { Q4K_STREAM, Q4K_SLAB, REG } kind;
    int r;  // waves per group (stream), rows per workgroup (slab), rows per wave (register kernels)
    size_t lds;
};
constexpr int GVR_NS = 4;  // stream ring depth

static GemvPlan gemv_plan(const hq_dev_mat *W) {
    const size_t N = W->rows, K = W->cols, rb = W->row_bytes;
    if (W->type == HQ_TYPE_Q4_K && K % 512 == 0 && N >= 8 * 1024 && (N + 8) * rb < ((size_t)1 << 32)) {
        const int S = K / 512 >= 2 ? 2 : 1;
        const size_t lds = K * 2 + K / 32 * 4 + 32 * (size_t)S + (size_t)S * GVR_NS * GVR_SLOT;
        if (lds <= 64 * 1024) return {GemvPlan::Q4K_STREAM, S, lds};
    }
    if (W->type == HQ_TYPE_Q4_K && (N + 32) * rb < ((size_t)1 << 32)) {
        const size_t fixed = K * 2 + K / 32 * 4;
        int R = 32;
        while (R > 1 && ((N + R - 1) / R < 512 || fixed + (size_t)R * (rb + 16) > 64 * 1024)) R >>= 1;
        const size_t lds = fixed + (size_t)R * (rb + 16);
        if (lds <= 64 * 1024) return {GemvPlan::Q4K_SLAB, R, lds};
    }
    return {GemvPlan::REG, N >= 4096 ? 2 : 1, 0};
}

hipError_t hq_launch_gemv(const hq_dev_mat *W, const uint16_t *a, void *C, int c_f32, int accumulate, hipStream_t st) {
    if (W->type == HQ_TYPE_Q6_K || hq_is_kq(W->type)) return hq_launch_gemv_kq(W, a, C, c_f32, accumulate, st);
    const GemvPlan pl = gemv_plan(W);
    const int N = (int)W->rows, K = (int)W->cols;
    const uint32_t rb = (uint32_t)W->row_bytes;
    if (pl.kind == GemvPlan::Q4K_STREAM) {
        k_gemv_q4_k_r<GVR_NS><<<(N + 7) / 8, 64 * pl.r, pl.lds, st>>>(W->qs, rb, a, N, K, C, c_f32, accumulate);
    } else if (pl.kind == GemvPlan::Q4K_SLAB) {
        const unsigned g = (unsigned)((N + pl.r - 1) / pl.r);
#define GVS(r) k_gemv_q4_k_s<r><<<g, 256, pl.lds, st>>>(W->qs, rb, a, N, K, C, c_f32, accumulate)
        switch (pl.r) {
        case 32: GVS(32); break;
        case 16: GVS(16); break;
        case 8: GVS(8); break;
        case 4: GVS(4); break;
        case 2: GVS(2); break;
        default: GVS(1); break;
        }
#undef GVS
    } else if (pl.r == 2) {
        launch_gemv_t<2>(W, a, C, c_f32, accumulate, st);
    } else {
        launch_gemv_t<1>(W, a, C, c_f32, accumulate, st);
    }
    return hipGetLastError();
}

template <int LPR>
static void launch_gather_t(const hq_dev_mat *W, const uint16_t *H, const uint32_t *ids, int B, int k, float *out,
                            hipStream_t st) {
    const int pairs = B * k, K = (int)W->cols;
    const unsigned g = (unsigned)((pairs + 256 / LPR - 1) / (256 / LPR));
    if (W->type == HQ_TYPE_Q8_0)
        k_gather_q8_0<LPR><<<g, 256, 0, st>>>(W->qs, W->d, W->ldd, H, ids, pairs, k, K, W->rows, out);
    else
        k_gather_q4_k<LPR><<<g, 256, 0, st>>>(W->qs, W->row_bytes, H, ids, pairs, k, K, W->rows, out);
}

hipError_t hq_launch_gather(const hq_dev_mat *W, const uint16_t *H, const uint32_t *ids, int B, int k, float *out,
                            hipStream_t st) {
    if (W->type == HQ_TYPE_Q6_K || hq_is_kq(W->type)) return hq_launch_gather_kq(W, H, ids, B, k, out, st);
    switch (lanes_per_row((long)B * k)) {
    case 16: launch_gather_t<16>(W, H, ids, B, k, out, st); break;
    case 32: launch_gather_t<32>(W, H, ids, B, k, out, st); break;
    default: launch_gather_t<64>(W, H, ids, B, k, out, st); break;
    }
    return hipGetLastError();
}

static SkPlan hq_sk_plan(int M, int N, int K, int bm, int bn, int n_cu) {
    SkPlan p;
    p.tm = (M + bm - 1) / bm;
    p.tiles = p.tm * ((N + bn - 1) / bn);
    p.upt = (K + KC - 1) / KC;
    const long units = (long)p.tiles * p.upt;
    int G = (int)(units < n_cu ? units : n_cu);
    if (G >= 8) G -= G % 8;
    p.G = G;
    p.base = (int)(units / G);
    p.extra = (int)(units % G);
    return p;
}

namespace {
// Launch plan of the register-decode tile kernels (128 x 192 full-K tiles, one workgroup per CU):
// launches of row_tiles x col_tiles tiles, each at most one round on every XCD. A launch deals its
// column tiles to the 8 XCDs in turn (all row tiles of a column tile on one XCD, which then fetches
// the weight slab once), so an XCD gets row_tiles x ceil(col_tiles / 8) tiles; more than its CUs
// would leave a second round on that XCD (measured: M = 640, 5 x 51 tiles in one launch, 59 us
// against 30 at M = 512). Chunks of rows come first (each launch reads all the weights, which stay
// in the last-level cache, and a slice of A), then chunks of columns. `fill` when the launches'
// tiles fill at least 70 % of the CU time.
struct WrPlan {
    int row_tiles, col_tiles, launches, tw;  // tw: tile width in columns (192, or 160 for k_gemm_q4_k_wr160)
    bool fill;
};
WrPlan wr_plan(int M, int N, int n_cu, int tw = 192) {
    WrPlan w;
    w.tw = tw;
    const int mt = (M + 127) / 128, nt = (N + tw - 1) / tw, per_xcd = std::max(1, n_cu / 8), ncx = (nt + 7) / 8;
    if (mt * ncx <= per_xcd) {
        w.row_tiles = mt, w.col_tiles = nt;
    } else if (ncx <= per_xcd) {
        w.row_tiles = per_xcd / ncx, w.col_tiles = nt;
    } else {
        w.row_tiles = std::min(mt, per_xcd), w.col_tiles = 8 * std::max(1, per_xcd / w.row_tiles);
    }
    w.launches = ((mt + w.row_tiles - 1) / w.row_tiles) * ((nt + w.col_tiles - 1) / w.col_tiles);
    w.fill = 10L * mt * nt >= 7L * w.launches * n_cu;
    return w;
}
// the plan's launches: launch(m0, rows, t0, t1) for row chunk m0 .. m0 + rows - 1 and column tiles
// t0 .. t1 - 1
template <class F>
hipError_t wr_launches(const WrPlan &pl, int M, int N, F &&launch) {
    const int mt = (M + 127) / 128, nt = (N + pl.tw - 1) / pl.tw;
    for (int r = 0; r < mt; r += pl.row_tiles)
        for (int t = 0; t < nt; t += pl.col_tiles) {
            const int m0 = 128 * r;
            const hipError_t e = launch(m0, std::min(M - m0, 128 * pl.row_tiles), t, std::min(nt, t + pl.col_tiles));
            if (e != hipSuccess) return e;
        }
    return hipSuccess;
}
// Launch plan of the Q4_K register-decode kernel over more than one round: 160-column tiles where
// they need no more launches than 192-column ones (M = 512, N = 19456: two launches of 4 x 122 / 2
// tiles, 244 of 256 CUs, instead of 204), and one launch where its tiles make two rounds on every XCD
// with the second at least 60 % full (the gate/up pair GEMM at M = 512, I = 9728: one launch of
// 4 x 122 tiles instead of two of 2 x 122, 68.5 -> 67.4 us in a same-box A/B)
WrPlan wr4_plan(int M, int N, int n_cu) {
    WrPlan pl = wr_plan(M, N, n_cu);
    const WrPlan p160 = wr_plan(M, N, n_cu, 160);
    if (p160.fill && p160.launches <= pl.launches) pl = p160;
    const int mt = (M + 127) / 128, nt = (N + pl.tw - 1) / pl.tw, per_xcd = std::max(1, n_cu / 8);
    const int on_xcd = mt * ((nt + 7) / 8);
    if (pl.fill && on_xcd > per_xcd && on_xcd <= 2 * per_xcd && 5 * on_xcd >= 8 * per_xcd)
        pl.row_tiles = mt, pl.col_tiles = nt, pl.launches = 1;
    return pl;
}
}  // namespace

namespace {
// Kernel choice for M >= 2: MB (16-row blocks of M per tile) grows with M up to 8 (Q4_K: at least 2);
// NB = 2 16-column blocks per wave. Q4_K with M > 64 uses the wide 8-wave kernel (tile 128 x 256).
// Stream-K removes the wave-quantization cost, so the tile only sets the operand reuse.
struct GemmCfg {
    int mb, nb, waves;
    bool wide;
    int ws_nb;     // > 0: the full-K tile kernel k_gemm_q4_k_ws with 32 * ws_nb columns per tile
    int ws_parts;  // with ws_nb: workgroups per tile, each a contiguous range of K (1: whole K)
    int ws8_nb;  // > 0: the Q8_0 full-K tile kernel k_gemm_q8_0_ws, 32 * ws8_nb columns per tile
    int ws8_parts;  // with ws8_nb: workgroups per tile (K split, as ws_parts)
    int rbm;        // Q4_K mid M: workgroups per tile of k_gemm_q4_k_rb (hq_gemm_rb.hip); 0: not used
    int rb8;        // Q8_0 M <= 64: workgroups per tile of k_gemm_q8_0_rb (hq_gemm_rb.hip); 0: not used
    bool bt;        // Q4_K large M: the 256 x 256 tile kernel k_gemm_q4_k_bt (hq_gemm_bt.hip)
    bool wr;        // Q4_K, one round of full-K tiles: the 128 x 192 tile kernel k_gemm_q4_k_wr (hq_gemm_wr.hip)
    int wr_parts;   // with wr: workgroups per tile (K split), 1: whole K
    int wr_tw;      // with wr: tile width, 192 or 160 columns (k_gemm_q4_k_wr160)
    bool wr_multi;  // with wr: launches of at most one round each (wr4_plan), no K split
    bool wr8;       // Q8_0, the same: k_gemm_q8_0_wr (hq_gemm_wr8.hip)
    bool nn;        // Q4_K with N <= 32 and many rows: k_gemm_q4_k_nn (hq_gemm_nn.hip)
};

// Q4_K with M > 64 runs the full-K tile kernel when its tiles fit in one round on the CUs and fill
// at least 70 % of them (e.g. M = 512, N = 9728: 244 tiles of 128 x 160 on 256 CUs), or, with each
// tile's K split over 2 or 4 workgroups, when few tiles cover a long K (M = 512, N = 2560,
// K = 9728); otherwise the Stream-K wide kernel (many tiles at large M, where its split-tile
// overhead is amortised: measured faster at M = 4096 and 16384).
GemmCfg gemm_cfg(const hq_dev_mat *W, int M, int n_cu) {
    GemmCfg c;
    c.mb = M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8;
    if ((W->type == HQ_TYPE_Q6_K || hq_is_kq(W->type)) && c.mb > 4) c.mb = 4;  // the narrow kernel, up to 64-row tiles
    c.nb = 2;
    if (W->type == HQ_TYPE_Q4_K && c.mb == 1) c.mb = 2;
    // (Q5_K: the Q4_K LDS-decode tile kernel where it is chosen below, else the Stream-K k-quant kernel)
    c.wide = (W->type == HQ_TYPE_Q4_K || W->type == HQ_TYPE_Q5_K) && M > 64;
    c.waves = c.wide ? WNW : 4;
    c.ws_nb = 0;
    c.ws_parts = 1;
    c.rbm = W->type == HQ_TYPE_Q4_K ? hq_rb_parts(M, (int)W->rows, (int)W->cols, n_cu) : 0;
    c.rb8 = W->type == HQ_TYPE_Q8_0 ? hq_rb8_parts(M, (int)W->rows, (int)W->cols, n_cu) : 0;
    if (c.wide && (size_t)M * W->cols * 2 < ((size_t)1 << 32)) {
        float eff = 0.f;
        const int nb = hq_ws_choose(M, (int)W->rows, n_cu, &eff);
        const long tiles = (long)((M + 127) / 128) * (((int)W->rows + 32 * nb - 1) / (32 * nb));
        if (eff >= 0.7f && tiles <= n_cu) c.ws_nb = nb;
        // few tiles over a long K (M = 512, N = 2560, K = 9728: 64 tiles of 128 x 160): split each
        // tile's K over 2 or 4 workgroups, the widest tiles for which that fills at least 3/4 of the
        // CUs in one round, with >= min_sb super-blocks per part
        auto split = [&](int min_sb) {
            for (int parts = 4; !c.ws_nb && parts >= 2; parts /= 2)
                for (int w = 5; !c.ws_nb && w >= 2; w--) {
                    const long t = (long)((M + 127) / 128) * (((int)W->rows + 32 * w - 1) / (32 * w));
                    if (t * parts <= n_cu && 4 * t * parts >= 3L * n_cu && (int)(W->cols / 256) >= min_sb * parts) {
                        c.ws_nb = w;
                        c.ws_parts = parts;
                    }
                }
        };
        split(8);
        // Q5_K has no large-M kernel of its own: the tile kernel over several rounds when they fill at
        // least half of the CU time (as the Q8_0 and k-quant tile kernels)
        if (W->type == HQ_TYPE_Q5_K && !c.ws_nb && eff >= 0.5f) c.ws_nb = nb;
        // then parts of >= 4 super-blocks (M = 128, N = 9728, K = 2560: 102 tiles of 128 x 96 in 2
        // parts, 22.2 us against 29.8 for Stream-K; M = 512, N = 1024, K = 4096: 18.9 against 37.1;
        // M = 1024, N = 1024, K = 2560: 19.2 against 29.1), where the Stream-K kernel is left
        if (!c.ws_nb) split(4);
    }
    if (W->type == HQ_TYPE_Q5_K && !c.ws_nb) {
        c.wide = false;
        c.waves = 4;
    }
    // Q4_K full-K tiles without a K split: the 128 x 192 tile kernel, whose waves decode their own
    // columns (M = 512, N = 9728: 204 tiles)
    c.wr = c.ws_nb && c.ws_parts == 1 && hq_wr_fits(W, M);
    c.wr_parts = 1;
    // 160-column tiles where they still make one round on every XCD and are more tiles than the
    // 192-column ones (M = 512, N = 9728: 244 tiles instead of 204 on 256 CUs); each wave issues
    // 40 MFMAs per stage instead of 48
    c.wr_tw = 192;
    if (c.wr) {
        const int mt = (M + 127) / 128, per_xcd = std::max(1, n_cu / 8);
        const int n192 = ((int)W->rows + 191) / 192, n160 = ((int)W->rows + 159) / 160;
        if (mt * ((n160 + 7) / 8) <= per_xcd && n160 > n192) c.wr_tw = 160;
    }
    // few tiles over a long K, where the LDS-decode kernel splits K (M = 512, N = 2560, K = 9728): the
    // register-decode kernel with each tile's K split over 4 or 2 workgroups of >= 5 super-blocks,
    // when its tiles x parts fit one round on every XCD and fill >= 70 % of the CUs (4 x 14 x 4 = 224;
    // M = 200, N = 9728, K = 2560: 2 x 51 x 2, 31.9 us against 36.3 for the LDS-decode kernel's split;
    // parts of 4 super-blocks measured slower than the LDS-decode kernel's, e.g. 34.4 against 29.0 us
    // at M = 512, N = 2560, K = 4096)
    // 160-column tiles first (more workgroups in the round: M = 512, N = 2560, 4 x 16 x 4 = 256)
    if (!c.wr && c.ws_nb && c.ws_parts > 1 && hq_wr_fits(W, M)) {
        const int mt = (M + 127) / 128, per_xcd = std::max(1, n_cu / 8);
        for (int parts = 4; !c.wr && parts >= 2; parts /= 2)
            for (int tw = 160; !c.wr && tw <= 192; tw += 32) {
                const int units = ((int)W->rows + tw - 1) / tw * parts;
                if (mt * ((units + 7) / 8) <= per_xcd && 10L * mt * units >= 7L * n_cu && (int)(W->cols / 256) >= 5 * parts) {
                    c.wr = true;
                    c.wr_parts = parts;
                    c.wr_tw = tw;
                }
            }
    }
    // Q4_K where the Stream-K wide kernel would run: the 256 x 256 tile kernel when its rounds of
    // tiles fill at least 3/4 of the CU time (M = 16384, N = 9728: 2432 tiles in 9.5 rounds)
    c.bt = false;
    if (c.wide && !c.ws_nb && hq_bt_fits(W, M)) {
        const long t = (long)((M + 255) / 256) * (((long)W->rows + 255) / 256), rounds = (t + n_cu - 1) / n_cu;
        c.bt = 4 * t >= 3 * rounds * n_cu;
    }
    // Q4_K where the Stream-K wide kernel would run otherwise (N beyond one round at M ~512, M of
    // several hundred rows and more at N ~10k, short of the 256 x 256 kernel's rule): the register-
    // decode kernel as launches of at most one round each (wr4_plan), when they fill at least 70 % of
    // the CU time. Per call against Stream-K in a same-box A/B (K = 2560): M = 512, N = 19456 80.9 ->
    // 63.6 us; M = 384, N = 19456 66.4 -> 60.0; M = 512, N = 14336 65.4 -> 58.0; M = 768, N = 9728
    // 66.0 -> 59.8; M = 1024 81.5 -> 63.3; M = 2048 140.6 -> 127.2; M = 4096, N = 2560 88.2 -> 71.4;
    // M = 2048, N = 4096 60.6 -> 61.6. Against the 256 x 256 kernel it was no faster (M = 1536, N = 9728:
    // 95.6 -> 96.0; M = 3072: 181.8 -> 191.0), so that one keeps its shapes.
    c.wr_multi = false;
    if (!c.wr && !c.bt && c.wide && W->type == HQ_TYPE_Q4_K && !(c.ws_nb && c.ws_parts > 1) && hq_wr_fits(W, M)) {
        const WrPlan pl = wr4_plan(M, (int)W->rows, n_cu);
        if (pl.fill) c.wr = c.wr_multi = true, c.wr_tw = pl.tw, c.ws_nb = 0;
    }
    // Q8_0 with M > 64: the Q8_0 tile kernel when its tiles fill at least half of the CU time
    // (rounds of tiles included; M = 128, N = 9728: 152 tiles of 128 x 64, 21.7 us against 24.9 for
    // the narrow kernel), K is whole 128-wide stages and the byte offsets fit 32 bits
    c.ws8_nb = 0;
    c.ws8_parts = 1;
    // (Q6_K, Q3_K and Q2_K: the same tile kernel with k-quant producers, k_gemm_kq_ws, on the same rule)
    const bool kqws = (W->type == HQ_TYPE_Q6_K || W->type == HQ_TYPE_Q3_K || W->type == HQ_TYPE_Q2_K) && M > 64 &&
                      hq_kqws_fits(W, M);
    if (kqws || (W->type == HQ_TYPE_Q8_0 && M > 64 && W->cols % 128 == 0 && (size_t)M * W->cols * 2 < ((size_t)1 << 32) &&
                 ((size_t)W->rows + 160) * W->cols < ((size_t)1 << 32))) {
        float eff = 0.f;
        const int nb = hq_ws_choose(M, (int)W->rows, n_cu, &eff);
        const long tiles = (long)((M + 127) / 128) * (((int)W->rows + 32 * nb - 1) / (32 * nb));
        if (eff >= 0.5f) c.ws8_nb = nb;
        // fewer tiles than 3/4 of the CUs over a long K (M = 512, N = 2560, K = 9728: 160 tiles of
        // 128 x 64 through 76 stages, 66 us): each tile's K split over 2 or 4 workgroups, the widest
        // tiles that fill >= 3/4 of the CUs in one round. Parts of >= 8 stages where no unsplit tiling
        // fills half the CU time (M = 96, N = 9728, K = 2560: Q8_0 24.6 -> 21.4 us, Q6_K 31.9 -> 21.5;
        // M = 128, N = K = 4096: 25.2 -> 17.6, 26.3 -> 17.4) and for Q8_0 (M = 128, N = 9728, K = 2560:
        // 22.7 -> 21.8); >= 16 stages for the k-quants otherwise (the same shape: Q6_K 21.0 unsplit
        // against 21.9 split, Q3_K 19.3 against 20.5)
        const int min_stages = c.ws8_nb && kqws ? 16 : 8;
        if (4 * tiles < 3L * n_cu || !c.ws8_nb)
            for (int parts = 4, done = 0; !done && parts >= 2; parts /= 2)
                for (int w = 5; !done && w >= 2; w--) {
                    const long t = (long)((M + 127) / 128) * (((int)W->rows + 32 * w - 1) / (32 * w));
                    if (t * parts <= n_cu && 4 * t * parts >= 3L * n_cu && (int)(W->cols / 128) >= min_stages * parts) {
                        c.ws8_nb = w;
                        c.ws8_parts = parts;
                        done = 1;
                    }
                }
    }
    // Q8_0 with M > 64: the register-decode tile kernel (128 x 192 full-K tiles) where its launches of
    // at most one round each fill at least 70 % of the CU time (M = 512, N = 9728: one launch of 204
    // tiles; M = 2048: four launches of 16 x 13 tiles)
    c.wr8 = W->type == HQ_TYPE_Q8_0 && M > 64 && hq_wr8_fits(W, M) && wr_plan(M, (int)W->rows, n_cu).fill;
    // N <= 32 with at least 64 workgroups of 64 rows (config 4's b / a projections at M = 16384: 256):
    // the skinny kernel, which reads A once with every CU streaming
    c.nn = W->type == HQ_TYPE_Q4_K && W->rows <= 32 && M >= 64 * 64 && hq_nn_fits(W, M);
    if (c.nn) {
        c.wide = c.wr = c.bt = false;
        c.ws_nb = c.rbm = 0;
        c.ws_parts = 1;
        c.waves = 4;
    }
    return c;
}

SkPlan gemm_plan(const hq_dev_mat *W, int M, const GemmCfg &c, int n_cu) {
    return hq_sk_plan(M, (int)W->rows, (int)W->cols, 16 * c.mb, 16 * c.nb * c.waves, n_cu);
}
}  // namespace

// device bytes of a row of K values (the upload's layout: Q8_0 quant plane, k-quant slots)
static size_t shape_row_bytes(int type, int K) {
    return type == HQ_TYPE_Q4_K ? (size_t)K / 256 * 144 : type == HQ_TYPE_Q8_0 ? (size_t)K
         : (size_t)K / 256 * (type == HQ_TYPE_Q6_K ? 224 : type == HQ_TYPE_Q5_K ? 176 : type == HQ_TYPE_Q3_K ? 112 : 96);
}

void hq_gemm_tile_shape(int type, int M, int N, int K, int n_cu, int *rows, int *cols) {
    hq_dev_mat W = {};
    W.type = type;
    W.rows = (uint32_t)N;
    W.cols = (uint32_t)K;
    W.row_bytes = shape_row_bytes(type, K);
    W.ldd = type == HQ_TYPE_Q8_0 ? (K / 32 + 7) / 8 * 8 : 0;
    const GemmCfg c = gemm_cfg(&W, M, n_cu);
    if (c.nn) {
        *rows = 64, *cols = 32;
        return;
    }
    *rows = c.bt ? 256 : c.wr || c.wr8 ? 128 : c.rbm ? 64 : c.rb8 ? (M <= 16 ? 16 : M <= 32 ? 32 : 64) : c.ws_nb || c.ws8_nb ? 128 : 16 * c.mb;
    *cols = c.bt ? 256 : c.wr ? c.wr_tw : c.wr8 ? 192 : c.rbm || c.rb8 ? 64 : c.ws_nb ? 32 * c.ws_nb : c.ws8_nb ? 32 * c.ws8_nb : 16 * c.nb * c.waves;
}

// Name of the kernel that does the work of an M x N x K hq_gemm call (the main kernel for GEMMs
// with a pre-pass), as rocprofv3 lists it.
void hq_gemm_kernel_name(int type, int M, int N, int K, int n_cu, char *buf, size_t n) {
    hq_dev_mat W = {};
    W.type = type;
    W.rows = (uint32_t)N;
    W.cols = (uint32_t)K;
    W.ldd = type == HQ_TYPE_Q8_0 ? (K / 32 + 7) / 8 * 8 : 0;
    W.row_bytes = shape_row_bytes(type, K);
    const char *kq = type == HQ_TYPE_Q2_K ? "10" : type == HQ_TYPE_Q3_K ? "11" : type == HQ_TYPE_Q5_K ? "13" : nullptr;
    if (M == 1 && (kq || type == HQ_TYPE_Q6_K)) {  // template arguments: the ggml type, rows per wave, gather, LDS copy of a
        snprintf(buf, n, "k_gemv_sb<%d, %d, false, %s>", type, hq_sb_rows(N), hq_sb_lds(type, K) ? "true" : "false");
        return;
    }
    const GemmCfg c = gemm_cfg(&W, M, n_cu);
    if (c.ws_nb && type == HQ_TYPE_Q5_K) {
        snprintf(buf, n, "k_gemm_q5_k_ws<%d>", c.ws_nb);
        return;
    }
    if (c.ws8_nb && type != HQ_TYPE_Q8_0) {  // template arguments: the ggml type, the tile width / 32
        snprintf(buf, n, "k_gemm_kq_ws<%d, %d>", type, c.ws8_nb);
        return;
    }
    if (kq) {  // template argument: the ggml type
        const int mb = M <= 16 ? 1 : M <= 32 ? 2 : 4;
        snprintf(buf, n, "k_gemm_kq<%s, %d, 2>", kq, mb);
        return;
    }
    if (M == 1) {
        const GemvPlan pl = gemv_plan(&W);
        if (pl.kind == GemvPlan::Q4K_STREAM) snprintf(buf, n, "k_gemv_q4_k_r<%d>", GVR_NS);
        else if (pl.kind == GemvPlan::Q4K_SLAB) snprintf(buf, n, "k_gemv_q4_k_s<%d>", pl.r);
        else snprintf(buf, n, "%s<%d>", type == HQ_TYPE_Q4_K ? "k_gemv_q4_k" : "k_gemv_q8_0", pl.r);
        return;
    }
    if (c.nn) snprintf(buf, n, "k_gemm_q4_k_nn<%d>", N <= 16 ? 1 : 2);
    else if (c.rbm) snprintf(buf, n, "k_gemm_q4_k_rb<1, 4, 3, 2>");
    else if (c.rb8) snprintf(buf, n, "k_gemm_q8_0_rb<%d, 3, 2>", M <= 16 ? 1 : M <= 32 ? 2 : 4);
    else if (c.bt) snprintf(buf, n, "k_gemm_q4_k_bt");
    else if (c.wr)
        snprintf(buf, n, c.wr_parts > 1 ? (c.wr_tw == 160 ? "k_gemm_q4_k_wr_ks160" : "k_gemm_q4_k_wr_ks<3>")
                                        : c.wr_tw == 160 ? "k_gemm_q4_k_wr160" : "k_gemm_q4_k_wr<3>");
    else if (c.wr8) snprintf(buf, n, "k_gemm_q8_0_wr");
    else if (c.ws_nb) snprintf(buf, n, "k_gemm_q4_k_ws<%d>", c.ws_nb);
    else if (c.ws8_nb) snprintf(buf, n, "k_gemm_q8_0_ws<%d>", c.ws8_nb);
    else if (c.wide) snprintf(buf, n, "k_gemm_q4_k_w<%d>", c.mb);  // template argument: row blocks
    else snprintf(buf, n, "%s<%d, %d>", type == HQ_TYPE_Q4_K ? "k_gemm_q4_k" : type == HQ_TYPE_Q6_K ? "k_gemm_q6_k" : "k_gemm_q8_0",
                  c.mb, c.nb);
}

void hq_gemm_work_bytes(const hq_dev_mat *W, int M, int n_cu, size_t *partial_bytes, size_t *counter_bytes,
                        size_t *sums_bytes) {
    const GemmCfg c = gemm_cfg(W, M, n_cu);
    if (c.nn) {  // no workspace
        *partial_bytes = *counter_bytes = *sums_bytes = 0;
        return;
    }
    const SkPlan p = gemm_plan(W, M, c, n_cu);
    const bool tile = c.ws_nb || c.ws8_nb || c.bt;  // tile kernels: partial tiles only when K is split (below)
    *partial_bytes = tile ? 0 : (size_t)2 * p.G * 64 * c.waves * c.mb * c.nb * 4 * sizeof(float);
    *counter_bytes = tile ? 0 : (size_t)p.tiles * sizeof(int);
    const int snb = c.ws_nb ? c.ws_nb : c.ws8_nb, sparts = c.ws_nb ? c.ws_parts : c.ws8_parts;
    if (snb && sparts > 1) {  // K-split tile kernels: one fp32 tile per (tile, part)
        const size_t tiles = (size_t)((M + 127) / 128) * ((W->rows + 32 * snb - 1) / (32 * snb));
        *partial_bytes = tiles * sparts * 128 * 32 * snb * sizeof(float);
        *counter_bytes = tiles * sizeof(int);
    }
    if (c.rbm == 1 || c.rb8 == 1) *partial_bytes = *counter_bytes = 0;  // mid-M kernels, one part per tile
    const int rparts = c.rbm > 1 ? c.rbm : c.rb8 > 1 ? c.rb8 : 0;
    if (rparts) {  // mid-M kernels with a K split: tiles of at most 64 x 64 fp32
        const size_t tiles = (W->rows + 63) / 64;
        *partial_bytes = tiles * rparts * 64 * 64 * sizeof(float);
        *counter_bytes = tiles * sizeof(int);
    }
    // (the Q4_K tile kernels wr, ws form their own)
    *sums_bytes = c.wide && !c.wr && !(c.ws_nb && W->type == HQ_TYPE_Q4_K) ? (size_t)M * (W->cols / KC) * 32 : 0;
    if (c.wr8) *partial_bytes = *counter_bytes = 0;  // (no K split)
    if (c.wr) {  // K split: one fp32 128 x wr_tw tile per (tile, part)
        const size_t tiles = (size_t)((M + 127) / 128) * ((W->rows + c.wr_tw - 1) / c.wr_tw);
        *partial_bytes = c.wr_parts > 1 ? tiles * c.wr_parts * 128 * c.wr_tw * sizeof(float) : 0;
        *counter_bytes = c.wr_parts > 1 ? tiles * sizeof(int) : 0;
    }
}

// Pre-pass of a GEMM (the activation sub-block sums of the Q4_K kernels that read them from HBM;
// nothing otherwise: the Q4_K tile kernels k_gemm_q4_k_wr, k_gemm_q4_k_ws and k_gemm_q4_k_rb form
// their own).
hipError_t hq_launch_gemm_pre(const hq_dev_mat *W, const uint16_t *A, int M, const HqGemmWork &wk, hipStream_t st) {
    const GemmCfg c = gemm_cfg(W, M, wk.n_cu);
    if (c.wide && !c.wr && !(c.ws_nb && W->type == HQ_TYPE_Q4_K)) {
        const size_t nsub = (size_t)M * (W->cols / 32);
        if (nsub >= ((size_t)1 << 31)) return hipErrorInvalidValue;
        if (c.ws_nb || c.bt) k_asums<true><<<grid_for(nsub, 256, 16384), 256, 0, st>>>(A, M, (int)W->cols, wk.sums);
        else k_asums<false><<<grid_for(nsub, 256, 16384), 256, 0, st>>>(A, M, (int)W->cols, wk.sums);
    }
    return hipGetLastError();
}

// Main kernel of a GEMM (needs hq_launch_gemm_pre's output for the same A).
hipError_t hq_launch_gemm_main(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                               const HqGemmWork &wk, hipStream_t st) {
    const GemmCfg c = gemm_cfg(W, M, wk.n_cu);
    if (c.nn) return hq_launch_gemm_nn(W, A, M, C, c_f32, accumulate, st);
    if (c.rbm) return hq_launch_gemm_rb(W, A, M, C, c_f32, accumulate, c.rbm, wk.partials, wk.counters, st);
    if (c.rb8) return hq_launch_gemm_rb8(W, A, M, C, c_f32, accumulate, c.rb8, wk.partials, wk.counters, st);
    if (c.bt) return hq_launch_gemm_bt(W, A, wk.sums, M, C, c_f32, accumulate, st);
    if (c.wr && c.wr_multi) {
        const size_t K = W->cols, N = W->rows, esize = c_f32 ? 4 : 2;
        return wr_launches(wr4_plan(M, (int)N, wk.n_cu), M, (int)N, [&](int m0, int rows, int t0, int t1) {
            return hq_launch_gemm_wr(W, A + (size_t)m0 * K, rows, (char *)C + (size_t)m0 * N * esize, c_f32, accumulate, t0, t1, 1,
                                     nullptr, nullptr, st, c.wr_tw);
        });
    }
    if (c.wr) return hq_launch_gemm_wr(W, A, M, C, c_f32, accumulate, 0, -1, c.wr_parts, wk.partials, wk.counters, st, c.wr_tw);
    if (c.wr8) {
        const size_t K = W->cols, N = W->rows, esize = c_f32 ? 4 : 2;
        return wr_launches(wr_plan(M, (int)N, wk.n_cu), M, (int)N, [&](int m0, int rows, int t0, int t1) {
            return hq_launch_gemm_wr8(W, A + (size_t)m0 * K, rows, (char *)C + (size_t)m0 * N * esize, c_f32, accumulate, t0, t1, st);
        });
    }
    if (c.ws_nb)
        return hq_launch_gemm_ws(W, A, wk.sums, M, C, c_f32, accumulate, c.ws_nb, c.ws_parts, wk.partials, wk.counters, st);
    if (c.ws8_nb && W->type != HQ_TYPE_Q8_0)
        return hq_launch_gemm_kqws(W, A, M, C, c_f32, accumulate, c.ws8_nb, c.ws8_parts, wk.partials, wk.counters, st);
    if (c.ws8_nb)
        return hq_launch_gemm_ws8(W, A, M, C, c_f32, accumulate, c.ws8_nb, c.ws8_parts, wk.partials, wk.counters, st);
    GemmArgs g;
    g.qs = W->qs, g.d = W->d, g.ldd = W->ldd, g.row_bytes = W->row_bytes, g.A = A;
    g.M = M, g.N = (int)W->rows, g.K = (int)W->cols, g.C = C, g.c_f32 = c_f32, g.accumulate = accumulate;
    g.plan = gemm_plan(W, M, c, wk.n_cu);
    g.partials = wk.partials, g.counters = wk.counters, g.sums = wk.sums;
    {
        size_t pb, cb, sb;
        hq_gemm_work_bytes(W, M, wk.n_cu, &pb, &cb, &sb);
        if (pb > 0xffffffffu) return hipErrorInvalidValue;
        g.partial_bytes = (uint32_t)pb;
    }
    if (c.wide) {
        k_gemm_q4_k_w<8><<<g.plan.G, 64 * WNW, 0, st>>>(g);
        return hipGetLastError();
    }
    if (W->type == HQ_TYPE_Q6_K) return hq_launch_gemm_q6k(g, c.mb, st);
    if (hq_is_kq(W->type)) return hq_launch_gemm_kq(W->type, g, c.mb, st);
#define CASE(a)                                                                                 \
    if (c.mb == a) {                                                                            \
        if (W->type == HQ_TYPE_Q8_0) k_gemm_q8_0<a, 2><<<g.plan.G, 256, 0, st>>>(g);            \
        else if constexpr (a % 2 == 0) k_gemm_q4_k<a, 2><<<g.plan.G, 256, 0, st>>>(g);          \
        return hipGetLastError();                                                               \
    }
    CASE(1) CASE(2) CASE(4) CASE(8)
#undef CASE
    return hipErrorInvalidValue;
}

// gate/up pair GEMM with the SwiGLU epilogue inside the full-K tile kernels (M > 64; any number of
// tile rounds, each tile's K in one workgroup). *fused = 0 when the shape does not suit them: the
// caller then runs hq_launch_gemm into fp32 and hq_launch_swiglu_pairs.
hipError_t hq_launch_gemm_swiglu(const hq_dev_mat *W, const uint16_t *A, int M, uint16_t *out, const HqGemmWork &wk,
                                 hipStream_t st, int *fused) {
    *fused = 0;
    const int N = (int)W->rows, K = (int)W->cols;
    if (M <= 64 || (size_t)M * K * 2 >= ((size_t)1 << 32) || N % 16) return hipSuccess;
    // the register-decode tile kernels (128 x 192 tiles) where their launches of at most one round
    // fill at least 70 % of the CU time (M = 512, pair matrix of I = 9728: 4 x 102 tiles as two
    // launches; measured faster than one launch of two rounds); the Q4_K one needs its upload-time
    // column tables
    // The Q4_K kernel takes 160-column tiles where they need no more launches than 192-column ones
    // (M = 512, I = 9728: two launches of 4 x 122 / 2 tiles, 244 of 256 CUs, instead of 204)
    const bool wr8 = W->type == HQ_TYPE_Q8_0 && hq_wr8_fits(W, M), wr4 = W->type == HQ_TYPE_Q4_K && W->tab && hq_wr_fits(W, M);
    // (wr4_plan; the Q8_0 kernel takes the same plan with 192-column tiles only: one launch of two
    // rounds, 63.8 -> 62.9 us at M = 512, I = 9728)
    WrPlan pl = wr4 ? wr4_plan(M, N, wk.n_cu) : wr_plan(M, N, wk.n_cu);
    if (wr8 && pl.fill) {
        const int mt = (M + 127) / 128, nt = (N + pl.tw - 1) / pl.tw, per_xcd = std::max(1, wk.n_cu / 8);
        const int on_xcd = mt * ((nt + 7) / 8);
        if (on_xcd > per_xcd && on_xcd <= 2 * per_xcd && 5 * on_xcd >= 8 * per_xcd) pl.row_tiles = mt, pl.col_tiles = nt, pl.launches = 1;
    }
    if (pl.fill && (wr8 || wr4)) {
        *fused = 1;
        return wr_launches(pl, M, N, [&](int m0, int rows, int t0, int t1) {
            const uint16_t *Am = A + (size_t)m0 * K;
            uint16_t *om = out + (size_t)m0 * (N / 2);
            return wr8 ? hq_launch_gemm_wr8(W, Am, rows, om, HQ_OUT_SWIGLU, 0, t0, t1, st)
                       : hq_launch_gemm_wr(W, Am, rows, om, HQ_OUT_SWIGLU, 0, t0, t1, 1, nullptr, nullptr, st, pl.tw);
        });
    }
    float eff = 0.f;
    const int nb = hq_ws_choose(M, N, wk.n_cu, &eff);
    if (W->type == HQ_TYPE_Q4_K && (size_t)M * K * 2 < ((size_t)1 << 32)) {
        *fused = 1;
        return hq_launch_gemm_ws(W, A, nullptr, M, out, HQ_OUT_SWIGLU, 0, nb, 1, nullptr, nullptr, st);
    }
    if (W->type == HQ_TYPE_Q5_K && wk.sums) {  // (the sums buffer of its own plan's tile kernel)
        const size_t nsub = (size_t)M * (W->cols / 32);
        if (nsub >= ((size_t)1 << 31)) return hipSuccess;
        k_asums<true><<<grid_for(nsub, 256, 16384), 256, 0, st>>>(A, M, K, wk.sums);
        *fused = 1;
        return hq_launch_gemm_ws(W, A, wk.sums, M, out, HQ_OUT_SWIGLU, 0, nb, 1, nullptr, nullptr, st);
    }
    if (W->type == HQ_TYPE_Q8_0 && K % 128 == 0 && ((size_t)N + 160) * K < ((size_t)1 << 32)) {
        *fused = 1;
        return hq_launch_gemm_ws8(W, A, M, out, HQ_OUT_SWIGLU, 0, nb, 1, nullptr, nullptr, st);
    }
    if ((W->type == HQ_TYPE_Q6_K || W->type == HQ_TYPE_Q3_K || W->type == HQ_TYPE_Q2_K) && hq_kqws_fits(W, M)) {
        *fused = 1;
        return hq_launch_gemm_kqws(W, A, M, out, HQ_OUT_SWIGLU, 0, nb, 1, nullptr, nullptr, st);
    }
    return hipSuccess;
}

// out[m][8k + e] = silu(C[m][16k + e]) * C[m][16k + 8 + e]: the pair epilogue as its own pass
__global__ void __launch_bounds__(256) k_swiglu_pairs(const float *__restrict__ C, uint16_t *__restrict__ out, size_t n_out) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n_out; i += (size_t)gridDim.x * blockDim.x) {
        const size_t k = i / 8, e = i % 8;
        const float g = C[16 * k + e], u = C[16 * k + 8 + e];
        out[i] = __builtin_bit_cast(uint16_t, (_Float16)(g / (1.0f + expf(-g)) * u));
    }
}

hipError_t hq_launch_swiglu_pairs(const float *C, uint16_t *out, size_t n_out, hipStream_t st) {
    k_swiglu_pairs<<<grid_for(n_out, 256, 16384), 256, 0, st>>>(C, out, n_out);
    return hipGetLastError();
}

hipError_t hq_launch_gemm(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                          const HqGemmWork &wk, hipStream_t st) {
    const hipError_t e = hq_launch_gemm_pre(W, A, M, wk, st);
    return e != hipSuccess ? e : hq_launch_gemm_main(W, A, M, C, c_f32, accumulate, wk, st);
}

hipError_t hq_launch_f32_to_f16(const float *in, uint16_t *out, size_t n, hipStream_t st) {
    k_f32_to_f16<<<grid_for(n, 256, 16384), 256, 0, st>>>(in, out, n);
    return hipGetLastError();
}
