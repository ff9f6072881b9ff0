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

#include "hq_kernels.h"

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

#define DEV static __device__ __forceinline__

DEV float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

DEV h2 as_h2(uint32_t x) { return __builtin_bit_cast(h2, x); }

// Bytes 4-7 of the v_perm_b32 source pair {S0, S1} come from S0 = 0x64646464 (the high byte of
// fp16 1024.0); bytes 0-3 from S1 = w. Result: [w.byte(i), 0x64, w.byte(j), 0x64].
DEV uint32_t perm_lo(uint32_t w) { return __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u); }  // bytes 0,1
DEV uint32_t perm_hi(uint32_t w) { return __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u); }  // bytes 2,3

// Q4_K scales/mins (ggml_quant.h:51-59) as four words of bytes: sw0 = s0..s3, sw1 = s4..s7,
// mw0 = m0..m3, mw1 = m4..m7, from the 12 scale bytes held in words q0 (bytes 0-3), q1 (4-7), q2 (8-11).
DEV void q4k_scale_words(uint32_t q0, uint32_t q1, uint32_t q2, uint32_t &sw0, uint32_t &sw1, uint32_t &mw0,
                         uint32_t &mw1) {
    sw0 = q0 & 0x3f3f3f3fu;
    mw0 = q1 & 0x3f3f3f3fu;
    sw1 = (q2 & 0x0f0f0f0fu) | ((q0 >> 2) & 0x30303030u);
    mw1 = ((q2 >> 4) & 0x0f0f0f0fu) | ((q1 >> 2) & 0x30303030u);
}

DEV uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

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
// 16 lanes per row; 4 rows per wave. Lane j of a row walks 16-byte chunks j, j+16, ... of the
// row's quant bytes and keeps an fp32 partial; a 16-lane butterfly reduces it.
DEV float sum16(float v) {
    v += __shfl_xor(v, 8, 16);
    v += __shfl_xor(v, 4, 16);
    v += __shfl_xor(v, 2, 16);
    v += __shfl_xor(v, 1, 16);
    return v;
}

// 16 fp16 activations starting at a (32-byte aligned) as fp32.
DEV void load_a16(const uint16_t *__restrict__ a, float *x) {
    const u4v v0 = *(const u4v *)a, v1 = *(const u4v *)(a + 8);
    const uint32_t w[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const h2 p = as_h2(w[i]);
        x[2 * i] = (float)p.x;
        x[2 * i + 1] = (float)p.y;
    }
}

// Q8_0 row dot: sum over the row of q*d*a. Chunk c = 16 values of block c/2.
DEV float dot_row_q8_0(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ d, const uint16_t *__restrict__ a,
                       int K, int j) {
    float acc = 0.f;
    for (int c = j; c < K / 16; c += 16) {
        const u4v q = *(const u4v *)(qs + 16 * c);
        const float dv = h2f(d[c >> 1]);
        float x[16];
        load_a16(a + 16 * c, x);
        const uint32_t w[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
        float p = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) p += (float)(int8_t)byte_of(w[i >> 2], i & 3) * x[i];
        acc += p * dv;
    }
    return acc;
}

// Q4_K row dot. Chunk c = 16 bytes of qs of super-block c/8: part t = c%8 -> p = t/2, h = t%2;
// low nibbles are values 64p+16h+i (sub 2p), high nibbles 64p+32+16h+i (sub 2p+1).
DEV float dot_row_q4_k(const uint8_t *__restrict__ row, const uint16_t *__restrict__ a, int K, int j) {
    float acc = 0.f;
    for (int c = j; c < K / 32; c += 16) {
        const uint8_t *b = row + (size_t)(c >> 3) * 144;
        const int t = c & 7, p = t >> 1, h = t & 1;
        const u4v hdr = *(const u4v *)b;
        const u4v q = *(const u4v *)(b + 16 + 16 * t);
        uint32_t sw0, sw1, mw0, mw1;
        q4k_scale_words(hdr.y, hdr.z, hdr.w, sw0, sw1, mw0, mw1);
        const int s0 = 2 * p, s1 = 2 * p + 1;
        const float d = h2f((uint16_t)hdr.x), dmin = h2f((uint16_t)(hdr.x >> 16));
        const float ds0 = d * (float)byte_of(s0 < 4 ? sw0 : sw1, s0 & 3);
        const float ds1 = d * (float)byte_of(s1 < 4 ? sw0 : sw1, s1 & 3);
        const float dm0 = dmin * (float)byte_of(s0 < 4 ? mw0 : mw1, s0 & 3);
        const float dm1 = dmin * (float)byte_of(s1 < 4 ? mw0 : mw1, s1 & 3);
        const int kb = (c >> 3) * 256 + 64 * p + 16 * h;
        float xl[16], xh[16];
        load_a16(a + kb, xl);
        load_a16(a + kb + 32, xh);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        float ql = 0.f, qh = 0.f, sl = 0.f, sh = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t by = byte_of(w[i >> 2], i & 3);
            ql += (float)(by & 0xfu) * xl[i];
            qh += (float)(by >> 4) * xh[i];
            sl += xl[i];
            sh += xh[i];
        }
        acc += (ds0 * ql - dm0 * sl) + (ds1 * qh - dm1 * sh);
    }
    return acc;
}

DEV void store_out(void *C, size_t idx, float v, int c_f32, int accumulate) {
    if (c_f32) {
        float *c = (float *)C + idx;
        *c = accumulate ? *c + v : v;
    } else {
        _Float16 *c = (_Float16 *)C + idx;
        *c = (_Float16)(accumulate ? (float)*c + v : v);
    }
}

__global__ void __launch_bounds__(256) k_gemv_q8_0(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ d,
                                                   int ldd, const uint16_t *__restrict__ a, int N, int K, void *C,
                                                   int c_f32, int accumulate) {
    const int n = blockIdx.x * 16 + (threadIdx.x >> 4), j = threadIdx.x & 15;
    const int nr = n < N ? n : N - 1;
    const float v = sum16(dot_row_q8_0(qs + (size_t)nr * K, d + (size_t)nr * ldd, a, K, j));
    if (j == 0 && n < N) store_out(C, n, v, c_f32, accumulate);
}

__global__ void __launch_bounds__(256) k_gemv_q4_k(const uint8_t *__restrict__ W, size_t row_bytes,
                                                   const uint16_t *__restrict__ a, int N, int K, void *C, int c_f32,
                                                   int accumulate) {
    const int n = blockIdx.x * 16 + (threadIdx.x >> 4), j = threadIdx.x & 15;
    const int nr = n < N ? n : N - 1;
    const float v = sum16(dot_row_q4_k(W + (size_t)nr * row_bytes, a, K, j));
    if (j == 0 && n < N) store_out(C, n, v, c_f32, accumulate);
}

// out[i] = dot(H[i / k], W[ids[i]]) for i < pairs. An id >= rows reads row 0 and stores NaN, so a
// bad id can never move a load outside the matrix.
__global__ void __launch_bounds__(256) k_gather_q8_0(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ d,
                                                     int ldd, const uint16_t *__restrict__ H,
                                                     const uint32_t *__restrict__ ids, int pairs, int k, int K,
                                                     uint32_t rows, float *__restrict__ out) {
    const int i = blockIdx.x * 16 + (threadIdx.x >> 4), j = threadIdx.x & 15;
    const int ic = i < pairs ? i : pairs - 1;
    const uint32_t id = ids[ic];
    const size_t r = id < rows ? id : 0;
    const float v = sum16(dot_row_q8_0(qs + r * K, d + r * ldd, H + (size_t)(ic / k) * K, K, j));
    if (j == 0 && i < pairs) out[i] = id < rows ? v : __builtin_nanf("");
}

__global__ void __launch_bounds__(256) k_gather_q4_k(const uint8_t *__restrict__ W, size_t row_bytes,
                                                     const uint16_t *__restrict__ H, const uint32_t *__restrict__ ids,
                                                     int pairs, int k, int K, uint32_t rows, float *__restrict__ out) {
    const int i = blockIdx.x * 16 + (threadIdx.x >> 4), j = threadIdx.x & 15;
    const int ic = i < pairs ? i : pairs - 1;
    const uint32_t id = ids[ic];
    const size_t r = id < rows ? id : 0;
    const float v = sum16(dot_row_q4_k(W + r * row_bytes, H + (size_t)(ic / k) * K, K, j));
    if (j == 0 && i < pairs) out[i] = id < rows ? v : __builtin_nanf("");
}

// ============================================================================ MFMA GEMM
// Tile: BM = 16*MB rows of A (M) by BN = 64*NB columns (N, weight rows); 4 waves, wave w owns
// columns [16*NB*w, 16*NB*(w+1)) of the tile and all BM rows. K advances in chunks of KC = 256
// activations staged in LDS (row stride LDA halves, padded against bank conflicts).
//
// v_mfma_f32_16x16x32_f16 operands (per lane l: ln = l % 16, lg = l / 16): A holds row ln,
// 8 k-slots of group lg; B holds column ln, the same 8 k-slots; D holds column ln, rows 4*lg..4*lg+3.
// The k-slot -> k mapping inside one MFMA is free as long as A and B agree; it is chosen so each
// lane's 8 weights come from one 16-byte load and each lane's 8 activations are 16 contiguous bytes.
namespace {
constexpr int KC = 256;
constexpr int LDA = KC + 8;

template <int MB>
struct Smem {
    _Float16 a[16 * MB * LDA];
    _Float16 s[16 * MB * 16];  // Q4_K: per row, fp16 hi[8] then lo[8] of the 8 sub-block sums
};

template <int MB>
DEV void stage_a(Smem<MB> &sm, const uint16_t *__restrict__ A, int M, int K, int m0, int k0, int kc) {
    constexpr int BM = 16 * MB;
    for (int i = threadIdx.x; i < BM * (KC / 8); i += 256) {
        const int r = i / (KC / 8), kk = (i % (KC / 8)) * 8, m = m0 + r;
        u4v v = {0u, 0u, 0u, 0u};
        if (m < M && kk < kc) v = *(const u4v *)(A + (size_t)m * K + k0 + kk);
        *(u4v *)(&sm.a[r * LDA + kk]) = v;
    }
}

// Q4_K: S[r][sub] = fp32 sum of the 32 staged activations of sub-block sub, split hi + lo fp16.
template <int MB>
DEV void stage_sums(Smem<MB> &sm) {
    constexpr int BM = 16 * MB;
    for (int i = threadIdx.x; i < BM * 8; i += 256) {
        const int r = i >> 3, sub = i & 7;
        const h8 *p = (const h8 *)&sm.a[r * LDA + 32 * sub];
        float s = 0.f;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const h8 x = p[v];
#pragma unroll
            for (int e = 0; e < 8; e++) s += (float)x[e];
        }
        const _Float16 hi = (_Float16)s;
        const _Float16 lo = (_Float16)(s - (float)hi);
        sm.s[r * 16 + sub] = hi;
        sm.s[r * 16 + 8 + sub] = lo;
    }
}

DEV f4 mfma(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

// B fragment from 4 bytes (u = q+128 biased int8) x 2 words -> fp16(q*d), 8 values.
DEV h8 frag_q8_0(uint32_t w0, uint32_t w1, h2 d2) {
    const h2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t w[2] = {w0, w1};
    h8 out;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const h2 a = (as_h2(perm_lo(w[i])) + bias) * d2;
        const h2 b = (as_h2(perm_hi(w[i])) + bias) * d2;
        out[4 * i + 0] = a.x;
        out[4 * i + 1] = a.y;
        out[4 * i + 2] = b.x;
        out[4 * i + 3] = b.y;
    }
    return out;
}

// B fragment of exact integers s*q from the low (hi_nib = false) or high nibbles of 8 bytes.
// fp16(1024 + q) * s - 1024*s, or fp16(1024 + 16q) * (s/16) - 64*s: one fused rounding of an
// exact integer <= 945, hence exact.
template <bool HI_NIB>
DEV h8 frag_q4_k(uint32_t w0, uint32_t w1, h2 mul, h2 add) {
    const uint32_t mask = HI_NIB ? 0xfff0fff0u : 0xff0fff0fu;
    const uint32_t w[2] = {w0, w1};
    h8 out;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const h2 a = __builtin_elementwise_fma(as_h2(perm_lo(w[i]) & mask), mul, add);
        const h2 b = __builtin_elementwise_fma(as_h2(perm_hi(w[i]) & mask), mul, add);
        out[4 * i + 0] = a.x;
        out[4 * i + 1] = a.y;
        out[4 * i + 2] = b.x;
        out[4 * i + 3] = b.y;
    }
    return out;
}

DEV h8 lds_frag(const _Float16 *p) { return *(const h8 *)p; }

}  // namespace

template <int MB, int NB>
__global__ void __launch_bounds__(256) k_gemm_q8_0(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ dpl,
                                                   int ldd, const uint16_t *__restrict__ A, int M, int N, int K,
                                                   void *C, int c_f32, int accumulate) {
    __shared__ Smem<MB> sm;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ln = lane & 15, lg = lane >> 4;
    const int m0 = blockIdx.y * 16 * MB, nw = blockIdx.x * 64 * NB + wave * 16 * NB;
    f4 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    const uint8_t *wrow[NB];
    const uint16_t *drow[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) {
        int n = nw + 16 * j + ln;
        n = n < N ? n : N - 1;
        wrow[j] = qs + (size_t)n * K;
        drow[j] = dpl + (size_t)n * ldd;
    }
    for (int k0 = 0; k0 < K; k0 += KC) {
        const int kc = K - k0 < KC ? K - k0 : KC;
        __syncthreads();
        stage_a<MB>(sm, A, M, K, m0, k0, kc);
        __syncthreads();
        // 64-value steps: lane (ln, lg) loads weights [kk + 16*lg, +16) of its row (one block);
        // MFMA t in {0, 1} takes bytes 8t..8t+7 of that load.
        for (int kk = 0; kk < kc; kk += 64) {
            const bool full = kk + 64 <= kc;  // a 32-value tail leaves lanes lg >= 2 without data
            h8 bf[NB][2];
#pragma unroll
            for (int j = 0; j < NB; j++) {
                u4v q = {0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
                uint16_t dv = 0;
                if (full || lg < 2) {
                    q = *(const u4v *)(wrow[j] + k0 + kk + 16 * lg);
                    dv = drow[j][(k0 + kk) / 32 + (lg >> 1)];
                }
                const _Float16 dh = __builtin_bit_cast(_Float16, dv);
                const h2 d2 = {dh, dh};
                bf[j][0] = frag_q8_0(q.x, q.y, d2);
                bf[j][1] = frag_q8_0(q.z, q.w, d2);
            }
#pragma unroll
            for (int t = 0; t < 2; t++) {
#pragma unroll
                for (int i = 0; i < MB; i++) {
                    const h8 af = lds_frag(&sm.a[(16 * i + ln) * LDA + kk + 16 * lg + 8 * t]);
#pragma unroll
                    for (int j = 0; j < NB; j++) acc[i][j] = mfma(af, bf[j][t], acc[i][j]);
                }
            }
        }
    }
    // D layout: lane holds column ln, rows 4*lg + e
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const int n = nw + 16 * j + ln;
        if (n >= N) continue;
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + 16 * i + 4 * lg + e;
                if (m < M) store_out(C, (size_t)m * N + n, acc[i][j][e], c_f32, accumulate);
            }
    }
}

template <int MB, int NB>
__global__ void __launch_bounds__(256) k_gemm_q4_k(const uint8_t *__restrict__ W, size_t row_bytes,
                                                   const uint16_t *__restrict__ A, int M, int N, int K, void *C,
                                                   int c_f32, int accumulate) {
    __shared__ Smem<MB> sm;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ln = lane & 15, lg = lane >> 4;
    const int m0 = blockIdx.y * 16 * MB, nw = blockIdx.x * 64 * NB + wave * 16 * NB;
    f4 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    const uint8_t *wrow[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) {
        int n = nw + 16 * j + ln;
        n = n < N ? n : N - 1;
        wrow[j] = W + (size_t)n * row_bytes;
    }
    // Lane (ln, lg) loads chunk c = 4L + lg (L = 0, 1) of the 128 quant bytes: p = 2L + lg/2,
    // h = lg%2. MFMA i = 4L + t: t = 0/1 low nibbles of bytes 0-7 / 8-15, t = 2/3 high nibbles;
    // its activations start at k = 64p + 16h + 8(t&1) + 32(t>>1); its sub-block is 2p + (t>>1).
    const int pA = lg >> 1, hA = lg & 1;
    for (int k0 = 0; k0 < K; k0 += KC) {
        __syncthreads();
        stage_a<MB>(sm, A, M, K, m0, k0, KC);
        __syncthreads();
        stage_sums<MB>(sm);
        __syncthreads();
        const int sb = k0 / 256;
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const uint8_t *b = wrow[j] + (size_t)sb * 144;
            const u4v hdr = *(const u4v *)b;
            const u4v q0 = *(const u4v *)(b + 16 + 16 * lg);
            const u4v q1 = *(const u4v *)(b + 16 + 64 + 16 * lg);
            uint32_t sw0, sw1, mw0, mw1;
            q4k_scale_words(hdr.y, hdr.z, hdr.w, sw0, sw1, mw0, mw1);
            // scales of this lane's sub-blocks: L=0 -> subs 2pA, 2pA+1 (sw0); L=1 -> 4+2pA, 5+2pA (sw1)
            h2 mulL[2][2], addL[2][2];  // [L][nibble half]
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
            h8 bf[8];
            bf[0] = frag_q4_k<false>(q0.x, q0.y, mulL[0][0], addL[0][0]);
            bf[1] = frag_q4_k<false>(q0.z, q0.w, mulL[0][0], addL[0][0]);
            bf[2] = frag_q4_k<true>(q0.x, q0.y, mulL[0][1], addL[0][1]);
            bf[3] = frag_q4_k<true>(q0.z, q0.w, mulL[0][1], addL[0][1]);
            bf[4] = frag_q4_k<false>(q1.x, q1.y, mulL[1][0], addL[1][0]);
            bf[5] = frag_q4_k<false>(q1.z, q1.w, mulL[1][0], addL[1][0]);
            bf[6] = frag_q4_k<true>(q1.x, q1.y, mulL[1][1], addL[1][1]);
            bf[7] = frag_q4_k<true>(q1.z, q1.w, mulL[1][1], addL[1][1]);
            // min-term operand: lanes lg 0,1 -> -(dmin*m) hi, lanes 2,3 -> lo; k-slot e = sub-block e
            const float dmin = h2f((uint16_t)(hdr.x >> 16));
            h8 bmin;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float v = dmin * (float)byte_of(e < 4 ? mw0 : mw1, e & 3);
                const _Float16 vh = (_Float16)v;
                bmin[e] = lg < 2 ? -vh : -(_Float16)(v - (float)vh);
            }
            const float d = h2f((uint16_t)hdr.x);
#pragma unroll
            for (int i = 0; i < MB; i++) {
                const _Float16 *arow = &sm.a[(16 * i + ln) * LDA];
                f4 part = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int L = 0; L < 2; L++)
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const int kA = 64 * (2 * L + pA) + 16 * hA + 8 * (t & 1) + 32 * (t >> 1);
                        part = mfma(lds_frag(arow + kA), bf[4 * L + t], part);
                    }
                acc[i][j] += part * d;
                // A side of the min term: lanes lg 0,2 -> S hi, lanes 1,3 -> S lo
                const h8 as = lds_frag(&sm.s[(16 * i + ln) * 16 + 8 * (lg & 1)]);
                acc[i][j] = mfma(as, bmin, acc[i][j]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const int n = nw + 16 * j + ln;
        if (n >= N) continue;
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + 16 * i + 4 * lg + e;
                if (m < M) store_out(C, (size_t)m * N + n, acc[i][j][e], c_f32, accumulate);
            }
    }
}

// ============================================================================ misc
__global__ void __launch_bounds__(256) k_f32_to_f16(const float *__restrict__ in, uint16_t *__restrict__ out,
                                                    size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = __builtin_bit_cast(uint16_t, (_Float16)in[i]);
}

// ============================================================================ launchers
static unsigned grid_for(size_t n, unsigned per, unsigned cap) {
    size_t g = (n + per - 1) / per;
    return (unsigned)(g < cap ? (g ? g : 1) : cap);
}

hipError_t hq_launch_dequant(const hq_dev_mat *W, uint32_t row0, const uint32_t *ids, uint32_t nrows, float *out,
                             hipStream_t st) {
    if (W->type == HQ_TYPE_Q8_0) {
        const size_t n = (size_t)nrows * W->cols / 4;
        k_dequant_q8_0<<<grid_for(n, 256, 65536), 256, 0, st>>>(W->qs, W->d, W->cols, W->ldd, row0, ids, nrows, out);
    } else {
        const size_t n = (size_t)nrows * W->cols / 8;
        k_dequant_q4_k<<<grid_for(n, 256, 65536), 256, 0, st>>>(W->qs, W->row_bytes, W->cols, row0, ids, nrows, out);
    }
    return hipGetLastError();
}

hipError_t hq_launch_gemv(const hq_dev_mat *W, const uint16_t *a, void *C, int c_f32, int accumulate, hipStream_t st) {
    const int N = (int)W->rows, K = (int)W->cols;
    const unsigned g = (unsigned)((N + 15) / 16);
    if (W->type == HQ_TYPE_Q8_0)
        k_gemv_q8_0<<<g, 256, 0, st>>>(W->qs, W->d, W->ldd, a, N, K, C, c_f32, accumulate);
    else
        k_gemv_q4_k<<<g, 256, 0, st>>>(W->qs, W->row_bytes, a, N, K, C, c_f32, accumulate);
    return hipGetLastError();
}

hipError_t hq_launch_gather(const hq_dev_mat *W, const uint16_t *H, const uint32_t *ids, int B, int k, float *out,
                            hipStream_t st) {
    const int pairs = B * k, K = (int)W->cols;
    const unsigned g = (unsigned)((pairs + 15) / 16);
    if (W->type == HQ_TYPE_Q8_0)
        k_gather_q8_0<<<g, 256, 0, st>>>(W->qs, W->d, W->ldd, H, ids, pairs, k, K, W->rows, out);
    else
        k_gather_q4_k<<<g, 256, 0, st>>>(W->qs, W->row_bytes, H, ids, pairs, k, K, W->rows, out);
    return hipGetLastError();
}

template <int MB, int NB>
static void launch_gemm_t(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                          hipStream_t st) {
    const int N = (int)W->rows, K = (int)W->cols;
    dim3 grid((unsigned)((N + 64 * NB - 1) / (64 * NB)), (unsigned)((M + 16 * MB - 1) / (16 * MB)));
    if (W->type == HQ_TYPE_Q8_0)
        k_gemm_q8_0<MB, NB><<<grid, 256, 0, st>>>(W->qs, W->d, W->ldd, A, M, N, K, C, c_f32, accumulate);
    else
        k_gemm_q4_k<MB, NB><<<grid, 256, 0, st>>>(W->qs, W->row_bytes, A, M, N, K, C, c_f32, accumulate);
}

// Tile choice: MB (16-row blocks of M per tile) grows with M up to 8; NB (16-column blocks per
// wave) is picked to minimise ceil(tiles / 256 CUs) * tile area, i.e. wave quantization.
void hq_gemm_config(int M, int N, int *mb, int *nb) {
    int m = M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8;
    const int mt = (M + 16 * m - 1) / (16 * m);
    int best = 1;
    double best_cost = 1e300;
    for (int n = 1; n <= 4; n++) {
        const long tiles = (long)mt * ((N + 64 * n - 1) / (64 * n));
        const long rounds = (tiles + 255) / 256;
        const double cost = (double)rounds * (16.0 * m) * (64.0 * n) * (1.0 + 0.08 / n);
        if (cost < best_cost - 1e-9) best_cost = cost, best = n;
    }
    *mb = m;
    *nb = best;
}

hipError_t hq_launch_gemm(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                          hipStream_t st) {
    int mb, nb;
    hq_gemm_config(M, (int)W->rows, &mb, &nb);
#define CASE(a, b) \
    if (mb == a && nb == b) return launch_gemm_t<a, b>(W, A, M, C, c_f32, accumulate, st), hipGetLastError();
#define ROW(a) CASE(a, 1) CASE(a, 2) CASE(a, 3) CASE(a, 4)
    ROW(1) ROW(2) ROW(4) ROW(8)
#undef ROW
#undef CASE
    return hipErrorInvalidValue;
}

hipError_t hq_launch_f32_to_f16(const float *in, uint16_t *out, size_t n, hipStream_t st) {
    k_f32_to_f16<<<grid_for(n, 256, 16384), 256, 0, st>>>(in, out, n);
    return hipGetLastError();
}
