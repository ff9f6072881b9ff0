// hq_kquant.hip - GGUF Q2_K, Q3_K and Q5_K matrices on gfx950: decode, GEMV (M = 1), option-row gather
// and the MFMA GEMM (M >= 2). Formats, device slots and the exact decode are in hq_kquant.h.
//
// Kernels (one template per kernel, instantiated for the three types)
//   k_dequant_kq  rows -> fp32, bit-identical to the reference decoder.
//   k_gemv_kq     M = 1: one wave per output row, lanes over 16-value chunks, exact fp32 weights,
//                 fp32 sums (HBM-bound).
//   k_gather_kq   option-row readout: the GEMV loop over (state, id) pairs.
//   k_gemm_kq     M >= 2: the Stream-K MFMA kernel of hq_sk.h (tile 16 MB x 128, K-units of one
//                 super-block). No weight is rounded to 16 bits: each weight is d * B1 - dmin * B2
//                 with B1, B2 exact fp16 integers per 8 consecutive k of a lane:
//                   Q5_K  B1 = s * q (q <= 31, s <= 63: <= 1953)   B2 = m (the sub-block's min code)
//                   Q2_K  B1 = (sm & 15) * q (<= 45)                B2 = sm >> 4
//                   Q3_K  B1 = (sc - 32) * q (-124 .. 128)           no B2
//                 so a k-step issues one MFMA per term into two fp32 unit accumulators, and at the end
//                 of the unit the tile accumulator adds d * U1 - dmin * U2 (the column's d and dmin).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hq_device.h"
#include "hq_kernels.h"
#include "hq_kquant.h"
#include "hq_sk.h"

namespace {

// one thread per (row, 16-value chunk); output row r is matrix row ids[r] when ids is given
template <int T>
__global__ void __launch_bounds__(256) k_dequant_kq(const uint8_t *__restrict__ W, size_t row_bytes, int K, uint32_t row0,
                                                    const uint32_t *__restrict__ ids, uint32_t nrows, float *__restrict__ out) {
    const size_t per_row = (size_t)K / 16, total = (size_t)nrows * per_row;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / per_row, v0 = (i % per_row) * 16, row = ids ? (size_t)ids[r] : row0 + r;
        const uint8_t *blk = W + row * row_bytes + (v0 / 256) * kq_slot(T);
        float w[2][8];
        kq_deq8<T>(blk, (int)(v0 % 256), w[0]);
        kq_deq8<T>(blk, (int)(v0 % 256) + 8, w[1]);
        float4 *o = (float4 *)(out + r * (size_t)K + v0);
#pragma unroll
        for (int q = 0; q < 4; q++) o[q] = float4{w[q >> 1][4 * (q & 1)], w[q >> 1][4 * (q & 1) + 1], w[q >> 1][4 * (q & 1) + 2],
                                                   w[q >> 1][4 * (q & 1) + 3]};
    }
}

// dot of one row with fp16 activations a [K]: lane j of 64 takes 16-value chunks j, j + 64, ...
template <int T>
DEV float kq_row_dot(const uint8_t *__restrict__ row, const uint16_t *__restrict__ a, int K, int j) {
    float acc = 0.f;
    for (int c = j; c < K / 16; c += 64) {
        const uint8_t *blk = row + (size_t)(c >> 4) * kq_slot(T);
        const h8 a0 = *(const h8 *)(a + 16 * c), a1 = *(const h8 *)(a + 16 * c + 8);
        float w[8];
        kq_deq8<T>(blk, (c & 15) * 16, w);
#pragma unroll
        for (int e = 0; e < 8; e++) acc = fmaf(w[e], (float)a0[e], acc);
        kq_deq8<T>(blk, (c & 15) * 16 + 8, w);
#pragma unroll
        for (int e = 0; e < 8; e++) acc = fmaf(w[e], (float)a1[e], acc);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    return acc;
}

// M = 1: one wave per output row
template <int T>
__global__ void __launch_bounds__(256) k_gemv_kq(const uint8_t *__restrict__ W, size_t row_bytes, const uint16_t *__restrict__ a,
                                                 int N, int K, void *C, int c_f32, int accumulate) {
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6), j = threadIdx.x & 63;
    if (n >= N) return;
    const float v = kq_row_dot<T>(W + (size_t)n * row_bytes, a, K, j);
    if (j == 0) store_out(C, (size_t)n, v, c_f32, accumulate);
}

// out[i] = dot(H[i / k], W[ids[i]]); an id >= rows stores NaN and reads row 0 instead
template <int T>
__global__ void __launch_bounds__(256) k_gather_kq(const uint8_t *__restrict__ W, size_t row_bytes, const uint16_t *__restrict__ H,
                                                   const uint32_t *__restrict__ ids, int pairs, int k, int K, uint32_t rows,
                                                   float *__restrict__ out) {
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6), j = threadIdx.x & 63;
    if (i >= pairs) return;
    const uint32_t id = ids[i];
    const float v = kq_row_dot<T>(W + (size_t)(id < rows ? id : 0) * row_bytes, H + (size_t)(i / k) * K, K, j);
    if (j == 0) out[i] = id < rows ? v : __builtin_nanf("");
}

// ---------------------------------------------------------------------------------------- GEMM
// Eight fp16 values (b - bias) * f for the 8 bytes b of words w0, w1 (b + 1024 - bias an exact small
// integer, f an fp16 integer whose product with it is exact).
DEV h8 scaled_bytes(uint32_t w0, uint32_t w1, _Float16 bias, _Float16 f) {
    const h2 k = {(_Float16)1024.0f + bias, (_Float16)1024.0f + bias}, ff = {f, f};
    const uint32_t w[2] = {w0, w1};
    h8 out;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const h2 x = (as_h2(perm_lo(w[i])) - k) * ff, y = (as_h2(perm_hi(w[i])) - k) * ff;
        out[4 * i] = x.x, out[4 * i + 1] = x.y, out[4 * i + 2] = y.x, out[4 * i + 3] = y.y;
    }
    return out;
}

DEV h8 splat8(_Float16 x) { return h8{x, x, x, x, x, x, x, x}; }

// Per-type lane loads of one super-block (NL 16-byte pieces at offsets off(i, lg) of the slot) and
// the B fragments of k-step (s, e): the lane's values 64 s + 16 lg + 8 e .. + 7 of the super-block.
template <int T>
struct KqB;

// Q5_K: pieces 0 header {d, dmin, scales}, 1 qh[16 (lg & 1) ..], 2 + s ql[32 s + 16 (lg & 1) ..]. The
// lane's values lie in sub-block 2 s + (lg >> 1), nibble lg >> 1 of its ql bytes.
template <>
struct KqB<HQ_TYPE_Q5_K> {
    static constexpr int NL = 6, HAS_MIN = 1;
    DEV uint32_t off(int i, int lg) { return i == 0 ? 0u : i == 1 ? 16u + 16u * (lg & 1) : 48u + 32u * (i - 2) + 16u * (lg & 1); }
    DEV void frags(const u4v (&x)[NL], int s, int e, int lg, h8 &b1, h8 &b2) {
        const int sub = 2 * s + (lg >> 1);
        uint32_t sw0, sw1, mw0, mw1;
        q4k_scale_words(x[0].y, x[0].z, x[0].w, sw0, sw1, mw0, mw1);
        const uint32_t sc = byte_of(sub < 4 ? sw0 : sw1, sub & 3), mn = byte_of(sub < 4 ? mw0 : mw1, sub & 3);
        const int sh = 4 * (lg >> 1);
        const uint32_t q0 = ((x[2 + s][2 * e] >> sh) & 0x0f0f0f0fu) | (((x[1][2 * e] >> sub) & 0x01010101u) << 4);
        const uint32_t q1 = ((x[2 + s][2 * e + 1] >> sh) & 0x0f0f0f0fu) | (((x[1][2 * e + 1] >> sub) & 0x01010101u) << 4);
        b1 = scaled_bytes(q0, q1, (_Float16)0.0f, (_Float16)(float)sc);
        b2 = splat8((_Float16)(float)mn);
    }
    DEV void scales(const u4v (&x)[NL], float &d, float &dmin) {
        d = h2f((uint16_t)x[0].x);
        dmin = h2f((uint16_t)(x[0].x >> 16));
    }
};

// Q2_K: pieces 0 scales[16], 1 {d, dmin}, 2 + h qs[32 h + 16 (lg & 1) ..]. The lane's values of
// k-step (s, e) are in half h = s / 2, bit pair j = 2 (s % 2) + (lg >> 1), scale byte 8 h + 2 j + (lg & 1).
template <>
struct KqB<HQ_TYPE_Q2_K> {
    static constexpr int NL = 4, HAS_MIN = 1;
    DEV uint32_t off(int i, int lg) { return i == 0 ? 0u : i == 1 ? 80u : 16u + 32u * (i - 2) + 16u * (lg & 1); }
    DEV void frags(const u4v (&x)[NL], int s, int e, int lg, h8 &b1, h8 &b2) {
        const int h = s >> 1, j = 2 * (s & 1) + (lg >> 1);
        const uint32_t sm = byte_of(x[0][2 * h + (s & 1)], lg);  // byte 8 h + 2 j + (lg & 1) = 4 (2 h + s % 2) + lg
        const uint32_t q0 = (x[2 + h][2 * e] >> (2 * j)) & 0x03030303u, q1 = (x[2 + h][2 * e + 1] >> (2 * j)) & 0x03030303u;
        b1 = scaled_bytes(q0, q1, (_Float16)0.0f, (_Float16)(float)(sm & 15u));
        b2 = splat8((_Float16)(float)(sm >> 4));
    }
    DEV void scales(const u4v (&x)[NL], float &d, float &dmin) {
        d = h2f((uint16_t)x[1].x);
        dmin = h2f((uint16_t)(x[1].x >> 16));
    }
};

// Q3_K: pieces 0 {scales[12], d}, 1 hmask[16 (lg & 1) ..], 2 + h qs[32 h + 16 (lg & 1) ..]; bit pair
// j = 2 (s % 2) + (lg >> 1) of the quants, hmask bit 4 h + j, scale 8 h + 2 j + (lg & 1).
template <>
struct KqB<HQ_TYPE_Q3_K> {
    static constexpr int NL = 4, HAS_MIN = 0;
    DEV uint32_t off(int i, int lg) { return i == 0 ? 96u : i == 1 ? 16u * (lg & 1) : 32u + 32u * (i - 2) + 16u * (lg & 1); }
    DEV void frags(const u4v (&x)[NL], int s, int e, int lg, h8 &b1, h8 &) {
        // scale 8 h + 2 j + (lg & 1) = 4 g + lg with g = 2 h + s % 2 (the code layout of hq_kquant.h)
        const int h = s >> 1, j = 2 * (s & 1) + (lg >> 1), g = 2 * h + (s & 1);
        const uint32_t lo = (byte_of(x[0][g & 1], lg) >> (4 * (g >> 1))) & 15u;
        const uint32_t hi = (byte_of(x[0][2], lg) >> (2 * g)) & 3u;
        const int sc = (int)(lo | (hi << 4)) - 32;
        const uint32_t q0 = ((x[2 + h][2 * e] >> (2 * j)) & 0x03030303u) | (((x[1][2 * e] >> (4 * h + j)) & 0x01010101u) << 2);
        const uint32_t q1 = ((x[2 + h][2 * e + 1] >> (2 * j)) & 0x03030303u) | (((x[1][2 * e + 1] >> (4 * h + j)) & 0x01010101u) << 2);
        b1 = scaled_bytes(q0, q1, (_Float16)4.0f, (_Float16)(float)sc);  // (q' - 4) * (sc - 32), q' = q2 + 4 hb
    }
    DEV void scales(const u4v (&x)[NL], float &d, float &dmin) {
        d = h2f((uint16_t)x[0].w);
        dmin = 0.f;
    }
};

// Stream-K GEMM (structure of k_gemm_q6_k in hq_q6k.hip): tile 16 MB rows x 64 NB columns per wave-set
// of 4 waves, K-units of one super-block; lane (ln, lg) of column block j loads its column's NL pieces.
template <int T, int MB, int NB>
__global__ void __launch_bounds__(256) k_gemm_kq(GemmArgs g) {
    using D = KqB<T>;
    constexpr int NL = D::NL;
    __shared__ __attribute__((aligned(16))) _Float16 sa[2][16 * MB * KC];
    __shared__ int s_flag;
    const SkPlan &p = g.plan;
    const int w = sk_worker(p.G), u0 = sk_start(p, w), u1 = sk_start(p, w + 1);
    const rsrc_t rpart = make_rsrc(g.partials, g.partial_bytes);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ln = lane & 15, lg = lane >> 4;
    const int M = g.M, N = g.N, K = g.K;
    const rsrc_t ra = make_rsrc(g.A, (uint32_t)((size_t)M * K * 2));
    const rsrc_t rw = make_rsrc(g.qs, (uint32_t)((size_t)N * g.row_bytes));  // rows >= N read as zero
    ADma adma;
    uint32_t vrow[NB];
    auto tile_setup = [&](int tile) {
        const int m0 = (tile % p.tm) * 16 * MB, nw = (tile / p.tm) * 64 * NB + wave * 16 * NB;
        adma = adma_setup<MB>(K, m0);
#pragma unroll
        for (int j = 0; j < NB; j++) vrow[j] = (uint32_t)(nw + 16 * j + ln) * (uint32_t)g.row_bytes;
    };
    auto load_w = [&](int unit, u4v (&x)[NB][NL]) {
        const uint32_t base = (uint32_t)unit * (uint32_t)kq_slot(T);
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
            for (int i = 0; i < NL; i++) x[j][i] = buf_load16(rw, vrow[j], base + D::off(i, lg));
    };
    f4 acc[MB][NB];
    u4v wc[NB][NL];
    int cur_tile = u0 / p.upt;
    tile_setup(cur_tile);
    dma_a<MB>(sa[0], ra, adma, K, (u0 % p.upt) * KC);
    load_w(u0 % p.upt, wc);
    for (int u = u0; u < u1; u++) {
        const int cb = (u - u0) & 1, tile = u / p.upt, ku = u % p.upt;
        const int m0 = (tile % p.tm) * 16 * MB, nw = (tile / p.tm) * 64 * NB + wave * 16 * NB;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        u4v wn[NB][NL];
        if (u + 1 < u1) {
            const int t1 = (u + 1) / p.upt;
            if (t1 != cur_tile) {
                cur_tile = t1;
                tile_setup(t1);
            }
            dma_a<MB>(sa[cb ^ 1], ra, adma, K, ((u + 1) % p.upt) * KC);
            load_w((u + 1) % p.upt, wn);
        }
        if (u == u0 || ku == 0) {
#pragma unroll
            for (int i = 0; i < MB; i++)
#pragma unroll
                for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
        }
        f4 au[MB][NB], am[MB][NB];
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) au[i][j] = am[i][j] = f4{0.f, 0.f, 0.f, 0.f};
        const _Float16 *buf = sa[cb];
#pragma unroll
        for (int f = 0; f < 8; f++) {
            const int s = f >> 1, e = f & 1;
            h8 b1[NB], b2[NB];
#pragma unroll
            for (int j = 0; j < NB; j++) D::frags(wc[j], s, e, lg, b1[j], b2[j]);
#pragma unroll
            for (int i = 0; i < MB; i++) {
                const h8 af = a_frag(buf, 16 * i + ln, 8 * s + 2 * lg + e);
#pragma unroll
                for (int j = 0; j < NB; j++) {
                    au[i][j] = mfma(af, b1[j], au[i][j]);
                    if constexpr (D::HAS_MIN) am[i][j] = mfma(af, b2[j], am[i][j]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < NB; j++) {
            float d, dmin;
            D::scales(wc[j], d, dmin);
#pragma unroll
            for (int i = 0; i < MB; i++) {
                acc[i][j] += au[i][j] * d;
                if constexpr (D::HAS_MIN) acc[i][j] -= am[i][j] * dmin;
            }
        }
        if (ku == p.upt - 1 || u == u1 - 1)
            finish_tile<MB, NB, 256>(acc, p, w, u0, u1, tile, &s_flag, rpart, g.counters, g.C, M, N, m0, nw, ln, lg, g.c_f32,
                                     g.accumulate);
        if (u + 1 < u1) {
#pragma unroll
            for (int j = 0; j < NB; j++)
#pragma unroll
                for (int i = 0; i < NL; i++) wc[j][i] = wn[j][i];
        }
    }
}

unsigned grid_cap(size_t n, unsigned per, unsigned cap) {
    const size_t gsz = (n + per - 1) / per;
    return (unsigned)(gsz < cap ? (gsz ? gsz : 1) : cap);
}

template <int T>
hipError_t gemm_t(const GemmArgs &g, int mb, hipStream_t st) {
    switch (mb) {
    case 1: k_gemm_kq<T, 1, 2><<<g.plan.G, 256, 0, st>>>(g); break;
    case 2: k_gemm_kq<T, 2, 2><<<g.plan.G, 256, 0, st>>>(g); break;
    case 4: k_gemm_kq<T, 4, 2><<<g.plan.G, 256, 0, st>>>(g); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
}  // namespace

#define KQ_SWITCH(type, CALL)                                      \
    switch (type) {                                                \
    case HQ_TYPE_Q2_K: CALL(HQ_TYPE_Q2_K); break;                  \
    case HQ_TYPE_Q3_K: CALL(HQ_TYPE_Q3_K); break;                  \
    case HQ_TYPE_Q5_K: CALL(HQ_TYPE_Q5_K); break;                  \
    default: return hipErrorInvalidValue;                          \
    }

hipError_t hq_launch_dequant_kq(const hq_dev_mat *W, uint32_t row0, const uint32_t *ids, uint32_t nrows, float *out,
                                hipStream_t st) {
    const size_t n = (size_t)nrows * (W->cols / 16);
#define DQ(t) k_dequant_kq<t><<<grid_cap(n, 256, 65536), 256, 0, st>>>(W->qs, W->row_bytes, (int)W->cols, row0, ids, nrows, out)
    KQ_SWITCH(W->type, DQ)
#undef DQ
    return hipGetLastError();
}

hipError_t hq_launch_gemv_kq(const hq_dev_mat *W, const uint16_t *a, void *C, int c_f32, int accumulate, hipStream_t st) {
#define GV(t) k_gemv_kq<t><<<(W->rows + 3) / 4, 256, 0, st>>>(W->qs, W->row_bytes, a, (int)W->rows, (int)W->cols, C, c_f32, accumulate)
    KQ_SWITCH(W->type, GV)
#undef GV
    return hipGetLastError();
}

hipError_t hq_launch_gather_kq(const hq_dev_mat *W, const uint16_t *H, const uint32_t *ids, int B, int k, float *out,
                               hipStream_t st) {
    const int pairs = B * k;
#define GA(t) k_gather_kq<t><<<(pairs + 3) / 4, 256, 0, st>>>(W->qs, W->row_bytes, H, ids, pairs, k, (int)W->cols, W->rows, out)
    KQ_SWITCH(W->type, GA)
#undef GA
    return hipGetLastError();
}

hipError_t hq_launch_gemm_kq(int type, const GemmArgs &g, int mb, hipStream_t st) {
    switch (type) {
    case HQ_TYPE_Q2_K: return gemm_t<HQ_TYPE_Q2_K>(g, mb, st);
    case HQ_TYPE_Q3_K: return gemm_t<HQ_TYPE_Q3_K>(g, mb, st);
    case HQ_TYPE_Q5_K: return gemm_t<HQ_TYPE_Q5_K>(g, mb, st);
    default: return hipErrorInvalidValue;
    }
}
