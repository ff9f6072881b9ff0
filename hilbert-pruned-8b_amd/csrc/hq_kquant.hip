// hq_kquant.hip - GGUF Q2_K, Q3_K and Q5_K matrices on gfx950: decode, GEMV (M = 1), option-row gather
// and the MFMA GEMM (M >= 2); the GEMV and gather also serve Q6_K. Formats, device slots and the exact
// decode are in hq_kquant.h.
//
// Kernels (one template per kernel, instantiated per type)
//   k_dequant_kq  rows -> fp32, bit-identical to the reference decoder.
//   k_gemv_sb     M = 1 and the option-row gather (Q2_K, Q3_K, Q5_K, Q6_K): lane tasks of one eighth
//                 of a super-block, exact fp16 integers in v_dot2_f32_f16, R rows per wave (HBM-bound).
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

// ------------------------------------------------------------------ GEMV / gather by super-block eighths
// A lane task is one eighth of a super-block of one row: 32 values, read with its own 8- or 16-byte
// loads (the eight lanes of a super-block are neighbours, so a super-block's bytes arrive as whole
// lines and its scale bytes as one broadcast load). The quantized integers become exact fp16 values
// (fp16 1024 + u from v_perm_b32, minus 1024 + bias) and meet the fp16 activations in v_dot2_f32_f16
// (exact products, fp32 sums); the scale, and for Q2_K / Q5_K the min against the activations' fp32
// sum, are applied per 8 or 16 values in fp32. A wave holds RW rows, 64 / RW lanes each: eight per
// super-block and S = 8 / RW super-blocks side by side, so a lane walks K / 256 / S super-blocks of its
// row with the next one's loads in flight while it computes the current one.

// 8 values: the bytes of w0, w1 (exact integers u <= 63), minus kb - 1024, dotted with the 8 fp16 a
DEV float dotu8(uint32_t w0, uint32_t w1, const u4v a, h2 kb, float s) {
    const h2 q[4] = {as_h2(perm_lo(w0)) - kb, as_h2(perm_hi(w0)) - kb, as_h2(perm_lo(w1)) - kb, as_h2(perm_hi(w1)) - kb};
    return dot8(q, a, s);
}

DEV h2 splat2(float x) { return h2{(_Float16)x, (_Float16)x}; }

// The loaded bytes of one lane task: up to three weight pieces and four 8-value activation vectors.
struct SbRaw {
    u4v w0, w1, w2;
    u4v a[4];
};

// Loads of eighth p of the super-block at blk (device slot) and of its 256 activations a (global
// memory, or the workgroup's LDS copy of the vector).
//   Q2_K, Q3_K, Q6_K: values 128 h + 32 j + l0 .. + 7 for j = 0 .. 3 (h = p / 4, l0 = 8 (p % 4)).
//   Q5_K: values 16 (p % 2) .. + 15 of sub-blocks 2 (p / 2) and 2 (p / 2) + 1.
template <int T, class AP>
DEV void sb_load_a(SbRaw &x, AP a, int p) {
    if constexpr (T == HQ_TYPE_Q5_K) {
        const int sp = p >> 1, l0 = 16 * (p & 1);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            x.a[2 * t] = ld_a16(a + 32 * (2 * sp + t) + l0);
            x.a[2 * t + 1] = ld_a16(a + 32 * (2 * sp + t) + l0 + 8);
        }
    } else {
        const int h = p >> 2, l0 = 8 * (p & 3);
#pragma unroll
        for (int j = 0; j < 4; j++) x.a[j] = ld_a16(a + 128 * h + 32 * j + l0);
    }
}
template <int T>
DEV void sb_load_w(SbRaw &x, const uint8_t *__restrict__ blk, int p) {
    if constexpr (T == HQ_TYPE_Q5_K) {
        const int sp = p >> 1, l0 = 16 * (p & 1);
        x.w0 = *(const u4v *)blk;                          // d, dmin, scales[12]
        x.w1 = *(const u4v *)(blk + 48 + 32 * sp + l0);    // qs
        x.w2 = *(const u4v *)(blk + 16 + l0);              // qh
    } else {
        const int h = p >> 2, l0 = 8 * (p & 3);
        if constexpr (T == HQ_TYPE_Q2_K) {
            x.w0 = *(const u4v *)blk;  // scales[16]
            const u2v qs = *(const u2v *)(blk + 16 + 32 * h + l0);
            x.w1 = u4v{qs.x, qs.y, *(const uint32_t *)(blk + 80), 0u};  // qs, {d, dmin}
        } else if constexpr (T == HQ_TYPE_Q3_K) {
            x.w0 = *(const u4v *)(blk + 96);  // scales[12], d
            const u2v qs = *(const u2v *)(blk + 32 + 32 * h + l0), hm = *(const u2v *)(blk + l0);
            x.w1 = u4v{qs.x, qs.y, hm.x, hm.y};
        } else {
            static_assert(T == HQ_TYPE_Q6_K, "k-quant type");
            x.w0 = *(const u4v *)(blk + 192);  // int8 scales[16]
            const u2v q0 = *(const u2v *)(blk + 64 * h + l0), q1 = *(const u2v *)(blk + 64 * h + 32 + l0);
            const u2v qh = *(const u2v *)(blk + 128 + 32 * h + l0);
            x.w1 = u4v{q0.x, q0.y, q1.x, q1.y};
            x.w2 = u4v{qh.x, qh.y, (uint32_t)*(const uint16_t *)(blk + 208), 0u};  // qh, d
        }
    }
}

// The lane task's dot product from its loaded bytes. For Q2_K, Q3_K, Q6_K the scale of group j is
// number 8 h + 2 j + (l0 >> 4): word 2 h + (j >> 1), byte 2 (j & 1) + (l0 >> 4) of the scale vector.
template <int T>
DEV float sb_dot(const SbRaw &x, int p) {
    float r = 0.f;
    if constexpr (T == HQ_TYPE_Q5_K) {
        // sub-block j = 2 sp + t: nibble t of the qs bytes, qh bit j; q = u (0 .. 31)
        const int sp = p >> 1;
        uint32_t sw0, sw1, mw0, mw1;
        q4k_scale_words(x.w0.y, x.w0.z, x.w0.w, sw0, sw1, mw0, mw1);
        const float d = h2f((uint16_t)x.w0.x), dm = h2f((uint16_t)(x.w0.x >> 16));
        const h2 kb = splat2(1024.0f);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int j = 2 * sp + t;
            uint32_t u[4];
#pragma unroll
            for (int w = 0; w < 4; w++) u[w] = ((x.w1[w] >> (4 * t)) & 0x0f0f0f0fu) | (((x.w2[w] >> j) & 0x01010101u) << 4);
            const float dq = dotu8(u[2], u[3], x.a[2 * t + 1], kb, dotu8(u[0], u[1], x.a[2 * t], kb, 0.f));
            const float sa = sum8(x.a[2 * t + 1], sum8(x.a[2 * t], 0.f));
            const uint32_t s = byte_of(j < 4 ? sw0 : sw1, j & 3), m = byte_of(j < 4 ? mw0 : mw1, j & 3);
            r += d * (float)s * dq - dm * (float)m * sa;
        }
    } else {
        const int h = p >> 2, hl = (p & 3) >> 1;  // hl = l0 >> 4
        if constexpr (T == HQ_TYPE_Q2_K) {
            // q = u (0 .. 3); scale byte sm: d (sm & 15), min dmin (sm >> 4)
            const float d = h2f((uint16_t)x.w1.z), dm = h2f((uint16_t)(x.w1.z >> 16));
            const h2 kb = splat2(1024.0f);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t sm = byte_of(x.w0[2 * h + (j >> 1)], 2 * (j & 1) + hl);
                const float dq = dotu8((x.w1.x >> (2 * j)) & 0x03030303u, (x.w1.y >> (2 * j)) & 0x03030303u, x.a[j], kb, 0.f);
                r += d * (float)(sm & 15u) * dq - dm * (float)(sm >> 4) * sum8(x.a[j], 0.f);
            }
        } else if constexpr (T == HQ_TYPE_Q3_K) {
            // u = q2 + 4 hb (0 .. 7), q = u - 4; the 6-bit scale codes as in q3k_code (e = 4 g + i)
            const float d = h2f((uint16_t)x.w0.w);
            const h2 kb = splat2(1028.0f);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int g = 2 * h + (j >> 1), i = 2 * (j & 1) + hl;
                const int s = (int)(((byte_of(g & 1 ? x.w0.y : x.w0.x, i) >> (4 * (g >> 1))) & 15u) |
                                    (((byte_of(x.w0.z, i) >> (2 * g)) & 3u) << 4)) - 32;
                const uint32_t u0 = ((x.w1.x >> (2 * j)) & 0x03030303u) | (((x.w1.z >> (4 * h + j)) & 0x01010101u) << 2);
                const uint32_t u1 = ((x.w1.y >> (2 * j)) & 0x03030303u) | (((x.w1.w >> (4 * h + j)) & 0x01010101u) << 2);
                r += d * (float)s * dotu8(u0, u1, x.a[j], kb, 0.f);
            }
        } else {
            // j: low (j < 2) or high nibble of ql[64 h + 32 (j & 1) + l], bits 2 j, 2 j + 1 of
            // qh[32 h + l]; u = nibble | bits << 4 (0 .. 63), q = u - 32; signed 8-bit scales
            const float d = h2f((uint16_t)x.w2.z);
            const h2 kb = splat2(1056.0f);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t q0 = (j & 1) ? x.w1.z : x.w1.x, q1 = (j & 1) ? x.w1.w : x.w1.y;
                const int sh = j >= 2 ? 4 : 0;
                const uint32_t u0 = ((q0 >> sh) & 0x0f0f0f0fu) | (((x.w2.x >> (2 * j)) & 0x03030303u) << 4);
                const uint32_t u1 = ((q1 >> sh) & 0x0f0f0f0fu) | (((x.w2.y >> (2 * j)) & 0x03030303u) << 4);
                const int s = (int)(int8_t)byte_of(x.w0[2 * h + (j >> 1)], 2 * (j & 1) + hl);
                r += d * (float)s * dotu8(u0, u1, x.a[j], kb, 0.f);
            }
        }
    }
    return r;
}

// GATHER = false: C[o] = dot(W[o], a) for o < n_out = N (store_out modes). GATHER = true:
// out[o] = dot(W[ids[o]], a + (o / k_opts) K) for o < n_out = B k; an id >= rows stores NaN (its lanes
// read row 0). Rows of a wave past n_out compute row n_out - 1 and store nothing.
// LDSA (GEMV): the workgroup copies the activation vector into LDS once (dynamic shared memory of
// 2 K bytes) and every lane reads its activations from there: the lanes of a row together read 2 K
// bytes of activations per row against K / 4 .. 7 K / 8 bytes of weights, so from L2 / L1 they
// would set the pace. The first weight loads are issued before the copy.
template <int T, int RW, bool GATHER, bool LDSA>
__global__ void __launch_bounds__(256) k_gemv_sb(const uint8_t *__restrict__ W, size_t row_bytes,
                                                 const uint16_t *__restrict__ a, const uint32_t *__restrict__ ids,
                                                 int n_out, int k_opts, int K, uint32_t rows, void *C, int c_f32,
                                                 int accumulate) {
    static_assert(!(GATHER && LDSA), "the gather reads one activation vector per state");
    extern __shared__ __attribute__((aligned(16))) uint16_t sb_act[];
    constexpr int S = 8 / RW, G = 8 * S;  // super-blocks side by side, lanes per row
    const int lane = threadIdx.x & 63, o0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RW;
    if (!LDSA && o0 >= n_out) return;
    const int p = lane & 7, s = (lane >> 3) & (S - 1), o = o0 + lane / G, oc = min(o, n_out - 1);
    uint32_t row = (uint32_t)oc;
    const uint16_t *av = a;
    if constexpr (GATHER) {
        const uint32_t id = ids[oc];
        row = id < rows ? id : 0u;
        av = a + (size_t)(oc / k_opts) * K;
    }
    const int nsb = K >> 8;
    const uint8_t *base = W + (size_t)row * row_bytes;
    float acc = 0.f;
    int u = min(s, nsb - 1);
    SbRaw x;
    sb_load_w<T>(x, base + (size_t)u * kq_slot(T), p);
    auto act = [&]() {
        if constexpr (LDSA) return stage_act<256>(a, K, sb_act);  // every wave takes part
        else return av;
    }();
    if constexpr (LDSA) {
        __syncthreads();
        if (o0 >= n_out) return;  // (waves past n_out leave after the barrier)
    }
    sb_load_a<T>(x, act + 256 * u, p);
    for (u = s; u < nsb; u += S) {
        const int un = min(u + S, nsb - 1);  // the next super-block (the last one again at the end)
        SbRaw y;
        sb_load_w<T>(y, base + (size_t)un * kq_slot(T), p);
        sb_load_a<T>(y, act + 256 * un, p);
        acc += sb_dot<T>(x, p);
        x = y;
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((lane & (G - 1)) == 0 && o < n_out) {
        if constexpr (GATHER) ((float *)C)[o] = ids[o] < rows ? acc : __builtin_nanf("");
        else store_out(C, (size_t)o, acc, c_f32, accumulate);
    }
}


template <int T, bool GATHER>
hipError_t launch_sb(const hq_dev_mat *W, const uint16_t *a, const uint32_t *ids, int n_out, int k_opts, void *C, int c_f32,
                     int accumulate, hipStream_t st) {
    const int R = hq_sb_rows(n_out);
    const unsigned grid = (unsigned)(((n_out + R - 1) / R + 3) / 4);
    // the GEMV's activation vector in LDS (up to 64 KB: K <= 32768; not Q5_K, whose lanes read 16
    // contiguous values per sub-block and measured no faster from LDS)
    const bool lds = hq_sb_lds(T, (int)W->cols) && !GATHER;
    const size_t shm = lds ? (size_t)W->cols * 2 : 0;
#define SB(r)                                                                                                          \
    if (lds) k_gemv_sb<T, r, GATHER, !GATHER><<<grid, 256, shm, st>>>(W->qs, W->row_bytes, a, ids, n_out, k_opts,        \
                                                                     (int)W->cols, W->rows, C, c_f32, accumulate);    \
    else k_gemv_sb<T, r, GATHER, false><<<grid, 256, 0, st>>>(W->qs, W->row_bytes, a, ids, n_out, k_opts, (int)W->cols, \
                                                             W->rows, C, c_f32, accumulate)
    switch (R) {
    case 1: SB(1); break;
    case 2: SB(2); break;
    case 4: SB(4); break;
    default: SB(8); break;
    }
#undef SB
    return hipGetLastError();
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

// rows per wave of k_gemv_sb (GEMV and gather): two at n_out >= 8192 (K = 2560: 2432 waves), else one
// (K = 9728, N = 2560: eight super-blocks side by side); measured over 1 .. 8 rows on both headline shapes
int hq_sb_rows(int n_out) { return n_out >= 8192 ? 2 : 1; }

// whether the k-quant GEMV stages its activation vector in LDS (k_gemv_sb<T, RW, false, true>)
int hq_sb_lds(int type, int K) { return type != HQ_TYPE_Q5_K && K <= 32768; }

hipError_t hq_launch_gemv_kq(const hq_dev_mat *W, const uint16_t *a, void *C, int c_f32, int accumulate, hipStream_t st) {
    const int n = (int)W->rows;
    switch (W->type) {
    case HQ_TYPE_Q2_K: return launch_sb<HQ_TYPE_Q2_K, false>(W, a, nullptr, n, 1, C, c_f32, accumulate, st);
    case HQ_TYPE_Q3_K: return launch_sb<HQ_TYPE_Q3_K, false>(W, a, nullptr, n, 1, C, c_f32, accumulate, st);
    case HQ_TYPE_Q5_K: return launch_sb<HQ_TYPE_Q5_K, false>(W, a, nullptr, n, 1, C, c_f32, accumulate, st);
    case HQ_TYPE_Q6_K: return launch_sb<HQ_TYPE_Q6_K, false>(W, a, nullptr, n, 1, C, c_f32, accumulate, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t hq_launch_gather_kq(const hq_dev_mat *W, const uint16_t *H, const uint32_t *ids, int B, int k, float *out,
                               hipStream_t st) {
    const int pairs = B * k;
    switch (W->type) {
    case HQ_TYPE_Q2_K: return launch_sb<HQ_TYPE_Q2_K, true>(W, H, ids, pairs, k, out, 1, 0, st);
    case HQ_TYPE_Q3_K: return launch_sb<HQ_TYPE_Q3_K, true>(W, H, ids, pairs, k, out, 1, 0, st);
    case HQ_TYPE_Q5_K: return launch_sb<HQ_TYPE_Q5_K, true>(W, H, ids, pairs, k, out, 1, 0, st);
    case HQ_TYPE_Q6_K: return launch_sb<HQ_TYPE_Q6_K, true>(W, H, ids, pairs, k, out, 1, 0, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t hq_launch_gemm_kq(int type, const GemmArgs &g, int mb, hipStream_t st) {
    switch (type) {
    case HQ_TYPE_Q2_K: return gemm_t<HQ_TYPE_Q2_K>(g, mb, st);
    case HQ_TYPE_Q3_K: return gemm_t<HQ_TYPE_Q3_K>(g, mb, st);
    case HQ_TYPE_Q5_K: return gemm_t<HQ_TYPE_Q5_K>(g, mb, st);
    default: return hipErrorInvalidValue;
    }
}
