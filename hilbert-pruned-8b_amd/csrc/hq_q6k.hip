// hq_q6k.hip - GGUF Q6_K matrices on gfx950: decode and the MFMA GEMM.
//
// Reference arithmetic (cleanroom-transformer/src/ggml_quant.h:151-169): a super-block of 256 values
// {u8 ql[128], u8 qh[64], int8 scales[16], fp16 d}; value 128h + 32r + l (half h, lane r = 0..3,
// l = 0..31) has q = (ql[64h + 32(r % 2) + l] low nibble for r < 2, high for r >= 2)
// | (bits 2r, 2r + 1 of qh[32h + l]) << 4, minus 32, and y = (d * sc) * q with sc = scales[8h + 2r + l/16]
// (d * sc is exact in fp32; the second product can round).
//
// Device layout (written by hq_mat_upload): each 210-byte super-block is stored in a 224-byte slot
// {ql[128], qh[64], scales[16], d, 14 zero bytes}, so every 16-byte load is aligned; hq_mat_download
// restores the GGUF bytes.
//
// Kernels
//   k_dequant_q6_k  rows -> fp32, bit-identical to the reference decoder ((d * sc) * q in fp32).
//   (M = 1 and the option-row gather: k_gemv_sb in hq_kquant.hip)
//   k_gemm_q6_k     M >= 2: the Stream-K MFMA kernel of hq_sk.h (tile 16 MB x 128, K-units of one
//                   super-block). No weight is rounded to 16 bits: with q = lo + 16 hb - 32 (lo the
//                   4-bit part, hb the 2-bit part), W / d = sc * lo + 16 sc * (hb - 2), and both terms
//                   are exact fp16 integers (|sc * lo| <= 1920, 16 sc (hb - 2) a multiple of 16 up to
//                   4096); each k-step issues one MFMA per term, the unit's fp32 accumulator is
//                   multiplied by the column's d once.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hq_device.h"
#include "hq_kernels.h"
#include "hq_sk.h"

namespace {
constexpr int Q6_SLOT = 224;  // device bytes per super-block

// Values v .. v + 15 (v a multiple of 16) of the super-block at blk as fp32, bit-identical to the
// reference decoder.
DEV void q6k_deq16(const uint8_t *blk, int v, float (&w)[16]) {
    const int h = v >> 7, r = (v >> 5) & 3, l0 = v & 16;
    const u4v ql = *(const u4v *)(blk + 64 * h + 32 * (r & 1) + l0);
    const u4v qh = *(const u4v *)(blk + 128 + 32 * h + l0);
    const float ds = h2f(*(const uint16_t *)(blk + 208)) * (float)(int8_t)blk[192 + 8 * h + 2 * r + (l0 >> 4)];
    const int shl = r >= 2 ? 4 : 0, shh = 2 * r;
    const uint32_t lw[4] = {ql.x, ql.y, ql.z, ql.w}, hw[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const int lo = (int)((lw[e >> 2] >> (8 * (e & 3) + shl)) & 0xfu);
        const int hb = (int)((hw[e >> 2] >> (8 * (e & 3) + shh)) & 3u);
        w[e] = ds * (float)((lo | (hb << 4)) - 32);
    }
}

// one thread per (row, 16-value chunk); output row r is matrix row ids[r] when ids is given
__global__ void __launch_bounds__(256) k_dequant_q6_k(const uint8_t *__restrict__ W, size_t row_bytes, int K,
                                                      uint32_t row0, const uint32_t *__restrict__ ids, uint32_t nrows,
                                                      float *__restrict__ out) {
    const size_t per_row = (size_t)K / 16, total = (size_t)nrows * per_row;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / per_row, v0 = (i % per_row) * 16, row = ids ? (size_t)ids[r] : row0 + r;
        float w[16];
        q6k_deq16(W + row * row_bytes + (v0 / 256) * Q6_SLOT, (int)(v0 % 256), w);
        float4 *o = (float4 *)(out + r * (size_t)K + v0);
#pragma unroll
        for (int q = 0; q < 4; q++) o[q] = float4{w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]};
    }
}

// The two exact fp16 B terms of 8 weights: bytes 8e .. 8e + 7 of the lane's ql / qh vectors, nibble
// `hi_nib`, 2-bit field at `shh`; sc = the group scale, s16 = 16 * sc.
DEV void q6k_frags(uint32_t l0, uint32_t l1, uint32_t h0, uint32_t h1, bool hi_nib, int shh, h2 sc, h2 s16, h8 &b1,
                   h8 &b2) {
    const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f}, k1026 = {(_Float16)1026.0f, (_Float16)1026.0f};
    const uint32_t n[2] = {(hi_nib ? l0 >> 4 : l0) & 0x0f0f0f0fu, (hi_nib ? l1 >> 4 : l1) & 0x0f0f0f0fu};
    const uint32_t q[2] = {(h0 >> shh) & 0x03030303u, (h1 >> shh) & 0x03030303u};
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const h2 a = (as_h2(perm_lo(n[i])) - k1024) * sc, b = (as_h2(perm_hi(n[i])) - k1024) * sc;
        const h2 c = (as_h2(perm_lo(q[i])) - k1026) * s16, d = (as_h2(perm_hi(q[i])) - k1026) * s16;
        b1[4 * i] = a.x, b1[4 * i + 1] = a.y, b1[4 * i + 2] = b.x, b1[4 * i + 3] = b.y;
        b2[4 * i] = c.x, b2[4 * i + 1] = c.y, b2[4 * i + 2] = d.x, b2[4 * i + 3] = d.y;
    }
}

// Stream-K Q6_K GEMM (structure of k_gemm_q8_0 in hq_kernels.hip): tile 16 MB rows x 64 NB columns per
// wave-set of 4 waves, K-units of one super-block. Lane (ln, lg) of column block j holds the
// unit's values 64 s + 16 lg .. + 16 for s = 0..3: ql bytes 64 h + 16 lg (h = s / 2, both s of a
// half share them), qh bytes 128 + 32 h + 16 (lg % 2), scale bytes 192 .. 207 and d.
template <int MB, int NB>
__global__ void __launch_bounds__(256) k_gemm_q6_k(GemmArgs g) {
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
    struct Wq {
        u4v ql[2], qh[2], sc;
        uint32_t d;
    };
    auto load_w = [&](int unit, Wq (&x)[NB]) {
        const uint32_t base = (uint32_t)unit * Q6_SLOT;
#pragma unroll
        for (int j = 0; j < NB; j++) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                x[j].ql[h] = buf_load16(rw, vrow[j], base + 64u * h + 16u * lg);
                x[j].qh[h] = buf_load16(rw, vrow[j], base + 128u + 32u * h + 16u * (lg & 1));
            }
            x[j].sc = buf_load16(rw, vrow[j], base + 192u);
            x[j].d = __builtin_amdgcn_raw_buffer_load_b32(rw, vrow[j], base + 208u, 0);
        }
    };
    f4 acc[MB][NB];
    Wq wc[NB];
    int cur_tile = u0 / p.upt;
    tile_setup(cur_tile);
    dma_a<MB>(sa[0], ra, adma, K, (u0 % p.upt) * KC);
    load_w(u0 % p.upt, wc);
    for (int u = u0; u < u1; u++) {
        const int cb = (u - u0) & 1, tile = u / p.upt, ku = u % p.upt;
        const int m0 = (tile % p.tm) * 16 * MB, nw = (tile / p.tm) * 64 * NB + wave * 16 * NB;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        Wq wn[NB];
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
        f4 au[MB][NB];
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) au[i][j] = f4{0.f, 0.f, 0.f, 0.f};
        const _Float16 *buf = sa[cb];
#pragma unroll
        for (int f = 0; f < 8; f++) {
            const int s = f >> 1, e = f & 1, h = s >> 1, t = s & 1;
            const int shh = 4 * t + 2 * (lg >> 1), sci = 8 * h + 4 * t + lg;
            h8 b1[NB], b2[NB];
#pragma unroll
            for (int j = 0; j < NB; j++) {
                const uint32_t scw[4] = {wc[j].sc.x, wc[j].sc.y, wc[j].sc.z, wc[j].sc.w};
                const int scv = (int)(int8_t)(scw[sci >> 2] >> (8 * (sci & 3)));
                const _Float16 sch = (_Float16)(float)scv, s16h = (_Float16)(float)(16 * scv);
                const uint32_t qlw[4] = {wc[j].ql[h].x, wc[j].ql[h].y, wc[j].ql[h].z, wc[j].ql[h].w};
                const uint32_t qhw[4] = {wc[j].qh[h].x, wc[j].qh[h].y, wc[j].qh[h].z, wc[j].qh[h].w};
                q6k_frags(qlw[2 * e], qlw[2 * e + 1], qhw[2 * e], qhw[2 * e + 1], t != 0, shh, h2{sch, sch},
                          h2{s16h, s16h}, b1[j], b2[j]);
            }
#pragma unroll
            for (int i = 0; i < MB; i++) {
                const h8 af = a_frag(buf, 16 * i + ln, 8 * s + 2 * lg + e);
#pragma unroll
                for (int j = 0; j < NB; j++) {
                    au[i][j] = mfma(af, b1[j], au[i][j]);
                    au[i][j] = mfma(af, b2[j], au[i][j]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const float d = h2f((uint16_t)wc[j].d);
#pragma unroll
            for (int i = 0; i < MB; i++) acc[i][j] += au[i][j] * d;
        }
        if (ku == p.upt - 1 || u == u1 - 1)
            finish_tile<MB, NB, 256>(acc, p, w, u0, u1, tile, &s_flag, rpart, g.counters, g.C, M, N, m0, nw, ln, lg,
                                     g.c_f32, g.accumulate);
        if (u + 1 < u1) {
#pragma unroll
            for (int j = 0; j < NB; j++) wc[j] = wn[j];
        }
    }
}

unsigned grid_cap(size_t n, unsigned per, unsigned cap) {
    const size_t g = (n + per - 1) / per;
    return (unsigned)(g < cap ? (g ? g : 1) : cap);
}
}  // namespace

hipError_t hq_launch_dequant_q6k(const hq_dev_mat *W, uint32_t row0, const uint32_t *ids, uint32_t nrows, float *out,
                                 hipStream_t st) {
    const size_t n = (size_t)nrows * (W->cols / 16);
    k_dequant_q6_k<<<grid_cap(n, 256, 65536), 256, 0, st>>>(W->qs, W->row_bytes, (int)W->cols, row0, ids, nrows, out);
    return hipGetLastError();
}

hipError_t hq_launch_gemm_q6k(const GemmArgs &g, int mb, hipStream_t st) {
    switch (mb) {
    case 1: k_gemm_q6_k<1, 2><<<g.plan.G, 256, 0, st>>>(g); break;
    case 2: k_gemm_q6_k<2, 2><<<g.plan.G, 256, 0, st>>>(g); break;
    case 4: k_gemm_q6_k<4, 2><<<g.plan.G, 256, 0, st>>>(g); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
