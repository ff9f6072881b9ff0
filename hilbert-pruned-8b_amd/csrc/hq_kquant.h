// hq_kquant.h - device layout and exact fp32 decode of the GGUF k-quants Q2_K, Q3_K and Q5_K, shared
// by their kernels (hq_kquant.hip) and the backend's single-token kernels (hq_backend.hip).
//
// Reference arithmetic (cleanroom-transformer/src/ggml_quant.h): 256-value super-blocks.
//   Q2_K (:100-111)  {u8 scales[16], u8 qs[64], fp16 d, fp16 dmin}        84 B
//                    value 128h + 32j + l: q = bits 2j, 2j+1 of qs[32h + l]; byte sm = scales[8h + 2j + l/16];
//                    y = (d * (sm & 15)) * q - dmin * (sm >> 4)
//   Q3_K (:112-134)  {u8 hmask[32], u8 qs[64], u8 scales[12], fp16 d}    110 B
//                    q = bits 2j, 2j+1 of qs[32h + l], minus 4 unless bit 4h + j of hmask[l] is set;
//                    y = (d * (sc - 32)) * q with sc the 6-bit scale 8h + 2j + l/16
//   Q5_K (:135-150)  {fp16 d, fp16 dmin, u8 scales[12], u8 qh[32], u8 qs[128]}  176 B
//                    sub-block j (32 values): q = nibble (j odd: high) of qs[32(j/2) + l] + 16 * bit j
//                    of qh[l]; y = (d * s) * q - dmin * m with (s, m) the 6-bit codes of scale_min_k4
// Every product above is exact in fp32 (at most 22 significant bits), so the one rounding is the
// final subtraction (Q2_K, Q5_K) or none (Q3_K), with or without a fused multiply-add: the decoders
// below are bit-identical to the reference's.
//
// Device layout (hq_mat_upload): Q5_K keeps the GGUF bytes (176 = 11 x 16, so every field sits at a
// 16-byte boundary); Q2_K and Q3_K super-blocks are stored in 96- and 112-byte slots (the GGUF
// bytes, then zeros), so that every 16-byte load of a row is aligned. Fields keep their GGUF offsets.
// (Q6_K, whose kernels live in hq_q6k.hip, uses 224-byte slots the same way; kq_slot covers it for
// the GEMV of hq_kquant.hip.)
#ifndef HQ_KQUANT_H
#define HQ_KQUANT_H

#include "hq_device.h"
#include "hq_kernels.h"

constexpr int kq_slot(int type) {
    return type == HQ_TYPE_Q2_K ? 96 : type == HQ_TYPE_Q3_K ? 112 : type == HQ_TYPE_Q6_K ? 224 : 176;
}

// 6-bit Q3_K scale e (0..15) from the 12 packed bytes: low nibble from byte 4 (g % 2) + i (high
// nibble when g >= 2), top two bits from bits 2g, 2g + 1 of byte 8 + i, for e = 4g + i.
DEV int q3k_code(const uint8_t *sc, int e) {
    const int g = e >> 2, i = e & 3;
    return (int)(((sc[4 * (g & 1) + i] >> (4 * (g >> 1))) & 15u) | (((sc[8 + i] >> (2 * g)) & 3u) << 4));
}

// Values v .. v + 7 (v a multiple of 8) of the super-block at blk (device slot) as fp32, bit-identical
// to the reference decoder.
template <int T>
DEV void kq_deq8(const uint8_t *blk, int v, float (&w)[8]) {
    const int l = v & 31;
    if constexpr (T == HQ_TYPE_Q5_K) {
        const int sub = v >> 5;
        const u4v hdr = *(const u4v *)blk;
        uint32_t sw0, sw1, mw0, mw1;
        q4k_scale_words(hdr.y, hdr.z, hdr.w, sw0, sw1, mw0, mw1);
        const float ds = h2f((uint16_t)hdr.x) * (float)byte_of(sub < 4 ? sw0 : sw1, sub & 3);
        const float dm = h2f((uint16_t)(hdr.x >> 16)) * (float)byte_of(sub < 4 ? mw0 : mw1, sub & 3);
        const u2v ql = *(const u2v *)(blk + 48 + 32 * (sub >> 1) + l), qh = *(const u2v *)(blk + 16 + l);
        const int shift = (sub & 1) ? 4 : 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t lw = e < 4 ? ql.x : ql.y, hw = e < 4 ? qh.x : qh.y;
            const int q = (int)((lw >> (8 * (e & 3) + shift)) & 15u) + 16 * (int)((hw >> (8 * (e & 3) + sub)) & 1u);
            w[e] = ds * (float)q - dm;
        }
    } else {
        const int h = v >> 7, j = (v >> 5) & 3;
        if constexpr (T == HQ_TYPE_Q2_K) {
            const uint32_t sm = blk[8 * h + 2 * j + (l >> 4)];
            const float ds = h2f(*(const uint16_t *)(blk + 80)) * (float)(sm & 15u);
            const float dm = h2f(*(const uint16_t *)(blk + 82)) * (float)(sm >> 4);
            const u2v qs = *(const u2v *)(blk + 16 + 32 * h + l);
#pragma unroll
            for (int e = 0; e < 8; e++) w[e] = ds * (float)(((e < 4 ? qs.x : qs.y) >> (8 * (e & 3) + 2 * j)) & 3u) - dm;
        } else {
            const float dl = h2f(*(const uint16_t *)(blk + 108)) * (float)(q3k_code(blk + 96, 8 * h + 2 * j + (l >> 4)) - 32);
            const u2v qs = *(const u2v *)(blk + 32 + 32 * h + l), hm = *(const u2v *)(blk + l);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int q2 = (int)(((e < 4 ? qs.x : qs.y) >> (8 * (e & 3) + 2 * j)) & 3u);
                const int hb = (int)(((e < 4 ? hm.x : hm.y) >> (8 * (e & 3) + 4 * h + j)) & 1u);
                w[e] = dl * (float)(q2 - (hb ? 0 : 4));
            }
        }
    }
}

// Runtime-type form for kernels that take any of the three.
DEV void kq_deq8_any(int type, const uint8_t *blk, int v, float (&w)[8]) {
    if (type == HQ_TYPE_Q2_K) kq_deq8<HQ_TYPE_Q2_K>(blk, v, w);
    else if (type == HQ_TYPE_Q3_K) kq_deq8<HQ_TYPE_Q3_K>(blk, v, w);
    else kq_deq8<HQ_TYPE_Q5_K>(blk, v, w);
}

#endif
