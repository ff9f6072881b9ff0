// hq_sk.h - shared pieces of the Stream-K MFMA GEMM kernels (hq_kernels.hip, hq_q6k.hip): the
// activation tile DMA and fragment layout, B-fragment decoders, the Stream-K work split and the
// partial-tile protocol, and the kernel argument block.
#ifndef HQ_SK_H
#define HQ_SK_H

#include "hq_device.h"
#include "hq_kernels.h"

// ============================================================================ MFMA GEMM
// Work decomposition (Stream-K): the output is cut into tiles of BM = 16*MB rows (M) by
// BN = 64*NB columns (N, weight rows), and each tile into K-units of KC = 256 activations (one
// Q4_K super-block, eight Q8_0 blocks). The tile-major list of (tile, unit) pairs is split into G
// equal contiguous ranges, one per persistent workgroup (G = number of CUs), so every CU gets the
// same MFMA work whatever the shape (no wave quantization). A tile cut between workgroups is
// combined through a workspace: each contributor stores its fp32 partial tile, then increments the
// tile's counter; the contributor that brings the counter to its final value adds the others'
// partials and writes C, then resets the counter. No workgroup ever waits on another.
//
// Inside a workgroup: 4 waves, wave w owns columns [16*NB*w, 16*NB*(w+1)) of the tile and all BM
// rows. Pipeline per unit: the next unit's activation tile is streamed global -> LDS by
// global_load_lds_dwordx4 (no registers) into the other half of a double buffer, and each wave
// prefetches the next unit's weight bytes into registers, while the current unit is decoded and
// multiplied. One barrier per unit.
//
// LDS tile layout: row r holds 32 slots of 16 bytes; slot p holds activation chunk p ^ (r & 15)
// (XOR swizzle), so the 16 lanes of an MFMA operand read (16 rows, same chunk) hit 16 distinct
// 4-bank groups and the DMA writes stay contiguous (two rows per 64-lane instruction).
//
// v_mfma_f32_16x16x32_f16 operands (per lane l: ln = l % 16, lg = l / 16): A holds row ln,
// 8 k-slots of group lg; B holds column ln, the same 8 k-slots; D holds column ln, rows 4*lg..4*lg+3.
// The k-slot -> k mapping inside one MFMA is free as long as A and B agree; it is chosen so each
// lane's 8 weights come from one 16-byte load and each lane's 8 activations are one 16-byte slot.
//
// Q4_K: the B operand is the exact integer s*q; the per-unit fp32 accumulator is folded with d.
// The min term dmin * sum_sub m_sub * S_sub (S = fp32 sum of the sub-block's 32 activations, from
// v_dot2_f32_f16 over the LDS tile, split hi + lo fp16) is one MFMA per unit with the integer m as
// B operand, folded with dmin. S of unit u is complete only after the next barrier, so the min
// term of unit u is applied in unit u + 1 (or right before a tile is finished).
namespace {
constexpr int KC = 256;


// Activation tile DMA: instruction qq of wave w moves rows r = 8qq + 2w + (lane >> 5) (two 256-half
// rows per 64-lane instruction) into LDS slots (r, lane & 31). The per-lane byte offset is
// a_base[qq & 1] (row and swizzled chunk) plus qq * 16 * K + 2 * k0, all of it in the VGPR offset:
// a buffer load range-checks only that offset (not soffset), so rows at or past M, and the tail of
// the last row past K, read zeros instead of memory beyond A.
struct ADma {
    uint32_t base[2];
};

template <int MB>
DEV ADma adma_setup(int K, int m0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, p = lane & 31;
    const int r0 = 2 * wave + (lane >> 5);
    ADma d;
#pragma unroll
    for (int x = 0; x < 2; x++) {
        const int c = p ^ ((8 * x + r0) & 15);
        d.base[x] = (uint32_t)((m0 + r0) * K + 8 * c) * 2u;
    }
    return d;
}

template <int MB>
DEV void dma_a(_Float16 *buf, rsrc_t ra, const ADma &d, int K, int k0) {
    constexpr int INSTR = 16 * MB / 2;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int qq = 0; qq < (INSTR + 3) / 4; qq++) {
        const int q = 4 * qq + wave;
        if (INSTR % 4 == 0 || q < INSTR)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, lds_ptr(buf + q * 512), 16,
                                                     d.base[qq & 1] + (uint32_t)(qq * 16 * K + 2 * k0), 0, 0, 0);
    }
}

// A fragment: row r (= 16*i + ln), activation chunk c (8 halves).
DEV h8 a_frag(const _Float16 *buf, int r, int c) { return *(const h8 *)(buf + r * KC + 8 * (c ^ (r & 15))); }


// B fragment from 8 bytes u = q + 128 (two words) -> fp16(q * d): one rounding of the exact product.
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

// B fragment of exact integers s*q from the low (HI_NIB = false) or high nibbles of 8 bytes:
// fp16(1024 + q) * s - 1024*s, or fp16(1024 + 16q) * (s/16) - 64*s, one fused rounding of an
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


struct SkPlan {
    int tm, tiles, upt;  // M-tiles, tiles, K-units per tile
    int base, extra;     // workgroup w owns units [w*base + min(w, extra), (w+1)*base + min(w+1, extra))
    int G;               // workgroups
};

DEV int sk_start(const SkPlan &p, int w) { return w * p.base + (w < p.extra ? w : p.extra); }
DEV int sk_owner(const SkPlan &p, int u) {
    const int big = p.extra * (p.base + 1);
    return u < big ? u / (p.base + 1) : p.extra + (u - big) / p.base;
}

// Partial tiles travel through device-scope (sc1) 16-byte accesses (buf_store16 / buf_load16_sc1).
// Tile finished by this workgroup (NT threads): store it, or run the partial-tile protocol. Partial
// slot layout: (row block i, column block j) of thread tid at 16 * ((i * NB + j) * NT + tid).
template <int MB, int NB, int NT>
DEV void finish_tile(f4 (&acc)[MB][NB], const SkPlan &p, int w, int u0, int u1, int tile, int *s_flag,
                     rsrc_t rpart, int *__restrict__ counters, void *C, int M, int N, int m0, int nw, int ln, int lg,
                     int c_f32, int accumulate) {
    const int t0 = tile * p.upt, t1 = t0 + p.upt;
    if (t0 >= u0 && t1 <= u1) {
        store_tile<MB, NB>(C, acc, M, N, m0, nw, ln, lg, c_f32, accumulate);
        return;
    }
    constexpr uint32_t PER = NT * MB * NB * 16;  // bytes per partial tile
    const int tid = threadIdx.x;
    // slot 2w: the tile this workgroup starts in; 2w + 1: the tile it ends in. The counter update
    // is ordered after the stores by waiting for them (stores count in vmcnt) before the barrier.
    const int slot = tile == u0 / p.upt ? 2 * w : 2 * w + 1;
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) buf_store16(rpart, acc[i][j], (uint32_t)tid * 16u + slot * PER + (i * NB + j) * NT * 16);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const int wf = sk_owner(p, t0), wl = sk_owner(p, t1 - 1);
    if (tid == 0) {
        const int prev = atomicAdd(&counters[tile], 1);
        const int last = prev == wl - wf;
        if (last) atomicExch(&counters[tile], 0);
        *s_flag = last;
    }
    __syncthreads();
    if (!*s_flag) return;
    // The partials are summed in owner order wf .. wl (this workgroup's own in its place), so the
    // result is the same whichever contributor arrives last.
    constexpr int IG = MB < 4 ? MB : 4;  // row blocks per batch of loads (bounds the registers)
#pragma unroll
    for (int i0 = 0; i0 < MB; i0 += IG) {
        f4 s[IG][NB];
#pragma unroll
        for (int i = 0; i < IG; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) s[i][j] = f4{0.f, 0.f, 0.f, 0.f};
        for (int o = wf; o <= wl; o++) {
            if (o == w) {
#pragma unroll
                for (int i = 0; i < IG; i++)
#pragma unroll
                    for (int j = 0; j < NB; j++) s[i][j] += acc[i0 + i][j];
                continue;
            }
            const uint32_t os = (uint32_t)(tile == sk_start(p, o) / p.upt ? 2 * o : 2 * o + 1) * PER;
            f4 v[IG][NB];
#pragma unroll
            for (int i = 0; i < IG; i++)
#pragma unroll
                for (int j = 0; j < NB; j++)
                    v[i][j] = buf_load16_sc1(rpart, (uint32_t)tid * 16u, os + ((i0 + i) * NB + j) * NT * 16);
#pragma unroll
            for (int i = 0; i < IG; i++)
#pragma unroll
                for (int j = 0; j < NB; j++) s[i][j] += v[i][j];
        }
#pragma unroll
        for (int i = 0; i < IG; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) acc[i0 + i][j] = s[i][j];
    }
    store_tile<MB, NB>(C, acc, M, N, m0, nw, ln, lg, c_f32, accumulate);
}
}  // namespace

struct GemmArgs {
    const uint8_t *qs;    // Q8_0 quant plane / Q4_K blocks
    const uint16_t *d;    // Q8_0 scale plane
    int ldd;
    size_t row_bytes;
    const uint16_t *A;
    int M, N, K;
    void *C;
    int c_f32, accumulate;
    SkPlan plan;
    float *partials;
    uint32_t partial_bytes;
    int *counters;
    const uint16_t *sums;  // wide Q4_K kernel: activation sub-block sums (k_asums)
};

DEV int sk_worker(int G) {
    // consecutive ranges (which share tiles and weight slabs) on the same XCD: workgroups are dealt
    // round-robin to the 8 XCDs
    const int bid = blockIdx.x;
    return G % 8 == 0 ? (bid % 8) * (G / 8) + bid / 8 : bid;
}

#endif
