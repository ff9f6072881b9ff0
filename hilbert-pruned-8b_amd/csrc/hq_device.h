// hq_device.h - device helpers shared by the gfx950 kernel sources (hq_kernels.hip, hq_gemm_ws.hip).
#ifndef HQ_DEVICE_H
#define HQ_DEVICE_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
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

DEV void store_out(void *C, size_t idx, float v, int c_f32, int accumulate) {
    if (c_f32) {
        float *c = (float *)C + idx;
        *c = accumulate ? *c + v : v;
    } else {
        _Float16 *c = (_Float16 *)C + idx;
        *c = (_Float16)(accumulate ? (float)*c + v : v);
    }
}

typedef __attribute__((address_space(3))) void lds_void;

DEV lds_void *lds_ptr(const void *p) { return (lds_void *)(uintptr_t)p; }

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer over `bytes` bytes: loads at offsets >= bytes return zero.
DEV rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}

// LDS DMA: lane i's 16 bytes at voff + soff land at lds + 16 i (lds is wave-uniform).
DEV void dma16(rsrc_t r, void *lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_ptr(lds), 16, voff, soff, 0, 0);
}

// The same 16-byte LDS DMA written as assembly, so the compiler does not track it: it would
// otherwise wait for every earlier LDS DMA before each later LDS read. The caller waits for it
// with an explicit s_waitcnt vmcnt. lds_addr is the wave-uniform LDS byte address; M0 is restored.
DEV void dma16_untracked(rsrc_t r, uint32_t lds_addr, uint32_t voff) {
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 1\n\tbuffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(save)
                 : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(r)
                 : "memory");
}

// 16-byte LDS DMA with an SGPR offset, untracked by the compiler (explicit s_waitcnt vmcnt).
DEV void dma16_so(rsrc_t r, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 1\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(save)
                 : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(r),
                   "s"(__builtin_amdgcn_readfirstlane(soff))
                 : "memory");
}

// s_waitcnt vmcnt(n) for a wave-uniform n in 0 .. 31 (the count is an immediate of the instruction).
DEV void wait_vmcnt(int n) {
    switch (n) {
#define HQ_VMW(i) case i: asm volatile("s_waitcnt vmcnt(" #i ")" ::: "memory"); break;
        HQ_VMW(0) HQ_VMW(1) HQ_VMW(2) HQ_VMW(3) HQ_VMW(4) HQ_VMW(5) HQ_VMW(6) HQ_VMW(7)
        HQ_VMW(8) HQ_VMW(9) HQ_VMW(10) HQ_VMW(11) HQ_VMW(12) HQ_VMW(13) HQ_VMW(14) HQ_VMW(15)
        HQ_VMW(16) HQ_VMW(17) HQ_VMW(18) HQ_VMW(19) HQ_VMW(20) HQ_VMW(21) HQ_VMW(22) HQ_VMW(23)
        HQ_VMW(24) HQ_VMW(25) HQ_VMW(26) HQ_VMW(27) HQ_VMW(28) HQ_VMW(29) HQ_VMW(30) HQ_VMW(31)
#undef HQ_VMW
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
}

// Partial tiles are written and read with device-scope (sc1) buffer accesses: they go to the
// cross-XCD coherent level, so no L2 write-back or invalidation is needed, and unlike atomics they
// are not serialized, so a 16-byte access per (row block, column block) is in flight at once.
constexpr int CPOL_SC1 = 16;

// The whole offset is in the VGPR operand (range-checked) and the scalar offset is the constant 0:
// with a scalar-register offset the compiler inserts no wait states between a 16-byte buffer store
// and a VALU write of its data registers, and on gfx950 such a write right behind the store was
// seen to reach memory in place of the store's first data word.
DEV void buf_store16(rsrc_t r, f4 v, uint32_t voff) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, v), r, voff, 0u, CPOL_SC1);
}

// 16 bytes of an fp16 activation vector, from global memory or from a workgroup's LDS copy
typedef const __attribute__((address_space(3))) uint16_t lds_u16c;
DEV u4v ld_a16(const uint16_t *p) { return *(const u4v *)p; }
DEV u4v ld_a16(lds_u16c *p) { return *(const __attribute__((address_space(3))) u4v *)p; }
// Copy of the K fp16 values at a into LDS at lds (K % 8 == 0) by the workgroup's NT threads; the caller
// waits at a barrier before reading it. Returns the copy's LDS pointer.
template <int NT>
DEV lds_u16c *stage_act(const uint16_t *__restrict__ a, int K, uint16_t *lds) {
    using lds_u4 = __attribute__((address_space(3))) u4v;
    const uint32_t base = (uint32_t)(uintptr_t)lds;
    for (int i = threadIdx.x; i < K / 8; i += NT) *(lds_u4 *)(uintptr_t)(base + 16u * (uint32_t)i) = *(const u4v *)(a + 8 * i);
    return (lds_u16c *)(uintptr_t)base;
}

DEV f4 buf_load16_sc1(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, CPOL_SC1));
}

// sum of 8 products q*a: q four exact fp16 pairs, a four words of fp16 pairs (v_dot2_f32_f16: exact
// products, fp32 sums)
DEV float dot8(const h2 (&q)[4], const u4v a, float s) {
    s = __builtin_amdgcn_fdot2(q[0], as_h2(a.x), s, false);
    s = __builtin_amdgcn_fdot2(q[1], as_h2(a.y), s, false);
    s = __builtin_amdgcn_fdot2(q[2], as_h2(a.z), s, false);
    s = __builtin_amdgcn_fdot2(q[3], as_h2(a.w), s, false);
    return s;
}

// sum of the 8 fp16 values of a (fp32)
DEV float sum8(const u4v a, float s) {
    const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
    s = __builtin_amdgcn_fdot2(as_h2(a.x), one, s, false);
    s = __builtin_amdgcn_fdot2(as_h2(a.y), one, s, false);
    s = __builtin_amdgcn_fdot2(as_h2(a.z), one, s, false);
    s = __builtin_amdgcn_fdot2(as_h2(a.w), one, s, false);
    return s;
}

// One GEMV unit from LDS: 64 values of a weight row (32-byte quant group p of the super-block at
// blk: low nibbles = sub-block 2p, high nibbles = sub-block 2p + 1) dotted with activations
// [64 ku, 64 ku + 64) of sa, using the 32-value sums ss[2 ku], ss[2 ku + 1]. The quants become the
// fp16 values 1024 + q (low) and 1024 + 16 q (high) under v_perm_b32, meet the activations in
// v_dot2_f32_f16 (exact products, fp32 sums), and the 1024 bias comes off in fp32 through the sums:
// d sc dot(q, a) - dmin m sum(a) per sub-block (ggml_quant.h:51-59 scale and min codes).
DEV float gemv_unit_q4_k(const char *blk, int p, const char *sa, const float *ss, int ku) {
    const u4v hd = *(const u4v *)blk;
    const u4v q0 = *(const u4v *)(blk + 16 + 32 * p), q1 = *(const u4v *)(blk + 32 + 32 * p);
    const u4v *const av = (const u4v *)(sa + 128 * ku);
    const float s0 = ss[2 * ku], s1 = ss[2 * ku + 1];
    uint32_t sw0, sw1, mw0, mw1;
    q4k_scale_words(hd.y, hd.z, hd.w, sw0, sw1, mw0, mw1);
    const uint32_t sh = 16u * (uint32_t)(p & 1);
    const uint32_t sw = (p < 2 ? sw0 : sw1) >> sh, mw = (p < 2 ? mw0 : mw1) >> sh;
    const float d = h2f((uint16_t)hd.x), dmin = h2f((uint16_t)(hd.x >> 16));
    const float ds0 = d * (float)(sw & 0xffu), ds1 = d * (float)((sw >> 8) & 0xffu);
    const float dm0 = dmin * (float)(mw & 0xffu), dm1 = dmin * (float)((mw >> 8) & 0xffu);
    float part[4];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const u4v q = c ? q1 : q0;
        const uint32_t wl[4] = {q.x & 0x0f0f0f0fu, q.y & 0x0f0f0f0fu, q.z & 0x0f0f0f0fu, q.w & 0x0f0f0f0fu};
        const uint32_t wh[4] = {q.x & 0xf0f0f0f0u, q.y & 0xf0f0f0f0u, q.z & 0xf0f0f0f0u, q.w & 0xf0f0f0f0u};
        const h2 l0[4] = {as_h2(perm_lo(wl[0])), as_h2(perm_hi(wl[0])), as_h2(perm_lo(wl[1])), as_h2(perm_hi(wl[1]))};
        const h2 l1[4] = {as_h2(perm_lo(wl[2])), as_h2(perm_hi(wl[2])), as_h2(perm_lo(wl[3])), as_h2(perm_hi(wl[3]))};
        const h2 g0[4] = {as_h2(perm_lo(wh[0])), as_h2(perm_hi(wh[0])), as_h2(perm_lo(wh[1])), as_h2(perm_hi(wh[1]))};
        const h2 g1[4] = {as_h2(perm_lo(wh[2])), as_h2(perm_hi(wh[2])), as_h2(perm_lo(wh[3])), as_h2(perm_hi(wh[3]))};
        part[c] = dot8(l1, av[2 * c + 1], dot8(l0, av[2 * c], 0.f));
        part[2 + c] = dot8(g1, av[4 + 2 * c + 1], dot8(g0, av[4 + 2 * c], 0.f));
    }
    const float ql = (part[0] + part[1]) - 1024.0f * s0;  // dot(q, a), sub-block 2p
    const float qh = (part[2] + part[3]) - 1024.0f * s1;  // 16 dot(q, a), sub-block 2p + 1
    return (ds0 * ql - dm0 * s0) + (0.0625f * ds1 * qh - dm1 * s1);
}

DEV u4v buf_load16(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Eight fp16 B values s*q for 8 consecutive k from the low (mask 0x0f0f0f0f) or high (0xf0f0f0f0)
// nibbles of 8 bytes: masked bytes under 0x64 are fp16 1024 + q (or 1024 + 16q); one fma with
// (s, -1024 s) (or (s/16, -64 s)) gives the exact integer. The mask may differ per lane.
DEV h8 decode8m(u2v q, uint32_t mask, h2 mul, h2 add) {
    const uint32_t w0 = q.x & mask, w1 = q.y & mask;
    const h2 v0 = __builtin_elementwise_fma(as_h2(perm_lo(w0)), mul, add);
    const h2 v1 = __builtin_elementwise_fma(as_h2(perm_hi(w0)), mul, add);
    const h2 v2 = __builtin_elementwise_fma(as_h2(perm_lo(w1)), mul, add);
    const h2 v3 = __builtin_elementwise_fma(as_h2(perm_hi(w1)), mul, add);
    return h8{v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
}

template <bool HI>
DEV h8 decode8(u2v q, h2 mul, h2 add) {
    return decode8m(q, HI ? 0xf0f0f0f0u : 0x0f0f0f0fu, mul, add);
}

DEV f4 mfma(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
// bf16 MFMA on operands held as 16-bit patterns (loaded through the same h8 path as fp16 ones)
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
DEV f4 mfma_bf16(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c, 0, 0, 0);
}

// fp16 pair (1024 + b0, 1024 + b1) minus 1024: the bytes as exact fp16 integers.
DEV h2 bytes_f16(uint32_t w, bool hi_pair) {
    const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    return as_h2(hi_pair ? perm_hi(w) : perm_lo(w)) - k1024;
}

// Output mode of the tile kernels besides fp32 (1) and fp16 (0) C: silu(gate) * up of a gate/up
// pair matrix, fp16 (see tile_finish).
constexpr int HQ_OUT_SWIGLU = 2;

// SwiGLU output from accumulators in the MFMA layout of the register-decode kernels (lane (ln, lg) of
// block (i, j): row 16i + ln, columns 16j + 4lg .. + 3 of the wave's columns). Each 16-column block of
// a gate/up pair matrix is 8 gate columns and the 8 matching up columns, so lanes 32 apart hold
// matching gate (lg = 0, 1) and up (lg = 2, 3) values of the same 4 pair columns 4 (lg & 1) .. + 3.
// The two lanes split them: each sends its partner the two values the partner lacks (all 64 lanes
// take part, so this comes before any per-lane bounds check) and returns silu(gate) * up of pair
// columns 4 (lg & 1) + 2 (lg >> 1) and + 1 of the block, as two fp16 in a word. silu(g) =
// g / (1 + e^-g) with the hardware exp2 and reciprocal (about 1 ulp of fp32 each, far below the
// fp16 rounding of the result; e^-g overflowing to inf gives -0 for very negative g).
DEV uint32_t swiglu_pair2(const f4 &v, int lg) {
    const bool gate = lg < 2;
    h2 y;
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const float own = gate ? v[k] : v[2 + k];
        const float got = __shfl_xor(gate ? v[2 + k] : v[k], 32, 64);
        const float gv = gate ? own : got, uv = gate ? got : own;
        const float silu = gv * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gv * -1.4426950408889634f));
        y[k] = (_Float16)(silu * uv);
    }
    return __builtin_bit_cast(uint32_t, y);
}

// fp16 output tiles through LDS. A tile kernel whose accumulators hold scattered 16 x 16 blocks puts
// its tile into LDS as fp16 (row r at r * tile_ldr<ROWB>() bytes, so that consecutive rows start 4
// banks apart), then all NT threads store whole 16-byte pieces, consecutive lanes on consecutive bytes
// of a row: a store instruction writes whole 128-byte lines, where an 8-byte store from the
// accumulators covers 16 rows x 32 bytes. (Measured on the register-decode kernels: faster for fp16 C
// and for the Q4_K kernel's SwiGLU output, slower for fp32 C, whose LDS pass costs more than the
// stores gain.)
// tile_store_ok: fp16 C without accumulate, rows of whole 16-byte pieces, C 16-byte aligned.
DEV bool tile_store_ok(int c_f32, int accumulate, int N, const void *C) {
    return c_f32 == 0 && !accumulate && N % 8 == 0 && ((uintptr_t)C & 15u) == 0;
}
template <int ROWB>
constexpr int tile_ldr() { return ROWB + 16; }
// the store: Ct the tile's first row in C, `rows` of them inside M, C's row pitch in bytes, the
// tile's first byte col0 in a row and its vb bytes inside the row (a multiple of 16). Write-through
// stores (SC1), measured faster than write-back where every tile stores at once.
template <int BM, int NT, int ROWB>
DEV void tile_store_rows(const char *lds, char *Ct, int rows, uint32_t pitch, uint32_t col0, uint32_t vb, int tid) {
    constexpr int CPR = ROWB / 16, TOT = BM * CPR;
    static_assert(ROWB % 16 == 0, "whole pieces");
    const rsrc_t rc = make_rsrc(Ct, (uint32_t)rows * pitch);
#pragma unroll
    for (int k = 0; k < (TOT + NT - 1) / NT; k++) {
        const int c = tid + k * NT;
        if (TOT % NT != 0 && c >= TOT) break;
        const int row = c / CPR, pc = c - row * CPR;
        if (row >= rows || (uint32_t)pc * 16u >= vb) continue;
        buf_store16(rc, *(const f4 *)(lds + row * tile_ldr<ROWB>() + pc * 16), (uint32_t)row * pitch + col0 + (uint32_t)pc * 16u);
    }
}

// Output values n .. n + 7 of row m (n < N) of C [rows][N] (fp32 or fp16, plain or added to):
// one 16-byte (fp16) or two (fp32) stores where the row holds all 8 and C allows it (wide), else
// element by element.
DEV void store8_out(void *C, int N, int m, int n, f4 v0, f4 v1, bool wide, int c_f32, int accumulate) {
    const size_t idx = (size_t)m * N + n;
    if (wide && n + 8 <= N) {
        if (c_f32) {
            f4 *q = (f4 *)((float *)C + idx);
            q[0] = accumulate ? q[0] + v0 : v0;
            q[1] = accumulate ? q[1] + v1 : v1;
        } else {
            h8 *q = (h8 *)((_Float16 *)C + idx);
            if (accumulate) {
                const h8 o = *q;
                v0 += f4{(float)o[0], (float)o[1], (float)o[2], (float)o[3]};
                v1 += f4{(float)o[4], (float)o[5], (float)o[6], (float)o[7]};
            }
            *q = h8{(_Float16)v0.x, (_Float16)v0.y, (_Float16)v0.z, (_Float16)v0.w,
                    (_Float16)v1.x, (_Float16)v1.y, (_Float16)v1.z, (_Float16)v1.w};
        }
    } else {
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        for (int e = 0; e < 8 && n + e < N; e++) store_out(C, idx + e, v[e], c_f32, accumulate);
    }
}

// End of a full-K tile kernel's tile, held in LDS as fp32 rows of LD floats (BM x BN, NT threads).
// parts == 1: stored to C. parts > 1 (a K split, at most MAXP parts): every part stores its tile to
// partials[tile][part] with device-scope (sc1) 16-byte stores, waits for them and counts itself in
// on counters[tile]; the last of the tile's parts loads the others' in one round trip and adds all
// of them in part order (its own from LDS in its place), so the sum is the same whichever part
// arrives last, then writes C; the counter is left at zero. flag: an LDS word outside the tile.
// A partial tile is laid out by store instruction, not by row: 16-byte piece h (0, 1) of thread
// chunk c at (h NCH + c) 16 bytes, so the 64 lanes of each store and load cover 1 KB contiguously
// (row order would leave every 32-byte sector half written by each of two instructions).
template <int BM, int BN, int NT, int MAXP, class Args>
DEV void tile_finish(const char *lds, const Args &g, int m0, int n0, int tile, int part, int *flag) {
    constexpr int LD = BN + 4, CH = BN / 8, NCH = BM * CH, CPT = (NCH + NT - 1) / NT;  // 8-value chunks
    static_assert(NCH % NT == 0 || NCH < NT, "chunks per thread");
    constexpr uint32_t TILE = BM * BN * 4;  // bytes per partial tile
    const int M = g.M, N = g.N;
    const bool wide = (N & 7) == 0 && ((uintptr_t)g.C & 15u) == 0;
    f4 pv[MAXP][CPT][2];
    if (g.parts > 1) {
        const rsrc_t rp = make_rsrc(g.partials, (uint32_t)g.ntiles * (uint32_t)g.parts * TILE);
        const uint32_t own = ((uint32_t)tile * (uint32_t)g.parts + (uint32_t)part) * TILE;
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int c = (int)threadIdx.x + NT * i, row = c / CH, ch = c - row * CH;
            if (c >= NCH) break;
            const uint32_t off = (uint32_t)c * 16u;
            buf_store16(rp, *(const f4 *)(lds + (row * LD + 8 * ch) * 4), own + off);
            buf_store16(rp, *(const f4 *)(lds + (row * LD + 8 * ch + 4) * 4), own + off + NCH * 16u);
        }
        if (!g.counters) return;  // parts stored only: a kernel of its own adds them (k_tile_reduce)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0) {
            const int last = atomicAdd(&g.counters[tile], 1) == g.parts - 1;
            if (last) atomicExch(&g.counters[tile], 0);
            *flag = last;
        }
        __syncthreads();
        if (!*flag) return;
#pragma unroll
        for (int p = 0; p < MAXP; p++)
#pragma unroll
            for (int i = 0; i < CPT; i++) {
                const int c = (int)threadIdx.x + NT * i, row = c / CH, ch = c - row * CH;
                const uint32_t off = (uint32_t)c * 16u;
                const uint32_t pb = ((uint32_t)tile * (uint32_t)g.parts + (uint32_t)p) * TILE;
                if (c >= NCH) {
                    pv[p][i][0] = pv[p][i][1] = f4{0.f, 0.f, 0.f, 0.f};
                } else if (p < g.parts && p != part) {
                    pv[p][i][0] = buf_load16_sc1(rp, off, pb);
                    pv[p][i][1] = buf_load16_sc1(rp, off + NCH * 16u, pb);
                } else {
                    pv[p][i][0] = *(const f4 *)(lds + (row * LD + 8 * ch) * 4);
                    pv[p][i][1] = *(const f4 *)(lds + (row * LD + 8 * ch + 4) * 4);
                }
            }
    }
    if (g.c_f32 == HQ_OUT_SWIGLU) {
        // gate/up pair matrix (one workgroup per tile, parts == 1): columns 16 c .. 16 c + 7 of the
        // tile are gate rows and 16 c + 8 .. + 15 the matching up rows; C is fp16 [M, N / 2] and
        // takes silu(gate) * up at columns (n0 + 16 c) / 2 .. + 7 (16-byte stores)
        constexpr int PCH = CH / 2, NP = BM * PCH, PPT = (NP + NT - 1) / NT;
        static_assert(CH % 2 == 0, "pairs of chunks");
        const int Nh = N / 2;
#pragma unroll
        for (int i = 0; i < PPT; i++) {
            const int pc = (int)threadIdx.x + NT * i, row = pc / PCH, c = pc - row * PCH, m = m0 + row, n = n0 + 16 * c;
            if (pc >= NP) break;
            if (m >= M || n >= N) continue;
            const float *r = (const float *)(lds + (row * LD + 16 * c) * 4);
            h8 y;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float gv = r[e], uv = r[8 + e];
                y[e] = (_Float16)(gv / (1.0f + expf(-gv)) * uv);
            }
            *(h8 *)((_Float16 *)g.C + (size_t)m * Nh + n / 2) = y;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < CPT; i++) {
        const int c = (int)threadIdx.x + NT * i, row = c / CH, ch = c - row * CH, m = m0 + row, n = n0 + 8 * ch;
        if (c >= NCH) break;
        f4 v0, v1;
        if (g.parts > 1) {
            v0 = f4{0.f, 0.f, 0.f, 0.f}, v1 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int p = 0; p < MAXP; p++)
                if (p < g.parts) {
                    v0 += pv[p][i][0];
                    v1 += pv[p][i][1];
                }
        } else {
            v0 = *(const f4 *)(lds + (row * LD + 8 * ch) * 4);
            v1 = *(const f4 *)(lds + (row * LD + 8 * ch + 4) * 4);
        }
        if (m >= M || n >= N) continue;
        store8_out(g.C, N, m, n, v0, v1, wide, g.c_f32, g.accumulate);
    }
}

// Quad permutes of one VGPR by DPP, written as inline assembly: this compiler merges
// __builtin_amdgcn_mov_dpp / update_dpp calls that share a DPP control but read different
// registers into one move of the first register (observed on gfx950, ROCm 7.2). The s_nop gives
// the source's producer 5 wait states (a plain VALU write needs 2 before a DPP read; a
// v_dot2c_f32_f16 result needs more).
DEV float dpp_quad_1032(float v) {
    float r;
    asm volatile("s_nop 4\n\tv_mov_b32_dpp %0, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(v));
    return r;
}
DEV float dpp_quad_2301(float v) {
    float r;
    asm volatile("s_nop 4\n\tv_mov_b32_dpp %0, %1 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(v));
    return r;
}

// 4 x 4 transpose inside each quad of lanes: on entry lane k of a quad holds x[e] = X[e][k], on
// return x[e] = X[k][e]. Two rounds, each swapping the (register bit, lane bit) off-diagonal pairs:
// bit 0 through quad_perm [1,0,3,2], bit 1 through quad_perm [2,3,0,1].
DEV f4 quad_transpose(f4 x) {
    const int k = threadIdx.x & 3;
    f4 y, z;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float t = dpp_quad_1032(x[e ^ 1]);
        y[e] = ((e ^ k) & 1) ? t : x[e];
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float t = dpp_quad_2301(y[e ^ 2]);
        z[e] = ((e ^ k) & 2) ? t : y[e];
    }
    return z;
}

// Output tile of one wave: block (i, j) holds rows m0 + 16i + 4lg + e, column nw + 16j + ln in
// register e of lane (ln, lg). A quad transpose gives lane (4c + k, lg) row 4lg + k, columns
// 4c .. 4c + 3, stored as one 8-byte (fp16) or 16-byte (fp32) access when N % 4 == 0, else
// element by element (the same values and roundings either way).
template <int MB, int NB>
DEV void store_tile(void *C, const f4 (&acc)[MB][NB], int M, int N, int m0, int nw, int ln, int lg, int c_f32,
                    int accumulate) {
    const int k = ln & 3, c4 = ln & ~3;
    const bool wide = (N & 3) == 0;
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
        for (int i = 0; i < MB; i++) {
            const f4 y = quad_transpose(acc[i][j]);
            const int m = m0 + 16 * i + 4 * lg + k, n = nw + 16 * j + c4;
            if (m >= M || n >= N) continue;
            const size_t idx = (size_t)m * N + n;
            if (wide) {
                if (c_f32) {
                    f4 *c = (f4 *)((float *)C + idx);
                    *c = accumulate ? *c + y : y;
                } else {
                    h4 *c = (h4 *)((_Float16 *)C + idx);
                    *c = __builtin_convertvector(accumulate ? __builtin_convertvector(*c, f4) + y : y, h4);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (n + e < N) store_out(C, idx + e, y[e], c_f32, accumulate);
            }
        }
}

#endif
