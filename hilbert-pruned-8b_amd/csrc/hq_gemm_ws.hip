// hq_gemm_ws.hip - Q4_K GEMM for prefill shapes (M > 64) on gfx950, one output tile per workgroup.
//
// C[M,N] (+)= A[M,K] . W^T with A fp16 and W GGUF Q4_K super-blocks resident in HBM (reference
// arithmetic: cleanroom-transformer/src/ggml_quant.h:51-59, :135-150; matmul src/cpu_backend.c:38-54).
//
// Decomposition. Each workgroup computes one tile of 128 rows by BN = 32*NB columns over the whole
// of K (no partial tiles, no cross-workgroup traffic). The tile width is chosen per shape so the
// number of tiles fills the CUs (M = 512, N = 9728: 4 x 61 = 244 tiles of 128 x 160 on 256 CUs).
// Workgroup b runs on XCD b % 8; the four M-tiles of one N-tile are placed on the same XCD, so a
// weight slab is fetched from HBM once per XCD and served from that XCD's L2 to the others.
//
// Eight waves, two roles (one of each per SIMD, so one role's VALU work issues while the other's
// MFMAs run):
//   consumers (waves 0-3): wave (wm, wn) owns rows 64wm .. +64 and columns (BN/2)wn .. +BN/2 of the
//     tile: 4 x NB blocks of v_mfma_f32_16x16x32_f16, operands read from LDS.
//   producers (waves 4-7): stream the activation tile into LDS (buffer_load ... lds, no registers),
//     load the Q4_K bytes and decode them once per workgroup into an LDS tile of fp16 B operands,
//     and stage the per-unit min-term operands.
// K is walked in stages of 128 (half a super-block); LDS holds two stages (double buffering) and one
// s_barrier per stage hands a stage from producers to consumers.
//
// Arithmetic (no weight is ever rounded to 16 bits). Column n's accumulators hold its dot products
// in units of c_u = d_u (the super-block scale; 1 where d_u = 0) during super-block u: the main B
// operand is then the integer s*q (<= 945, exact in fp16; 0 where d_u = 0), where a super-block
// ends the accumulators are multiplied by c_u / c_{u+1} (fp32), and at the end by c_{U-1}. The min
// term -dmin * sum_sub m_sub * S_sub (S_sub = fp32 sum of the sub-block's 32 activations, as bf16
// hi + lo) is one bf16 MFMA per (row block, column block, super-block), after the rescale: A slots
// hold S_hi, S_lo, S_hi, S_lo of the 8 sub-blocks, B slots Bh, Bh, Bl, Bl with x = -dmin * m / c
// (fp32), Bh = bf16(x), Bl = bf16(x - Bh); the four products sum to S * x to about 2^-16 relative
// (bf16 keeps fp32's exponent range, so no S or x overflows). Q4_K: the producers form S from the
// staged activation tiles, so a super-block's min step runs at its end, once both of its stages are
// in LDS, in the next one's units (c = c_{u+1}; c_U = c_{U-1}). Q5_K (whose producers have no
// VALU time to spare for the sums): S comes from k_asums in HBM and the min step runs at the
// super-block's start, in its own units (c = c_u; the rescale by c_{u-1} / c_u comes first).
//
// LDS layouts (16-byte slots; a stage row is 128 k = 16 slots):
//   A tile [128 rows][16 slots], slot p of row r at p ^ (r & 15);
//   B tile [BN columns][16 slots], slot p of column c at p ^ (c & 15);
//   (the XOR swizzle makes the 16 lanes of an MFMA operand read hit 16 distinct slots: such reads run
//   at the full 256 bytes per clock)
//   S [128 rows][16 bf16] = hi[8], lo[8]; Bmin [BN][16 bf16] = Bh[8], Bl[8]; R [BN] fp32
//   c_{u-1} / c_u; CL [BN] fp32 c_u of the latest super-block staged; scale words [2][BN][2] (two
//   super-blocks: 6-bit scales of sub-blocks 0-3 and 4-7, zero where d = 0).
#include <type_traits>

#include "hq_device.h"
#include "hq_kernels.h"

namespace {
constexpr int WS_BM = 128;  // tile rows
constexpr int WS_KS = 128;  // K per pipeline stage
constexpr int WS_NT = 512;  // threads per workgroup

struct WsArgs {
    const uint8_t *W;  // Q4_K super-blocks, row n at n * row_bytes
    uint32_t row_bytes;
    const uint16_t *A;  // fp16 [M][K]
    int M, N, K;
    void *C;
    int c_f32, accumulate;
    const uint16_t *S;  // Q5_K: activation sub-block sums [M][K/256][16] (k_asums); Q4_K: unused
    int mt, nt;  // M-tiles, N-tiles
    // K split: each tile's super-blocks are cut into `parts` contiguous ranges, one workgroup each;
    // with parts > 1 every part stores its fp32 tile in partials[tile][part] and the last to arrive
    // (per-tile counter, left at zero) sums them in part order and writes C
    int parts;
    float *partials;
    int *counters;
    int ntiles;  // mt * nt
};

// Workgroup barrier without a memory fence: each role waits for exactly the memory operations the
// hand-off needs (explicit s_waitcnt before the call). A __syncthreads() fence would make the
// producers wait for every outstanding load, including weight loads meant for later stages.
DEV void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

DEV u2v buf_load8(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

// L2 prefetch: a 4-byte-per-lane LDS DMA of the bytes at voff into a scratch LDS slot that is never
// read (256 bytes at lds_addr). Written as assembly: the compiler waits for every LDS DMA it knows
// of before any later LDS access, which would put the fetch's latency in front of the next LDS
// read. The issuing wave waits for it (s_waitcnt vmcnt) before it ends. M0 is restored.
DEV void l2_touch(rsrc_t r, uint32_t voff, uint32_t lds_addr) {
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 1\n\tbuffer_load_dword %2, %3, 0 offen lds\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(save)
                 : "s"(lds_addr), "v"(voff), "s"(r)
                 : "memory");
}

// Epilogue through LDS. The output leaves the consumers' MFMA layout (lane (ln, lg) of block (i, j):
// row 16i + ln, 4 consecutive columns) as 16-byte pieces of 16 rows, which the memory system writes
// as partial lines; instead the consumers park the fp32 tile in LDS (rows padded by 4 floats against
// bank conflicts; the stage buffers are free once the main loop is done) and all 512 threads store
// it as whole row segments, 8 values per thread and access (tile_finish).
template <int NB>
DEV void ws_tile_to_lds(char *lds, const f4 (&acc)[4][NB], int wm, int wn, int ln, int lg) {
    constexpr int BN = 32 * NB, LD = BN + 4;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int r = 64 * wm + 16 * i + ln, c = (BN / 2) * wn + 16 * j + 4 * lg;
            *(f4 *)(lds + (r * LD + c) * 4) = acc[i][j];
        }
}

// LDS arena (bytes): A stages, B stages, S, Bmin, R, CL, scale words, prefetch scratch.
template <int NB>
struct WsLds {
    static constexpr int BN = 32 * NB;
    static constexpr int A = 0, A_BYTES = WS_BM * WS_KS * 2;  // per stage buffer
    static constexpr int B = 2 * A_BYTES, B_BYTES = BN * WS_KS * 2;
    static constexpr int S = B + 2 * B_BYTES;
    static constexpr int BM = S + WS_BM * 32;
    static constexpr int R = BM + BN * 32;
    static constexpr int CL = R + BN * 4;
    static constexpr int H = CL + BN * 4;
    static constexpr int PF = H + 2 * BN * 8;  // prefetch scratch, 4 x 256 bytes (never read)
    static constexpr int TOTAL = PF + 1024;
    static_assert(TOTAL <= 160 * 1024, "LDS budget");
};

// One consumer k-step (compile-time): A register set P (main k-steps); operand source SRC (0 / 1 =
// stage buffer, 2 = min-term tiles) at k-step F of the stage; BAR = last k-step of a stage (holds
// the stage barrier); NSRC / NF = the next k-step's source and k-step.
template <int P_, int SRC_, int F_, bool BAR_, int NSRC_, int NF_>
struct WsStep {
    static constexpr int P = P_, SRC = SRC_, F = F_, NSRC = NSRC_, NF = NF_;
    static constexpr bool BAR = BAR_;
};

// The tile body of k_gemm_q4_k_ws (T = Q4_K) and k_gemm_q5_k_ws (T = Q5_K: the same header, scale / min
// packing and sub-blocks, 176-byte super-blocks with the quants at byte 48 and a fifth bit per value in
// qh[32] at byte 16; its B operand s * q, q <= 31, s <= 63, is still an exact fp16 integer <= 1953).
template <int T, int NB>
DEV void ws_q4_tile(const WsArgs &g) {
    static_assert(T == HQ_TYPE_Q4_K || T == HQ_TYPE_Q5_K, "ws_q4_tile types");
    constexpr int SLOT = T == HQ_TYPE_Q5_K ? 176 : 144, QS = T == HQ_TYPE_Q5_K ? 48 : 16;
    constexpr int QL = T == HQ_TYPE_Q5_K ? 2 : 1;  // quant loads per column and stage
    using QR = std::conditional_t<T == HQ_TYPE_Q5_K, u4v, u2v>;  // Q5_K: qs bytes in .xy, qh bytes in .zw
    constexpr bool SUMS = T == HQ_TYPE_Q4_K;  // the producers form the activation sums
    constexpr int BN = 32 * NB;
    using L = WsLds<NB>;
    __shared__ __attribute__((aligned(256))) char lds[L::TOTAL];  // fragment addresses XOR bits 6-7
    _Float16 *const sA0 = (_Float16 *)(lds + L::A);
    _Float16 *const sB0 = (_Float16 *)(lds + L::B);
    uint16_t *const sS = (uint16_t *)(lds + L::S);
    uint16_t *const sBm = (uint16_t *)(lds + L::BM);
    uint32_t *const sH = (uint32_t *)(lds + L::H);
    float *const sR = (float *)(lds + L::R);
    float *const sCL = (float *)(lds + L::CL);
    auto sA = [&](int h) { return sA0 + h * (L::A_BYTES / 2); };
    auto sB = [&](int h) { return sB0 + h * (L::B_BYTES / 2); };

    // tile of this workgroup: XCD x = b % 8 takes N-tiles x, x + 8, ...; its slots run over the
    // M-tiles of one N-tile first
    const int b = blockIdx.x, x = b & 7, j8 = b >> 3, per = g.mt * g.parts;
    const int nt_i = x + 8 * (j8 / per), part = (j8 % per) / g.mt, mt_i = j8 % g.mt;
    if (nt_i >= g.nt) return;
    const int m0 = mt_i * WS_BM, n0 = nt_i * BN;
    // this part's super-blocks u0 .. u0 + U - 1 of UT; the operand bases are moved to u0 (row
    // strides stay K, UT), so the body below indexes super-blocks from 0
    const int M = g.M, N = g.N, K = g.K, UT = K / 256;
    const int u0 = part * UT / g.parts, U = (part + 1) * UT / g.parts - u0;
    const uint8_t *const Wb = g.W + (size_t)u0 * SLOT;
    const uint16_t *const Ab = g.A + (size_t)u0 * 256, *const Sb = SUMS ? g.A : g.S + (size_t)u0 * 16;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const rsrc_t ra = make_rsrc(Ab, (uint32_t)((size_t)M * K * 2 - (size_t)u0 * 512));
    const rsrc_t rw = make_rsrc(Wb, (uint32_t)((size_t)N * g.row_bytes - (size_t)u0 * SLOT));

    if (wave >= 4) {
        // ------------------------------------------------------------------ producers
        // Stage s's work, done in stage s - 1: its activation tile (LDS DMA) and its decoded B tile; in
        // an odd stage the min-term operands of the super-block it ends (Q4_K, with its activation
        // sums) or of the next one (Q5_K, with its S tile from HBM). Vector-memory
        // instructions are spread over the decode of the thread's columns (the texture path takes
        // ~20 clocks per instruction per CU, so a burst of them would stall the wave for the whole
        // burst); the end-of-stage wait covers the DMAs only (loads issued after them retire later).
        const int pw = __builtin_amdgcn_readfirstlane(wave - 4);  // wave-uniform LDS targets
        const int pt = tid - 256, xi = pt & 7;
        // activation DMA: instruction qq of wave pw fills rows 4(pw + 4qq) .. +4 (1 KB); lane l takes
        // row 4(pw + 4qq) + l/16, LDS slot l % 16, global chunk (l % 16) ^ (row & 15) (the row in the
        // VGPR offset, the one a buffer load range-checks: rows past M read zeros, none past A's end)
        const int arow = 4 * pw + (lane >> 4);
        const uint32_t a_voff = (uint32_t)(((m0 + arow) * K + 8 * ((lane & 15) ^ (arow & 15))) * 2);
        auto dma_a = [&](int s, int qq) {
            dma16(ra, sA(s & 1) + (pw + 4 * qq) * 512, a_voff + (uint32_t)(qq * 16 * K * 2), (uint32_t)(s * WS_KS * 2));
        };
        // Q5_K: S tile of unit u from HBM, 32 rows (1 KB) per wave; lane l: row 32pw + l/2, half l % 2
        const rsrc_t rs = make_rsrc(Sb, SUMS ? 0u : (uint32_t)((size_t)M * UT * 32 - (size_t)u0 * 32));
        const uint32_t s_voff = (uint32_t)(((m0 + 32 * pw + (lane >> 1)) * UT) * 32 + 16 * (lane & 1));
        auto dma_s = [&](int u) { dma16(rs, sS + pw * 512, s_voff, (uint32_t)(u * 32)); };
        // Q4_K: activation sub-block sums, from the stage buffers (the consumers read the same tiles): thread
        // pt takes row s_row = pt / 2 and, of a stage's four 32-value sub-blocks, 2 s_h and 2 s_h + 1
        // (chunks 8 s_h .. + 7, at slots chunk ^ (row & 15)); fp32 sums in the order of the stored
        // fp16 values, eight at a time (the order of the k_asums pre-pass, so S is the same bits);
        // the even stage's two wait in registers for the odd stage's, then the unit's S row goes out
        // as bf16 hi, lo
        const int s_row = pt >> 1, s_h = pt & 1;
        auto stage_sums = [&](int buf, float &t0, float &t1) {
            using lds_u4 = const __attribute__((address_space(3))) u4v;
            const uint32_t base = (uint32_t)(uintptr_t)sA(buf) + (uint32_t)s_row * (WS_KS * 2);
            u4v v[8];
#pragma unroll
            for (int q = 0; q < 8; q++)
                v[q] = *(lds_u4 *)(uintptr_t)(base + 16u * ((uint32_t)(8 * s_h + q) ^ (uint32_t)(s_row & 15)));
            t0 = sum8(v[3], sum8(v[2], sum8(v[1], sum8(v[0], 0.f))));
            t1 = sum8(v[7], sum8(v[6], sum8(v[5], sum8(v[4], 0.f))));
        };
        auto bf_pair = [](float a, float b, uint32_t &hi, uint32_t &lo) {
            const __bf16 ha = (__bf16)a, hb = (__bf16)b;
            const __bf16 la = (__bf16)(a - (float)ha), lb = (__bf16)(b - (float)hb);
            hi = (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
            lo = (uint32_t)__builtin_bit_cast(uint16_t, la) | ((uint32_t)__builtin_bit_cast(uint16_t, lb) << 16);
        };
        float se0 = 0.f, se1 = 0.f;  // this unit's even-stage sums
        auto write_sums = [&](float so0, float so1) {
            using lds_u32 = __attribute__((address_space(3))) uint32_t;
            uint32_t he, le, ho, lo;
            bf_pair(se0, se1, he, le);
            bf_pair(so0, so1, ho, lo);
            const uint32_t row = (uint32_t)(uintptr_t)(sS + s_row * 16);
            *(lds_u32 *)(uintptr_t)(row + 4u * (uint32_t)s_h) = he;          // hi of sub-blocks 2 s_h, + 1
            *(lds_u32 *)(uintptr_t)(row + 4u * (uint32_t)(2 + s_h)) = ho;    // hi of 4 + 2 s_h, + 1
            *(lds_u32 *)(uintptr_t)(row + 16u + 4u * (uint32_t)s_h) = le;    // lo
            *(lds_u32 *)(uintptr_t)(row + 16u + 4u * (uint32_t)(2 + s_h)) = lo;
        };
        // quant bytes: this thread's columns c_i = pt/8 + 32i (i < NB), half-chunk xi of each stage
        // (bytes QS + 8(8(s % 2) + xi) of super-block s/2; Q5_K also qh bytes 8(xi % 4) .. + 7, the
        // fifth bits of the same values). Four register sets: stage s's go to Q[s % 4], three stages
        // before its decode.
        uint32_t w_voff[NB], h_voff[NB];
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const uint32_t row = (uint32_t)(n0 + (pt >> 3) + 32 * i) * g.row_bytes;
            w_voff[i] = row + (uint32_t)QS + 8u * (uint32_t)xi;
            h_voff[i] = row + 16u + 8u * (uint32_t)(xi & 3);
        }
        QR Q[4][NB];
        auto load_q = [&](QR (&q)[NB], int s, int i) {
            const u2v w = buf_load8(rw, w_voff[i], (uint32_t)((s >> 1) * SLOT + 64 * (s & 1)));
            if constexpr (QL == 2) {
                const u2v h = buf_load8(rw, h_voff[i], (uint32_t)((s >> 1) * SLOT));
                q[i] = u4v{w.x, w.y, h.x, h.y};
            } else {
                q[i] = w;
            }
        };
        // super-block headers, one column per thread (pt < BN; the other threads load column 0's
        // and drop it, so that every wave issues the same loads): H[u % 2] holds unit u's
        const bool colt = pt < BN;
        const uint32_t m_voff = (uint32_t)(n0 + (colt ? pt : 0)) * g.row_bytes;
        u4v H[2];
        auto load_hdr = [&](u4v &h, int u) { h = buf_load16(rw, m_voff, (uint32_t)(u * SLOT)); };
        // a unit's scale words for the decode (sub-blocks 0-3 / 4-7; zero where d = 0, so that B = 0
        // there) -> sH[u % 2][pt]
        auto write_scales = [&](const u4v hm, int buf) {
            if (!colt) return;
            uint32_t sw0, sw1, mw0, mw1;
            q4k_scale_words(hm.y, hm.z, hm.w, sw0, sw1, mw0, mw1);
            const uint32_t nz = (hm.x & 0x7fffu) ? 0xffffffffu : 0u;
            *(u2v *)(sH + (buf * BN + pt) * 2) = u2v{sw0 & nz, sw1 & nz};
        };
        // Q4_K: min-term operands of a super-block (header hm of column pt) in the units of the next
        // one (header hn; the last super-block: hn = hm), the rescale ratio c_u / c_{u+1} (1 for the
        // last) and c_{u+1}
        auto write_min = [&](const u4v hm, const u4v hn, bool last) {
            if (!colt) return;
            uint32_t sw0, sw1, mw0, mw1;
            q4k_scale_words(hm.y, hm.z, hm.w, sw0, sw1, mw0, mw1);
            const float d = h2f((uint16_t)hm.x), dmin = h2f((uint16_t)(hm.x >> 16)), dn = h2f((uint16_t)hn.x);
            const float c_u = d != 0.0f ? d : 1.0f, c = dn != 0.0f ? dn : 1.0f, inv = 1.0f / c;
            u4v bh, bl;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t w = q < 2 ? mw0 : mw1;
                const float x0 = (-dmin * (float)byte_of(w, 2 * (q & 1))) * inv;  // -dmin * m is exact
                const float x1 = (-dmin * (float)byte_of(w, 2 * (q & 1) + 1)) * inv;
                const __bf16 h0 = (__bf16)x0, h1 = (__bf16)x1;
                const __bf16 l0 = (__bf16)(x0 - (float)h0), l1 = (__bf16)(x1 - (float)h1);
                bh[q] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                bl[q] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
            }
            *(u4v *)(sBm + pt * 16) = bh;
            *(u4v *)(sBm + pt * 16 + 8) = bl;
            sR[pt] = last ? 1.0f : c_u * inv;
            sCL[pt] = c;
        };
        // Q5_K: min-term operands, rescale ratio and unit of a super-block (header hm of column pt;
        // c_prev = the column's previous unit, 1 before the first)
        float c_prev = 1.0f;
        auto write_min_start = [&](const u4v hm) {
            if (!colt) return;
            uint32_t sw0, sw1, mw0, mw1;
            q4k_scale_words(hm.y, hm.z, hm.w, sw0, sw1, mw0, mw1);
            const float d = h2f((uint16_t)hm.x), dmin = h2f((uint16_t)(hm.x >> 16));
            const float c = d != 0.0f ? d : 1.0f, inv = 1.0f / c;
            u4v bh, bl;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t w = q < 2 ? mw0 : mw1;
                const float x0 = (-dmin * (float)byte_of(w, 2 * (q & 1))) * inv;  // -dmin * m is exact
                const float x1 = (-dmin * (float)byte_of(w, 2 * (q & 1) + 1)) * inv;
                const __bf16 h0 = (__bf16)x0, h1 = (__bf16)x1;
                const __bf16 l0 = (__bf16)(x0 - (float)h0), l1 = (__bf16)(x1 - (float)h1);
                bh[q] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                bl[q] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
            }
            *(u4v *)(sBm + pt * 16) = bh;
            *(u4v *)(sBm + pt * 16 + 8) = bl;
            sR[pt] = c_prev * inv;
            sCL[pt] = c;
            c_prev = c;
        };
        // The vector-memory items of a stage: 8 activation DMAs, (Q5_K) the S DMA, a header load
        // (into hd), NB quant loads (into qd; s_* / u_* < 0: item absent); item k is issued before
        // column k * NB / NI of the decode. Whatever is issued after the DMAs may still be in flight at
        // the end of the stage: a load has until the end of the next stage.
        constexpr int KH = SUMS ? 8 : 9, NI = KH + 1 + NB;  // the header's item, items
        auto issue = [&](int i, int s_dma, int u_s, int u_h, u4v &hd, int s_q, QR (&qd)[NB]) {
#pragma unroll
            for (int k = 0; k < NI; k++) {
                if (k * NB / NI != i) continue;
                if (k < 8) {
                    if (s_dma >= 0) dma_a(s_dma, k);
                } else if (k < KH) {
                    if (u_s >= 0) dma_s(u_s);
                } else if (k == KH) {
                    if (u_h >= 0) load_hdr(hd, u_h);
                } else if (s_q >= 0) {
                    load_q(qd, s_q, k - KH - 1);
                }
            }
        };
        // decode stage s (H = s % 2) into sB(H): column c_i's half-chunk X = 8H + xi covers
        // sub-blocks 2p (low nibbles) and 2p + 1 (high) with p = 2H + xi/4; its 8 + 8 values sit at
        // stage slots 8(xi/4) + (xi % 4) and that + 4. The scale words of a unit are read from sH
        // once, at the start of its even stage's decode (both words: Sw1 keeps the odd stage's).
        const int slot_lo = 8 * (xi >> 2) + (xi & 3);
        const uint32_t ssel = (xi >> 2) ? 0x04030402u : 0x04010400u;  // scale bytes 2(p%2), 2(p%2)+1
        uint32_t Sw1[NB];
        auto decode = [&](auto hc, auto sbc, const QR (&q)[NB], int s_dma, int u_s, int u_h, u4v &hd, int s_q,
                          QR (&qd)[NB]) {
            constexpr int HS = decltype(hc)::value, SB = decltype(sbc)::value;
            _Float16 *dst = sB(HS);
            const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
            // Q4_K: low nibbles as 1024 + q, high as 1024 + 16q; Q5_K: both as 1024 + q (5 bits)
            const h2 kmul = {(_Float16)1.0f, (_Float16)(QL == 2 ? 1.0f : 0.0625f)};
            const h2 kadd = {(_Float16)-1024.0f, (_Float16)(QL == 2 ? -1024.0f : -64.0f)};
            uint32_t Sw0[NB];
            if constexpr (HS == 0) {
#pragma unroll
                for (int i = 0; i < NB; i++) {
                    const u2v w = *(const u2v *)(sH + (SB * BN + (pt >> 3) + 32 * i) * 2);
                    Sw0[i] = w.x;
                    Sw1[i] = w.y;
                }
            }
#pragma unroll
            for (int i = 0; i < NB; i++) {
                issue(i, s_dma, u_s, u_h, hd, s_q, qd);
                const uint32_t c = (uint32_t)((pt >> 3) + 32 * i), sg = c & 15u;
                const uint32_t sw = HS ? Sw1[i] : Sw0[i];
                const h2 sp = as_h2(__builtin_amdgcn_perm(0x64646464u, sw, ssel)) - k1024;
                const h2 mu = sp * kmul, ad = sp * kadd;
                h8 lo, hi;
                if constexpr (QL == 2) {
                    // sub-blocks 2p (low nibbles, qh bit 2p) and 2p + 1 (high, bit 2p + 1), p = 2H + xi / 4
                    const int p = 2 * HS + (xi >> 2);
                    const u4v w = q[i];
                    const u2v l5 = {(w.x & 0x0f0f0f0fu) | (((w.z >> (2 * p)) & 0x01010101u) << 4),
                                    (w.y & 0x0f0f0f0fu) | (((w.w >> (2 * p)) & 0x01010101u) << 4)};
                    const u2v h5 = {((w.x >> 4) & 0x0f0f0f0fu) | (((w.z >> (2 * p + 1)) & 0x01010101u) << 4),
                                    ((w.y >> 4) & 0x0f0f0f0fu) | (((w.w >> (2 * p + 1)) & 0x01010101u) << 4)};
                    lo = decode8m(l5, 0xffffffffu, h2{mu.x, mu.x}, h2{ad.x, ad.x});
                    hi = decode8m(h5, 0xffffffffu, h2{mu.y, mu.y}, h2{ad.y, ad.y});
                } else {
                    lo = decode8<false>(q[i], h2{mu.x, mu.x}, h2{ad.x, ad.x});
                    hi = decode8<true>(q[i], h2{mu.y, mu.y}, h2{ad.y, ad.y});
                }
                *(h8 *)(dst + c * WS_KS + 8 * ((uint32_t)slot_lo ^ sg)) = lo;
                *(h8 *)(dst + c * WS_KS + 8 * ((uint32_t)(slot_lo + 4) ^ sg)) = hi;
            }
        };
        // end of a stage: this wave's LDS writes done, and every load issued before the last
        // n_in_flight ones (the DMAs among them) landed; then the barrier
        auto end_stage = [&](int n_in_flight) {
            if (n_in_flight == 2 * QL * NB + 1) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(2 * QL * NB + 1) : "memory");
            else if (n_in_flight == QL * NB + 1) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(QL * NB + 1) : "memory");
            else if (n_in_flight == QL * NB) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(QL * NB) : "memory");
            else if (n_in_flight == 1) asm volatile("s_waitcnt vmcnt(1) lgkmcnt(0)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
            wg_barrier();
        };
        using i0 = std::integral_constant<int, 0>;
        using i1 = std::integral_constant<int, 1>;
        const int S2 = 2 * U;  // stages
        // prologue, phase 1: headers of units 0 and 1, stage 0's quants and activation tile (Q5_K:
        // and unit 0's S tile), all in flight together (the compiler waits for the outstanding DMAs
        // before the LDS writes that follow, so they cost one memory latency, not two); unit 0's scale
        // words; the min-term tiles of the consumers' first min step: Q4_K, "unit -1" (zero S and
        // Bmin, ratio 1), Q5_K, unit 0's; the quants of stages 1 and 2, the header of unit 2
        load_hdr(H[0], 0);
        load_hdr(H[1], U > 1 ? 1 : 0);
#pragma unroll
        for (int i = 0; i < NB; i++) load_q(Q[0], 0, i);
#pragma unroll
        for (int k = 0; k < 8; k++) dma_a(0, k);
        if constexpr (!SUMS) dma_s(0);
        write_scales(H[0], 0);
        if constexpr (SUMS) {
            *(u4v *)(sS + pt * 8) = u4v{0u, 0u, 0u, 0u};
            if (colt) {
                *(u4v *)(sBm + pt * 16) = u4v{0u, 0u, 0u, 0u};
                *(u4v *)(sBm + pt * 16 + 8) = u4v{0u, 0u, 0u, 0u};
                sR[pt] = 1.0f;
            }
        } else {
            write_min_start(H[0]);
        }
        u4v hcur = H[0];  // Q4_K: header of the super-block whose min-term operands go out next
#pragma unroll
        for (int i = 0; i < NB; i++) load_q(Q[1], 1, i);
#pragma unroll
        for (int i = 0; i < NB; i++) load_q(Q[2], S2 > 2 ? 2 : 0, i);
        load_hdr(H[0], U > 2 ? 2 : 0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wg_barrier();  // unit 0's scale words are visible
        // phase 2: decode stage 0; the stage-0 barrier
        decode(i0{}, i0{}, Q[0], -1, -1, -1, H[1], -1, Q[3]);
        end_stage(2 * QL * NB + 1);  // DMAs of phase 1 landed (Q[1], Q[2], H[0] may be in flight)
        // Super-block u, in stages 2u (P = u % 2 picks the register sets) and 2u + 1.
        auto unit = [&](auto par, int u) {
            constexpr int P = decltype(par)::value;
            const int t = 2 * u;
            const bool q3 = t + 3 < S2, q4 = t + 4 < S2, nx = u + 1 < U, h3 = u + 3 < U;
            // stage 2u: decode stage 2u + 1 (this unit, odd half); activation tile 2u + 1; quants
            // of stage 2u + 3; the next unit's scale words; Q4_K: the sums of stage 2u (buffer 0)
            decode(i1{}, std::integral_constant<int, P>{}, Q[(2 * P + 1) & 3], t + 1, -1, -1, H[P], q3 ? t + 3 : -1,
                   Q[(2 * P + 3) & 3]);
            if (nx) write_scales(H[P ^ 1], P ^ 1);
            if constexpr (SUMS) stage_sums(0, se0, se1);
            end_stage(q3 ? QL * NB : 0);
            // stage 2u + 1, Q4_K: this unit's S tile (with the sums of stage 2u + 1, buffer 1) and
            // min-term operands in the next unit's units (read by the consumers' min step at this
            // stage's end); Q5_K: the next unit's min-term operands (its S tile comes by DMA below)
            if constexpr (SUMS) {
                float so0, so1;
                stage_sums(1, so0, so1);
                write_sums(so0, so1);
                if (!nx) {  // the last stage: nothing else to stage; the LDS writes land before its barrier
                    write_min(hcur, hcur, true);
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    return;
                }
                write_min(hcur, H[P ^ 1], false);
                hcur = H[P ^ 1];
            } else {
                if (!nx) return;  // the last stage has nothing to stage
                write_min_start(H[P ^ 1]);
            }
            // (the next unit's header's last use here: the register then takes the header of unit
            // u + 3); decode stage 2u + 2 (next unit, even half); activation tile 2u + 2, (Q5_K) the
            // next unit's S tile, header u + 3, quants of stage 2u + 4
            decode(i0{}, std::integral_constant<int, P ^ 1>{}, Q[(2 * P + 2) & 3], t + 2, SUMS ? -1 : u + 1,
                   h3 ? u + 3 : -1, H[P ^ 1], q4 ? t + 4 : -1, Q[(2 * P) & 3]);
            end_stage((q4 ? QL * NB : 0) + (h3 ? 1 : 0));
        };
        int u = 0;
        for (; u + 1 < U; u += 2) {
            unit(i0{}, u);
            unit(i1{}, u + 1);
        }
        if (u < U) unit(i0{}, u);
        wg_barrier();  // the last stage's barrier
        wg_barrier();  // the consumers' output tile is in LDS
        tile_finish<WS_BM, 32 * NB, WS_NT, 4>(lds, g, m0, n0, nt_i * g.mt + mt_i, part, (int *)(lds + L::PF));
        return;
    }

    // ---------------------------------------------------------------------- consumers
    // A consumer wave's work is a stream of k-steps of 4 x NB MFMAs into acc: per super-block one min
    // k-step (S x Bmin, bf16; its MFMA groups first rescale the blocks they update by c_{u-1} / c_u)
    // and 8 main k-steps (32 k of a stage buffer). Every k-step reads the operands of the next one
    // while its own MFMAs run: the next A fragments first (into the other A register set; after the
    // second group in a min k-step), the next B fragment j right after the MFMAs that used B fragment
    // j. The last k-step of a stage passes the stage barrier after its first MFMA groups (its own
    // operands are in registers by then) and reads the next stage's operands after it. Scheduling
    // barriers keep that order: left alone, the compiler sinks every LDS read next to its first
    // use, and the MFMAs wait for LDS latency at every group.
    const int wm = wave & 1, wn = wave >> 1, ln = lane & 15, lg = lane >> 4;
    // slot (4f + lg) ^ ln of row ln: bits 4-5 of the byte offset from (lg ^ ln) & 3, bits 6-7 from
    // f ^ (ln >> 2), so the k-step-f address is the k-step-0 address with 64 f XORed in (rows are
    // 256-byte aligned)
    const uint32_t sw0 = 16u * ((uint32_t)lg ^ (uint32_t)ln);
    const uint32_t a_lane = (uint32_t)(uintptr_t)sA(0) + (uint32_t)((64 * wm + ln) * WS_KS * 2) + sw0;
    const uint32_t b_lane = (uint32_t)(uintptr_t)sB(0) + (uint32_t)(((BN / 2) * wn + ln) * WS_KS * 2) + sw0;
    using lds_h8 = const __attribute__((address_space(3))) h8;
    using lds_f4 = const __attribute__((address_space(3))) f4;
    auto lds_at = [](uint32_t byte) { return *(lds_h8 *)(uintptr_t)byte; };
    const uint32_t s_base = (uint32_t)(uintptr_t)(sS + (64 * wm + ln) * 16 + 8 * (lg & 1));
    const uint32_t m_base = (uint32_t)(uintptr_t)(sBm + ((BN / 2) * wn + ln) * 16 + 8 * (lg >> 1));
    // per-column fp32 factors of lane (ln, lg) in block j: columns 16j + 4lg .. + 3
    const uint32_t r_base = (uint32_t)(uintptr_t)(sR + (BN / 2) * wn + 4 * lg);
    const uint32_t cl_base = (uint32_t)(uintptr_t)(sCL + (BN / 2) * wn + 4 * lg);
    // operand sources: 0 / 1 = stage buffer, 2 = min-term tiles; A fragment i rows 16i.., B fragment
    // j columns 16j.. of the wave's block
    auto ldA = [&](int src, int i, int f) -> h8 {
        return src == 2 ? lds_at(s_base + i * 16 * 32)
                        : lds_at((a_lane ^ (64u * f)) + src * L::A_BYTES + i * 16 * WS_KS * 2);
    };
    auto ldB = [&](int src, int j, int f) -> h8 {
        return src == 2 ? lds_at(m_base + j * 16 * 32)
                        : lds_at((b_lane ^ (64u * f)) + src * L::B_BYTES + j * 16 * WS_KS * 2);
    };
    auto ldR = [&](int j) { return *(lds_f4 *)(uintptr_t)(r_base + j * 16 * 4); };
    f4 acc[4][NB];
    h8 fa[2][4], am[4], fb[NB];  // A fragments: main k-steps alternate fa[0] / fa[1]; min k-step am
    f4 rr[2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    constexpr int JB = NB >= 3 ? 2 : 1;  // MFMA groups of a stage's last k-step before its barrier
    auto kstep = [&](auto cfg) {
        using C = decltype(cfg);
        constexpr int P = C::P;
        auto read_next_a = [&]() {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if constexpr (C::NSRC == 2) am[i] = ldA(2, i, 0);
                else fa[P ^ 1][i] = ldA(C::NSRC, i, C::NF);
            }
            if constexpr (C::NSRC == 2) rr[0] = ldR(0);
        };
        // the next k-step's A fragments: at the start, or (min k-step) after group JA
        constexpr int JA = C::SRC == 2 ? JB : 0;
#pragma unroll
        for (int j = 0; j < NB; j++) {
            if (!C::BAR && j == JA) read_next_a();
            if (C::BAR && j == JB) {
                // every read of this stage's buffers has been issued: wait for them, hand the
                // buffers back, then read the next stage's first operands
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                wg_barrier();
                read_next_a();
#pragma unroll
                for (int jj = 0; jj < JB; jj++) fb[jj] = ldB(C::NSRC, jj, C::NF);
            }
            if constexpr (C::SRC == 2) {
                if (j + 1 < NB) rr[(j + 1) & 1] = ldR(j + 1);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i][j] *= rr[j & 1];
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i][j] = mfma_bf16(fb[j], am[i], acc[i][j]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i][j] = mfma(fb[j], fa[P][i], acc[i][j]);
            }
            if (!(C::BAR && j < JB)) fb[j] = ldB(C::NSRC, j, C::NF);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    wg_barrier();  // the producers' prologue, phase 1
    wg_barrier();  // stage 0 and unit 0's min-term tiles are in LDS
#pragma unroll
    for (int i = 0; i < 4; i++) am[i] = ldA(2, i, 0);
#pragma unroll
    for (int j = 0; j < NB; j++) fb[j] = ldB(2, j, 0);
    rr[0] = ldR(0);
    // Weight prefetch: the producers' loads retire in issue order, so a load that misses L2 would
    // hold up the end-of-stage wait for the activation DMA issued after it. The consumers (whose
    // own waits cover only LDS reads) touch every cache line of super-block u + 3 of the tile's
    // columns at the start of super-block u; the mt workgroups that share an N-tile (same XCD, same
    // L2) split the columns. Lane e of the four consumer waves (and of e + 256, ...) touches bytes
    // {0, 72, 143} (e % 3) of column mt_i + mt (e / 3).
    const int pf_cols = (BN - mt_i + g.mt - 1) / g.mt, pf_lanes = 3 * pf_cols;
    const rsrc_t rw_pf = rw;
    const uint32_t pf_lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds + L::PF) + 256u * (uint32_t)wave);
    auto prefetch = [&](int v) {
        for (int e0 = 64 * wave; e0 < pf_lanes; e0 += 256) {
            const int e = e0 + lane, jc = e / 3, t = e - 3 * jc;
            const int c = mt_i + g.mt * (e < pf_lanes ? jc : 0);
            const uint32_t voff = (uint32_t)(n0 + c) * g.row_bytes + (uint32_t)SLOT * (uint32_t)v +
                                  (t == 0 ? 0u : t == 1 ? (uint32_t)SLOT / 2 : (uint32_t)SLOT - 1);
            l2_touch(rw_pf, voff, pf_lds);
        }
    };
    // per super-block: a min k-step (Q4_K: the previous super-block's, before the first with zero
    // operands and ratio 1; Q5_K: its own), 4 k-steps of the even stage (buffer 0), 4 of the odd stage
    // (buffer 1); the last k-step reads the next min k-step's operands. Q4_K: the last super-block's
    // min k-step follows the loop; Q5_K: after the last super-block those reads return stale LDS
    // contents that are never used.
    for (int u = 0; u < U; u++) {
        if (u + 3 < U) prefetch(u + 3);
        kstep(WsStep<1, 2, 0, false, 0, 0>{});  // P = 1: E0's A fragments go to fa[0]
        kstep(WsStep<0, 0, 0, false, 0, 1>{});
        kstep(WsStep<1, 0, 1, false, 0, 2>{});
        kstep(WsStep<0, 0, 2, false, 0, 3>{});
        kstep(WsStep<1, 0, 3, true, 1, 0>{});
        kstep(WsStep<0, 1, 0, false, 1, 1>{});
        kstep(WsStep<1, 1, 1, false, 1, 2>{});
        kstep(WsStep<0, 1, 2, false, 1, 3>{});
        kstep(WsStep<1, 1, 3, true, 2, 0>{});
    }
    if constexpr (SUMS) kstep(WsStep<1, 2, 0, false, 0, 0>{});  // the last super-block's min k-step (ratio 1)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the prefetches
    // back to true units: multiply by the last super-block's c (written with its min-term tiles)
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const f4 cl = *(lds_f4 *)(uintptr_t)(cl_base + j * 16 * 4);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i][j] *= cl;
    }
    ws_tile_to_lds<NB>(lds, acc, wm, wn, ln, lg);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wg_barrier();
    tile_finish<WS_BM, 32 * NB, WS_NT, 4>(lds, g, m0, n0, nt_i * g.mt + mt_i, part, (int *)(lds + L::PF));
}

template <int NB>
__global__ void __launch_bounds__(WS_NT) k_gemm_q4_k_ws(WsArgs g) {
    ws_q4_tile<HQ_TYPE_Q4_K, NB>(g);
}
template <int NB>
__global__ void __launch_bounds__(WS_NT) k_gemm_q5_k_ws(WsArgs g) {
    ws_q4_tile<HQ_TYPE_Q5_K, NB>(g);
}

// ---------------------------------------------------------------------------------------------
// Q8_0 tile kernel: the same decomposition, roles and consumer k-step stream as k_gemm_q4_k_ws,
// without the min term and the rescale (a Q8_0 weight is q * d with one scale per 32 values, so the
// B operand carries the scale: fp16(q * d), one rounding of the exact product, as in the other
// Q8_0 kernels). Weights: the quant plane (bytes u = q + 128, row n at n * K) and the fp16 scale
// plane (row n at n * ldd). Per 128-K stage, producer thread (column c = pt / 8 + 32 i, xi = pt % 8)
// takes values 16 xi .. 16 xi + 15 of the stage: one 16-byte quant load and one 2-byte scale load
// per column, three stages ahead (four register sets), decoded into B-tile slots 2 xi, 2 xi + 1.
template <int NB>
struct Ws8Lds {
    static constexpr int BN = 32 * NB;
    static constexpr int A = 0, A_BYTES = WS_BM * WS_KS * 2;
    static constexpr int B = 2 * A_BYTES, B_BYTES = BN * WS_KS * 2;
    static constexpr int PF = B + 2 * B_BYTES;  // prefetch scratch, 4 x 256 bytes (never read)
    static constexpr int TOTAL = PF + 1024;
    static_assert(TOTAL <= 160 * 1024, "LDS budget");
};

struct Ws8Args {
    const uint8_t *Q;   // quant plane, bytes u = q + 128
    const uint16_t *D;  // fp16 scale plane
    int ldd;
    const uint16_t *A;
    int M, N, K;
    void *C;
    int c_f32, accumulate;
    int mt, nt;
    int parts;  // K split as in WsArgs (ranges of 128-wide stages)
    float *partials;
    int *counters;
    int ntiles;
};

// 16 fp16 values fp16(q * d) from 16 stored bytes u = q + 128: fp16(1024 + u) - 1152 = q exactly,
// then one rounding of q * d
DEV void decode16_q8_0(const u4v q, h2 d2, h8 &lo, h8 &hi) {
    const h2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    h2 v[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = (as_h2(perm_lo(w[i])) + bias) * d2;
        v[2 * i + 1] = (as_h2(perm_hi(w[i])) + bias) * d2;
    }
    lo = h8{v[0].x, v[0].y, v[1].x, v[1].y, v[2].x, v[2].y, v[3].x, v[3].y};
    hi = h8{v[4].x, v[4].y, v[5].x, v[5].y, v[6].x, v[6].y, v[7].x, v[7].y};
}

// Consumers of the LDS-decode kernels whose B tile holds the weights themselves (Q8_0 and the
// k-quants of k_gemm_kq_ws: no min term, no rescale): the k-step stream of k_gemm_q4_k_ws without
// its min k-step, 4 main k-steps per 128-K stage, each reading the next k-step's operands while its
// MFMAs run, the stage barrier inside a stage's last k-step. S2 stages; prefetch(s) warms L2 with the
// weights of stages s and s + 1 (issued every second stage, four stages ahead). Ends with the fp32
// tile in LDS and a barrier, for tile_finish.
template <int NB, class L, class Pf>
DEV void ws_plain_consumers(char *lds, int wave, int lane, int S2, Pf &prefetch) {
    constexpr int BN = 32 * NB;
    _Float16 *const sA0 = (_Float16 *)(lds + L::A);
    _Float16 *const sB0 = (_Float16 *)(lds + L::B);
    const int wm = wave & 1, wn = wave >> 1, ln = lane & 15, lg = lane >> 4;
    const uint32_t sw0 = 16u * ((uint32_t)lg ^ (uint32_t)ln);
    const uint32_t a_lane = (uint32_t)(uintptr_t)sA0 + (uint32_t)((64 * wm + ln) * WS_KS * 2) + sw0;
    const uint32_t b_lane = (uint32_t)(uintptr_t)sB0 + (uint32_t)(((BN / 2) * wn + ln) * WS_KS * 2) + sw0;
    using lds_h8 = const __attribute__((address_space(3))) h8;
    auto lds_at = [](uint32_t byte) { return *(lds_h8 *)(uintptr_t)byte; };
    auto ldA = [&](int src, int i, int f) -> h8 {
        return lds_at((a_lane ^ (64u * f)) + src * L::A_BYTES + i * 16 * WS_KS * 2);
    };
    auto ldB = [&](int src, int j, int f) -> h8 {
        return lds_at((b_lane ^ (64u * f)) + src * L::B_BYTES + j * 16 * WS_KS * 2);
    };
    f4 acc[4][NB];
    h8 fa[2][4], fb[NB];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    constexpr int JB = NB >= 3 ? 2 : 1;
    auto kstep = [&](auto cfg) {
        using C = decltype(cfg);
        constexpr int P = C::P;
        auto read_next_a = [&]() {
#pragma unroll
            for (int i = 0; i < 4; i++) fa[P ^ 1][i] = ldA(C::NSRC, i, C::NF);
        };
#pragma unroll
        for (int j = 0; j < NB; j++) {
            if (!C::BAR && j == 0) read_next_a();
            if (C::BAR && j == JB) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                wg_barrier();
                read_next_a();
#pragma unroll
                for (int jj = 0; jj < JB; jj++) fb[jj] = ldB(C::NSRC, jj, C::NF);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i][j] = mfma(fb[j], fa[P][i], acc[i][j]);
            if (!(C::BAR && j < JB)) fb[j] = ldB(C::NSRC, j, C::NF);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    wg_barrier();  // stage 0 is in LDS
#pragma unroll
    for (int i = 0; i < 4; i++) fa[0][i] = ldA(0, i, 0);
#pragma unroll
    for (int j = 0; j < NB; j++) fb[j] = ldB(0, j, 0);
    int t = 0;
    for (; t + 2 <= S2; t += 2) {
        if (t + 5 < S2) prefetch(t + 4);
        kstep(WsStep<0, 0, 0, false, 0, 1>{});
        kstep(WsStep<1, 0, 1, false, 0, 2>{});
        kstep(WsStep<0, 0, 2, false, 0, 3>{});
        kstep(WsStep<1, 0, 3, true, 1, 0>{});
        kstep(WsStep<0, 1, 0, false, 1, 1>{});
        kstep(WsStep<1, 1, 1, false, 1, 2>{});
        kstep(WsStep<0, 1, 2, false, 1, 3>{});
        kstep(WsStep<1, 1, 3, true, 0, 0>{});
    }
    if (t < S2) {  // odd stage count: the last stage sits in buffer 0
        kstep(WsStep<0, 0, 0, false, 0, 1>{});
        kstep(WsStep<1, 0, 1, false, 0, 2>{});
        kstep(WsStep<0, 0, 2, false, 0, 3>{});
        kstep(WsStep<1, 0, 3, true, 1, 0>{});
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the prefetches
    ws_tile_to_lds<NB>(lds, acc, wm, wn, ln, lg);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wg_barrier();
}

template <int NB>
__global__ void __launch_bounds__(WS_NT) k_gemm_q8_0_ws(Ws8Args g) {
    constexpr int BN = 32 * NB;
    using L = Ws8Lds<NB>;
    __shared__ __attribute__((aligned(256))) char lds[L::TOTAL];
    _Float16 *const sA0 = (_Float16 *)(lds + L::A);
    _Float16 *const sB0 = (_Float16 *)(lds + L::B);
    auto sA = [&](int h) { return sA0 + h * (L::A_BYTES / 2); };
    auto sB = [&](int h) { return sB0 + h * (L::B_BYTES / 2); };
    const int b = blockIdx.x, x = b & 7, j8 = b >> 3, per = g.mt * g.parts;
    const int nt_i = x + 8 * (j8 / per), part = (j8 % per) / g.mt, mt_i = j8 % g.mt;
    if (nt_i >= g.nt) return;
    const int m0 = mt_i * WS_BM, n0 = nt_i * BN;
    // this part's stages s0 .. s0 + S2 - 1 of K / 128; operand bases moved to s0 (row strides stay
    // K and ldd), so the body below indexes stages from 0
    const int M = g.M, N = g.N, K = g.K, ST = K / WS_KS;
    const int s0 = part * ST / g.parts, S2 = (part + 1) * ST / g.parts - s0;
    const uint16_t *const Ab = g.A + (size_t)s0 * WS_KS;
    const uint8_t *const Qb = g.Q + (size_t)s0 * WS_KS;
    const uint16_t *const Db = g.D + (size_t)s0 * (WS_KS / 32);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const rsrc_t ra = make_rsrc(Ab, (uint32_t)((size_t)M * K * 2 - (size_t)s0 * WS_KS * 2));
    const rsrc_t rq = make_rsrc(Qb, (uint32_t)((size_t)N * K - (size_t)s0 * WS_KS));  // columns >= N read as zero

    if (wave >= 4) {
        // ------------------------------------------------------------------ producers
        // Stage s's activation tile (LDS DMA) and decoded B tile are made in stage s - 1; the quant
        // and scale loads of stage s + 3 are issued then too, one column's pair after each column's
        // decode. The end-of-stage wait covers the DMAs (issued first) and everything older.
        const int pw = __builtin_amdgcn_readfirstlane(wave - 4);
        const int pt = tid - 256, xi = pt & 7;
        const rsrc_t rd = make_rsrc(Db, (uint32_t)((size_t)N * g.ldd * 2 - (size_t)s0 * (WS_KS / 32) * 2));
        const int arow = 4 * pw + (lane >> 4);
        const uint32_t a_voff = (uint32_t)(((m0 + arow) * K + 8 * ((lane & 15) ^ (arow & 15))) * 2);
        auto dma_a = [&](int s, int qq) {
            dma16(ra, sA(s & 1) + (pw + 4 * qq) * 512, a_voff + (uint32_t)(qq * 16 * K * 2), (uint32_t)(s * WS_KS * 2));
        };
        uint32_t q_voff[NB], d_voff[NB];
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const uint32_t n = (uint32_t)(n0 + (pt >> 3) + 32 * i);
            q_voff[i] = n * (uint32_t)K + 16u * (uint32_t)xi;
            d_voff[i] = (n * (uint32_t)g.ldd + (uint32_t)(xi >> 1)) * 2u;
        }
        u4v Q[4][NB];
        uint32_t D[4][NB];
        auto load = [&](int set, int s, int i) {
            Q[set][i] = buf_load16(rq, q_voff[i], (uint32_t)(s * WS_KS));
            D[set][i] = __builtin_amdgcn_raw_buffer_load_b16(rd, d_voff[i], (uint32_t)(s * 8), 0);
        };
        const int slot0 = 2 * xi;
        auto decode = [&](auto setc, int s) {
            constexpr int SET = decltype(setc)::value;
            _Float16 *dst = sB(s & 1);
#pragma unroll
            for (int i = 0; i < NB; i++) {
                const uint32_t c = (uint32_t)((pt >> 3) + 32 * i), sg = c & 15u;
                const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)D[SET][i]);
                h8 lo, hi;
                decode16_q8_0(Q[SET][i], h2{dh, dh}, lo, hi);
                *(h8 *)(dst + c * WS_KS + 8 * ((uint32_t)slot0 ^ sg)) = lo;
                *(h8 *)(dst + c * WS_KS + 8 * ((uint32_t)(slot0 + 1) ^ sg)) = hi;
                if (s + 3 < S2) load((SET + 3) & 3, s + 3, i);
            }
        };
        auto end_stage = [&](bool loads_issued) {
            if (loads_issued) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(2 * NB) : "memory");
            else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
            wg_barrier();
        };
        using i0 = std::integral_constant<int, 0>;
        using i1 = std::integral_constant<int, 1>;
        using i2 = std::integral_constant<int, 2>;
        using i3 = std::integral_constant<int, 3>;
        // prologue: quants and scales of stages 0, 1, 2; stage 0's activation tile; decode stage 0
#pragma unroll
        for (int i = 0; i < NB; i++) load(0, 0, i);
#pragma unroll
        for (int i = 0; i < NB; i++) load(1, S2 > 1 ? 1 : 0, i);
#pragma unroll
        for (int i = 0; i < NB; i++) load(2, S2 > 2 ? 2 : 0, i);
#pragma unroll
        for (int k = 0; k < 8; k++) dma_a(0, k);
        decode(i0{}, 0);
        end_stage(3 < S2);
        // stage t (consumers on stage t): make stage t + 1 (register set (t + 1) % 4)
        auto step = [&](auto setc, int t) {
            const int s = t + 1;
            if (s < S2) {
#pragma unroll
                for (int k = 0; k < 8; k++) dma_a(s, k);
                decode(setc, s);
            }
            end_stage(s + 3 < S2);
        };
        int t = 0;
        for (; t + 4 <= S2; t += 4) {
            step(i1{}, t);
            step(i2{}, t + 1);
            step(i3{}, t + 2);
            step(i0{}, t + 3);
        }
        if (t < S2) step(i1{}, t++);
        if (t < S2) step(i2{}, t++);
        if (t < S2) step(i3{}, t++);
        wg_barrier();  // the consumers' output tile is in LDS
        tile_finish<WS_BM, 32 * NB, WS_NT, 4>(lds, g, m0, n0, nt_i * g.mt + mt_i, part, (int *)(lds + L::PF));
        return;
    }

    // ---------------------------------------------------------------------- consumers
    // L2 warm-up of the quants of stages s, s + 1 (one 128-byte line per column and stage; the mt
    // workgroups of an N-tile split the columns), as in k_gemm_q4_k_ws
    const int pf_cols = (BN - mt_i + g.mt - 1) / g.mt, pf_lanes = 2 * pf_cols;
    const uint32_t pf_lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds + L::PF) + 256u * (uint32_t)wave);
    auto prefetch = [&](int s) {
        for (int e0 = 64 * wave; e0 < pf_lanes; e0 += 256) {
            const int e = e0 + lane, jc = e >> 1;
            const int c = mt_i + g.mt * (e < pf_lanes ? jc : 0);
            const uint32_t voff = (uint32_t)(n0 + c) * (uint32_t)K + (uint32_t)(s + (e & 1)) * WS_KS;
            l2_touch(rq, voff, pf_lds);
        }
    };
    ws_plain_consumers<NB, L>(lds, wave, lane, S2, prefetch);
    tile_finish<WS_BM, 32 * NB, WS_NT, 4>(lds, g, m0, n0, nt_i * g.mt + mt_i, part, (int *)(lds + L::PF));
}

// ---------------------------------------------------------------------------------------------
// Q6_K, Q3_K and Q2_K tile kernel: the Q8_0 kernel's decomposition, roles and consumers, with producers
// that decode the k-quant super-blocks (device slots of hq_kquant.h / hq_q6k.hip). A 128-K stage is
// half h of a super-block; producer thread (column c = pt / 8 + 32 i, xi = pt % 8) takes the values
// 32 j + 8 lq .. + 7 of the stage for j = jp and jp + 2 (jp = xi / 4, lq = xi % 4): for both types
// these share the thread's quant bytes (Q6_K: low and high nibbles of the same ql bytes; Q3_K, Q2_K:
// bit pairs of the same qs bytes), and each 8 of them share one scale. Q6_K, Q3_K: B =
// fp16(q * fp16(d * s)): q exact, d * s exact in fp32 and rounded to fp16, then one rounding of the
// product (two roundings of the exact weight, each at most 2^-11 relative). Q2_K: B = fp16 of the
// fp32 weight (one rounding). The fp16 range bounds |w| < 65504, as for Q8_0.
//   Q6_K (:151-169)  q = (ql nibble | 2 bits of qh << 4) - 32, s = int8 scales[8h + 2j + l/16]
//   Q3_K (:112-134)  q = (2 bits of qs | hmask bit 4h + j << 2) - 4, s = 6-bit code 8h + 2j + l/16 - 32
//   Q2_K (:100-111)  q = 2 bits of qs, w = d (sm & 15) q - dmin (sm >> 4), sm = scales[8h + 2j + l/16]
struct KqwsArgs {
    const uint8_t *W;  // device slots, row n at n * row_bytes
    uint32_t row_bytes;
    const uint16_t *A;
    int M, N, K;
    void *C;
    int c_f32, accumulate;
    int mt, nt;
    int parts;  // K split as in WsArgs (ranges of whole super-blocks)
    float *partials;
    int *counters;
    int ntiles;
};

// one producer thread's loaded bytes of one column and stage
struct KqwsRaw {
    u2v q0, q1;  // Q6_K: ql, qh; Q3_K: qs, hmask (8 bytes each, the thread's l range)
    u4v sc;      // Q6_K: scales 8h .. 8h + 7, d; Q3_K: the 12 scale bytes and d
};

template <int T>
struct KqwsSrc {
    static_assert(T == HQ_TYPE_Q6_K || T == HQ_TYPE_Q3_K || T == HQ_TYPE_Q2_K, "k-quant tile kernel types");
    static constexpr int SLOT = T == HQ_TYPE_Q6_K ? 224 : T == HQ_TYPE_Q3_K ? 112 : 96;
    static constexpr int NLD = T == HQ_TYPE_Q6_K ? 4 : 3;  // loads per column and stage
    // vo = the column's row offset; so = the super-block's offset in the part's slots; h = half
    DEV void load(rsrc_t r, uint32_t vo, uint32_t so, int h, int jp, int lq, KqwsRaw &x) {
        if constexpr (T == HQ_TYPE_Q6_K) {
            x.q0 = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(r, vo + 32u * jp + 8u * lq, so + 64u * h, 0));
            x.q1 = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(r, vo + 128u + 8u * lq, so + 32u * h, 0));
            const u2v sc = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(r, vo + 192u, so + 8u * h, 0));
            x.sc = u4v{sc.x, sc.y, (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, vo + 208u, so, 0), 0u};
        } else if constexpr (T == HQ_TYPE_Q3_K) {
            x.q0 = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(r, vo + 32u + 8u * lq, so + 32u * h, 0));
            x.q1 = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(r, vo + 8u * lq, so, 0));
            x.sc = buf_load16(r, vo + 96u, so);
        } else {  // Q2_K: qs, scales 8h .. 8h + 7, {d, dmin}
            x.q0 = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(r, vo + 16u + 8u * lq, so + 32u * h, 0));
            x.q1 = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(r, vo, so + 8u * h, 0));
            x.sc = u4v{__builtin_amdgcn_raw_buffer_load_b32(r, vo + 80u, so, 0), 0u, 0u, 0u};
        }
    }
    // the 8 fp16 B values of j = jp + 2 t
    DEV h8 decode(const KqwsRaw &x, int h, int jp, int lq, int t) {
        const int j = jp + 2 * t;
        if constexpr (T == HQ_TYPE_Q2_K) {
            // w = (d * (sm & 15)) * q - dmin * (sm >> 4) in fp32 (the products exact, as in the
            // reference decoder), rounded once to fp16: a packed fp16 form would round both terms of a
            // difference that can cancel. Scale byte 2 j + (lq >> 1) of the half's 8: word j >> 1.
            const uint32_t sm = byte_of(j < 2 ? x.q1.x : x.q1.y, 2 * (j & 1) + (lq >> 1));
            const float ds = h2f((uint16_t)x.sc.x) * (float)(sm & 15u), dm = h2f((uint16_t)(x.sc.x >> 16)) * (float)(sm >> 4);
            h8 out;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t q = ((e < 4 ? x.q0.x : x.q0.y) >> (8 * (e & 3) + 2 * j)) & 3u;
                out[e] = (_Float16)__builtin_fmaf((float)q, ds, -dm);
            }
            return out;
        } else {
            uint32_t u[2];
            float d;
            int s;
            _Float16 bias;
            if constexpr (T == HQ_TYPE_Q6_K) {
#pragma unroll
                for (int w = 0; w < 2; w++) u[w] = ((x.q0[w] >> (4 * t)) & 0x0f0f0f0fu) | (((x.q1[w] >> (2 * j)) & 0x03030303u) << 4);
                const int e = 2 * j + (lq >> 1);  // scale byte of the half's 8
                s = (int)(int8_t)byte_of(e < 4 ? x.sc.x : x.sc.y, e & 3);
                d = h2f((uint16_t)x.sc.z);
                bias = (_Float16)1056.0f;  // 1024 + 32
            } else {
#pragma unroll
                for (int w = 0; w < 2; w++) u[w] = ((x.q0[w] >> (2 * j)) & 0x03030303u) | (((x.q1[w] >> (4 * h + j)) & 0x01010101u) << 2);
                const int e = 8 * h + 2 * j + (lq >> 1), g = e >> 2, i = e & 3;  // the 6-bit code, as q3k_code
                s = (int)(((byte_of(g & 1 ? x.sc.y : x.sc.x, i) >> (4 * (g >> 1))) & 15u) | (((byte_of(x.sc.z, i) >> (2 * g)) & 3u) << 4)) - 32;
                d = h2f((uint16_t)x.sc.w);
                bias = (_Float16)1028.0f;  // 1024 + 4
            }
            const _Float16 ds = (_Float16)(d * (float)s);
            const h2 kb = {bias, bias}, m2 = {ds, ds};
            h2 v[4];
#pragma unroll
            for (int w = 0; w < 2; w++) {
                v[2 * w] = (as_h2(perm_lo(u[w])) - kb) * m2;
                v[2 * w + 1] = (as_h2(perm_hi(u[w])) - kb) * m2;
            }
            return h8{v[0].x, v[0].y, v[1].x, v[1].y, v[2].x, v[2].y, v[3].x, v[3].y};
        }
    }
};

template <int T, int NB>
__global__ void __launch_bounds__(WS_NT) k_gemm_kq_ws(KqwsArgs g) {
    using Src = KqwsSrc<T>;
    constexpr int BN = 32 * NB, SLOT = Src::SLOT, NLD = Src::NLD;
    using L = Ws8Lds<NB>;
    __shared__ __attribute__((aligned(256))) char lds[L::TOTAL];
    _Float16 *const sA0 = (_Float16 *)(lds + L::A);
    _Float16 *const sB0 = (_Float16 *)(lds + L::B);
    auto sA = [&](int h) { return sA0 + h * (L::A_BYTES / 2); };
    auto sB = [&](int h) { return sB0 + h * (L::B_BYTES / 2); };
    const int b = blockIdx.x, x = b & 7, j8 = b >> 3, per = g.mt * g.parts;
    const int nt_i = x + 8 * (j8 / per), part = (j8 % per) / g.mt, mt_i = j8 % g.mt;
    if (nt_i >= g.nt) return;
    const int m0 = mt_i * WS_BM, n0 = nt_i * BN;
    // this part's super-blocks u0 .. u0 + U - 1 (stages 2 u0 .. ); operand bases moved to u0
    const int M = g.M, N = g.N, K = g.K, UT = K / 256;
    const int u0 = part * UT / g.parts, U = (part + 1) * UT / g.parts - u0, S2 = 2 * U;
    const uint16_t *const Ab = g.A + (size_t)u0 * 256;
    const uint8_t *const Wb = g.W + (size_t)u0 * SLOT;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const rsrc_t ra = make_rsrc(Ab, (uint32_t)((size_t)M * K * 2 - (size_t)u0 * 512));
    const rsrc_t rw = make_rsrc(Wb, (uint32_t)((size_t)N * g.row_bytes - (size_t)u0 * SLOT));  // rows >= N read as zero

    if (wave >= 4) {
        // ------------------------------------------------------------------ producers
        // as in k_gemm_q8_0_ws: stage s's activation tile and decoded B tile are made in stage s - 1,
        // the weight loads of stage s + 3 issued then too, one column's after each column's decode
        const int pw = __builtin_amdgcn_readfirstlane(wave - 4);
        const int pt = tid - 256, xi = pt & 7, jp = xi >> 2, lq = xi & 3;
        const int arow = 4 * pw + (lane >> 4);
        const uint32_t a_voff = (uint32_t)(((m0 + arow) * K + 8 * ((lane & 15) ^ (arow & 15))) * 2);
        auto dma_a = [&](int s, int qq) {
            dma16(ra, sA(s & 1) + (pw + 4 * qq) * 512, a_voff + (uint32_t)(qq * 16 * K * 2), (uint32_t)(s * WS_KS * 2));
        };
        uint32_t w_voff[NB];
#pragma unroll
        for (int i = 0; i < NB; i++) w_voff[i] = (uint32_t)(n0 + (pt >> 3) + 32 * i) * g.row_bytes;
        // NS register sets, loads AHEAD = NS - 1 stages before their decode (three sets for the wide
        // tiles: four would not fit the registers)
        constexpr int NS = NB >= 4 ? 3 : 4, AHEAD = NS - 1;
        KqwsRaw Q[NS][NB];
        auto load = [&](int set, int s, int i) {
            Src::load(rw, w_voff[i], (uint32_t)((s >> 1) * SLOT), s & 1, jp, lq, Q[set][i]);
        };
        auto decode = [&](auto setc, int s) {
            constexpr int SET = decltype(setc)::value;
            _Float16 *dst = sB(s & 1);
            const int h = s & 1;
#pragma unroll
            for (int i = 0; i < NB; i++) {
                const uint32_t c = (uint32_t)((pt >> 3) + 32 * i), sg = c & 15u;
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint32_t slot = (uint32_t)(4 * (jp + 2 * t) + lq);
                    *(h8 *)(dst + c * WS_KS + 8 * (slot ^ sg)) = Src::decode(Q[SET][i], h, jp, lq, t);
                }
                if (s + AHEAD < S2) load((SET + AHEAD) % NS, s + AHEAD, i);
            }
        };
        auto end_stage = [&](bool loads_issued) {
            if (loads_issued) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(NLD * NB) : "memory");
            else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
            wg_barrier();
        };
        using i0 = std::integral_constant<int, 0>;
        using i1 = std::integral_constant<int, 1>;
        using i2 = std::integral_constant<int, 2>;
        using i3 = std::integral_constant<int, 3>;
#pragma unroll
        for (int k = 0; k < AHEAD; k++)
#pragma unroll
            for (int i = 0; i < NB; i++) load(k, S2 > k ? k : 0, i);
#pragma unroll
        for (int k = 0; k < 8; k++) dma_a(0, k);
        decode(i0{}, 0);
        end_stage(AHEAD < S2);
        // stage t (consumers on stage t): make stage t + 1 from register set (t + 1) % NS
        auto step = [&](auto setc, int t) {
            const int s = t + 1;
            if (s < S2) {
#pragma unroll
                for (int k = 0; k < 8; k++) dma_a(s, k);
                decode(setc, s);
            }
            end_stage(s + AHEAD < S2);
        };
        int t = 0;
        if constexpr (NS == 4) {
            for (; t + 4 <= S2; t += 4) {
                step(i1{}, t);
                step(i2{}, t + 1);
                step(i3{}, t + 2);
                step(i0{}, t + 3);
            }
            if (t < S2) step(i1{}, t++);
            if (t < S2) step(i2{}, t++);
            if (t < S2) step(i3{}, t++);
        } else {
            for (; t + 3 <= S2; t += 3) {
                step(i1{}, t);
                step(i2{}, t + 1);
                step(i0{}, t + 2);
            }
            if (t < S2) step(i1{}, t++);
            if (t < S2) step(i2{}, t++);
        }
        wg_barrier();  // the consumers' output tile is in LDS
        tile_finish<WS_BM, BN, WS_NT, 4>(lds, g, m0, n0, nt_i * g.mt + mt_i, part, (int *)(lds + L::PF));
        return;
    }

    // ---------------------------------------------------------------------- consumers
    // L2 warm-up of super-block s / 2 of the tile's columns (bytes 0, SLOT / 2, SLOT - 1 of each
    // column's slot; the mt workgroups of an N-tile split the columns)
    const int pf_cols = (BN - mt_i + g.mt - 1) / g.mt, pf_lanes = 3 * pf_cols;
    const uint32_t pf_lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds + L::PF) + 256u * (uint32_t)wave);
    auto prefetch = [&](int s) {
        for (int e0 = 64 * wave; e0 < pf_lanes; e0 += 256) {
            const int e = e0 + lane, jc = e / 3, k = e - 3 * jc;
            const int c = mt_i + g.mt * (e < pf_lanes ? jc : 0);
            const uint32_t voff = (uint32_t)(n0 + c) * g.row_bytes + (uint32_t)(s >> 1) * SLOT +
                                  (k == 0 ? 0u : k == 1 ? (uint32_t)SLOT / 2 : (uint32_t)SLOT - 1);
            l2_touch(rw, voff, pf_lds);
        }
    };
    ws_plain_consumers<NB, L>(lds, wave, lane, S2, prefetch);
    tile_finish<WS_BM, BN, WS_NT, 4>(lds, g, m0, n0, nt_i * g.mt + mt_i, part, (int *)(lds + L::PF));
}
}  // namespace

// Tile width for the shape: the NB (BN = 32 NB columns, NB <= 5 for the LDS budget) with the least
// rounds-of-tiles x (NB + 1) (a tile's time grows with its width plus a per-tile share of fixed
// costs: narrow tiles reuse each activation fragment fewer times); the fraction of CU time doing
// useful work is returned in *eff.
int hq_ws_choose(int M, int N, int n_cu, float *eff) {
    const int mt = (M + WS_BM - 1) / WS_BM;
    int best = 5;
    double best_cost = 1e30, best_eff = 0.0;
    for (int nb = 5; nb >= 2; nb--) {
        const int nt = (N + 32 * nb - 1) / (32 * nb);
        const long tiles = (long)mt * nt, rounds = (tiles + n_cu - 1) / n_cu;
        const double cost = (double)rounds * (nb + 1);
        if (cost < best_cost - 1e-9) {
            best_cost = cost;
            best = nb;
            best_eff = (double)M * N / ((double)rounds * n_cu * WS_BM * 32.0 * nb);
        }
    }
    if (eff) *eff = (float)best_eff;
    return best;
}

hipError_t hq_launch_gemm_ws(const hq_dev_mat *W, const uint16_t *A, const uint16_t *S, int M, void *C, int c_f32,
                             int accumulate, int nb, int parts, float *partials, int *counters, hipStream_t st) {
    if (W->type == HQ_TYPE_Q5_K && !S) return hipErrorInvalidValue;
    WsArgs g;
    g.W = W->qs, g.row_bytes = (uint32_t)W->row_bytes, g.A = A, g.S = S;
    g.M = M, g.N = (int)W->rows, g.K = (int)W->cols, g.C = C, g.c_f32 = c_f32, g.accumulate = accumulate;
    g.mt = (M + WS_BM - 1) / WS_BM;
    g.nt = (g.N + 32 * nb - 1) / (32 * nb);
    g.parts = parts, g.partials = partials, g.counters = counters, g.ntiles = g.mt * g.nt;
    if (parts < 1 || parts > 4 || parts > g.K / 256 || (parts > 1 && (!partials || !counters))) return hipErrorInvalidValue;
    if (parts > 1 && (size_t)g.mt * g.nt * parts * WS_BM * 32 * nb * 4 >= ((size_t)1 << 32)) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)(8 * ((g.nt + 7) / 8) * g.mt * parts);
    const bool q5 = W->type == HQ_TYPE_Q5_K;
    if (!q5 && W->type != HQ_TYPE_Q4_K) return hipErrorInvalidValue;
#define WSQ(nbv)                                                 \
    if (q5) k_gemm_q5_k_ws<nbv><<<grid, WS_NT, 0, st>>>(g);      \
    else k_gemm_q4_k_ws<nbv><<<grid, WS_NT, 0, st>>>(g);
    switch (nb) {
    case 2: WSQ(2) break;
    case 3: WSQ(3) break;
    case 4: WSQ(4) break;
    case 5: WSQ(5) break;
    default: return hipErrorInvalidValue;
    }
#undef WSQ
    return hipGetLastError();
}

hipError_t hq_launch_gemm_ws8(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                              int nb, int parts, float *partials, int *counters, hipStream_t st) {
    if (W->cols % WS_KS) return hipErrorInvalidValue;
    Ws8Args g;
    g.Q = W->qs, g.D = W->d, g.ldd = W->ldd, g.A = A;
    g.M = M, g.N = (int)W->rows, g.K = (int)W->cols, g.C = C, g.c_f32 = c_f32, g.accumulate = accumulate;
    g.mt = (M + WS_BM - 1) / WS_BM;
    g.nt = (g.N + 32 * nb - 1) / (32 * nb);
    g.parts = parts, g.partials = partials, g.counters = counters, g.ntiles = g.mt * g.nt;
    if (parts < 1 || parts > 4 || parts > g.K / WS_KS || (parts > 1 && (!partials || !counters))) return hipErrorInvalidValue;
    if (parts > 1 && (size_t)g.mt * g.nt * parts * WS_BM * 32 * nb * 4 >= ((size_t)1 << 32)) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)(8 * ((g.nt + 7) / 8) * g.mt * parts);
    switch (nb) {
    case 2: k_gemm_q8_0_ws<2><<<grid, WS_NT, 0, st>>>(g); break;
    case 3: k_gemm_q8_0_ws<3><<<grid, WS_NT, 0, st>>>(g); break;
    case 4: k_gemm_q8_0_ws<4><<<grid, WS_NT, 0, st>>>(g); break;
    case 5: k_gemm_q8_0_ws<5><<<grid, WS_NT, 0, st>>>(g); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t hq_launch_gemm_kqws(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                               int nb, int parts, float *partials, int *counters, hipStream_t st) {
    if ((W->type != HQ_TYPE_Q6_K && W->type != HQ_TYPE_Q3_K && W->type != HQ_TYPE_Q2_K) || W->cols % 256 || !hq_kqws_fits(W, M))
        return hipErrorInvalidValue;
    KqwsArgs g;
    g.W = W->qs, g.row_bytes = (uint32_t)W->row_bytes, g.A = A;
    g.M = M, g.N = (int)W->rows, g.K = (int)W->cols, g.C = C, g.c_f32 = c_f32, g.accumulate = accumulate;
    g.mt = (M + WS_BM - 1) / WS_BM;
    g.nt = (g.N + 32 * nb - 1) / (32 * nb);
    g.parts = parts, g.partials = partials, g.counters = counters, g.ntiles = g.mt * g.nt;
    if (parts < 1 || parts > 4 || parts > g.K / 256 || (parts > 1 && (!partials || !counters))) return hipErrorInvalidValue;
    if (parts > 1 && (size_t)g.mt * g.nt * parts * WS_BM * 32 * nb * 4 >= ((size_t)1 << 32)) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)(8 * ((g.nt + 7) / 8) * g.mt * parts);
#define KQWS(t)                                                                          \
    switch (nb) {                                                                        \
    case 2: k_gemm_kq_ws<t, 2><<<grid, WS_NT, 0, st>>>(g); break;                        \
    case 3: k_gemm_kq_ws<t, 3><<<grid, WS_NT, 0, st>>>(g); break;                        \
    case 4: k_gemm_kq_ws<t, 4><<<grid, WS_NT, 0, st>>>(g); break;                        \
    case 5: k_gemm_kq_ws<t, 5><<<grid, WS_NT, 0, st>>>(g); break;                        \
    default: return hipErrorInvalidValue;                                                \
    }
    if (W->type == HQ_TYPE_Q6_K) {
        KQWS(HQ_TYPE_Q6_K)
    } else if (W->type == HQ_TYPE_Q3_K) {
        KQWS(HQ_TYPE_Q3_K)
    } else {
        KQWS(HQ_TYPE_Q2_K)
    }
#undef KQWS
    return hipGetLastError();
}

// every byte offset of k_gemm_kq_ws fits 32 bits (tile rows and columns past the matrix included)
int hq_kqws_fits(const hq_dev_mat *W, int M) {
    const size_t lim = (size_t)1 << 32;
    return (W->type == HQ_TYPE_Q6_K || W->type == HQ_TYPE_Q3_K || W->type == HQ_TYPE_Q2_K) && W->cols % 256 == 0 && M >= 1 &&
           ((size_t)M + WS_BM) * W->cols * 2 < lim && ((size_t)W->rows + 160) * W->row_bytes < lim;
}
