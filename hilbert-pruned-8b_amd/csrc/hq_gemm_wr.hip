// hq_gemm_wr.hip - Q4_K GEMM for prefill shapes of one tile round (M = 128 .. ~512 at N ~ 10k; with
// each tile's K split over workgroups for few tiles over a long K, k_gemm_q4_k_wr_ks; the gate/up pair
// GEMM with the SwiGLU epilogue) on gfx950: 128 x 64NB output tiles; 4 MFMA waves that each own all
// 128 rows and 16NB columns, and 4 loader waves.
//
// C[M,N] (+)= A[M,K] . W^T with A fp16 and W GGUF Q4_K super-blocks resident in HBM (reference
// arithmetic: cleanroom-transformer/src/ggml_quant.h:51-59, :135-150; matmul src/cpu_backend.c:38-54).
//
// Why this shape. Measured on gfx950 (one CU): an MFMA 16x16x32 takes 16 clocks and two independent
// VALU instructions issued behind it in the same wave cost nothing (each one more costs ~4 clocks);
// LDS reads run at 256 bytes per clock but ds_write_b128 at ~64. A Q4_K weight fragment (16 columns
// x 32 k) costs 10 VALU instructions to decode, so it has to feed 8 row blocks (128 rows) to stay
// inside that budget: each MFMA wave decodes, in registers, only its own 16NB columns and uses them
// against all 128 rows of the tile (no decode is repeated, no decoded weight goes through LDS). The
// activation tile is the only operand shared through LDS. An LDS DMA instruction holds its wave until
// the address unit takes it (~20-25 clocks per 1 KB per CU, ~30 per stage here), which would idle the
// MFMA pipe of a multiplying wave: the loads are issued by the loader waves, one beside each MFMA wave
// on its SIMD. M = 512, N = 9728: 4 x 51 tiles of 128 x 192 on 256 CUs, one round.
//
// Pipeline. K is walked in stages of 64 (one 32-byte quant group p of a super-block u). Per stage an
// MFMA wave runs 16 groups of NB MFMAs (group g: k-step g / 8, row block g % 8), each closed by a
// scheduling barrier, and spreads the rest of its work over the groups so that it issues while the
// MFMAs run: the activation read of the group three ahead, half a weight fragment's decode per group
// (k-step 1 in groups 0 .. 5, the next stage's k-step 0 in groups 9 .. 14; each pinned to its group,
// the loop body has no branches for the compiler to sink work across). The 8 waves meet at one
// s_barrier per stage, in group 6; after it the loaders fill ring slot s + 2 (4 stages of activations
// and quants; each load has two stages to land) and the MFMA waves read the next stage's quant words.
//
// Arithmetic: as hq_gemm_ws.hip and hq_gemm_bt.hip (accumulators in units of c_u = d_u, weight operand
// the exact integer s*q). The row blocks are rescaled by c_u / c_{u+1} right after their last MFMA of
// super-block u; at the end by c_{U-1}. The min term of super-block u (bf16 hi/lo S x Bmin) is added
// one super-block late, in stage p = 1 of super-block u + 1 and in its units (x = -dmin*m/c_{u+1}),
// each row block four groups away from its own MFMAs; the last super-block's after the loop, in its
// own units. The activation sub-block sums S come from the loader waves: each stage's ring slot is
// summed in LDS while the stage is being multiplied (no pass over A before the kernel), so S of
// super-block u is whole one barrier after its last stage. The per-column tables (scale words, Bmin,
// F = c_u / c_{u+1}, CN = c_{u+1}) depend on the weights only: they are computed once at upload
// (k_q4k_tables) and moved into LDS with the loads.
//
// LDS (111 KB for NB = 3): A [4][128 rows][64 k] fp16 (16-byte slot p of row r at p ^ ((r >> 1) & 7));
// quant groups [4][64NB columns][32 B] (the two halves of column c swapped where (c >> 3) & 1);
// S [2][128][hi x 8, lo x 8] bf16; the tile's Bmin [64NB][32 B] and records [3][64NB][16 B]. The
// output goes from the accumulators straight to C.
#include "hq_device.h"
#include "hq_kernels.h"

namespace {
constexpr int WR_BM = 128, WR_KS = 64, WR_NT = 512, WR_RING = 4;
// activation operand read-ahead in groups (< WR_AF; reads of the next stage start after its barrier)
// and the ring they land in: 7 of 8 takes the 128-row tile kernel to 220 VGPRs (two waves per SIMD
// still) and saved 2 % at M = 512, N = 9728, K = 2560 against 3 of 4 in a same-box A/B
#ifndef WR_AD
#define WR_AD 7
#endif
#ifndef WR_AFN
#define WR_AFN 8
#endif
constexpr int WR_AF = WR_AFN;
static_assert(WR_AD < WR_AF && 16 - WR_AD > 6 && 16 % WR_AF == 0, "activation read-ahead");

struct WrArgs {
    const uint8_t *W;  // Q4_K super-blocks, row n at n * row_bytes
    uint32_t row_bytes;
    const uint16_t *A;  // fp16 [M][K]
    const uint8_t *tab; // per-super-block column tables (hq_launch_q4k_tables)
    int M, N, K;
    void *C;
    int c_f32, accumulate;
    int mt, nt0, nt;  // M-tiles; this launch's column tiles nt0 .. nt - 1
    // K split: each tile's super-blocks cut into `parts` contiguous ranges, one workgroup each, whose
    // fp32 tiles meet in partials (tile_finish: the last to arrive adds them in part order); 1: whole K
    int parts;
    float *partials;
    int *counters;
    int ntiles;  // mt * nt (the counter and partial-tile index range)
};

// Tile geometry. TW = 192: MFMA wave w owns column blocks 3w .. 3w + 2 for all 8 row blocks. TW = 160
// (10 column blocks; 4 x 61 = 244 tiles at N = 9728 instead of 4 x 51 = 204 of 192 columns): wave w owns
// blocks 2w and 2w + 1 for all rows and the half (row blocks 4h .. 4h + 3, h = w % 2) of block
// 8 + w / 2, so every wave issues the same 40 MFMAs per stage (48 at TW = 192).
template <int TW>
struct WrGeo {
    static_assert(TW == 192 || TW == 160, "tile width");
    static constexpr bool SPLIT = TW == 160;
    static constexpr int BN = TW, QK = TW / 32;  // quant (and Bmin) DMA instructions: 32 columns each
    static constexpr int RC = 192;               // record slot width in columns (TW = 160 over-fetches)
    // column block of the wave's operand j, and whether it covers processing row i (TW = 160 rotates
    // a wave's row blocks by 4 h, so its half block is always processing rows 0 .. 3)
    DEV int cb(int w, int j) { return SPLIT ? (j < 2 ? 2 * w + j : 8 + (w >> 1)) : 3 * w + j; }
    static constexpr bool has(int i, int j) { return !SPLIT || j < 2 || i < 4; }
};

// (the tables first: their reads then take their constant offsets in the instruction's 16-bit offset
// field; the activation ring's reads do from their own base)
template <int TW>
struct WrLds {
    static constexpr int BN = TW;
    static constexpr int T_REC = 0;                                       // column tables: records [3][192][16 B],
    static constexpr int T_BM = T_REC + 3 * WrGeo<TW>::RC * 16;           // Bmin [BN][32 B]
    static constexpr int S = T_BM + BN * 32, S_BYTES = WR_BM * 32;        // sub-block sums, per parity
    static constexpr int Q = S + 2 * S_BYTES, Q_BYTES = BN * 32;          // quant groups per ring slot
    static constexpr int A = Q + WR_RING * Q_BYTES, A_BYTES = WR_BM * WR_KS * 2;  // activations per ring slot
    static constexpr int TOTAL = A + WR_RING * A_BYTES;
    static_assert(TOTAL <= 160 * 1024, "LDS budget");
    static_assert(T_BM + BN * 32 <= 65536, "table offsets in the offset field");
};

DEV void wr_barrier() { asm volatile("s_barrier" ::: "memory"); }
// a loader wave's wait before a barrier: every LDS DMA but the last n issued, and its LDS stores
template <int n>
DEV void wr_wait() { asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(n) : "memory"); }
// keeps a computed operand in the group that computes it (the compiler would otherwise sink the work
// to the operand's first use)
DEV void wr_pin(h8 &x) { asm volatile("" : "+v"(x)); }
// half hf of a weight operand (decode8m's values 4hf .. 4hf + 3, from quant word hf), in place
DEV void wr_dec_half(h8 &b, u2v q, int hf, uint32_t mask, h2 mul, h2 add) {
    const uint32_t w = (hf ? q.y : q.x) & mask;
    const h2 v0 = __builtin_elementwise_fma(as_h2(perm_lo(w)), mul, add);
    const h2 v1 = __builtin_elementwise_fma(as_h2(perm_hi(w)), mul, add);
    b[4 * hf] = v0.x, b[4 * hf + 1] = v0.y, b[4 * hf + 2] = v1.x, b[4 * hf + 3] = v1.y;
    wr_pin(b);
}


// whether the tile kernels store their output staged in LDS: fp16 C (tile_store_ok) or the SwiGLU
// output of a pair matrix (C 16-byte aligned; N is a multiple of 16); the SwiGLU pair GEMM at
// M = 512, I = 9728, K = 2560 measured 2-3 us faster so in same-box A/Bs
DEV bool wr_staged(const WrArgs &g) {
    return tile_store_ok(g.c_f32, g.accumulate, g.N, g.C) || (g.c_f32 == HQ_OUT_SWIGLU && ((uintptr_t)g.C & 15u) == 0);
}
// the store phase of an output tile staged in LDS (tile_store_rows): fp16 C [M][N], or the SwiGLU
// output fp16 [M][N / 2] (the tile's BN / 2 output columns from n0 / 2)
template <int BN>
DEV void wr_store(const char *lds, const WrArgs &g, int m0, int n0, int tid) {
    const int rows = min(WR_BM, g.M - m0), cols = min(BN, g.N - n0);
    if (g.c_f32 == HQ_OUT_SWIGLU) {
        const uint32_t pitch = (uint32_t)g.N;
        tile_store_rows<WR_BM, WR_NT, BN>(lds, (char *)g.C + (size_t)m0 * pitch, rows, pitch, (uint32_t)n0, (uint32_t)cols, tid);
    } else {
        const uint32_t pitch = (uint32_t)g.N * 2u;
        tile_store_rows<WR_BM, WR_NT, BN * 2>(lds, (char *)g.C + (size_t)m0 * pitch, rows, pitch, (uint32_t)n0 * 2u, (uint32_t)cols * 2u, tid);
    }
}

// The tile body; KS: with the K split (parts > 1; the split-only work is compiled out of the whole-K
// kernels, which are the headline's); TW: the tile width (192 or 160 columns)
template <bool KS, int TW>
DEV void wr_tile(const WrArgs &g) {
    using L = WrLds<TW>;
    using G = WrGeo<TW>;
    constexpr int NB = 3, BN = L::BN;
    static_assert(WR_BM * tile_ldr<BN * 2>() <= L::TOTAL && WR_BM * (BN + 4) * 4 <= L::TOTAL - 16, "output tile in LDS");
    __shared__ __attribute__((aligned(256))) char lds[L::TOTAL];
    // tile and K part: XCD x = b % 8 takes column units x, x + 8, ... (unit = N-tile x parts + part);
    // its slots run over the M-tiles of one unit first (the unit's weight slab is then fetched once
    // per XCD)
    const int b = blockIdx.x, x = b & 7, j8 = b >> 3;
    const int parts = KS ? g.parts : 1;
    const int cu = g.nt0 * parts + x + 8 * (j8 / g.mt), mt_i = j8 % g.mt;
    const int nt_i = KS ? cu / parts : cu, part = KS ? cu - nt_i * parts : 0;
    if (nt_i >= g.nt) return;
    const int m0 = mt_i * WR_BM, n0 = nt_i * BN;
    const int M = g.M, N = g.N, K = g.K, Ut = K / 256;
    // this part's super-blocks u0 .. u0 + U - 1: the operand bases move to u0 (row strides stay), so
    // the body below counts super-blocks and stages from 0 (the column tables are global: F and c of
    // a part's last super-block look at the next part's first)
    const int u0 = KS ? part * Ut / parts : 0, U = KS ? (part + 1) * Ut / parts - u0 : Ut, S2 = 4 * U;
    const uint16_t *const Ab = g.A + (size_t)u0 * 256;
    const uint8_t *const Wb = g.W + (size_t)u0 * 144;
    const uint8_t *const Tb = g.tab + (size_t)u0 * N * HQ_Q4K_TAB_BYTES;
    // (the wave index through readfirstlane: the role and every LDS DMA address derived from it are
    // then scalar values, not per-lane ones read back with a VALU instruction per DMA)
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, ln = lane & 15,
              lg = lane >> 4;
    // roles: waves 0-3 multiply (wave w: columns 16NB w .. of the tile, all 128 rows); waves 4-7 load
    // (wave 4 + w: a quarter of the activation tile and of its sub-block sums, and a share of the quant
    // groups and column tables)
    const int role = wave >> 2, w4 = wave & 3;
    const rsrc_t ra = make_rsrc(Ab, (uint32_t)((size_t)M * K * 2 - (size_t)u0 * 512));
    const rsrc_t rw = make_rsrc(Wb, (uint32_t)((size_t)N * g.row_bytes - (size_t)u0 * 144));
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
    // tile-relative first column of the wave's operand j; TW = 160: the wave's row blocks are processed
    // rotated by 4 hr (processing row i is row block (i + 4 hr) % 8), so its half block's rows come first
    int c0[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) c0[j] = 16 * G::cb(w4, j);
    const int hr = G::SPLIT ? (w4 & 1) : 0;
    auto rb_of = [&](int i) { return (i + 4 * hr) & 7; };  // row block of processing row i

    // ---- loads. A buffer load checks only its VGPR offset against the buffer's size (the scalar offset
    // is not range-checked), so every row and column index is in the VGPR offset: rows past M and
    // columns past N read zeros, and no load reads past the end of A or W.
    // Activation DMA of stage s into ring slot buf: instruction q (0..3) of wave w fills rows
    // 8(4w + q) .. + 8; lane i: row r = 8(4w + q) + i/8, LDS slot i % 8, global chunk
    // (i % 8) ^ ((r >> 1) & 7) (the q = 0 chunk ^ 4 for odd q)
    const int a_row0 = 32 * w4 + (lane >> 3);
    const uint32_t a_ch = (uint32_t)((lane & 7) ^ ((a_row0 >> 1) & 7));
    uint32_t a_voff[4];
#pragma unroll
    for (int q = 0; q < 4; q++) a_voff[q] = (uint32_t)(m0 + a_row0 + 8 * q) * (uint32_t)K * 2u + 16u * (q & 1 ? a_ch ^ 4u : a_ch);
    auto dma_a1 = [&](int s, int buf, int q) {
        dma16_so(ra, lds0 + (uint32_t)(L::A + buf * L::A_BYTES + w4 * 4096 + q * 1024), a_voff[q], (uint32_t)(s * WR_KS * 2));
    };
    // quant DMA of stage s, 32 of the tile's 192 columns per instruction: instruction k (wave w issues
    // k = w, and k = 4 + w for w < 2), lane i: column c = 32k + i/2, LDS half i % 2 of the column's 32
    // bytes, holding the group's half (i % 2) ^ ((c >> 3) & 1)
    constexpr int QK = G::QK;
    const int qw = w4 + 4 < QK ? 2 : 1;  // this wave's quant DMAs per stage
    uint32_t q_voff[2];
#pragma unroll
    for (int t = 0; t < 2; t++)
        q_voff[t] = (uint32_t)(n0 + 32 * (w4 + 4 * t) + (lane >> 1)) * g.row_bytes + 16u * (uint32_t)((lane & 1) ^ ((lane >> 4) & 1));
    auto dma_q1 = [&](int s, int buf, int t) {
        const uint32_t dst = lds0 + (uint32_t)(L::Q + buf * L::Q_BYTES + (w4 + 4 * t) * 1024);
        dma16_so(rw, dst, q_voff[t], (uint32_t)((s >> 2) * 144 + 16 + 32 * (s & 3)));
    };
    // activation sub-block sums of stage s (sub-blocks 2p, 2p + 1 of super-block u; s = 4u + p) from
    // its ring slot into S parity u & 1, on the matrix core (one VALU instruction on this SIMD costs
    // the MFMA wave beside it as much as a quarter of an MFMA): loader wave w sums rows 32w + 16b + i
    // (b = 0, 1) with two MFMAs per row block, activations as the B operand and a 0/1 A operand whose
    // rows 0-7 select the stage's first sub-block and rows 8-15 the second. Lane (i, q) then holds the
    // fp32 sum of row 32w + 16b + i, sub-block 2p + h for b = q & 1, h = q >> 1 (exact products, fp32
    // sums) and stores its bf16 hi and lo parts
    const int s_b = lg & 1, s_h = lg >> 1;
    uint32_t s_src[2][2];
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int row = 32 * w4 + 16 * b + ln;
            s_src[b][h] = lds0 + (uint32_t)(L::A + row * 128) + 16u * ((uint32_t)(4 * h + lg) ^ (uint32_t)((row >> 1) & 7));
        }
    const uint32_t s_dst = lds0 + (uint32_t)(L::S + (32 * w4 + 16 * s_b + ln) * 32 + 2 * s_h);
    const _Float16 one_lo = (_Float16)(ln < 8 ? 1.0f : 0.0f), one_hi = (_Float16)(ln < 8 ? 0.0f : 1.0f);
    const h8 sel0 = {one_lo, one_lo, one_lo, one_lo, one_lo, one_lo, one_lo, one_lo};
    const h8 sel1 = {one_hi, one_hi, one_hi, one_hi, one_hi, one_hi, one_hi, one_hi};
    auto sums = [&](int s) {
        using lds_h8 = const __attribute__((address_space(3))) h8;
        const uint32_t so = (uint32_t)((s & 3) * L::A_BYTES);
        f4 c[2];
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const h8 x0 = *(lds_h8 *)(uintptr_t)(s_src[b][0] + so), x1 = *(lds_h8 *)(uintptr_t)(s_src[b][1] + so);
            c[b] = mfma(sel1, x1, mfma(sel0, x0, f4{0.f, 0.f, 0.f, 0.f}));
        }
        const float v = s_b ? c[1][0] : c[0][0];
        const __bf16 hi = (__bf16)v, lo = (__bf16)(v - (float)hi);
        using lds_u16 = __attribute__((address_space(3))) uint16_t;
        const uint32_t d = s_dst + (uint32_t)(((s >> 2) & 1) * L::S_BYTES + 4 * (s & 3));
        *(lds_u16 *)(uintptr_t)d = __builtin_bit_cast(uint16_t, hi);
        *(lds_u16 *)(uintptr_t)(d + 16) = __builtin_bit_cast(uint16_t, lo);
    };
    // column tables of the tile, 1 KB per instruction: Bmin of super-block u, instruction k (0 .. QK - 1):
    // columns 32k .. + 32; the records of super-block u in record slot u % 3 (they stay until the
    // super-block's rescale and the tile's end read them, two super-blocks after the next one's
    // loads), instruction k (0..2): columns 64k .. + 64 (for TW = 160 the last 32 are the next tile's,
    // never read). The loader waves with one quant DMA per stage issue them. Past column N these read
    // other table bytes (the upload leaves HQ_Q4K_TAB_PAD zero bytes after the tables for the last
    // tile's), used only for outputs that are not stored
    const rsrc_t rt = make_rsrc(Tb, (uint32_t)((size_t)N * U * HQ_Q4K_TAB_BYTES));
    auto dma_bm = [&](int u, int k) {
        dma16_so(rt, lds0 + (uint32_t)(L::T_BM + 1024 * k), 16u * (uint32_t)lane,
                 (uint32_t)u * (uint32_t)N * HQ_Q4K_TAB_BYTES + (uint32_t)(n0 + 32 * k) * 32u);
    };
    auto dma_rec = [&](int u, int slot, int k) {
        dma16_so(rt, lds0 + (uint32_t)(L::T_REC + slot * G::RC * 16 + 1024 * k), 16u * (uint32_t)lane,
                 (uint32_t)u * (uint32_t)N * HQ_Q4K_TAB_BYTES + (uint32_t)N * 32u + (uint32_t)(n0 + 64 * k) * 16u);
    };

    // ---- operand addresses. Activation fragment of row block i, k-step f, ring slot buf: lane (ln, lg)
    // reads row 16i + ln, slot (4f + lg) ^ ((ln >> 1) & 7)
    // (processing rows 0 .. 3 and 4 .. 7 have their own bases, which differ by the rotation)
    const uint32_t a_lane = lds0 + (uint32_t)(L::A + ln * 128) + 16u * ((uint32_t)lg ^ (uint32_t)((ln >> 1) & 7));
    const uint32_t a_lo = a_lane + (uint32_t)(4 * hr * 16 * 128), a_hi = a_lane - (uint32_t)(4 * hr * 16 * 128);
    auto rd = [&](int buf, int gg) {
        return *(const __attribute__((address_space(3))) h8 *)(uintptr_t)(((((gg & 7) < 4 ? a_lo : a_hi) ^ (64u * (uint32_t)(gg >> 3))) +
                                                                           (uint32_t)(buf * L::A_BYTES)) +
                                                                          (uint32_t)((gg & 7) * 16 * 128));
    };
    // quant words of operand j (column c0[j] + ln of the tile, bytes 8lg .. + 7 of the group)
    uint32_t q_lane[NB];
#pragma unroll
    for (int j = 0; j < NB; j++)
        q_lane[j] = lds0 + (uint32_t)(L::Q + (c0[j] + ln) * 32 + 16 * ((lg >> 1) ^ ((ln >> 3) & 1)) + 8 * (lg & 1));
    auto rdq = [&](int buf, int j) {
        return *(const __attribute__((address_space(3))) u2v *)(uintptr_t)(q_lane[j] + (uint32_t)(buf * L::Q_BYTES));
    };
    // the scales of sub-blocks 2p, 2p + 1 of operand j in record slot v (16 bits of scale word p / 2,
    // read as such: no shift, which the compiler would place right behind the read and wait for)
    auto rdsw = [&](int p, int v, int j) {
        return (uint32_t) * (const __attribute__((address_space(3))) uint16_t *)(uintptr_t)(lds0 + (uint32_t)(L::T_REC + (v * G::RC + c0[j] + ln) * 16 +
                                                                                                             (p >> 1) * 4 + (p & 1) * 2));
    };
    const uint32_t s_lane = lds0 + (uint32_t)(L::S + ln * 32 + 16 * (lg & 1));
    const uint32_t s_lo = s_lane + (uint32_t)(4 * hr * 16 * 32), s_hi = s_lane - (uint32_t)(4 * hr * 16 * 32);
    auto rds = [&](int par, int i) {  // processing row i
        return *(const __attribute__((address_space(3))) h8 *)(uintptr_t)((i < 4 ? s_lo : s_hi) + (uint32_t)(par * L::S_BYTES + i * 16 * 32));
    };
    auto rdbm = [&](int j) {
        return *(const __attribute__((address_space(3))) h8 *)(uintptr_t)(lds0 + (uint32_t)(L::T_BM + (c0[j] + ln) * 32 + 16 * (lg >> 1)));
    };
    // field f (2: F, 3: CN) of the records of columns c0[j] + 4lg .. + 3 in record slot v
    auto rdr = [&](int j, int v, int f) {
        f4 r;
#pragma unroll
        for (int c = 0; c < 4; c++)
            r[c] = *(const __attribute__((address_space(3))) float *)(uintptr_t)(lds0 + (uint32_t)(L::T_REC + (v * G::RC + c0[j] + 4 * lg + c) * 16 + 4 * f));
        return r;
    };

    f4 acc[8][NB];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    // decode scales of stage p: (s_lo, s_hi) of sub-blocks 2p, 2p + 1 -> multipliers (s_lo, s_hi / 16)
    // and addends (-1024 s_lo, -64 s_hi) for the low (x) and high (y) nibbles: the scales as the fp16
    // (1024 + s), then one fma for both multipliers ((1024 + s) / 16 - 64 = s / 16, exact) and one
    // product for both addends
    auto scales = [&](uint32_t w, h2 &mu, h2 &ad) {
        const h2 x = as_h2(__builtin_amdgcn_perm(0x64646464u, w, 0x04010400u));
        mu = __builtin_elementwise_fma(x, h2{(_Float16)1.0f, (_Float16)0.0625f}, h2{(_Float16)-1024.0f, (_Float16)-64.0f});
        ad = mu * h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
    };

    const int u_last = U - 1;
    if (role == 1) {
        // ------------------------------------------------------------------------------ loaders
        // prologue: stage 0 of activations and quants, the records of unit 0, then stage 1, which (as
        // in every loader stage) is still in flight at the barrier. S parity 1 is zeroed: the min step
        // of unit 0 (the late one of unit -1, with Bmin zero in the MFMA waves' registers) adds zeros
#pragma unroll
        for (int q = 0; q < 4; q++) dma_a1(0, 0, q);
        dma_q1(0, 0, 0);
        if (qw == 2) dma_q1(0, 0, 1);
        if constexpr (G::SPLIT) {
            if (w4 >= 1) dma_rec(0, 0, w4 - 1);
        } else {
            if (w4 == 2) dma_rec(0, 0, 0), dma_rec(0, 0, 2);
            if (w4 == 3) dma_rec(0, 0, 1);
        }
        *(__attribute__((address_space(3))) u4v *)(uintptr_t)(lds0 + (uint32_t)(L::S + L::S_BYTES + w4 * 1024 + 16 * lane)) =
            u4v{0u, 0u, 0u, 0u};
        {
            const int s1 = S2 > 1 ? 1 : 0;
#pragma unroll
            for (int q = 0; q < 4; q++) dma_a1(s1, 1, q);
            dma_q1(s1, 1, 0);
            if (qw == 2) dma_q1(s1, 1, 1);
        }
        if (qw == 2) wr_wait<6>();
        else wr_wait<5>();
        wr_barrier();
        // loader stage s = 4u + p runs between the MFMA waves' barriers of stages s - 1 and s (the
        // prologue's barrier counts as stage -1's), while they finish stage s - 1 and start stage s:
        // the loads of stage s + 2 (ring slot (s + 2) % 4, last read in stage s - 2); the records of
        // unit u + 1 at p = 0, 1 (parity (u + 1) & 1: unit u - 1's were last read in stage 4u - 2) and
        // Bmin of unit u at p = 1, 2 (unit u - 1's was read in stage 4u - 1, it is read in stage 4u + 3);
        // the sums of stage s (landed by the last barrier); then wait for everything but this stage's
        // loads (stage s + 1's land: each load has two stages) and for the sums' stores, and meet the
        // MFMA waves at their barrier. Per stage a loader wave issues 4 activation DMAs, 2 (waves 0, 1)
        // or 1 (waves 2, 3) quant DMAs and, waves 2 and 3, 0 to 2 table DMAs. Past the last unit the
        // record loads repeat it (same bytes). TW = 160: waves 1-3 issue record instruction w - 1 at
        // p = 0 and Bmin instructions w - 1, w + 2 (up to 4) at p = 1 and p = 2.
        int rs_next = 0;
        for (int u = 0; u < U; u++) {
            const int u_next = u < u_last ? u + 1 : u_last;
            rs_next = u < u_last ? (rs_next == 2 ? 0 : rs_next + 1) : rs_next;  // u_next % 3
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const int s = 4 * u + p, ld = (s + 2) & 3, s_src = s + 2 < S2 ? s + 2 : S2 - 1;
#pragma unroll
                for (int q = 0; q < 4; q++) dma_a1(s_src, ld, q);
                dma_q1(s_src, ld, 0);
                if (qw == 2) dma_q1(s_src, ld, 1);
                if constexpr (G::SPLIT) {
                    if (w4 >= 1) {
                        if (p == 0) dma_rec(u_next, rs_next, w4 - 1);
                        if (p == 1) dma_bm(u, w4 - 1);
                        if (p == 2 && w4 + 2 < QK) dma_bm(u, w4 + 2);
                    }
                } else if (w4 == 2) {
                    if (p == 0) dma_rec(u_next, rs_next, 0);
                    if (p == 1) dma_rec(u_next, rs_next, 2);
                    if (p == 2) dma_bm(u, 2), dma_bm(u, 3);
                } else if (w4 == 3) {
                    if (p == 0) dma_rec(u_next, rs_next, 1);
                    if (p == 1) dma_bm(u, 0), dma_bm(u, 1);
                    if (p == 2) dma_bm(u, 4), dma_bm(u, 5);
                }
                sums(s);
                // wait for all but this stage's DMAs (4 activation, qw quant, and the table ones)
                if constexpr (G::SPLIT) {
                    if (qw == 2 || p < 2 || (p == 2 && w4 + 2 < QK)) wr_wait<6>();
                    else wr_wait<5>();
                } else {
                    if (qw == 2) wr_wait<6>();
                    else if (p == 3) wr_wait<5>();
                    else if (p == 0 || (p == 1 && w4 == 2)) wr_wait<6>();
                    else wr_wait<7>();
                }
                wr_barrier();
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last (clamped, unused) loads
        if constexpr (KS) {
            // meet the MFMA waves once they are done with the rings and tables and once their tile is
            // in LDS, then store or reduce it with them
            wr_barrier();
            wr_barrier();
            tile_finish<WR_BM, BN, WR_NT, 4>(lds, g, m0, n0, nt_i * g.mt + mt_i, part, (int *)(lds + L::TOTAL - 16));
        } else if (wr_staged(g)) {
            // the same two meetings, then store the tile with them
            wr_barrier();
            wr_barrier();
            wr_store<BN>(lds, g, m0, n0, tid);
        }
        return;
    }

    // ---------------------------------------------------------------------------------- MFMA waves
    wr_barrier();  // the loaders' prologue
    // stage 0's first operands and k-step 0 weights
    // af: ring of WR_AF (a stage's 16 groups wrap it exactly), each read WR_AD groups ahead
    h8 af[WR_AF], b0[NB], b1[NB];
    u2v qc[NB];
    h2 muh[NB], adh[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) {
        qc[j] = rdq(0, j);
        h2 mu, ad;
        scales(rdsw(0, 0, j), mu, ad);  // (super-block 0's records: slot 0)
        muh[j] = h2{mu.y, mu.y}, adh[j] = h2{ad.y, ad.y};
        b0[j] = decode8<false>(qc[j], h2{mu.x, mu.x}, h2{ad.x, ad.x});
    }
    // the activation reads last and in group order, as the loop leaves them pending at its back edge
    // (the wait before the loop's first MFMA then counts the same on both ways in)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < WR_AD; k++) {
        af[k] = rd(0, k);
        __builtin_amdgcn_sched_barrier(0);
    }
    h8 bm[NB], sa[3];
    f4 r[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) r[j] = f4{1.f, 1.f, 1.f, 1.f}, bm[j] = h8{};

    // main loop: one super-block (4 stages) per iteration; stage s = 4u + p, ring slot s % 4. The
    // previous super-block's min k-step (S of unit u - 1 x its Bmin in units of c_u, read at p = 3 of
    // unit u - 1) runs at p = 1: group g < 8 adds it to block row (g + 4) % 8, four groups away from
    // that row's own MFMAs on either side. Rescale to the next super-block's units: block row i two
    // groups after its last MFMA of the super-block (group 10 + i at p = 3; rows 6 and 7 in the next
    // super-block's groups 0 and 1, ahead of their first MFMAs there).
    uint32_t swn[NB];  // the next stage's scale words
    h2 mul0[NB], add0[NB];  // and its k-step 0 multipliers and addends
    int rs = 0;  // record slot of super-block u (u % 3)
    for (int u = 0; u < U; u++) {
        const int rsn = rs == 2 ? 0 : rs + 1;  // record slot of the next super-block
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int s = 4 * u + p, cur = s & 3, nxt = (s + 1) & 3;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int gg = 0; gg < 16; gg++) {
                // the activation operand WR_AD groups ahead (the next stage's first ones from group
                // 16 - WR_AD, after the barrier)
                if (gg + WR_AD < 16) af[(gg + WR_AD) % WR_AF] = rd(cur, gg + WR_AD);
                else af[(gg + WR_AD) % WR_AF] = rd(nxt, gg + WR_AD - 16);
#pragma unroll
                for (int j = 0; j < NB; j++)
                    if (G::has(gg & 7, j)) acc[gg & 7][j] = mfma(gg < 8 ? b0[j] : b1[j], af[gg % WR_AF], acc[gg & 7][j]);
                if (p == 1 && gg < 8) {
                    const int i = (gg + 4) & 7;
#pragma unroll
                    for (int j = 0; j < NB; j++)
                        if (G::has(i, j)) acc[i][j] = mfma_bf16(bm[j], sa[gg % 3], acc[i][j]);
                }
                // unit u - 1's sub-block sums of the row the min k-step reaches three groups later (p = 1,
                // group g < 8: row (g + 4) % 8, read from group 13 of p = 0, after this group's use of
                // the slot)
                if ((p == 0 && gg >= 13) || (p == 1 && gg < 5)) {
                    const int g = p == 0 ? gg - 13 : gg + 3;
                    sa[g % 3] = rds((u + 1) & 1, (g + 4) & 7);
                }
                // this stage's k-step 1 weights, half a column block per group
                if (gg < 2 * NB) wr_dec_half(b1[gg / 2], qc[gg / 2], gg & 1, 0xf0f0f0f0u, muh[gg / 2], adh[gg / 2]);
                if (p == 3 && gg >= 10) {
                    const int i = gg - 10;
#pragma unroll
                    for (int j = 0; j < NB; j++)
                        if (G::has(i, j)) acc[i][j] *= r[j];
                }
                if (p == 0 && gg < 2)
#pragma unroll
                    for (int j = 0; j < NB; j++)
                        if (G::has(6 + gg, j)) acc[6 + gg][j] *= r[j];
                if (gg == 6) {
                    // the loaders' wait before the barrier lands the next stage's activations and
                    // quants; after it they refill the slot of stage s - 1, whose reads have all been
                    // consumed (this stage's quants are decoded, so qc is free)
                    wr_barrier();
                    const int pn = (p + 1) & 3, un = p == 3 ? rsn : rs;
#pragma unroll
                    for (int j = 0; j < NB; j++) qc[j] = rdq(nxt, j), swn[j] = rdsw(pn, un, j);
                }
                // at p = 3 this super-block's rescale factor F = c_u / c_{u+1} and its Bmin (landed by the
                // barrier; the loaders rewrite Bmin from p = 1 of the next one), one group each after
                // the barrier's reads (one burst would exceed what an LDS wait count can leave
                // outstanding, and the next MFMA would wait for part of it)
                if (p == 3 && gg == 7)
#pragma unroll
                    for (int j = 0; j < NB; j++) r[j] = rdr(j, rs, 2);
                if (p == 3 && gg == 8)
#pragma unroll
                    for (int j = 0; j < NB; j++) bm[j] = rdbm(j);
                // the next stage's scales and k-step 0 weights (b0 is free after group 7), half a
                // column block per group
                if (gg >= 9 && gg < 9 + 2 * NB) {
                    const int j = (gg - 9) / 2, hf = (gg - 9) & 1;
                    if (hf == 0) {
                        h2 mu, ad;
                        scales(swn[j], mu, ad);
                        muh[j] = h2{mu.y, mu.y}, adh[j] = h2{ad.y, ad.y};
                        mul0[j] = h2{mu.x, mu.x}, add0[j] = h2{ad.x, ad.x};
                    }
                    wr_dec_half(b0[j], qc[j], hf, 0x0f0f0f0fu, mul0[j], add0[j]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        rs = rsn;
    }
    // ---- rows 6 and 7 to the units of the next super-block (rows 0-5 were rescaled in the last stage;
    // F is 1 for the matrix's last super-block, c_u / c_{u+1} where a K part ends before it), the last
    // super-block's min k-step (its Bmin, in those units, read at p = 3, and its sums landed by the
    // last barrier), then back to true units (c_{u+1}, or the last super-block's c) and straight from
    // the accumulators (or, with a K split, through LDS to tile_finish):
    // lane (ln, lg) of block (i, j) holds row 16i + ln, columns 16j + 4lg .. + 3 of the wave's
    // columns (one 16-byte fp32 or 8-byte fp16 store; element by element at the matrix edge or where
    // N % 4 or C's alignment does not allow it)
    if constexpr (KS)
#pragma unroll
        for (int j = 0; j < NB; j++) {
            if (G::has(6, j)) acc[6][j] *= r[j];
            if (G::has(7, j)) acc[7][j] *= r[j];
        }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const h8 si = rds(u_last & 1, i);
#pragma unroll
        for (int j = 0; j < NB; j++)
            if (G::has(i, j)) acc[i][j] = mfma_bf16(bm[j], si, acc[i][j]);
    }
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const f4 cl = rdr(j, u_last % 3, 3);
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (G::has(i, j)) acc[i][j] *= cl;
    }
    if constexpr (KS) {
        constexpr int LD = BN + 4;  // tile_finish's row stride in floats
        wr_barrier();               // every wave is done with the rings and tables
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < NB; j++)
                if (G::has(i, j)) *(f4 *)(lds + ((16 * rb_of(i) + ln) * LD + c0[j] + 4 * lg) * 4) = acc[i][j];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wr_barrier();
        tile_finish<WR_BM, BN, WR_NT, 4>(lds, g, m0, n0, nt_i * g.mt + mt_i, part, (int *)(lds + L::TOTAL - 16));
        return;
    }
    // fp16 C, or the SwiGLU output, through LDS (tile_store_rows) where C allows it: the accumulators
    // as fp16 (or the pairs' fp16 products silu(gate) * up) at their rows and columns, then all 8
    // waves store
    if (wr_staged(g)) {
        wr_barrier();  // every wave is done with the rings, sums and tables
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) {
                if (!G::has(i, j)) continue;
                const int row = 16 * rb_of(i) + ln;
                const f4 v = acc[i][j];
                if (g.c_f32 == HQ_OUT_SWIGLU)
                    *(uint32_t *)(lds + row * tile_ldr<BN>() + (c0[j] / 2 + 4 * (lg & 1) + 2 * (lg >> 1)) * 2) = swiglu_pair2(v, lg);
                else
                    *(h4 *)(lds + row * tile_ldr<BN * 2>() + (c0[j] + 4 * lg) * 2) = h4{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wr_barrier();
        wr_store<BN>(lds, g, m0, n0, tid);
        return;
    }
    // (vector stores write through to memory: SC1, measured faster than write-back here, where every
    // tile stores its whole output at the end)
    if (g.c_f32 == HQ_OUT_SWIGLU) {
        // gate/up pair matrix: C is fp16 [M, N / 2] and takes silu(gate) * up (N a multiple of 16)
        const int Nh = N / 2;
        const rsrc_t ro = make_rsrc(g.C, (uint32_t)((size_t)M * Nh * 2));
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int m = m0 + 16 * rb_of(i) + ln;
#pragma unroll
            for (int j = 0; j < NB; j++) {
                if (!G::has(i, j)) continue;
                const uint32_t y = swiglu_pair2(acc[i][j], lg);
                const int n = n0 + c0[j];
                if (m < M && n < N)
                    __builtin_amdgcn_raw_buffer_store_b32(y, ro, (uint32_t)(((size_t)m * Nh + n / 2 + 4 * (lg & 1) + 2 * (lg >> 1)) * 2),
                                                          0u, CPOL_SC1);
            }
        }
        return;
    }
    const bool vec = (N & 3) == 0 && ((uintptr_t)g.C & (g.c_f32 ? 15u : 7u)) == 0;
    const rsrc_t rc = make_rsrc(g.C, (uint32_t)((size_t)M * N * (g.c_f32 ? 4 : 2)));
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int m = m0 + 16 * rb_of(i) + ln;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int n = n0 + c0[j] + 4 * lg;
            if (!G::has(i, j) || n >= N) continue;
            const size_t idx = (size_t)m * N + n;
            f4 v = acc[i][j];
            if (vec) {
                if (g.c_f32) {
                    if (g.accumulate) v += *(const f4 *)((const float *)g.C + idx);
                    buf_store16(rc, v, (uint32_t)(idx * 4));
                } else {
                    if (g.accumulate) {
                        const h4 o = *(const h4 *)((const _Float16 *)g.C + idx);
                        v += f4{(float)o[0], (float)o[1], (float)o[2], (float)o[3]};
                    }
                    const h4 hv = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
                    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2v, hv), rc, (uint32_t)(idx * 2), 0u, CPOL_SC1);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if (n + e >= N) break;
                    if (g.c_f32) {
                        float *q = (float *)g.C + idx + e;
                        *q = g.accumulate ? *q + v[e] : v[e];
                    } else {
                        _Float16 *q = (_Float16 *)g.C + idx + e;
                        *q = (_Float16)(g.accumulate ? (float)*q + v[e] : v[e]);
                    }
                }
            }
        }
    }
}

template <int NB>
__global__ void __launch_bounds__(WR_NT) k_gemm_q4_k_wr(WrArgs g) {
    wr_tile<false, 64 * NB>(g);
}
// the same for 160-column tiles (more tiles in one round where 192-column ones leave CUs idle)
__global__ void __launch_bounds__(WR_NT) k_gemm_q4_k_wr160(WrArgs g) { wr_tile<false, 160>(g); }
template <int NB>
__global__ void __launch_bounds__(WR_NT) k_gemm_q4_k_wr_ks(WrArgs g) {
    wr_tile<true, 64 * NB>(g);
}
// the K split with 160-column tiles (M = 512, N = 2560: 4 x 16 tiles x 4 parts = 256 workgroups
// instead of 4 x 14 x 4 = 224)
__global__ void __launch_bounds__(WR_NT) k_gemm_q4_k_wr_ks160(WrArgs g) { wr_tile<true, 160>(g); }
}  // namespace

namespace {
// The K split's sum: the parts' tiles (tile_finish's layout: 16-byte piece h of 8-value chunk c of
// tile t, part p at ((t parts + p) TILE) + (h NCH + c) 16 bytes) added in part order, as tile_finish's
// last part would, by one thread per chunk over all CUs, then stored to C
template <int BN>
__global__ void __launch_bounds__(256) k_tile_reduce(const float *__restrict__ partials, int parts, int ntiles, int mt,
                                                     int M, int N, void *C, int c_f32, int accumulate) {
    constexpr int CH = BN / 8, NCH = WR_BM * CH;
    constexpr size_t TILE = (size_t)WR_BM * BN * 4;
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    if (t >= (uint32_t)ntiles * (uint32_t)NCH) return;
    const int tile = (int)(t / NCH), c = (int)(t - (uint32_t)tile * NCH), row = c / CH, ch = c - row * CH;
    const int nt_i = tile / mt, mt_i = tile - nt_i * mt, m = mt_i * WR_BM + row, n = nt_i * BN + 8 * ch;
    if (m >= M || n >= N) return;
    const char *base = (const char *)partials + (size_t)tile * parts * TILE + (size_t)c * 16;
    f4 pv[4][2];
#pragma unroll
    for (int p = 0; p < 4; p++)
        if (p < parts) pv[p][0] = *(const f4 *)(base + p * TILE), pv[p][1] = *(const f4 *)(base + p * TILE + NCH * 16);
    f4 v0 = f4{0.f, 0.f, 0.f, 0.f}, v1 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < 4; p++)
        if (p < parts) v0 += pv[p][0], v1 += pv[p][1];
    const bool wide = (N & 7) == 0 && ((uintptr_t)C & 15u) == 0;
    store8_out(C, N, m, n, v0, v1, wide, c_f32, accumulate);
}
}  // namespace

// the launch of k_tile_reduce for the register-decode kernel's tile widths (160, 192). (The LDS-decode
// tile kernels keep the last-part sum of tile_finish: their parts of a tile share one XCD's L2, and a
// separate sum measured slower there, e.g. Q8_0 M = 128, N = 9728, two parts: 19.2 -> 20.3 us.)
hipError_t hq_launch_tile_reduce(const float *partials, int parts, int ntiles, int mt, int bn, int M, int N, void *C, int c_f32,
                                 int accumulate, hipStream_t st) {
    if (parts < 2 || parts > 4 || mt < 1 || ntiles < 1) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)(((size_t)ntiles * WR_BM * (bn / 8) + 255) / 256);
    if (bn == 160) k_tile_reduce<160><<<grid, 256, 0, st>>>(partials, parts, ntiles, mt, M, N, C, c_f32, accumulate);
    else if (bn == 192) k_tile_reduce<192><<<grid, 256, 0, st>>>(partials, parts, ntiles, mt, M, N, C, c_f32, accumulate);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}


// Per-column tables of every super-block of a Q4_K matrix (one thread per row, super-blocks in order):
// for super-block v, Bmin [rows][32 B] = bf16 hi[8], lo[8] of x_i = -dmin * m_i / c_{v+1} at
// v * rows * 48, then records [rows][16 B] = scale words sw0, sw1 (zero where d = 0),
// F = c_v / c_{v+1}, CN = c_{v+1}; c_v = d_v, or 1 where d_v = 0, and c_{v+1} reads c_v for the last
// super-block (F = 1). The GEMM accumulates super-block v in units of c_v, rescales by F after it and
// adds its min term in the next units (the last super-block's in its own; -dmin * m_i is exact in
// fp32).
__global__ void __launch_bounds__(256) k_q4k_tables(const uint8_t *W, uint32_t rows, uint32_t nb, uint32_t row_bytes,
                                                    uint8_t *tab) {
    const uint32_t n = blockIdx.x * 256u + threadIdx.x;
    if (n >= rows) return;
    for (uint32_t v = 0; v < nb; v++) {
        const u4v hm = *(const u4v *)(W + (size_t)n * row_bytes + (size_t)v * 144);
        uint32_t sw0, sw1, mw0, mw1;
        q4k_scale_words(hm.y, hm.z, hm.w, sw0, sw1, mw0, mw1);
        const uint32_t nz = (hm.x & 0x7fffu) ? 0xffffffffu : 0u;
        const float d = h2f((uint16_t)hm.x), dmin = h2f((uint16_t)(hm.x >> 16));
        const float c = d != 0.0f ? d : 1.0f;
        float cn = c;
        if (v + 1 < nb) {
            const float dn = h2f(*(const uint16_t *)(W + (size_t)n * row_bytes + (size_t)(v + 1) * 144));
            cn = dn != 0.0f ? dn : 1.0f;
        }
        const float inv = 1.0f / cn;
        uint32_t bh[4], bl[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t w = q < 2 ? mw0 : mw1;
            const float x0 = (-dmin * (float)byte_of(w, 2 * (q & 1))) * inv;
            const float x1 = (-dmin * (float)byte_of(w, 2 * (q & 1) + 1)) * inv;
            const __bf16 h0 = (__bf16)x0, h1 = (__bf16)x1;
            const __bf16 l0 = (__bf16)(x0 - (float)h0), l1 = (__bf16)(x1 - (float)h1);
            bh[q] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            bl[q] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
        }
        uint8_t *t = tab + (size_t)v * rows * HQ_Q4K_TAB_BYTES;
        *(u4v *)(t + (size_t)n * 32) = u4v{bh[0], bh[1], bh[2], bh[3]};
        *(u4v *)(t + (size_t)n * 32 + 16) = u4v{bl[0], bl[1], bl[2], bl[3]};
        *(u4v *)(t + (size_t)rows * 32 + (size_t)n * 16) =
            u4v{sw0 & nz, sw1 & nz, __builtin_bit_cast(uint32_t, c / cn), __builtin_bit_cast(uint32_t, cn)};
    }
}

hipError_t hq_launch_q4k_tables(const hq_dev_mat *W, uint8_t *tab, hipStream_t st) {
    if (W->type != HQ_TYPE_Q4_K || W->cols % 256) return hipErrorInvalidValue;
    k_q4k_tables<<<(W->rows + 255) / 256, 256, 0, st>>>(W->qs, W->rows, W->cols / 256, (uint32_t)W->row_bytes, tab);
    return hipGetLastError();
}

// every byte offset of the kernel (tile rows and columns past the matrix included, C's) fits 32 bits
int hq_wr_fits(const hq_dev_mat *W, int M) {
    const size_t lim = (size_t)1 << 32, mr = (size_t)M + WR_BM;
    return W->type == HQ_TYPE_Q4_K && W->cols % 256 == 0 && M >= 1 && mr * W->cols * 2 < lim && (size_t)M * W->rows * 4 < lim &&
           ((size_t)W->rows + 64 * 3) * (W->cols / 256) * HQ_Q4K_TAB_BYTES < lim &&
           ((size_t)W->rows + 64 * 3) * W->row_bytes < lim;
}

hipError_t hq_launch_gemm_wr(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                             int nt0, int nt1, int parts, float *partials, int *counters, hipStream_t st, int tw) {
    if (!hq_wr_fits(W, M) || !W->tab) return hipErrorInvalidValue;  // (every uploaded Q4_K matrix has its tables)
    if (tw != 192 && tw != 160) return hipErrorInvalidValue;
    constexpr int NB = 3;
    WrArgs g;
    g.W = W->qs, g.row_bytes = (uint32_t)W->row_bytes, g.A = A, g.tab = W->tab;
    g.M = M, g.N = (int)W->rows, g.K = (int)W->cols, g.C = C, g.c_f32 = c_f32, g.accumulate = accumulate;
    g.mt = (M + WR_BM - 1) / WR_BM;
    const int nt_all = (g.N + tw - 1) / tw;
    g.nt0 = nt0, g.nt = nt1 < 0 || nt1 > nt_all ? nt_all : nt1;
    if (nt0 < 0 || nt0 >= g.nt) return hipErrorInvalidValue;
    // K split: whole super-blocks per part, the full column range, a workspace of one fp32 tile per
    // (tile, part) and a zeroed counter per tile, 32-bit offsets
    g.parts = parts, g.partials = partials, g.counters = counters, g.ntiles = g.mt * g.nt;
    if (parts < 1 || parts > 4 || parts > g.K / 256) return hipErrorInvalidValue;
    if (parts > 1 && (!partials || !counters || nt0 != 0 || c_f32 == HQ_OUT_SWIGLU ||
                      (size_t)g.ntiles * parts * WR_BM * tw * 4 >= ((size_t)1 << 32)))
        return hipErrorInvalidValue;
    // fp32 or fp16 C, or the SwiGLU output of a gate/up pair matrix (N a multiple of 16, no accumulate)
    if (c_f32 != 0 && c_f32 != 1 && !(c_f32 == HQ_OUT_SWIGLU && W->rows % 16 == 0 && !accumulate)) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)(8 * (((g.nt - g.nt0) * parts + 7) / 8) * g.mt);
    if (parts > 1) {
        // every part stores its tile; k_tile_reduce adds them
        g.counters = nullptr;
        if (tw == 160) k_gemm_q4_k_wr_ks160<<<grid, WR_NT, 0, st>>>(g);
        else k_gemm_q4_k_wr_ks<NB><<<grid, WR_NT, 0, st>>>(g);
        return hq_launch_tile_reduce(partials, parts, g.ntiles, g.mt, tw, M, g.N, C, c_f32, accumulate, st);
    }
    else if (tw == 160) k_gemm_q4_k_wr160<<<grid, WR_NT, 0, st>>>(g);
    else k_gemm_q4_k_wr<NB><<<grid, WR_NT, 0, st>>>(g);
    return hipGetLastError();
}
