// hq_gemm_bt.hip - Q4_K GEMM for large M on gfx950: 256 x 256 output tiles, 8 cooperating waves.
//
// C[M,N] (+)= A[M,K] . W^T with A fp16 and W GGUF Q4_K super-blocks resident in HBM (reference
// arithmetic: cleanroom-transformer/src/ggml_quant.h:51-59, :135-150; matmul src/cpu_backend.c:38-54).
//
// Why this shape. A 256 x 256 tile over the whole of K, 8 waves of 128 x 64 each (two per SIMD, so
// one wave's LDS waits and decode run under the other's MFMAs). Decoded weights never pass through
// LDS: in a 16 x 16 x 32 MFMA the weight operand of lane (ln, lg) is column ln, k 8lg .. 8lg + 7,
// and in a Q4_K quant group byte l holds k = l (low nibble) and k = 32 + l (high nibble), so the 8
// quant bytes 8lg .. 8lg + 7 of a column's 32-byte group decode in registers into that lane's
// operands of both 32-k steps of a 64-k stage. The raw quant groups are staged in LDS by DMA (8 KB
// per stage) and the two waves sharing a column block (one per row half) each decode it. Per stage
// LDS then carries the activation tile (32 KB written, 128 KB read: the 8 waves read 128 rows
// each), the quant groups (8 KB written, 16 KB read) and the per-super-block tables.
//
// Pipeline. K is walked in stages of 64 (one 32-byte quant group p of a super-block u: low nibbles
// = sub-block 2p, high = 2p + 1). Activations and quant groups are triple-buffered in LDS and one
// s_barrier ends each stage. In stage s = 4u + p every wave issues, in this order: the activation
// DMA of stage s + 2 (4 of the tile's 32 1-KB DMAs) and its quant DMA (1 of 8), at p = 1 the next
// super-block's activation sums (S DMA), at p = 0 the next super-block's 16-byte header (a register
// load); then, at p = 0, the super-block's min k-step (below), and the stage's two 32-k k-steps
// (weight operands decoded from the stage's quant groups, 32 MFMAs each); at p = 3 the column owners
// write the next super-block's tables. Every load is issued as assembly, out of the compiler's
// count: the end of stage s waits (s_waitcnt vmcnt) for everything issued before stage s, so each
// load has between one and two stages to land.
//
// Arithmetic: as hq_gemm_ws.hip (accumulators in units of c_u = d_u, the weight operand the exact
// integer s*q, rescale by c_{u-1}/c_u where a super-block begins and by c_{U-1} at the end; the min
// term one bf16 MFMA per (16 x 16 block, super-block) with hi/lo splits of the sub-block sums S and
// of x = -dmin*m/c_u). Output lane (ln, lg) of a 16 x 16 block holds row ln, columns 4lg .. 4lg + 3.
//
// LDS (142 KB): A [3][256 rows][64 k] fp16, 128 B per row, 16-byte slot p at p ^ ((row >> 1) & 7)
// (the 16 lanes of an operand read hit 16 distinct 4-bank groups); quant groups [3][256 columns][32
// B], the two 16-byte halves of column c swapped where (c >> 3) & 1 (conflict-free 8-byte reads); S
// [256 rows][16] bf16 (hi[8], lo[8]); per column of the next super-block: Bmin [256][16] bf16 (Bh[8],
// Bl[8]), R and CL [256] fp32; scale words SW [2][256][2] (sub-blocks 0-3, 4-7; zero where d = 0) by
// super-block parity.
#include <type_traits>

#include "hq_device.h"
#include "hq_kernels.h"

namespace {
constexpr int BT_BM = 256, BT_BN = 256, BT_KS = 64, BT_NT = 512;

struct BtArgs {
    const uint8_t *W;  // Q4_K super-blocks, row n at n * row_bytes
    uint32_t row_bytes;
    const uint16_t *A;  // fp16 [M][K]
    const uint16_t *S;  // activation sub-block sums [M][K/256][16] (k_asums, bf16 hi/lo)
    int M, N, K;
    void *C;
    int c_f32, accumulate;
    int mt, nt;
};

struct BtLds {
    static constexpr int A = 0, A_BYTES = BT_BM * BT_KS * 2;  // per buffer (3 buffers)
    static constexpr int Q = 3 * A_BYTES, Q_BYTES = BT_BN * 32;  // quant groups, per buffer (3 buffers)
    static constexpr int S = Q + 3 * Q_BYTES;        // [256][16] bf16
    static constexpr int BM = S + BT_BM * 32;        // [256][16] bf16
    static constexpr int R = BM + BT_BN * 32;        // [256] fp32
    static constexpr int CL = R + BT_BN * 4;         // [256] fp32
    static constexpr int SW = CL + BT_BN * 4;        // [2][256][2] u32, by super-block parity
    static constexpr int TOTAL = SW + 2 * BT_BN * 8;
    static_assert(TOTAL <= 160 * 1024, "LDS budget");
};

DEV void bt_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Buffer loads into registers, written as assembly so that the compiler does not track them (its own
// count of outstanding loads leaves out the LDS DMAs, so any wait it placed for such a load would
// also wait for DMAs issued after it). A value is valid only after an explicit s_waitcnt that takes
// it as an in-out operand (which also keeps every use after that wait).
DEV u4v bt_load16(rsrc_t r, uint32_t voff, uint32_t soff) {
    u4v v;
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(r), "s"(soff) : "memory");
    return v;
}


__global__ void __launch_bounds__(BT_NT) k_gemm_q4_k_bt(BtArgs g) {
    using L = BtLds;
    __shared__ __attribute__((aligned(256))) char lds[L::TOTAL];
    const int M = g.M, N = g.N, K = g.K, U = K / 256, S2 = 4 * U;
    // tile of this workgroup: XCD x = b % 8 runs the x-th eighth of the tile list (M-tile major, so an
    // XCD's workgroups share activation tiles in its L2)
    const int T = g.mt * g.nt, per = (T + 7) / 8, b = blockIdx.x, t = (b & 7) * per + (b >> 3);
    if (t >= T) return;
    const int m0 = (t / g.nt) * BT_BM, n0 = (t % g.nt) * BT_BN;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave & 1, wn = wave >> 1, ln = lane & 15, lg = lane >> 4;
    const rsrc_t ra = make_rsrc(g.A, (uint32_t)((size_t)M * K * 2));
    const rsrc_t rw = make_rsrc(g.W, (uint32_t)((size_t)N * g.row_bytes));
    const rsrc_t rs = make_rsrc(g.S, (uint32_t)((size_t)M * U * 32));
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;

    // ---- activation DMA: instruction q (0..3) of wave w fills rows 8(4w + q) .. + 8 of a buffer;
    // lane i: row r = 8(4w + q) + i/8, LDS slot i % 8, global 8-value chunk (i % 8) ^ ((r >> 1) & 7),
    // which is the q = 0 chunk ^ 4 for odd q
    // (the row in the VGPR offset, the one a buffer load range-checks: rows past M read zeros and no
    // load reads past the end of A)
    const int a_row0 = 32 * wave + (lane >> 3);
    const uint32_t a_ch = (uint32_t)((lane & 7) ^ ((a_row0 >> 1) & 7));
    uint32_t a_voff[4];
#pragma unroll
    for (int q = 0; q < 4; q++) a_voff[q] = (uint32_t)(m0 + a_row0 + 8 * q) * (uint32_t)K * 2u + 16u * (q & 1 ? a_ch ^ 4u : a_ch);
    auto dma_a1 = [&](int s, int buf, int q) {
        dma16_so(ra, lds0 + (uint32_t)(L::A + buf * L::A_BYTES + wave * 4096 + q * 1024), a_voff[q], (uint32_t)(s * BT_KS * 2));
    };
    auto dma_a = [&](int s, int buf) {
#pragma unroll
        for (int q = 0; q < 4; q++) dma_a1(s, buf, q);
    };
    // S of super-block u: wave w moves rows 32w .. + 32 (1 KB); lane i: row 32w + i/2, half i % 2
    const uint32_t s_voff = (uint32_t)(m0 + 32 * wave + (lane >> 1)) * (uint32_t)U * 32u + 16u * (uint32_t)(lane & 1);
    auto dma_s = [&](int u) { dma16_so(rs, lds0 + (uint32_t)(L::S + wave * 1024), s_voff, (uint32_t)(u * 32)); };
    // quant DMA of stage s (group s % 4 of super-block s / 4, 32 bytes per column): wave w moves
    // columns 32w .. + 32; lane i: column c = 32w + i/2, LDS half i % 2 of the column's 32 bytes, which
    // holds the group's half (i % 2) ^ ((c >> 3) & 1) (so that the 8-byte operand reads below hit
    // distinct banks)
    const int q_col = 32 * wave + (lane >> 1);
    const uint32_t q_voff = (uint32_t)(n0 + q_col) * g.row_bytes + 16u * (uint32_t)((lane & 1) ^ ((q_col >> 3) & 1));
    auto dma_q = [&](int s, int buf) {
        dma16_so(rw, lds0 + (uint32_t)(L::Q + buf * L::Q_BYTES + wave * 1024), q_voff,
                 (uint32_t)((s >> 2) * 144 + 16 + 32 * (s & 3)));
    };
    // header of super-block u for the column owners (thread t: column t / 2; both threads of a column
    // load it, the even one writes the tables)
    const int col = tid >> 1, half = tid & 1;
    const uint32_t h_voff = (uint32_t)(n0 + col) * g.row_bytes;
    auto load_h = [&](int u) { return bt_load16(rw, h_voff, (uint32_t)(u * 144)); };

    // ---- per-column tables of a super-block (threads with half == 0): scale words, min-term
    // operands, rescale ratio and unit
    float c_prev = 1.0f;
    auto write_tables = [&](const u4v hm, int u) {
        uint32_t sw0, sw1, mw0, mw1;
        q4k_scale_words(hm.y, hm.z, hm.w, sw0, sw1, mw0, mw1);
        const uint32_t nz = (hm.x & 0x7fffu) ? 0xffffffffu : 0u;  // d = 0: B = 0 (min term only)
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
        *(u4v *)(lds + L::BM + col * 32) = bh;
        *(u4v *)(lds + L::BM + col * 32 + 16) = bl;
        *(float *)(lds + L::R + col * 4) = c_prev * inv;
        *(float *)(lds + L::CL + col * 4) = c;
        // read in every stage of unit u, while the tables of unit u + 1 are written: two buffers
        *(u2v *)(lds + L::SW + (u & 1) * BT_BN * 8 + col * 8) = u2v{sw0 & nz, sw1 & nz};
        c_prev = c;
    };

    // ---- MFMA work of wave (wm, wn): rows 128 wm + 16 i (i < 8), columns 64 wn + 16 j (j < 4)
    const uint32_t xs = 16u * ((uint32_t)lg ^ (uint32_t)((ln >> 1) & 7));  // k-step 0 slot; k-step f: ^ 64 f
    const uint32_t a_lane = lds0 + (uint32_t)(L::A + (128 * wm + ln) * 128) + xs;
    const uint32_t s_lane = lds0 + (uint32_t)(L::S + (128 * wm + ln) * 32 + 16 * (lg & 1));
    const uint32_t m_lane = lds0 + (uint32_t)(L::BM + (64 * wn + ln) * 32 + 16 * (lg >> 1));
    const uint32_t r_lane = lds0 + (uint32_t)(L::R + (64 * wn + 4 * lg) * 4);
    const uint32_t cl_lane = lds0 + (uint32_t)(L::CL + (64 * wn + 4 * lg) * 4);
    const uint32_t sw_lane = lds0 + (uint32_t)(L::SW + (64 * wn + ln) * 8);
    // quants of column block j for lane (ln, lg): column c = 64 wn + 16 j + ln, bytes 8 lg .. + 7 of the
    // group (((c >> 3) & 1) is j-independent)
    const uint32_t q_lane = lds0 + (uint32_t)(L::Q + (64 * wn + ln) * 32 +
                                              16 * ((lg >> 1) ^ ((ln >> 3) & 1)) + 8 * (lg & 1));
    using lds_h8 = const __attribute__((address_space(3))) h8;
    using lds_f4 = const __attribute__((address_space(3))) f4;
    using lds_u1 = const __attribute__((address_space(3))) uint32_t;
    using lds_u2 = const __attribute__((address_space(3))) u2v;
    auto at = [](uint32_t byte) { return *(lds_h8 *)(uintptr_t)byte; };
    auto at4 = [](uint32_t byte) { return *(lds_f4 *)(uintptr_t)byte; };
    auto at1 = [](uint32_t byte) { return *(lds_u1 *)(uintptr_t)byte; };
    auto at2 = [](uint32_t byte) { return *(lds_u2 *)(uintptr_t)byte; };
    f4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    // The MFMA sequences below are written in issue order, one group of 4 MFMAs (one 16-row block
    // against the wave's 4 column blocks) between scheduling barriers: each group first issues the
    // LDS read of the operand two groups ahead, and VALU work (rescale, decode) that the next groups
    // need is placed behind the MFMAs it overlaps. Left alone, the compiler reads each operand right
    // before its MFMAs and the LDS latency is exposed at every group.
    //
    // The min k-step of a super-block: rescale block row i by c_{u-1}/c_u, then S x Bmin (bf16).
    auto min_step = [&]() {
        f4 r[4];
        h8 bm[4], sa[3];
#pragma unroll
        for (int j = 0; j < 4; j++) r[j] = at4(r_lane + j * 16 * 4);
#pragma unroll
        for (int j = 0; j < 4; j++) bm[j] = at(m_lane + j * 16 * 32);
        sa[0] = at(s_lane);
        sa[1] = at(s_lane + 16 * 32);
#pragma unroll
        for (int j = 0; j < 4; j++) acc[0][j] *= r[j];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (i + 2 < 8) sa[(i + 2) % 3] = at(s_lane + (i + 2) * 16 * 32);
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = mfma_bf16(bm[j], sa[i % 3], acc[i][j]);
            if (i + 1 < 8)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i + 1][j] *= r[j];
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // a stage's two 32-k steps: weight operands decoded from the quants q with the super-block's
    // scale words sw (sub-blocks 2p, 2p + 1: bytes 2(p % 2), 2(p % 2) + 1 of word p / 2), activation
    // operands from A buffer at offset boff. Group g (0 .. 15): k-step g / 8, block row g % 8; the
    // k-step 1 weight operands are decoded behind the first four groups.
    auto stage_mfma = [&](int p, int buf, int u, auto issue) {
        const uint32_t boff = (uint32_t)(buf * L::A_BYTES);
        u2v q[4];
#pragma unroll
        for (int j = 0; j < 4; j++) q[j] = at2(q_lane + (uint32_t)(buf * L::Q_BYTES + j * 16 * 32));
        auto rd = [&](int g) { return at(((a_lane ^ (64u * (uint32_t)(g >> 3))) + boff) + (uint32_t)((g & 7) * 16 * 128)); };
        h8 af[3], b0[4], b1[4];
        h2 mu[4], ad[4];
        af[0] = rd(0);
        af[1] = rd(1);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t w = at1(sw_lane + (uint32_t)((u & 1) * BT_BN * 8 + j * 16 * 8 + (p >> 1) * 4)) >> ((p & 1) * 16);
            const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
            const h2 sp = as_h2(__builtin_amdgcn_perm(0x64646464u, w, 0x04010400u)) - k1024;  // (s_lo, s_hi)
            mu[j] = sp * h2{(_Float16)1.0f, (_Float16)0.0625f};
            ad[j] = sp * h2{(_Float16)-1024.0f, (_Float16)-64.0f};
            b0[j] = decode8<false>(q[j], h2{mu[j].x, mu[j].x}, h2{ad[j].x, ad[j].x});
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < 16; g++) {
            if (g + 2 < 16) af[(g + 2) % 3] = rd(g + 2);
#pragma unroll
            for (int j = 0; j < 4; j++) acc[g & 7][j] = mfma(g < 8 ? b0[j] : b1[j], af[g % 3], acc[g & 7][j]);
            if (g < 4) b1[g] = decode8<true>(q[g], h2{mu[g].y, mu[g].y}, h2{ad[g].y, ad[g].y});
            issue(g);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // ---- prologue: activations and quants of stages 0 and 1, S and header of unit 0; unit 0's tables
    u4v H;
    dma_a(0, 0);
    dma_a(1, 1);
    dma_q(0, 0);
    dma_q(1, 1);
    dma_s(0);
    H = load_h(0);
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(H)::"memory");
    if (half == 0) write_tables(H, 0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    bt_barrier();

    // ---- main loop: one super-block (4 stages) per iteration; stage s = 4u + p. H: the header of
    // unit u until stage 4u (unit u's tables are written by then), then of unit u + 1. Every stage
    // issues the same loads whatever u is (sources past the end of K are clamped to the last unit or
    // stage; what they bring is never used), so the wait counts are constants.
    const int u_last = U - 1;
    int ab = 0;  // A buffer of stage s (s % 3)
    for (int u = 0; u < U; u++) {
        const int u_next = u < u_last ? u + 1 : u_last;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int s = 4 * u + p;
            const int ab2 = ab == 0 ? 2 : ab - 1;  // (s + 2) % 3
            const int s_src = s + 2 < S2 ? s + 2 : S2 - 1;
            // the stage's loads, issued between its MFMA groups (a burst of them at the stage start
            // would hold up every wave's first MFMAs while the address unit works through them)
            auto issue = [&](int g) {
                if (g == 1 || g == 3 || g == 5 || g == 7) dma_a1(s_src, ab2, g >> 1);
                if (g == 9) dma_q(s_src, ab2);
                if (p == 1 && g == 11) dma_s(u_next);  // unit u's min k-step is behind the previous barrier
                if (p == 0 && g == 13) H = load_h(u_next);
            };
            __builtin_amdgcn_sched_barrier(0);
            if (p == 0) min_step();
            stage_mfma(p, ab, u, issue);
            __builtin_amdgcn_sched_barrier(0);
            if (p == 3 && u + 1 < U && half == 0) write_tables(H, u + 1);
            // end of stage s: every load issued before this stage has landed (the loads this stage
            // issued may stay in flight): the activations and quants of stage s + 1 and, at p = 1,
            // the header loaded at p = 0.
            if (p == 0) asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)" ::: "memory");
            if (p == 1) asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)" : "+v"(H)::"memory");
            if (p >= 2) asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)" ::: "memory");
            bt_barrier();
            ab = ab == 2 ? 0 : ab + 1;
        }
    }
    // the last stages' (clamped, unused) loads still write LDS and the header register: land them
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(H)::"memory");

    // ---- output: back to true units (the last unit's c), rows 128 wm + 16 i + ln, columns
    // 64 wn + 16 j + 4 lg .. + 3
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const f4 cl = at4(cl_lane + j * 16 * 4);
        const int n = n0 + 64 * wn + 16 * j + 4 * lg;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int m = m0 + 128 * wm + 16 * i + ln;
            const f4 v = acc[i][j] * cl;
            if (m >= M || n >= N) continue;
            const size_t idx = (size_t)m * N + n;
            if (n + 4 <= N && (N & 3) == 0) {
                if (g.c_f32) {
                    f4 *c = (f4 *)((float *)g.C + idx);
                    *c = g.accumulate ? *c + v : v;
                } else {
                    typedef _Float16 hh4 __attribute__((ext_vector_type(4)));
                    hh4 *c = (hh4 *)((_Float16 *)g.C + idx);
                    *c = __builtin_convertvector(g.accumulate ? __builtin_convertvector(*c, f4) + v : v, hh4);
                }
            } else {
                for (int e = 0; e < 4 && n + e < N; e++) store_out(g.C, idx + e, v[e], g.c_f32, g.accumulate);
            }
        }
    }
}
}  // namespace

// every byte offset of the kernel (tile rows and columns past the matrix included) fits 32 bits
int hq_bt_fits(const hq_dev_mat *W, int M) {
    const size_t lim = (size_t)1 << 32, mr = (size_t)M + BT_BM;
    return W->type == HQ_TYPE_Q4_K && W->cols % 256 == 0 && M >= 1 && mr * W->cols * 2 < lim &&
           mr * (W->cols / 256) * 32 < lim && ((size_t)W->rows + BT_BN) * W->row_bytes < lim;
}

hipError_t hq_launch_gemm_bt(const hq_dev_mat *W, const uint16_t *A, const uint16_t *S, int M, void *C, int c_f32,
                             int accumulate, hipStream_t st) {
    if (!hq_bt_fits(W, M)) return hipErrorInvalidValue;
    BtArgs g;
    g.W = W->qs, g.row_bytes = (uint32_t)W->row_bytes, g.A = A, g.S = S;
    g.M = M, g.N = (int)W->rows, g.K = (int)W->cols, g.C = C, g.c_f32 = c_f32, g.accumulate = accumulate;
    g.mt = (M + BT_BM - 1) / BT_BM;
    g.nt = (g.N + BT_BN - 1) / BT_BN;
    const int T = g.mt * g.nt, per = (T + 7) / 8;
    k_gemm_q4_k_bt<<<(unsigned)(8 * per), BT_NT, 0, st>>>(g);
    return hipGetLastError();
}
