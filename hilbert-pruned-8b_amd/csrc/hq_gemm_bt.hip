// hq_gemm_bt.hip - Q4_K GEMM for large M on gfx950: 256 x 256 output tiles, 8 cooperating waves.
//
// C[M,N] (+)= A[M,K] . W^T with A fp16 and W GGUF Q4_K super-blocks resident in HBM (reference
// arithmetic: cleanroom-transformer/src/ggml_quant.h:51-59, :135-150; matmul src/cpu_backend.c:38-54).
//
// Why this shape. Per CU and per k, a BM x BN tile costs BM*BN MACs, BM*2 + BN*0.5625 bytes from
// L2 (fp16 activations, Q4_K weights), and, with wave tiles WM x WN, 2*(BM*BN/WN + BM*BN/WM)/... LDS
// reads; at 256 x 256 with 128 x 64 wave tiles the L2 bytes per MAC are 0.59x and the LDS reads per
// MAC 0.84x those of the 128 x 160 tile kernel (hq_gemm_ws.hip), and each weight is decoded once
// for 256 rows instead of 128. Every wave loads, decodes and multiplies (no producer / consumer
// roles): two waves per SIMD, so one wave's loads, decode and LDS waits run under the other's MFMAs.
//
// Pipeline. K is walked in stages of 64 (one 32-byte quant group p of a super-block: low nibbles =
// sub-block 2p, high = 2p + 1), double-buffered in LDS, one s_barrier per stage. In stage s every
// wave issues the activation DMA of stage s + 1 (4 of the tile's 32 1-KB DMAs), the 16-byte quant
// load of stage s + 3 (a 4-deep register ring), at a super-block's first stage the next
// super-block's 16-byte header, at its second stage the next super-block's activation sums (S DMA);
// runs stage s's two 32-k MFMA k-steps; decodes stage s + 1 into the other B buffer; and at a
// super-block's third stage writes the next super-block's min-term operands.
//
// Arithmetic: as hq_gemm_ws.hip (accumulators in units of c_u = d_u, the B operand the exact integer
// s*q, rescale by c_{u-1}/c_u where a super-block begins and by c_{U-1} at the end; the min term one
// bf16 MFMA per (16 x 16 block, super-block) with hi/lo splits of the sub-block sums S and of
// x = -dmin*m/c_u). The weight fragment is the MFMA's first operand: lane (ln, lg) of a 16 x 16 block
// holds row ln, columns 4lg .. 4lg + 3.
//
// LDS (146 KB): A [2][256 rows][64 k] fp16 and B [2][256 cols][64 k] fp16, 128 B per row / column,
// 16-byte slot p at p ^ ((row or col >> 1) & 7) (16 lanes of an operand read hit 16 distinct 4-bank
// groups); S [256 rows][16] bf16 (hi[8], lo[8]); Bmin [256 cols][16] bf16 (Bh[8], Bl[8]); R, CL
// [256] fp32.
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
    static constexpr int A = 0, A_BYTES = BT_BM * BT_KS * 2;  // per buffer
    static constexpr int B = 2 * A_BYTES, B_BYTES = BT_BN * BT_KS * 2;
    static constexpr int S = B + 2 * B_BYTES;       // [256][16] bf16
    static constexpr int BM = S + BT_BM * 32;       // [256][16] bf16
    static constexpr int R = BM + BT_BN * 32;       // [256] fp32
    static constexpr int CL = R + BT_BN * 4;        // [256] fp32
    static constexpr int TOTAL = CL + BT_BN * 4;
    static_assert(TOTAL <= 160 * 1024, "LDS budget");
};

DEV void bt_barrier() { asm volatile("s_barrier" ::: "memory"); }

// 16-byte buffer load into registers, written as assembly so that the compiler does not track it
// (its own count of outstanding loads leaves out the LDS DMAs, so any wait it placed for this load
// would also wait for DMAs issued after it). The value is valid only after an explicit s_waitcnt
// that takes it as an in-out operand (which also keeps every use after that wait).
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
    if ((b >> 3) >= per || t >= T) return;
    const int m0 = (t / g.nt) * BT_BM, n0 = (t % g.nt) * BT_BN;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const rsrc_t ra = make_rsrc(g.A, (uint32_t)((size_t)M * K * 2));
    const rsrc_t rw = make_rsrc(g.W, (uint32_t)((size_t)N * g.row_bytes));
    const rsrc_t rs = make_rsrc(g.S, (uint32_t)((size_t)M * U * 32));

    // ---- loads. The LDS DMAs are untracked by the compiler (it would wait for each before every later
    // LDS read); the end of a stage waits for them explicitly. Activation DMA: instruction q (0..3) of
    // wave w fills rows 8(4w + q) .. + 8 of a buffer; lane i: row r = 8(4w + q) + i/8, LDS slot i % 8,
    // global 8-value chunk (i % 8) ^ ((r >> 1) & 7), which is the q = 0 chunk ^ 4 for odd q
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
    const int a_row0 = 32 * wave + (lane >> 3);
    const uint32_t a_ch = (uint32_t)((lane & 7) ^ ((a_row0 >> 1) & 7));
    const uint32_t a_rowoff = (uint32_t)(m0 + a_row0) * (uint32_t)K * 2u;
    const uint32_t a_voff0 = a_rowoff + 16u * a_ch, a_voff1 = a_rowoff + 16u * (a_ch ^ 4u);
    auto dma_a = [&](int s, int buf) {
        const uint32_t dst = lds0 + (uint32_t)(L::A + buf * L::A_BYTES + wave * 4096);
#pragma unroll
        for (int q = 0; q < 4; q++)
            dma16_so(ra, dst + q * 1024, q & 1 ? a_voff1 : a_voff0, (uint32_t)(q * 8 * K * 2 + s * BT_KS * 2));
    };
    // S of super-block u: wave w moves rows 32w .. + 32 (1 KB); lane i: row 32w + i/2, half i % 2
    const uint32_t s_voff = (uint32_t)(m0 + 32 * wave + (lane >> 1)) * (uint32_t)U * 32u + 16u * (uint32_t)(lane & 1);
    auto dma_s = [&](int u) { dma16_so(rs, lds0 + (uint32_t)(L::S + wave * 1024), s_voff, (uint32_t)(u * 32)); };
    // quants: thread t decodes column c = t / 2 (bytes 16h .. 16h + 15 of each quant group, h = t % 2)
    const int col = tid >> 1, half = tid & 1;
    const uint32_t w_row = (uint32_t)(n0 + col) * g.row_bytes, w_q = w_row + 16u * (uint32_t)half;
    auto load_q = [&](int s) { return bt_load16(rw, w_q, (uint32_t)((s >> 2) * 144 + 16 + 32 * (s & 3))); };
    auto load_h = [&](int u) { return bt_load16(rw, w_row, (uint32_t)(u * 144)); };

    // ---- decode of stage s into B buffer s & 1: low nibbles -> k 16h .. 16h + 15 (slots 2h, 2h + 1),
    // high nibbles -> k 32 + 16h .. (slots 4 + 2h, 5 + 2h), of column c's 128-byte row
    const uint32_t cx = (uint32_t)((col >> 1) & 7);
    char *const b_col = lds + L::B + col * 128;
    auto decode = [&](int s, const u4v q, uint32_t sw0, uint32_t sw1) {
        const int p = s & 3;
        const uint32_t sw = p < 2 ? sw0 : sw1, sh = (uint32_t)(p & 1) * 16u;
        // (1024 + s_lo, 1024 + s_hi) from scale bytes 2(p % 2), 2(p % 2) + 1
        const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
        const h2 sp = as_h2(__builtin_amdgcn_perm(0x64646464u, sw >> sh, 0x04010400u)) - k1024;
        const h2 mu = sp * h2{(_Float16)1.0f, (_Float16)0.0625f}, ad = sp * h2{(_Float16)-1024.0f, (_Float16)-64.0f};
        char *dst = b_col + (s & 1) * L::B_BYTES;
        const u2v q01 = {q.x, q.y}, q23 = {q.z, q.w};
        *(h8 *)(dst + 16 * ((uint32_t)(2 * half) ^ cx)) = decode8<false>(q01, h2{mu.x, mu.x}, h2{ad.x, ad.x});
        *(h8 *)(dst + 16 * ((uint32_t)(2 * half + 1) ^ cx)) = decode8<false>(q23, h2{mu.x, mu.x}, h2{ad.x, ad.x});
        *(h8 *)(dst + 16 * ((uint32_t)(4 + 2 * half) ^ cx)) = decode8<true>(q01, h2{mu.y, mu.y}, h2{ad.y, ad.y});
        *(h8 *)(dst + 16 * ((uint32_t)(5 + 2 * half) ^ cx)) = decode8<true>(q23, h2{mu.y, mu.y}, h2{ad.y, ad.y});
    };
    // scale words of a header (zero where d = 0, so that B = 0 there)
    auto scale_words = [&](const u4v hm, uint32_t &sw0, uint32_t &sw1) {
        uint32_t mw0, mw1;
        q4k_scale_words(hm.y, hm.z, hm.w, sw0, sw1, mw0, mw1);
        const uint32_t nz = (hm.x & 0x7fffu) ? 0xffffffffu : 0u;
        sw0 &= nz, sw1 &= nz;
    };
    // min-term operands, rescale ratio and unit of a super-block (threads with half == 0, one per column)
    float c_prev = 1.0f;
    auto write_min = [&](const u4v hm) {
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
        *(u4v *)(lds + L::BM + col * 32) = bh;
        *(u4v *)(lds + L::BM + col * 32 + 16) = bl;
        *(float *)(lds + L::R + col * 4) = c_prev * inv;
        *(float *)(lds + L::CL + col * 4) = c;
        c_prev = c;
    };

    // ---- MFMA work of wave (wm, wn): rows 128 wm + 16 i (i < 8), columns 64 wn + 16 j (j < 4)
    const int wm = wave & 1, wn = wave >> 1, ln = lane & 15, lg = lane >> 4;
    const uint32_t xs = 16u * ((uint32_t)lg ^ (uint32_t)((ln >> 1) & 7));  // k-step 0 slot; k-step f: ^ 64 f
    const uint32_t a_lane = (uint32_t)(uintptr_t)(lds + L::A) + (uint32_t)((128 * wm + ln) * 128) + xs;
    const uint32_t b_lane = (uint32_t)(uintptr_t)(lds + L::B) + (uint32_t)((64 * wn + ln) * 128) + xs;
    const uint32_t s_lane = (uint32_t)(uintptr_t)(lds + L::S) + (uint32_t)((128 * wm + ln) * 32 + 16 * (lg & 1));
    const uint32_t m_lane = (uint32_t)(uintptr_t)(lds + L::BM) + (uint32_t)((64 * wn + ln) * 32 + 16 * (lg >> 1));
    const uint32_t r_lane = (uint32_t)(uintptr_t)(lds + L::R) + (uint32_t)((64 * wn + 4 * lg) * 4);
    const uint32_t cl_lane = (uint32_t)(uintptr_t)(lds + L::CL) + (uint32_t)((64 * wn + 4 * lg) * 4);
    using lds_h8 = const __attribute__((address_space(3))) h8;
    using lds_f4 = const __attribute__((address_space(3))) f4;
    auto at = [](uint32_t byte) { return *(lds_h8 *)(uintptr_t)byte; };
    auto at4 = [](uint32_t byte) { return *(lds_f4 *)(uintptr_t)byte; };
    f4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    // the min k-step of a super-block: rescale, then S x Bmin (bf16)
    auto min_step = [&]() {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const f4 r = at4(r_lane + j * 16 * 4);
#pragma unroll
            for (int i = 0; i < 8; i++) acc[i][j] *= r;
        }
        h8 bm[4];
#pragma unroll
        for (int j = 0; j < 4; j++) bm[j] = at(m_lane + j * 16 * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const h8 sa = at(s_lane + i * 16 * 32);
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = mfma_bf16(bm[j], sa, acc[i][j]);
        }
    };
    // the two 32-k steps of a stage from buffer buf
    auto stage_mfma = [&](int buf) {
#pragma unroll
        for (int f = 0; f < 2; f++) {
            const uint32_t ao = a_lane ^ (64u * f), bo = b_lane ^ (64u * f);
            h8 bf[4];
#pragma unroll
            for (int j = 0; j < 4; j++) bf[j] = at(bo + buf * L::B_BYTES + j * 16 * 128);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const h8 af = at(ao + buf * L::A_BYTES + i * 16 * 128);
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = mfma(bf[j], af, acc[i][j]);
            }
        }
    };

    // ---- prologue: headers of units 0 and 1, quants of stages 0 .. 2, stage 0's activations, S of
    // unit 0; unit 0's min-term operands and stage 0's B tile
    u4v H, Q[4];
    H = load_h(0);
    Q[0] = load_q(0);
    Q[1] = load_q(1);
    Q[2] = load_q(2);
    dma_a(0, 0);
    dma_s(0);
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(H), "+v"(Q[0]), "+v"(Q[1]), "+v"(Q[2])::"memory");
    uint32_t sw0, sw1;
    scale_words(H, sw0, sw1);
    if (half == 0) write_min(H);
    decode(0, Q[0], sw0, sw1);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    bt_barrier();

    // ---- main loop: one super-block (4 stages) per iteration; stage s = 4u + p. H: the header of
    // unit u until stage 4u (its scale words and min-term operands are taken by then), then of u + 1.
    // Every stage issues the same loads whatever u is (sources past the end of K are clamped to the
    // last unit or stage; what they bring is never used), so the compiler counts its own loads
    // exactly and waits for each only where it is used.
    const int u_last = U - 1;
    for (int u = 0; u < U; u++) {
        const int u_next = u < u_last ? u + 1 : u_last;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int s = 4 * u + p;
            if (p == 0) min_step();
            __builtin_amdgcn_sched_barrier(0);
            // decode stage s + 1 (its quants were loaded two stages ago) before this stage's loads
            // are issued, so that the wait for them is not also a wait for the new loads
            if (s + 1 < S2) {
                // stage s + 1's scale words: this unit's, or (p == 3) the next unit's header
                uint32_t w0 = sw0, w1 = sw1;
                if (p == 3) scale_words(H, w0, w1);
                decode(s + 1, Q[(p + 1) & 3], w0, w1);
                if (p == 3) sw0 = w0, sw1 = w1;
            }
            __builtin_amdgcn_sched_barrier(0);
            dma_a(s + 1 < S2 ? s + 1 : s, (s + 1) & 1);
            if (p == 1) dma_s(u_next);  // the min k-step of unit u is behind the previous barrier
            Q[(p + 3) & 3] = load_q(s + 3 < S2 ? s + 3 : S2 - 1);
            if (p == 0) H = load_h(u_next);
            __builtin_amdgcn_sched_barrier(0);
            stage_mfma(s & 1);
            __builtin_amdgcn_sched_barrier(0);
            if (p == 2 && u + 1 < U && half == 0) write_min(H);
            // end of the stage: this wave's LDS writes done, and every load issued before this
            // stage's activation DMA landed, the DMA itself included (those issued after it may stay
            // in flight): the quants of stage s + 2 and, at p = 1, the header of unit u + 1
            if (p == 0) asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)" : "+v"(Q[2])::"memory");
            if (p == 1) asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)" : "+v"(Q[3]), "+v"(H)::"memory");
            if (p == 2) asm volatile("s_waitcnt vmcnt(1) lgkmcnt(0)" : "+v"(Q[0])::"memory");
            if (p == 3) asm volatile("s_waitcnt vmcnt(1) lgkmcnt(0)" : "+v"(Q[1])::"memory");
            bt_barrier();
        }
    }
    // the last stages' (clamped, unused) loads still write their registers: land them first
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(H), "+v"(Q[0]), "+v"(Q[1]), "+v"(Q[2]), "+v"(Q[3])::"memory");

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
