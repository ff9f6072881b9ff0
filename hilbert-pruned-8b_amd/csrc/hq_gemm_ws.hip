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
// Exactness (no weight is ever rounded to 16 bits). The B operand is the integer s*q (<= 945, exact
// in fp16). A super-block's products accumulate in fp32 (part), which is folded into the output
// accumulator as acc += d * part once per super-block. The min term -dmin * sum_sub m_sub * S_sub
// (S_sub = fp32 sum of the sub-block's 32 activations, from k_asums as fp16 hi + lo) is one MFMA per
// (row block, column block, super-block) accumulating into acc: A slots hold S_hi, S_lo, S_hi, S_lo
// of the 8 sub-blocks, B slots Bh, Bh, Bl, Bl with Bh = fp16(-dmin*m), Bl = fp16(-dmin*m - Bh)
// (exact: -dmin*m has at most 17 significant bits), so the four products sum to S * (-dmin*m) to
// about 2^-22 relative.
//
// LDS layouts (16-byte slots; a stage row is 128 k = 16 slots):
//   A tile [128 rows][16 slots], slot p of row r at p ^ (r & 15);
//   B tile [BN columns][16 slots], slot p of column c at p ^ (c & 15);
//   (the XOR swizzle makes the 16 lanes of an MFMA operand read hit 16 distinct slots: such reads run
//   at the full 256 bytes per clock)
//   S [128 rows][16 halves] = hi[8], lo[8]; Bmin [BN][16 halves] = Bh[8], Bl[8]; D [BN] fp16 d.
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
    const uint16_t *S;  // activation sub-block sums [M][K/256][16] (k_asums)
    int M, N, K;
    void *C;
    int c_f32, accumulate;
    int mt, nt;  // M-tiles, N-tiles
};

// Workgroup barrier without a memory fence: each role waits for exactly the memory operations the
// hand-off needs (explicit s_waitcnt before the call). A __syncthreads() fence would make the
// producers wait for every outstanding load, including weight loads meant for later stages.
DEV void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

DEV u2v buf_load8(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

DEV void dma16(rsrc_t r, void *lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_ptr(lds), 16, voff, soff, 0, 0);
}

// Eight fp16 B values s*q for 8 consecutive k from the low (HI = false) or high nibbles of 8 bytes:
// masked bytes under 0x64 are fp16 1024 + q (or 1024 + 16q); one fma with (s, -1024 s) (or
// (s/16, -64 s)) gives the exact integer.
template <bool HI>
DEV h8 decode8(u2v q, h2 mul, h2 add) {
    const uint32_t mask = HI ? 0xf0f0f0f0u : 0x0f0f0f0fu;
    const uint32_t w0 = q.x & mask, w1 = q.y & mask;
    const h2 v0 = __builtin_elementwise_fma(as_h2(perm_lo(w0)), mul, add);
    const h2 v1 = __builtin_elementwise_fma(as_h2(perm_hi(w0)), mul, add);
    const h2 v2 = __builtin_elementwise_fma(as_h2(perm_lo(w1)), mul, add);
    const h2 v3 = __builtin_elementwise_fma(as_h2(perm_hi(w1)), mul, add);
    return h8{v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
}

// Output block (i, j) of a consumer wave: lane (ln, lg) holds C[r0 + 16i + ln][c0 + 16j + 4lg + e]
// in register e. Stored as one 8-byte (fp16) or 16-byte (fp32) access when the 4 columns lie inside
// C and are aligned for it (N % 4 == 0 and C aligned to the access), else element by element (same
// values and roundings either way).
template <int MB, int NB>
DEV void store_rows4(void *C, const f4 (&acc)[MB][NB], int M, int N, int r0, int c0, int ln, int lg, int c_f32,
                     int accumulate) {
    const bool wide = (N & 3) == 0 && ((uintptr_t)C & (c_f32 ? 15u : 7u)) == 0;
#pragma unroll
    for (int i = 0; i < MB; i++) {
        const int m = r0 + 16 * i + ln;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int n = c0 + 16 * j + 4 * lg;
            if (n >= N) continue;
            const f4 y = acc[i][j];
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
}

// LDS arena (bytes): A stages, B stages, S, Bmin, D.
template <int NB>
struct WsLds {
    static constexpr int BN = 32 * NB;
    static constexpr int A = 0, A_BYTES = WS_BM * WS_KS * 2;  // per stage buffer
    static constexpr int B = 2 * A_BYTES, B_BYTES = BN * WS_KS * 2;
    static constexpr int S = B + 2 * B_BYTES;
    static constexpr int BM = S + WS_BM * 32;
    static constexpr int D = BM + BN * 32;
    static constexpr int TOTAL = D + BN * 2;
    static_assert(TOTAL <= 160 * 1024, "LDS budget");
};

template <int NB>
__global__ void __launch_bounds__(WS_NT) k_gemm_q4_k_ws(WsArgs g) {
    constexpr int BN = 32 * NB;
    using L = WsLds<NB>;
    __shared__ __attribute__((aligned(16))) char lds[L::TOTAL];
    _Float16 *const sA0 = (_Float16 *)(lds + L::A);
    _Float16 *const sB0 = (_Float16 *)(lds + L::B);
    uint16_t *const sS = (uint16_t *)(lds + L::S);
    uint16_t *const sBm = (uint16_t *)(lds + L::BM);
    uint16_t *const sD = (uint16_t *)(lds + L::D);
    auto sA = [&](int h) { return sA0 + h * (L::A_BYTES / 2); };
    auto sB = [&](int h) { return sB0 + h * (L::B_BYTES / 2); };

    // tile of this workgroup: XCD x = b % 8 takes N-tiles x, x + 8, ...; its slots run over the
    // M-tiles of one N-tile first
    const int b = blockIdx.x, x = b & 7, j8 = b >> 3;
    const int nt_i = x + 8 * (j8 / g.mt), mt_i = j8 % g.mt;
    if (nt_i >= g.nt) return;
    const int m0 = mt_i * WS_BM, n0 = nt_i * BN;
    const int M = g.M, N = g.N, K = g.K, U = K / 256;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const rsrc_t ra = make_rsrc(g.A, (uint32_t)((size_t)M * K * 2));
    const rsrc_t rw = make_rsrc(g.W, (uint32_t)((size_t)N * g.row_bytes));

    if (wave >= 4) {
        // ------------------------------------------------------------------ producers
        const int pt = tid - 256, pw = wave - 4, xi = pt & 7;
        const rsrc_t rs = make_rsrc(g.S, (uint32_t)((size_t)M * U * 32));
        // activation DMA: instruction qq of wave pw fills rows 4(pw + 4qq) .. +4 (1 KB); lane l takes
        // row 4(pw + 4qq) + l/16, LDS slot l % 16, global chunk (l % 16) ^ (row & 15)
        const int arow = 4 * pw + (lane >> 4);
        const uint32_t a_voff = (uint32_t)(((m0 + arow) * K + 8 * ((lane & 15) ^ (arow & 15))) * 2);
        auto dma_a = [&](int s) {
            _Float16 *dst = sA(s & 1);
#pragma unroll
            for (int qq = 0; qq < 8; qq++)
                dma16(ra, dst + (pw + 4 * qq) * 512, a_voff, (uint32_t)(qq * 16 * K * 2 + s * WS_KS * 2));
        };
        // S tile of unit u: 32 rows (1 KB) per wave; lane l: row 32pw + l/2, half l % 2
        const uint32_t s_voff = (uint32_t)(((m0 + 32 * pw + (lane >> 1)) * U) * 32 + 16 * (lane & 1));
        auto dma_s = [&](int u) { dma16(rs, sS + pw * 512, s_voff, (uint32_t)(u * 32)); };
        // weight bytes: this thread's columns c_i = pt/8 + 32i (i < NB), half-chunk xi of each stage
        uint32_t w_voff[NB];
#pragma unroll
        for (int i = 0; i < NB; i++) w_voff[i] = (uint32_t)(n0 + (pt >> 3) + 32 * i) * g.row_bytes;
        // Register sets with compile-time roles (no dynamic indexing): Hc = header of the current unit,
        // Hn = header of the next; Q0 / Q1 = quant half-chunks of the unit's even / odd stage.
        u4v Hc[NB], Hn[NB];
        u2v Q0[NB], Q1[NB];
        // header of column pt (pt < BN) for the min-term operands: current / next unit
        const uint32_t m_voff = (uint32_t)(n0 + (pt < BN ? pt : 0)) * g.row_bytes;
        u4v Mc, Mn;
        auto load_h = [&](u4v (&h)[NB], int u) {
#pragma unroll
            for (int i = 0; i < NB; i++) h[i] = buf_load16(rw, w_voff[i], (uint32_t)(u * 144));
        };
        // half-chunk xi of stage s: bytes 16 + 8(8(s % 2) + xi) of super-block s/2 (the lane part in
        // the vector offset, the stage part in the uniform one)
        const uint32_t q_voff = 16u + 8u * (uint32_t)xi;
        auto load_q = [&](u2v (&q)[NB], int s) {
            const uint32_t so = (uint32_t)((s >> 1) * 144 + 64 * (s & 1));
#pragma unroll
            for (int i = 0; i < NB; i++) q[i] = buf_load8(rw, w_voff[i] + q_voff, so);
        };
        // decode a stage into sB(h) (h = stage parity): half-chunk X = 8h + xi covers sub-blocks 2p
        // (low nibbles) and 2p + 1 (high) with p = 2h + xi/4; its 8 + 8 values sit at stage slots
        // 8(xi/4) + (xi % 4) and that + 4
        const int slot_lo = 8 * (xi >> 2) + (xi & 3);
        const uint32_t ssel = (xi >> 2) ? 0x04030402u : 0x04010400u;  // scale bytes 2(p%2), 2(p%2)+1
        auto decode = [&](const u4v (&hd_)[NB], const u2v (&q)[NB], int h) {
            _Float16 *dst = sB(h);
            const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
            const h2 kmul = {(_Float16)1.0f, (_Float16)0.0625f}, kadd = {(_Float16)-1024.0f, (_Float16)-64.0f};
#pragma unroll
            for (int i = 0; i < NB; i++) {
                const u4v hd = hd_[i];
                uint32_t sw0, sw1, mw0, mw1;
                q4k_scale_words(hd.y, hd.z, hd.w, sw0, sw1, mw0, mw1);
                // sub-block pair p = 2h + xi/4: scales in sw0 (p < 2) or sw1
                const h2 sp = as_h2(__builtin_amdgcn_perm(0x64646464u, h ? sw1 : sw0, ssel)) - k1024;
                const h2 mu = sp * kmul, ad = sp * kadd;
                const h8 lo = decode8<false>(q[i], h2{mu.x, mu.x}, h2{ad.x, ad.x});
                const h8 hi = decode8<true>(q[i], h2{mu.y, mu.y}, h2{ad.y, ad.y});
                const uint32_t c = (uint32_t)((pt >> 3) + 32 * i), sg = c & 15u;
                *(h8 *)(dst + c * WS_KS + 8 * ((uint32_t)slot_lo ^ sg)) = lo;
                *(h8 *)(dst + c * WS_KS + 8 * ((uint32_t)(slot_lo + 4) ^ sg)) = hi;
            }
        };
        // min-term operands and d of a unit, one thread per column (pt < BN, header hm of column pt):
        // Bh = fp16(-dmin * m), Bl = fp16(-dmin * m - Bh) for the 8 sub-blocks, in fp16 pairs
        auto write_min = [&](const u4v hm) {
            if (pt >= BN) return;
            uint32_t sw0, sw1, mw0, mw1;
            q4k_scale_words(hm.y, hm.z, hm.w, sw0, sw1, mw0, mw1);
            const _Float16 ndm = -__builtin_bit_cast(_Float16, (uint16_t)(hm.x >> 16));
            const h2 nd2 = {ndm, ndm};
            const h2 mv[4] = {bytes_f16(mw0, false), bytes_f16(mw0, true), bytes_f16(mw1, false), bytes_f16(mw1, true)};
            h8 bh, bl;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const h2 h = mv[q] * nd2;                                  // one rounding of the exact product
                const h2 l = __builtin_elementwise_fma(mv[q], nd2, -h);    // the remainder
                bh[2 * q] = h.x, bh[2 * q + 1] = h.y;
                bl[2 * q] = l.x, bl[2 * q + 1] = l.y;
            }
            *(h8 *)(sBm + pt * 16) = bh;
            *(h8 *)(sBm + pt * 16 + 8) = bl;
            sD[pt] = (uint16_t)hm.x;
        };
        // A stage ends when this wave's LDS writes are done and the loads the next stage reads from
        // LDS (the activation tile, the S tile) have landed. Vector-memory loads retire in issue
        // order, so those are issued first in every stage and the weight loads for later stages
        // after them; the end-of-stage wait leaves the latter in flight (vmcnt(n) = n newest loads
        // may be outstanding). A weight load issued in stage s is read by the decode in stage s + 1
        // and is waited for by the end of stage s + 1 at the latest: about two stages of latency.
        auto end_stage = [&](auto n_in_flight) {
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(decltype(n_in_flight)::value) : "memory");
            wg_barrier();
        };
        using keep0 = std::integral_constant<int, 0>;
        using keepq = std::integral_constant<int, NB>;
        using keephq = std::integral_constant<int, 2 * NB + 1>;
        // prologue: stage 0 decoded and its activation tile in LDS before the first barrier
        load_h(Hc, 0);
        load_q(Q0, 0);
        Mc = buf_load16(rw, m_voff, 0);
        dma_a(0);
        load_q(Q1, 1);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NB + 8) : "memory");  // Hc, Q0, Mc
        decode(Hc, Q0, 0);
        end_stage(keepq{});  // Q1 may still be in flight
        for (int u = 0; u < U; u++) {
            const bool last = u + 1 == U;
            // stage 2u: activation tile 2u + 1, then the next headers and quants 2u + 2; decode
            // stage 2u + 1
            dma_a(2 * u + 1);
            if (!last) {
                load_h(Hn, u + 1);
                Mn = buf_load16(rw, m_voff, (uint32_t)((u + 1) * 144));
                load_q(Q0, 2 * u + 2);
            }
            decode(Hc, Q1, 1);
            if (!last) end_stage(keephq{});
            else end_stage(keep0{});
            // stage 2u + 1: activation tile 2u + 2 and the S tile of unit u, then quants 2u + 3;
            // decode stage 2u + 2 (next unit), min-term operands of unit u
            if (!last) dma_a(2 * u + 2);
            dma_s(u);
            if (!last) load_q(Q1, 2 * u + 3);
            if (!last) decode(Hn, Q0, 0);
            write_min(Mc);
            if (!last) end_stage(keepq{});
            else end_stage(keep0{});
#pragma unroll
            for (int i = 0; i < NB; i++) Hc[i] = Hn[i];
            Mc = Mn;
        }
        return;
    }

    // ---------------------------------------------------------------------- consumers
    const int wm = wave & 1, wn = wave >> 1, ln = lane & 15, lg = lane >> 4;
    // byte offsets inside a stage buffer: A row 64wm + 16i + ln, B column (BN/2)wn + 16j + ln
    const uint32_t a_row = (uint32_t)((64 * wm + ln) * WS_KS * 2);
    const uint32_t b_col = (uint32_t)(((BN / 2) * wn + ln) * WS_KS * 2);
    auto a_frag = [&](int buf, int i, int f) {
        const char *base = (const char *)sA(buf) + a_row + i * 16 * WS_KS * 2;
        return *(const h8 *)(base + 16 * ((uint32_t)(4 * f + lg) ^ (uint32_t)ln));
    };
    auto b_frag = [&](int buf, int j, int f) {
        const char *base = (const char *)sB(buf) + b_col + j * 16 * WS_KS * 2;
        return *(const h8 *)(base + 16 * ((uint32_t)(4 * f + lg) ^ (uint32_t)ln));
    };
    f4 acc[4][NB], part[4][NB];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    // Fold of the super-block just completed: acc += d * part, then its min-term MFMA. With the
    // weight fragment as the MFMA's first operand, lane (ln, lg) of block (i, j) holds row 16i + ln,
    // columns 16j + 4lg .. + 3 of the wave's tile, so it needs the 4 d values of those columns.
    auto fold = [&]() {
        h8 am[4];
#pragma unroll
        for (int i = 0; i < 4; i++) am[i] = *(const h8 *)(sS + (64 * wm + 16 * i + ln) * 16 + 8 * (lg & 1));
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int c = (BN / 2) * wn + 16 * j;
            const h8 bm = *(const h8 *)(sBm + (c + ln) * 16 + 8 * (lg >> 1));
            const h4 d4 = *(const h4 *)(sD + c + 4 * lg);
            const f4 dv = __builtin_convertvector(d4, f4);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc[i][j] += part[i][j] * dv;
                acc[i][j] = mfma(bm, am[i], acc[i][j]);
            }
        }
    };
    // One stage: 4 k-steps of 32. A fragments of k-step f + 1 are read (into the other register set)
    // before the MFMAs of k-step f; a B fragment is re-read for k-step f + 1 right after its 4 MFMAs
    // of k-step f are issued. The scheduling barriers keep this order (the compiler would otherwise
    // sink each read next to its first use and stall on it). An even stage (the first of a
    // super-block) starts with the previous super-block's fold.
    auto stage = [&](int buf, bool first, bool do_fold) {
        if (do_fold) fold();
        h8 fa[2][4], fb[NB];
#pragma unroll
        for (int i = 0; i < 4; i++) fa[0][i] = a_frag(buf, i, 0);
#pragma unroll
        for (int j = 0; j < NB; j++) fb[j] = b_frag(buf, j, 0);
#pragma unroll
        for (int f = 0; f < 4; f++) {
            const int cur = f & 1;

            if (f < 3) {
#pragma unroll
                for (int i = 0; i < 4; i++) fa[cur ^ 1][i] = a_frag(buf, i, f + 1);
            }
    #pragma unroll
            for (int j = 0; j < NB; j++) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    part[i][j] = mfma(fb[j], fa[cur][i], (f == 0 && first) ? f4{0.f, 0.f, 0.f, 0.f} : part[i][j]);
                if (f < 3) fb[j] = b_frag(buf, j, f + 1);
            }

        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wg_barrier();
    };
    wg_barrier();
    for (int u = 0; u < U; u++) {
        stage(0, true, u > 0);
        stage(1, false, false);
    }
    fold();  // last super-block
    // Output: lane (ln, lg) of block (i, j) holds row 16i + ln, 4 consecutive columns: one 8-byte
    // (fp16) or 16-byte (fp32) store per block when the 4 columns are inside C and aligned.
    store_rows4<4, NB>(g.C, acc, M, N, m0 + 64 * wm, n0 + (BN / 2) * wn, ln, lg, g.c_f32, g.accumulate);
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
                             int accumulate, int nb, hipStream_t st) {
    WsArgs g;
    g.W = W->qs, g.row_bytes = (uint32_t)W->row_bytes, g.A = A, g.S = S;
    g.M = M, g.N = (int)W->rows, g.K = (int)W->cols, g.C = C, g.c_f32 = c_f32, g.accumulate = accumulate;
    g.mt = (M + WS_BM - 1) / WS_BM;
    g.nt = (g.N + 32 * nb - 1) / (32 * nb);
    const unsigned grid = (unsigned)(8 * ((g.nt + 7) / 8) * g.mt);
    switch (nb) {
    case 2: k_gemm_q4_k_ws<2><<<grid, WS_NT, 0, st>>>(g); break;
    case 3: k_gemm_q4_k_ws<3><<<grid, WS_NT, 0, st>>>(g); break;
    case 4: k_gemm_q4_k_ws<4><<<grid, WS_NT, 0, st>>>(g); break;
    case 5: k_gemm_q4_k_ws<5><<<grid, WS_NT, 0, st>>>(g); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
