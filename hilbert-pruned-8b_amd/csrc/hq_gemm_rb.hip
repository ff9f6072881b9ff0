// hq_gemm_rb.hip - Q4_K and Q8_0 GEMMs for mid-size M on gfx950 (Q4_K: 33 <= M <= 64; Q8_0:
// 2 <= M <= 64): full-K tiles of up to 64 rows x 64 columns, one per workgroup; where a shape has
// too few tiles for the CUs, each tile's K is split over up to 8 workgroups whose partial tiles are
// added in a fixed order (tile_finish).
//
// C[M,N] (+)= A[M,K] . W^T with A fp16 and W GGUF Q4_K super-blocks resident in HBM (reference
// arithmetic: cleanroom-transformer/src/ggml_quant.h:51-59, :135-150; matmul src/cpu_backend.c:38-54).
//
// A workgroup holds PIPE independent pipelines of four waves (PIPE = 2: one wave of each per SIMD);
// pipeline kh takes the super-blocks u = kh, kh + PIPE, ... of K, so one pipeline's LDS and memory
// latency is covered by the other's work. In a pipeline, wave w owns all 64 rows and the 16 columns
// 16w .. 16w + 15 of the tile and decodes its own columns' Q4_K bytes from LDS straight into MFMA
// fragments (v_mfma_f32_16x16x32_f16, activations as the first operand, so each lane's four
// accumulators belong to one output column); no decoded B tile is stored. Per pipeline, an LDS ring
// of NSTG 128-K stages (activation tile + the quant bytes of its columns, both LDS-DMA'd, written as
// assembly and waited with explicit s_waitcnt vmcnt) and a ring of super-block slots (the
// activations' sub-block sums in (hi, lo) pair layout, which the waves form from the staged tiles,
// one (row, sub-block) per lane and stage, and the column headers).
//
// Arithmetic as in the full-K tile kernel of hq_gemm_ws.hip: the B operand is the exact integer
// s*q (fp16 1024 + q via v_perm_b32, one v_pk_fma_f16 with (s, -1024 s) or (s/16, -64 s)); a
// column's accumulators are in units of c_u = d_u (1 where d_u = 0) during super-block u and are
// rescaled by c_{u'} / c_u when the pipeline moves on (u' its previous super-block), then by its
// last c; the min term -dmin * sum_sub m_sub * S_sub is one bf16 MFMA per row block and super-block
// whose k slots pair (S hi, S lo, S hi, S lo) with (x hi, x hi, x lo, x lo), so a lane needs only the
// two sub-blocks of its own lane group. It runs one super-block late (S of u is whole once u's last
// stage is summed): at the start of u's successor u', after the rescale, with x = -dmin_u m_u / c_{u'};
// the last super-block's after the loop, in its own units. Each lane reads its column's 16-byte
// header and forms every per-column value itself (no cross-lane exchange). The two pipelines' tiles
// are added in pipeline order through LDS before the store.
#include <type_traits>

#include "hq_device.h"
#include "hq_kernels.h"

namespace {
struct RbArgs {
    const uint8_t *W;  // Q4_K super-blocks, row n at n * row_bytes
    uint32_t row_bytes;
    const uint16_t *A;  // fp16 [M][K]
    int M, N, K;
    void *C;
    int c_f32, accumulate;
    int mt, nt;  // M-tiles, N-tiles
    // K split (few tiles, long K): each tile's pairs of super-blocks are cut into `parts` ranges,
    // one workgroup each, finished by tile_finish (partials[tile][part], per-tile counters)
    int parts;
    float *partials;
    int *counters;
    int ntiles;
};
}  // namespace

namespace {
constexpr int RB_KS = 128, RB_NT = 256;

template <int NB, int MBK, int NSTG>
struct RbLds {
    static constexpr int BN = 64 * NB;
    static constexpr int BM = 16 * MBK;
    static constexpr int A_BYTES = BM * RB_KS * 2;  // activation stage tile
    static constexpr int B_BYTES = 4 * NB * 1024;      // quant bytes [wave][j][16 cols][64 B]
    static constexpr int STG = A_BYTES + B_BYTES;      // one stage slot (NSTG slots)
    static constexpr int S_BYTES = BM * 32;            // sub-block sums of a super-block
    static constexpr int H_BYTES = BN * 16;            // headers [wave][16 NB cols][16 B]
    static constexpr int SBS = S_BYTES + H_BYTES;      // one super-block slot (NSB slots)
    static constexpr int NSB = NSTG / 2 + 2;
    static constexpr int SB0 = NSTG * STG;
    static constexpr int TOTAL = SB0 + NSB * SBS;
    static_assert(TOTAL <= 160 * 1024, "LDS budget");
    static_assert(BM * (BN + 4) * 4 <= NSTG * STG, "epilogue tile");
};

using rb_lds_h8 = const __attribute__((address_space(3))) h8;
using rb_lds_u4 = const __attribute__((address_space(3))) u4v;
DEV h8 rb_ld8(uint32_t a) { return *(rb_lds_h8 *)(uintptr_t)a; }
DEV u4v rb_ld16(uint32_t a) { return *(rb_lds_u4 *)(uintptr_t)a; }
using rb_lds_u2 = const __attribute__((address_space(3))) u2v;
DEV h8 rb_lds_pairs(uint32_t a) {
    const u2v p = *(rb_lds_u2 *)(uintptr_t)a;
    return __builtin_bit_cast(h8, u4v{p.x, p.x, p.y, p.y});
}
template <int I, int N, class F>
DEV void sfor(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        sfor<I + 1, N>(f);
    }
}
DEV void rb_wait_lgkm() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

template <int NB, int MBK, int NSTG, int PIPE>
__global__ void __launch_bounds__(RB_NT * PIPE) k_gemm_q4_k_rb(RbArgs g) {
    constexpr int BM = 16 * MBK, HG = MBK / 2, D = NSTG - 1;
    constexpr int BN = 64 * NB;
    using L = RbLds<NB, MBK, NSTG>;
    constexpr int NSB = L::NSB;
    static_assert(L::TOTAL % 256 == 0, "arena alignment");
    __shared__ __attribute__((aligned(256))) char lds[L::TOTAL * PIPE];
    const int b = blockIdx.x, x = b & 7, j8 = b >> 3, per = g.mt * g.parts;
    const int nt_i = x + 8 * (j8 / per), part = (j8 % per) / g.mt, mt_i = j8 % g.mt;
    if (nt_i >= g.nt) return;
    const int m0 = mt_i * BM, n0 = nt_i * BN;
    // this part's super-blocks u0 .. u0 + PIPE U - 1 (whole groups of PIPE); the operand bases are
    // moved to u0 (row strides stay K and UT). PIPE independent pipelines of 4 waves; pipeline kh
    // takes the part's super-blocks kh, kh + PIPE, ...
    const int M = g.M, N = g.N, K = g.K, UT = K / 256, GT = UT / PIPE;
    const int g0 = part * GT / g.parts, U = (part + 1) * GT / g.parts - g0, u0 = PIPE * g0, S2 = 2 * U;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3), kh = __builtin_amdgcn_readfirstlane(tid >> 8);
    auto ru = [&](int u) __attribute__((always_inline)) { return PIPE * u + kh; };  // real super-block
    const int ln = lane & 15, lg = lane >> 4;
    const rsrc_t ra = make_rsrc(g.A + (size_t)u0 * 256, (uint32_t)((size_t)M * K * 2 - (size_t)u0 * 512));
    const rsrc_t rw = make_rsrc(g.W + (size_t)u0 * 144, (uint32_t)((size_t)N * g.row_bytes - (size_t)u0 * 144));
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds + (uint32_t)(kh * L::TOTAL);
    const int nw = n0 + 16 * NB * wave;  // the wave's first column
    const uint32_t rb = g.row_bytes;

    // ---- DMA issue (every lane offset holds the row / column part, so rows >= M and columns >= N
    // fall outside the buffer ranges and read zero)
    const int arow = 4 * wave + (lane >> 4);
    const uint32_t a_voff = ((uint32_t)(m0 + arow) * (uint32_t)K + 8u * (uint32_t)((lane & 15) ^ (arow & 15))) * 2u;
    const uint32_t a_qq = 16u * (uint32_t)K * 2u;
    auto dma_a = [&](int s, int qq) __attribute__((always_inline)) {
        dma16_so(ra, lds0 + (uint32_t)((s % NSTG) * L::STG + (wave + 4 * qq) * 1024), a_voff + (uint32_t)qq * a_qq,
                 (uint32_t)((2 * ru(s >> 1) + (s & 1)) * RB_KS * 2));
    };
    uint32_t b_voff[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) b_voff[j] = (uint32_t)(nw + 16 * j + (lane >> 2)) * rb + 16u + 16u * (uint32_t)(lane & 3);
    auto dma_b = [&](int s, int j) __attribute__((always_inline)) {
        dma16_so(rw, lds0 + (uint32_t)((s % NSTG) * L::STG + L::A_BYTES + (wave * NB + j) * 1024), b_voff[j],
                 (uint32_t)(ru(s >> 1) * 144 + 64 * (s & 1)));
    };
    const uint32_t h_voff = (uint32_t)(nw + (lane < 16 * NB ? lane : 0)) * rb;
    auto dma_h = [&](int u) __attribute__((always_inline)) {
        if (lane < 16 * NB)
            dma16_so(rw, lds0 + (uint32_t)(L::SB0 + (u % NSB) * L::SBS + L::S_BYTES + wave * 256 * NB), h_voff,
                     (uint32_t)(ru(u) * 144));
    };

    // ---- operands
    // A fragment of row block i, k-step kk of the stage in slot s % NSTG: row 16i + ln, 16-byte slot
    // p = 8(lg>>1) + 4(kk>>1) + 2(lg&1) + (kk&1) stored at p ^ ln
    const uint32_t a_lane = (uint32_t)(ln * 256) + 16u * (uint32_t)((8 * (lg >> 1) + 2 * (lg & 1)) ^ ln);
    auto a_base = [&](int s, int kk) __attribute__((always_inline)) {
        return (lds0 + (uint32_t)((s % NSTG) * L::STG) + a_lane) ^ (uint32_t)(64 * (kk >> 1) + 16 * (kk & 1));
    };
    // S fragment (min k-step) of row block i: row 16i + ln, the (hi, lo) pairs of sub-blocks 2lg and
    // 2lg + 1, each pair twice
    const uint32_t s_lane = (uint32_t)(ln * 32 + 8 * lg);
    auto s_base = [&](int u) __attribute__((always_inline)) { return lds0 + (uint32_t)(L::SB0 + (u % NSB) * L::SBS) + s_lane; };
    const uint32_t raw_lane = (uint32_t)(L::A_BYTES + wave * NB * 1024 + ln * 64 + lg * 16);
    const uint32_t hdr_lane = (uint32_t)(L::SB0 + L::S_BYTES + wave * 256 * NB + ln * 16);

    f4 acc[MBK][NB];
#pragma unroll
    for (int i = 0; i < MBK; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    h8 fa[MBK], fb[NB], fbn[NB], bm[NB];
    float rr[NB];
    u4v raw[NB], hd[NB];
    uint32_t sws[NB][2], pm[NB][4];
    float cprev[NB], xprev[NB][2];  // c of the previous super-block; -dmin m of its lane sub-blocks
#pragma unroll
    for (int j = 0; j < NB; j++) cprev[j] = 1.0f, xprev[j][0] = xprev[j][1] = 0.0f;

    auto read_hdr = [&](int u) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NB; j++) hd[j] = rb_ld16(lds0 + (uint32_t)((u % NSB) * L::SBS) + hdr_lane + (uint32_t)(j * 256));
    };
    // min-term B fragment of x0, x1 (sub-blocks 2lg, 2lg + 1): (hi, hi), (lo, lo) bf16 pairs, matching
    // the S fragment's (hi, lo), (hi, lo) pairs
    auto min_frag = [&](float x0, float x1) __attribute__((always_inline)) {
        const __bf16 h0 = (__bf16)x0, h1 = (__bf16)x1;
        const __bf16 l0 = (__bf16)(x0 - (float)h0), l1 = (__bf16)(x1 - (float)h1);
        const uint32_t uh0 = __builtin_bit_cast(uint16_t, h0), uh1 = __builtin_bit_cast(uint16_t, h1);
        const uint32_t ul0 = __builtin_bit_cast(uint16_t, l0), ul1 = __builtin_bit_cast(uint16_t, l1);
        return __builtin_bit_cast(h8, u4v{uh0 * 0x10001u, ul0 * 0x10001u, uh1 * 0x10001u, ul1 * 0x10001u});
    };
    // super-block values of column 16j + ln (from hd[j] of super-block u; every lane of the column
    // holds its header): scale words of sub-blocks 0-3 / 4-7 (zero where d = 0), the lane's min-term B
    // fragment of the PREVIOUS super-block in units of c_u (x = -dmin_{u-1} m_{u-1} / c_u: its sums are
    // whole only once its last stage is summed, so its min k-step runs at the start of u, after the
    // rescale), and the column's rescale ratio c_{u-1} / c_u
    auto sb_col = [&](int j) __attribute__((always_inline)) {
        const u4v h = hd[j];
        uint32_t sw0, sw1, mw0, mw1;
        q4k_scale_words(h.y, h.z, h.w, sw0, sw1, mw0, mw1);
        const uint32_t nz = (h.x & 0x7fffu) ? 0xffffffffu : 0u;
        sws[j][0] = sw0 & nz;
        sws[j][1] = sw1 & nz;
        const uint32_t mw = lg < 2 ? mw0 : mw1;
        const float d = h2f((uint16_t)h.x), dmin = h2f((uint16_t)(h.x >> 16));
        const float c = d != 0.0f ? d : 1.0f, inv = 1.0f / c;
        bm[j] = min_frag(xprev[j][0] * inv, xprev[j][1] * inv);
        xprev[j][0] = -dmin * (float)byte_of(mw, 2 * (lg & 1));
        xprev[j][1] = -dmin * (float)byte_of(mw, 2 * (lg & 1) + 1);
        rr[j] = cprev[j] * inv;
        cprev[j] = c;
    };
    // activation sub-block sums (no pass over A before the kernel): in stage s = 2u + h, lane (r, b) of
    // wave w sums row 16w + r (r = lane % 16) of the stage's tile over sub-block b = lane / 16 (fp32,
    // the sum8 order) and stores it as a (hi, lo) bf16 pair in S(u)[row][4h + b] (the slot u % NSB
    // that the min k-step of super-block u + 1 reads)
    static_assert(MBK == 4 && RB_KS == 128, "one (row, sub-block) of the stage per lane of the 4 waves");
    const int srow = 16 * wave + (lane & 15), sblk = lane >> 4;
    u4v sx[4];
    auto sums_rd = [&](int s) __attribute__((always_inline)) {
        const uint32_t base = lds0 + (uint32_t)((s % NSTG) * L::STG + srow * 256);
#pragma unroll
        for (int c = 0; c < 4; c++) sx[c] = rb_ld16(base + (uint32_t)(((4 * sblk + c) ^ (srow & 15)) * 16));
    };
    auto sums_wr = [&](int s) __attribute__((always_inline)) {
        const float v = sum8(sx[3], sum8(sx[2], sum8(sx[1], sum8(sx[0], 0.f))));
        const __bf16 hi = (__bf16)v, lo = (__bf16)(v - (float)hi);
        const uint32_t w = (uint32_t)__builtin_bit_cast(uint16_t, hi) | ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
        *(__attribute__((address_space(3))) uint32_t *)(uintptr_t)(lds0 + (uint32_t)(L::SB0 + ((s >> 1) % NSB) * L::SBS + srow * 32 +
                                                                                     (4 * (s & 1) + sblk) * 4)) = w;
    };
    // main decode parameters of stage half h: the lane's quant group p = 2h + lg/2 covers sub-blocks
    // 2p (low nibbles: s, -1024 s) and 2p + 1 (high nibbles: s/16, -64 s)
    auto make_pm = [&](int h) __attribute__((always_inline)) {
        const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
        const h2 kmul = {(_Float16)1.0f, (_Float16)0.0625f}, kadd = {(_Float16)-1024.0f, (_Float16)-64.0f};
        const uint32_t ssel = (lg >> 1) ? 0x04030402u : 0x04010400u;
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const h2 sp = as_h2(__builtin_amdgcn_perm(0x64646464u, sws[j][h], ssel)) - k1024;
            const h2 mu = sp * kmul, ad = sp * kadd;
            pm[j][0] = __builtin_bit_cast(uint32_t, h2{mu.x, mu.x});
            pm[j][1] = __builtin_bit_cast(uint32_t, h2{ad.x, ad.x});
            pm[j][2] = __builtin_bit_cast(uint32_t, h2{mu.y, mu.y});
            pm[j][3] = __builtin_bit_cast(uint32_t, h2{ad.y, ad.y});
        }
    };
    auto read_raw = [&](int s) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NB; j++) raw[j] = rb_ld16(lds0 + (uint32_t)((s % NSTG) * L::STG) + raw_lane + (uint32_t)(j * 1024));
    };
    auto decode_j = [&](int kk, int j) __attribute__((always_inline)) {
        const u2v q = (kk & 1) ? u2v{raw[j].z, raw[j].w} : u2v{raw[j].x, raw[j].y};
        if (kk >> 1) fbn[j] = decode8<true>(q, as_h2(pm[j][2]), as_h2(pm[j][3]));
        else fbn[j] = decode8<false>(q, as_h2(pm[j][0]), as_h2(pm[j][1]));
    };
    auto mfma_row = [&](int i) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = mfma(fa[i], fb[j], acc[i][j]);
    };
    auto rescale_row = [&](int i) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] *= rr[j];
    };

    // vector-memory items issued in stage s = 2u + h for stage t = s + D (if t < S2): H of super-block
    // t / 2 + 1 when t is even (one super-block early: its values are computed during stage t + 1),
    // then A 0..MBK-1 and B 0..NB-1 of stage t. They are spread over the groups of the stage's first
    // k-steps (h = 0: min k-step and main k-steps 0-1; h = 1: main k-steps 0-1). count_t = the
    // instructions of stage t.
    auto count_t = [&](int t) __attribute__((always_inline)) {
        return t < S2 ? MBK + NB + (((t & 1) == 0 && (t >> 1) + 1 < U) ? 1 : 0) : 0;
    };
    auto issue_at = [&](int u, auto hc, auto fc) __attribute__((always_inline)) {
        constexpr int H = decltype(hc)::value, F = decltype(fc)::value;
        constexpr bool SH = ((H + D) & 1) == 0;
        constexpr int NI = (SH ? 1 : 0) + MBK + NB, G = (H == 0 ? 3 : 2) * MBK;
        static_assert(NI <= G, "issue slots");
        constexpr int n = (F * NI + G - 1) / G;
        if constexpr (n < NI && (n * G) / NI == F) {
            const int t = 2 * u + H + D;
            if (t < S2) {
                constexpr int it = SH ? n : n + 1;  // 0 = H, 1.. = A, then B
                if constexpr (it == 0) {
                    if ((t >> 1) + 1 < U) dma_h((t >> 1) + 1);
                } else if constexpr (it < 1 + MBK) {
                    dma_a(t, it - 1);
                } else {
                    dma_b(t, it - 1 - MBK);
                }
            }
        }
    };
    auto sched_fence = []() __attribute__((always_inline)) { __builtin_amdgcn_sched_barrier(0); };

    // ---- prologue: super-block 0's headers, then stages 0 .. D - 1 as in the main loop
    dma_h(0);
    int n_pro = 0;
    for (int t = 0; t < D && t < S2; t++) {
        if ((t & 1) == 0 && (t >> 1) + 1 < U) dma_h((t >> 1) + 1);
        for (int qq = 0; qq < MBK; qq++) dma_a(t, qq);
#pragma unroll
        for (int j = 0; j < NB; j++) dma_b(t, j);
        n_pro += count_t(t);
    }
    wait_vmcnt(n_pro);  // H(0)
    read_hdr(0);
#pragma unroll
    for (int j = 0; j < NB; j++) sb_col(j);
    make_pm(0);
    wait_vmcnt(n_pro - count_t(0));  // stage 0
    read_raw(0);
#pragma unroll
    for (int j = 0; j < NB; j++) decode_j(0, j);
    rb_wait_lgkm();
    __syncthreads();
    // (super-block 0's min k-step adds the zero term of a super-block -1)
#pragma unroll
    for (int i = 0; i < MBK; i++) fa[i] = h8{};

    // ---- k-steps: 8 groups (row blocks) each, pinned in order by scheduling fences
    // min k-step of super-block u (stage s = 2u): rescale + S x Bmin; reads stage s's kk = 0 A fragments
    auto kmin = [&](auto mode, int u) __attribute__((always_inline)) {
        const int s = 2 * u;
        const uint32_t ab = a_base(s, 0);
        rescale_row(0);
        sched_fence();
        sfor<0, MBK>([&](auto gc) __attribute__((always_inline)) {
            constexpr int i = decltype(gc)::value;
#pragma unroll
            for (int j = 0; j < NB; j++) {
                acc[i][j] = mfma_bf16(fa[i], bm[j], acc[i][j]);
            }
            if constexpr (i + 1 < MBK) rescale_row(i + 1);
            fa[i] = rb_ld8(ab + (uint32_t)(i * 16 * 256));
            issue_at(u, std::integral_constant<int, 0>{}, std::integral_constant<int, i>{});
            sched_fence();
        });
#pragma unroll
        for (int j = 0; j < NB; j++) fb[j] = fbn[j];
    };
    // main k-step kk < 3 of stage s = 2u + h (k = kk + 1): decodes kk + 1's B fragments (block j in
    // group 2j), reads its A fragments; in k-step 2 waits for the previous stage's DMAs (group 5),
    // reads the next stage's quant bytes and receives its decode parameters (group 6). In stage
    // 2u + 1 of a super-block with a successor, k-steps 0-1 compute the next super-block's values.
    auto kmain = [&](auto mode, auto hc, int u, auto kc, auto nvc) __attribute__((always_inline)) {
        constexpr int MODE = decltype(mode)::value, H = decltype(hc)::value, KK = decltype(kc)::value;
        (void)nvc;  // (the call sites still name the register set; the body no longer needs it)
        constexpr bool MORE = !(MODE == 2 && H == 1);
        const int s = 2 * u + H;
        const uint32_t ab = a_base(s, KK + 1);
        sfor<0, MBK>([&](auto gc) __attribute__((always_inline)) {
            constexpr int i = decltype(gc)::value;
            mfma_row(i);
            fa[i] = rb_ld8(ab + (uint32_t)(i * 16 * 256));
            if constexpr ((i & 1) == 0 && (i >> 1) < NB) decode_j(KK + 1, i >> 1);
            if constexpr (KK < 2) issue_at(u, hc, std::integral_constant<int, (H == 0 ? MBK : 0) + MBK * KK + i>{});
            if constexpr (KK == 0 && i == 1) sums_rd(s);
            if constexpr (KK == 1 && i == 0) sums_wr(s);
            if constexpr (H == 1 && MORE) {
                if constexpr (KK == 0 && i == 1) read_hdr(u + 1);
                if constexpr (KK == 0 && i == 3)
#pragma unroll
                    for (int j = 0; j < NB; j++) sb_col(j);
            }
            if constexpr (KK == 2 && i == 0 && MORE) {
                int nv = 0;
#pragma unroll
                for (int t = 2; t <= D; t++) nv += count_t(s + t);
                wait_vmcnt(nv);
                read_raw(s + 1);
            }
            if constexpr (KK == 2 && i == 1 && MORE) make_pm(H == 0 ? 1 : 0);
            sched_fence();
        });
#pragma unroll
        for (int j = 0; j < NB; j++) fb[j] = fbn[j];
    };
    // last k-step of stage s: groups 0-3 (decoding the next stage's first B fragments), the stage
    // hand-off (every wave done with stage s; its DMAs for stage s + 1 landed), the next stage's
    // first A (or S) fragments, groups 4-7
    auto klast = [&](auto mode, auto hc, int u) __attribute__((always_inline)) {
        constexpr int MODE = decltype(mode)::value, H = decltype(hc)::value;
        constexpr bool MORE = !(MODE == 2 && H == 1), NSB = H == 1;
        const int s = 2 * u + H;
        sfor<0, HG>([&](auto gc) __attribute__((always_inline)) {
            constexpr int i = decltype(gc)::value;
            mfma_row(i);
            if constexpr (MORE && i == 1)
#pragma unroll
                for (int j = 0; j < NB; j++) decode_j(0, j);
            sched_fence();
        });
        rb_wait_lgkm();
        __syncthreads();
        uint32_t nb = 0;
        constexpr uint32_t nstep = NSB ? 16u * 32u : 16u * 256u;
        if constexpr (MORE) {
            nb = NSB ? s_base(u) : a_base(s + 1, 0);
#pragma unroll
            for (int i = 0; i < HG; i++) fa[i] = NSB ? rb_lds_pairs(nb + (uint32_t)i * nstep) : rb_ld8(nb + (uint32_t)i * nstep);
        }
        sched_fence();
        sfor<HG, MBK>([&](auto gc) __attribute__((always_inline)) {
            constexpr int i = decltype(gc)::value;
            mfma_row(i);
            if constexpr (MORE) fa[i] = NSB ? rb_lds_pairs(nb + (uint32_t)i * nstep) : rb_ld8(nb + (uint32_t)i * nstep);
            sched_fence();
        });
        if constexpr (MORE && !NSB)
#pragma unroll
            for (int j = 0; j < NB; j++) fb[j] = fbn[j];
    };
    using i0 = std::integral_constant<int, 0>;
    using i1 = std::integral_constant<int, 1>;
    using i2 = std::integral_constant<int, 2>;
    auto sb_body = [&](auto mode, int u) __attribute__((always_inline)) {
        constexpr int MODE = decltype(mode)::value;
        using nv0 = std::integral_constant<int, MODE == 0 ? 2 + MBK + NB : MODE == 1 ? MBK + NB : 0>;
        using nv1 = std::integral_constant<int, MODE == 2 ? 0 : MBK + NB>;
        kmin(mode, u);
        kmain(mode, i0{}, u, i0{}, nv0{});
        kmain(mode, i0{}, u, i1{}, nv0{});
        kmain(mode, i0{}, u, i2{}, nv0{});
        klast(mode, i0{}, u);
        kmain(mode, i1{}, u, i0{}, nv1{});
        kmain(mode, i1{}, u, i1{}, nv1{});
        kmain(mode, i1{}, u, i2{}, nv1{});
        klast(mode, i1{}, u);
    };
    int u = 0;
    for (; u + 2 < U; u++) sb_body(std::integral_constant<int, 0>{}, u);
    if (U >= 2) sb_body(std::integral_constant<int, 1>{}, U - 2);
    sb_body(std::integral_constant<int, 2>{}, U - 1);

    // the last super-block's min k-step, in its own units (its sums were whole at the last hand-off)
    {
        const uint32_t sb = s_base(U - 1);
#pragma unroll
        for (int i = 0; i < MBK; i++) fa[i] = rb_lds_pairs(sb + (uint32_t)(i * 16 * 32));
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const float inv = 1.0f / cprev[j];
            bm[j] = min_frag(xprev[j][0] * inv, xprev[j][1] * inv);
        }
#pragma unroll
        for (int i = 0; i < MBK; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) acc[i][j] = mfma_bf16(fa[i], bm[j], acc[i][j]);
    }
    // back to true units: x c of the last super-block (the lane's column of each block)
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
        for (int i = 0; i < MBK; i++) acc[i][j] *= cprev[j];
    // epilogue through LDS (the stage slots are free: every wave passed the last barrier). With two
    // pipelines, the odd super-blocks' tile is parked first and added to the even ones' (fixed order).
    constexpr int LD = BN + 4;
    auto tile_at = [&](int i, int j, int e) __attribute__((always_inline)) {
        const int r = 16 * i + 4 * lg + e, c = 16 * NB * wave + 16 * j + ln;
        return (float *)(lds + (r * LD + c) * 4);
    };
    if constexpr (PIPE == 2) {
        if (kh == 1)
#pragma unroll
            for (int i = 0; i < MBK; i++)
#pragma unroll
                for (int j = 0; j < NB; j++)
#pragma unroll
                    for (int e = 0; e < 4; e++) *tile_at(i, j, e) = acc[i][j][e];
        rb_wait_lgkm();
        __syncthreads();
    }
    if (kh == 0)
#pragma unroll
        for (int i = 0; i < MBK; i++)
#pragma unroll
            for (int j = 0; j < NB; j++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float *t = tile_at(i, j, e);
                    *t = PIPE == 2 ? acc[i][j][e] + *t : acc[i][j][e];
                }
    rb_wait_lgkm();
    __syncthreads();
    tile_finish<BM, BN, RB_NT * PIPE, 8>(lds, g, m0, n0, nt_i * g.mt + mt_i, part,
                                        (int *)(lds + L::TOTAL * PIPE - 16));
}
}  // namespace


int hq_rb_fits(int M, int K) { return M > 32 && M <= 64 && K % 512 == 0 && (size_t)M * K * 2 < ((size_t)1 << 32); }

// Workgroups per 64 x 64 tile for the mid-M Q4_K kernel, or 0 where the narrow kernel serves better:
// one when the tiles alone number >= n_cu / 2 (N >= 8192 on 256 CUs), else the most parts (<= 8,
// >= 2 super-block pairs each) that keep one round, when they reach >= n_cu / 2 workgroups
int hq_rb_parts(int M, int N, int K, int n_cu) {
    if (!hq_rb_fits(M, K) || (size_t)N * (K / 256) * 144 >= ((size_t)1 << 32)) return 0;
    const int tiles = (N + 63) / 64, pairs = K / 512;
    if (2 * tiles >= n_cu) return 1;
    for (int p = 8; p >= 2; p--)
        if (tiles * p <= n_cu && 2 * tiles * p >= n_cu && pairs >= 2 * p) return p;
    return 0;
}

hipError_t hq_launch_gemm_rb(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32,
                             int accumulate, int parts, float *partials, int *counters, hipStream_t st) {
    if (W->type != HQ_TYPE_Q4_K || !hq_rb_fits(M, (int)W->cols)) return hipErrorInvalidValue;
    if (parts < 1 || parts > 8 || (parts > 1 && (4 * parts > (int)W->cols / 256 || !partials || !counters)))
        return hipErrorInvalidValue;
    RbArgs g;
    g.W = W->qs, g.row_bytes = (uint32_t)W->row_bytes, g.A = A;
    g.M = M, g.N = (int)W->rows, g.K = (int)W->cols, g.C = C, g.c_f32 = c_f32, g.accumulate = accumulate;
    g.mt = 1;
    g.nt = (g.N + 63) / 64;
    g.parts = parts, g.partials = partials, g.counters = counters, g.ntiles = g.nt;
    if ((size_t)W->rows * W->row_bytes >= ((size_t)1 << 32)) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)(8 * ((g.nt + 7) / 8) * parts);
    k_gemm_q4_k_rb<1, 4, 3, 2><<<grid, 2 * RB_NT, 0, st>>>(g);
    return hipGetLastError();
}

// ============================================================================ Q8_0, mid M
// The same structure for Q8_0 (M <= 64; N >= 8192, or a K split as for Q4_K): 16 MBK x 64 tiles, PIPE pipelines of
// four waves taking 128-wide stages kh, kh + PIPE, ...; wave w decodes columns 16w .. 16w + 15. No
// min term and no rescale: the B operand is fp16(q * d), one rounding of the exact weight (as in the
// other Q8_0 kernels), from the biased byte u = q + 128 (fp16 1024 + u by v_perm_b32, minus 1152).
// Per stage and pipeline, LDS holds the activation tile (rows of 256 B, 16-byte slot p of row r at
// p ^ (r & 15)), the quant bytes of the wave's 16 columns (16-byte chunk c of column n at chunk
// c ^ (n & 7)) and their scales (4 per column).
namespace {
struct Rb8Args {
    const uint8_t *Q;   // quant plane [N][K], bytes u = q + 128
    const uint16_t *D;  // fp16 scale plane [N][ldd]
    int ldd;
    const uint16_t *A;  // fp16 [M][K]
    int M, N, K;
    void *C;
    int c_f32, accumulate;
    int nt;  // N-tiles
    int parts;  // K split as for the Q4_K kernel (groups of PIPE stages)
    float *partials;
    int *counters;
    int ntiles;
};

template <int MBK, int NSTG>
struct Rb8Lds {
    static constexpr int BM = 16 * MBK;
    static constexpr int A_BYTES = BM * RB_KS * 2;
    static constexpr int Q_BYTES = 4 * 16 * RB_KS;  // [wave][16 cols][128 B]
    static constexpr int D_BYTES = 4 * 16 * 16;     // [wave][16 cols][16 B] (scales of 2 stages; 4 used)
    static constexpr int STG = A_BYTES + Q_BYTES + D_BYTES;
    static constexpr int TOTAL = NSTG * STG;
    static_assert(TOTAL % 256 == 0, "arena alignment");
    static_assert(BM * 68 * 4 <= TOTAL, "epilogue tile");
};

// 8 fp16 B values fp16(q * d) from 8 stored bytes u = q + 128
DEV h8 decode8_q8_0(u2v w, h2 d2) {
    const h2 k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
    const h2 v0 = (as_h2(perm_lo(w.x)) - k1152) * d2, v1 = (as_h2(perm_hi(w.x)) - k1152) * d2;
    const h2 v2 = (as_h2(perm_lo(w.y)) - k1152) * d2, v3 = (as_h2(perm_hi(w.y)) - k1152) * d2;
    return h8{v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
}

using rb_lds_u2v = const __attribute__((address_space(3))) u2v;
DEV u2v rb_ld64(uint32_t a) { return *(rb_lds_u2v *)(uintptr_t)a; }

template <int MBK, int NSTG, int PIPE>
__global__ void __launch_bounds__(RB_NT * PIPE) k_gemm_q8_0_rb(Rb8Args g) {
    constexpr int BM = 16 * MBK, BN = 64;
    using L = Rb8Lds<MBK, NSTG>;
    __shared__ __attribute__((aligned(256))) char lds[L::TOTAL * PIPE];
    const int b = blockIdx.x, j8 = b >> 3, nt_i = (b & 7) + 8 * (j8 / g.parts), part = j8 % g.parts;
    if (nt_i >= g.nt) return;
    const int n0 = nt_i * BN;
    // this part's stages s0 .. s0 + PIPE S2 - 1 (whole groups of PIPE); operand bases moved to s0
    const int M = g.M, N = g.N, K = g.K, GT = K / RB_KS / PIPE;
    const int g0 = part * GT / g.parts, S2 = (part + 1) * GT / g.parts - g0, s0 = PIPE * g0;
    const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3), kh = __builtin_amdgcn_readfirstlane(tid >> 8);
    auto rs = [&](int s) __attribute__((always_inline)) { return PIPE * s + kh; };  // real stage
    const rsrc_t ra = make_rsrc(g.A + (size_t)s0 * RB_KS, (uint32_t)((size_t)M * K * 2 - (size_t)s0 * RB_KS * 2));
    const rsrc_t rq = make_rsrc(g.Q + (size_t)s0 * RB_KS, (uint32_t)((size_t)N * K - (size_t)s0 * RB_KS));
    const rsrc_t rd = make_rsrc(g.D + (size_t)s0 * 4, (uint32_t)((size_t)N * g.ldd * 2 - (size_t)s0 * 8));
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds + (uint32_t)(kh * L::TOTAL);
    const int nw = n0 + 16 * wave;

    // DMAs of stage s (MBK + 3 per wave): activation rows 4(wave + 4qq) .. + 3 (1 KB each); quant
    // bytes of columns nw + 8h .. + 7 (lane l: column l / 8, LDS chunk l % 8 <- global chunk
    // (l % 8) ^ (column & 7)); the 16 columns' scales (16 lanes, 16 bytes from the stage's first)
    const int arow = 4 * wave + (lane >> 4);
    const uint32_t a_voff = ((uint32_t)arow * (uint32_t)K + 8u * (uint32_t)((lane & 15) ^ (arow & 15))) * 2u;
    const uint32_t a_qq = 16u * (uint32_t)K * 2u;
    uint32_t q_voff[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int c = 8 * h + (lane >> 3);
        q_voff[h] = (uint32_t)(nw + c) * (uint32_t)K + 16u * (uint32_t)((lane & 7) ^ (c & 7));
    }
    const uint32_t d_voff = (uint32_t)(nw + (lane & 15)) * (uint32_t)g.ldd * 2u;
    auto slot = [&](int s) __attribute__((always_inline)) { return lds0 + (uint32_t)((s % NSTG) * L::STG); };
    auto issue_stage = [&](int s) __attribute__((always_inline)) {
        const uint32_t sl = slot(s);
        for (int qq = 0; qq < MBK; qq++)
            dma16_so(ra, sl + (uint32_t)((wave + 4 * qq) * 1024), a_voff + (uint32_t)qq * a_qq, (uint32_t)(rs(s) * RB_KS * 2));
#pragma unroll
        for (int h = 0; h < 2; h++)
            dma16_so(rq, sl + (uint32_t)(L::A_BYTES + wave * 2048 + h * 1024), q_voff[h], (uint32_t)(rs(s) * RB_KS));
        if (lane < 16)
            dma16_so(rd, sl + (uint32_t)(L::A_BYTES + L::Q_BYTES + wave * 256), d_voff, (uint32_t)(rs(s) * 8));
    };
    constexpr int NI = MBK + 3;

    // operand addresses: A fragment i of k-step kk: row 16i + ln, slot (4kk + lg) ^ ln; quant bytes of
    // k-step kk: column ln, bytes 32kk + 8lg .. + 7 (chunk 2kk + lg/2, stored at chunk ^ (ln & 7))
    const uint32_t a_lane = (uint32_t)(ln * 256) + 16u * (uint32_t)(lg ^ ln);
    const uint32_t q_lane = (uint32_t)(L::A_BYTES + wave * 2048 + ln * RB_KS + 8 * (lg & 1));
    const uint32_t d_lane = (uint32_t)(L::A_BYTES + L::Q_BYTES + wave * 256 + ln * 16);

    f4 acc[MBK];
#pragma unroll
    for (int i = 0; i < MBK; i++) acc[i] = f4{0.f, 0.f, 0.f, 0.f};

    for (int s = 0; s < NSTG - 1 && s < S2; s++) issue_stage(s);
    for (int s = 0; s < S2; s++) {
        // this wave's DMAs of stage s have landed (those of the later stages issued so far may not)
        const int later = (s + NSTG - 2 < S2 - 1 ? s + NSTG - 2 : S2 - 1) - s;
        wait_vmcnt(NI * later);
        rb_wait_lgkm();
        __syncthreads();  // every wave's stage-s DMAs landed; every wave done with stage s - 1
        if (s + NSTG - 1 < S2) issue_stage(s + NSTG - 1);
        const uint32_t sl = slot(s);
        const u2v dd = rb_ld64(sl + d_lane);  // the column's 4 block scales of the stage
        h8 fa[4][MBK], fb[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
#pragma unroll
            for (int i = 0; i < MBK; i++) fa[kk][i] = rb_ld8(sl + (uint32_t)(i * 16 * 256) + (a_lane ^ (uint32_t)(64 * kk)));
            const uint32_t chunk = (uint32_t)(2 * kk + (lg >> 1)) ^ (uint32_t)(ln & 7);
            const u2v w = rb_ld64(sl + q_lane + 16u * chunk);
            const uint32_t dw = (kk & 2) ? dd.y : dd.x;
            const uint16_t dh = (uint16_t)((kk & 1) ? (dw >> 16) : (dw & 0xffffu));
            const _Float16 d = __builtin_bit_cast(_Float16, dh);
            fb[kk] = decode8_q8_0(w, h2{d, d});
        }
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int i = 0; i < MBK; i++) acc[i] = mfma(fa[kk][i], fb[kk], acc[i]);
    }

    // epilogue: pipeline 1's tile is parked in LDS and added to pipeline 0's (fixed order); the
    // lane's accumulators are rows 16i + 4lg + e of column 16 wave + ln
    constexpr int LD = BN + 4;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    rb_wait_lgkm();
    __syncthreads();
    auto tile_at = [&](int i, int e) __attribute__((always_inline)) {
        return (float *)(lds + ((16 * i + 4 * lg + e) * LD + 16 * wave + ln) * 4);
    };
    if constexpr (PIPE == 2) {
        if (kh == 1)
#pragma unroll
            for (int i = 0; i < MBK; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) *tile_at(i, e) = acc[i][e];
        rb_wait_lgkm();
        __syncthreads();
    }
    if (kh == 0)
#pragma unroll
        for (int i = 0; i < MBK; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float *t = tile_at(i, e);
                *t = PIPE == 2 ? acc[i][e] + *t : acc[i][e];
            }
    rb_wait_lgkm();
    __syncthreads();
    tile_finish<BM, BN, RB_NT * PIPE, 8>(lds, g, 0, n0, nt_i, part, (int *)(lds + L::TOTAL * PIPE - 16));
}
}  // namespace

// Workgroups per tile of the mid-M Q8_0 kernel (2 <= M <= 64, K a multiple of 256), or 0: one when
// the tiles number >= n_cu / 2 (N >= 8192 on 256 CUs), else the most parts (<= 8, >= 2 pairs of
// 128-wide stages each) that keep one round and reach >= n_cu / 2 workgroups
int hq_rb8_parts(int M, int N, int K, int n_cu) {
    if (M < 2 || M > 64 || K % 256 || (size_t)64 * K * 2 >= ((size_t)1 << 32) || ((size_t)N + 64) * K >= ((size_t)1 << 32))
        return 0;
    const int tiles = (N + 63) / 64, groups = K / 256;
    if (2 * tiles >= n_cu) return 1;
    for (int p = 8; p >= 2; p--)
        if (tiles * p <= n_cu && 2 * tiles * p >= n_cu && groups >= 2 * p) return p;
    return 0;
}

hipError_t hq_launch_gemm_rb8(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                              int parts, float *partials, int *counters, hipStream_t st) {
    if (W->type != HQ_TYPE_Q8_0 || M < 2 || M > 64 || W->cols % 256) return hipErrorInvalidValue;
    if (parts < 1 || parts > 8 || (parts > 1 && (2 * parts > (int)W->cols / 256 || !partials || !counters)))
        return hipErrorInvalidValue;
    if ((size_t)64 * W->cols * 2 >= ((size_t)1 << 32) || ((size_t)W->rows + 64) * W->cols >= ((size_t)1 << 32))
        return hipErrorInvalidValue;
    Rb8Args g;
    g.Q = W->qs, g.D = W->d, g.ldd = W->ldd, g.A = A;
    g.M = M, g.N = (int)W->rows, g.K = (int)W->cols, g.C = C, g.c_f32 = c_f32, g.accumulate = accumulate;
    g.nt = (g.N + 63) / 64;
    g.parts = parts, g.partials = partials, g.counters = counters, g.ntiles = g.nt;
    const unsigned grid = (unsigned)(8 * ((g.nt + 7) / 8) * parts);
    if (M <= 16) k_gemm_q8_0_rb<1, 3, 2><<<grid, 2 * RB_NT, 0, st>>>(g);
    else if (M <= 32) k_gemm_q8_0_rb<2, 3, 2><<<grid, 2 * RB_NT, 0, st>>>(g);
    else k_gemm_q8_0_rb<4, 3, 2><<<grid, 2 * RB_NT, 0, st>>>(g);
    return hipGetLastError();
}
