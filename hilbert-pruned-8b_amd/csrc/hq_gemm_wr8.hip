// hq_gemm_wr8.hip - Q8_0 GEMM for prefill shapes (M = 512 at N ~ 10k in one launch; larger M and the
// gate/up pair GEMM with the SwiGLU epilogue as launches of one round each, planned by the caller) on
// gfx950: 128 x 192 output tiles; 4 MFMA waves that each own all 128 rows and 48 columns, and 4
// loader waves.
//
// C[M,N] (+)= A[M,K] . W^T with A fp16 and W GGUF Q8_0 blocks resident in HBM (reference arithmetic:
// cleanroom-transformer/src/ggml_quant.h:42-49; matmul src/cpu_backend.c:38-54).
//
// The shape of k_gemm_q4_k_wr (hq_gemm_wr.hip) for Q8_0, which has neither a min term nor a rescale:
// a weight is q * d with one fp16 scale per 32 values, and the MFMA operand is fp16(q * d) (one
// rounding of the exact product, as in the other Q8_0 kernels). Decoding a lane's 8 values costs 12
// VALU instructions (4 byte permutes into fp16 1024 + u, 4 subtractions of 1152 giving q exactly, 4
// multiplications by d); each decoded fragment feeds the 8 row blocks of the tile: 1.5 instructions
// per MFMA. Measured on gfx950 (one CU, groups of three 16x16x32 MFMAs): two independent VALU
// instructions behind each MFMA cost ~5 clocks per group of 48, but ~2 clocks each while LDS operand
// reads are in flight, as they always are here; six dependent ones bunched behind the last MFMA ~25.
// The activation tile is the only operand the MFMA waves share through LDS; the loader waves issue
// every load as an LDS DMA, so no multiplying wave waits for an address unit. (Two MFMA waves per
// SIMD splitting K, with or without loader waves, hid more of the VALU cost in isolation but were
// slower in this kernel: 32.7 and 35.5 us against 30.2 at M = 512.)
//
// K order. An MFMA sums over its 32 k in any order as long as both operands use the same one: in
// k-step f (0, 1) of a 64-wide stage, lane group lg holds k = 16 lg + 8 f .. + 7 (not 32 f + 8 lg),
// so one 16-byte chunk of a column's 64 stage bytes (chunk lg) holds the lane's quants of both k-steps
// and the activation fragment is 16-byte chunk 2 lg + f of the row. The lane's k then lie in Q8_0
// block lg / 2 of the stage in both k-steps: one scale per lane and stage.
//
// Pipeline as k_gemm_q4_k_wr: stages of 64 k, 16 groups of 3 MFMAs per stage (k-step g / 8, row block
// g % 8); the activation read 3 groups ahead; half a weight fragment decoded per group, two
// instructions behind each MFMA (k-step 1 in groups 0 .. 5, the next stage's k-step 0 in groups
// 9 .. 14); one s_barrier per stage, in group 6, after which the loaders fill ring slot s + 2 and the
// MFMA waves read the next stage's quant chunks and scales.
//
// LDS (118 KB): A [4][128 rows][64 k] fp16 (16-byte chunk p of row r at p ^ ((r >> 1) & 7));
// quants [4][12 column blocks][64 slots of 16 B] (slot 4c + (h ^ ((c >> 2) & 3)) holds chunk h of
// column c of the block: a block's 64 lanes read 64 distinct 16-byte slots, 16 of them per 256-byte
// bank cycle); scales [2][192 columns][8 fp16] (the 8 blocks of a 256-wide super-stage).
#include "hq_device.h"
#include "hq_kernels.h"

namespace {
constexpr int W8_BM = 128, W8_KS = 64, W8_NT = 512, W8_RING = 4, W8_NB = 3;
constexpr int W8_AD = 3, W8_AF = 4;  // activation read-ahead in groups, ring of fragments
static_assert(W8_AD < W8_AF && 16 - W8_AD > 6 && 16 % W8_AF == 0, "activation read-ahead");

struct Wr8Args {
    const uint8_t *Q;   // quant plane, bytes u = q + 128, row n at n * K
    const uint16_t *D;  // fp16 scale plane, row n at n * ldd
    int ldd;
    const uint16_t *A;  // fp16 [M][K]
    int M, N, K;
    void *C;
    int c_f32, accumulate;
    int mt, nt0, nt;  // M-tiles; this launch's column tiles nt0 .. nt - 1
};

struct Wr8Lds {
    static constexpr int BN = 64 * W8_NB, WC = 16 * W8_NB, CB = BN / 16;  // tile columns, per MFMA wave, column blocks
    static constexpr int A = 0, A_BYTES = W8_BM * W8_KS * 2;                // per ring slot
    static constexpr int Q = W8_RING * A_BYTES, Q_BYTES = CB * 1024;        // per ring slot
    static constexpr int D = Q + W8_RING * Q_BYTES, D_BYTES = BN * 16;      // per super-stage parity
    static constexpr int TOTAL = D + 2 * D_BYTES;
    static_assert(TOTAL <= 160 * 1024, "LDS budget");
};

DEV void w8_barrier() { asm volatile("s_barrier" ::: "memory"); }
// the store phase of an fp16 output tile staged in LDS (tile_store_rows)
DEV void w8_store(const char *lds, const Wr8Args &g, int m0, int n0, int tid) {
    constexpr int BN = Wr8Lds::BN;
    static_assert(W8_BM * tile_ldr<BN * 2>() <= Wr8Lds::TOTAL, "output tile in LDS");
    const uint32_t pitch = (uint32_t)g.N * 2u;
    tile_store_rows<W8_BM, W8_NT, BN * 2>(lds, (char *)g.C + (size_t)m0 * pitch, min(W8_BM, g.M - m0), pitch, (uint32_t)n0 * 2u,
                                          (uint32_t)min(BN, g.N - n0) * 2u, tid);
}
// a loader wave's wait before a barrier: every LDS DMA but the last n issued
template <int n>
DEV void w8_wait() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory"); }
// keeps a computed operand where it is computed (the compiler would otherwise sink the work to the
// operand's first use)
DEV void w8_pin(h8 &x) { asm volatile("" : "+v"(x)); }
// half hf of a weight operand in C (the prologue's): values 4hf .. 4hf + 3 = fp16(q * d) from quant
// word w (bytes q + 128): fp16(1024 + u) from a byte permute, minus 1152 (q exactly), times d
DEV void w8_dec_half(h8 &b, uint32_t w, int hf, h2 d2) {
    const h2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const h2 v0 = (as_h2(perm_lo(w)) + bias) * d2;
    const h2 v1 = (as_h2(perm_hi(w)) + bias) * d2;
    b[4 * hf] = v0.x, b[4 * hf + 1] = v0.y, b[4 * hf + 2] = v1.x, b[4 * hf + 3] = v1.y;
    w8_pin(b);
}

// The MFMA groups of the main loop are written as assembly so that their instruction order is fixed:
// the compiler places plain arithmetic and MFMAs freely within a basic block (measured: the decode's
// dependent VALU chains bunched behind a group's last MFMA, each instruction then costing its full
// issue time and more). Hazards the compiler cannot see inside the statements: none arise within a
// group (no instruction reads a result of the group's MFMAs; each VALU result is read two
// instructions later); an accumulator is next read by an MFMA 8 groups later; a decoded operand is
// first read by an MFMA at least one group later; only MFMAs read the accumulators until the loop
// ends, after which the caller waits out the last MFMAs' latency (w8_mfma_drain).
//
// group without decode: acc_j += b_j x a, j = 0 .. 2
DEV void w8_grp(f4 &c0, f4 &c1, f4 &c2, const u4v &b0, const u4v &b1, const u4v &b2, const h8 &a) {
    asm volatile(
        "v_mfma_f32_16x16x32_f16 %[c0], %[b0], %[a], %[c0]\n\t"
        "v_mfma_f32_16x16x32_f16 %[c1], %[b1], %[a], %[c1]\n\t"
        "v_mfma_f32_16x16x32_f16 %[c2], %[b2], %[a], %[c2]"
        : [c0] "+v"(c0), [c1] "+v"(c1), [c2] "+v"(c2)
        : [b0] "v"(b0), [b1] "v"(b1), [b2] "v"(b2), [a] "v"(a));
}
// group with half a decode: the same MFMAs, each followed by two independent VALU instructions of
// the decode of quant word w with scale d (the low half of the 32-bit value): two byte permutes into
// fp16 1024 + u, two subtractions of 1152, two multiplications by d (each pair independent, each
// result read two instructions later); the results are dwords o0, o1 of the operand
DEV void w8_grp_dec(f4 &c0, f4 &c1, f4 &c2, const u4v &b0, const u4v &b1, const u4v &b2, const h8 &a, uint32_t w,
                    uint32_t d, uint32_t &o0, uint32_t &o1) {
    uint32_t x0, x1;
    asm volatile(
        "v_mfma_f32_16x16x32_f16 %[c0], %[b0], %[a], %[c0]\n\t"
        "v_perm_b32 %[x0], %[k], %[w], %[slo]\n\t"
        "v_perm_b32 %[x1], %[k], %[w], %[shi]\n\t"
        "v_mfma_f32_16x16x32_f16 %[c1], %[b1], %[a], %[c1]\n\t"
        "v_pk_add_f16 %[x0], %[x0], %[bias]\n\t"
        "v_pk_add_f16 %[x1], %[x1], %[bias]\n\t"
        "v_mfma_f32_16x16x32_f16 %[c2], %[b2], %[a], %[c2]\n\t"
        "v_pk_mul_f16 %[o0], %[x0], %[d] op_sel_hi:[1,0]\n\t"
        "v_pk_mul_f16 %[o1], %[x1], %[d] op_sel_hi:[1,0]"
        : [c0] "+v"(c0), [c1] "+v"(c1), [c2] "+v"(c2), [x0] "=&v"(x0), [x1] "=&v"(x1), [o0] "=&v"(o0), [o1] "=&v"(o1)
        : [b0] "v"(b0), [b1] "v"(b1), [b2] "v"(b2), [a] "v"(a), [w] "v"(w), [d] "v"(d), [k] "s"(0x64646464u),
          [slo] "v"(0x04010400u), [shi] "v"(0x04030402u), [bias] "s"(0xe480e480u));  // (fp16 -1152 = 0xe480)
}
// the latency of the last MFMAs before their accumulators are read by other instructions
DEV void w8_mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

__global__ void __launch_bounds__(W8_NT) k_gemm_q8_0_wr(Wr8Args g) {
    using L = Wr8Lds;
    constexpr int NB = W8_NB, BN = L::BN, WC = L::WC;
    __shared__ __attribute__((aligned(256))) char lds[L::TOTAL];
    // tile: XCD x = b % 8 takes N-tiles x, x + 8, ...; its slots run over the M-tiles of one N-tile
    // first (the weight slab is then fetched once per XCD)
    const int b = blockIdx.x, x = b & 7, j8 = b >> 3;
    const int nt_i = g.nt0 + x + 8 * (j8 / g.mt), mt_i = j8 % g.mt;
    if (nt_i >= g.nt) return;
    const int m0 = mt_i * W8_BM, n0 = nt_i * BN;
    const int M = g.M, N = g.N, K = g.K, U = K / 256, S2 = 4 * U;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, ln = lane & 15,
              lg = lane >> 4;
    // roles: waves 0-3 multiply (wave w: columns 48w .. 48w + 47 of the tile, all 128 rows); waves 4-7
    // load (wave 4 + w: a quarter of the activation tile, column blocks w, w + 4, w + 8 of the quants
    // and, w < 3, a third of the scales)
    const int role = wave >> 2, w4 = wave & 3;
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
    const int wc0 = WC * w4, nw = n0 + wc0;  // first column of MFMA wave w4 (in the tile, in W)

    if (role == 1) {
        // ------------------------------------------------------------------------------ loaders
        // A buffer load checks only its VGPR offset against the buffer's size (the scalar offset is not
        // range-checked), so every row and column index is in the VGPR offset: rows past M and columns
        // past N read zeros, and no load reads past the end of A, the quants or the scales.
        const rsrc_t ra = make_rsrc(g.A, (uint32_t)((size_t)M * K * 2));
        const rsrc_t rq = make_rsrc(g.Q, (uint32_t)((size_t)N * K));
        const rsrc_t rd = make_rsrc(g.D, (uint32_t)((size_t)N * g.ldd * 2));
        // activations of stage s into ring slot buf: instruction q (0..3) fills rows 8(4w + q) .. + 8;
        // lane i: row r = 8(4w + q) + i/8, LDS chunk i % 8, global chunk (i % 8) ^ ((r >> 1) & 7) (the
        // q = 0 chunk ^ 4 for odd q)
        const int a_row0 = 32 * w4 + (lane >> 3);
        const uint32_t a_ch = (uint32_t)((lane & 7) ^ ((a_row0 >> 1) & 7));
        uint32_t a_voff[4];
#pragma unroll
        for (int q = 0; q < 4; q++)
            a_voff[q] = (uint32_t)(m0 + a_row0 + 8 * q) * (uint32_t)K * 2u + 16u * (q & 1 ? a_ch ^ 4u : a_ch);
        // quants of stage s, column block w + 4t: lane i loads chunk (i % 4) ^ ((i >> 4) % 4) of column
        // i / 4 (four lanes read one column's 64 stage bytes) into slot i
        uint32_t q_voff[3];
#pragma unroll
        for (int t = 0; t < 3; t++)
            q_voff[t] = (uint32_t)(n0 + 16 * (w4 + 4 * t) + (lane >> 2)) * (uint32_t)K +
                        16u * (uint32_t)((lane & 3) ^ ((lane >> 4) & 3));
        // scales of super-stage v (8 fp16 of a column), instruction w (w < 3): columns 64w .. + 64
        const uint32_t d_voff = (uint32_t)(n0 + 64 * w4 + lane) * (uint32_t)g.ldd * 2u;
        auto dma_a = [&](int s, int buf) {
#pragma unroll
            for (int q = 0; q < 4; q++)
                dma16_so(ra, lds0 + (uint32_t)(L::A + buf * L::A_BYTES + w4 * 4096 + q * 1024), a_voff[q],
                         (uint32_t)(s * W8_KS * 2));
        };
        auto dma_q = [&](int s, int buf) {
#pragma unroll
            for (int t = 0; t < 3; t++)
                dma16_so(rq, lds0 + (uint32_t)(L::Q + buf * L::Q_BYTES + (w4 + 4 * t) * 1024), q_voff[t],
                         (uint32_t)(s * W8_KS));
        };
        auto dma_d = [&](int v) {
            dma16_so(rd, lds0 + (uint32_t)(L::D + (v & 1) * L::D_BYTES + w4 * 1024), d_voff, (uint32_t)(16 * v));
        };
        // prologue: stage 0 and the scales of super-stage 0, then stage 1 (still in flight at the
        // barrier, as every loader stage's loads are)
        dma_a(0, 0);
        dma_q(0, 0);
        if (w4 < 3) dma_d(0);
        dma_a(S2 > 1 ? 1 : 0, 1);
        dma_q(S2 > 1 ? 1 : 0, 1);
        w8_wait<7>();
        w8_barrier();
        // loader stage s = 4u + p runs between the MFMA waves' barriers of stages s - 1 and s (the
        // prologue's barrier counts as stage -1's): the loads of stage s + 2 (ring slot (s + 2) % 4,
        // last read in stage s - 2) and, at p = 1, the scales of super-stage u + 1 (parity (u + 1) & 1,
        // last read at the barrier of stage 4u - 2; first read at that of stage 4u + 3); then wait for
        // everything but this stage's loads (each load has two stages to land) and meet the MFMA
        // waves at their barrier. Past the end the loads repeat the last stage into free slots.
        for (int u = 0; u < U; u++) {
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const int s = 4 * u + p, ld = (s + 2) & 3, s_src = s + 2 < S2 ? s + 2 : S2 - 1;
                dma_a(s_src, ld);
                dma_q(s_src, ld);
                if (p == 1 && w4 < 3) {
                    dma_d(u + 1 < U ? u + 1 : u);
                    w8_wait<8>();
                } else {
                    w8_wait<7>();
                }
                w8_barrier();
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last (clamped, unused) loads
        if (tile_store_ok(g.c_f32, g.accumulate, g.N, g.C)) {
            // meet the MFMA waves once they are done with the rings and once their tile is in LDS,
            // then store it with them
            w8_barrier();
            w8_barrier();
            w8_store(lds, g, m0, n0, tid);
        }
        return;
    }

    // ---------------------------------------------------------------------------------- MFMA waves
    // activation fragment of row block i, k-step f, ring slot buf: lane (ln, lg) reads row 16i + ln,
    // chunk (2lg + f) ^ ((ln >> 1) & 7)
    const uint32_t a_lane = lds0 + (uint32_t)(L::A + ln * 128) + 16u * ((2u * (uint32_t)lg) ^ (uint32_t)((ln >> 1) & 7));
    auto rd = [&](int buf, int gg) {
        return *(const __attribute__((address_space(3))) h8 *)(uintptr_t)(((a_lane ^ (16u * (uint32_t)(gg >> 3))) +
                                                                           (uint32_t)(buf * L::A_BYTES)) +
                                                                          (uint32_t)((gg & 7) * 16 * 128));
    };
    // quant chunk lg of column 16j + ln of the wave (16 bytes: k-step 0 in words 0, 1, k-step 1 in 2, 3)
    const uint32_t q_lane = lds0 + (uint32_t)(L::Q + 3 * w4 * 1024 + 16 * (4 * ln + (lg ^ ((ln >> 2) & 3))));
    auto rdq = [&](int buf, int j) {
        return *(const __attribute__((address_space(3))) u4v *)(uintptr_t)(q_lane + (uint32_t)(buf * L::Q_BYTES + j * 1024));
    };
    // scale of the lane's Q8_0 block (2p + lg / 2 of the super-stage) for stage p, column block j
    const uint32_t d_lane = lds0 + (uint32_t)(L::D + (wc0 + ln) * 16 + 2 * (lg >> 1));
    auto rdd = [&](int par, int p, int j) {
        return (uint32_t) * (const __attribute__((address_space(3))) uint16_t *)(uintptr_t)(d_lane + (uint32_t)(par * L::D_BYTES +
                                                                                                          j * 16 * 16 + 4 * p));
    };

    f4 acc[8][NB];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    w8_barrier();  // the loaders' prologue
    h8 af[W8_AF];
    u4v b0[NB], b1[NB], qc[NB];
    uint32_t dn[NB];  // the scale of the lane's block, in the low half
#pragma unroll
    for (int k = 0; k < W8_AD; k++) af[k] = rd(0, k);
#pragma unroll
    for (int j = 0; j < NB; j++) {
        qc[j] = rdq(0, j);
        dn[j] = rdd(0, 0, j);
        const _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)dn[j]);
        h8 t;
        w8_dec_half(t, qc[j].x, 0, h2{h, h});
        w8_dec_half(t, qc[j].y, 1, h2{h, h});
        b0[j] = __builtin_bit_cast(u4v, t);
    }
    asm volatile("s_nop 4" ::: "memory");  // (the prologue's VALU results before the first MFMA reads them)

    // main loop: one super-stage (4 stages) per iteration; stage s = 4u + p, ring slot s % 4
    for (int u = 0; u < U; u++) {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int s = 4 * u + p, cur = s & 3, nxt = (s + 1) & 3;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int gg = 0; gg < 16; gg++) {
                // the activation operand W8_AD groups ahead (the next stage's first ones from group
                // 16 - W8_AD, after the barrier)
                if (gg + W8_AD < 16) af[(gg + W8_AD) % W8_AF] = rd(cur, gg + W8_AD);
                else af[(gg + W8_AD) % W8_AF] = rd(nxt, gg + W8_AD - 16);
                f4 *c = acc[gg & 7];
                const u4v *bk = gg < 8 ? b0 : b1;
                const h8 a = af[gg % W8_AF];
                // half a weight fragment per group: this stage's k-step 1 (groups 0 .. 5: quant words 2,
                // 3), the next stage's k-step 0 (groups 9 .. 14: words 0, 1, read after the barrier;
                // b0 is free after group 7)
                uint32_t o0, o1;
                if (gg < 2 * NB) {
                    const int j = gg / 2, hf = gg & 1;
                    w8_grp_dec(c[0], c[1], c[2], bk[0], bk[1], bk[2], a, hf ? qc[j].w : qc[j].z, dn[j], o0, o1);
                    b1[j][2 * hf] = o0, b1[j][2 * hf + 1] = o1;
                } else if (gg >= 9 && gg < 9 + 2 * NB) {
                    const int j = (gg - 9) / 2, hf = (gg - 9) & 1;
                    w8_grp_dec(c[0], c[1], c[2], bk[0], bk[1], bk[2], a, hf ? qc[j].y : qc[j].x, dn[j], o0, o1);
                    b0[j][2 * hf] = o0, b0[j][2 * hf + 1] = o1;
                } else {
                    w8_grp(c[0], c[1], c[2], bk[0], bk[1], bk[2], a);
                }
                if (gg == 6) {
                    // the loaders' wait before the barrier lands the next stage's activations and quants
                    // (and, before stage 4u + 4, its super-stage's scales); after it they refill the slot
                    // of stage s - 1, whose reads have all been consumed (this stage's quants are
                    // decoded, so qc and dn are free)
                    w8_barrier();
                    const int sn = s + 1;
#pragma unroll
                    for (int j = 0; j < NB; j++) qc[j] = rdq(nxt, j), dn[j] = rdd((sn >> 2) & 1, sn & 3, j);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    w8_mfma_drain();
    // fp16 C through LDS (tile_store_rows) where C allows it: the accumulators as fp16 at their rows
    // and columns, then all 8 waves store
    if (tile_store_ok(g.c_f32, g.accumulate, g.N, g.C)) {
        w8_barrier();  // every wave is done with the rings and scales
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) {
                const int row = 16 * i + ln, col = wc0 + 16 * j;
                const f4 v = acc[i][j];
                *(h4 *)(lds + row * tile_ldr<BN * 2>() + (col + 4 * lg) * 2) = h4{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        w8_barrier();
        w8_store(lds, g, m0, n0, tid);
        return;
    }
    // lane (ln, lg) of block (i, j) holds row 16i + ln, columns 16j + 4lg .. + 3 of the wave's columns
    // (one 16-byte fp32 or 8-byte fp16 store; element by element at the matrix edge or where N % 4 or
    // C's alignment does not allow it). Vector stores write through to memory (SC1), measured faster
    // than write-back where every tile stores its whole output at the end.
    if (g.c_f32 == HQ_OUT_SWIGLU) {
        // gate/up pair matrix: C is fp16 [M, N / 2] and takes silu(gate) * up (N a multiple of 16)
        const int Nh = N / 2;
        const rsrc_t ro = make_rsrc(g.C, (uint32_t)((size_t)M * Nh * 2));
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int m = m0 + 16 * i + ln;
#pragma unroll
            for (int j = 0; j < NB; j++) {
                const uint32_t y = swiglu_pair2(acc[i][j], lg);
                const int n = nw + 16 * j;
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
        const int m = m0 + 16 * i + ln;
        if (m >= M) break;
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int n = nw + 16 * j + 4 * lg;
            if (n >= N) continue;
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
}  // namespace

// every byte offset of the kernel (tile rows and columns past the matrix included, C's) fits 32 bits
int hq_wr8_fits(const hq_dev_mat *W, int M) {
    const size_t lim = (size_t)1 << 32, mr = (size_t)M + W8_BM, nr = (size_t)W->rows + 64 * W8_NB;
    return W->type == HQ_TYPE_Q8_0 && W->cols % 256 == 0 && W->ldd % 8 == 0 && M >= 1 && mr * W->cols * 2 < lim &&
           (size_t)M * W->rows * 4 < lim && nr * W->cols < lim && nr * (size_t)W->ldd * 2 < lim;
}

hipError_t hq_launch_gemm_wr8(const hq_dev_mat *W, const uint16_t *A, int M, void *C, int c_f32, int accumulate,
                              int nt0, int nt1, hipStream_t st) {
    if (!hq_wr8_fits(W, M)) return hipErrorInvalidValue;
    // fp32 or fp16 C, or the SwiGLU output of a gate/up pair matrix (N a multiple of 16, no accumulate)
    if (c_f32 != 0 && c_f32 != 1 && !(c_f32 == HQ_OUT_SWIGLU && W->rows % 16 == 0 && !accumulate)) return hipErrorInvalidValue;
    Wr8Args g;
    g.Q = W->qs, g.D = W->d, g.ldd = W->ldd, g.A = A;
    g.M = M, g.N = (int)W->rows, g.K = (int)W->cols, g.C = C, g.c_f32 = c_f32, g.accumulate = accumulate;
    g.mt = (M + W8_BM - 1) / W8_BM;
    const int nt_all = (g.N + 64 * W8_NB - 1) / (64 * W8_NB);
    g.nt0 = nt0, g.nt = nt1 < 0 || nt1 > nt_all ? nt_all : nt1;
    if (nt0 < 0 || nt0 >= g.nt) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)(8 * ((g.nt - g.nt0 + 7) / 8) * g.mt);
    k_gemm_q8_0_wr<<<grid, W8_NT, 0, st>>>(g);
    return hipGetLastError();
}
