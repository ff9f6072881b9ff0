// hq_backend.hip - the HIP inference backend (include/hq_backend.h): the reference's backend_t
// vtable (cleanroom-transformer/src/transformer.h:347-364) over a device-resident layer loop.
//
// Per chunk of T tokens at position pos0 (the reference's run_layers, src/cuda_backend.cu:783-850,
// for LAYER_FULL layers), on the backend's stream:
//   x [T, H] fp32      residual stream (embedding rows decoded from the GGUF blocks)
//   hb [T, H] fp16     RMSNorm(x) * (off + w): the GEMM operand (k_rmsnorm_f16)
//   q/k/v fp32         hq_gemm(q|k|v, hb)            (q rows interleave [q_h | gate_h] with the output gate)
//   qr fp32, kc/vc     q/k RMSNorm (optional) + RoPE with the model's inverse frequencies, k and v
//                      appended to the per-layer fp32 KV cache at pos0 .. pos0 + T - 1 (k_qk_rope)
//   ob [T, nh*hd] fp16 causal softmax attention over the cache, grouped-query, optional sigmoid gate
//                      (k_attention)
//   x += hq_gemm(o, ob)                               (accumulate into the residual)
//   hb = RMSNorm(x) fp16
//   fb = silu(gate . hb) * (up . hb) fp16: where gate and up share a block type and shape they are
//        resident as one gate/up pair matrix (hq_mat_upload_pair) and fb comes from hq_gemm_swiglu
//        (any T: the SwiGLU epilogue inside the GEMM's tiles for prefill shapes, the tuned GEMV over
//        both halves at T = 1); otherwise (a Q4_K gate with a Q6_K up, as Q4_K_M files pair them)
//        T = 1 runs k_gateup_swiglu (one pass over both matrices) and larger T two hq_gemm calls and
//        k_swiglu
//   x += hq_gemm(down, fb)
// then, with readout ids, one kernel normalises the last position (final RMSNorm, fp32) and dots it
// with each id's lm_head row decoded from its blocks (k_norm_readout; src/cuda_backend.cu:561-592).
// Every projection is an hq_gemm call (GEMV at T = 1, MFMA GEMM above), so the quantized matmul path
// is the one the rest of the library measures; the surrounding kernels are simple fp32 code.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <vector>

#include "hq.h"
#include "hq_backend.h"
#include "hq_device.h"
#include "hq_internal.h"
#include "hq_kernels.h"
#include "hq_kquant.h"

namespace {

#define BCK(call)                                                                                         \
    do {                                                                                                  \
        hipError_t e_ = (call);                                                                           \
        if (e_ != hipSuccess)                                                                             \
            return hq_internal_fail("HIP %s failed: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__); \
    } while (0)

constexpr int CHUNK = 1024;    // tokens per layer-loop pass
constexpr int MAX_IDS = 4096;  // readout ids per forward

// ------------------------------------------------------------------------------------ kernels
// Eight consecutive weights 8g .. 8g + 7 of row r as fp32, bit-identical to the reference decoder
// (src/ggml_quant.h:95-99 Q8_0, :100-134 Q2_K / Q3_K, :135-150 Q4_K / Q5_K, :151-169 Q6_K; device
// layouts as in hq_kernels.hip, hq_kquant.h and hq_q6k.hip).
DEV void deq8(const hq_dev_mat &W, size_t r, int g, float (&w)[8]) {
    if (hq_is_kq(W.type)) {
        const uint8_t *b = W.qs + r * W.row_bytes + (size_t)(8 * g / 256) * kq_slot(W.type);
        kq_deq8_any(W.type, b, (8 * g) % 256, w);
        return;
    }
    if (W.type == HQ_TYPE_Q8_0) {
        const u2v q = *(const u2v *)(W.qs + r * W.cols + 8 * (size_t)g);
        const float d = h2f(W.d[r * (size_t)W.ldd + g / 4]);
#pragma unroll
        for (int j = 0; j < 8; j++) w[j] = (float)(int8_t)(byte_of(j < 4 ? q.x : q.y, j & 3) ^ 0x80u) * d;
        return;
    }
    if (W.type == HQ_TYPE_Q6_K) {  // src/ggml_quant.h:151-169, 224-byte device slots
        const int v = (8 * g) % 256, h = v >> 7, rr = (v >> 5) & 3, l0 = v & 31;
        const uint8_t *b = W.qs + r * W.row_bytes + (size_t)(8 * g / 256) * 224;
        const u2v ql = *(const u2v *)(b + 64 * h + 32 * (rr & 1) + l0), qh = *(const u2v *)(b + 128 + 32 * h + l0);
        const float ds = h2f(*(const uint16_t *)(b + 208)) * (float)(int8_t)b[192 + 8 * h + 2 * rr + (l0 >> 4)];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int lo = (int)((((j < 4 ? ql.x : ql.y) >> (8 * (j & 3))) >> (rr >= 2 ? 4 : 0)) & 0xfu);
            const int hb = (int)((((j < 4 ? qh.x : qh.y) >> (8 * (j & 3))) >> (2 * rr)) & 3u);
            w[j] = ds * (float)((lo | (hb << 4)) - 32);
        }
        return;
    }
    const int v0 = 8 * g, sub = (v0 % 256) / 32, l0 = v0 % 32;
    const uint8_t *b = W.qs + r * W.row_bytes + (size_t)(v0 / 256) * 144;
    const u4v hdr = *(const u4v *)b;
    uint32_t sw0, sw1, mw0, mw1;
    q4k_scale_words(hdr.y, hdr.z, hdr.w, sw0, sw1, mw0, mw1);
    const uint32_t s = byte_of(sub < 4 ? sw0 : sw1, sub & 3), m = byte_of(sub < 4 ? mw0 : mw1, sub & 3);
    const float ds = h2f((uint16_t)hdr.x) * (float)s, dm = h2f((uint16_t)(hdr.x >> 16)) * (float)m;
    const u2v q = *(const u2v *)(b + 16 + 32 * (sub >> 1) + l0);
    const int shift = (sub & 1) ? 4 : 0;
#pragma unroll
    for (int j = 0; j < 8; j++) w[j] = ds * (float)((((j < 4 ? q.x : q.y) >> (8 * (j & 3))) >> shift) & 0xfu) - dm;
}

DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
DEV float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sum over a 256-thread block (red: 4 floats of LDS); every thread gets the total.
DEV float block_sum(float v, float *red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

DEV float silu(float x) { return x / (1.0f + expf(-x)); }  // src/ops_common.h:56

// RMSNorm of row blockIdx.x (src/cpu_backend.c:57-62): out = x * (1 / sqrt(mean(x^2) + eps)) * (off + w)
template <typename T>
__global__ void __launch_bounds__(256) k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, float off,
                                                 float eps, T *__restrict__ out, int H) {
    __shared__ float red[4];
    const float *xr = x + (size_t)blockIdx.x * H;
    float ss = 0.f;
    for (int i = threadIdx.x; i < H; i += 256) ss += xr[i] * xr[i];
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
    for (int i = threadIdx.x; i < H; i += 256) out[(size_t)blockIdx.x * H + i] = (T)(xr[i] * inv * (off + w[i]));
}

// One wave per (token t, head j): heads j < nh are queries (q rows of qb, stride qw, [q | gate]
// per head when gated), the others keys of kv head j - nh (whose value row is copied alongside).
// Optional q/k RMSNorm, then RoPE on the first rot dims (pairs i, i + rot/2) at position pos0 + t
// (src/cpu_backend.c:86-102). Queries go to qr [T, nh, hd]; keys and values to the caches.
__global__ void __launch_bounds__(64) k_qk_rope(const float *__restrict__ qb, const float *__restrict__ kb,
                                                const float *__restrict__ vb, const float *__restrict__ qn,
                                                const float *__restrict__ kn, float off, float eps,
                                                const float *__restrict__ inv_freq, float *__restrict__ qr,
                                                float *__restrict__ kc, float *__restrict__ vc, int nh, int nkv, int hd,
                                                int rot, int qw, int gated, int pos0, int qk_norm) {
    __shared__ float xs[256];
    const int t = blockIdx.x, j = blockIdx.y, lane = threadIdx.x, kvw = nkv * hd;
    const bool is_q = j < nh;
    const float *src = is_q ? qb + (size_t)t * qw + (size_t)j * hd * (gated ? 2 : 1) : kb + (size_t)t * kvw + (size_t)(j - nh) * hd;
    float *dst = is_q ? qr + ((size_t)t * nh + j) * hd : kc + (size_t)(pos0 + t) * kvw + (size_t)(j - nh) * hd;
    float v[4];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int d = lane + 64 * i;
        v[i] = d < hd ? src[d] : 0.f;
        ss += v[i] * v[i];
    }
    if (qk_norm) {
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
        const float *nw = is_q ? qn : kn;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int d = lane + 64 * i;
            if (d < hd) v[i] = v[i] * inv * (off + nw[d]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (lane + 64 * i < hd) xs[lane + 64 * i] = v[i];
    __syncthreads();
    const float p = (float)(pos0 + t);
    const int half = rot / 2;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int d = lane + 64 * i;
        if (d >= hd) continue;
        float y = xs[d];
        if (d < rot) {
            const int f = d < half ? d : d - half;
            const float a = inv_freq[f] * p, cs = cosf(a), sn = sinf(a);
            y = d < half ? xs[d] * cs - xs[d + half] * sn : xs[d] * cs + xs[d - half] * sn;
        }
        dst[d] = y;
        if (!is_q) vc[(size_t)(pos0 + t) * kvw + (size_t)(j - nh) * hd + d] = vb[(size_t)t * kvw + (size_t)(j - nh) * hd + d];
    }
}

// One wave per (token t, query head j): causal softmax attention of query pos0 + t over cache
// positions 0 .. pos0 + t of kv head j / (nh / nkv), online over chunks of 64 positions (lane s
// scores position s0 + s); output fp16 [T, nh * hd], times sigmoid(gate) when gated
// (src/cpu_backend.c:103-131).
__global__ void __launch_bounds__(64) k_attention(const float *__restrict__ qr, const float *__restrict__ qb,
                                                  const float *__restrict__ kc, const float *__restrict__ vc,
                                                  _Float16 *__restrict__ out, int nh, int nkv, int hd, int qw,
                                                  int gated, int pos0, float scale) {
    __shared__ float qs[256];
    const int t = blockIdx.x, j = blockIdx.y, lane = threadIdx.x, kvw = nkv * hd, g = j / (nh / nkv);
    const int n = pos0 + t + 1;
    for (int d = lane; d < hd; d += 64) qs[d] = qr[((size_t)t * nh + j) * hd + d];
    __syncthreads();
    float m = -INFINITY, l = 0.f, o[4] = {0.f, 0.f, 0.f, 0.f};
    const float *kh = kc + (size_t)g * hd, *vh = vc + (size_t)g * hd;
    for (int s0 = 0; s0 < n; s0 += 64) {
        const int s = s0 + lane;
        float sc = -INFINITY;
        if (s < n) {
            const float *kr = kh + (size_t)s * kvw;
            float acc = 0.f;
            for (int d = 0; d < hd; d += 4) {
                const float4 k4 = *(const float4 *)(kr + d);
                acc += qs[d] * k4.x + qs[d + 1] * k4.y + qs[d + 2] * k4.z + qs[d + 3] * k4.w;
            }
            sc = acc * scale;
        }
        const float mn = fmaxf(m, wave_max(sc));
        const float pr = s < n ? expf(sc - mn) : 0.f;
        const float alpha = expf(m - mn);  // 0 before the first chunk (m = -inf)
        l = l * alpha + wave_sum(pr);
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] *= alpha;
        const int cnt = n - s0 < 64 ? n - s0 : 64;
        for (int e = 0; e < cnt; e++) {
            const float pe = __shfl(pr, e, 64);
            const float *vr = vh + (size_t)(s0 + e) * kvw;
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (lane + 64 * i < hd) o[i] += pe * vr[lane + 64 * i];
        }
        m = mn;
    }
    const float *gate = qb + (size_t)t * qw + (size_t)j * hd * 2 + hd;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int d = lane + 64 * i;
        if (d >= hd) continue;
        float y = o[i] / l;
        if (gated) y *= 1.0f / (1.0f + expf(-gate[d]));
        out[((size_t)t * nh + j) * hd + d] = (_Float16)y;
    }
}

__global__ void __launch_bounds__(256) k_swiglu(const float *__restrict__ g, const float *__restrict__ u,
                                                _Float16 *__restrict__ out, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = (_Float16)(silu(g[i]) * u[i]);
}

// Single-token FFN input (src/cuda_backend.cu:548-559): out[i] = silu(gate_i . a) * (up_i . a) for
// one fp16 activation row a [H]; one wave per output row, both weight rows decoded in registers.
__global__ void __launch_bounds__(256) k_gateup_swiglu(hq_dev_mat Wg, hq_dev_mat Wu, const _Float16 *__restrict__ a,
                                                       _Float16 *__restrict__ out, int I, int H) {
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (i >= I) return;
    float sg = 0.f, su = 0.f;
    for (int g = lane; g < H / 8; g += 64) {
        float wg[8], wu[8];
        deq8(Wg, (size_t)i, g, wg);
        deq8(Wu, (size_t)i, g, wu);
        const h8 av = *(const h8 *)(a + 8 * g);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            sg += wg[e] * (float)av[e];
            su += wu[e] * (float)av[e];
        }
    }
    sg = wave_sum(sg);
    su = wave_sum(su);
    if (lane == 0) out[i] = (_Float16)(silu(sg) * su);
}

// Readout (src/cuda_backend.cu:561-592, src/cpu_backend.c:253-259): workgroup b normalises the last
// position x [H] (final RMSNorm, fp32) into LDS and dots it with lm_head row ids[b].
__global__ void __launch_bounds__(256) k_norm_readout(const float *__restrict__ x, const float *__restrict__ w,
                                                      float off, float eps, hq_dev_mat Wh,
                                                      const uint32_t *__restrict__ ids, float *__restrict__ logits,
                                                      int H) {
    extern __shared__ float hs[];
    __shared__ float red[4];
    float ss = 0.f;
    for (int i = threadIdx.x; i < H; i += 256) ss += x[i] * x[i];
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
    for (int i = threadIdx.x; i < H; i += 256) hs[i] = x[i] * inv * (off + w[i]);
    __syncthreads();
    const size_t r = ids[blockIdx.x];
    float acc = 0.f;
    for (int g = threadIdx.x; g < H / 8; g += 256) {
        float wv[8];
        deq8(Wh, r, g, wv);
#pragma unroll
        for (int e = 0; e < 8; e++) acc += wv[e] * hs[8 * g + e];
    }
    acc = block_sum(acc, red);
    if (threadIdx.x == 0) logits[blockIdx.x] = acc;
}

unsigned blocks_for(size_t n, unsigned per) { return (unsigned)((n + per - 1) / per < 65535 ? (n + per - 1) / per : 65535); }

// ------------------------------------------------------------------------------------ backend
struct DevLayer {
    hq_mat *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr, *gate = nullptr, *up = nullptr, *down = nullptr;
    hq_mat *pair = nullptr;  // gate and up as one pair matrix (then gate and up are null)
    float *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    float *kc = nullptr, *vc = nullptr;  // [max_seq, kvw] fp32
};

struct HipBackend {
    hq_ref_backend_t base;  // first member: callers hold a pointer to it
    const hq_ref_model_t *m = nullptr;
    int device = 0;
    hipStream_t st = nullptr;
    hq_mat *embed = nullptr, *lm_head = nullptr;
    float *final_norm = nullptr, *inv_freq = nullptr;
    std::vector<DevLayer> L;
    std::vector<void *> allocs;  // device buffers owned by the backend
    float *x = nullptr, *qb = nullptr, *kb = nullptr, *vb = nullptr, *qr = nullptr, *gb = nullptr, *ub = nullptr;
    _Float16 *hb = nullptr, *ob = nullptr, *fb = nullptr;
    uint32_t *d_tok = nullptr, *d_ids = nullptr;
    float *d_logits = nullptr, *d_hidden = nullptr;
    int chunk = CHUNK, last_T = 0;
    size_t snap_pos = 0;
    bool has_snap = false;
};

int dalloc(HipBackend *b, void **p, size_t bytes) {
    BCK(hipMalloc(p, bytes ? bytes : 16));
    b->allocs.push_back(*p);
    return 0;
}

int upload_vec(HipBackend *b, float **out, const float *src, size_t n) {
    *out = nullptr;
    if (!src) return hq_internal_fail("hip backend: a norm vector of the model is missing");
    if (dalloc(b, (void **)out, n * sizeof(float))) return -1;
    BCK(hipMemcpy(*out, src, n * sizeof(float), hipMemcpyHostToDevice));
    return 0;
}

int upload_mat(HipBackend *b, hq_mat **out, const hq_wmat_t *w, const char *what) {
    if (hq_mat_upload(w, b->device, out)) {
        char msg[512];
        snprintf(msg, sizeof msg, "%s", hq_last_error());
        return hq_internal_fail("hip backend: %s: %s", what, msg);
    }
    return 0;
}

void release(HipBackend *b) {
    if (!b) return;
    (void)hipSetDevice(b->device);
    if (b->st) (void)hipStreamSynchronize(b->st);
    for (DevLayer &l : b->L)
        for (hq_mat *m : {l.q, l.k, l.v, l.o, l.gate, l.up, l.down, l.pair}) hq_mat_free(m);
    if (b->lm_head != b->embed) hq_mat_free(b->lm_head);
    hq_mat_free(b->embed);
    for (void *p : b->allocs) (void)hipFree(p);
    if (b->st) {
        (void)hq_stream_destroy(b->st);  // also frees the stream's GEMM workspace
    }
    delete b;
}

HipBackend *self(hq_ref_backend_t *b) { return (HipBackend *)b; }

int be_reset(hq_ref_backend_t *bb) {
    bb->pos = 0;
    self(bb)->last_T = 0;
    return 0;
}

int be_snapshot(hq_ref_backend_t *bb) {
    // full-attention state is the KV cache, which later tokens only append to: the position is the
    // whole snapshot (the reference's cu_snapshot copies only Gated-DeltaNet state besides it)
    HipBackend *b = self(bb);
    b->snap_pos = bb->pos;
    b->has_snap = true;
    return 0;
}

int be_restore(hq_ref_backend_t *bb) {
    HipBackend *b = self(bb);
    if (!b->has_snap) return hq_internal_fail("restore: no snapshot");
    bb->pos = b->snap_pos;
    return 0;
}

void be_destroy(hq_ref_backend_t *bb) { release(self(bb)); }

int gemm(HipBackend *b, const hq_mat *W, const _Float16 *A, int T, float *C, bool accumulate) {
    return hq_gemm(W, (const uint16_t *)A, T, C, 1, accumulate ? 1 : 0, b->st);
}

// The layer loop over T tokens at position pos0; x holds their embedding rows.
int run_layers(HipBackend *b, int T, int pos0) {
    const hq_ref_config_t &c = b->m->cfg;
    const int H = (int)c.hidden, I = (int)c.intermediate, nh = (int)c.n_heads, nkv = (int)c.n_kv_heads;
    const int hd = (int)c.head_dim, qw = nh * hd * (c.attn_gate ? 2 : 1);
    const float off = c.norm_offset, eps = c.eps, scale = 1.0f / sqrtf((float)hd);
    hipStream_t st = b->st;
    for (uint32_t li = 0; li < c.n_layers; li++) {
        const DevLayer &L = b->L[li];
        k_rmsnorm<_Float16><<<T, 256, 0, st>>>(b->x, L.in_norm, off, eps, b->hb, H);
        BCK(hipGetLastError());
        if (gemm(b, L.q, b->hb, T, b->qb, false) || gemm(b, L.k, b->hb, T, b->kb, false) ||
            gemm(b, L.v, b->hb, T, b->vb, false))
            return -1;
        k_qk_rope<<<dim3(T, nh + nkv), 64, 0, st>>>(b->qb, b->kb, b->vb, L.q_norm, L.k_norm, off, eps, b->inv_freq, b->qr,
                                                    L.kc, L.vc, nh, nkv, hd, (int)c.rot_dim, qw, c.attn_gate, pos0,
                                                    c.qk_norm);
        BCK(hipGetLastError());
        k_attention<<<dim3(T, nh), 64, 0, st>>>(b->qr, b->qb, L.kc, L.vc, b->ob, nh, nkv, hd, qw, c.attn_gate, pos0, scale);
        BCK(hipGetLastError());
        if (gemm(b, L.o, b->ob, T, b->x, true)) return -1;
        k_rmsnorm<_Float16><<<T, 256, 0, st>>>(b->x, L.post_norm, off, eps, b->hb, H);
        BCK(hipGetLastError());
        if (L.pair) {
            if (hq_gemm_swiglu(L.pair, (const uint16_t *)b->hb, T, (uint16_t *)b->fb, st)) return -1;
        } else if (T == 1) {
            k_gateup_swiglu<<<(I + 3) / 4, 256, 0, st>>>(*hq_mat_dev(L.gate), *hq_mat_dev(L.up), b->hb, b->fb, I, H);
            BCK(hipGetLastError());
        } else {
            if (gemm(b, L.gate, b->hb, T, b->gb, false) || gemm(b, L.up, b->hb, T, b->ub, false)) return -1;
            k_swiglu<<<blocks_for((size_t)T * I, 256), 256, 0, st>>>(b->gb, b->ub, b->fb, (size_t)T * I);
            BCK(hipGetLastError());
        }
        if (gemm(b, L.down, b->fb, T, b->x, true)) return -1;
    }
    return 0;
}

int be_forward(hq_ref_backend_t *bb, const uint32_t *tokens, size_t n, const uint32_t *ids, uint32_t n_ids,
               float *logits) {
    HipBackend *b = self(bb);
    const hq_ref_config_t &c = b->m->cfg;
    if (n == 0) return hq_internal_fail("forward: no tokens");
    if (bb->pos + n > bb->max_seq) return hq_internal_fail("forward: %zu tokens exceed context %zu", bb->pos + n, bb->max_seq);
    if (n_ids > MAX_IDS) return hq_internal_fail("forward: too many readout ids (%u > %d)", n_ids, MAX_IDS);
    if (n_ids && (!ids || !logits)) return hq_internal_fail("forward: readout ids without an output buffer");
    for (size_t t = 0; t < n; t++)
        if (tokens[t] >= c.vocab) return hq_internal_fail("forward: token %u out of range", tokens[t]);
    for (uint32_t k = 0; k < n_ids; k++)
        if (ids[k] >= c.vocab) return hq_internal_fail("forward: readout id %u out of range", ids[k]);
    BCK(hipSetDevice(b->device));
    const int H = (int)c.hidden;
    int last_T = 0;
    for (size_t c0 = 0; c0 < n; c0 += (size_t)b->chunk) {
        const int T = (int)(n - c0 < (size_t)b->chunk ? n - c0 : (size_t)b->chunk);
        BCK(hipMemcpyAsync(b->d_tok, tokens + c0, (size_t)T * sizeof(uint32_t), hipMemcpyHostToDevice, b->st));
        BCK(hq_launch_dequant(hq_mat_dev(b->embed), 0, b->d_tok, (uint32_t)T, b->x, b->st));
        if (run_layers(b, T, (int)bb->pos)) return -1;
        bb->pos += (size_t)T;
        last_T = T;
    }
    b->last_T = last_T;
    if (n_ids) {
        BCK(hipMemcpyAsync(b->d_ids, ids, n_ids * sizeof(uint32_t), hipMemcpyHostToDevice, b->st));
        k_norm_readout<<<n_ids, 256, (size_t)H * sizeof(float), b->st>>>(b->x + (size_t)(last_T - 1) * H, b->final_norm,
                                                                         c.norm_offset, c.eps, *hq_mat_dev(b->lm_head),
                                                                         b->d_ids, b->d_logits, H);
        BCK(hipGetLastError());
        BCK(hipMemcpyAsync(logits, b->d_logits, n_ids * sizeof(float), hipMemcpyDeviceToHost, b->st));
    }
    BCK(hipStreamSynchronize(b->st));
    return 0;
}

int be_last_hidden(hq_ref_backend_t *bb, float *out) {
    HipBackend *b = self(bb);
    const hq_ref_config_t &c = b->m->cfg;
    if (b->last_T < 1) return hq_internal_fail("last_hidden: no forward pass yet");
    BCK(hipSetDevice(b->device));
    const int H = (int)c.hidden;
    k_rmsnorm<float><<<1, 256, 0, b->st>>>(b->x + (size_t)(b->last_T - 1) * H, b->final_norm, c.norm_offset, c.eps,
                                           b->d_hidden, H);
    BCK(hipGetLastError());
    BCK(hipMemcpyAsync(out, b->d_hidden, (size_t)H * sizeof(float), hipMemcpyDeviceToHost, b->st));
    BCK(hipStreamSynchronize(b->st));
    return 0;
}

// Shapes the kernels support, checked before anything is uploaded.
int check_model(const hq_ref_model_t *m, size_t max_seq) {
    const hq_ref_config_t &c = m->cfg;
    if (!c.hidden || !c.n_layers || !c.vocab || !c.n_heads || !c.n_kv_heads || !c.head_dim || !c.intermediate)
        return hq_internal_fail("hip backend: empty model config");
    if (c.n_layers > 256) return hq_internal_fail("hip backend: %u layers (at most 256)", c.n_layers);
    for (uint32_t l = 0; l < c.n_layers; l++)
        if (m->layers[l].type != HQ_REF_LAYER_FULL)
            return hq_internal_fail("hip backend: layer %u is a Gated-DeltaNet (linear attention) layer; this backend runs "
                                    "full-attention layers only", l);
    if (c.head_dim > 256 || c.head_dim % 4) return hq_internal_fail("hip backend: head_dim %u (a multiple of 4, at most 256)", c.head_dim);
    if (c.rot_dim > c.head_dim || c.rot_dim % 2) return hq_internal_fail("hip backend: rot_dim %u", c.rot_dim);
    if (c.n_heads % c.n_kv_heads) return hq_internal_fail("hip backend: %u heads over %u kv heads", c.n_heads, c.n_kv_heads);
    if (c.hidden % 8 || c.hidden > 16384) return hq_internal_fail("hip backend: hidden %u (a multiple of 8, at most 16384)", c.hidden);
    if (!m->rope_inv_freq || !m->final_norm || !m->layers) return hq_internal_fail("hip backend: model tables missing");
    if (max_seq == 0 || max_seq > (1u << 24)) return hq_internal_fail("hip backend: max_seq %zu", max_seq);
    return 0;
}

int init(HipBackend *b, const hq_ref_model_t *m, size_t max_seq) {
    const hq_ref_config_t &c = m->cfg;
    if (check_model(m, max_seq)) return -1;
    if (hq_device_init(b->device)) return -1;
    void *s;
    if (hq_stream_create(&s)) return -1;
    b->st = (hipStream_t)s;
    if (upload_mat(b, &b->embed, &m->embed, "token_embd")) return -1;
    if (c.tied) b->lm_head = b->embed;
    else if (upload_mat(b, &b->lm_head, &m->lm_head, "output")) return -1;
    const size_t H = c.hidden, hd = c.head_dim, I = c.intermediate, kvw = (size_t)c.n_kv_heads * hd;
    if (upload_vec(b, &b->final_norm, m->final_norm, H) || upload_vec(b, &b->inv_freq, m->rope_inv_freq, c.rot_dim / 2 ? c.rot_dim / 2 : 1))
        return -1;
    b->L.resize(c.n_layers);
    for (uint32_t l = 0; l < c.n_layers; l++) {
        const hq_ref_layer_t &s = m->layers[l];
        DevLayer &d = b->L[l];
        char what[64];
        snprintf(what, sizeof what, "layer %u", l);
        if (upload_vec(b, &d.in_norm, s.in_norm, H) || upload_vec(b, &d.post_norm, s.post_norm, H) ||
            upload_mat(b, &d.q, &s.q, what) || upload_mat(b, &d.k, &s.k, what) || upload_mat(b, &d.v, &s.v, what) ||
            upload_mat(b, &d.o, &s.o, what) || upload_mat(b, &d.down, &s.down, what))
            return -1;
        // gate and up of one block type and shape (rows a multiple of 8): one pair matrix
        const bool pair = s.gate.dtype == HQ_DT_GGML && s.up.dtype == HQ_DT_GGML && s.gate.ggml_type == s.up.ggml_type &&
                          s.gate.rows == s.up.rows && s.gate.cols == s.up.cols && s.gate.rows % 8 == 0;
        if (pair) {
            if (hq_mat_upload_pair(&s.gate, &s.up, b->device, &d.pair)) {
                char msg[512];
                snprintf(msg, sizeof msg, "%s", hq_last_error());
                return hq_internal_fail("hip backend: %s gate/up: %s", what, msg);
            }
        } else if (upload_mat(b, &d.gate, &s.gate, what) || upload_mat(b, &d.up, &s.up, what)) {
            return -1;
        }
        if (c.qk_norm && (upload_vec(b, &d.q_norm, s.q_norm, hd) || upload_vec(b, &d.k_norm, s.k_norm, hd))) return -1;
        if (dalloc(b, (void **)&d.kc, max_seq * kvw * sizeof(float)) || dalloc(b, (void **)&d.vc, max_seq * kvw * sizeof(float)))
            return -1;
    }
    const size_t CH = (size_t)(max_seq < (size_t)CHUNK ? max_seq : (size_t)CHUNK);
    b->chunk = (int)CH;
    const size_t qw = (size_t)c.n_heads * hd * (c.attn_gate ? 2 : 1), ow = (size_t)c.n_heads * hd;
    if (dalloc(b, (void **)&b->x, CH * H * 4) || dalloc(b, (void **)&b->qb, CH * qw * 4) ||
        dalloc(b, (void **)&b->kb, CH * kvw * 4) || dalloc(b, (void **)&b->vb, CH * kvw * 4) ||
        dalloc(b, (void **)&b->qr, CH * ow * 4) || dalloc(b, (void **)&b->gb, CH * I * 4) ||
        dalloc(b, (void **)&b->ub, CH * I * 4) || dalloc(b, (void **)&b->hb, CH * H * 2) ||
        dalloc(b, (void **)&b->ob, CH * ow * 2) || dalloc(b, (void **)&b->fb, CH * I * 2) ||
        dalloc(b, (void **)&b->d_tok, CH * 4) || dalloc(b, (void **)&b->d_ids, MAX_IDS * 4) ||
        dalloc(b, (void **)&b->d_logits, MAX_IDS * 4) || dalloc(b, (void **)&b->d_hidden, H * 4))
        return -1;
    // every projection must take its input width and give the next one's
    for (uint32_t l = 0; l < c.n_layers; l++) {
        const DevLayer &d = b->L[l];
        uint32_t r, k;
        struct {
            const hq_mat *w;
            uint32_t rows, cols;
            const char *name;
        } want[] = {{d.q, (uint32_t)qw, (uint32_t)H, "q"},        {d.k, (uint32_t)kvw, (uint32_t)H, "k"},
                    {d.v, (uint32_t)kvw, (uint32_t)H, "v"},        {d.o, (uint32_t)H, (uint32_t)ow, "o"},
                    {d.gate, (uint32_t)I, (uint32_t)H, "gate"},   {d.up, (uint32_t)I, (uint32_t)H, "up"},
                    {d.pair, 2 * (uint32_t)I, (uint32_t)H, "gate/up"}, {d.down, (uint32_t)H, (uint32_t)I, "down"}};
        for (auto &w : want) {
            if (!w.w) continue;  // (gate and up, or their pair)
            if (hq_mat_shape(w.w, &r, &k, nullptr)) return -1;
            if (r != w.rows || k != w.cols)
                return hq_internal_fail("hip backend: layer %u %s is [%u, %u], the config needs [%u, %u]", l, w.name, r, k,
                                        w.rows, w.cols);
        }
    }
    uint32_t r, k;
    if (hq_mat_shape(b->embed, &r, &k, nullptr) || hq_mat_shape(b->lm_head, nullptr, nullptr, nullptr)) return -1;
    if (r != c.vocab || k != H) return hq_internal_fail("hip backend: embedding is [%u, %u]", r, k);
    if (hq_mat_shape(b->lm_head, &r, &k, nullptr)) return -1;
    if (r != c.vocab || k != H) return hq_internal_fail("hip backend: lm_head is [%u, %u]", r, k);
    return 0;
}

// ------------------------------------------------------------------------------------ selftest
uint64_t lcg(uint64_t *s) {  // the public MMIX LCG, as the reference's selftest
    *s = *s * 6364136223846793005ull + 1442695040888963407ull;
    return *s >> 33;
}

double now_s() {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

uint16_t to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
float from_f16(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// hq_gemm at several M on W against a float64 host product of W's decoded rows (hq_dequant_f32,
// bit-exact with the reference decoder) on up to 64 sampled columns.
int selftest_gemm(const hq_mat *W, const char *name, int verbose, int *failed, hipStream_t st) {
    uint32_t N, K;
    if (hq_mat_shape(W, &N, &K, nullptr)) return -1;
    const int Ms[] = {1, 5, 33, 64, 200};
    uint64_t seed = 42 + N + K;
    const int ncol = N < 64 ? (int)N : 64;
    std::vector<uint32_t> cols(ncol);
    for (int j = 0; j < ncol; j++) cols[j] = (uint32_t)((uint64_t)j * N / ncol);
    std::vector<float> w((size_t)ncol * K);
    float *dw;
    BCK(hipMalloc(&dw, (size_t)K * 4));
    for (int j = 0; j < ncol; j++) {
        if (hq_dequant_f32(W, cols[j], 1, dw, st)) return -1;
        BCK(hipMemcpyAsync(w.data() + (size_t)j * K, dw, (size_t)K * 4, hipMemcpyDeviceToHost, st));
    }
    BCK(hipStreamSynchronize(st));
    BCK(hipFree(dw));
    for (int M : Ms) {
        std::vector<uint16_t> A((size_t)M * K);
        for (auto &a : A) a = to_f16((float)((double)lcg(&seed) / (double)(1ull << 31) * 2.0 - 1.0));
        void *dA, *dC;
        BCK(hipMalloc(&dA, A.size() * 2));
        BCK(hipMalloc(&dC, (size_t)M * N * 4));
        BCK(hipMemcpy(dA, A.data(), A.size() * 2, hipMemcpyHostToDevice));
        if (hq_gemm(W, (const uint16_t *)dA, M, dC, 1, 0, st)) return -1;
        std::vector<float> C((size_t)M * N);
        BCK(hipMemcpyAsync(C.data(), dC, C.size() * 4, hipMemcpyDeviceToHost, st));
        BCK(hipStreamSynchronize(st));
        BCK(hipFree(dA));
        BCK(hipFree(dC));
        double worst = 0, num = 0, den = 0;
        for (int m = 0; m < M; m++)
            for (int j = 0; j < ncol; j++) {
                double ref = 0;
                for (uint32_t k = 0; k < K; k++) ref += (double)from_f16(A[(size_t)m * K + k]) * (double)w[(size_t)j * K + k];
                const double err = fabs(ref - (double)C[(size_t)m * N + cols[j]]);
                worst = err > worst ? err : worst;
                num += err * err, den += ref * ref;
            }
        const double rel = den > 0 ? sqrt(num / den) : sqrt(num);
        const bool ok = rel <= 1e-3 && worst <= 1e-2;
        if (!ok) (*failed)++;
        if (verbose || !ok)
            printf("  gemm %-8s M=%-4d N=%-6u K=%-6u rel-L2 %.2e max-abs %.2e  %s\n", name, M, N, K, rel, worst, ok ? "ok" : "FAIL");
    }
    return 0;
}

// hq_gemm_swiglu on a gate/up pair matrix at several M against silu(g) * u in float64 from the
// decoded gate and up rows (hq_dequant_f32) on up to 64 sampled output columns; the output is fp16,
// so half an ulp of |y| is allowed on top of the 1e-2 bar.
int selftest_swiglu(const hq_mat *P, int verbose, int *failed, hipStream_t st) {
    uint32_t N2, K;
    if (hq_mat_shape(P, &N2, &K, nullptr)) return -1;
    const uint32_t I = N2 / 2;
    const int Ms[] = {1, 5, 64, 200};
    uint64_t seed = 17 + I + K;
    const int ncol = I < 64 ? (int)I : 64;
    std::vector<uint32_t> cols(ncol);
    for (int j = 0; j < ncol; j++) cols[j] = (uint32_t)((uint64_t)j * I / ncol);
    std::vector<float> wg((size_t)ncol * K), wu((size_t)ncol * K);
    float *dw;
    BCK(hipMalloc(&dw, (size_t)K * 4));
    for (int j = 0; j < ncol; j++) {
        const uint32_t i = cols[j], rg = 16 * (i / 8) + i % 8;  // pair rows of gate i and up i
        if (hq_dequant_f32(P, rg, 1, dw, st)) return -1;
        BCK(hipMemcpyAsync(wg.data() + (size_t)j * K, dw, (size_t)K * 4, hipMemcpyDeviceToHost, st));
        if (hq_dequant_f32(P, rg + 8, 1, dw, st)) return -1;
        BCK(hipMemcpyAsync(wu.data() + (size_t)j * K, dw, (size_t)K * 4, hipMemcpyDeviceToHost, st));
        BCK(hipStreamSynchronize(st));
    }
    BCK(hipFree(dw));
    for (int M : Ms) {
        std::vector<uint16_t> A((size_t)M * K), O((size_t)M * I);
        for (auto &a : A) a = to_f16((float)((double)lcg(&seed) / (double)(1ull << 31) * 2.0 - 1.0));
        void *dA, *dO;
        BCK(hipMalloc(&dA, A.size() * 2));
        BCK(hipMalloc(&dO, O.size() * 2));
        BCK(hipMemcpy(dA, A.data(), A.size() * 2, hipMemcpyHostToDevice));
        if (hq_gemm_swiglu(P, (const uint16_t *)dA, M, (uint16_t *)dO, st)) return -1;
        BCK(hipMemcpyAsync(O.data(), dO, O.size() * 2, hipMemcpyDeviceToHost, st));
        BCK(hipStreamSynchronize(st));
        BCK(hipFree(dA));
        BCK(hipFree(dO));
        double worst = 0, num = 0, den = 0;
        bool ok = true;
        for (int m = 0; m < M; m++)
            for (int j = 0; j < ncol; j++) {
                double g = 0, u = 0;
                for (uint32_t k = 0; k < K; k++) {
                    const double a = from_f16(A[(size_t)m * K + k]);
                    g += a * wg[(size_t)j * K + k], u += a * wu[(size_t)j * K + k];
                }
                const double want = g / (1.0 + exp(-g)) * u, got = from_f16(O[(size_t)m * I + cols[j]]);
                const double err = fabs(want - got);
                ok = ok && err <= 1e-2 + fabs(want) * 0x1p-11;
                worst = err > worst ? err : worst;
                num += err * err, den += want * want;
            }
        const double rel = den > 0 ? sqrt(num / den) : sqrt(num);
        ok = ok && rel <= 1e-3;
        if (!ok) (*failed)++;
        if (verbose || !ok)
            printf("  gate/up+SwiGLU M=%-4d I=%-6u K=%-6u rel-L2 %.2e max-abs %.2e  %s\n", M, I, K, rel, worst, ok ? "ok" : "FAIL");
    }
    return 0;
}

// The fused single-token gate/up+SwiGLU kernel against hq_gemm on gate and up plus k_swiglu.
int selftest_fused(HipBackend *b, int verbose, int *failed) {
    const hq_ref_config_t &c = b->m->cfg;
    const int H = (int)c.hidden, I = (int)c.intermediate;
    uint64_t seed = 99;
    std::vector<uint16_t> a(H);
    for (auto &x : a) x = to_f16((float)((double)lcg(&seed) / (double)(1ull << 31) * 2.0 - 1.0));
    BCK(hipMemcpy(b->hb, a.data(), (size_t)H * 2, hipMemcpyHostToDevice));
    const DevLayer &L = b->L[0];
    k_gateup_swiglu<<<(I + 3) / 4, 256, 0, b->st>>>(*hq_mat_dev(L.gate), *hq_mat_dev(L.up), b->hb, b->fb, I, H);
    BCK(hipGetLastError());
    std::vector<uint16_t> fused(I), plain(I);
    BCK(hipMemcpyAsync(fused.data(), b->fb, (size_t)I * 2, hipMemcpyDeviceToHost, b->st));
    if (gemm(b, L.gate, b->hb, 1, b->gb, false) || gemm(b, L.up, b->hb, 1, b->ub, false)) return -1;
    k_swiglu<<<blocks_for((size_t)I, 256), 256, 0, b->st>>>(b->gb, b->ub, b->fb, (size_t)I);
    BCK(hipGetLastError());
    BCK(hipMemcpyAsync(plain.data(), b->fb, (size_t)I * 2, hipMemcpyDeviceToHost, b->st));
    BCK(hipStreamSynchronize(b->st));
    double worst = 0, scale = 0;
    for (int i = 0; i < I; i++) {
        const double p = from_f16(plain[i]), f = from_f16(fused[i]);
        worst = fabs(p - f) > worst ? fabs(p - f) : worst;
        scale = fabs(p) > scale ? fabs(p) : scale;
    }
    const bool ok = worst <= 1e-3 * (1.0 + scale);
    if (!ok) (*failed)++;
    if (verbose || !ok) printf("  fused gate/up+SwiGLU (T = 1) vs unfused: max-abs %.2e (max |y| %.2f)  %s\n", worst, scale, ok ? "ok" : "FAIL");
    return 0;
}

void compare(const char *what, const float *ref, const float *got, uint32_t n, double tol, int *failed) {
    double worst = 0;
    uint32_t ar = 0, ag = 0;
    for (uint32_t k = 0; k < n; k++) {
        worst = fabs((double)ref[k] - got[k]) > worst ? fabs((double)ref[k] - got[k]) : worst;
        if (ref[k] > ref[ar]) ar = k;
        if (got[k] > got[ag]) ag = k;
    }
    const bool ok = worst <= tol && ar == ag;
    if (!ok) (*failed)++;
    printf("  %-40s max|dlogit| %.2e  argmax %s  %s\n", what, worst, ar == ag ? "same" : "DIFF", ok ? "ok" : "FAIL");
}

}  // namespace

extern "C" int hq_gemv_swiglu(const hq_mat *gate, const hq_mat *up, const uint16_t *a, uint16_t *out, void *stream) {
    if (!gate || !up || !a || !out) return hq_internal_fail("hq_gemv_swiglu: null argument");
    uint32_t rg, kg, ru, ku;
    if (hq_mat_shape(gate, &rg, &kg, nullptr) || hq_mat_shape(up, &ru, &ku, nullptr)) return -1;
    if (rg != ru || kg != ku) return hq_internal_fail("hq_gemv_swiglu: gate [%u, %u] and up [%u, %u] differ", rg, kg, ru, ku);
    if (hq_mat_device(gate) != hq_mat_device(up)) return hq_internal_fail("hq_gemv_swiglu: gate and up on different devices");
    if ((uintptr_t)a % 16 || (uintptr_t)out % 2) return hq_internal_fail("hq_gemv_swiglu: a must be 16-byte aligned");
    BCK(hipSetDevice(hq_mat_device(gate)));
    k_gateup_swiglu<<<(rg + 3) / 4, 256, 0, (hipStream_t)stream>>>(*hq_mat_dev(gate), *hq_mat_dev(up), (const _Float16 *)a,
                                                                  (_Float16 *)out, (int)rg, (int)kg);
    BCK(hipGetLastError());
    return 0;
}

// The reference CPU backend, when the program that loads this library provides it (the reference
// binary does: src/cpu_backend.c); a weak reference, so the library loads without it.
extern "C" hq_ref_backend_t *cpu_backend_create(const hq_ref_model_t *m, size_t max_seq) __attribute__((weak));

extern "C" hq_ref_backend_t *hip_backend_create(const hq_ref_model_t *m, size_t max_seq, int device, bool keep_quantized) {
    if (!m) {
        hq_internal_fail("hip_backend_create: no model");
        return nullptr;
    }
    if (!keep_quantized) {
        hq_internal_fail("hip_backend_create: weights are kept in their GGUF blocks (keep_quantized must be true)");
        return nullptr;
    }
    HipBackend *b = new HipBackend();
    b->m = m;
    b->device = device;
    b->base.name = "hip-gguf-quantized";
    b->base.reset = be_reset;
    b->base.forward = be_forward;
    b->base.snapshot = be_snapshot;
    b->base.restore = be_restore;
    b->base.destroy = be_destroy;
    b->base.last_hidden = be_last_hidden;
    b->base.max_seq = max_seq;
    b->base.pos = 0;
    if (init(b, m, max_seq)) {
        char msg[512];
        snprintf(msg, sizeof msg, "%s", hq_last_error());
        release(b);
        hq_internal_fail("%s", msg);
        return nullptr;
    }
    return &b->base;
}

extern "C" int hip_selftest(const hq_ref_model_t *m, int device, size_t n_tokens, int verbose) {
    if (!m) return hq_internal_fail("hip_selftest: no model");
    if (n_tokens < 2) n_tokens = 2;
    const hq_ref_config_t &c = m->cfg;
    const size_t ctx = n_tokens > 2048 ? n_tokens : 2048;
    hq_ref_backend_t *gpu = hip_backend_create(m, ctx, device, true);
    if (!gpu) return -1;
    HipBackend *b = self(gpu);
    int failed = 0, rc = 0;
    printf("hq_gemm on the model's matrices vs a float64 host product of the decoded weights:\n");
    const DevLayer &L0 = b->L[0];
    rc = selftest_gemm(L0.q, "q", verbose, &failed, b->st) || selftest_gemm(L0.down, "down", verbose, &failed, b->st) ||
         (!L0.pair && selftest_gemm(L0.gate, "gate", verbose, &failed, b->st));
    if (L0.pair) {
        printf("hq_gemm_swiglu on the gate/up pair vs silu(g) * u from the decoded weights in float64:\n");
        rc = rc || selftest_swiglu(L0.pair, verbose, &failed, b->st);
    } else {
        printf("fused single-token kernel vs the unfused kernels:\n");
        rc = rc || selftest_fused(b, verbose, &failed);
    }
    uint64_t seed = 7;
    std::vector<uint32_t> tok(n_tokens), ids(16);
    for (auto &t : tok) t = (uint32_t)(lcg(&seed) % c.vocab);
    for (auto &i : ids) i = (uint32_t)(lcg(&seed) % c.vocab);
    float full[16], split[16], step[16], ref[16];
    std::vector<float> hg(c.hidden), hc(c.hidden);
    const size_t half = n_tokens / 2;
    double t0 = now_s();
    rc = rc || gpu->reset(gpu) || gpu->forward(gpu, tok.data(), n_tokens, ids.data(), 16, full);
    const double gpu_s = now_s() - t0;
    rc = rc || gpu->last_hidden(gpu, hg.data());  // after the full prefill
    rc = rc || gpu->reset(gpu) || gpu->forward(gpu, tok.data(), half, nullptr, 0, nullptr) || gpu->snapshot(gpu) ||
         gpu->forward(gpu, tok.data() + half, n_tokens - half, ids.data(), 16, split) || gpu->restore(gpu) ||
         gpu->forward(gpu, tok.data() + half, n_tokens - half, ids.data(), 16, split);
    rc = rc || gpu->reset(gpu) || gpu->forward(gpu, tok.data(), n_tokens - 1, nullptr, 0, nullptr) ||
         gpu->forward(gpu, tok.data() + n_tokens - 1, 1, ids.data(), 16, step);
    if (!rc) {
        printf("forward pass, %zu tokens (hip %.4f s):\n", n_tokens, gpu_s);
        compare("prefix+restore+suffix vs full prefill", full, split, 16, 1e-3, &failed);
        compare("prefill + 1-token step vs full prefill", full, step, 16, 1e-3, &failed);
        if (cpu_backend_create) {
            hq_ref_backend_t *cpu = cpu_backend_create(m, n_tokens);
            if (!cpu || cpu->reset(cpu) || cpu->forward(cpu, tok.data(), n_tokens, ids.data(), 16, ref) ||
                cpu->last_hidden(cpu, hc.data())) {
                if (cpu) cpu->destroy(cpu);
                rc = hq_internal_fail("hip_selftest: the CPU reference forward failed");
            } else {
                cpu->destroy(cpu);
                compare("hip vs cpu (full prefill)", ref, full, 16, 1e-2, &failed);
                // the reference's direction check of the final hidden state (src/cuda_backend.cu:1440-1446)
                double dot = 0, nc = 0, ng = 0;
                for (uint32_t k = 0; k < c.hidden; k++)
                    dot += (double)hc[k] * hg[k], nc += (double)hc[k] * hc[k], ng += (double)hg[k] * hg[k];
                const double cosine = nc > 0 && ng > 0 ? dot / sqrt(nc * ng) : 0;
                const bool ok = cosine >= 0.999;
                if (!ok) failed++;
                printf("  %-40s cosine %.6f  %s\n", "hip vs cpu final hidden state", cosine, ok ? "ok" : "FAIL");
            }
        } else {
            printf("  (no cpu_backend_create in this program: the CPU comparison is left to the caller)\n");
        }
        // prefill throughput at a realistic prompt length (src/cuda_backend.cu:1447-1457): one warm-up
        // pass, then the timed one
        const size_t bench = ctx < 2048 ? ctx : 2048;
        std::vector<uint32_t> bt(bench);
        for (size_t t = 0; t < bench; t++) bt[t] = tok[t % n_tokens];
        rc = gpu->reset(gpu) || gpu->forward(gpu, bt.data(), bench, ids.data(), 2, full);
        t0 = now_s();
        rc = rc || gpu->reset(gpu) || gpu->forward(gpu, bt.data(), bench, ids.data(), 2, full);
        const double dt = now_s() - t0;
        if (!rc) printf("  hip prefill %zu tokens: %.2f ms (%.0f tokens/s)\n", bench, dt * 1e3, (double)bench / dt);
    }
    gpu->destroy(gpu);
    if (rc) return -1;
    if (failed) return hq_internal_fail("hip_selftest: %d check(s) failed", failed);
    printf("selftest passed\n");
    return 0;
}
