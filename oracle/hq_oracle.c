/* hq_oracle.c - CPU oracle for the quantized matmul path (TEST INFRASTRUCTURE ONLY).
 *
 * Restates the reference engine's CPU arithmetic (cleanroom-transformer/src/...) in this
 * project's own code. Built with the reference's flags (-O2 -std=c11 -fopenmp, no -march, so no
 * FMA contraction) so that float results are bit-identical to the reference CPU backend.
 * Only tests/, bench.py (cpu_baseline) and __graft_entry__.smoke() use this file.
 */
#include "hq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* src/ops_common.h:32-53. Exact for every bit pattern: normals rebias the exponent, subnormals
 * are f * 2^-24 (exact in float), inf/NaN keep their payload shifted into the float mantissa. */
float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, f = h & 1023u;
    uint32_t bits;
    if (e == 31u) {
        bits = sign | 0x7f800000u | (f << 13);
    } else if (e != 0u) {
        bits = sign | ((e + 112u) << 23) | (f << 13);
    } else if (f == 0u) {
        bits = sign;
    } else {
        float v = (float)f * 0x1p-24f;
        return sign ? -v : v;
    }
    float out;
    memcpy(&out, &bits, sizeof out);
    return out;
}

void or_f16_to_f32_array(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(in[i]);
}

/* src/ggml_quant.h:22-47 (the formats on this path; 0 = unsupported) */
uint32_t or_block_values(int type) {
    switch (type) {
    case OR_GGML_Q8_0: return 32u;
    case OR_GGML_Q2_K: case OR_GGML_Q3_K: case OR_GGML_Q4_K: case OR_GGML_Q5_K: case OR_GGML_Q6_K: return 256u;
    default: return 0u;
    }
}
uint32_t or_block_bytes(int type) {
    switch (type) {
    case OR_GGML_Q8_0: return 34u;
    case OR_GGML_Q2_K: return 84u;
    case OR_GGML_Q3_K: return 110u;
    case OR_GGML_Q4_K: return 144u;
    case OR_GGML_Q5_K: return 176u;
    case OR_GGML_Q6_K: return 210u;
    default: return 0u;
    }
}

/* src/gguf.c:54-57 */
size_t or_row_bytes(int type, uint64_t cols) {
    const uint32_t per = or_block_values(type);
    return per ? (size_t)(cols / per) * or_block_bytes(type) : 0;
}

static float le_f16(const uint8_t *p) { return or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* src/ggml_quant.h:51-59. Twelve bytes hold eight 6-bit scales and eight 6-bit mins: entries
 * 0-3 sit in the low 6 bits of bytes 0-3 (scale) and 4-7 (min); entries 4-7 take their low
 * nibble from bytes 8-11 (scale: low nibble, min: high nibble) and their top 2 bits from the
 * spare top bits of bytes 0-3 (scale) and 4-7 (min). */
void or_scale_min_k4(int j, const uint8_t *q, uint8_t *s, uint8_t *m) {
    if (j < 4) {
        *s = (uint8_t)(q[j] & 0x3f);
        *m = (uint8_t)(q[4 + j] & 0x3f);
        return;
    }
    const uint8_t lo = q[4 + j];
    *s = (uint8_t)((lo & 0x0f) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((lo >> 4) | ((q[j] >> 6) << 4));
}

/* Q3_K 6-bit scale e (0..15) from the 12 packed bytes at sc (src/ggml_quant.h:118-128): the low
 * nibble of scale 4g + i (g = 0..3, i = 0..3) is nibble g / 2 of byte 4 (g % 2) + i, its top two
 * bits are bits 2g, 2g + 1 of byte 8 + i. */
static int q3k_scale(const uint8_t *sc, int e) {
    const int g = e >> 2, i = e & 3;
    const int lo = (sc[4 * (g & 1) + i] >> (4 * (g >> 1))) & 0x0f, hi = (sc[8 + i] >> (2 * g)) & 3;
    return lo | (hi << 4);
}

/* Sub-block `sub` (32 values) of one block.
 * Q8_0 (src/ggml_quant.h:95-99): {fp16 d; int8 q[32]}, y = q * d (exact in float).
 * Q4_K / Q5_K (src/ggml_quant.h:135-150): {fp16 d, fp16 dmin, u8 scales[12], [Q5_K: u8 qh[32],]
 * u8 qs[128]}; sub-block j reads nibble (j odd: high, even: low) of qs[32*(j/2) + l], Q5_K adds
 * 16 where bit j of qh[l] is set; y = (d*s)*q - dmin*m, where the two products are exact in float
 * and only the subtraction rounds. */
void or_dequant_sub32(int type, const uint8_t *b, int sub, float *y) {
    if (type == OR_GGML_Q8_0) {
        const float d = le_f16(b);
        for (int l = 0; l < 32; l++) y[l] = (float)(int8_t)b[2 + l] * d;
        return;
    }
    if (type == OR_GGML_Q4_K || type == OR_GGML_Q5_K) {
        const int five = type == OR_GGML_Q5_K;
        uint8_t s, m;
        or_scale_min_k4(sub, b + 4, &s, &m);
        const float ds = le_f16(b) * (float)s, dm = le_f16(b + 2) * (float)m;
        const uint8_t *qs = b + (five ? 48 : 16) + 32 * (sub >> 1), *qh = b + 16;
        const int shift = (sub & 1) ? 4 : 0;
        for (int l = 0; l < 32; l++) {
            const int q = ((qs[l] >> shift) & 0x0f) + (five ? 16 * ((qh[l] >> sub) & 1) : 0);
            y[l] = ds * (float)q - dm;
        }
        return;
    }
    if (type == OR_GGML_Q2_K) {
        /* Q2_K (src/ggml_quant.h:100-111): {u8 scales[16], u8 qs[64], fp16 d, fp16 dmin}. Value
         * 128h + 32j + l (h = 0, 1; j = 0..3) is bits 2j, 2j + 1 of qs[32h + l]; each 16 values have
         * their own byte scales[8h + 2j + l/16]: low nibble s, high nibble m;
         * y = (d*s)*q - dmin*m (both products exact in float, the subtraction rounds). */
        const int h = sub >> 2, j = sub & 3;
        const uint8_t *qs = b + 16 + 32 * h;
        const float d = le_f16(b + 80), dmin = le_f16(b + 82);
        for (int l = 0; l < 32; l++) {
            const uint8_t sm = b[8 * h + 2 * j + (l >> 4)];
            const float ds = d * (float)(sm & 0x0f), dm = dmin * (float)(sm >> 4);
            y[l] = ds * (float)((qs[l] >> (2 * j)) & 3) - dm;
        }
        return;
    }
    if (type == OR_GGML_Q3_K) {
        /* Q3_K (src/ggml_quant.h:112-134): {u8 hmask[32], u8 qs[64], u8 scales[12], fp16 d}. Value
         * 128h + 32j + l is bits 2j, 2j + 1 of qs[32h + l] minus 4 unless bit 4h + j of hmask[l] is
         * set; 16 values share the 6-bit scale 8h + 2j + l/16 (q3k_scale), offset by -32;
         * y = (d * (sc - 32)) * q, both products exact in float. */
        const int h = sub >> 2, j = sub & 3;
        const uint8_t *qs = b + 32 + 32 * h;
        const float d = le_f16(b + 108);
        for (int l = 0; l < 32; l++) {
            const float dl = d * (float)(q3k_scale(b + 96, 8 * h + 2 * j + (l >> 4)) - 32);
            const int q = ((qs[l] >> (2 * j)) & 3) - ((b[l] >> (4 * h + j)) & 1 ? 0 : 4);
            y[l] = dl * (float)q;
        }
        return;
    }
    if (type == OR_GGML_Q6_K) {
        /* Q6_K (src/ggml_quant.h:151-169): {u8 ql[128], u8 qh[64], int8 scales[16], fp16 d}. The
         * 256 values form two halves of 128; in half h, value 32r + l (r = 0..3, l = 0..31) takes
         * its low 4 bits from ql[64h + l + 32(r % 2)] (low nibble for r < 2, high for r >= 2), its
         * top 2 bits from bits 2r, 2r+1 of qh[32h + l], is offset by -32, and is scaled by
         * scales[8h + 2r + l/16] and d: y = (d * sc) * q, where d * sc is exact in float and the
         * second product can round. */
        const int h = sub >> 2, r = sub & 3;
        const uint8_t *ql = b + 64 * h + 32 * (r & 1), *qh = b + 128 + 32 * h;
        const int8_t *sc = (const int8_t *)(b + 192) + 8 * h + 2 * r;
        const float d = le_f16(b + 208);
        for (int l = 0; l < 32; l++) {
            const int lo = (r < 2 ? ql[l] : ql[l] >> 4) & 0x0f, hi = (qh[l] >> (2 * r)) & 3;
            const int q = (lo | (hi << 4)) - 32;
            y[l] = d * (float)sc[l >> 4] * (float)q;
        }
    }
}

/* src/gguf.c:59-73: a row is decoded 32 values at a time; value u*32 lies in block u*32/per. */
void or_dequantize_row(int type, const void *src, float *out, uint64_t cols) {
    const uint8_t *p = (const uint8_t *)src;
    const uint32_t per = or_block_values(type), bytes = or_block_bytes(type);
    if (!per) return;
    for (uint64_t u = 0; u < cols / 32; u++) {
        const uint64_t first = u * 32;
        or_dequant_sub32(type, p + (first / per) * bytes, (int)((first % per) / 32), out + first);
    }
}

/* src/model.c:283-289. llama.cpp stores each head's rotary pairs interleaved: storage row
 * 2i+j of a head holds Hugging Face row j*(hd/2)+i. Returns the storage row of HF row r. */
uint32_t or_src_row(const or_wmat_t *w, uint32_t r) {
    if (!w->perm_heads) return r;
    const uint32_t hd = w->rows / w->perm_heads, half = hd / 2, within = r % hd;
    return (r - within) + 2 * (within % half) + within / half;
}

/* src/model.c:291-307 (DT_GGML branch) */
void or_wmat_row_f32(const or_wmat_t *w, uint32_t r, float *out) {
    const size_t rb = or_row_bytes(w->ggml_type, w->cols);
    or_dequantize_row(w->ggml_type, (const uint8_t *)w->data + (size_t)or_src_row(w, r) * rb, out, w->cols);
}

/* src/cpu_backend.c:28-36: eight float partial sums over k mod 8, combined as
 * ((p0+p1)+(p2+p3))+((p4+p5)+(p6+p7)), then a scalar tail. */
float or_dot(const float *a, const float *b, size_t n) {
    float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t k;
    for (k = 0; k + 8 <= n; k += 8)
        for (int j = 0; j < 8; j++) p[j] += a[k + j] * b[k + j];
    float s = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    for (; k < n; k++) s += a[k] * b[k];
    return s;
}

/* src/cpu_backend.c:39-54: each thread widens one weight row at a time, then forms the T dots
 * against it; rows are split statically across threads. */
void or_matmul_rows(const or_wmat_t *w, const float *x, size_t T, float *y, int accumulate, uint32_t r0, uint32_t r1) {
    const size_t N = w->rows, K = w->cols;
    const long lo = (long)r0, hi = (long)r1;
#pragma omp parallel
    {
        float *row = (float *)malloc(K * sizeof *row);
#pragma omp for schedule(static)
        for (long r = lo; r < hi; r++) {
            or_wmat_row_f32(w, (uint32_t)r, row);
            for (size_t t = 0; t < T; t++) {
                const float v = or_dot(x + t * K, row, K);
                float *dst = y + t * N + (size_t)r;
                *dst = accumulate ? *dst + v : v;
            }
        }
        free(row);
    }
}

void or_matmul(const or_wmat_t *w, const float *x, size_t T, float *y, int accumulate) {
    or_matmul_rows(w, x, T, y, accumulate, 0, w->rows);
}

/* src/cpu_backend.c:253-259: each selected row is widened and dotted with the hidden state. */
void or_gather_dot(const or_wmat_t *w, const float *h, const uint32_t *ids, size_t B, size_t k, float *out) {
    const size_t K = w->cols;
    const long pairs = (long)(B * k);
#pragma omp parallel
    {
        float *row = (float *)malloc(K * sizeof *row);
#pragma omp for schedule(static)
        for (long i = 0; i < pairs; i++) {
            or_wmat_row_f32(w, ids[i], row);
            out[i] = or_dot(h + (size_t)(i / (long)k) * K, row, K);
        }
        free(row);
    }
}

/* ----------------------------------------------------------------- config-1 forward */

/* src/cpu_backend.c:57-62: sum of squares in double; out = x * inv * (0 + w) for Llama. */
static void rms_norm(const float *x, const float *w, float *out, size_t n, float eps) {
    double ss = 0.0;
    for (size_t i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float inv = 1.0f / sqrtf((float)(ss / (double)n) + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] * inv * (0.0f + w[i]);
}

static float silu(float v) { return v / (1.0f + expf(-v)); }

/* src/cpu_backend.c:77-133 for a Llama layer (no q/k norm, no output gate), positions 0..T-1. */
static void attention(const or_llama_t *m, const or_layer_t *L, const float *h, size_t T, float *out,
                      const float *inv_freq) {
    const size_t nh = m->n_heads, nkv = m->n_kv_heads, hd = m->head_dim, rot = m->rot_dim;
    const size_t qw = nh * hd, kvw = nkv * hd;
    float *q = (float *)malloc(T * qw * sizeof *q), *k = (float *)malloc(T * kvw * sizeof *k);
    float *v = (float *)malloc(T * kvw * sizeof *v);
    or_matmul(&L->q, h, T, q, 0);
    or_matmul(&L->k, h, T, k, 0);
    or_matmul(&L->v, h, T, v, 0);
    for (size_t t = 0; t < T; t++) {
        const float pos = (float)t;
        for (size_t j = 0; j < nh + nkv; j++) {
            float *x = j < nh ? q + t * qw + j * hd : k + t * kvw + (j - nh) * hd;
            for (size_t i = 0; i < rot / 2; i++) {
                const float ang = inv_freq[i] * pos, c = cosf(ang), s = sinf(ang);
                const float x1 = x[i], x2 = x[i + rot / 2];
                x[i] = x1 * c - x2 * s;
                x[i + rot / 2] = x2 * c + x1 * s;
            }
        }
    }
    const float scale = 1.0f / sqrtf((float)hd);
    const long work = (long)(T * nh);
#pragma omp parallel
    {
        float *sc = (float *)malloc(T * sizeof *sc);
#pragma omp for schedule(dynamic, 4)
        for (long wi = 0; wi < work; wi++) {
            const size_t t = (size_t)wi / nh, j = (size_t)wi % nh, g = j / (nh / nkv), n = t + 1;
            const float *qv = q + t * qw + j * hd;
            float mx = -INFINITY;
            for (size_t s = 0; s < n; s++) {
                sc[s] = or_dot(qv, k + s * kvw + g * hd, hd) * scale;
                if (sc[s] > mx) mx = sc[s];
            }
            float sum = 0.0f;
            for (size_t s = 0; s < n; s++) sum += (sc[s] = expf(sc[s] - mx));
            float *o = out + t * qw + j * hd;
            memset(o, 0, hd * sizeof *o);
            for (size_t s = 0; s < n; s++) {
                const float *vs = v + s * kvw + g * hd;
                const float pr = sc[s] / sum;
                for (size_t d = 0; d < hd; d++) o[d] += pr * vs[d];
            }
        }
        free(sc);
    }
    free(q), free(k), free(v);
}

/* src/cpu_backend.c:218-263 for a Llama model at position 0; RoPE frequencies the caller's table
 * (model_t.rope_inv_freq, src/model.c:449-477) or, without one, src/model.c:453 (theta powers).
 * hidden (optional, H floats): the final-normalised last position, the CPU backend's last_hidden
 * (src/cpu_backend.c:253-254, :294-298). */
int or_llama_forward_h(const or_llama_t *m, const uint32_t *tokens, size_t T, const uint32_t *ids, uint32_t n_ids,
                       float *logits, float *hidden) {
    if (T == 0) return -1;
    for (size_t t = 0; t < T; t++)
        if (tokens[t] >= m->vocab) return -1;
    for (uint32_t i = 0; i < n_ids; i++)
        if (ids[i] >= m->vocab) return -1;
    const size_t H = m->hidden, I = m->intermediate, qw = (size_t)m->n_heads * m->head_dim;
    float *inv_freq = (float *)malloc(m->rot_dim / 2 * sizeof(float));
    for (uint32_t i = 0; i < m->rot_dim / 2; i++)
        inv_freq[i] = m->rope_inv_freq ? m->rope_inv_freq[i] : 1.0f / powf(m->rope_theta, (float)(2 * i) / (float)m->rot_dim);
    float *x = (float *)malloc(T * H * sizeof *x), *h = (float *)malloc(T * H * sizeof *h);
    float *mix = (float *)malloc(T * qw * sizeof *mix);
    float *g = (float *)malloc(T * I * sizeof *g), *u = (float *)malloc(T * I * sizeof *u);
    for (size_t t = 0; t < T; t++) or_wmat_row_f32(&m->embed, tokens[t], x + t * H);
    for (uint32_t l = 0; l < m->n_layers; l++) {
        const or_layer_t *L = &m->layers[l];
        for (size_t t = 0; t < T; t++) rms_norm(x + t * H, L->in_norm, h + t * H, H, m->eps);
        attention(m, L, h, T, mix, inv_freq);
        or_matmul(&L->o, mix, T, x, 1);
        for (size_t t = 0; t < T; t++) rms_norm(x + t * H, L->post_norm, h + t * H, H, m->eps);
        or_matmul(&L->gate, h, T, g, 0);
        or_matmul(&L->up, h, T, u, 0);
        for (size_t i = 0; i < T * I; i++) g[i] = silu(g[i]) * u[i];
        or_matmul(&L->down, g, T, x, 1);
    }
    rms_norm(x + (T - 1) * H, m->final_norm, h, H, m->eps);
    if (hidden) memcpy(hidden, h, H * sizeof *hidden);
    float *row = (float *)malloc(H * sizeof *row);
    for (uint32_t i = 0; i < n_ids; i++) {
        or_wmat_row_f32(&m->lm_head, ids[i], row);
        logits[i] = or_dot(h, row, H);
    }
    free(row), free(x), free(h), free(mix), free(g), free(u), free(inv_freq);
    return 0;
}

int or_llama_forward(const or_llama_t *m, const uint32_t *tokens, size_t T, const uint32_t *ids, uint32_t n_ids,
                     float *logits) {
    return or_llama_forward_h(m, tokens, T, ids, n_ids, logits, NULL);
}
