/* hq_llama.c - config-1 caller context: the reference CPU forward pass of a Llama-architecture
 * model (cleanroom-transformer/src/cpu_backend.c:218-263) with every linear layer on the GPU.
 *
 * Host fp32 work, in the reference's order: embedding rows (decoded on the device,
 * hq_embed_f32), RMSNorm with a double sum of squares (src/cpu_backend.c:57-62), RoPE and causal
 * softmax attention (:77-133), SwiGLU (:250). Every projection is hq_matmul_host, the host-pointer
 * drop-in for the reference's static matmul (:39); the readout is hq_gather_dot on the fp16 final
 * hidden state (:253-259). RoPE frequencies follow src/model.c:450-454.
 */
#include "hq_llama.h"

#include "hq_internal.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static void rms_norm(const float *x, const float *w, float *out, size_t n, float eps) {
    double ss = 0.0;
    for (size_t i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float inv = 1.0f / sqrtf((float)(ss / (double)n) + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

static float dot8(const float *a, const float *b, size_t n) {
    float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t k = 0;
    for (; k + 8 <= n; k += 8)
        for (int j = 0; j < 8; j++) p[j] += a[k + j] * b[k + j];
    float s = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    for (; k < n; k++) s += a[k] * b[k];
    return s;
}

static uint16_t f32_to_f16_bits(float f) {
    /* round to nearest even; values here are hidden-state activations, far from fp16 limits */
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const float a = fabsf(f);
    if (!(a == a)) return (uint16_t)(sign | 0x7e00u);
    if (a >= 65520.0f) return (uint16_t)(sign | 0x7c00u);
    if (a < 6.103515625e-05f) {                      /* fp16 subnormal range: multiples of 2^-24 */
        const float q = rintf(a * 16777216.0f);       /* rint: round half to even */
        return (uint16_t)(sign | (uint32_t)q);
    }
    memcpy(&u, &a, 4);
    uint32_t e = (u >> 23) - 127 + 15, man = u & 0x7fffffu;
    uint32_t h = (e << 10) | (man >> 13);
    const uint32_t rest = man & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

typedef struct {
    float *x, *h, *q, *k, *v, *mix, *g, *u, *sc, *inv_freq;
} work_t;

static void work_free(work_t *w) {
    free(w->x), free(w->h), free(w->q), free(w->k), free(w->v), free(w->mix), free(w->g), free(w->u), free(w->sc);
    free(w->inv_freq);
}

int hq_llama_forward(const hq_llama_t *m, const uint32_t *tokens, size_t T, const uint32_t *ids, uint32_t n_ids,
                     float *logits) {
    if (T == 0) return hq_internal_fail("forward: no tokens");
    for (size_t t = 0; t < T; t++)
        if (tokens[t] >= m->vocab) return hq_internal_fail("forward: token %u out of range", tokens[t]);
    for (uint32_t i = 0; i < n_ids; i++)
        if (ids[i] >= m->vocab) return hq_internal_fail("forward: readout id %u out of range", ids[i]);
    const size_t H = m->hidden, I = m->intermediate, nh = m->n_heads, nkv = m->n_kv_heads, hd = m->head_dim;
    const size_t qw = nh * hd, kvw = nkv * hd, rot = m->rot_dim;
    work_t w = {0};
    w.x = malloc(T * H * sizeof(float)), w.h = malloc(T * H * sizeof(float));
    w.q = malloc(T * qw * sizeof(float)), w.k = malloc(T * kvw * sizeof(float)), w.v = malloc(T * kvw * sizeof(float));
    w.mix = malloc(T * qw * sizeof(float)), w.g = malloc(T * I * sizeof(float)), w.u = malloc(T * I * sizeof(float));
    w.sc = malloc(T * sizeof(float)), w.inv_freq = malloc((rot / 2 + 1) * sizeof(float));
    int rc = -1;
    void *dbuf = NULL;
    uint16_t *hf = NULL;
    if (!w.x || !w.h || !w.q || !w.k || !w.v || !w.mix || !w.g || !w.u || !w.sc || !w.inv_freq) {
        hq_internal_fail("forward: out of host memory");
        goto done;
    }
    for (size_t i = 0; i < rot / 2; i++)
        w.inv_freq[i] = m->rope_inv_freq ? m->rope_inv_freq[i] : 1.0f / powf(m->rope_theta, (float)(2 * i) / (float)rot);

    /* embedding rows, decoded on the device */
    const size_t out_off = (n_ids * sizeof(float) + 255) / 256 * 256, emb_bytes = T * H * sizeof(float);
    const size_t dbytes = emb_bytes > out_off + H * sizeof(uint16_t) ? emb_bytes : out_off + H * sizeof(uint16_t);
    if (hq_malloc(&dbuf, dbytes + 64)) goto done;
    if (hq_embed_f32(m->embed, tokens, (int)T, (float *)dbuf, NULL) || hq_device_synchronize() ||
        hq_memcpy_d2h(w.x, dbuf, T * H * sizeof(float), NULL))
        goto done;

    const float scale = 1.0f / sqrtf((float)hd);
    for (uint32_t l = 0; l < m->n_layers; l++) {
        const hq_llama_layer_t *L = &m->layers[l];
        for (size_t t = 0; t < T; t++) rms_norm(w.x + t * H, L->in_norm, w.h + t * H, H, m->eps);
        if (hq_matmul_host(L->q, w.h, T, w.q, false) || hq_matmul_host(L->k, w.h, T, w.k, false) ||
            hq_matmul_host(L->v, w.h, T, w.v, false))
            goto done;
        for (size_t t = 0; t < T; t++) {
            const float pos = (float)t;
            for (size_t j = 0; j < nh + nkv; j++) {
                float *x = j < nh ? w.q + t * qw + j * hd : w.k + t * kvw + (j - nh) * hd;
                for (size_t i = 0; i < rot / 2; i++) {
                    const float ang = w.inv_freq[i] * pos, c = cosf(ang), s = sinf(ang);
                    const float x1 = x[i], x2 = x[i + rot / 2];
                    x[i] = x1 * c - x2 * s;
                    x[i + rot / 2] = x2 * c + x1 * s;
                }
            }
        }
        for (size_t t = 0; t < T; t++)
            for (size_t j = 0; j < nh; j++) {
                const size_t g = j / (nh / nkv), n = t + 1;
                const float *qv = w.q + t * qw + j * hd;
                float mx = -INFINITY;
                for (size_t s = 0; s < n; s++) {
                    w.sc[s] = dot8(qv, w.k + s * kvw + g * hd, hd) * scale;
                    if (w.sc[s] > mx) mx = w.sc[s];
                }
                float sum = 0.0f;
                for (size_t s = 0; s < n; s++) sum += (w.sc[s] = expf(w.sc[s] - mx));
                float *o = w.mix + t * qw + j * hd;
                memset(o, 0, hd * sizeof *o);
                for (size_t s = 0; s < n; s++) {
                    const float *vs = w.v + s * kvw + g * hd, pr = w.sc[s] / sum;
                    for (size_t d = 0; d < hd; d++) o[d] += pr * vs[d];
                }
            }
        if (hq_matmul_host(L->o, w.mix, T, w.x, true)) goto done;
        for (size_t t = 0; t < T; t++) rms_norm(w.x + t * H, L->post_norm, w.h + t * H, H, m->eps);
        if (hq_matmul_host(L->gate, w.h, T, w.g, false) || hq_matmul_host(L->up, w.h, T, w.u, false)) goto done;
        for (size_t i = 0; i < T * I; i++) w.g[i] = w.g[i] / (1.0f + expf(-w.g[i])) * w.u[i];
        if (hq_matmul_host(L->down, w.g, T, w.x, true)) goto done;
    }
    rms_norm(w.x + (T - 1) * H, m->final_norm, w.h, H, m->eps);

    /* readout: fp16 hidden state, gathered option rows */
    if (n_ids) {
        hf = malloc(H * sizeof *hf);
        if (!hf) goto done;
        for (size_t i = 0; i < H; i++) hf[i] = f32_to_f16_bits(w.h[i]);
        float *d_out = (float *)dbuf;
        uint16_t *d_h = (uint16_t *)((char *)dbuf + out_off);
        if (hq_memcpy_h2d(d_h, hf, H * sizeof *hf, NULL) || hq_gather_dot(m->lm_head, d_h, ids, 1, (int)n_ids, d_out, NULL) ||
            hq_memcpy_d2h(logits, d_out, n_ids * sizeof(float), NULL))
            goto done;
    }
    rc = 0;
done:
    if (dbuf) hq_free(dbuf);
    free(hf);
    work_free(&w);
    return rc;
}
