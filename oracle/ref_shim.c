/* ref_shim.c - exports the reference CPU backend's static matmul/dot (TEST INFRASTRUCTURE ONLY).
 *
 * Compiled by oracle/Makefile together with the reference's own sources, in place under
 * /root/reference/cleanroom-transformer/src, into oracle/_ref/libref.so. The reference source
 * is included, not copied: this file only adds exported wrappers around functions that the
 * reference declares static (src/cpu_backend.c:28, :39; src/ops_common.h:32;
 * src/ggml_quant.h:51, :63), a one-call model + CPU-forward driver (as src/main.c:351-387) and
 * two probes of the reference GGUF reader (src/gguf.c).
 * Used only by tests/ to pin the oracle restatement (oracle/hq_oracle.c) bit for bit.
 */
#include "cpu_backend.c"
#include "ggml_quant.h"

int ref_matmul(const wmat_t *w, const float *x, size_t T, float *y, int accumulate) {
    matmul(w, x, T, y, accumulate != 0);
    return 0;
}

float ref_dot(const float *a, const float *b, size_t n) { return dot(a, b, n); }

float ref_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

void ref_scale_min_k4(int j, const unsigned char *q, uint8_t *s, uint8_t *m) { ggml_scale_min_k4(j, q, s, m); }

void ref_dequant_sub32(int type, const unsigned char *b, int sub, float *y) { ggml_dequant_sub32(type, b, sub, y); }

const char *ref_last_error(void) { return last_error(); }

/* model_load(path) -> CPU backend -> one prefill of n tokens -> logits at ids. 0 / -1. */
int ref_logits(const char *path, const uint32_t *tokens, size_t n, const uint32_t *ids, uint32_t n_ids,
               float *logits, float *last_hidden) {
    model_t m;
    if (model_load(path, &m)) return -1;
    backend_t *be = cpu_backend_create(&m, n);
    int rc = be->reset(be);
    if (!rc) rc = be->forward(be, tokens, n, ids, n_ids, logits);
    if (!rc && last_hidden) rc = be->last_hidden(be, last_hidden);
    be->destroy(be);
    model_free(&m);
    return rc;
}

/* gguf_open + gguf_tensor + gguf_tensor_data (src/gguf.c:134-219, :317-344): the tensor's type,
 * extents and data bytes as the reference reader locates them. 0, or -1 (ref_last_error). */
int ref_gguf_tensor(const char *path, const char *name, int *type, uint64_t ne[4], void *out, size_t cap, size_t *bytes) {
    gguf_t *g;
    if (gguf_open(path, &g)) return -1;
    const gguf_tensor_t *t = gguf_tensor(g, name);
    const void *p = t ? gguf_tensor_data(g, t) : NULL;
    if (!p) {
        if (!t) set_error("no tensor %s", name);
        gguf_close(g);
        return -1;
    }
    *type = t->type;
    for (int d = 0; d < 4; d++) ne[d] = t->ne[d];
    const size_t n = ggml_row_bytes(t->type, t->ne[0]) * (size_t)(t->ne[1] * t->ne[2] * t->ne[3]);
    *bytes = n;
    if (n <= cap) memcpy(out, p, n);
    gguf_close(g);
    return n <= cap ? 0 : -1;
}

/* gguf_open alone (src/gguf.c:134-219): 0 when the reference reader accepts the file's header,
 * metadata and tensor table, else -1 (ref_last_error). */
int ref_gguf_open_ok(const char *path) {
    gguf_t *g;
    if (gguf_open(path, &g)) return -1;
    gguf_close(g);
    return 0;
}
