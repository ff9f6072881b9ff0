/* hq_backend.h - the HIP inference backend: the reference's backend_t vtable over a device-resident
 * layer loop whose every projection goes through hq_gemm (include/hq.h).
 *
 * Drop-in for cuda_backend_create / cuda_selftest (cleanroom-transformer/src/transformer.h:366-372,
 * src/cuda_backend.cu:1003-1024, :1392-1466), selected where the reference's make_backend picks a
 * backend (src/main.c:144-151). The structs below are layout mirrors of the reference's config_t,
 * layer_t, st_set_t, model_t and backend_t (src/transformer.h:229-235, :278-364): a caller passes its
 * model_t * as an hq_ref_model_t * and gets back a backend_t * (field offsets are checked against the
 * reference header by the tests). Names are prefixed; layouts are the reference's, unchanged.
 *
 * Scope: models whose layers are all full attention (LAYER_FULL), as the Llama architecture
 * (src/model.c:60-107) and full-attention Qwen-style layers (optional output gate, q/k RMSNorm,
 * RMSNorm offset); weights in GGUF blocks of a type hq_mat_upload accepts, kept quantized in HBM
 * (keep_quantized must be true: there is no bf16 upload path). A model with Gated-DeltaNet
 * (LAYER_LINEAR) layers, or non-GGUF weights, is refused by hip_backend_create with a message.
 * Errors: NULL / -1 with the message in hq_last_error().
 */
#ifndef HQ_BACKEND_H
#define HQ_BACKEND_H

#include "hq.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { HQ_REF_LAYER_LINEAR = 0, HQ_REF_LAYER_FULL = 1 };  /* src/transformer.h:276 */
enum { HQ_REF_ARCH_QWEN35 = 0, HQ_REF_ARCH_LLAMA = 1 };   /* src/transformer.h:277 */

/* config_t (src/transformer.h:279-293) */
typedef struct {
    uint32_t hidden, n_layers, intermediate, vocab;
    uint32_t n_heads, n_kv_heads, head_dim, rot_dim;
    uint32_t lin_k_heads, lin_v_heads, lin_k_dim, lin_v_dim, conv_k;
    uint32_t arch;
    float eps, rope_theta;
    float norm_offset; /* RMSNorm scale is (norm_offset + w) */
    bool attn_gate, qk_norm, tied;
    bool rope_llama3;
    float rope_factor, rope_low_freq, rope_high_freq, rope_orig_ctx;
    uint8_t layer_type[256];
    uint32_t n_full, n_linear;
} hq_ref_config_t;

/* layer_t (src/transformer.h:307-318); matrices are wmat_t = hq_wmat_t */
typedef struct {
    uint32_t type, slot;
    float *in_norm, *post_norm;
    hq_wmat_t gate, up, down;
    hq_wmat_t q, k, v, o;
    float *q_norm, *k_norm;
    hq_wmat_t qkv, z, b, a, out;
    float *conv_w;
    float *A_log, *dt_bias, *lin_norm;
} hq_ref_layer_t;

/* st_set_t (src/transformer.h:229-235); opaque here */
typedef struct {
    void **files;
    size_t n_files;
    void *tensors;
    size_t n_tensors;
} hq_ref_st_set_t;

/* model_t (src/transformer.h:320-329) */
typedef struct {
    hq_ref_config_t cfg;
    hq_ref_st_set_t st;
    hq_wmat_t embed, lm_head;
    float *final_norm;
    hq_ref_layer_t *layers;
    float *rope_inv_freq; /* [rot_dim / 2], with any Llama 3.1 scaling already applied (src/model.c:450-477) */
    void *gguf;
    char source[512];
} hq_ref_model_t;

/* backend_t (src/transformer.h:347-364) */
typedef struct hq_ref_backend hq_ref_backend_t;
struct hq_ref_backend {
    const char *name;
    int (*reset)(hq_ref_backend_t *);
    int (*forward)(hq_ref_backend_t *, const uint32_t *tokens, size_t n, const uint32_t *ids, uint32_t n_ids,
                   float *logits);
    int (*snapshot)(hq_ref_backend_t *);
    int (*restore)(hq_ref_backend_t *);
    void (*destroy)(hq_ref_backend_t *);
    size_t pos, max_seq;
    int (*last_hidden)(hq_ref_backend_t *, float *out);
};

/* cuda_backend_create (src/cuda_backend.cu:1003-1024): uploads the model to `device` (matrices with
 * hq_mat_upload, norm vectors and RoPE frequencies as fp32) and returns the vtable, reset to
 * position 0. forward is synchronous at return, as the reference's; prompts longer than one chunk
 * are processed in chunks with a KV cache of max_seq positions per layer. */
hq_ref_backend_t *hip_backend_create(const hq_ref_model_t *m, size_t max_seq, int device, bool keep_quantized);

/* cuda_selftest (src/cuda_backend.cu:1392-1466), for this backend: every GEMM path of hq_gemm on
 * the model's own matrices against a float64 host product of the decoded weights; the gate/up +
 * SwiGLU path (hq_gemm_swiglu on the pair matrix at M = 1 .. 200 against float64, or the fused
 * single-token kernel against the unfused kernels where gate and up differ in type); then a forward
 * pass of n_tokens (>= 2) seeded tokens three ways (full prefill; prefix + snapshot + suffix +
 * restore + suffix; prefill of n - 1 tokens + one step) whose logits must agree, and against the
 * reference CPU backend when the program provides cpu_backend_create (logits, and the final hidden
 * state by cosine >= 0.999 as the reference checks it); last, a timed prefill of 2048 tokens
 * (tokens/s printed). Prints a report; returns 0 when every check passes, else -1. */
int hip_selftest(const hq_ref_model_t *m, int device, size_t n_tokens, int verbose);

#ifdef __cplusplus
}
#endif
#endif
