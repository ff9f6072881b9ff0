/* hq_llama.h - config-1 caller context: the reference CPU forward pass for a Llama-architecture
 * model with every linear layer and the option readout routed through the HIP matmul path.
 *
 * Mirrors cpu_forward (cleanroom-transformer/src/cpu_backend.c:218-263) for LAYER_FULL layers of a
 * Llama config (src/model.c:60-107: no q/k norm, no output gate, RMSNorm offset 0): embedding
 * rows, RMSNorm, RoPE, causal attention and SwiGLU run on the host in fp32 as the reference does;
 * q/k/v/o/gate/up/down go through hq_matmul_host (src/cpu_backend.c:82-84, :242, :248-251) and
 * the lm_head readout through hq_gather_dot (src/cpu_backend.c:253-259).
 */
#ifndef HQ_LLAMA_H
#define HQ_LLAMA_H

#include "hq.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Subset of the reference layer_t (src/transformer.h:307-318) for full-attention layers. */
typedef struct {
    hq_mat *q, *k, *v, *o, *gate, *up, *down; /* resident; q/k uploaded with perm_heads */
    const float *in_norm, *post_norm;         /* host, hidden floats */
} hq_llama_layer_t;

/* Subset of the reference config_t / model_t (src/transformer.h:278-329). */
typedef struct {
    uint32_t hidden, n_layers, intermediate, vocab, n_heads, n_kv_heads, head_dim, rot_dim;
    float eps, rope_theta;
    hq_mat *embed, *lm_head;
    const float *final_norm;
    const hq_llama_layer_t *layers;
    /* Optional [rot_dim / 2] RoPE inverse frequencies, as the reference's model_t.rope_inv_freq
     * (src/model.c:449-477: Llama 3.1 frequency scaling and GGUF rope_freqs divisors applied); NULL:
     * 1 / powf(rope_theta, 2k / rot_dim), the unscaled table (src/model.c:453). */
    const float *rope_inv_freq;
} hq_llama_t;

/* One prefill of T tokens from position 0; logits[i] for ids[i] at the last position.
 * Returns 0, or -1 (hq_last_error) on an empty prompt, an out-of-range token or id, or a device
 * error (src/cpu_backend.c:223-228). */
int hq_llama_forward(const hq_llama_t *m, const uint32_t *tokens, size_t T, const uint32_t *ids, uint32_t n_ids,
                     float *logits);

/* Embedding rows from a resident matrix: out[i] = row ids[i] as fp32 (device memory, n x cols).
 * ids on the host, range-checked. Replaces k_embed_q (src/cuda_backend.cu:483-488). */
int hq_embed_f32(const hq_mat *W, const uint32_t *ids, int n, float *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif
