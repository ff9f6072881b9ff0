/* hq_oracle.h - CPU oracle for the quantized matmul path (TEST INFRASTRUCTURE ONLY).
 *
 * A plain-C restatement of the reference engine's CPU arithmetic on the hot path, used
 * by tests/, bench.py's cpu_baseline leg and __graft_entry__.smoke() as the checker.
 * Nothing in the product library links, loads or calls this code.
 *
 * Reference files restated (paths relative to cleanroom-transformer/):
 *   src/ops_common.h:32-53      fp16 -> fp32                      or_f16_to_f32
 *   src/ggml_quant.h:22-47      block values / bytes              or_block_values, or_block_bytes
 *   src/gguf.c:54-57            bytes per row                     or_row_bytes
 *   src/ggml_quant.h:51-59      6-bit scale/min unpack (k-quants) or_scale_min_k4
 *   src/ggml_quant.h:95-99      Q8_0 32-value block decode        or_dequant_sub32 (Q8_0)
 *   src/ggml_quant.h:100-111    Q2_K sub-block decode             or_dequant_sub32 (Q2_K)
 *   src/ggml_quant.h:112-134    Q3_K sub-block decode             or_dequant_sub32 (Q3_K), q3k_scale
 *   src/ggml_quant.h:135-150    Q4_K / Q5_K sub-block decode      or_dequant_sub32 (Q4_K, Q5_K)
 *   src/ggml_quant.h:151-169    Q6_K sub-block decode             or_dequant_sub32 (Q6_K)
 *   src/gguf.c:59-73            row decode                        or_dequantize_row
 *   src/model.c:283-307         q/k row un-permute, row widen     or_src_row, or_wmat_row_f32
 *   src/cpu_backend.c:28-36     8-partial dot                     or_dot
 *   src/cpu_backend.c:39-54     row-parallel matmul               or_matmul
 *   src/cpu_backend.c:253-259   option-row readout                or_gather_dot
 *   src/cpu_backend.c:57-62, 77-133, 218-263, src/model.c:450-469
 *                               Llama forward (config 1)          or_llama_forward
 *
 * Pinning: every function is checked in tests/ against the reference compiled from its own
 * sources (oracle/_ref, bit-exact), against committed golden vectors produced by that build,
 * and against closed forms (brute force over all 6-bit scale/min codes, all nibble and int8
 * values, fp16 subnormal/inf/NaN scales, double-precision products).
 */
#ifndef HQ_ORACLE_H
#define HQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_GGML_Q8_0 = 8, OR_GGML_Q2_K = 10, OR_GGML_Q3_K = 11, OR_GGML_Q4_K = 12, OR_GGML_Q5_K = 13, OR_GGML_Q6_K = 14 };

/* Same field order and types as the reference wmat_t (src/transformer.h:293-300). dtype is
 * always 3 (DT_GGML) here; only block-quantized matrices are on this path. */
typedef struct {
    int dtype;
    uint32_t rows, cols;
    const void *data;
    int ggml_type;
    uint32_t perm_heads;
} or_wmat_t;

float or_f16_to_f32(uint16_t h);
uint32_t or_block_values(int type);
uint32_t or_block_bytes(int type);
size_t or_row_bytes(int type, uint64_t cols);
void or_scale_min_k4(int j, const uint8_t *q, uint8_t *s, uint8_t *m);
void or_dequant_sub32(int type, const uint8_t *block, int sub, float *y);
void or_dequantize_row(int type, const void *src, float *out, uint64_t cols);
uint32_t or_src_row(const or_wmat_t *w, uint32_t r);
void or_wmat_row_f32(const or_wmat_t *w, uint32_t r, float *out);
float or_dot(const float *a, const float *b, size_t n);
/* y[t*rows + r] (+)= dot(x[t*cols ..], W[r]) for t < T; OpenMP over rows when built with -fopenmp. */
void or_matmul(const or_wmat_t *w, const float *x, size_t T, float *y, int accumulate);
/* Same, for rows [r0, r1) only: the CPU-baseline timing sample. */
void or_matmul_rows(const or_wmat_t *w, const float *x, size_t T, float *y, int accumulate, uint32_t r0, uint32_t r1);
/* out[b*k + j] = dot(h[b*cols ..], W[ids[b*k + j]]) for b < B, j < k. */
void or_gather_dot(const or_wmat_t *w, const float *h, const uint32_t *ids, size_t B, size_t k, float *out);
/* Widen fp16 bit patterns to float (exact). */
void or_f16_to_f32_array(const uint16_t *in, float *out, size_t n);

/* Tiny Llama model for config 1 (subset of the reference model_t / layer_t / config_t). */
typedef struct {
    or_wmat_t q, k, v, o, gate, up, down;
    const float *in_norm, *post_norm;
} or_layer_t;

typedef struct {
    uint32_t hidden, n_layers, intermediate, vocab, n_heads, n_kv_heads, head_dim, rot_dim;
    float eps, rope_theta;
    or_wmat_t embed, lm_head;
    const float *final_norm;
    const or_layer_t *layers;
    const float *rope_inv_freq; /* optional [rot_dim / 2] table (model_t.rope_inv_freq); NULL: theta powers */
} or_llama_t;

/* One prefill from position 0 of T tokens; logits for ids at the last position.
 * Returns 0, or -1 on an empty prompt or an out-of-range token / id. */
int or_llama_forward(const or_llama_t *m, const uint32_t *tokens, size_t T, const uint32_t *ids, uint32_t n_ids,
                     float *logits);
/* The same, also writing the final-normalised last position (the CPU backend's last_hidden) to
 * hidden [hidden floats] when it is not NULL. */
int or_llama_forward_h(const or_llama_t *m, const uint32_t *tokens, size_t T, const uint32_t *ids, uint32_t n_ids,
                       float *logits, float *hidden);

#ifdef __cplusplus
}
#endif
#endif
