/* hq_gguf.h - GGUF files straight into HBM: a read-only mapping of the file, its tensor table, and
 * hq_wmat_t views of the quantized matrices for hq_mat_upload (include/hq.h), which streams them to
 * the device through pinned staging buffers with asynchronous copies and repacks on the device.
 *
 * Replaces the path the reference takes from disk to GPU memory: gguf_open / gguf_tensor /
 * gguf_tensor_data (cleanroom-transformer/src/gguf.c:134-219, :317-344: mmap, header and tensor
 * table with the general.alignment rule, bounds and block checks) feeding upload_mat
 * (src/cuda_backend.cu:677-699). Errors: -1 with the message in hq_last_error().
 */
#ifndef HQ_GGUF_H
#define HQ_GGUF_H

#include "hq.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hq_gguf hq_gguf;

/* Maps `path` read-only and parses the header (GGUF v2 or v3), metadata and tensor table; tensor
 * data offsets are relative to the data section, aligned to general.alignment (default 32).
 * Malformed or truncated files are refused. */
int hq_gguf_open(const char *path, hq_gguf **out);
void hq_gguf_close(hq_gguf *g);

size_t hq_gguf_n_tensors(const hq_gguf *g);
/* Tensor i: name (NUL-terminated, valid until close), ggml type, dimensions (ne[0] contiguous;
 * unused ones are 1) and the byte offset of its data from the start of the file. */
int hq_gguf_tensor_info(const hq_gguf *g, size_t i, const char **name, int *ggml_type, uint32_t *n_dims, uint64_t ne[4],
                        uint64_t *file_offset);
/* Index of the tensor called `name`; -1 (and a message) when there is none. */
int hq_gguf_find(const hq_gguf *g, const char *name, size_t *index);
/* A scalar unsigned metadata value (u8/u16/u32/u64 types); -1 when absent or of another type. */
int hq_gguf_get_uint(const hq_gguf *g, const char *key, uint64_t *out);

/* hq_wmat_t view of a quantized matrix in the mapping (rows = ne[1] * ne[2] * ne[3], cols = ne[0],
 * dtype DT_GGML, the given perm_heads). Checks that the block type is one hq_mat_upload accepts,
 * that a row is whole blocks and that the data lies inside the file (src/gguf.c:324-344). The
 * view is valid until hq_gguf_close. */
int hq_gguf_wmat(const hq_gguf *g, const char *name, uint32_t perm_heads, hq_wmat_t *out);

#ifdef __cplusplus
}
#endif
#endif
