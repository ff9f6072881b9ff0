/* hq_internal.h - helpers shared by the library's C and HIP sources (not part of the ABI). */
#ifndef HQ_INTERNAL_H
#define HQ_INTERNAL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Records a message for hq_last_error() and returns -1. */
int hq_internal_fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

/* Values and bytes per block of a ggml block type hq_mat_upload accepts: 0, or -1 for other types. */
int hq_internal_block_shape(int ggml_type, uint32_t *values, uint32_t *bytes);
/* The accepted block types, for messages ("Q8_0 = 8, ..."). */
const char *hq_internal_supported_types(void);

#ifdef __cplusplus
}
#endif
#endif
