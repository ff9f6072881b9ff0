/* hq_internal.h - helpers shared by the library's C and HIP sources (not part of the ABI). */
#ifndef HQ_INTERNAL_H
#define HQ_INTERNAL_H

#ifdef __cplusplus
extern "C" {
#endif

/* Records a message for hq_last_error() and returns -1. */
int hq_internal_fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

#ifdef __cplusplus
}
#endif
#endif
