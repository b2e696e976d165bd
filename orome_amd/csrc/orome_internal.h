/* orome_internal.h -- private helpers shared by the C and HIP translation units. */
#ifndef OROME_INTERNAL_H
#define OROME_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Records `msg` as the last error, prints "[hip] msg" to stderr, returns code. */
int orome_fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

struct orome_hip_ctx;
/* Repacks `nblocks` consecutive Q4_K blocks at device address `blocks` from
 * the ggml scale packing to the reference's, on the context's stream, and
 * waits for it. */
int orome_hip_q4k_ggml_to_reference(struct orome_hip_ctx *ctx, void *blocks, size_t nblocks);

#ifdef __cplusplus
}
#endif
#endif
