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

#ifdef __cplusplus
}
#endif
#endif
