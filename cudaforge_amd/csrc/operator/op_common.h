/* op_common.h — helpers shared by the HIP operator host code (internal). */
#ifndef CF_OP_COMMON_H_
#define CF_OP_COMMON_H_

#include <stddef.h>
#include <stdint.h>
#include "platform.h"

/* Compute units of the current device (cached after the first query; 256 on MI355X). */
int cf_cu_count(void);

/* Bump carve-up of one workspace region: returns the aligned offset of `bytes` and
 * advances *cursor. */
static inline size_t cf_ws_take(size_t* cursor, size_t bytes) {
    const size_t at = (*cursor + 255) / 256 * 256;
    *cursor = at + bytes;
    return at;
}

static inline void* cf_stream_of(const stream_t* s) { return s ? s->cuda_stream : NULL; }

static inline int64_t cf_ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

#endif /* CF_OP_COMMON_H_ */
