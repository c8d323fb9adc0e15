/* op_common.c — device facts the operator planners need. */
#include "op_common.h"
#include "gpu_ops.h"

#define CF_MAX_DEV 16

int cf_cu_count(void) {
    static int cached[CF_MAX_DEV];
    gpu_caps_t caps;
    int dev = gpu_current_device();
    if (dev < 0 || dev >= CF_MAX_DEV) dev = 0;
    if (cached[dev] > 0) return cached[dev];
    if (gpu_get_gpu_caps(&caps, dev) != 0 || caps.cu_count <= 0) return 256;
    cached[dev] = caps.cu_count;
    return cached[dev];
}
