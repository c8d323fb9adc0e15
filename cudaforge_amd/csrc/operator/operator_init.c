/* operator_init.c — registers every operator listed in operator_registry.def
 * (X-macro expansion as in src/operator/operator_init.c:25-45). */
#include "operator.h"
#include "mha_ops.h"
#include "rope_ops.h"
#include "layer_ops.h"

int operator_init_all(void) {
    int ret = 0;
#define REGISTER_GPU(fn) ret += fn();
#include "operator_registry.def"
#undef REGISTER_GPU
    return ret;
}
