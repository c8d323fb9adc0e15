/*
 * operator.h — operator-layer API: op signature, registry entry, lookup.
 *
 * Same types, signature and semantics as the reference operator layer
 * (src/operator/include/operator.h:14-46): an op receives packed input and output
 * pointer arrays, an op-specific params struct and a stream, and returns 0 on success,
 * -1 on invalid arguments, or a positive HIP error code on a failed launch.
 */
#ifndef CF_OPERATOR_H_
#define CF_OPERATOR_H_

#include "platform.h"
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque base of every op's params struct (operator.h:14-16). */
typedef struct {
    char _reserved;
} operator_params_t;

/* operator.h:21-25 */
typedef int (*operator_func_t)(const void* inputs[], void* outputs[],
                               const operator_params_t* params, stream_t* stream);

#define OP_FLAG_NONE        (0)
#define OP_FLAG_IN_PLACE    (1 << 0)
#define OP_FLAG_ALLOW_ALIAS (1 << 1)

/* operator.h:34-40 */
typedef struct {
    const char*     name;       /* e.g. "mha_decode_f16_cuda" */
    const char*     data_type;  /* "f32", "f16" */
    operator_func_t func;
    int             version;
    uint32_t        flags;
} operator_registry_t;

/* Registry (operator.h:45-46; operator_registry.c:9-22). Not thread-safe; filled once. */
const operator_registry_t* operator_find(const char* name);
int operator_register(const operator_registry_t* op);

/* Registers every op this library provides (operator_init.c:25-45).  Returns the sum
 * of the individual register_* return codes (0 on success). */
int operator_init_all(void);

/* Number of registered entries and indexed access (used by tests to enumerate). */
int operator_count(void);
const operator_registry_t* operator_at(int index);

#ifdef __cplusplus
}
#endif

#endif /* CF_OPERATOR_H_ */
