/* operator_registry.c — global name -> op table (src/operator/operator_registry.c:9-22
 * of the reference: fixed capacity, linear search, filled once at init). */
#include "operator.h"

#include <string.h>

#define MAX_REGISTERED_OPS 128

static const operator_registry_t* g_ops[MAX_REGISTERED_OPS];
static int g_nops = 0;

int operator_register(const operator_registry_t* op) {
    if (!op || !op->name || g_nops >= MAX_REGISTERED_OPS) return -1;
    /* Re-registering the same entry (operator_init_all called twice) is a no-op. */
    for (int i = 0; i < g_nops; i++)
        if (g_ops[i] == op) return 0;
    g_ops[g_nops++] = op;
    return 0;
}

const operator_registry_t* operator_find(const char* name) {
    if (!name) return NULL;
    for (int i = 0; i < g_nops; i++)
        if (strcmp(g_ops[i]->name, name) == 0) return g_ops[i];
    return NULL;
}

int operator_count(void) { return g_nops; }

const operator_registry_t* operator_at(int index) {
    return (index >= 0 && index < g_nops) ? g_ops[index] : NULL;
}
