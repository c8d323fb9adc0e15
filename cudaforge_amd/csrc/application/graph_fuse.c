/*
 * graph_fuse.c — recognition of the self-attention subgraph that graph_execute runs as
 * one OP_MHA_FUSED node (the reference's detect_and_fuse_mha, graph.c:347-665, and its
 * helper mha_unique_consumer, graph.c:301-314).
 *
 * Pattern, from the tensor X that exactly three MatMuls read:
 *   each MatMul -> optional bias Add -> Reshape -> Transpose      (Q, K and V chains)
 *   MatMul(Q, K) -> Mul(scale) -> optional Add(mask) -> Softmax -> MatMul(probs, V)
 *   -> Transpose -> Reshape -> MatMul(W_O) -> optional bias Add -> optional residual Add
 * where the mask Add's second input is the (S, S) output of a CausalMask node.
 * Q is the chain whose output is the first operand of a MatMul, K the chain that is its
 * second operand, V the third (graph.c:431-467).  B, S, D come from X's shape, H and d
 * from Q's transposed shape (B, H, S, d) (graph.c:564-576).
 *
 * Where this differs from the reference, it is stricter or more general, never looser:
 *   - the scale is the Mul's scalar operand (the reference assumed 1/sqrt(d) whatever
 *     the graph multiplied by): the scores must be the Mul's first input and its other
 *     operand a 1-element weight, or a 1-element tensor no node produces, so its host
 *     value is the one the graph computes with; anything else is not fused;
 *   - projection weights, their biases and b_O are node weights only; an Add whose second
 *     operand is a graph tensor is taken as the residual when it is (B, S, D), so a
 *     missing bias Add cannot swallow the residual (graph.c:512-540 took the first Add as
 *     the bias) and no graph input is uploaded once as if it were a weight;
 *   - H_kv is read from K's transposed shape (GQA, H % H_kv == 0);
 *   - causal = 1 when the scaled scores go through Add(scores, mask) with `mask` the
 *     output of a CausalMask node of seq_len S (its 0 / -inf pattern is exactly the
 *     fused op's causal rule, causal_mask.c:17-21); the CausalMask node is part of the
 *     match when the Add is its only reader, else it still runs;
 *   - weights must be present with the sizes the fused operator reads, and every tensor
 *     must share one dtype (F32 or F16), else the subgraph is left unfused;
 *   - every non-overlapping match is found, not just the first.
 */
#include "graph.h"
#include "causal_mask_int.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int n;
    int ids[GRAPH_MHA_MAX_NODES];
} node_list_t;

static void take(node_list_t* l, int nid) {
    if (l->n < GRAPH_MHA_MAX_NODES) l->ids[l->n++] = nid;
}

static int in_list(const node_list_t* l, int nid) {
    for (int i = 0; i < l->n; i++)
        if (l->ids[i] == nid) return 1;
    return 0;
}

static int reads(const graph_node_t* n, int tid) {
    for (int j = 0; j < n->num_inputs; j++)
        if (n->input_tensors[j] == tid) return 1;
    return 0;
}

/* The one node outside `used` that reads tensor tid; -1 if there is none or more than one
 * (graph.c:301-314). */
static int sole_reader(const inference_graph_t* g, int tid, const unsigned char* used) {
    if (tid < 0) return -1;
    int found = -1;
    for (int i = 0; i < g->num_nodes; i++) {
        if (used[i] || !reads(&g->nodes[i], tid)) continue;
        if (found >= 0) return -1;
        found = i;
    }
    return found;
}

static int out0(const inference_graph_t* g, int nid) {
    const graph_node_t* n = &g->nodes[nid];
    return n->num_outputs > 0 ? n->output_tensors[0] : -1;
}

static tensor_t* tensor_of(const inference_graph_t* g, int tid) {
    return (tid >= 0 && tid < g->num_tensors) ? g->tensors[tid].tensor : NULL;
}

static int is(const inference_graph_t* g, int nid, op_type_t type) {
    return nid >= 0 && g->nodes[nid].type == type;
}

/* The node's first weight (a MatMul's W, an Add's bias, a Mul's scale), or NULL. */
static tensor_t* weight_of(const graph_node_t* n) {
    return (n->num_weights >= 1 && n->weights) ? n->weights[0] : NULL;
}

/* Node that writes tensor tid, or -1. */
static int producer_of(const inference_graph_t* g, int tid) {
    for (int i = 0; i < g->num_nodes; i++) {
        const graph_node_t* n = &g->nodes[i];
        for (int j = 0; j < n->num_outputs; j++)
            if (n->output_tensors[j] == tid) return i;
    }
    return -1;
}

/* MatMul -> (bias Add) -> Reshape -> Transpose from MatMul `mm` (graph.c:391-429).
 * Returns the Transpose's output tensor or -1; w/b receive the MatMul's weight and the
 * bias (NULL without a bias Add). */
static int proj_chain(const inference_graph_t* g, const unsigned char* used, int mm, node_list_t* l,
                      tensor_t** w, tensor_t** b) {
    const graph_node_t* n = &g->nodes[mm];
    *w = weight_of(n);
    *b = NULL;
    take(l, mm);
    int cur = out0(g, mm);
    int nx = sole_reader(g, cur, used);
    if (is(g, nx, OP_ADD) && g->nodes[nx].num_inputs >= 1 && g->nodes[nx].input_tensors[0] == cur) {
        tensor_t* bias = weight_of(&g->nodes[nx]);
        const tensor_t* y = tensor_of(g, cur);
        if (!bias || !y || y->ndim < 1 || bias->numel != y->shape[y->ndim - 1]) return -1;
        *b = bias;
        take(l, nx);
        cur = out0(g, nx);
        nx = sole_reader(g, cur, used);
    }
    if (!is(g, nx, OP_RESHAPE)) return -1;
    take(l, nx);
    cur = out0(g, nx);
    nx = sole_reader(g, cur, used);
    if (!is(g, nx, OP_TRANSPOSE)) return -1;
    take(l, nx);
    return out0(g, nx);
}

static int same_dtype(const tensor_t* t, data_type_t dt) { return t == NULL || t->dtype == dt; }

/* IEEE binary16 -> float. */
static float half_to_float(uint16_t h) {
    const int e = (h >> 10) & 0x1F;
    const uint32_t man = h & 0x3FFu;
    float v;
    if (e == 0) v = ldexpf((float)man, -24);                    /* zero, subnormal */
    else if (e == 31) v = man ? NAN : INFINITY;
    else v = ldexpf((float)(man | 0x400u), e - 25);             /* (1 + man/1024) * 2^(e-15) */
    return (h & 0x8000u) ? -v : v;
}

static float scalar_value(const tensor_t* t) {
    if (t->dtype == DATA_TYPE_F16) return half_to_float(*(const uint16_t*)t->data);
    return *(const float*)t->data;
}

/* Tries the pattern rooted at X = x_tid with the three projection MatMuls mm[3]. */
static int match_at(const inference_graph_t* g, const unsigned char* used, int x_tid, const int mm[3],
                    graph_mha_match_t* m) {
    node_list_t l = {0};
    int chain_out[3];
    tensor_t* w[3];
    tensor_t* b[3];
    for (int c = 0; c < 3; c++) {
        chain_out[c] = proj_chain(g, used, mm[c], &l, &w[c], &b[c]);
        if (chain_out[c] < 0) return 0;
    }
    /* Q: a chain that is the first operand of a MatMul; K: that MatMul's second operand. */
    int qi = -1, attn = -1;
    for (int c = 0; c < 3 && attn < 0; c++)
        for (int i = 0; i < g->num_nodes; i++) {
            const graph_node_t* n = &g->nodes[i];
            if (used[i] || in_list(&l, i) || n->type != OP_MATMUL || n->num_inputs < 2) continue;
            if (n->input_tensors[0] == chain_out[c]) {
                qi = c;
                attn = i;
                break;
            }
        }
    if (attn < 0) return 0;
    int ki = -1;
    for (int c = 0; c < 3; c++)
        if (c != qi && chain_out[c] == g->nodes[attn].input_tensors[1]) ki = c;
    if (ki < 0) return 0;
    const int vi = 3 - qi - ki;
    take(&l, attn);

    int cur = out0(g, attn);
    int nx = sole_reader(g, cur, used);
    if (!is(g, nx, OP_MUL) || g->nodes[nx].num_inputs < 1 || g->nodes[nx].input_tensors[0] != cur) return 0;
    /* The scale: a 1-element node weight.  Its host value becomes a kernel argument,
     * which a recorded replay keeps; a graph tensor the caller may rewrite between
     * executions would then go stale, so a scale that is not a weight is not fused. */
    const tensor_t* scale_t = weight_of(&g->nodes[nx]);
    if (!scale_t || scale_t->numel != 1 || !scale_t->data) return 0;
    take(&l, nx);
    cur = out0(g, nx);
    nx = sole_reader(g, cur, used);
    /* Causal: Add(scores, mask) with mask the output of a CausalMask node (its seq_len is
     * checked against S below). */
    int mask_node = -1;
    if (is(g, nx, OP_ADD) && g->nodes[nx].num_weights == 0 && g->nodes[nx].num_inputs == 2 &&
        g->nodes[nx].input_tensors[0] == cur) {
        mask_node = producer_of(g, g->nodes[nx].input_tensors[1]);
        if (!is(g, mask_node, OP_CAUSAL_MASK) || used[mask_node]) return 0;
        take(&l, nx);
        if (sole_reader(g, g->nodes[nx].input_tensors[1], used) == nx) take(&l, mask_node);
        cur = out0(g, nx);
        nx = sole_reader(g, cur, used);
    }
    if (!is(g, nx, OP_SOFTMAX)) return 0;
    take(&l, nx);
    cur = out0(g, nx);
    nx = sole_reader(g, cur, used);
    if (!is(g, nx, OP_MATMUL) || g->nodes[nx].num_inputs < 2 || g->nodes[nx].input_tensors[0] != cur ||
        g->nodes[nx].input_tensors[1] != chain_out[vi])
        return 0;
    take(&l, nx);
    cur = out0(g, nx);
    nx = sole_reader(g, cur, used);
    if (!is(g, nx, OP_TRANSPOSE)) return 0;
    take(&l, nx);
    cur = out0(g, nx);
    nx = sole_reader(g, cur, used);
    if (!is(g, nx, OP_RESHAPE)) return 0;
    take(&l, nx);
    cur = out0(g, nx);
    nx = sole_reader(g, cur, used);
    if (!is(g, nx, OP_MATMUL)) return 0;
    tensor_t* wo = weight_of(&g->nodes[nx]);
    take(&l, nx);
    cur = out0(g, nx);

    /* Shapes (graph.c:564-576). */
    const tensor_t* x = tensor_of(g, x_tid);
    const tensor_t* qt = tensor_of(g, chain_out[qi]);
    const tensor_t* kt = tensor_of(g, chain_out[ki]);
    const tensor_t* y = tensor_of(g, cur);
    if (!x || x->ndim < 3 || !qt || qt->ndim < 4 || !kt || kt->ndim < 4 || !y) return 0;
    const int64_t B = x->shape[0], S = x->shape[1], D = x->shape[2];
    const int64_t H = qt->shape[1], d = qt->shape[3], H_kv = kt->shape[1];
    if (B <= 0 || S <= 0 || D <= 0 || H <= 0 || d <= 0 || H_kv <= 0 || H % H_kv != 0 || H * d != D) return 0;
    if (mask_node >= 0) {
        const graph_node_t* mn = &g->nodes[mask_node];
        const tensor_t* mt = tensor_of(g, out0(g, mask_node));
        if (!mn->params || mn->params_size < sizeof(causal_mask_params_t) ||
            ((const causal_mask_params_t*)mn->params)->seq_len != S || !mt || mt->numel != S * S)
            return 0;
    }

    /* Optional bias Add, then optional residual Add (graph.c:512-540). */
    tensor_t* bo = NULL;
    int residual = -1;
    nx = sole_reader(g, cur, used);
    if (is(g, nx, OP_ADD) && g->nodes[nx].num_inputs >= 1 && g->nodes[nx].input_tensors[0] == cur) {
        tensor_t* op = weight_of(&g->nodes[nx]);
        if (op && op->numel == D) {
            bo = op;
            take(&l, nx);
            cur = out0(g, nx);
            nx = sole_reader(g, cur, used);
        }
    }
    if (is(g, nx, OP_ADD) && g->nodes[nx].num_inputs >= 2 && g->nodes[nx].num_weights == 0 &&
        g->nodes[nx].input_tensors[0] == cur) {
        const int r = g->nodes[nx].input_tensors[1];
        const tensor_t* rt = tensor_of(g, r);
        if (rt && rt->numel == B * S * D) {
            residual = r;
            take(&l, nx);
            cur = out0(g, nx);
        }
    }
    if (l.n >= GRAPH_MHA_MAX_NODES) return 0;   /* a list that overflowed is not trusted */
    y = tensor_of(g, cur);
    if (!y || y->numel != B * S * D) return 0;

    /* Weights with the sizes mha_fused reads (mha_fused.c:9-20), one dtype throughout. */
    const int64_t kvd = H_kv * d;
    tensor_t* wq = w[qi];
    tensor_t* wk = w[ki];
    tensor_t* wv = w[vi];
    if (!wq || !wk || !wv || !wo) return 0;
    if (wq->numel != D * D || wk->numel != D * kvd || wv->numel != D * kvd || wo->numel != D * D) return 0;
    if ((b[qi] && b[qi]->numel != D) || (b[ki] && b[ki]->numel != kvd) || (b[vi] && b[vi]->numel != kvd)) return 0;
    const data_type_t dt = x->dtype;
    if (dt != DATA_TYPE_F32 && dt != DATA_TYPE_F16) return 0;
    tensor_t* ws[8] = {wq, b[qi], wk, b[ki], wv, b[vi], wo, bo};
    for (int i = 0; i < 8; i++)
        if (!same_dtype(ws[i], dt)) return 0;
    if (!same_dtype(y, dt) || (residual >= 0 && !same_dtype(tensor_of(g, residual), dt))) return 0;

    memset(m, 0, sizeof(*m));
    m->num_nodes = l.n;
    memcpy(m->nodes, l.ids, (size_t)l.n * sizeof(int));
    m->out_node = l.ids[l.n - 1];
    m->input_tid = x_tid;
    m->residual_tid = residual;
    m->output_tid = cur;
    memcpy(m->weights, ws, sizeof(ws));
    mha_fused_params_t* p = &m->params;
    p->batch_size = B;
    p->seq_len = S;
    p->hidden_size = D;
    p->num_heads = H;
    p->num_kv_heads = H_kv;
    p->head_dim = d;
    p->scale = scalar_value(scale_t);
    p->has_residual = residual >= 0;
    p->causal = mask_node >= 0;
    return 1;
}

int graph_detect_mha(const inference_graph_t* g, graph_mha_match_t* matches, int max_matches) {
    if (!g || !matches || max_matches <= 0 || g->num_nodes <= 0) return 0;
    unsigned char* used = (unsigned char*)calloc((size_t)g->num_nodes, 1);
    if (!used) return 0;
    /* Nodes absorbed by a permanent fusion take part in no match. */
    for (int i = 0; i < g->num_nodes && i < g->fused_away_cap; i++) used[i] = g->fused_away[i];
    int count = 0;
    for (int tid = 0; tid < g->num_tensors && count < max_matches; tid++) {
        /* X: read by exactly three MatMuls (graph.c:363-380). */
        int mm[3], n_mm = 0;
        for (int i = 0; i < g->num_nodes && n_mm <= 3; i++) {
            const graph_node_t* n = &g->nodes[i];
            if (used[i] || n->type != OP_MATMUL || n->num_outputs < 1 || !reads(n, tid)) continue;
            if (n_mm < 3) mm[n_mm] = i;
            n_mm++;
        }
        if (n_mm != 3) continue;
        if (match_at(g, used, tid, mm, &matches[count])) {
            for (int i = 0; i < matches[count].num_nodes; i++) used[matches[count].nodes[i]] = 1;
            count++;
        }
    }
    free(used);
    return count;
}
