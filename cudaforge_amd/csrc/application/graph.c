/*
 * graph.c — graph construction, topological build and name-based execution for the
 * attention operators (src/application/engine/graph.c:17-220 and :670-1115 of the
 * reference give the behaviour this follows).
 *
 * Execution contract kept from the reference:
 *   - op lookup by name: "<base>_f16_cuda" when the node's first output is F16 (except
 *     layout ops), else "<base>_cuda", else the CPU "<base>" (graph.c:836-884);
 *     unresolved -> -2;
 *   - input slots = node inputs then weights, outputs right after (graph.c:900-925);
 *   - GPU ops get device pointers; outputs stay on the device until the end, when
 *     graph outputs are copied back (lazy D2H, graph.c:1051-1083);
 *   - an op's nonzero return aborts execution and is returned (graph.c:1019-1025).
 * Changes: graph inputs are re-uploaded on every execution (the reference uploaded once,
 * tensor.c:54, and reused stale data); KV-cache tensors are device-authoritative and
 * uploaded once; a CPU op that writes a KV cache refreshes its device copy.  GPU
 * executions run each self-attention subgraph that graph_detect_mha finds (graph_fuse.c,
 * the reference's detect_and_fuse_mha, graph.c:347-665) as one OP_MHA_FUSED node, without
 * rewriting the graph.
 * GPU executions run on a non-blocking stream the graph owns and, once an execution has
 * run every node on the GPU, are recorded into a HIP graph and replayed (the reference's
 * CUDA-graph path, graph.c:681-742, which it left disabled because every launch went to
 * the legacy stream).  Graph inputs are uploaded, and graph outputs downloaded, on the
 * graph's own stream, ordered with its launches, so a GPU execution synchronises the host
 * once (in the first output download); first uploads of weights, caches and new device
 * copies go through the legacy stream, which is synchronised before the next launch.
 */
#include "graph.h"
#include "gpu_ops.h"
#include "mha_decode_int.h"
#include "../kernels/kernels.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* Device-held length of a uniform-length decode node (GPU executions).  The node runs in
 * the operator's advancing device-uniform mode (cache_len
 * MHA_DECODE_CACHE_LEN_DEVICE_ADVANCE, lengths in slot 11), so its launches do not depend
 * on cache_len and its last kernel adds one: a recorded execution therefore replays at
 * every length of a decode loop.  `held` is the value the device array holds after the
 * work issued so far. */
typedef struct {
    int32_t* lens;   /* device, B entries; NULL until the node first runs on the GPU */
    int64_t  B;
    int64_t  held;   /* -1 = unknown */
} decode_lens_t;

static decode_lens_t* decode_lens_at(inference_graph_t* g, int nid) {
    if (nid < 0) return NULL;
    if (nid >= g->decode_lens_cap) {
        const int cap = g->num_nodes > nid ? g->num_nodes : nid + 1;
        decode_lens_t* p = (decode_lens_t*)realloc(g->decode_lens, (size_t)cap * sizeof(decode_lens_t));
        if (!p) return NULL;
        memset(p + g->decode_lens_cap, 0, (size_t)(cap - g->decode_lens_cap) * sizeof(decode_lens_t));
        g->decode_lens = p;
        g->decode_lens_cap = cap;
    }
    return &((decode_lens_t*)g->decode_lens)[nid];
}

static void decode_lens_free(inference_graph_t* g) {
    decode_lens_t* v = (decode_lens_t*)g->decode_lens;
    for (int i = 0; i < g->decode_lens_cap; i++)
        if (v[i].lens) gpu_device_free(v[i].lens);
    free(v);
    g->decode_lens = NULL;
    g->decode_lens_cap = 0;
}

/* A decode node whose GPU execution uses a device-held uniform length. */
static int uniform_decode(const graph_node_t* n) {
    return n->type == OP_MHA_DECODE && n->params && n->params_size >= sizeof(mha_decode_params_t) &&
           ((const mha_decode_params_t*)n->params)->cache_len >= 0;
}

/* Sets the device lengths of node nid to its cache_len (a kernel on the graph's stream)
 * unless they hold it already.  Not while recording: the recording must advance the
 * lengths, never set them. */
static int decode_lens_sync(inference_graph_t* g, int nid) {
    const graph_node_t* n = &g->nodes[nid];
    decode_lens_t* dl = decode_lens_at(g, nid);
    if (!dl) return -1;
    const mha_decode_params_t* p = (const mha_decode_params_t*)n->params;
    if (dl->lens && dl->B < p->batch_size) {   /* the node's batch grew: a larger array */
        gpu_device_free(dl->lens);
        dl->lens = NULL;
        gpu_buffer_generation_bump();          /* a recording may point at the old one */
    }
    if (!dl->lens) {
        if (p->batch_size <= 0 || p->batch_size > 65535) return -1;
        dl->lens = (int32_t*)gpu_device_alloc((size_t)p->batch_size * sizeof(int32_t));
        if (!dl->lens) return -1;
        dl->B = p->batch_size;
        dl->held = -1;
    }
    if (dl->held == p->cache_len) return 0;
    const int rc = cf_launch_i32_update(dl->lens, (int32_t)dl->B, (int32_t)p->cache_len, 0, g->hip_graph);
    if (rc != 0) return rc;
    dl->held = p->cache_len;
    return 0;
}

static void pinned_free(inference_graph_t* g);

/* Drops the recorded execution; the next all-GPU execution starts over. */
static void replay_reset(inference_graph_t* g) {
    if (g->hip_graph_exec) gpu_graph_exec_destroy(g->hip_graph_exec);
    g->hip_graph_exec = NULL;
    g->hip_graph_state = 0;
}

void graph_set_replay(inference_graph_t* g, int enable) {
    if (!g) return;
    g->replay_off = !enable;
    replay_reset(g);
}

int graph_replay_state(const inference_graph_t* g) { return g ? g->hip_graph_state : 0; }

inference_graph_t* graph_create(void) {
    inference_graph_t* g = (inference_graph_t*)calloc(1, sizeof(inference_graph_t));
    if (!g) return NULL;
    g->kv_cache_K_tid = -1;
    g->kv_cache_V_tid = -1;
    return g;
}

int graph_add_tensor(inference_graph_t* g, tensor_t* t) {
    if (!g || !t) return -1;
    replay_reset(g);
    graph_tensor_t* p = (graph_tensor_t*)realloc(g->tensors, (size_t)(g->num_tensors + 1) * sizeof(graph_tensor_t));
    if (!p) return -1;
    g->tensors = p;
    const int id = g->num_tensors++;
    g->tensors[id].tensor = t;
    g->tensors[id].producer = -1;
    g->tensors[id].consumer = -1;
    return id;
}

int graph_add_node(inference_graph_t* g, op_type_t type,
                   int num_inputs, const int* input_tensors,
                   int num_outputs, const int* output_tensors,
                   int num_weights, tensor_t** weights,
                   void* params, size_t params_size) {
    if (!g || num_inputs < 0 || num_outputs < 0 || num_weights < 0) return -1;
    if ((num_inputs > 0 && !input_tensors) || (num_outputs > 0 && !output_tensors)) return -1;
    replay_reset(g);
    graph_node_t* p = (graph_node_t*)realloc(g->nodes, (size_t)(g->num_nodes + 1) * sizeof(graph_node_t));
    if (!p) return -1;
    g->nodes = p;
    const int id = g->num_nodes++;
    graph_node_t* n = &g->nodes[id];
    memset(n, 0, sizeof(*n));
    n->type = type;
    n->num_inputs = num_inputs;
    n->num_outputs = num_outputs;
    n->num_weights = num_weights;
    if (num_weights > 0 && weights) {
        n->weights = (tensor_t**)malloc((size_t)num_weights * sizeof(tensor_t*));
        if (!n->weights) return -1;
        memcpy(n->weights, weights, (size_t)num_weights * sizeof(tensor_t*));
    } else {
        n->num_weights = 0;
    }
    if (params && params_size > 0) {
        n->params = malloc(params_size);
        if (!n->params) return -1;
        memcpy(n->params, params, params_size);
        n->params_size = params_size;
    }
    if (num_inputs > 0) {
        n->input_tensors = (int*)malloc((size_t)num_inputs * sizeof(int));
        if (!n->input_tensors) return -1;
        memcpy(n->input_tensors, input_tensors, (size_t)num_inputs * sizeof(int));
    }
    if (num_outputs > 0) {
        n->output_tensors = (int*)malloc((size_t)num_outputs * sizeof(int));
        if (!n->output_tensors) return -1;
        memcpy(n->output_tensors, output_tensors, (size_t)num_outputs * sizeof(int));
    }
    for (int i = 0; i < num_inputs; i++)
        if (input_tensors[i] >= 0 && input_tensors[i] < g->num_tensors) g->tensors[input_tensors[i]].consumer = id;
    for (int i = 0; i < num_outputs; i++) {
        const int tid = output_tensors[i];
        if (tid < 0 || tid >= g->num_tensors) continue;
        /* A node that reads and writes the same tensor (in-place KV cache) is not its
         * own producer for ordering purposes. */
        int self = 0;
        for (int j = 0; j < num_inputs; j++) if (input_tensors[j] == tid) self = 1;
        if (!self) g->tensors[tid].producer = id;
    }
    return id;
}

static int append_id(int** arr, int* count, int value) {
    int* p = (int*)realloc(*arr, (size_t)(*count + 1) * sizeof(int));
    if (!p) return -1;
    *arr = p;
    p[(*count)++] = value;
    return 0;
}

int graph_set_input(inference_graph_t* g, int node_id) {
    if (!g || node_id < 0 || node_id >= g->num_nodes) return -1;
    return append_id(&g->input_node_ids, &g->num_inputs, node_id);
}

int graph_set_output(inference_graph_t* g, int node_id) {
    if (!g || node_id < 0 || node_id >= g->num_nodes) return -1;
    return append_id(&g->output_node_ids, &g->num_outputs, node_id);
}

void graph_set_kv_cache(inference_graph_t* g, int K_tensor_id, int V_tensor_id) {
    if (!g) return;
    replay_reset(g);
    g->kv_cache_K_tid = K_tensor_id;
    g->kv_cache_V_tid = V_tensor_id;
}

/* (graph.c:139-149.)  GPU executions read a uniform length from the device, so a new
 * length keeps the recording; only a switch between a uniform and a per-sequence
 * (ragged, cache_len < 0) length changes the launches and drops it. */
void graph_update_cache_len(inference_graph_t* g, int64_t new_cache_len) {
    if (!g) return;
    for (int i = 0; i < g->num_nodes; i++) {
        graph_node_t* n = &g->nodes[i];
        if (n->type == OP_MHA_DECODE && n->params && n->params_size >= sizeof(mha_decode_params_t)) {
            mha_decode_params_t* p = (mha_decode_params_t*)n->params;
            if ((p->cache_len < 0) != (new_cache_len < 0)) replay_reset(g);
            p->cache_len = new_cache_len;
        }
    }
}

void graph_set_permanent_fusion(inference_graph_t* g, int enable) {
    if (g) g->permanent_fusion = enable;
}

/* Kahn's algorithm (graph.c:158-220): a node depends on the producers of its inputs. */
int graph_build(inference_graph_t* g) {
    if (!g) return -1;
    replay_reset(g);
    const int n = g->num_nodes;
    int* indeg = (int*)calloc((size_t)(n > 0 ? n : 1), sizeof(int));
    int* queue = (int*)malloc((size_t)(n > 0 ? n : 1) * sizeof(int));
    int* order = (int*)malloc((size_t)(n > 0 ? n : 1) * sizeof(int));
    if (!indeg || !queue || !order) { free(indeg); free(queue); free(order); return -1; }
    for (int i = 0; i < n; i++)
        for (int j = 0; j < g->nodes[i].num_inputs; j++) {
            const int tid = g->nodes[i].input_tensors[j];
            if (tid >= 0 && tid < g->num_tensors) {
                const int prod = g->tensors[tid].producer;
                if (prod >= 0 && prod != i) indeg[i]++;
            }
        }
    int head = 0, tail = 0, done = 0;
    for (int i = 0; i < n; i++) if (indeg[i] == 0) queue[tail++] = i;
    while (head < tail) {
        const int v = queue[head++];
        order[done++] = v;
        for (int k = 0; k < n; k++) {
            if (k == v) continue;
            for (int l = 0; l < g->nodes[k].num_inputs; l++) {
                const int tid = g->nodes[k].input_tensors[l];
                if (tid >= 0 && tid < g->num_tensors && g->tensors[tid].producer == v) {
                    if (--indeg[k] == 0) queue[tail++] = k;
                }
            }
        }
    }
    free(indeg);
    free(queue);
    if (done != n) { free(order); return -1; }   /* cycle */
    free(g->topo_order);
    g->topo_order = order;
    return 0;
}

void graph_destroy(inference_graph_t* g) {
    if (!g) return;
    replay_reset(g);
    if (g->hip_graph) {
        (void)gpu_stream_synchronize(g->hip_graph);
        gpu_stream_destroy(g->hip_graph);
    }
    decode_lens_free(g);
    pinned_free(g);
    free(g->fused_away);
    for (int i = 0; i < g->num_nodes; i++) {
        free(g->nodes[i].input_tensors);
        free(g->nodes[i].output_tensors);
        free(g->nodes[i].weights);
        free(g->nodes[i].params);
    }
    free(g->nodes);
    for (int i = 0; i < g->num_tensors; i++) tensor_destroy(g->tensors[i].tensor);
    free(g->tensors);
    free(g->topo_order);
    free(g->input_node_ids);
    free(g->output_node_ids);
    free(g);
}

/* Op type -> CPU base name (graph.c:254-294). */
static const char* op_name(op_type_t type) {
    switch (type) {
        case OP_RELU: return "relu_f32";
        case OP_SIGMOID: return "sigmoid_f32";
        case OP_GELU: return "gelu_f32";
        case OP_MATMUL: return "matmul_f32";
        case OP_CONV2D: return "conv2d_f32";
        case OP_MAXPOOL2D: return "maxpool2d_f32";
        case OP_AVGPOOL2D: return "avgpool2d_f32";
        case OP_BATCHNORM: return "batchnorm_f32";
        case OP_ADD: return "add_f32";
        case OP_RESHAPE: return "reshape_f32";
        case OP_GLOBALAVGPOOL: return "globalavgpool_f32";
        case OP_SOFTMAX: return "softmax_f32";
        case OP_SILU: return "silu_f32";
        case OP_MUL: return "mul_f32";
        case OP_CONCAT: return "concat_f32";
        case OP_RESIZE: return "resize_f32";
        case OP_TRANSPOSE: return "transpose_f32";
        case OP_SUB: return "sub_f32";
        case OP_DIV: return "div_f32";
        case OP_SLICE: return "slice_f32";
        case OP_SPLIT: return "split_f32";
        case OP_LAYERNORM: return "layernorm_f32";
        case OP_GATHER: return "gather_f32";
        case OP_SQUEEZE_UNSQUEEZE: return "squeeze_unsqueeze_f32";
        case OP_EXP: return "exp_f32";
        case OP_REDUCE: return "reduce_f32";
        case OP_CAST: return "cast_f32";
        case OP_ARGMAX: return "argmax_f32";
        case OP_MHA_FUSED: return "mha_fused_f32";
        case OP_MHA_DECODE: return "mha_decode_f32";
        case OP_CAUSAL_MASK: return "causal_mask_f32";
        case OP_ROPE: return "rope_f32";
        case OP_PAD: return "pad_f32";
        case OP_CLIP: return "clip_f32";
        case OP_WHERE: return "where_f32";
        case OP_TANH: return "tanh_f32";
        default: return NULL;
    }
}

static const operator_registry_t* resolve_node(const inference_graph_t* g, const graph_node_t* n, bool use_cuda,
                                               char* buf, size_t buf_len) {
    const char* base = op_name(n->type);
    buf[0] = '\0';
    if (!base) return NULL;
    int out_f16 = 0;
    if (n->num_outputs > 0 && n->output_tensors && n->output_tensors[0] >= 0 &&
        n->output_tensors[0] < g->num_tensors && g->tensors[n->output_tensors[0]].tensor)
        out_f16 = g->tensors[n->output_tensors[0]].tensor->dtype == DATA_TYPE_F16;
    const operator_registry_t* op = NULL;
    const int layout_op = n->type == OP_CAST || n->type == OP_RESHAPE || n->type == OP_TRANSPOSE ||
                          n->type == OP_SLICE || n->type == OP_SPLIT || n->type == OP_SQUEEZE_UNSQUEEZE;
    if (out_f16 && !layout_op) {
        const size_t bl = strlen(base);
        char b16[64];
        if (bl > 3 && strcmp(base + bl - 3, "f32") == 0) snprintf(b16, sizeof(b16), "%.*sf16", (int)(bl - 3), base);
        else snprintf(b16, sizeof(b16), "%s", base);
        /* mha_fused_f16_cuda keeps the reference's FP32 buffers; F16 tensors take the
         * fp16-I/O op. */
        if (n->type == OP_MHA_FUSED && use_cuda) snprintf(b16, sizeof(b16), "mha_fused_f16io");
        snprintf(buf, buf_len, use_cuda ? "%s_cuda" : "%s", b16);
        op = operator_find(buf);
    }
    if (!op) {
        snprintf(buf, buf_len, use_cuda ? "%s_cuda" : "%s", base);
        op = operator_find(buf);
    }
    if (!op && use_cuda) {
        op = operator_find(base);
        if (op) snprintf(buf, buf_len, "%s", base);
    }
    return op;
}

const operator_registry_t* graph_resolve_op(const inference_graph_t* g, int node_id, bool use_cuda,
                                            char* buf, size_t buf_len) {
    if (!g || node_id < 0 || node_id >= g->num_nodes || !buf || buf_len < 8) return NULL;
    return resolve_node(g, &g->nodes[node_id], use_cuda, buf, buf_len);
}

static size_t tensor_nbytes(const tensor_t* t) {
    const data_type_info_t* info = data_type_get_info(t->dtype);
    return info ? (size_t)t->numel * info->size : 0;
}

static int is_kv(const inference_graph_t* g, int tid) {
    return tid >= 0 && (tid == g->kv_cache_K_tid || tid == g->kv_cache_V_tid);
}

/* Pinned host staging of a graph input or output tensor (allocated on first use, freed
 * with the graph).  The device reads and writes it directly, so a copy kernel on the
 * graph's stream moves the data between launches: a DMA-engine copy there measured
 * ~25 us of hand-over latency before the next kernel and ~16 us after the last one.
 * NULL when the tensor is large (its copy is bandwidth-bound, not latency-bound) or
 * pinned memory is unavailable. */
typedef struct {
    void*  host;
    size_t bytes;
    int    rec_in;    /* its upload copy is a node of the recording */
    int    rec_out;   /* its download copy is a node of the recording */
} pinned_t;

#define GRAPH_PINNED_MAX ((size_t)16 << 20)

static void* pinned_of(inference_graph_t* g, int tid, size_t bytes) {
    if (tid < 0 || bytes == 0 || bytes > GRAPH_PINNED_MAX) return NULL;
    if (tid >= g->pinned_cap) {
        const int cap = g->num_tensors > tid ? g->num_tensors : tid + 1;
        pinned_t* p = (pinned_t*)realloc(g->pinned, (size_t)cap * sizeof(pinned_t));
        if (!p) return NULL;
        memset(p + g->pinned_cap, 0, (size_t)(cap - g->pinned_cap) * sizeof(pinned_t));
        g->pinned = p;
        g->pinned_cap = cap;
    }
    pinned_t* e = &((pinned_t*)g->pinned)[tid];
    if (e->host && e->bytes >= bytes) return e->host;
    if (e->host) {
        gpu_host_free_pinned(e->host);
        gpu_buffer_generation_bump();   /* a recording may copy through the old buffer */
    }
    e->host = gpu_host_alloc_pinned(bytes);
    e->bytes = e->host ? bytes : 0;
    return e->host;
}

static pinned_t* pinned_entry(inference_graph_t* g, int tid) {
    return tid >= 0 && tid < g->pinned_cap ? &((pinned_t*)g->pinned)[tid] : NULL;
}

static void pinned_clear_recorded(inference_graph_t* g) {
    for (int i = 0; i < g->pinned_cap; i++) ((pinned_t*)g->pinned)[i].rec_in = ((pinned_t*)g->pinned)[i].rec_out = 0;
}

static void pinned_free(inference_graph_t* g) {
    pinned_t* v = (pinned_t*)g->pinned;
    for (int i = 0; i < g->pinned_cap; i++)
        if (v[i].host) gpu_host_free_pinned(v[i].host);
    free(v);
    g->pinned = NULL;
    g->pinned_cap = 0;
}

/* How an execution moves a staged graph input to the device. */
enum {
    UPLOAD_NOW = 0,     /* copy kernel on the graph's stream now */
    UPLOAD_RECORD = 1,  /* fill the staging and mark it: the recording's first nodes copy it */
    UPLOAD_REPLAY = 2,  /* fill the staging of the inputs whose copy is in the recording */
};

/* Host -> device copy of graph input tid: through its pinned staging on the graph's
 * stream, ordered before the launches that read it (no host synchronisation).  The first
 * upload of a tensor, and tensors without staging, go through tensor_upload (legacy
 * stream); *legacy is then set so the caller waits for it. */
static int upload_input(inference_graph_t* g, int tid, tensor_t* t, int* legacy, int mode) {
    const size_t bytes = tensor_nbytes(t);
    void* stage = t->data_device ? pinned_of(g, tid, bytes) : NULL;
    if (stage && mode == UPLOAD_REPLAY && !pinned_entry(g, tid)->rec_in) stage = NULL;
    if (!stage) {
        *legacy = 1;
        return tensor_upload(t);
    }
    memcpy(stage, t->data, bytes);
    if (mode == UPLOAD_RECORD) pinned_entry(g, tid)->rec_in = 1;
    if (mode != UPLOAD_NOW) return 0;
    return cf_launch_copy_bytes(t->data_device, stage, bytes, g->hip_graph) == 0 ? 0 : -1;
}

/* Inside a capture: the copies of the staged inputs (first) or of the graph outputs
 * (last) as nodes of the recording, so a replay runs them back to back with the
 * operators' launches instead of as separate launches around the graph. */
static int record_input_copies(inference_graph_t* g) {
    for (int tid = 0; tid < g->pinned_cap && tid < g->num_tensors; tid++) {
        const pinned_t* e = pinned_entry(g, tid);
        if (!e->rec_in) continue;
        tensor_t* t = g->tensors[tid].tensor;
        if (cf_launch_copy_bytes(t->data_device, e->host, tensor_nbytes(t), g->hip_graph) != 0) return -1;
    }
    return 0;
}

static int record_output_copies(inference_graph_t* g) {
    for (int i = 0; i < g->num_outputs; i++) {
        const graph_node_t* n = &g->nodes[g->output_node_ids[i]];
        if (n->type != OP_OUTPUT || n->num_inputs <= 0) continue;
        const int tid = n->input_tensors[0];
        if (tid < 0 || tid >= g->num_tensors) continue;
        tensor_t* src = g->tensors[tid].tensor;
        if (!src->data_device) continue;
        const size_t bytes = tensor_nbytes(src);
        void* stage = pinned_of(g, tid, bytes);
        if (!stage) continue;
        if (cf_launch_copy_bytes(stage, src->data_device, bytes, g->hip_graph) != 0) return -1;
        pinned_entry(g, tid)->rec_out = 1;
    }
    return 0;
}

/* Written by an operator during execution (so its device copy is the current one), as
 * opposed to a graph input (no producer, or an OP_INPUT node), whose host data the
 * caller may change between executions. */
static int op_produced(const inference_graph_t* g, int tid) {
    const int prod = g->tensors[tid].producer;
    return prod >= 0 && g->nodes[prod].type != OP_INPUT;
}

/* Runs one node: resolves its operator, moves its tensors to where the operator runs,
 * calls it (graph.c:820-1030). */
static int run_node(inference_graph_t* g, int nid, const graph_node_t* n, bool use_cuda, unsigned char* fresh,
                    int* ran_on_gpu, int recording) {
    int ret = 0;
    char name[64];
    const operator_registry_t* op = resolve_node(g, n, use_cuda, name, sizeof(name));
    if (!op) return -2;
    const int on_gpu = use_cuda && strstr(name, "_cuda") != NULL;
    if (ran_on_gpu) *ran_on_gpu = on_gpu;
    /* A CPU operator reads host copies of device data: let the graph's stream finish. */
    if (use_cuda && !on_gpu && g->hip_graph && (ret = gpu_stream_synchronize(g->hip_graph)) != 0) return ret;
    int copied = 0;                 /* a host-to-device copy was issued for this node */

    /* Input slots: tensor inputs, then weights, padded with NULLs to the count some ops
     * always read (graph.c:886-895: activations 2, Conv/MatMul 3 for the optional bias,
     * BatchNorm 6), so no op reads an output slot as an input. */
    int in_slots = n->num_inputs + n->num_weights;
    int reserve = 0;
    switch (n->type) {
        case OP_RELU: case OP_SIGMOID: case OP_GELU: case OP_SILU: case OP_EXP: case OP_TANH: reserve = 2; break;
        case OP_CONV2D: case OP_MATMUL: reserve = 3; break;
        case OP_BATCHNORM: reserve = 6; break;
        default: break;
    }
    /* Decode on the GPU: a uniform length runs from device-held lengths (slot 11); the
     * reference's bound on cache_len (mha_decode.c:14-16) is checked here, where it is
     * still a host value.  Per-sequence lengths (the node's 9th weight) are checked on
     * their host copy. */
    const mha_decode_params_t* dp = n->type == OP_MHA_DECODE && n->params &&
                                    n->params_size >= sizeof(mha_decode_params_t)
                                        ? (const mha_decode_params_t*)n->params : NULL;
    const int dev_len = on_gpu && dp && dp->cache_len >= 0 && nid >= 0;
    mha_decode_params_t dev_params;
    decode_lens_t* dl = NULL;
    if (dp && dp->cache_len >= dp->max_seq) return -1;
    if (dp && dp->cache_len < 0 && n->num_weights >= 9) {
        const tensor_t* lt = n->weights[8];
        if (!lt || !lt->data || lt->dtype != DATA_TYPE_I32 || lt->numel < dp->batch_size) return -1;
        for (int64_t b = 0; b < dp->batch_size; b++) {
            const int32_t v = ((const int32_t*)lt->data)[b];
            if (v < 0 || v >= dp->max_seq) return -1;
        }
    }
    /* Per-sequence lengths change between steps: their host copy, checked above, is
     * uploaded on every GPU execution, which a recording could not repeat, so such a
     * step is not recorded (the graph then runs eagerly until the mode changes). */
    const int ragged_lens = on_gpu && dp && dp->cache_len < 0 && n->num_weights >= 9;
    if (ragged_lens && recording) return -1;
    if (dev_len) {
        if (!recording && (ret = decode_lens_sync(g, nid)) != 0) return ret;
        dl = decode_lens_at(g, nid);
        if (!dl || !dl->lens || dl->held != dp->cache_len) return -1;
        dev_params = *dp;
        dev_params.cache_len = MHA_DECODE_CACHE_LEN_DEVICE_ADVANCE;
        if (reserve < MHA_DECODE_SLOT_SEQLENS + 1) reserve = MHA_DECODE_SLOT_SEQLENS + 1;
    }
    if (in_slots < reserve) in_slots = reserve;
    const int total = in_slots + n->num_outputs;
    const void* local[32];
    const void** slots = total <= 32 ? local : (const void**)malloc((size_t)total * sizeof(void*));
    if (!slots) return -1;
    void** outs = (void**)&slots[in_slots];
    for (int i = n->num_inputs + n->num_weights; i < in_slots; i++) slots[i] = NULL;

    for (int i = 0; i < n->num_inputs && ret == 0; i++) {
        const int tid = n->input_tensors[i];
        slots[i] = NULL;
        if (tid < 0 || tid >= g->num_tensors) continue;
        tensor_t* t = g->tensors[tid].tensor;
        if (on_gpu) {
            if (is_kv(g, tid) || op_produced(g, tid)) {
                copied |= !t->data_device;
                if (tensor_copy_to_device(t) != 0) ret = -1;
            } else if (!fresh[tid]) {
                if (upload_input(g, tid, t, &copied, UPLOAD_NOW) != 0) ret = -1;
                fresh[tid] = 1;
            }
            slots[i] = t->data_device;
        } else {
            if (t->data_device && op_produced(g, tid) && tensor_copy_to_host(t) != 0) ret = -1;
            if (is_kv(g, tid) && t->data_device && tensor_copy_to_host(t) != 0) ret = -1;
            slots[i] = t->data;
        }
    }
    for (int w = 0; w < n->num_weights && ret == 0; w++) {
        tensor_t* t = n->weights[w];
        slots[n->num_inputs + w] = NULL;
        if (!t) continue;
        if (on_gpu) {
            if (ragged_lens && w == 8) {
                copied = 1;
                if (tensor_upload(t) != 0) ret = -1;
            } else {
                copied |= !t->data_device;
                if (tensor_copy_to_device(t) != 0) ret = -1;
            }
            slots[n->num_inputs + w] = t->data_device;
        } else {
            slots[n->num_inputs + w] = t->data;
        }
    }
    /* A uniform length runs from the node's device-held lengths, never from a 9th
     * weight the node may also carry for its ragged steps (that weight is left as the
     * caller wrote it). */
    if (dev_len) slots[MHA_DECODE_SLOT_SEQLENS] = dl->lens;
    for (int i = 0; i < n->num_outputs && ret == 0; i++) {
        const int tid = n->output_tensors[i];
        outs[i] = NULL;
        if (tid < 0 || tid >= g->num_tensors) continue;
        tensor_t* t = g->tensors[tid].tensor;
        if (on_gpu) {
            if (!t->data_device) {
                t->data_device = gpu_device_alloc(tensor_nbytes(t));
                if (!t->data_device) ret = -1;
            }
            outs[i] = t->data_device;
        } else {
            outs[i] = t->data;
        }
    }
    /* Host copies go on the legacy stream, which the graph's non-blocking stream does not
     * wait for: let them land before the operator's launches. */
    if (ret == 0 && copied) ret = gpu_stream_synchronize(NULL);
    if (ret == 0) {
        stream_t stream = {g->hip_graph};
        const void* params = dev_len ? (const void*)&dev_params : n->params;
        ret = op->func(slots, outs, (const operator_params_t*)params, use_cuda ? &stream : NULL);
        /* The op's last kernel moved the lengths to the next position. */
        if (ret == 0 && dev_len) dl->held = dp->cache_len + 1;
    }
    if (ret == 0 && use_cuda && !on_gpu) {
        /* A CPU op wrote host data: device copies are stale.  KV caches stay
         * device-authoritative, so refresh them; drop the others. */
        for (int i = 0; i < n->num_outputs; i++) {
            const int tid = n->output_tensors[i];
            if (tid < 0 || tid >= g->num_tensors) continue;
            tensor_t* t = g->tensors[tid].tensor;
            if (!t->data_device) continue;
            if (is_kv(g, tid)) {
                if (tensor_upload(t) != 0 || gpu_stream_synchronize(NULL) != 0) ret = -1;
            } else {
                gpu_device_free(t->data_device);
                t->data_device = NULL;
            }
        }
    }
    if (slots != local) free((void*)slots);
    return ret;
}

/* Uploads every tensor a GPU execution reads from the host that is neither a KV cache nor
 * produced by an operator (the graph inputs and constant inputs), marking it fresh, and
 * makes sure the KV caches and weights are on the device: a recorded execution may not
 * copy from the host. */
static int preload_inputs(inference_graph_t* g, unsigned char* fresh, int mode) {
    int legacy = 0;
    for (int i = 0; i < g->num_nodes; i++) {
        const graph_node_t* n = &g->nodes[i];
        for (int k = 0; k < n->num_inputs; k++) {
            const int tid = n->input_tensors[k];
            if (tid < 0 || tid >= g->num_tensors || fresh[tid]) continue;
            tensor_t* t = g->tensors[tid].tensor;
            if (is_kv(g, tid) || op_produced(g, tid)) {
                if (is_kv(g, tid) && tensor_copy_to_device(t) != 0) return -1;
                continue;
            }
            if (upload_input(g, tid, t, &legacy, mode) != 0) return -1;
            fresh[tid] = 1;
        }
        for (int w = 0; w < n->num_weights; w++)
            if (n->weights[w] && tensor_copy_to_device(n->weights[w]) != 0) return -1;
    }
    /* Device lengths of the decode nodes, set on the graph's stream before the recorded
     * (or replayed) work. */
    for (int i = 0; i < g->num_nodes; i++) {
        if (!uniform_decode(&g->nodes[i])) continue;
        const mha_decode_params_t* p = (const mha_decode_params_t*)g->nodes[i].params;
        if (p->cache_len >= p->max_seq) return -1;
        const int rc = decode_lens_sync(g, i);
        if (rc != 0) return rc;
    }
    /* First uploads (weights, caches, new device copies) ran on the legacy stream, which
     * the graph's stream does not wait for. */
    return legacy ? gpu_stream_synchronize(NULL) : 0;
}

/* After a replay: the recording advanced every decode node's lengths by one. */
static void decode_lens_replayed(inference_graph_t* g) {
    for (int i = 0; i < g->num_nodes && i < g->decode_lens_cap; i++) {
        decode_lens_t* dl = &((decode_lens_t*)g->decode_lens)[i];
        if (dl->lens && uniform_decode(&g->nodes[i]))
            dl->held = ((const mha_decode_params_t*)g->nodes[i].params)->cache_len + 1;
    }
}

/* Permanent fusion (graph_set_permanent_fusion): node m->out_node becomes the match's
 * OP_MHA_FUSED node and the match's other nodes are marked absorbed.  The fused node
 * keeps its id, its output tensor and so its place in the topological order; its new
 * inputs (X, the residual) are produced before the pattern's last node, which read
 * them too.  Returns -1 (graph unchanged) if memory runs out. */
static int make_fusion_permanent(inference_graph_t* g, const graph_mha_match_t* m) {
    if (g->fused_away_cap < g->num_nodes) {
        unsigned char* p = (unsigned char*)realloc(g->fused_away, (size_t)g->num_nodes);
        if (!p) return -1;
        memset(p + g->fused_away_cap, 0, (size_t)(g->num_nodes - g->fused_away_cap));
        g->fused_away = p;
        g->fused_away_cap = g->num_nodes;
    }
    int* in = (int*)malloc(2 * sizeof(int));
    int* out = (int*)malloc(sizeof(int));
    tensor_t** w = (tensor_t**)malloc(8 * sizeof(tensor_t*));
    mha_fused_params_t* fp = (mha_fused_params_t*)malloc(sizeof(mha_fused_params_t));
    if (!in || !out || !w || !fp) {
        free(in); free(out); free(w); free(fp);
        return -1;
    }
    in[0] = m->input_tid;
    in[1] = m->residual_tid;
    out[0] = m->output_tid;
    memcpy(w, m->weights, 8 * sizeof(tensor_t*));
    *fp = m->params;
    graph_node_t* n = &g->nodes[m->out_node];
    free(n->input_tensors);
    free(n->output_tensors);
    free(n->weights);
    free(n->params);
    n->type = OP_MHA_FUSED;
    n->num_inputs = 2;
    n->input_tensors = in;
    n->num_outputs = 1;
    n->output_tensors = out;
    n->num_weights = 8;
    n->weights = w;
    n->params = fp;
    n->params_size = sizeof(*fp);
    for (int i = 0; i < m->num_nodes; i++)
        if (m->nodes[i] != m->out_node) g->fused_away[m->nodes[i]] = 1;
    return 0;
}

/* Runs every node once, in topological order, with MHA subgraph fusion on GPU
 * executions.  *all_gpu tells whether every node ran on the GPU. */
static int run_nodes(inference_graph_t* g, bool use_cuda, unsigned char* fresh, int* all_gpu, int recording) {
    /* MHA subgraph fusion (graph.c:766-815, GPU executions only): each match runs as one
     * OP_MHA_FUSED node in place of its last node; its other nodes are skipped. */
    graph_mha_match_t* fz = NULL;
    int* fused_at = NULL;
    int n_fused = 0;
    *all_gpu = use_cuda;
    if (use_cuda && g->num_nodes > 0) {
        const int cap = g->num_nodes / 8 + 1;
        fz = (graph_mha_match_t*)malloc((size_t)cap * sizeof(*fz));
        fused_at = (int*)malloc((size_t)g->num_nodes * sizeof(int));
        if (!fz || !fused_at) { free(fz); free(fused_at); return -1; }
        n_fused = graph_detect_mha(g, fz, cap);
        if (g->permanent_fusion && n_fused > 0) {
            /* Rewrite once; this and every later execution run the fused nodes as
             * ordinary nodes. */
            for (int k = 0; k < n_fused; k++)
                if (make_fusion_permanent(g, &fz[k]) != 0) { free(fz); free(fused_at); return -1; }
            n_fused = 0;
        }
        for (int i = 0; i < g->num_nodes; i++) fused_at[i] = -1;
        for (int k = 0; k < n_fused; k++)
            for (int i = 0; i < fz[k].num_nodes; i++)
                fused_at[fz[k].nodes[i]] = fz[k].nodes[i] == fz[k].out_node ? k : -2;
    }

    int ret = 0;
    for (int oi = 0; oi < g->num_nodes && ret == 0; oi++) {
        const int nid = g->topo_order[oi];
        graph_node_t* n = &g->nodes[nid];
        if (n->type == OP_INPUT || n->type == OP_OUTPUT) continue;
        if (nid < g->fused_away_cap && g->fused_away[nid]) continue;
        if (fused_at && fused_at[nid] == -2) continue;
        int gpu = 0;
        if (fused_at && fused_at[nid] >= 0) {
            graph_mha_match_t* m = &fz[fused_at[nid]];
            int fin[2] = {m->input_tid, m->residual_tid};
            int fout[1] = {m->output_tid};
            graph_node_t fn;
            memset(&fn, 0, sizeof(fn));
            fn.type = OP_MHA_FUSED;
            fn.num_inputs = 2;
            fn.input_tensors = fin;
            fn.num_outputs = 1;
            fn.output_tensors = fout;
            fn.num_weights = 8;
            fn.weights = m->weights;
            fn.params = &m->params;
            fn.params_size = sizeof(m->params);
            ret = run_node(g, -1, &fn, use_cuda, fresh, &gpu, recording);
        } else {
            ret = run_node(g, nid, n, use_cuda, fresh, &gpu, recording);
        }
        if (!gpu) *all_gpu = 0;
    }
    free(fz);
    free(fused_at);
    return ret;
}

int graph_execute(inference_graph_t* g, tensor_t* inputs[], tensor_t* outputs[], bool use_cuda) {
    if (!g || !g->topo_order) return -1;
    if (g->num_inputs > 0 && !inputs) return -1;
    if (g->num_outputs > 0 && !outputs) return -1;
    if (use_cuda && !g->hip_graph && gpu_stream_create(&g->hip_graph) != 0) {
        g->hip_graph = NULL;
        return -1;
    }

    /* Graph inputs -> input-node tensors (host). */
    for (int i = 0; i < g->num_inputs; i++) {
        const graph_node_t* n = &g->nodes[g->input_node_ids[i]];
        if (n->num_outputs <= 0 || !inputs[i]) continue;
        const int tid = n->output_tensors[0];
        if (tid < 0 || tid >= g->num_tensors) continue;
        tensor_t* dst = g->tensors[tid].tensor;
        if (dst->data != inputs[i]->data) {
            if (inputs[i]->numel != dst->numel || inputs[i]->dtype != dst->dtype) return -1;
            memcpy(dst->data, inputs[i]->data, tensor_nbytes(dst));
        }
    }

    /* Tensors uploaded during this execution (so each external input moves once). */
    unsigned char* fresh = (unsigned char*)calloc((size_t)(g->num_tensors > 0 ? g->num_tensors : 1), 1);
    if (!fresh) return -1;

    int ret = 0;
    int in_graph = 0;   /* this execution launched the recording, its I/O copies included */
    const int replay = use_cuda && !g->replay_off;
    /* A buffer the recording points at was freed or handed to another stream since it was
     * made: record again. */
    if (replay && g->hip_graph_state == 2 && g->replay_generation != gpu_buffer_generation()) replay_reset(g);
    if (replay && g->hip_graph_state == 2 && g->hip_graph_exec) {
        ret = preload_inputs(g, fresh, UPLOAD_REPLAY);
        if (ret == 0 && g->replay_generation != gpu_buffer_generation()) {
            /* The preload itself replaced such a buffer: this execution runs eagerly. */
            replay_reset(g);
            pinned_clear_recorded(g);
            memset(fresh, 0, (size_t)(g->num_tensors > 0 ? g->num_tensors : 1));
            int all_gpu = 0;
            ret = run_nodes(g, use_cuda, fresh, &all_gpu, 0);
            if (ret == 0 && all_gpu) g->hip_graph_state = 1;
        } else if (ret == 0) {
            ret = gpu_graph_launch(g->hip_graph_exec, g->hip_graph);
            if (ret == 0) {
                decode_lens_replayed(g);
                in_graph = 1;
            }
        }
    } else if (replay && g->hip_graph_state == 1) {
        /* Record this execution's launches, then run the recording. */
        int all_gpu = 0, recorded = 0;
        void* exec = NULL;
        pinned_clear_recorded(g);
        ret = preload_inputs(g, fresh, UPLOAD_RECORD);
        /* Output staging is allocated before the capture (no allocation inside it). */
        for (int i = 0; i < g->num_outputs && ret == 0; i++) {
            const graph_node_t* n = &g->nodes[g->output_node_ids[i]];
            const int tid = n->type == OP_OUTPUT && n->num_inputs > 0 ? n->input_tensors[0] : -1;
            if (tid >= 0 && tid < g->num_tensors && g->tensors[tid].tensor->data_device)
                (void)pinned_of(g, tid, tensor_nbytes(g->tensors[tid].tensor));
        }
        const uint64_t gen = gpu_buffer_generation();
        if (ret == 0 && gpu_capture_begin(g->hip_graph) == 0) {
            int rrc = record_input_copies(g);
            if (rrc == 0) rrc = run_nodes(g, use_cuda, fresh, &all_gpu, 1);
            if (rrc == 0 && all_gpu) rrc = record_output_copies(g);
            const int crc = gpu_capture_end(g->hip_graph, &exec);
            if (rrc == 0 && crc == 0 && all_gpu && gen == gpu_buffer_generation()) {
                g->hip_graph_exec = exec;
                g->hip_graph_state = 2;
                g->replay_generation = gen;
                recorded = 1;
                ret = gpu_graph_launch(exec, g->hip_graph);
                in_graph = ret == 0;
            }
        }
        if (ret == 0 && !recorded) {
            /* Not recordable: run it eagerly, and do not try again until the graph or
             * its parameters change. */
            gpu_graph_exec_destroy(exec);
            (void)gpu_get_last_error();
            g->hip_graph_state = -1;
            pinned_clear_recorded(g);
            memset(fresh, 0, (size_t)(g->num_tensors > 0 ? g->num_tensors : 1));
            /* The failed recording's lengths bookkeeping ran ahead of the device. */
            for (int i = 0; i < g->decode_lens_cap; i++) ((decode_lens_t*)g->decode_lens)[i].held = -1;
            ret = run_nodes(g, use_cuda, fresh, &all_gpu, 0);
        }
    } else {
        int all_gpu = 0;
        ret = run_nodes(g, use_cuda, fresh, &all_gpu, 0);
        if (ret == 0 && replay && all_gpu && g->hip_graph_state == 0) g->hip_graph_state = 1;
    }
    free(fresh);
    if (ret != 0) return ret;

    /* Outputs come back on the graph's stream (one synchronisation, in the first
     * download); without device outputs, the stream is synchronised here. */
    int synced = 0;
    for (int i = 0; i < g->num_outputs; i++) {
        const graph_node_t* n = &g->nodes[g->output_node_ids[i]];
        if (n->type != OP_OUTPUT || n->num_inputs <= 0) continue;
        const int tid = n->input_tensors[0];
        if (tid < 0 || tid >= g->num_tensors) continue;
        tensor_t* src = g->tensors[tid].tensor;
        if (use_cuda && src->data_device) {
            const size_t bytes = tensor_nbytes(src);
            const pinned_t* rec = in_graph ? pinned_entry(g, tid) : NULL;
            void* stage = rec && rec->rec_out ? NULL : pinned_of(g, tid, bytes);
            if (rec && rec->rec_out) {
                /* The recording's last nodes copied it into the staging. */
                if (!synced && gpu_stream_synchronize(g->hip_graph) != 0) return -1;
                memcpy(src->data, rec->host, bytes);
            } else if (stage) {
                if (cf_launch_copy_bytes(stage, src->data_device, bytes, g->hip_graph) != 0 ||
                    gpu_stream_synchronize(g->hip_graph) != 0)
                    return -1;
                memcpy(src->data, stage, bytes);
            } else {
                if (gpu_stream_synchronize(g->hip_graph) != 0 || tensor_copy_to_host(src) != 0) return -1;
            }
            synced = 1;
        }
        if (outputs[i] && outputs[i]->data != src->data) {
            if (outputs[i]->numel != src->numel || outputs[i]->dtype != src->dtype) return -1;
            memcpy(outputs[i]->data, src->data, tensor_nbytes(src));
        }
    }
    /* Every launch has finished when graph_execute returns (caches included). */
    if (use_cuda && !synced) {
        const int rc = gpu_stream_synchronize(g->hip_graph);
        if (rc != 0) return rc;
    }
    return 0;
}
