/*
 * graph.h — the application-layer graph API, restricted to what the attention hot path
 * needs (construction, topological build, name-based dispatch, KV-cache hooks).
 *
 * Types and signatures follow src/application/engine/graph.h:13-122 of the reference:
 * the op_type_t enumerator values are identical (OP_MHA_FUSED = 28, OP_MHA_DECODE = 29)
 * and inference_graph_t keeps its field order.  graph_execute dispatches by the
 * reference's name rule (graph.c:836-884): "<base>_f16_cuda" when the node's output
 * tensor is F16, else "<base>_cuda", else the CPU "<base>"; only HIP operators are
 * registered by this library, so a CPU-only execution finds no op and returns -2 unless
 * the caller registered CPU ops itself.
 */
#ifndef CF_GRAPH_H_
#define CF_GRAPH_H_

#include "platform.h"
#include "operator.h"
#include "mha_fused_int.h"
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    OP_RELU,
    OP_SIGMOID,
    OP_GELU,
    OP_MATMUL,
    OP_CONV2D,
    OP_MAXPOOL2D,
    OP_AVGPOOL2D,
    OP_BATCHNORM,
    OP_ADD,
    OP_RESHAPE,
    OP_GLOBALAVGPOOL,
    OP_SOFTMAX,
    OP_SILU,
    OP_MUL,
    OP_CONCAT,
    OP_RESIZE,
    OP_TRANSPOSE,
    OP_SUB,
    OP_DIV,
    OP_SLICE,
    OP_SPLIT,
    OP_LAYERNORM,
    OP_GATHER,
    OP_SQUEEZE_UNSQUEEZE,
    OP_EXP,
    OP_REDUCE,
    OP_CAST,
    OP_ARGMAX,
    OP_MHA_FUSED,
    OP_MHA_DECODE,
    OP_CAUSAL_MASK,
    OP_ROPE,
    OP_PAD,
    OP_CLIP,
    OP_WHERE,
    OP_TANH,
    OP_INPUT,
    OP_OUTPUT
} op_type_t;

typedef struct {
    op_type_t  type;
    int        num_inputs;
    int        num_outputs;
    int*       input_tensors;   /* indices into graph->tensors[] */
    int*       output_tensors;
    int        num_weights;
    tensor_t** weights;         /* caller keeps ownership of the pointed-to tensors */
    void*      params;          /* copy of the op params */
    size_t     params_size;
} graph_node_t;

typedef struct {
    tensor_t* tensor;
    int       producer;  /* node writing it, -1 for a graph input */
    int       consumer;  /* last node reading it, -1 for a graph output */
} graph_tensor_t;

typedef struct {
    int             num_nodes;
    graph_node_t*   nodes;
    int             num_tensors;
    graph_tensor_t* tensors;
    int*            topo_order;
    int             num_inputs;
    int             num_outputs;
    int*            input_node_ids;
    int*            output_node_ids;
    /* KV-cache support for autoregressive decode */
    int             kv_cache_K_tid;  /* -1 if unused */
    int             kv_cache_V_tid;
    int             permanent_fusion;
    /* Stream and graph-replay state (the reference's CUDA-graph slots, graph.h:89-94):
     * hip_graph_state 0 = nothing recorded, 1 = one all-GPU execution done (the next
     * one is captured), 2 = captured (executions replay hip_graph_exec), -1 = not
     * capturable until the graph or its parameters change. */
    int             hip_graph_state;
    void*           hip_graph;       /* stream owned by this graph (hipStream_t, non-blocking) */
    void*           hip_graph_exec;  /* instantiated recording of one execution */
    int64_t         graph_cache_B;
    int64_t         graph_cache_S;
    int             replay_off;      /* graph_set_replay(g, 0) */
    uint64_t        replay_generation; /* gpu_buffer_generation() when hip_graph_exec was recorded */
    void*           decode_lens;     /* per node: device-held lengths of uniform decode nodes */
    int             decode_lens_cap; /* entries in decode_lens */
    void*           pinned;          /* per tensor: pinned host staging of graph inputs/outputs */
    int             pinned_cap;      /* entries in pinned */
    unsigned char*  fused_away;      /* per node: absorbed by a permanent MHA fusion (never runs) */
    int             fused_away_cap;  /* entries in fused_away */
} inference_graph_t;

inference_graph_t* graph_create(void);
int   graph_add_node(inference_graph_t* g, op_type_t type,
                     int num_inputs, const int* input_tensors,
                     int num_outputs, const int* output_tensors,
                     int num_weights, tensor_t** weights,
                     void* params, size_t params_size);
int   graph_add_tensor(inference_graph_t* g, tensor_t* t);
int   graph_set_input(inference_graph_t* g, int node_id);
int   graph_set_output(inference_graph_t* g, int node_id);
int   graph_build(inference_graph_t* g);
void  graph_destroy(inference_graph_t* g);

void  graph_set_kv_cache(inference_graph_t* g, int K_tensor_id, int V_tensor_id);
void  graph_update_cache_len(inference_graph_t* g, int64_t new_cache_len);
/* graph.c:151-153 and :810-815.  Off (the default): each GPU execution finds the
 * attention subgraphs again and runs each as one fused node without changing the graph.
 * On: the next GPU execution that finds them rewrites the graph for good: each match's
 * last node becomes that OP_MHA_FUSED node (inputs X and the residual, the 8 weights,
 * its params) and the match's other nodes are marked absorbed, so no later execution
 * runs them or looks for the pattern again.  Turning the flag off afterwards does not
 * undo a rewrite (the reference kept no restore record either).  A rewritten graph runs
 * its fused nodes through mha_fused_*_cuda, so it needs use_cuda. */
void  graph_set_permanent_fusion(inference_graph_t* g, int enable);

int   graph_execute(inference_graph_t* g, tensor_t* inputs[],
                    tensor_t* outputs[], bool use_cuda);

/* HIP-graph replay of GPU executions (on by default).  GPU executions run on a
 * non-blocking stream the graph owns.  After one execution in which every node ran on
 * the GPU, the next execution uploads the graph inputs, records the node launches into a
 * HIP graph and launches it; later executions only upload the inputs, replay the
 * recording and download the outputs.  A decode node's uniform cache_len is held on
 * the device and advanced by the recording, so a decode loop that moves cache_len by
 * one per step keeps replaying.  Adding nodes or tensors, graph_build,
 * graph_set_kv_cache, switching a decode node between uniform and per-sequence lengths,
 * and a change of gpu_buffer_generation() (a buffer the recording points at was freed)
 * discard the recording.  An execution with a CPU operator, or whose recording fails,
 * stays eager.  graph_set_replay(g, 0) turns it off; graph_replay_state(g) returns
 * hip_graph_state. */
void  graph_set_replay(inference_graph_t* g, int enable);
int   graph_replay_state(const inference_graph_t* g);

/* One self-attention subgraph, the pattern of the reference's detect_and_fuse_mha
 * (graph.c:347-665):
 *   X -> 3 x [MatMul (-> Add bias) -> Reshape -> Transpose] -> Q, K, V
 *   MatMul(Q, K) -> Mul(scale) (-> CausalMask) -> Softmax -> MatMul(., V)
 *   -> Transpose -> Reshape -> MatMul(W_O) (-> Add b_O) (-> Add residual)
 * Every intermediate tensor must have exactly one reader.  When use_cuda is set,
 * graph_execute runs each match as one OP_MHA_FUSED node in place of the pattern's last
 * node and skips the others; the graph itself is modified only under
 * graph_set_permanent_fusion. */
#define GRAPH_MHA_MAX_NODES 24
typedef struct {
    int       out_node;                      /* the pattern's last node */
    int       num_nodes;
    int       nodes[GRAPH_MHA_MAX_NODES];    /* every node of the pattern */
    int       input_tid;                     /* X (B, S, D) */
    int       residual_tid;                  /* -1 without a residual Add */
    int       output_tid;
    tensor_t* weights[8];                    /* W_Q, b_Q, W_K, b_K, W_V, b_V, W_O, b_O */
    mha_fused_params_t params;
} graph_mha_match_t;

/* Finds up to max_matches non-overlapping attention subgraphs (all of them, where the
 * reference fused the first only); returns how many.  No counterpart in the reference,
 * which keeps the detection static: it lets callers and tests see what graph_execute
 * will fuse. */
int   graph_detect_mha(const inference_graph_t* g, graph_mha_match_t* matches, int max_matches);

/* Name the executor would dispatch a node to (for tests): writes into buf, returns the
 * registry entry or NULL. */
const operator_registry_t* graph_resolve_op(const inference_graph_t* g, int node_id,
                                            bool use_cuda, char* buf, size_t buf_len);

#ifdef __cplusplus
}
#endif

#endif /* CF_GRAPH_H_ */
