/*
 * inference_engine.c — session wrapper over a graph
 * (src/application/engine/inference_engine.c:10-53 of the reference).
 */
#include "inference_engine.h"
#include "operator.h"

#include <stdio.h>
#include <stdlib.h>

struct inference_session_t {
    inference_graph_t* graph;
    int num_inputs;
    int num_outputs;
};

int inference_engine_init(void) {
    platform_init();
    return operator_init_all();
}

void inference_engine_finalize(void) { platform_finalize(); }

inference_session_t* inference_session_load(const char* onnx_path) {
    fprintf(stderr, "inference_session_load(%s): ONNX parsing is not part of this build; "
                    "use inference_session_from_graph\n", onnx_path ? onnx_path : "(null)");
    return NULL;
}

inference_session_t* inference_session_from_graph(inference_graph_t* graph, int num_inputs, int num_outputs) {
    if (!graph || !graph->topo_order) return NULL;
    inference_session_t* s = (inference_session_t*)calloc(1, sizeof(*s));
    if (!s) return NULL;
    s->graph = graph;
    s->num_inputs = num_inputs >= 0 ? num_inputs : graph->num_inputs;
    s->num_outputs = num_outputs >= 0 ? num_outputs : graph->num_outputs;
    return s;
}

/* inference_engine.c:31-37 */
int inference_session_run(inference_session_t* session, tensor_t* inputs[], tensor_t* outputs[], int use_cuda) {
    if (!session || !session->graph) return -1;
    return graph_execute(session->graph, inputs, outputs, use_cuda != 0);
}

int inference_session_num_inputs(inference_session_t* session) { return session ? session->num_inputs : 0; }
int inference_session_num_outputs(inference_session_t* session) { return session ? session->num_outputs : 0; }

void inference_session_destroy(inference_session_t* session) {
    if (!session) return;
    graph_destroy(session->graph);
    free(session);
}
