/*
 * inference_engine.h — session API (src/application/include/inference_engine.h:8-17).
 *
 * inference_session_run has the reference's contract (inference_engine.c:31-37): it
 * executes the session's graph with graph_execute.  ONNX parsing is not part of this
 * build, so inference_session_load reports an error and returns NULL; sessions are made
 * from an already-built graph with inference_session_from_graph (the graph is owned by
 * the session afterwards and destroyed with it).
 */
#ifndef CF_INFERENCE_ENGINE_H_
#define CF_INFERENCE_ENGINE_H_

#include "platform.h"
#include "graph.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct inference_session_t inference_session_t;

int  inference_engine_init(void);
void inference_engine_finalize(void);

inference_session_t* inference_session_load(const char* onnx_path);
inference_session_t* inference_session_from_graph(inference_graph_t* graph,
                                                  int num_inputs, int num_outputs);
int  inference_session_run(inference_session_t* session,
                           tensor_t* inputs[], tensor_t* outputs[], int use_cuda);
int  inference_session_num_inputs(inference_session_t* session);
int  inference_session_num_outputs(inference_session_t* session);
void inference_session_destroy(inference_session_t* session);

#ifdef __cplusplus
}
#endif

#endif /* CF_INFERENCE_ENGINE_H_ */
