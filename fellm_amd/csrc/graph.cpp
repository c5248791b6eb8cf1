// Stream capture and replay of launch sequences as HIP graphs.
//
// replaces: crates/backend-cuda/src/graph.rs (CudaGraphCapture::begin /
// finish, CudaGraphExec::launch / drop).  Capture runs in thread-local mode
// on the caller's stream; finishing instantiates the graph and uploads it to
// the same stream, so the first replay pays no set-up.  An unfinished capture
// can be abandoned with fellm_rocm_graph_abort, which ends it and destroys
// what was recorded, leaving the stream out of capture mode.
//
// Every kernel of this library reads its per-step values (positions, row
// lengths, ids, the DeviceStepParams block) from device memory, so a graph
// recorded once is replayed with new values by updating that memory between
// replays; kernel arguments never change.
#include <hip/hip_runtime.h>

#include <new>

#include "fellm_abi.h"
#include "fellm_rocm.h"

namespace {

struct GraphExec {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace

extern "C" int fellm_rocm_graph_begin(void *stream) {
    if (!stream) return FELLM_ERR_ARITY;  // the null stream cannot be captured
    return hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal) == hipSuccess
               ? FELLM_OK
               : FELLM_ERR_LAUNCH;
}

extern "C" int fellm_rocm_graph_end(void *stream, void **graph_exec) {
    if (!stream || !graph_exec) return FELLM_ERR_ARITY;
    *graph_exec = nullptr;
    hipGraph_t graph = nullptr;
    if (hipStreamEndCapture(as_stream(stream), &graph) != hipSuccess || !graph) return FELLM_ERR_LAUNCH;
    hipGraphExec_t exec = nullptr;
    if (hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return FELLM_ERR_LAUNCH;
    }
    if (hipGraphUpload(exec, as_stream(stream)) != hipSuccess) {
        (void)hipGraphExecDestroy(exec);
        (void)hipGraphDestroy(graph);
        return FELLM_ERR_LAUNCH;
    }
    GraphExec *g = new (std::nothrow) GraphExec{graph, exec};
    if (!g) {
        (void)hipGraphExecDestroy(exec);
        (void)hipGraphDestroy(graph);
        return FELLM_ERR_ALLOC;
    }
    *graph_exec = g;
    return FELLM_OK;
}

extern "C" int fellm_rocm_graph_abort(void *stream) {
    if (!stream) return FELLM_ERR_ARITY;
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(as_stream(stream), &status) != hipSuccess) return FELLM_ERR_LAUNCH;
    if (status == hipStreamCaptureStatusNone) return FELLM_OK;
    hipGraph_t graph = nullptr;
    (void)hipStreamEndCapture(as_stream(stream), &graph);
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipGetLastError();  // clear the error an invalidated capture leaves behind
    return FELLM_OK;
}

extern "C" int fellm_rocm_graph_launch(void *graph_exec, void *stream) {
    if (!graph_exec) return FELLM_ERR_ARITY;
    const GraphExec *g = static_cast<const GraphExec *>(graph_exec);
    return hipGraphLaunch(g->exec, as_stream(stream)) == hipSuccess ? FELLM_OK : FELLM_ERR_LAUNCH;
}

extern "C" void fellm_rocm_graph_destroy(void *graph_exec) {
    if (!graph_exec) return;
    GraphExec *g = static_cast<GraphExec *>(graph_exec);
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

extern "C" int fellm_rocm_stream_is_capturing(void *stream) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(as_stream(stream), &status) != hipSuccess) return FELLM_ERR_LAUNCH;
    return status == hipStreamCaptureStatusActive ? 1 : 0;
}
