// graph.cpp -- capture a sequence of library calls on a stream into a HIP graph
// and replay it: the decode step of a serving loop (every layer's launches plus
// the logits) becomes one submission instead of ~16 launches per layer.
//
// Capture runs in thread-local mode: a call on the capturing thread that may not
// be recorded (hipMalloc, a synchronisation) fails instead of silently leaving
// the graph, so the first call of each GEMM shape (which creates the library
// plan and the stream's workspace) must run once eagerly before capture.  The
// library's kernels take every per-step value that changes between replays from
// device memory (positions, slots, context lengths, block tables); host
// arguments (row and sequence counts, the maximum context used for the decode
// grid, pointers) are fixed at capture.
#include "quantlib_amd.h"

#include <new>

struct ql_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

extern "C" hipError_t ql_graph_begin(hipStream_t stream) {
    if (!stream) return hipErrorInvalidValue;   // the null stream cannot be captured
    return hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal);
}

extern "C" hipError_t ql_graph_end(hipStream_t stream, ql_graph** out) {
    if (!stream || !out) return hipErrorInvalidValue;
    *out = nullptr;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(stream, &g);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return e;
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return e;
    }
    ql_graph* r = new (std::nothrow) ql_graph();
    if (!r) {
        (void)hipGraphExecDestroy(exec);
        (void)hipGraphDestroy(g);
        return hipErrorOutOfMemory;
    }
    r->graph = g;
    r->exec = exec;
    *out = r;
    return hipSuccess;
}

extern "C" hipError_t ql_graph_launch(ql_graph* g, hipStream_t stream) {
    if (!g || !g->exec) return hipErrorInvalidValue;
    return hipGraphLaunch(g->exec, stream);
}

extern "C" hipError_t ql_graph_destroy(ql_graph* g) {
    if (!g) return hipSuccess;
    hipError_t e = hipSuccess;
    if (g->exec) e = hipGraphExecDestroy(g->exec);
    if (g->graph) {
        const hipError_t e2 = hipGraphDestroy(g->graph);
        if (e == hipSuccess) e = e2;
    }
    delete g;
    return e;
}
