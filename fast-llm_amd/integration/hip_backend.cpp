// hip_backend.cpp -- the binding a maintainer adds to the reference runtime
// (as src/runtime/hip_backend.cpp) so that its frozen decode graph runs the
// quantized matvec tasks through libfastllm_hip.  It is not part of the
// library; tests/test_integration_binding.py compiles and links it against
// the reference's own headers (include/fastllm/fastllm.h,
// src/runtime/runtime_internal.h) where they are present.
// Built only with -DFASTLLM_HIP=ON; links -lfastllm_hip.
#include <cstdio>
#include <cstdlib>

#include "fastllm_hip.h"
#include "runtime_internal.h"

namespace fastllm {

struct HipBackend {
    void * stream = nullptr;
    void * graph  = nullptr;          // captured once per frozen graph
    flh_arena * arena = nullptr;

    static void check(int rc, const char * what) {
        if (rc != FLH_OK) {
            fprintf(stderr, "fastllm: %s failed (%d): %s\n", what, rc, flh_last_error());
            abort();                  // the reference's error behaviour
        }
    }

    // replaces Arena::create's cudaMallocManaged region
    void init(int device, size_t arena_bytes) {
        check(flh_init(device), "flh_init");
        check(flh_stream_create(&stream), "flh_stream_create");
        check(flh_arena_create(arena_bytes, &arena), "flh_arena_create");
    }

    void * alloc(size_t bytes, size_t align) {
        void * p = nullptr;
        check(flh_arena_alloc(arena, bytes, align, &p), "flh_arena_alloc");
        return p;
    }

    // The decoder's aux_alloc (src/model/decoder.cpp:779) for the decode-op
    // param blocks (RmsNormP, RouterSelP, SiluMulP, WmergeP): flh_exec_tasks
    // reads them on the host, so they live in pinned host memory, not in the
    // device arena.  Freed by the caller with flh_host_free at shutdown.
    void * aux_alloc(size_t bytes) {
        void * p = nullptr;
        check(flh_host_alloc(bytes, &p), "flh_host_alloc");
        return p;
    }

    // One token: the frozen task table in topological order (run_serial's
    // order, src/runtime/graph.cpp:116-148).  `tasks` is the host copy of
    // Graph::tasks_; all pointers inside refer to arena memory.
    void run_token(const Task * tasks, uint32_t n, const RtShared * sh) {
        static_assert(sizeof(Task) == sizeof(flh_task), "Task layout");
        if (!graph) {                 // capture once, replay per token
            check(flh_graph_capture_begin(stream), "capture_begin");
            check(flh_exec_tasks(reinterpret_cast<const flh_task *>(tasks), n,
                                 sh->fast_kernels, sh->i8_cpu_mask,
                                 sh->i8k_cpu_mask, stream), "flh_exec_tasks");
            check(flh_graph_capture_end(stream, &graph), "capture_end");
        }
        check(flh_graph_launch(graph, stream), "flh_graph_launch");
        check(flh_stream_sync(stream), "flh_stream_sync");
    }

    void shutdown() {
        if (graph) flh_graph_destroy(graph);
        flh_stream_destroy(stream);
        flh_arena_destroy(arena);
    }
};

}  // namespace fastllm
