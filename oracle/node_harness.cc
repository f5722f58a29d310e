// node_harness.cc — test infrastructure: the reference's expert node with this
// repository's AMD backend plugin, for tests/test_gpu_node.py.
//
// oracle/Makefile (target `node`) compiles the reference's node sources where
// they lie under /root/reference (control loop, worker loop, registry, expert
// format, node info, backend registry, common/ codecs) with
// EXPERT_NODE_V2_ENABLE_AMD=1 and the other backends off, puts
// constellation_amd/backend_amd/ in front of the reference's AMD stub headers,
// and links this file and libcx_moe.so.  Nothing of the reference is copied.
//
// main() follows expert_node_v2/main.cc:94-157: BuildStaticNodeInfo through
// the backend registry, the control loop on its thread (it starts the
// resident_bg upload thread itself), one RunGpuWorkerLoopV2 thread per worker.
// Additions a test needs:
//  * CreateBackendWorkspaceV2 with the AMD case that the integration adds to
//    backend_workspace_v2.cc:79-80 (the reference's file, which returns
//    nullptr for AMD, is not linked);
//  * RunGpuWorkerLoopV2 is the reference's worker.cc with the integration's
//    one-branch edit (oracle/integrate_worker.awk streams it to the compiler):
//    each worker port answers InferRequest and MoeLayerRequest
//    (HandleMoeLayerRequestAmdV2);
//  * stdin: "quit" frees every resident expert through the registry
//    (ExpertRegistryV2::Reset -> FreeExpertWeightsAmdV2), whose
//    ExpertDeviceStorageV2 destructors abort on a leaked buffer
//    (expert_format_v2.h:141-157), reports the arena and exits 0 when it is
//    empty.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <memory>
#include <mutex>
#include <shared_mutex>
#include <string>
#include <thread>
#include <vector>

#include "cx_moe.h"
#include "expert_node_v2/backend/amd/backend_workspace_amd_v2.h"
#include "expert_node_v2/backend/backend_workspace_v2.h"
#include "expert_node_v2/control.h"
#include "expert_node_v2/node_info.h"
#include "expert_node_v2/worker.h"

namespace expert_node_v2 {

// The factory with the integration's AMD case; every other vendor is off in
// this build.
std::unique_ptr<BackendWorkspaceV2> CreateBackendWorkspaceV2(common::GpuVendor vendor,
                                                             const common::VendorWorkerSpan& span,
                                                             int worker_id) {
    if (vendor != common::GpuVendor::AMD) return nullptr;
    if (worker_id < span.worker_id_begin || worker_id >= span.worker_id_begin + span.worker_count)
        return nullptr;
    ExpertWorkspaceConfigV2 cfg;
    cfg.hidden_dim = 7168;
    cfg.inter_dim = 2048;
    auto p = std::make_unique<BackendWorkspaceAmdV2>(worker_id - span.worker_id_begin, cfg);
    if (!p->ok()) return nullptr;
    return p;
}

}  // namespace expert_node_v2

namespace {

bool ParsePort(const char* s, int* out) {
    char* end = nullptr;
    const long v = std::strtol(s, &end, 10);
    if (end == s || *end != '\0' || v <= 0 || v > 65535) return false;
    *out = static_cast<int>(v);
    return true;
}

}  // namespace

int main(int argc, char** argv) {
    int control_port = 0, worker_base = 0;
    for (int i = 1; i + 1 < argc; i += 2) {
        if (std::strcmp(argv[i], "--control-port") == 0 && ParsePort(argv[i + 1], &control_port)) continue;
        if (std::strcmp(argv[i], "--worker-base-port") == 0 && ParsePort(argv[i + 1], &worker_base)) continue;
        std::fprintf(stderr, "usage: %s --control-port P --worker-base-port W\n", argv[0]);
        return 2;
    }
    if (control_port == 0 || worker_base == 0) {
        std::fprintf(stderr, "usage: %s --control-port P --worker-base-port W\n", argv[0]);
        return 2;
    }
    setvbuf(stdout, nullptr, _IOLBF, 0);
    auto* state = new ControlState();  // lives until exit, as in main.cc
    if (!BuildStaticNodeInfo("amd_node0", "127.0.0.1", control_port, worker_base,
                             &state->static_info)) {
        std::fprintf(stderr, "BuildStaticNodeInfo failed\n");
        return 1;
    }
    std::printf("[harness] num_gpus=%zu\n", state->static_info.gpus.size());
    std::thread(RunControlLoop, state).detach();
    std::vector<GpuWorkerContextV2*> ctxs;
    for (const auto& gpu : state->static_info.gpus) {
        auto* c = new GpuWorkerContextV2();
        c->worker_id = gpu.worker_id;
        c->worker_port = static_cast<int>(gpu.worker_port);
        c->state = state;
        std::thread(RunGpuWorkerLoopV2, c).detach();
        ctxs.push_back(c);
    }
    std::string line;
    while (std::getline(std::cin, line)) {
        if (line != "quit") continue;
        std::uint64_t before = 0, after = 0;
        {
            std::unique_lock<std::shared_mutex> lock(state->mu);
            cx_arena_stats(0, &before, nullptr);
            state->registry.Reset();
            cx_arena_stats(0, &after, nullptr);
        }
        std::printf("[harness] reset: arena used %llu -> %llu bytes\n",
                    static_cast<unsigned long long>(before), static_cast<unsigned long long>(after));
        std::fflush(stdout);
        std::_Exit(after == 0 ? 0 : 3);
    }
    std::_Exit(0);  // stdin closed without "quit": no teardown under the detached threads
}
