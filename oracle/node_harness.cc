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
//  * per worker, a second listener on worker_port + kLayerPortOffset whose
//    loop is the integrated worker loop: InferRequest as worker.cc:256-267,
//    plus the MoeLayerRequest branch (HandleMoeLayerRequestAmdV2);
//  * stdin: "quit" frees every resident expert through the registry
//    (ExpertRegistryV2::Reset -> FreeExpertWeightsAmdV2), whose
//    ExpertDeviceStorageV2 destructors abort on a leaked buffer
//    (expert_format_v2.h:141-157), reports the arena and exits 0 when it is
//    empty.
#include <sys/socket.h>
#include <netinet/in.h>
#include <unistd.h>

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

#include "common/header_codec.h"
#include "common/protocol.h"
#include "common/socket_utils.h"
#include "cx_moe.h"
#include "expert_node_v2/backend/amd/backend_workspace_amd_v2.h"
#include "expert_node_v2/backend/amd/moe_layer_worker_amd_v2.h"
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

constexpr int kLayerPortOffset = 100;

int Listen(int port) {
    int fd = ::socket(AF_INET, SOCK_STREAM, 0);
    if (fd < 0) return -1;
    int one = 1;
    ::setsockopt(fd, SOL_SOCKET, SO_REUSEADDR, &one, sizeof(one));
    sockaddr_in a{};
    a.sin_family = AF_INET;
    a.sin_addr.s_addr = htonl(INADDR_LOOPBACK);
    a.sin_port = htons(static_cast<std::uint16_t>(port));
    if (::bind(fd, reinterpret_cast<sockaddr*>(&a), sizeof(a)) != 0 || ::listen(fd, 16) != 0) {
        ::close(fd);
        return -1;
    }
    return fd;
}

// The worker loop with the integration's MoeLayerRequest branch.
void RunLayerWorkerLoop(GpuWorkerContextV2* ctx) {
    const auto& gpu = ctx->state->static_info.gpus[static_cast<std::size_t>(ctx->worker_id)];
    const auto& span = ctx->state->static_info.vendor_spans[static_cast<std::size_t>(gpu.gpu_vendor)];
    ctx->workspace = expert_node_v2::CreateBackendWorkspaceV2(gpu.gpu_vendor, span, ctx->worker_id);
    const int lfd = ctx->workspace ? Listen(ctx->worker_port) : -1;
    if (lfd < 0) {
        std::fprintf(stderr, "[harness] layer worker %d failed to start on port %d\n",
                     ctx->worker_id, ctx->worker_port);
        return;
    }
    std::printf("[harness] layer worker started worker_id=%d port=%d\n", ctx->worker_id,
                ctx->worker_port);
    std::fflush(stdout);
    for (;;) {
        const int fd = ::accept(lfd, nullptr, nullptr);
        if (fd < 0) continue;
        for (;;) {
            std::uint8_t hb[16];
            if (!common::RecvAll(fd, hb, sizeof(hb))) break;
            common::MsgHeader h{};
            if (!common::DecodeHeader(hb, sizeof(hb), &h) || h.magic != common::kMagic ||
                h.version != common::kVersion)
                break;
            std::string body(h.body_len, '\0');
            if (h.body_len > 0 && !common::RecvAll(fd, body.data(), h.body_len)) break;
            bool ok = false;
            if (h.msg_type == static_cast<std::uint16_t>(common::MsgType::InferRequest))
                ok = HandleInferRequest(fd, ctx, h, body);
            else if (h.msg_type == expert_node_v2::kMsgMoeLayerRequestV2)
                ok = expert_node_v2::HandleMoeLayerRequestAmdV2(fd, ctx, h, body);
            if (!ok) break;
        }
        ::close(fd);
    }
}

bool ParsePort(const char* s, int* out) {
    char* end = nullptr;
    const long v = std::strtol(s, &end, 10);
    if (end == s || *end != '\0' || v <= 0 || v > 65535 - kLayerPortOffset) return false;
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
        auto* l = new GpuWorkerContextV2();
        l->worker_id = gpu.worker_id;
        l->worker_port = static_cast<int>(gpu.worker_port) + kLayerPortOffset;
        l->state = state;
        std::thread(RunLayerWorkerLoop, l).detach();
        ctxs.push_back(c);
        ctxs.push_back(l);
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
