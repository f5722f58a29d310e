// moe_layer_worker_amd_v2.cc — see moe_layer_worker_amd_v2.h.
#include "expert_node_v2/backend/amd/moe_layer_worker_amd_v2.h"

#include <cstdio>
#include <shared_mutex>
#include <vector>

#include "common/socket_utils.h"
#include "cx_moe.h"
#include "expert_node_v2/backend/amd/backend_workspace_amd_v2.h"
#include "expert_node_v2/control.h"

namespace expert_node_v2 {

bool HandleMoeLayerRequestAmdV2(int fd, GpuWorkerContextV2* ctx, const common::MsgHeader& req,
                                const std::string& req_body, int experts_per_layer) {
    if (ctx == nullptr || ctx->state == nullptr || !ctx->workspace || experts_per_layer <= 0) {
        std::fprintf(stderr, "[worker] HandleMoeLayerRequestAmdV2: invalid context\n");
        return false;
    }
    auto* ws = dynamic_cast<BackendWorkspaceAmdV2*>(ctx->workspace.get());
    if (ws == nullptr) {
        std::fprintf(stderr, "[worker] MoeLayerRequest needs the AMD workspace\n");
        return false;
    }
    cx_moe_layer_request_info info{};
    if (cx_moe_layer_request_peek(reinterpret_cast<const std::uint8_t*>(req_body.data()),
                                  req_body.size(), &info) != CX_OK) {
        std::fprintf(stderr, "[%s] failed to decode MoeLayerRequest: %s\n",
                     ctx->state->static_info.node_id.c_str(), cx_last_error());
        return false;
    }
    std::string resp_body;
    bool ok = false;
    {
        std::shared_lock<std::shared_mutex> lock(ctx->state->mu);
        const ExpertRegistryV2& reg = ctx->state->registry;
        std::vector<const ExpertDeviceStorageV2*> experts(static_cast<std::size_t>(experts_per_layer),
                                                          nullptr);
        const std::int64_t base = static_cast<std::int64_t>(info.layer_id) * experts_per_layer;
        if (info.layer_id >= 0 && base + experts_per_layer <= kSharedExpertIdBaseV2) {
            for (int i = 0; i < experts_per_layer; ++i)
                experts[static_cast<std::size_t>(i)] =
                    reg.FindDeviceStorage(static_cast<int>(base + i), ctx->worker_id);
        }
        const ExpertDeviceStorageV2* shared =
            (info.flags & CX_MOE_LAYER_FLAG_SHARED) && info.layer_id >= 0
                ? reg.FindDeviceStorage(SharedExpertIdV2(info.layer_id), ctx->worker_id)
                : nullptr;
        ok = ws->RunMoeLayerRequest(info.layer_id, experts, shared, req_body, &resp_body);
    }
    if (!ok) return false;
    common::MsgHeader resp{};
    resp.magic = common::kMagic;
    resp.version = common::kVersion;
    resp.msg_type = kMsgMoeLayerResponseV2;
    resp.request_id = req.request_id;
    resp.body_len = static_cast<std::uint32_t>(resp_body.size());
    return common::SendMessage(fd, resp, resp_body);
}

}  // namespace expert_node_v2
