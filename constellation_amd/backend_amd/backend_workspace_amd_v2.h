// backend_workspace_amd_v2.h — per-worker execution state of the AMD backend:
// the BackendWorkspaceV2 implementation that CreateBackendWorkspaceV2 returns
// for GpuVendor::AMD (backend_workspace_v2.cc:79-80 currently returns
// nullptr).
#pragma once

#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "expert_node_v2/backend/backend_workspace_v2.h"

struct cx_ctx;
struct cx_layer;

namespace expert_node_v2 {

class BackendWorkspaceAmdV2 final : public BackendWorkspaceV2 {
public:
    BackendWorkspaceAmdV2(int local_gpu_id, const ExpertWorkspaceConfigV2& config);
    ~BackendWorkspaceAmdV2() override;

    // RunExpertRequest (backend_workspace_v2.h:18-21): any batch >= 1,
    // fp16/bf16 in and out; persistent device + pinned buffers, no
    // per-request allocation.  Echoes batch_size, hidden_dim and
    // output_dtype like backend_workspace_cuda_v2.cc:91-95.
    bool RunExpertRequest(const ExpertDeviceStorageV2& storage,
                          const common::InferRequestMsg& req,
                          common::InferResponseMsg* resp) override;

    // Whole-layer request (MoeLayerRequest, msg_type 42; no counterpart in
    // the reference's v1 protocol): layer_experts[i] is the device storage of
    // the layer's local expert i on this worker (nullptr: not resident here),
    // shared the layer's shared expert (nullable).  Fills resp_body with the
    // MoeLayerResponse body; request-level failures are status codes in it
    // (1 unknown expert, 2 not resident, 4 execution failure, as
    // worker.cc:113-132).  Returns false only for a body that does not decode.
    // The device expert table of a layer is built once and reused while its
    // storages stay the same.
    bool RunMoeLayerRequest(int layer_id,
                            const std::vector<const ExpertDeviceStorageV2*>& layer_experts,
                            const ExpertDeviceStorageV2* shared, const std::string& req_body,
                            std::string* resp_body);

    bool ok() const { return ctx_ != nullptr; }

private:
    // Cached device table of one layer, keyed by the descriptors it was
    // built from (device pointers and blocks, so a re-uploaded expert at the
    // same storage address still invalidates it).
    struct LayerTable {
        std::vector<unsigned char> key;
        cx_layer* layer = nullptr;
    };
    cx_layer* layer_for(int layer_id, const std::vector<const ExpertDeviceStorageV2*>& experts,
                        const ExpertDeviceStorageV2* shared);

    int local_gpu_id_ = -1;
    cx_ctx* ctx_ = nullptr;
    std::unordered_map<int, LayerTable> layers_;
};

}  // namespace expert_node_v2
