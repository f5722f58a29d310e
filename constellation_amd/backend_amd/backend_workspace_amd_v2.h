// backend_workspace_amd_v2.h — per-worker execution state of the AMD backend:
// the BackendWorkspaceV2 implementation that CreateBackendWorkspaceV2 returns
// for GpuVendor::AMD (backend_workspace_v2.cc:79-80 currently returns
// nullptr).
#pragma once

#include <memory>

#include "expert_node_v2/backend/backend_workspace_v2.h"

struct cx_ctx;

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

    bool ok() const { return ctx_ != nullptr; }

private:
    int local_gpu_id_ = -1;
    cx_ctx* ctx_ = nullptr;
};

}  // namespace expert_node_v2
