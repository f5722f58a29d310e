// backend_workspace_amd_v2.cc — see backend_workspace_amd_v2.h.
#include "expert_node_v2/backend/amd/backend_workspace_amd_v2.h"

#include <cstdio>

#include "cx_moe.h"

namespace expert_node_v2 {

BackendWorkspaceAmdV2::BackendWorkspaceAmdV2(int local_gpu_id,
                                             const ExpertWorkspaceConfigV2& config)
    : BackendWorkspaceV2(config), local_gpu_id_(local_gpu_id) {
    if (local_gpu_id_ < 0) return;
    if (cx_ctx_create(local_gpu_id_, &ctx_) != CX_OK) {
        std::fprintf(stderr, "[BackendWorkspaceAmdV2] cx_ctx_create(%d): %s\n", local_gpu_id_,
                     cx_last_error());
        ctx_ = nullptr;
    }
}

BackendWorkspaceAmdV2::~BackendWorkspaceAmdV2() {
    if (ctx_ != nullptr) cx_ctx_destroy(ctx_);
}

bool BackendWorkspaceAmdV2::RunExpertRequest(const ExpertDeviceStorageV2& storage,
                                             const common::InferRequestMsg& req,
                                             common::InferResponseMsg* resp) {
    if (ctx_ == nullptr || resp == nullptr) return false;
    if (req.batch_size <= 0 || req.hidden_dim != config_.hidden_dim) return false;
    const int in = static_cast<int>(req.input_dtype);
    const int out = static_cast<int>(req.output_dtype);
    if ((in != CX_DTYPE_FP16 && in != CX_DTYPE_BF16) ||
        (out != CX_DTYPE_FP16 && out != CX_DTYPE_BF16)) {
        return false;
    }
    cx_expert_desc d{};
    d.w_up = storage.w_up_weight.data;
    d.s_up = storage.w_up_scale.data;
    d.w_gate = storage.w_gate_weight.data;
    d.s_gate = storage.w_gate_scale.data;
    d.w_down = storage.w_down_weight.data;
    d.s_down = storage.w_down_scale.data;
    d.hidden = storage.w_up_meta.cols;
    d.inter = storage.w_up_meta.rows;
    d.up_rb = storage.w_up_scale_meta.row_block;
    d.up_cb = storage.w_up_scale_meta.col_block;
    d.gate_rb = storage.w_gate_scale_meta.row_block;
    d.gate_cb = storage.w_gate_scale_meta.col_block;
    d.down_rb = storage.w_down_scale_meta.row_block;
    d.down_cb = storage.w_down_scale_meta.col_block;
    if (d.hidden != req.hidden_dim) return false;

    const std::size_t out_bytes =
        static_cast<std::size_t>(req.batch_size) * static_cast<std::size_t>(req.hidden_dim) * 2;
    resp->output.resize(out_bytes);
    const int rc = cx_expert_run_host(ctx_, &d, req.activation.data(), req.activation.size(), in,
                                      req.batch_size, resp->output.data(), out_bytes, out);
    if (rc != CX_OK) {
        std::fprintf(stderr, "[BackendWorkspaceAmdV2] cx_expert_run_host rc=%d: %s\n", rc,
                     cx_last_error());
        resp->output.clear();
        return false;
    }
    resp->status_code = 0;
    resp->batch_size = req.batch_size;
    resp->hidden_dim = req.hidden_dim;
    resp->output_dtype = req.output_dtype;
    return true;
}

}  // namespace expert_node_v2
