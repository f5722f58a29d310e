// backend_workspace_amd_v2.cc — see backend_workspace_amd_v2.h.
#include "expert_node_v2/backend/amd/backend_workspace_amd_v2.h"

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <utility>

#include "cx_moe.h"
#include "expert_node_v2/backend/amd/backend_amd_v2.h"

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
    for (auto& kv : layers_)
        if (kv.second.layer != nullptr) cx_layer_destroy(ctx_, kv.second.layer);
    if (ctx_ != nullptr) cx_ctx_destroy(ctx_);
}

namespace {

// The device pointers and block metadata of one resident expert.
cx_expert_desc describe(const ExpertDeviceStorageV2& storage) {
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
    d.gu_layout = AmdGateUpLayout(storage.w_up_meta.rows, storage.w_up_meta.cols);  // as uploaded
    return d;
}

}  // namespace

cx_layer* BackendWorkspaceAmdV2::layer_for(
    int layer_id, const std::vector<const ExpertDeviceStorageV2*>& experts,
    const ExpertDeviceStorageV2* shared) {
    std::vector<cx_expert_desc> descs(experts.size());
    std::vector<const cx_expert_desc*> ptrs(experts.size(), nullptr);
    for (std::size_t i = 0; i < experts.size(); ++i) {
        if (experts[i] == nullptr) continue;
        descs[i] = describe(*experts[i]);
        ptrs[i] = &descs[i];
    }
    cx_expert_desc sd{};
    if (shared != nullptr) sd = describe(*shared);
    // key: residency bits, then every descriptor (zeroed where absent)
    std::vector<unsigned char> key(experts.size() + 1 + sizeof(cx_expert_desc) * (descs.size() + 1));
    for (std::size_t i = 0; i < experts.size(); ++i) key[i] = experts[i] != nullptr;
    key[experts.size()] = shared != nullptr;
    std::memcpy(key.data() + experts.size() + 1, descs.data(), sizeof(cx_expert_desc) * descs.size());
    std::memcpy(key.data() + experts.size() + 1 + sizeof(cx_expert_desc) * descs.size(), &sd,
                sizeof(sd));
    LayerTable& t = layers_[layer_id];
    if (t.layer != nullptr && t.key == key) return t.layer;
    if (t.layer != nullptr) cx_layer_destroy(ctx_, t.layer);
    t.layer = nullptr;
    t.key.clear();
    if (cx_layer_create(ctx_, static_cast<int>(experts.size()), ptrs.data(),
                        shared != nullptr ? &sd : nullptr, &t.layer) != CX_OK) {
        std::fprintf(stderr, "[BackendWorkspaceAmdV2] cx_layer_create(layer %d): %s\n", layer_id,
                     cx_last_error());
        t.layer = nullptr;
        return nullptr;
    }
    t.key = std::move(key);
    return t.layer;
}

bool BackendWorkspaceAmdV2::RunMoeLayerRequest(
    int layer_id, const std::vector<const ExpertDeviceStorageV2*>& layer_experts,
    const ExpertDeviceStorageV2* shared, const std::string& req_body, std::string* resp_body) {
    if (ctx_ == nullptr || resp_body == nullptr) return false;
    const auto* body = reinterpret_cast<const std::uint8_t*>(req_body.data());
    cx_moe_layer_request_info info{};
    if (cx_moe_layer_request_peek(body, req_body.size(), &info) != CX_OK) {
        std::fprintf(stderr, "[BackendWorkspaceAmdV2] bad MoeLayerRequest: %s\n", cx_last_error());
        return false;
    }
    resp_body->assign(cx_moe_layer_response_size(info.batch_size, info.hidden_dim), '\0');
    auto* out = reinterpret_cast<std::uint8_t*>(resp_body->data());
    cx_layer* layer = layer_for(layer_id, layer_experts, shared);
    std::size_t n = 0;
    if (layer == nullptr) {
        // no resident expert of this layer here: status 2, no output
        const std::uint32_t hdr[5] = {2u, static_cast<std::uint32_t>(info.batch_size),
                                      static_cast<std::uint32_t>(info.hidden_dim),
                                      info.output_dtype, 0u};
        std::memcpy(out, hdr, sizeof(hdr));
        resp_body->resize(sizeof(hdr));
        return true;
    }
    const int rc = cx_moe_layer_request_run(ctx_, layer, body, req_body.size(), out,
                                            resp_body->size(), &n);
    if (rc != CX_OK) {
        std::fprintf(stderr, "[BackendWorkspaceAmdV2] cx_moe_layer_request_run rc=%d: %s\n", rc,
                     cx_last_error());
        return false;
    }
    resp_body->resize(n);
    return true;
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
    const cx_expert_desc d = describe(storage);
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
