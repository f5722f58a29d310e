// backend_amd_v2.cc — see backend_amd_v2.h.
#include "expert_node_v2/backend/amd/backend_amd_v2.h"

#include <cstdio>

#include "cx_moe.h"

namespace expert_node_v2 {

namespace {

bool UploadOneMatrixAmd(int device, const MatrixBlockScaleViewV2& view, bool gate_up,
                        MatrixMetaV2* meta, BlockScaleMetaV2* scale_meta,
                        DeviceBufferV2<std::uint8_t>* weight, DeviceBufferV2<float>* scale) {
    std::uint8_t* dw = nullptr;
    float* ds = nullptr;
    const std::uint64_t rows = static_cast<std::uint64_t>(view.matrix.rows);
    const std::uint64_t cols = static_cast<std::uint64_t>(view.matrix.cols);
    const bool tiled = gate_up && AmdGateUpLayout(rows, cols) == CX_LAYOUT_TILE16;
    const int rc = (tiled ? cx_upload_matrix_tiled : cx_upload_matrix)(
        device, view.weight.data.data(), rows, cols, view.scale.data.data(), view.scale.data.size(),
        &dw, &ds);
    if (rc != CX_OK) {
        std::fprintf(stderr, "[UploadExpertAmdV2] %s rc=%d: %s\n",
                     tiled ? "cx_upload_matrix_tiled" : "cx_upload_matrix", rc, cx_last_error());
        return false;
    }
    *meta = view.matrix;
    *scale_meta = view.scale_meta;
    weight->data = dw;
    weight->size = view.weight.data.size();
    scale->data = ds;
    scale->size = view.scale.data.size();
    return true;
}

template <class T>
void FreeOne(DeviceBufferV2<T>* b) {
    if (b->data != nullptr) cx_free_device(-1, b->data);
    b->data = nullptr;
    b->size = 0;
}

}  // namespace

bool UploadExpertAmdV2(int local_gpu_id, const ExpertTensorBundleV2& host_bundle,
                       ExpertDeviceStorageV2* out_storage) {
    if (local_gpu_id < 0 || out_storage == nullptr) return false;
    FreeExpertWeightsAmdV2(out_storage);
    ExpertWeightsViewV2 v;
    if (!BuildExpertWeightsViewV2(host_bundle, &v)) {
        std::fprintf(stderr, "[UploadExpertAmdV2] BuildExpertWeightsViewV2 failed local_gpu_id=%d\n",
                     local_gpu_id);
        host_bundle.debug_print("  ");
        return false;
    }
    ExpertDeviceStorageV2& s = *out_storage;
    if (!UploadOneMatrixAmd(local_gpu_id, v.w_up, true, &s.w_up_meta, &s.w_up_scale_meta,
                            &s.w_up_weight, &s.w_up_scale) ||
        !UploadOneMatrixAmd(local_gpu_id, v.w_gate, true, &s.w_gate_meta, &s.w_gate_scale_meta,
                            &s.w_gate_weight, &s.w_gate_scale) ||
        !UploadOneMatrixAmd(local_gpu_id, v.w_down, false, &s.w_down_meta, &s.w_down_scale_meta,
                            &s.w_down_weight, &s.w_down_scale)) {
        FreeExpertWeightsAmdV2(out_storage);
        return false;
    }
    return true;
}

void FreeExpertWeightsAmdV2(ExpertDeviceStorageV2* storage) {
    if (storage == nullptr) return;
    FreeOne(&storage->w_up_weight);
    FreeOne(&storage->w_up_scale);
    FreeOne(&storage->w_gate_weight);
    FreeOne(&storage->w_gate_scale);
    FreeOne(&storage->w_down_weight);
    FreeOne(&storage->w_down_scale);
    storage->w_up_meta = MatrixMetaV2{};
    storage->w_gate_meta = MatrixMetaV2{};
    storage->w_down_meta = MatrixMetaV2{};
    storage->w_up_scale_meta = BlockScaleMetaV2{};
    storage->w_gate_scale_meta = BlockScaleMetaV2{};
    storage->w_down_scale_meta = BlockScaleMetaV2{};
}

}  // namespace expert_node_v2
