// backend_amd_v2.h — AMD (MI355X) residency functions for the expert node's
// backend registry.  Drop-in replacement for the stub header of the same name
// (expert_node_v2/backend/amd/backend_amd_v2.h:7-23); the registry entry
// (backend_registry_v2.cc:72-80) binds these unchanged.  All device work goes
// through the C ABI of include/cx_moe.h (libcx_moe.so).
#pragma once

#include <cstdint>

#include "cx_moe.h"
#include "expert_node_v2/expert_format_v2.h"

namespace expert_node_v2 {

// How UploadExpertAmdV2 stores w_up and w_gate ([inter, hidden]): re-tiled
// on the device (CX_LAYOUT_TILE16, cx_upload_matrix_tiled) whenever the shape
// allows, else row-major.  BackendWorkspaceAmdV2 describes resident experts
// with the same rule, so the two always agree.
inline int AmdGateUpLayout(std::uint64_t rows, std::uint64_t cols) {
    return rows % 16 == 0 && cols % 128 == 0 ? CX_LAYOUT_TILE16 : CX_LAYOUT_ROWS;
}

// UploadExpertFnV2 (backend_registry_v2.h:21-24).  Validates the bundle with
// BuildExpertWeightsViewV2, then places each fp8 matrix and its fp32 scales
// in the device's HBM arena (cx_upload_matrix; up and gate through
// cx_upload_matrix_tiled where AmdGateUpLayout says so).  On failure the
// storage is left fully reset, as the contract requires.
bool UploadExpertAmdV2(
    int local_gpu_id,
    const ExpertTensorBundleV2& host_bundle,
    ExpertDeviceStorageV2* out_storage);

// FreeExpertWeightsFnV2 (backend_registry_v2.h:26-27): releases the six
// arena buffers and resets every field.
void FreeExpertWeightsAmdV2(ExpertDeviceStorageV2* storage);

}  // namespace expert_node_v2
