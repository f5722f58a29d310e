// gpu_info_amd_v2.cc — replaces the stubs of the same file
// (expert_node_v2/backend/amd/gpu_info_amd_v2.cc:3-21; contract
// backend_registry_v2.h:12-19 and backend/SKILL.md "Static/Dynamic info should
// fill").  One worker per visible AMD GPU, worker ids contiguous from
// worker_id_begin, worker_port = base + worker_id as the CUDA backend does
// (backend/cuda/gpu_info_cuda_v2.cc:59-64).
#include "expert_node_v2/backend/amd/gpu_info_amd_v2.h"

#include <utility>

#include "cx_moe.h"

bool BuildLocalAmdGpuInfosV2(std::int32_t worker_id_begin, std::uint32_t worker_port_base,
                             std::vector<common::StaticGpuInfo>* out) {
    if (out == nullptr) return false;
    out->clear();
    int count = 0;
    if (cx_device_count(&count) != CX_OK) return false;  // as gpu_info_cuda_v2.cc:47-50
    for (int i = 0; i < count; ++i) {
        cx_device_info info;
        if (cx_device_query(i, &info) != CX_OK) continue;
        common::StaticGpuInfo g;
        g.worker_id = worker_id_begin + i;
        g.gpu_name = info.name;
        g.total_mem_bytes = info.total_mem_bytes;
        g.worker_port = worker_port_base + static_cast<std::uint32_t>(g.worker_id);
        g.gpu_vendor = common::GpuVendor::AMD;
        g.capability_flags = info.capability_flags;
        g.arch_name = info.arch;
        out->push_back(std::move(g));
    }
    return true;
}

bool BuildLocalAmdDynamicGpuInfosV2(std::int32_t worker_id_begin,
                                    std::vector<common::DynamicGpuInfo>* out) {
    if (out == nullptr) return false;
    out->clear();
    int count = 0;
    if (cx_device_count(&count) != CX_OK) return false;
    for (int i = 0; i < count; ++i) {
        cx_device_info info;
        if (cx_device_query(i, &info) != CX_OK) continue;
        common::DynamicGpuInfo g;
        g.worker_id = worker_id_begin + i;
        g.free_mem_bytes = info.free_mem_bytes;
        g.gpu_status = common::GpuStatus::Idle;
        out->push_back(std::move(g));
    }
    return true;
}
