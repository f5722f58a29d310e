// ref_shim.cc — extern "C" entry points over the reference's own CPU expert
// sources, so tests can use the unmodified reference C++ as a checker.
//
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile into oracle/_ref/
// together with these reference files, compiled where they lie under
// /root/reference (nothing is copied):
//   expert_node_v2/expert_format_v2.cc            (BuildExpertWeightsViewV2)
//   expert_node_v2/backend/fp8_lut_v2.cc          (DecodeFp8ByteV2)
//   expert_node_v2/backend/expert_reference_v2.cc (RunExpertReferenceV2)
//   expert_node_v2/backend/dummy_expert_data_v2.cc(FillDummyExpertBundleV2)
//   expert_node_v2/backend/cpu/{backend_cpu_v2,fused_up_gate_cpu_v2,
//                                down_cpu_v2}.cc  (the CPU expert path)
// Only the wrappers below are this repository's code.
#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "expert_node_v2/backend/activation_codec_v2.h"
#include "expert_node_v2/backend/cpu/backend_cpu_v2.h"
#include "expert_node_v2/backend/cpu/down_cpu_v2.h"
#include "expert_node_v2/backend/cpu/fused_up_gate_cpu_v2.h"
#include "expert_node_v2/backend/dummy_expert_data_v2.h"
#include "expert_node_v2/backend/expert_reference_v2.h"
#include "expert_node_v2/backend/fp8_lut_v2.h"
#include "expert_node_v2/expert_format_v2.h"

#define REF_API extern "C" __attribute__((visibility("default")))

namespace {

void SetTensor(HostTensorV2* t, const void* data, std::size_t nbytes,
               std::uint64_t d0, std::uint64_t d1, const char* dtype,
               int rb, int cb) {
    t->bytes.assign(static_cast<const std::uint8_t*>(data),
                    static_cast<const std::uint8_t*>(data) + nbytes);
    t->meta.shape = {d0, d1};
    t->meta.dtype = dtype;
    t->meta.row_block = static_cast<std::uint32_t>(rb);
    t->meta.col_block = static_cast<std::uint32_t>(cb);
    t->ready = true;
}

bool MakeBundle(const std::uint8_t* wu, const float* su,
                const std::uint8_t* wg, const float* sg,
                const std::uint8_t* wd, const float* sd,
                int hidden, int inter, int rb, int cb,
                ExpertTensorBundleV2* b) {
    const std::uint64_t H = hidden, I = inter;
    const std::uint64_t ur = (I + rb - 1) / rb, uc = (H + cb - 1) / cb;
    const std::uint64_t dr = (H + rb - 1) / rb, dc = (I + cb - 1) / cb;
    SetTensor(&b->w_up, wu, I * H, I, H, "float8_e4m3fn", rb, cb);
    SetTensor(&b->w_up_scale, su, ur * uc * 4, ur, uc, "float32", rb, cb);
    SetTensor(&b->w_gate, wg, I * H, I, H, "float8_e4m3fn", rb, cb);
    SetTensor(&b->w_gate_scale, sg, ur * uc * 4, ur, uc, "float32", rb, cb);
    SetTensor(&b->w_down, wd, H * I, H, I, "float8_e4m3fn", rb, cb);
    SetTensor(&b->w_down_scale, sd, dr * dc * 4, dr, dc, "float32", rb, cb);
    return true;
}

struct CpuExpert {
    ExpertTensorBundleV2 bundle;
    ExpertDeviceStorageV2 storage;
    ExpertWorkspaceCpuV2 ws{};
    bool storage_ok = false;
    bool ws_ok = false;
    ~CpuExpert() {
        if (ws_ok) FreeExpertWorkspaceCpuV2(&ws);
        if (storage_ok) FreeExpertWeightsCpuV2(&storage);
    }
};

}  // namespace

REF_API float ref_fp8_decode(int fmt, std::uint8_t v) {
    return DecodeFp8ByteV2(static_cast<Fp8Format>(fmt), v);
}

REF_API std::uint16_t ref_encode(int dtype, float v) {
    return EncodeActivationFromFloatV2(static_cast<common::ActivationDType>(dtype), v);
}

REF_API float ref_decode(int dtype, std::uint16_t v) {
    return DecodeActivationToFloatV2(static_cast<common::ActivationDType>(dtype), v);
}

// FillDummyExpertBundleV2 (dummy_expert_data_v2.cc:9-132) copied out.
REF_API int ref_fill_dummy(int hidden, int inter, int rb, int cb,
                           std::uint8_t* wu, float* su, std::uint8_t* wg, float* sg,
                           std::uint8_t* wd, float* sd) {
    DummyExpertShapeV2 shape;
    shape.hidden_dim = hidden;
    shape.inter_dim = inter;
    shape.row_block = rb;
    shape.col_block = cb;
    ExpertTensorBundleV2 b;
    FillDummyExpertBundleV2(&b, shape);
    std::memcpy(wu, b.w_up.bytes.data(), b.w_up.bytes.size());
    std::memcpy(su, b.w_up_scale.bytes.data(), b.w_up_scale.bytes.size());
    std::memcpy(wg, b.w_gate.bytes.data(), b.w_gate.bytes.size());
    std::memcpy(sg, b.w_gate_scale.bytes.data(), b.w_gate_scale.bytes.size());
    std::memcpy(wd, b.w_down.bytes.data(), b.w_down.bytes.size());
    std::memcpy(sd, b.w_down_scale.bytes.data(), b.w_down_scale.bytes.size());
    return 0;
}

// FillDummyInputActivationV2 (dummy_expert_data_v2.cc:134-150).
REF_API int ref_fill_dummy_input(int hidden, int dtype, float* xf, std::uint16_t* xe) {
    std::vector<float> f;
    std::vector<std::uint16_t> e;
    FillDummyInputActivationV2(hidden, static_cast<common::ActivationDType>(dtype), &f, &e);
    std::memcpy(xf, f.data(), f.size() * 4);
    std::memcpy(xe, e.data(), e.size() * 2);
    return 0;
}

// RunExpertReferenceV2 (expert_reference_v2.cc:146-178) on one token.
REF_API int ref_expert_reference(const std::uint8_t* wu, const float* su,
                                 const std::uint8_t* wg, const float* sg,
                                 const std::uint8_t* wd, const float* sd,
                                 int hidden, int inter, int rb, int cb,
                                 const std::uint16_t* x, int in_dtype, int out_dtype,
                                 std::uint16_t* y, float* h) {
    ExpertTensorBundleV2 b;
    MakeBundle(wu, su, wg, sg, wd, sd, hidden, inter, rb, cb, &b);
    ExpertWeightsViewV2 view;
    if (!BuildExpertWeightsViewV2(b, &view)) return -1;
    std::vector<std::uint8_t> yb;
    std::vector<float> hv;
    if (!RunExpertReferenceV2(view, x, static_cast<common::ActivationDType>(in_dtype),
                              static_cast<common::ActivationDType>(out_dtype), &yb, &hv)) {
        return -2;
    }
    std::memcpy(y, yb.data(), yb.size());
    std::memcpy(h, hv.data(), hv.size() * 4);
    return 0;
}

// The reference CPU backend: UploadExpertCpuV2 + InitExpertWorkspaceCpuV2,
// then RunFusedUpGateCpuV2 / RunDownCpuV2 with an explicit OpenMP thread
// count (RunExpertCpuV2 itself fixes 12, backend_cpu_v2.cc:245-246).
REF_API void* ref_cpu_expert_create(const std::uint8_t* wu, const float* su,
                                    const std::uint8_t* wg, const float* sg,
                                    const std::uint8_t* wd, const float* sd,
                                    int hidden, int inter, int rb, int cb) {
    auto* e = new (std::nothrow) CpuExpert();
    if (e == nullptr) return nullptr;
    MakeBundle(wu, su, wg, sg, wd, sd, hidden, inter, rb, cb, &e->bundle);
    if (!UploadExpertCpuV2(0, e->bundle, &e->storage)) { delete e; return nullptr; }
    e->storage_ok = true;
    e->bundle.clear();
    ExpertWorkspaceConfigV2 cfg;
    cfg.hidden_dim = hidden;
    cfg.inter_dim = inter;
    if (!InitExpertWorkspaceCpuV2(cfg, &e->ws)) { delete e; return nullptr; }
    e->ws_ok = true;
    return e;
}

REF_API int ref_cpu_expert_run(void* handle, const std::uint16_t* x, int in_dtype,
                               std::uint16_t* y, int out_dtype, int omp_threads) {
    auto* e = static_cast<CpuExpert*>(handle);
    if (e == nullptr) return -1;
    const ExpertWeightsViewV2 v = e->storage.view();
    if (omp_threads <= 0) {
        return RunExpertCpuV2(v, &e->ws, x, static_cast<common::ActivationDType>(in_dtype), y,
                              static_cast<common::ActivationDType>(out_dtype)) ? 0 : -2;
    }
    if (!RunFusedUpGateCpuV2(v.w_up, v.w_gate, x, static_cast<common::ActivationDType>(in_dtype),
                             e->ws.tmp.data, omp_threads)) {
        return -2;
    }
    if (!RunDownCpuV2(v.w_down, e->ws.tmp.data, y, static_cast<common::ActivationDType>(out_dtype),
                      omp_threads)) {
        return -3;
    }
    return 0;
}

REF_API void ref_cpu_expert_destroy(void* handle) {
    delete static_cast<CpuExpert*>(handle);
}
