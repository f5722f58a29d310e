// cx_internal.h — shared declarations of the gfx950 MoE engine (not part of
// the public ABI; include/cx_moe.h is).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "cx_moe.h"

namespace cx {

// ---------------------------------------------------------------------------
// Vector types for the gfx950 builtins.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Geometry of the fast grouped kernels.
constexpr int kKB = 128;        // k-block: one scale per 128 columns
constexpr int kTileRows = 16;   // MFMA 16x16x32: 16 weight rows per wave
constexpr int kTileTok = 16;    // 16 token (pair) columns per MFMA tile
constexpr int kBigPairs = 128;  // pairs per item of the LDS-ring grouped GEMM (many tokens per expert)
constexpr int kWaves = 4;       // waves per workgroup

// ---------------------------------------------------------------------------
// Grouped-execution plan, built on the device by k_plan from (topk_ids,
// topk_w) and consumed by the gate/up, down and combine kernels.
//   slot   : one active expert (ascending expert id), the shared expert last
//   pair   : one (token, expert) assignment, grouped by slot.  The shared
//            expert's pairs are [0, T) (pair t = token t), so its h can be
//            produced before the routing is known; routed pairs follow.
//   item   : a run of <= item_cap pairs of one slot (one grouped work unit);
//            routed items first, the shared expert's items last
struct PlanHdr {
    int n_slots;
    int n_items;
    int n_pairs;
    int n_routed_slots;  // slots [0, n_routed_slots) are routed experts
    int n_routed_items;  // items [0, n_routed_items) belong to routed slots
    int pad[3];
};
constexpr int kPlanHdrInts = 8;

// Gate/up weight layouts (cx_expert_desc::gu_layout).  CX_LAYOUT_TILE16
// keeps each 16-row group's k-blocks as consecutive 2 KB tiles, and inside a
// tile the 32-byte pieces in MFMA lane order (quarter q of the 128 columns,
// then row): the 32 bytes a lane (row r % 16, quarter q) loads for a k-block
// sit at tile + (16 q + r % 16) * 32, and the k-blocks of a wave are 2 KB
// apart instead of 128 bytes, so a wave's weight range is one contiguous run.
// Byte offset of row r, columns 32 q .. 32 q + 31 of k-block kb in a matrix
// of `cols` columns (cols % 128 == 0, rows % 16 == 0 for TILE16):
__host__ __device__ inline size_t gu_piece_off(int layout, int cols, int r, int kb, int q) {
    return layout == CX_LAYOUT_TILE16
               ? ((((size_t)(r >> 4) * (size_t)(cols >> 7) + (size_t)kb) << 11) + (size_t)((q << 4) + (r & 15)) * 32)
               : (size_t)r * (size_t)cols + (size_t)kb * 128 + (size_t)q * 32;
}
// Distance between consecutive k-blocks of one row.
__host__ __device__ inline int gu_kstep(int layout) { return layout == CX_LAYOUT_TILE16 ? 2048 : 128; }
// Byte offset of element (r, c).
__host__ __device__ inline size_t gu_elem_off(int layout, int cols, int r, int c) {
    return gu_piece_off(layout, cols, r, c >> 7, (c >> 5) & 3) + (size_t)(c & 31);
}
__host__ __device__ inline bool gu_tile16_ok(uint64_t rows, uint64_t cols) {
    return rows % 16 == 0 && cols % 128 == 0;
}

// Flat per-item / per-slot records written by the planner, so a workgroup
// reaches its weight pointers with one dependent load.
struct ItemRec {
    const uint8_t* w_up;
    const uint8_t* w_gate;
    const uint8_t* w_down;
    const float* s_up;     // scale grids; the kernel adds its row block
    const float* s_gate;
    const float* s_down;
    int pb, np;            // pair range
    int up_rb, gate_rb, down_rb, gu_layout;
    int tok[4];            // tokens of the item's first (up to) 4 pairs
};

struct SlotRec {
    const uint8_t* w_down;
    const float* s_down;
    int down_rb;
    int pad;
};

struct PlanPtrs {
    PlanHdr* hdr;
    ItemRec* item_rec;     // [max_items]
    SlotRec* slot_rec;     // [max_slots]
    int* slot_expert;      // [max_slots]  index into the layer table
    int* slot_pair_begin;  // [max_slots]
    int* slot_pair_count;  // [max_slots]
    int* item_slot;        // [max_items]
    int* item_pair_begin;  // [max_items]
    int* item_pair_count;  // [max_items]
    int* pair_token;       // [max_pairs]
    float* pair_weight;    // [max_pairs]
    int* token_pairs;      // [T * (K+1)], pair index or -1 (shared in column K)
    int* pair_row;         // [max_pairs] y_part row of a pair: t for the shared expert's,
                           // T + t*K + k for (token t, route k); decode plans only (nullable:
                           // row = pair)
};

// Device error bits (ORed into the context's flag, read by cx_ctx_sync).
enum : int {
    kErrBadExpertId = 1,
    kErrNotResident = 2,
    kErrPlanOverflow = 4,
    kErrDuplicateRoute = 8,
    kErrBadWeight = 16,  // negative or non-finite route weight (validate_routes, moe_layer_runtime.py:96-97)
};

// A route weight the planners accept: finite and >= 0 (validate_routes
// rejects negative weights, server/moe_layer_runtime.py:96-97; a NaN or an
// infinity cannot come out of the router and is rejected too).
__device__ __forceinline__ bool route_weight_ok(float w) {
    return w >= 0.0f && w <= 3.402823466e38f;
}

// ---------------------------------------------------------------------------
// Kernel-duration timing.  While a LaunchTimer is current on the calling
// thread, cx_launch passes its events to hipExtLaunchKernelGGL, so the start
// event takes the first kernel's start timestamp and the stop event the last
// kernel's end timestamp (dispatch timestamps, without launch gaps).
struct LaunchTimer {
    hipEvent_t start = nullptr, stop = nullptr;
    bool started = false;
};
LaunchTimer*& current_launch_timer();

template <typename F, typename... Args>
inline void cx_launch(F kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t s, Args... args) {
    LaunchTimer* t = current_launch_timer();
    if (t == nullptr) {
        kernel<<<grid, block, lds, s>>>(args...);
        return;
    }
    hipExtLaunchKernelGGL(kernel, grid, block, lds, s, t->started ? nullptr : t->start, t->stop, 0u,
                          args...);
    t->started = true;
}

// ---------------------------------------------------------------------------
// Launchers (defined in the .hip files).  All return hipError_t of the launch.

struct ExpertLaunch {
    // Either a device table + plan (grouped mode) or one descriptor by value
    // with an implicit identity plan over n_tokens tokens (single mode).
    const cx_expert_desc* table;  // grouped mode; nullptr in single mode
    cx_expert_desc single;        // single mode
    PlanPtrs plan;                // grouped mode
    int max_items;                // grid bound in grouped mode
    int n_tokens;
    int hidden, inter;
    int maxt;                     // token tiles per item: 1 (decode) or 4 (prefill)
    const void* x;                // [T, hidden] fp16/bf16
    int in_dtype;
    uint16_t* h_hi;               // [pairs, inter] bf16 hi part of h
    uint16_t* h_lo;               // [pairs, inter] bf16 lo part of h
    float* h_f32;                 // optional [pairs, inter] fp32 h (debug/parity)
    float* y_part;                // [pairs, hidden] fp32 per-pair down output (grouped)
    void* y;                      // single mode: [T, hidden] out dtype
    float* y_f32;                 // single mode / fused decode: optional fp32 output
    int out_dtype;
    int fold_weight;              // phase A multiplies h by the pair's route weight
    int np_lds;                   // >0: stage up to np_lds activation rows per item in LDS
    int skip_shared;              // grouped mode: routed items only (shared expert done apart)
    int max_lds;                  // dynamic LDS per workgroup the device allows (0: unknown)
    float* gu_part;               // k-part gate/up sums of the shared expert [kparts][2][T][inter]
                                  // (written by the split stage-2 tiles; the routed gate/up
                                  // launch finalises them into h when non-null)
    int gu_kparts;
};

hipError_t launch_gate_up(const ExpertLaunch& L, hipStream_t s);
// Grouped mode with items of up to kBigPairs (128) pairs, for calls with
// many tokens per expert (cx_big.h): gate/up writes h, down writes y_part,
// as launch_gate_up / launch_down do.  big_ok: the shapes they take.
bool big_shape_ok(int hidden, int inter, int in_dtype);
bool big_ok(const ExpertLaunch& L);
hipError_t launch_gate_up_big(const ExpertLaunch& L, hipStream_t s);
hipError_t launch_down_big(const ExpertLaunch& L, hipStream_t s);
// Down projection per work item: grouped mode writes fp32 y_part[pair]
// (combined afterwards by launch_combine), single mode writes y / y_f32.
hipError_t launch_down(const ExpertLaunch& L, hipStream_t s);
hipError_t launch_combine(const PlanPtrs& plan, const float* y_part, int n_tokens,
                          int top_k, int hidden, void* y, int out_dtype, float* y_f32,
                          hipStream_t s);
// Combine of a decode plan (y_part rows by pair_row): weights read straight
// from the routes, every load independent of the others.
hipError_t launch_combine_dec(const PlanPtrs& plan, const float* topk_w, const float* y_part,
                              int n_tokens, int top_k, int has_shared, int hidden, void* y,
                              int out_dtype, float* y_f32, hipStream_t s);
// One-token decode (n_tokens == 1, decode plan): down of every item and the
// weighted combine in one launch, writing y / y_f32 directly (no y_part).
// Needs top_k <= 8, hidden % 16 == 0, inter / 128 in {4, 8, 16} and
// down_comb1_lds(inter) bytes of LDS (L.max_lds).  Workgroups of
// down_comb1_rows(hidden, n_cu) output rows (n_cu: the device's CUs).
size_t down_comb1_lds(int inter);
bool down_comb1_ok(int hidden, int inter, int top_k, int max_lds);
int down_comb1_rows(int hidden, int n_cu);
hipError_t launch_down_comb1(const ExpertLaunch& L, const int* token_pairs, const float* topk_w,
                             int top_k, int n_cu, hipStream_t s);
hipError_t launch_plan(const int32_t* ids, const float* w, int n_tokens, int top_k,
                       const cx_expert_desc* table, int n_experts, int has_shared,
                       int item_cap, int max_items, PlanPtrs plan, int* err_flag,
                       hipStream_t s);

// One expert at 1..4 tokens (single mode): gate/up as 2 k-part sums
// (L.gu_part, L.gu_kparts = 2), then down with K split over the waves of each
// workgroup, h finalised from the part sums.
bool expert_small_ok(const ExpertLaunch& L);
hipError_t launch_gate_up_kpart(const ExpertLaunch& L, hipStream_t s);
hipError_t launch_down_ks(const ExpertLaunch& L, hipStream_t s);

// Generic (any shape, any block size) single-expert path: correctness only.
hipError_t launch_generic_expert(const cx_expert_desc& e, const void* x, int in_dtype,
                                 int n_tokens, float* h_scratch, void* y, int out_dtype,
                                 float* y_f32, hipStream_t s);

// Router (optionally followed by the planner in the same launch for T <= 16).
struct RouteArgs {
    const void* x;
    int x_dtype;
    const void* w;
    int w_dtype;
    const float* bias;
    const uint8_t* resident;
    int n_tokens, hidden, n_experts, n_group, topk_group, top_k, norm;
    float scale;
    double* logits;         // scratch [T, E]
    int32_t* ids;           // [T, top_k]
    float* wout;            // [T, top_k]
    // planner (nullable plan = route only)
    const PlanPtrs* plan;
    const cx_expert_desc* table;
    int has_shared, item_cap, max_items;
    int* err_flag;
};
hipError_t launch_route(const RouteArgs& r, hipStream_t s);
int route_max_experts();

// Decode pipeline for T <= 16 tokens, E <= 256 experts.
//  cx_moe_layer:  stage 1 = router logits;
//                 stage 2 = selection + planner beside the shared expert's
//                 gate/up (sg nullable: no shared expert).
//  cx_moe_decode: planner from given routes beside the shared expert's gate/up.
// The shared-expert launch is a single-mode ExpertLaunch record whose pairs
// are the tokens (pair t = token t, the plan's shared pairs).
bool dec_route_ok(int n_experts, int n_group);
bool dec_shared_ok(int hidden, int inter);
// The shared expert's stage-2 gate/up can run as two k-parts (T <= 8):
// ExpertLaunch::gu_part set on both the stage-2 record and the routed
// gate/up launch, which then finalises the shared h.
bool dec_shared_split_ok(int hidden, int inter, int n_tokens);
// Activation rows the shared expert's gate/up tiles of stage 2 stage in LDS
// (0: stream them from L2).
int dec_sgu_np_lds(int hidden, int n_tokens, int max_lds);
hipError_t launch_dec_logits(const RouteArgs& r, hipStream_t s);
hipError_t launch_dec_select_sgu(const RouteArgs& r, const ExpertLaunch* sg, hipStream_t s);
hipError_t launch_dec_plan_sgu(const int32_t* ids, const float* w, int n_tokens, int top_k,
                               const cx_expert_desc* table, int n_experts, int has_shared,
                               PlanPtrs plan, int* err_flag, const ExpertLaunch* sg,
                               hipStream_t s);

// One-token decode with the selection inside the routed gate/up launch (no
// resident mask, every expert of the table resident, 256 experts in 8
// groups, at most 8 picks, bf16 x, x staged in LDS): stage 1 = router
// logits and scores (sc: s [E] then c [E], fp64) beside the
// shared expert's gate/up k-parts (sg nullable; else its gu_part with 2
// k-parts); stage 2 = the routed gate/up, each workgroup selecting for
// itself, writing the routes (R.ids / R.wout) and the one-token plan for
// launch_down_comb1, and finalising the shared h (L.gu_part).
bool dec_fused_sel_ok(int n_experts, int n_group, int topk_group, int hidden, int top_k, int x_dtype);
hipError_t launch_dec_logits_sgu(const RouteArgs& r, const ExpertLaunch* sg, double* sc, hipStream_t s);
hipError_t launch_gate_up_sel(const ExpertLaunch& L, const RouteArgs& r, const double* sc, hipStream_t s);

// Upload helpers / generator.
hipError_t launch_canonicalize_fp8(uint8_t* p, uint64_t n, hipStream_t s);
// layout: where element (r, c) goes (gu_elem_off); CX_LAYOUT_TILE16 needs
// gu_tile16_ok(rows, cols).
hipError_t launch_gen_fp8(uint64_t seed, uint64_t stream_id, int rows, int cols, int rb,
                          int cb, float std_dev, uint8_t* q, float* scale, hipStream_t s,
                          int layout = CX_LAYOUT_ROWS);
// Row-major fp8 `src` -> CX_LAYOUT_TILE16 `dst` (distinct buffers), with the
// 0x7F/0xFF canonicalisation of launch_canonicalize_fp8.
hipError_t launch_tile16_fp8(const uint8_t* src, uint8_t* dst, int rows, int cols, hipStream_t s);
hipError_t launch_gen_normal(uint64_t seed, uint64_t stream_id, uint64_t count,
                             float std_dev, int dtype, void* out, hipStream_t s);

bool fast_path_ok(const cx_expert_desc& e);

}  // namespace cx
