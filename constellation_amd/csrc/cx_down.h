// cx_down.h — the down projection of one work item of the grouped fp8
// expert MLP (<= 16 pairs), as a device function: per-pair fp32 output,
// combined afterwards in a fixed order.
// Semantics: RunDownReferenceV2 (expert_node_v2/backend/expert_reference_v2.cc:
// 92-144) per expert, combine_outputs_torch (server/moe_layer_runtime.py:
// 148-167) across experts, shared expert added last (full_model_runtime.py:348).
//
// h enters the MFMA as its bf16 hi/lo split (two MFMAs per step).  The B
// operand is read with raw buffer loads: a column whose token does not use
// the slot gets an out-of-range offset and reads zero without any memory
// traffic, so at one token per expert only 4 of 64 lanes fetch h.
#pragma once

#include "cx_gate_up.h"

namespace cx {

// One 16-column MFMA step of the down projection: A = 16 weight rows x 128 k
// (two dwordx4 per lane), B = h hi / lo (4 dwordx4 each).
__device__ __forceinline__ f32x4 down_step(const u32x4 w[2], const u32x4 hb[8]) {
    typedef Mma<false> M;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 t = M::mma(M::cvt(w[0][0], w[0][1]), M::bits(hb[0]), zero);
    t = M::mma(M::cvt(w[0][0], w[0][1]), M::bits(hb[4]), t);
    t = M::mma(M::cvt(w[0][2], w[0][3]), M::bits(hb[1]), t);
    t = M::mma(M::cvt(w[0][2], w[0][3]), M::bits(hb[5]), t);
    t = M::mma(M::cvt(w[1][0], w[1][1]), M::bits(hb[2]), t);
    t = M::mma(M::cvt(w[1][0], w[1][1]), M::bits(hb[6]), t);
    t = M::mma(M::cvt(w[1][2], w[1][3]), M::bits(hb[3]), t);
    t = M::mma(M::cvt(w[1][2], w[1][3]), M::bits(hb[7]), t);
    return t;
}

__device__ __forceinline__ void load_h8g(const uint16_t* hi, const uint16_t* lo, u32x4 hb[8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        hb[j] = ld16(hi + 8 * j);
        hb[4 + j] = ld16(lo + 8 * j);
    }
}

// Down projection of one work item (one expert, <= 16 pairs): workgroup =
// 4 waves x 16 rows = 64 output rows (`tile`), each wave streams its rows
// over the full K with a D-deep weight ring.  Output: fp32 per pair into
// y_part[pair][hidden] (the weighted combine runs after, k_combine), or the
// final output in single mode (pair = token).
// h of the item's pairs is never loaded from L2 inside the loop behind older
// weight loads (vmcnt completes in order, so such a load would collapse the
// ring to one step):
//  * XL (np <= 4): the rows go to LDS by direct global->LDS DMA before the
//    weight prologue; the loop issues weight loads only;
//  * otherwise (more pairs) h is loaded one step ahead in the order that
//    keeps its wait independent of younger weight loads (2-deep ring).
constexpr int kDownRowsPerWG = kTileRows * kWaves;  // 64
constexpr int kDownLdsRows = 4;

template <int NKB, int D, bool SINGLE, bool XL>
__device__ __forceinline__ void down_item_path(const ExpertLaunch& L, const Unit& u, int tile);

// Per item: h staged in LDS (D-deep weight ring) when the item has <= 4
// pairs, else h rides a 2-deep ring; both in one launch (uniform branch).
template <int NKB, int D, bool SINGLE>
__device__ __forceinline__ void down_item_tile(const ExpertLaunch& L, int tile, int item) {
    Unit u;
    if (!resolve_unit<SINGLE>(L, item, kTileTok, &u)) return;
    if (u.np <= kDownLdsRows) down_item_path<NKB, D, SINGLE, true>(L, u, tile);
    else down_item_path<NKB, 2, SINGLE, false>(L, u, tile);
}

template <int NKB, int D, bool SINGLE, bool XL>
__device__ __forceinline__ void down_item_path(const ExpertLaunch& L, const Unit& u, int tile) {
    const int H = u.e.hidden, I = u.e.inter;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const int rw = tile * kDownRowsPerWG + wave * kTileRows;
    const uint8_t* pd = u.e.w_down + (size_t)(rw + c) * I + g * 32;
    const int rbd = __builtin_amdgcn_readfirstlane(rw / u.e.down_rb);
    const float* sd = u.e.s_down + (size_t)rbd * (I / kKB);
    extern __shared__ __attribute__((aligned(16))) unsigned char hlds[];
    const size_t hs = (size_t)I * 2 + 16;  // LDS row stride (bytes) of one h plane
    const size_t hrow = (size_t)min(c, u.np - 1);
    // 0) XL: h rows -> LDS (hi rows then lo rows), 1 KB per wave instruction
    if (XL) {
        const int cpr = I / 512;
        const int nwc = 2 * u.np * cpr;
        for (int wc = wave; wc < nwc; wc += kWaves) {
            const int r = wc / cpr, j0 = (wc - r * cpr) * 64;  // r = plane * np + q
            const int plane = r >= u.np ? 1 : 0, q = r - plane * u.np;
            const uint16_t* src = (plane ? L.h_lo : L.h_hi) + (size_t)(u.pb + q) * I + (size_t)(j0 + lane) * 8;
            __builtin_amdgcn_global_load_lds(src, hlds + ((size_t)plane * kDownLdsRows + q) * hs + j0 * 16, 16, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // y_part row of this lane's pair (decode plans index rows by route)
    const int prow = SINGLE || L.plan.pair_row == nullptr ? u.pb + c
                                                          : L.plan.pair_row[u.pb + min(c, u.np - 1)];
    const uint16_t* gh = L.h_hi + (size_t)(u.pb + hrow) * I + g * 32;
    const uint16_t* gl = L.h_lo + (size_t)(u.pb + hrow) * I + g * 32;
    // 1) ring prologue.  Without XL, h is loaded one step ahead, issued
    //    after the weights of that step and before the weights D steps
    //    ahead, so waiting for it never waits for younger weight loads.
    u32x4 wb[D][2];
    u32x4 hr[8];
#pragma unroll
    for (int s = 0; s < D && s < NKB; ++s) {
        wb[s][0] = ld16(pd + s * kKB);
        wb[s][1] = ld16(pd + s * kKB + 16);
        if (!XL && s == 0) load_h8g(gh, gl, hr);
    }
    __builtin_amdgcn_sched_barrier(0);
    float scd[NKB];
#pragma unroll
    for (int k = 0; k < NKB; ++k) scd[k] = ldsc(sd + k);
    const unsigned char* lh = hlds + hrow * hs + g * 64;
    const unsigned char* ll = hlds + (kDownLdsRows + hrow) * hs + g * 64;
    if (XL) {
        vm_wait<2 * (D < NKB ? D : NKB)>();
        lds_dma_barrier();
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < NKB; ++k) {
        const int s = k % D;
        if (XL) {
            u32x4 hb[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                hb[j] = *reinterpret_cast<const u32x4*>(lh + k * (kKB * 2) + 16 * j);
                hb[4 + j] = *reinterpret_cast<const u32x4*>(ll + k * (kKB * 2) + 16 * j);
            }
            acc += scd[k] * down_step(wb[s], hb);
        } else {
            acc += scd[k] * down_step(wb[s], hr);
        }
        // one k-block's product tile live at a time
        __builtin_amdgcn_sched_barrier(0);
        if (!XL && k + 1 < NKB) load_h8g(gh + (k + 1) * kKB, gl + (k + 1) * kKB, hr);
        if (k + D < NKB) {
            wb[s][0] = ld16(pd + (k + D) * kKB);
            wb[s][1] = ld16(pd + (k + D) * kKB + 16);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if (c < u.np) {
        const size_t p = (size_t)prow;
        if (SINGLE)  // pair = token: final output
            store_out4(L.y, L.y_f32, p * H + rw + 4 * g, acc, L.out_dtype);
        else
            *reinterpret_cast<float4*>(L.y_part + p * H + rw + 4 * g) = float4{acc[0], acc[1], acc[2], acc[3]};
    }
}

inline size_t down_item_lds(int inter) { return (size_t)2 * kDownLdsRows * ((size_t)inter * 2 + 16); }

}  // namespace cx
