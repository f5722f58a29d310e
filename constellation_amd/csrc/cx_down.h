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

namespace cx {

// ---------------------------------------------------------------------------
// One-token decode: down projection of every item and the weighted combine in
// one launch.  Workgroup = a tile of <= 16 output rows x all items: wave w
// streams routed item w's rows over the full K (NKB k-blocks), then its share (NKS
// k-blocks) of the shared expert's K, as one weight ring; the h rows it needs
// (routed item: all of K; shared expert: its k range) are DMA'd into the
// wave's own LDS slice first.  The output rows are then combined in LDS —
// routes in route order weighted by topk_w, the shared expert's k-range
// partials in wave order, added last — cast, and stored.  Every CU streams
// from eight experts at once, and neither y_part nor a combine launch is
// needed.  Semantics: RunDownReferenceV2 (expert_reference_v2.cc:92-144) per
// expert and combine_outputs_torch (server/moe_layer_runtime.py:148-167),
// shared expert last (full_model_runtime.py:348).
// Plan layout at T = 1 (dec_plan_core): routed item i = slot i owns pair
// s0 + i (s0 = 1 with a shared expert, whose pair is 0), token_pairs[k] =
// pair of route k or -1.
constexpr int kDc1Waves = 8;

template <int NKB>
struct Dc1Geom {
    static constexpr int NKS = NKB >= kDc1Waves ? NKB / kDc1Waves : 1;  // shared k-blocks per wave
    static constexpr int kRoutedBytes = NKB * kKB * 2;                   // one h plane of a routed item
    static constexpr int kSharedBytes = NKS * kKB * 2;                   // one plane of a shared slice
    static constexpr int kWaveBytes = 2 * kRoutedBytes + 2 * kSharedBytes;
    static constexpr int kRedOff = kDc1Waves * kWaveBytes;
    static constexpr int kLds = kRedOff + 2 * kDc1Waves * 4 * 16;      // + routed / shared row partials
};

// Scale rows of one item for a tile of output rows: rows of the tile at or
// past `split` (tile-relative) lie in the next row block.  Row blocks are
// multiples of 16 rows and tiles at most 16, so a tile spans at most two.
struct Dc1Scales {
    const float* lo;
    const float* hi;
    int split;
};

__device__ __forceinline__ Dc1Scales dc1_scales(const float* s_down, int down_rb, int r0, int rows,
                                                int nkb, int k0) {
    const int rb = __builtin_amdgcn_readfirstlane(r0 / down_rb);
    const int split = (rb + 1) * down_rb - r0;
    Dc1Scales q;
    q.lo = s_down + (size_t)rb * nkb + k0;
    q.hi = split < rows ? q.lo + nkb : q.lo;
    q.split = split;
    return q;
}

// One wave's ring: NR routed stages (item weights pd, scales qd) then NS
// shared stages (ps, qs); h of stage k read from the wave's LDS slice.  The
// lane holds output rows 4g..4g+3 of the tile; each takes its own row
// block's scale.  dma() issues the wave's h DMA after the first PRE weight
// stages (PRE = 0: before any weight load).
template <int NR, int NS, int D, int NKB, int PRE, class Dma>
__device__ __forceinline__ void dc1_ring(const uint8_t* pd, const uint8_t* ps, Dc1Scales qd,
                                         Dc1Scales qs, const unsigned char* hw, int g,
                                         f32x4* acc_r, f32x4* acc_s, Dma dma) {
    typedef Dc1Geom<NKB> G;
    constexpr int NK = NR + NS;
    constexpr int DP = D < NK ? D : NK;  // prologue stages
    constexpr int P0 = PRE < DP ? PRE : DP;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 ar = zero, as = zero;
    auto wptr = [&](int k) { return k < NR ? pd + k * kKB : ps + (k - NR) * kKB; };
    u32x4 wb[D][2];
#pragma unroll
    for (int s = 0; s < P0; ++s) {
        wb[s][0] = ld16(wptr(s));
        wb[s][1] = ld16(wptr(s) + 16);
    }
    __builtin_amdgcn_sched_barrier(0);
    dma();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = P0; s < DP; ++s) {
        wb[s][0] = ld16(wptr(s));
        wb[s][1] = ld16(wptr(s) + 16);
    }
    __builtin_amdgcn_sched_barrier(0);
    float sc[NK], sc_hi[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) {
        sc[k] = k < NR ? ldsc(qd.lo + k) : ldsc(qs.lo + (k - NR));
        sc_hi[k] = k < NR ? ldsc(qd.hi + k) : ldsc(qs.hi + (k - NR));
    }
    bool hi_r[4], hi_s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        hi_r[i] = 4 * g + i >= qd.split;
        hi_s[i] = 4 * g + i >= qs.split;
    }
    // the DMA'd h (and the first P0 stages) are older than the remaining
    // prologue loads; nothing of the loop may move above this wait (the
    // compiler cannot count LDS DMA exactly and would drain the ring with
    // vmcnt(0))
    vm_wait<2 * (DP - P0)>();
    lds_dma_barrier();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < NK; ++k) {
        const int s = k % D;
        const unsigned char* hp = k < NR ? hw + k * (kKB * 2) + g * 64
                                         : hw + 2 * G::kRoutedBytes + (k - NR) * (kKB * 2) + g * 64;
        const int lo = k < NR ? G::kRoutedBytes : G::kSharedBytes;
        u32x4 hb[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            hb[j] = *reinterpret_cast<const u32x4*>(hp + 16 * j);
            hb[4 + j] = *reinterpret_cast<const u32x4*>(hp + lo + 16 * j);
        }
        const f32x4 t = down_step(wb[s], hb);
        f32x4 sv;
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = (k < NR ? hi_r[i] : hi_s[i]) ? sc_hi[k] : sc[k];
        if (k < NR) ar += sv * t;
        else as += sv * t;
        __builtin_amdgcn_sched_barrier(0);
        if (k + D < NK) {
            wb[s][0] = ld16(wptr(k + D));
            wb[s][1] = ld16(wptr(k + D) + 16);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    *acc_r = ar;
    *acc_s = as;
}

// Row tile `rtile` of `rows` (<= 16) output rows.  The plan header and the
// wave's item record come first, then the h DMA and the ring.  Wave 0
// fetches the route table with the DMA, so the combine needs no memory
// round trip.  With rows < 16, the MFMA's spare rows repeat the tile's last
// weight row (the same addresses, so no extra bytes) and are not stored.
template <int NKB, int D, int PRE = 0>
__device__ __forceinline__ void down_comb1_tile(const ExpertLaunch& L, const int* token_pairs,
                                                const float* topk_w, int top_k, unsigned char* lds,
                                                int rtile, int rows) {
    typedef Dc1Geom<NKB> G;
    constexpr int NKS = G::NKS;
    const int I = L.inter;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const int r0 = rtile * rows;
    const int wr = r0 + min(c, rows - 1);  // weight row of this lane
    const PlanHdr hd = ld_uniform(L.plan.hdr);
    const int ts = hd.n_routed_items;
    const bool shared = hd.n_items > ts;
    const bool has_r = wave < ts;
    const bool has_s = shared && wave * NKS < NKB;
    unsigned char* hw = lds + wave * G::kWaveBytes;
    const uint8_t* pd = nullptr;
    const uint8_t* ps = nullptr;
    Dc1Scales qd{nullptr, nullptr, kTileRows}, qs{nullptr, nullptr, kTileRows};
    // 0) h into this wave's LDS slice (1 KB per wave instruction), issued by
    //    the ring after its first PRE weight stages
    const uint16_t *hh = nullptr, *hl = nullptr, *hs = nullptr;
    constexpr int LPP = G::kSharedBytes / 16;  // lanes per shared plane
    if (has_r) {
        const ItemRec ri = ld_uniform(L.plan.item_rec + wave);
        hh = L.h_hi + (size_t)ri.pb * I + lane * 8;
        hl = L.h_lo + (size_t)ri.pb * I + lane * 8;
        pd = ri.w_down + (size_t)wr * I + g * 32;
        qd = dc1_scales(ri.s_down, ri.down_rb, r0, rows, I / kKB, 0);
    }
    if (has_s) {
        const ItemRec rs = ld_uniform(L.plan.item_rec + ts);
        const size_t k0 = (size_t)wave * NKS * kKB;
        hs = (lane < LPP ? L.h_hi : L.h_lo) + (size_t)rs.pb * I + k0 + (lane % LPP) * 8;
        ps = rs.w_down + (size_t)wr * I + k0 + g * 32;
        qs = dc1_scales(rs.s_down, rs.down_rb, r0, rows, I / kKB, wave * NKS);
    }
    auto dma = [&] {
        if (has_r) {
#pragma unroll
            for (int j = 0; j < G::kRoutedBytes / 1024; ++j) {
                __builtin_amdgcn_global_load_lds(hh + j * 512, hw + j * 1024, 16, 0, 0);
                __builtin_amdgcn_global_load_lds(hl + j * 512, hw + G::kRoutedBytes + j * 1024, 16, 0, 0);
            }
        }
        if (has_s && lane < 2 * LPP) __builtin_amdgcn_global_load_lds(hs, hw + 2 * G::kRoutedBytes, 16, 0, 0);
    };
    // wave 0: the route table (lane k: pair and weight of route k), issued
    // with the DMA so that the ring's first wait covers it
    int tpl = -1;
    float twl = 0.f;
    if (wave == 0 && lane <= top_k) {
        tpl = token_pairs[lane];
        if (lane < top_k) twl = topk_w[lane];
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x4 ar, as;
    if (has_r && has_s) dc1_ring<NKB, NKS, D, NKB, PRE>(pd, ps, qd, qs, hw, g, &ar, &as, dma);
    else if (has_r) dc1_ring<NKB, 0, D, NKB, PRE>(pd, ps, qd, qs, hw, g, &ar, &as, dma);
    else if (has_s) dc1_ring<0, NKS, D, NKB, PRE>(pd, ps, qd, qs, hw, g, &ar, &as, dma);
    else {
        lds_dma_barrier();
        ar = as = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // 1) column 0 (the token) of each wave's tiles: rows 4g..4g+3 on lane 16g
    f32x4* red_r = reinterpret_cast<f32x4*>(lds + G::kRedOff);
    f32x4* red_s = red_r + kDc1Waves * 4;
    if (c == 0) {
        red_r[wave * 4 + g] = ar;
        red_s[wave * 4 + g] = as;
    }
    __syncthreads();
    if (wave == 0) {
        const int s0 = shared ? 1 : 0;
        f32x4 sum = {0.f, 0.f, 0.f, 0.f};
        for (int k = 0; k < top_k; ++k) {
            const int p = __shfl(tpl, k);
            const float wk = __shfl(twl, k);
            if (p >= s0) sum += wk * red_r[(p - s0) * 4 + (lane & 3)];
        }
        if (shared && __shfl(tpl, top_k) >= 0) {
#pragma unroll
            for (int w = 0; w < kDc1Waves; ++w) sum += red_s[w * 4 + (lane & 3)];
        }
        if (lane < 4 && 4 * lane < rows) {
            if (rows % 4 == 0) store_out4(L.y, L.y_f32, (size_t)r0 + 4 * lane, sum, L.out_dtype);
            else store_out_n(L.y, L.y_f32, (size_t)r0 + 4 * lane, sum, min(4, rows - 4 * lane), L.out_dtype);
        }
    }
}

}  // namespace cx
