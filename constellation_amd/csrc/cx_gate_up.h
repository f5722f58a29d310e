// cx_gate_up.h — the gate/up (phase A) tile of the grouped fp8 expert MLP,
// as a device function so that both the stand-alone gate/up kernel and the
// decode kernels that overlap the shared expert with the router can run it.
//
// One workgroup tile = TR (16, or 8 to spread a small grid over more CUs)
// rows of gate and up of one expert for all pairs of one work item
// (<= 16*MAXT), K split over the KS waves; the partial tiles
// are summed in LDS in a fixed order and the SiLU(gate)*up epilogue writes h
// as a bf16 hi/lo split (h = hi + lo to 2^-17 relative).
// Semantics: RunFusedUpGateReferenceV2 (expert_node_v2/backend/
// expert_reference_v2.cc:11-90): dequantise-then-fp32 dot products.
#pragma once

#include "cx_device.h"

namespace cx {

// Resolves the work unit of a workgroup.  Returns false if the unit has no
// work (grids are sized for the worst case).
struct Unit {
    cx_expert_desc e;
    int pb;      // first pair
    int np;      // pairs in this unit
    int tok[4];  // tokens of the first (up to) 4 pairs
};

// SINGLE: one descriptor by value with pairs = tokens (no plan); otherwise
// the plan's item record.  A compile-time choice, so every field of the unit
// stays in SGPRs (a run-time choice merges the two sources into flat loads).
template <bool SINGLE>
__device__ __forceinline__ bool resolve_unit(const ExpertLaunch& L, int item, int unit_cap, Unit* u) {
    if (!SINGLE) {
        const PlanHdr hd = ld_uniform(L.plan.hdr);
        const int n_items = L.skip_shared ? hd.n_routed_items : hd.n_items;
        if (item >= n_items) return false;
        const ItemRec r = ld_uniform(L.plan.item_rec + item);
        u->pb = r.pb;
        u->np = r.np;
        u->e.w_up = r.w_up;
        u->e.w_gate = r.w_gate;
        u->e.w_down = r.w_down;
        u->e.s_up = r.s_up;
        u->e.s_gate = r.s_gate;
        u->e.s_down = r.s_down;
        u->e.hidden = L.hidden;
        u->e.inter = L.inter;
        u->e.up_rb = r.up_rb;
        u->e.gate_rb = r.gate_rb;
        u->e.down_rb = r.down_rb;
        u->e.up_cb = u->e.gate_cb = u->e.down_cb = kKB;  // grouped layers are 128-column blocks
        u->e.gu_layout = r.gu_layout;
#pragma unroll
        for (int q = 0; q < 4; ++q) u->tok[q] = r.tok[q];
    } else {
        u->pb = item * unit_cap;
        if (u->pb >= L.n_tokens) return false;
        u->np = min(unit_cap, L.n_tokens - u->pb);
        u->e = L.single;
#pragma unroll
        for (int q = 0; q < 4; ++q) u->tok[q] = u->pb + q;
    }
    return u->np > 0;
}

// Run-time form for the generic kernels.
__device__ __forceinline__ bool resolve_unit_rt(const ExpertLaunch& L, int item, int unit_cap, Unit* u) {
    return L.table != nullptr ? resolve_unit<false>(L, item, unit_cap, u)
                              : resolve_unit<true>(L, item, unit_cap, u);
}

__device__ __forceinline__ int pair_token(const ExpertLaunch& L, int p) {
    return L.table != nullptr ? L.plan.pair_token[p] : p;
}

// Phase A with a compile-time trip count (the fast path at DeepSeek shapes).
// NKB = k-blocks per wave (K split over the KS waves of the workgroup), D =
// k-blocks of weights in flight per wave; every loop is unrolled with
// constant bounds, so the compiler keeps D stages of loads outstanding
// (exact vmcnt waits) instead of draining the memory pipe every stage.
// XLDS: the item's activation rows are staged once in LDS (np <= np_lds
// rows, row stride hidden*2+16 bytes so the 16 token rows fall on different
// banks); otherwise they ride the same prefetch ring from global memory.
// The wave index is made uniform (wave_id), so the per-k-block scales of the
// tile are scalar loads held in SGPRs.
// Requires col blocks of 128 and row blocks multiple of 16 (fast_path_ok).
// LDS (dynamic, from `lds`): the cross-wave reduction tile, then the staged
// activation rows (gate_up_lds_bytes).  KSA <= KS waves do the work; the
// others (when a launch's block is wider than the K split) only join the
// barriers and the DMA.
constexpr size_t gate_up_red_bytes(int ksa, int maxt) { return (size_t)ksa * maxt * 2 * 64 * 16; }

inline size_t gate_up_lds_bytes(int ksa, int maxt, int np_lds, int hidden) {
    return gate_up_red_bytes(ksa, maxt) + (maxt == 1 ? (size_t)np_lds * ((size_t)hidden * 2 + 16) : 0);
}

// PARTIAL (single mode): the tile covers k-part `kpart` of the row (KSA * NKB
// k-blocks starting at kpart * KSA * NKB) and writes its fp32 gate and up
// sums to L.gu_part[kpart][gate, up][token][row] instead of h; the parts are
// summed in order and SiLU'd later (shared_h_finalize), so a small grid can
// spread one expert's rows over twice the CUs.
// gate_up_tile_unit: the tile of a work unit the caller has resolved (u.np
// > 0); gate_up_tile resolves it from the launch first.
// GL: the weights' layout (gu_layout), a compile-time choice per instance so
// that each keeps constant k-block strides.
template <int NKB, int D, int MAXT, bool F16, bool XLDS, int KS, bool SINGLE, int KSA, int TR,
          bool PARTIAL, int GL>
__device__ __forceinline__ void gate_up_tile_body(const ExpertLaunch& L, int tile, const Unit& u,
                                                  unsigned char* lds, int kpart) {
    static_assert(!PARTIAL || (SINGLE && MAXT == 1), "k-part sums: single mode, <= 16 tokens");
    typedef Mma<F16> M;
    typedef typename M::V V;
    f32x4* red = reinterpret_cast<f32x4*>(lds);  // [KSA][MAXT][2][64]
    unsigned char* xlds = lds + gate_up_red_bytes(KSA, MAXT);
    const int H = u.e.hidden, I = u.e.inter;
    static_assert(TR == 16 || TR == 8, "tile rows");
    const int r0 = tile * TR;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const bool active = KSA == KS || wave < KSA;  // wave-uniform
    const int kb0 = ((PARTIAL ? kpart * KSA : 0) + (active ? wave : 0)) * NKB;

    // TR = 8: lanes c and c + 8 read the same row (one fetch per wave
    // instruction); MFMA rows 8..15 are discarded
    constexpr int KW = GL == CX_LAYOUT_TILE16 ? 2048 : kKB;  // weight bytes between k-blocks
    const size_t roff = gu_piece_off(GL, H, r0 + (c & (TR - 1)), kb0, g);
    const uint8_t* pg = u.e.w_gate + roff;
    const uint8_t* pu = u.e.w_up + roff;
    // integer division runs on the VALU: pin the (uniform) results to SGPRs
    // so the scale addresses stay scalar
    const int rbg = __builtin_amdgcn_readfirstlane(r0 / u.e.gate_rb);
    const int rbu = __builtin_amdgcn_readfirstlane(r0 / u.e.up_rb);
    const float* sg = u.e.s_gate + (size_t)rbg * (H / kKB) + kb0;
    const float* su = u.e.s_up + (size_t)rbu * (H / kKB) + kb0;
    const int ntile = (u.np + kTileTok - 1) / kTileTok;
    const size_t xs = (size_t)H * 2 + 16;  // LDS row stride in bytes
    constexpr bool XRING = !XLDS && MAXT == 1;

    // 0) activations.  XLDS: the np rows go to LDS by direct global->LDS
    //    DMA (global_load_lds_dwordx4: 1 KB per wave instruction, no VGPRs),
    //    issued before the weights so that waiting for them leaves the
    //    weight ring in flight.  Otherwise each lane's column token is
    //    resolved now, for the same reason.
    const unsigned char* xl = nullptr;
    const uint16_t* xp[MAXT];
    if (XLDS) {
        const int cpr = H / 512;  // 1 KB wave chunks per row (hidden % 512 == 0)
        const int nwc = u.np * cpr;
        for (int wc = wave; wc < nwc; wc += KS) {
            const int q = wc / cpr, j0 = (wc - q * cpr) * 64;
            const int tok = SINGLE ? u.pb + q : q == 0 ? u.tok[0] : q == 1 ? u.tok[1] : q == 2 ? u.tok[2] : u.tok[3];
            const uint16_t* src = static_cast<const uint16_t*>(L.x) + (size_t)tok * H + (size_t)(j0 + lane) * 8;
            __builtin_amdgcn_global_load_lds(src, xlds + q * xs + j0 * 16, 16, 0, 0);
        }
        // keep the DMA ahead of the weight loads: the wait below counts on it
        __builtin_amdgcn_sched_barrier(0);
        xl = xlds + min(c, u.np - 1) * xs + ((size_t)kb0 * kKB + g * 32) * 2;
    } else {
#pragma unroll
        for (int tt = 0; tt < MAXT; ++tt) {
            const int q = min(tt * kTileTok + c, u.np - 1);
            xp[tt] = static_cast<const uint16_t*>(L.x) + (size_t)(SINGLE ? u.pb + q : L.plan.pair_token[u.pb + q]) * H +
                     (size_t)kb0 * kKB + g * 32;
        }
    }

    f32x4 accg[MAXT], accu[MAXT];
#pragma unroll
    for (int tt = 0; tt < MAXT; ++tt) {
        accg[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
        accu[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (!active) {  // only the DMA and the barriers
        if (XLDS) {
            vm_wait<0>();
            lds_dma_barrier();
        }
    } else {
    // 1) weight prologue: HBM latency is the long pole
    u32x4 wb[D][4];
#pragma unroll
    for (int s = 0; s < D && s < NKB; ++s) {
        wb[s][0] = ld16(pg + s * KW);
        wb[s][1] = ld16(pg + s * KW + 16);
        wb[s][2] = ld16(pu + s * KW);
        wb[s][3] = ld16(pu + s * KW + 16);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2) scales (scalar loads)
    float scg[NKB], scu[NKB];
#pragma unroll
    for (int k = 0; k < NKB; ++k) {
        scg[k] = ldsc(sg + k);
        scu[k] = ldsc(su + k);
    }
    u32x4 xb[XRING ? D : 1][4];
    if (XRING) {
#pragma unroll
        for (int s = 0; s < D && s < NKB; ++s) {
#pragma unroll
            for (int j = 0; j < 4; ++j) xb[s][j] = ld16(xp[0] + s * kKB + 8 * j);
        }
    }
    if (XLDS) {
        // the DMA'd rows are older than the D*4 weight loads in flight
        vm_wait<(D < NKB ? D : NKB) * 4>();
        lds_dma_barrier();
    }

    __builtin_amdgcn_sched_barrier(0);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < NKB; ++k) {
        const int s = k % D;
#pragma unroll
        for (int tt = 0; tt < MAXT; ++tt) {
            if (MAXT == 1 || tt < ntile) {
                V bx[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (XLDS) bx[j] = M::bits(*reinterpret_cast<const u32x4*>(xl + (k * kKB + 8 * j) * 2));
                    else if (XRING) bx[j] = M::bits(xb[s][j]);
                    else bx[j] = M::bits(ld16(xp[tt] + k * kKB + 8 * j));
                }
                // gate then up: only one converted operand set live at a time
                f32x4 tg = M::mma(M::cvt(wb[s][0][0], wb[s][0][1]), bx[0], zero);
                tg = M::mma(M::cvt(wb[s][0][2], wb[s][0][3]), bx[1], tg);
                tg = M::mma(M::cvt(wb[s][1][0], wb[s][1][1]), bx[2], tg);
                tg = M::mma(M::cvt(wb[s][1][2], wb[s][1][3]), bx[3], tg);
                f32x4 tu = M::mma(M::cvt(wb[s][2][0], wb[s][2][1]), bx[0], zero);
                tu = M::mma(M::cvt(wb[s][2][2], wb[s][2][3]), bx[1], tu);
                tu = M::mma(M::cvt(wb[s][3][0], wb[s][3][1]), bx[2], tu);
                tu = M::mma(M::cvt(wb[s][3][2], wb[s][3][3]), bx[3], tu);
                accg[tt] += scg[k] * tg;
                accu[tt] += scu[k] * tu;
            }
        }
        if (k + D < NKB) {
            // refill this stage right after its last use, D stages ahead
            __builtin_amdgcn_sched_barrier(0);
            const int kn = k + D;
            wb[s][0] = ld16(pg + kn * KW);
            wb[s][1] = ld16(pg + kn * KW + 16);
            wb[s][2] = ld16(pu + kn * KW);
            wb[s][3] = ld16(pu + kn * KW + 16);
            if (XRING) {
#pragma unroll
                for (int j = 0; j < 4; ++j) xb[s][j] = ld16(xp[0] + kn * kKB + 8 * j);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int tt = 0; tt < MAXT; ++tt) {
        red[((wave * MAXT + tt) * 2 + 0) * 64 + lane] = accg[tt];
        red[((wave * MAXT + tt) * 2 + 1) * 64 + lane] = accu[tt];
    }
    }  // active

    __syncthreads();
    for (int tt = wave; tt < ntile; tt += KS) {
        f32x4 G = red[(tt * 2 + 0) * 64 + lane], U = red[(tt * 2 + 1) * 64 + lane];
#pragma unroll
        for (int w = 1; w < KSA; ++w) {
            G += red[((w * MAXT + tt) * 2 + 0) * 64 + lane];
            U += red[((w * MAXT + tt) * 2 + 1) * 64 + lane];
        }
        const int q = tt * kTileTok + c;
        if (PARTIAL) {
            if (q < u.np && 4 * g < TR) {
                const size_t p = (size_t)(u.pb + q), T = (size_t)L.n_tokens;
                const int row = r0 + 4 * g;
                *reinterpret_cast<float4*>(L.gu_part + (((size_t)kpart * 2 + 0) * T + p) * I + row) =
                    float4{G[0], G[1], G[2], G[3]};
                *reinterpret_cast<float4*>(L.gu_part + (((size_t)kpart * 2 + 1) * T + p) * I + row) =
                    float4{U[0], U[1], U[2], U[3]};
            }
            continue;
        }
        if (q < u.np && 4 * g < TR) {
            const size_t p = (size_t)(u.pb + q);
            const float wf = !SINGLE && L.fold_weight ? L.plan.pair_weight[p] : 1.0f;
            const int row = r0 + 4 * g;
            uint32_t hi[4], lo[4];
            float hv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float gate = G[i], up = U[i];
                const float h = (gate / (1.0f + expf(-gate))) * up;
                hv[i] = h;
                const float hw = h * wf;
                hi[i] = bf16_rne(hw);
                lo[i] = bf16_rne(hw - __uint_as_float(hi[i] << 16));
            }
            *reinterpret_cast<uint2*>(L.h_hi + p * I + row) =
                uint2{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
            *reinterpret_cast<uint2*>(L.h_lo + p * I + row) =
                uint2{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
            if (L.h_f32 != nullptr)
                *reinterpret_cast<float4*>(L.h_f32 + p * I + row) = float4{hv[0], hv[1], hv[2], hv[3]};
        }
    }
}

template <int NKB, int D, int MAXT, bool F16, bool XLDS, int KS, bool SINGLE, int KSA = KS,
          int TR = kTileRows, bool PARTIAL = false>
__device__ __forceinline__ void gate_up_tile_unit(const ExpertLaunch& L, int tile, const Unit& u,
                                                  unsigned char* lds, int kpart = 0) {
    if (u.e.gu_layout == CX_LAYOUT_TILE16)
        gate_up_tile_body<NKB, D, MAXT, F16, XLDS, KS, SINGLE, KSA, TR, PARTIAL, CX_LAYOUT_TILE16>(L, tile, u, lds, kpart);
    else
        gate_up_tile_body<NKB, D, MAXT, F16, XLDS, KS, SINGLE, KSA, TR, PARTIAL, CX_LAYOUT_ROWS>(L, tile, u, lds, kpart);
}

template <int NKB, int D, int MAXT, bool F16, bool XLDS, int KS, bool SINGLE, int KSA = KS,
          int TR = kTileRows, bool PARTIAL = false>
__device__ __forceinline__ void gate_up_tile(const ExpertLaunch& L, int tile, int item,
                                             unsigned char* lds, int kpart = 0) {
    Unit u;
    if (!resolve_unit<SINGLE>(L, item, kTileTok * MAXT, &u)) return;
    gate_up_tile_unit<NKB, D, MAXT, F16, XLDS, KS, SINGLE, KSA, TR, PARTIAL>(L, tile, u, lds, kpart);
}


// h of the single-mode expert whose gate/up ran as k-part sums (PARTIAL):
// rows [16*tile, 16*tile + 16) of every token, parts summed in order 0, 1, ...
// One thread per (token, row); pairs are the tokens [0, n_tokens).
__device__ __forceinline__ void shared_h_finalize(const ExpertLaunch& L, int tile) {
    const int I = L.inter, T = L.n_tokens;
    for (int cell = threadIdx.x; cell < kTileRows * T; cell += blockDim.x) {
        const int t = cell / kTileRows, row = tile * kTileRows + cell % kTileRows;
        float gate = 0.f, up = 0.f;
        for (int kp = 0; kp < L.gu_kparts; ++kp) {
            gate += L.gu_part[(((size_t)kp * 2 + 0) * T + t) * I + row];
            up += L.gu_part[(((size_t)kp * 2 + 1) * T + t) * I + row];
        }
        const float h = (gate / (1.0f + expf(-gate))) * up;
        const uint32_t hi = bf16_rne(h);
        L.h_hi[(size_t)t * I + row] = static_cast<uint16_t>(hi);
        L.h_lo[(size_t)t * I + row] = static_cast<uint16_t>(bf16_rne(h - __uint_as_float(hi << 16)));
    }
}

}  // namespace cx
