// cx_expert.hip — grouped fp8 block-scaled expert MLP for gfx950.
//
// Computes, for every (token, expert) pair of a plan,
//   h = silu(Wg . x) * (Wu . x)          (fp32, k-block scales applied in fp32)
//   y_pair = Wd . h                       (fp32)
// and combines y[t] = sum_k w_k * y_pair(t,k) + y_pair(t, shared).
// Semantics: RunFusedUpGateReferenceV2 / RunDownReferenceV2
// (expert_node_v2/backend/expert_reference_v2.cc:11-144) and the fp32 combine
// of combine_outputs_torch (server/moe_layer_runtime.py:148-167).
//
// Design (MI355X-first, not a translation of the CUDA matvecs):
//  * The fp8 weights are streamed once per launch in their uploaded row-major
//    layout with dwordx4 loads (each lane reads 32 contiguous bytes of one row
//    per 128-column k-block; 16 lanes x 4 groups cover a 16x128 tile = 2 KB).
//  * They are converted in registers to bf16 (or fp16 when the activations
//    are fp16) by the gfx950 converter v_cvt_scalef32_pk_{bf16,f16}_fp8 —
//    exact, e4m3 fits both — and fed to v_mfma_f32_16x16x32_{bf16,f16} with
//    the tokens of one expert as the 16 MFMA columns.  Even at one token per
//    expert the matrix cores do the multiply-adds, leaving the VALU only the
//    conversion (0.5 op per weight byte) and the per-k-block scale FMA.
//  * The 128x128 block scale is uniform over a 16-row x 128-column MFMA tile,
//    so each k-block's 4 MFMAs accumulate into a fresh fp32 tile that is then
//    scaled and added to the running fp32 accumulator: dequantise-then-fp32
//    exactly, products of exact bf16/fp16 values accumulated in fp32.
//  * h stays fp32; the down projection consumes it as a two-term bf16 split
//    (h = hi + lo, |h - hi - lo| <= 2^-17 |h|) with two MFMAs per step.
//  * The k order inside a k-block is permuted identically for the weight
//    (A) and activation (B) operands, so any lane->k assignment of the MFMA
//    is valid; loads stay contiguous.

#include "cx_down.h"
#include "cx_gate_up.h"
#include "cx_grouped.h"
#include "cx_big.h"

namespace cx {
namespace {

// ---------------------------------------------------------------------------
// Phase A: gate/up.  Workgroup = 16 rows of gate and up of one expert, all
// pairs of one work item (<= 16*MAXT), K split over the 4 waves; the four
// partial tiles are summed in LDS in a fixed order.
// grid = (inter/16, max_items), block = 256.
template <int MAXT, bool F16>
__global__ __launch_bounds__(256) void k_gate_up_rt(ExpertLaunch L) {
    typedef Mma<F16> M;
    typedef typename M::V V;
    Unit u;
    if (!resolve_unit_rt(L, blockIdx.y, kTileTok * MAXT, &u)) return;
    const int H = u.e.hidden, I = u.e.inter;
    const int r0 = blockIdx.x * kTileRows;
    if (r0 >= I) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const int nkb = H / kKB;
    const int kb0 = (wave * nkb) / kWaves, kb1 = ((wave + 1) * nkb) / kWaves;

    const int gl = __builtin_amdgcn_readfirstlane(u.e.gu_layout);
    const size_t roff = gu_piece_off(gl, H, r0 + c, 0, g);
    const size_t kw = gu_kstep(gl);  // weight bytes between k-blocks
    const uint8_t* pg = u.e.w_gate + roff;
    const uint8_t* pu = u.e.w_up + roff;
    const float* sg = u.e.s_gate + (size_t)(r0 / u.e.gate_rb) * ((H + u.e.gate_cb - 1) / u.e.gate_cb);
    const float* su = u.e.s_up + (size_t)(r0 / u.e.up_rb) * ((H + u.e.up_cb - 1) / u.e.up_cb);
    const int kpg = u.e.gate_cb / kKB, kpu = u.e.up_cb / kKB;  // k-blocks per scale column

    const int ntile = (u.np + kTileTok - 1) / kTileTok;
    const uint16_t* xp[MAXT];
#pragma unroll
    for (int tt = 0; tt < MAXT; ++tt) {
        const int q = min(tt * kTileTok + c, u.np - 1);
        xp[tt] = static_cast<const uint16_t*>(L.x) + (size_t)pair_token(L, u.pb + q) * H + g * 32;
    }

    f32x4 accg[MAXT], accu[MAXT];
#pragma unroll
    for (int tt = 0; tt < MAXT; ++tt) {
        accg[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
        accu[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    constexpr int D = 4;  // k-blocks in flight per wave
    u32x4 wb[D][4];
    u32x4 xb[D][4];
#pragma unroll
    for (int s = 0; s < D; ++s) {
        const int k = kb0 + s;
        if (k < kb1) {
            wb[s][0] = ld16(pg + k * kw);
            wb[s][1] = ld16(pg + k * kw + 16);
            wb[s][2] = ld16(pu + k * kw);
            wb[s][3] = ld16(pu + k * kw + 16);
            if (MAXT == 1) {
#pragma unroll
                for (int j = 0; j < 4; ++j) xb[s][j] = ld16(xp[0] + k * kKB + 8 * j);
            }
        }
    }

    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    for (int kb = kb0; kb < kb1; kb += D) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int k = kb + s;
            if (k < kb1) {
                V ag[4], au[4];
                ag[0] = M::cvt(wb[s][0][0], wb[s][0][1]);
                ag[1] = M::cvt(wb[s][0][2], wb[s][0][3]);
                ag[2] = M::cvt(wb[s][1][0], wb[s][1][1]);
                ag[3] = M::cvt(wb[s][1][2], wb[s][1][3]);
                au[0] = M::cvt(wb[s][2][0], wb[s][2][1]);
                au[1] = M::cvt(wb[s][2][2], wb[s][2][3]);
                au[2] = M::cvt(wb[s][3][0], wb[s][3][1]);
                au[3] = M::cvt(wb[s][3][2], wb[s][3][3]);
                const float scg = sg[k / kpg];
                const float scu = su[k / kpu];
#pragma unroll
                for (int tt = 0; tt < MAXT; ++tt) {
                    if (tt < ntile) {
                        V bx[4];
                        if (MAXT == 1) {
#pragma unroll
                            for (int j = 0; j < 4; ++j) bx[j] = M::bits(xb[s][j]);
                        } else {
#pragma unroll
                            for (int j = 0; j < 4; ++j) bx[j] = M::bits(ld16(xp[tt] + k * kKB + 8 * j));
                        }
                        f32x4 tg = M::mma(ag[0], bx[0], zero);
                        f32x4 tu = M::mma(au[0], bx[0], zero);
#pragma unroll
                        for (int j = 1; j < 4; ++j) {
                            tg = M::mma(ag[j], bx[j], tg);
                            tu = M::mma(au[j], bx[j], tu);
                        }
                        accg[tt] += scg * tg;
                        accu[tt] += scu * tu;
                    }
                }
                const int kn = k + D;
                if (kn < kb1) {
                    wb[s][0] = ld16(pg + kn * kKB);
                    wb[s][1] = ld16(pg + kn * kKB + 16);
                    wb[s][2] = ld16(pu + kn * kKB);
                    wb[s][3] = ld16(pu + kn * kKB + 16);
                    if (MAXT == 1) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) xb[s][j] = ld16(xp[0] + kn * kKB + 8 * j);
                    }
                }
            }
        }
    }

    // Cross-wave K reduction in a fixed order, then the SiLU epilogue.
    __shared__ f32x4 red[kWaves][MAXT][2][64];
#pragma unroll
    for (int tt = 0; tt < MAXT; ++tt) {
        red[wave][tt][0][lane] = accg[tt];
        red[wave][tt][1][lane] = accu[tt];
    }
    __syncthreads();
    for (int tt = wave; tt < ntile; tt += kWaves) {
        f32x4 G = red[0][tt][0][lane], U = red[0][tt][1][lane];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) {
            G += red[w][tt][0][lane];
            U += red[w][tt][1][lane];
        }
        const int q = tt * kTileTok + c;
        if (q < u.np) {
            const size_t p = (size_t)(u.pb + q);
            const int row = r0 + 4 * g;
            uint32_t hi[4], lo[4];
            float hv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float gate = G[i], up = U[i];
                const float silu = gate / (1.0f + expf(-gate));
                const float h = silu * up;
                hv[i] = h;
                hi[i] = bf16_rne(h);
                lo[i] = bf16_rne(h - __uint_as_float(hi[i] << 16));
            }
            uint2 vhi = {hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
            uint2 vlo = {lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
            *reinterpret_cast<uint2*>(L.h_hi + p * I + row) = vhi;
            *reinterpret_cast<uint2*>(L.h_lo + p * I + row) = vlo;
            if (L.h_f32 != nullptr) {
                *reinterpret_cast<float4*>(L.h_f32 + p * I + row) =
                    float4{hv[0], hv[1], hv[2], hv[3]};
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Phase B: down.  Each wave owns 16 rows of Wd (full K = inter), the
// workgroup 64 rows; B operand = the bf16 hi/lo split of h for <= 16*MAXT
// pairs.  Writes fp32 per-pair outputs (grouped) or the final output
// (single mode).  grid = (hidden/64, max_items), block = 256.
template <int MAXT>
__global__ __launch_bounds__(256) void k_down_rt(ExpertLaunch L) {
    typedef Mma<false> M;
    typedef M::V V;
    Unit u;
    if (!resolve_unit_rt(L, blockIdx.y, kTileTok * MAXT, &u)) return;
    const int H = u.e.hidden, I = u.e.inter;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const int rw = blockIdx.x * (kTileRows * kWaves) + wave * kTileRows;
    if (rw >= H) return;
    const int nkb = I / kKB;

    const uint8_t* pd = u.e.w_down + (size_t)(rw + c) * I + g * 32;
    const float* sd = u.e.s_down + (size_t)(rw / u.e.down_rb) * ((I + u.e.down_cb - 1) / u.e.down_cb);
    const int kpd = u.e.down_cb / kKB;

    const int ntile = (u.np + kTileTok - 1) / kTileTok;
    const uint16_t* hh[MAXT];
    const uint16_t* hl[MAXT];
#pragma unroll
    for (int tt = 0; tt < MAXT; ++tt) {
        const int q = min(tt * kTileTok + c, u.np - 1);
        const size_t p = (size_t)(u.pb + q);
        hh[tt] = L.h_hi + p * I + g * 32;
        hl[tt] = L.h_lo + p * I + g * 32;
    }

    f32x4 acc[MAXT];
#pragma unroll
    for (int tt = 0; tt < MAXT; ++tt) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};

    constexpr int D = 4;
    u32x4 wb[D][2];
    u32x4 hb[D][8];
#pragma unroll
    for (int s = 0; s < D; ++s) {
        const int k = s;
        if (k < nkb) {
            wb[s][0] = ld16(pd + k * kKB);
            wb[s][1] = ld16(pd + k * kKB + 16);
            if (MAXT == 1) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    hb[s][j] = ld16(hh[0] + k * kKB + 8 * j);
                    hb[s][4 + j] = ld16(hl[0] + k * kKB + 8 * j);
                }
            }
        }
    }

    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < nkb; kb += D) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int k = kb + s;
            if (k < nkb) {
                V a[4];
                a[0] = M::cvt(wb[s][0][0], wb[s][0][1]);
                a[1] = M::cvt(wb[s][0][2], wb[s][0][3]);
                a[2] = M::cvt(wb[s][1][0], wb[s][1][1]);
                a[3] = M::cvt(wb[s][1][2], wb[s][1][3]);
                const float sc = sd[k / kpd];
#pragma unroll
                for (int tt = 0; tt < MAXT; ++tt) {
                    if (tt < ntile) {
                        V bh[4], bl[4];
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            if (MAXT == 1) {
                                bh[j] = M::bits(hb[s][j]);
                                bl[j] = M::bits(hb[s][4 + j]);
                            } else {
                                bh[j] = M::bits(ld16(hh[tt] + k * kKB + 8 * j));
                                bl[j] = M::bits(ld16(hl[tt] + k * kKB + 8 * j));
                            }
                        }
                        f32x4 t = M::mma(a[0], bh[0], zero);
                        t = M::mma(a[0], bl[0], t);
#pragma unroll
                        for (int j = 1; j < 4; ++j) {
                            t = M::mma(a[j], bh[j], t);
                            t = M::mma(a[j], bl[j], t);
                        }
                        acc[tt] += sc * t;
                    }
                }
                const int kn = k + D;
                if (kn < nkb) {
                    wb[s][0] = ld16(pd + kn * kKB);
                    wb[s][1] = ld16(pd + kn * kKB + 16);
                    if (MAXT == 1) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            hb[s][j] = ld16(hh[0] + kn * kKB + 8 * j);
                            hb[s][4 + j] = ld16(hl[0] + kn * kKB + 8 * j);
                        }
                    }
                }
            }
        }
    }

    const int row = rw + 4 * g;
#pragma unroll
    for (int tt = 0; tt < MAXT; ++tt) {
        const int q = tt * kTileTok + c;
        if (tt < ntile && q < u.np) {
            const size_t p = (size_t)(u.pb + q);
            const f32x4 v = acc[tt];
            if (L.table != nullptr) {
                *reinterpret_cast<float4*>(L.y_part + p * H + row) = float4{v[0], v[1], v[2], v[3]};
            } else {
                // single mode: pair == token
                uint16_t* yo = static_cast<uint16_t*>(L.y) + p * H + row;
                const uint2 o = {cast_out(v[0], L.out_dtype) | (cast_out(v[1], L.out_dtype) << 16),
                                 cast_out(v[2], L.out_dtype) | (cast_out(v[3], L.out_dtype) << 16)};
                *reinterpret_cast<uint2*>(yo) = o;
                if (L.y_f32 != nullptr) {
                    *reinterpret_cast<float4*>(L.y_f32 + p * H + row) = float4{v[0], v[1], v[2], v[3]};
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Phase A with a compile-time trip count: gate_up_tile (cx_gate_up.h) over
// grid = (inter/16, items).
// With L.gu_part set (decode, grouped mode), the last row of the grid
// finalises the shared expert's h from its stage-2 k-part sums.
template <int NKB, int D, int MAXT, bool F16, bool XLDS, int KS, bool SINGLE>
__global__ __launch_bounds__(64 * KS) void k_gate_up_t(ExpertLaunch L) {
    extern __shared__ __attribute__((aligned(16))) unsigned char gu_lds[];
    if (!SINGLE && MAXT == 1 && L.gu_part != nullptr && blockIdx.y == gridDim.y - 1) {
        shared_h_finalize(L, blockIdx.x);
        return;
    }
    gate_up_tile<NKB, D, MAXT, F16, XLDS, KS, SINGLE>(L, blockIdx.x, blockIdx.y, gu_lds);
}

// ---------------------------------------------------------------------------
// Phase B per work item with a compile-time trip count (prefill / single
// expert): each wave owns 16 rows of Wd over the full K = NKB k-blocks.
template <int NKB, int D, int MAXT>
__global__ __launch_bounds__(256) void k_down_t(ExpertLaunch L) {
    typedef Mma<false> M;
    typedef M::V V;
    Unit u;
    if (!resolve_unit_rt(L, blockIdx.y, kTileTok * MAXT, &u)) return;
    const int H = u.e.hidden, I = u.e.inter;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const int rw = blockIdx.x * (kTileRows * kWaves) + wave * kTileRows;
    const uint8_t* pd = u.e.w_down + (size_t)(rw + c) * I + g * 32;
    const float* sd = u.e.s_down + (size_t)(rw / u.e.down_rb) * (I / kKB);
    float scd[NKB];
#pragma unroll
    for (int k = 0; k < NKB; ++k) scd[k] = ldf(sd + k);
    const int ntile = (u.np + kTileTok - 1) / kTileTok;
    const uint16_t* hh[MAXT];
    const uint16_t* hl[MAXT];
#pragma unroll
    for (int tt = 0; tt < MAXT; ++tt) {
        const size_t p = (size_t)(u.pb + min(tt * kTileTok + c, u.np - 1));
        hh[tt] = L.h_hi + p * I + g * 32;
        hl[tt] = L.h_lo + p * I + g * 32;
    }
    f32x4 acc[MAXT];
#pragma unroll
    for (int tt = 0; tt < MAXT; ++tt) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 wb[D][2];
    u32x4 hb[8];  // MAXT == 1: h of the next step, loaded one step ahead
#pragma unroll
    for (int s = 0; s < D && s < NKB; ++s) {
        wb[s][0] = ld16(pd + s * kKB);
        wb[s][1] = ld16(pd + s * kKB + 16);
    }
    if (MAXT == 1) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            hb[j] = ld16(hh[0] + 8 * j);
            hb[4 + j] = ld16(hl[0] + 8 * j);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < NKB; ++k) {
        const int s = k % D;
        V a[4];
        a[0] = M::cvt(wb[s][0][0], wb[s][0][1]);
        a[1] = M::cvt(wb[s][0][2], wb[s][0][3]);
        a[2] = M::cvt(wb[s][1][0], wb[s][1][1]);
        a[3] = M::cvt(wb[s][1][2], wb[s][1][3]);
#pragma unroll
        for (int tt = 0; tt < MAXT; ++tt) {
            if (MAXT == 1 || tt < ntile) {
                V bh[4], bl[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (MAXT == 1) {
                        bh[j] = M::bits(hb[j]);
                        bl[j] = M::bits(hb[4 + j]);
                    } else {
                        bh[j] = M::bits(ld16(hh[tt] + k * kKB + 8 * j));
                        bl[j] = M::bits(ld16(hl[tt] + k * kKB + 8 * j));
                    }
                }
                f32x4 t = M::mma(a[0], bh[0], zero);
                t = M::mma(a[0], bl[0], t);
#pragma unroll
                for (int j = 1; j < 4; ++j) {
                    t = M::mma(a[j], bh[j], t);
                    t = M::mma(a[j], bl[j], t);
                }
                acc[tt] += scd[k] * t;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (MAXT == 1 && k + 1 < NKB) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                hb[j] = ld16(hh[0] + (k + 1) * kKB + 8 * j);
                hb[4 + j] = ld16(hl[0] + (k + 1) * kKB + 8 * j);
            }
        }
        if (k + D < NKB) {
            wb[s][0] = ld16(pd + (k + D) * kKB);
            wb[s][1] = ld16(pd + (k + D) * kKB + 16);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    const int row = rw + 4 * g;
#pragma unroll
    for (int tt = 0; tt < MAXT; ++tt) {
        const int q = tt * kTileTok + c;
        if (tt < ntile && q < u.np) {
            const size_t p = (size_t)(u.pb + q);
            const f32x4 v = acc[tt];
            if (L.table != nullptr) {
                *reinterpret_cast<float4*>(L.y_part + p * H + row) = float4{v[0], v[1], v[2], v[3]};
            } else {
                uint16_t* yo = static_cast<uint16_t*>(L.y) + p * H + row;
                *reinterpret_cast<uint2*>(yo) =
                    uint2{cast_out(v[0], L.out_dtype) | (cast_out(v[1], L.out_dtype) << 16),
                          cast_out(v[2], L.out_dtype) | (cast_out(v[3], L.out_dtype) << 16)};
                if (L.y_f32 != nullptr)
                    *reinterpret_cast<float4*>(L.y_f32 + p * H + row) = float4{v[0], v[1], v[2], v[3]};
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Down projection per work item of <= 16 pairs: down_item_tile (cx_down.h),
// grid = (hidden/64, items).
template <int NKB, int D, bool SINGLE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_down_item(ExpertLaunch L) {
    down_item_tile<NKB, D, SINGLE>(L, blockIdx.x, blockIdx.y);
}

// ---------------------------------------------------------------------------
// One-token decode: down projection of every item plus the weighted combine
// (down_comb1_tile, cx_down.h), grid = hidden/rows workgroups of 8 waves.
template <int NKB, int D, int PRE = 0>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void k_down_comb1(
    ExpertLaunch L, const int* __restrict__ token_pairs, const float* __restrict__ topk_w, int top_k,
    int rows) {
    extern __shared__ __attribute__((aligned(16))) unsigned char dc_lds[];
    down_comb1_tile<NKB, D, PRE>(L, token_pairs, topk_w, top_k, dc_lds, blockIdx.x, rows);
}

// ---------------------------------------------------------------------------
// One expert at 1..4 tokens (single mode), as two launches in which every
// wave's weights are one round trip of loads.  At this size the launches are
// bound by per-wave latency and MFMA work, not by HBM: the 16-row x full-K
// waves of k_gate_up_t<14, 4> / k_down_item took 12.7 and 7.1 us at 4 tokens
// even with all 44 MB resident in the MALL (13.4 and 7.6 from HBM).
//  * Gate/up (k_gate_up_kpart): 2 k-parts x inter/16 tiles of 8-wave
//    workgroups (KSA active waves x NKB k-blocks, the shared-expert split of
//    k_dec_select_sgu), fp32 part sums to L.gu_part[kpart][gate, up][t][row].
//    Twice the workgroups of one 16-row tile per workgroup, so every CU
//    streams; K over 8 waves of one workgroup instead keeps half the CUs idle.
//  * Down (k_down_ks): workgroup = 2 row groups of 16 output rows x 4 k
//    ranges (8 waves, NKBW k-blocks each, all loads in flight at once).  The
//    waves of a k range first turn its part sums into h = silu(g0 + g1) *
//    (u0 + u1) (the order of shared_h_finalize), bf16 hi + lo, in a shared
//    LDS slice, half each; the 4 partial tiles of a row group are summed in
//    LDS in k order.
template <int NKB, int KSA, bool F16, bool XLDS>
__global__ __launch_bounds__(512) void k_gate_up_kpart(ExpertLaunch L) {
    extern __shared__ __attribute__((aligned(16))) unsigned char gk_lds[];
    gate_up_tile<NKB, (NKB < 4 ? NKB : 4), 1, F16, XLDS, 8, true, KSA, kTileRows, true>(
        L, blockIdx.x, 0, gk_lds, blockIdx.y);
}

constexpr int kDownKsRows = 4;   // tokens of the split-K down launch
constexpr int kDownKsGroups = 2;  // 16-row groups per workgroup

constexpr size_t down_ks_lds(int nkbw) {
    return (size_t)4 * 2 * kDownKsRows * ((size_t)nkbw * kKB * 2 + 16) + (size_t)4 * kDownKsGroups * 64 * 16;
}

// The down k-split in pieces (the measured one-launch form of this expert,
// cx_kbench one-launch, issues the weights long before the part sums exist
// and runs the same pieces):
//  * down_ks_parts: this wave's half of its k range's part sums (global loads)
//  * down_ks_weights: this wave's 16 rows x NKBW k-blocks of Wd (all in flight)
//  * down_ks_h: h = silu(g0 + g1) * (u0 + u1) into LDS
//  * down_ks_mma: MFMA on the weights (fp8, or converted ahead), k-order sum, store
// Workgroup `blk` covers row groups 2 blk, 2 blk + 1 (wave >> 2) x 4 k ranges (wave & 3).
template <int NKBW>
struct DownKsParts {
    static constexpr int KW = NKBW * kKB;  // k per range
    static constexpr int NI = KW / 4;      // 4-k items per token and range
    static constexpr int ITEMS = (NI + 127) / 128;
    float4 g0[kDownKsRows][ITEMS], g1[kDownKsRows][ITEMS], u0[kDownKsRows][ITEMS], u1[kDownKsRows][ITEMS];
};

template <int NKBW>
__device__ __forceinline__ void down_ks_parts(const ExpertLaunch& L, DownKsParts<NKBW>& P) {
    typedef DownKsParts<NKBW> DP;
    const int I = L.inter, np = L.n_tokens;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int rg = wave >> 2, kb0 = (wave & 3) * NKBW;
    const size_t T = (size_t)np;
    const float* gp = L.gu_part + (size_t)kb0 * kKB;
#pragma unroll
    for (int q = 0; q < kDownKsRows; ++q) {
        if (q < np) {
#pragma unroll
            for (int it = 0; it < DP::ITEMS; ++it) {
                const int i = it * 128 + rg * 64 + lane;
                if (DP::NI % 128 != 0 && i >= DP::NI) continue;
                const size_t k4 = (size_t)i * 4;
                P.g0[q][it] = *reinterpret_cast<const float4*>(gp + ((0 * 2 + 0) * T + q) * I + k4);
                P.g1[q][it] = *reinterpret_cast<const float4*>(gp + ((1 * 2 + 0) * T + q) * I + k4);
                P.u0[q][it] = *reinterpret_cast<const float4*>(gp + ((0 * 2 + 1) * T + q) * I + k4);
                P.u1[q][it] = *reinterpret_cast<const float4*>(gp + ((1 * 2 + 1) * T + q) * I + k4);
            }
        }
    }
}

template <int NKBW>
__device__ __forceinline__ const uint8_t* down_ks_row(const ExpertLaunch& L, int blk) {
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int r0 = (blk * kDownKsGroups + (wave >> 2)) * kTileRows;
    return L.single.w_down + (size_t)(r0 + (lane & 15)) * L.inter + (size_t)(wave & 3) * NKBW * kKB +
           (lane >> 4) * 32;
}

template <int NKBW>
__device__ __forceinline__ void down_ks_weights(const uint8_t* pd, u32x4 (&wb)[NKBW][2]) {
#pragma unroll
    for (int k = 0; k < NKBW; ++k) {
        wb[k][0] = ld16(pd + k * kKB);
        wb[k][1] = ld16(pd + k * kKB + 16);
    }
}

// This wave's down scales (scalar loads, held in SGPRs).
template <int NKBW>
__device__ __forceinline__ void down_ks_scales(const ExpertLaunch& L, int blk, float (&scd)[NKBW]) {
    const cx_expert_desc& e = L.single;
    const int wave = wave_id();
    const int r0 = (blk * kDownKsGroups + (wave >> 2)) * kTileRows;
    const int rbd = __builtin_amdgcn_readfirstlane(r0 / e.down_rb);
    const float* sd = e.s_down + (size_t)rbd * (L.inter / kKB) + (wave & 3) * NKBW;
#pragma unroll
    for (int k = 0; k < NKBW; ++k) scd[k] = ldsc(sd + k);
}

// h = silu(g0 + g1) * (u0 + u1), bf16 hi + lo, into the k range's LDS slice,
// then a workgroup barrier.
template <int NKBW>
__device__ __forceinline__ void down_ks_h(const ExpertLaunch& L, const DownKsParts<NKBW>& P, unsigned char* lds) {
    typedef DownKsParts<NKBW> DP;
    constexpr size_t HS = DP::KW * 2 + 16;  // LDS row stride (bytes) of one h plane
    const int np = L.n_tokens;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int rg = wave >> 2, kq = wave & 3;
    unsigned char* hw = lds + (size_t)kq * (2 * kDownKsRows * HS);
#pragma unroll
    for (int q = 0; q < kDownKsRows; ++q) {
        if (q < np) {
#pragma unroll
            for (int it = 0; it < DP::ITEMS; ++it) {
                const int i = it * 128 + rg * 64 + lane;
                if (DP::NI % 128 != 0 && i >= DP::NI) continue;
                const float4 a = P.g0[q][it], b = P.g1[q][it], u = P.u0[q][it], v = P.u1[q][it];
                const float gs[4] = {a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w};
                const float us[4] = {u.x + v.x, u.y + v.y, u.z + v.z, u.w + v.w};
                uint32_t hi[4], lo[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float h = (gs[j] / (1.0f + expf(-gs[j]))) * us[j];
                    hi[j] = bf16_rne(h);
                    lo[j] = bf16_rne(h - __uint_as_float(hi[j] << 16));
                }
                const size_t off = (size_t)i * 8;
                *reinterpret_cast<uint2*>(hw + q * HS + off) = uint2{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
                *reinterpret_cast<uint2*>(hw + (kDownKsRows + q) * HS + off) =
                    uint2{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
            }
        }
    }
    __syncthreads();
}

// MFMA steps over this wave's rows and k range (step(k, hb): the product of
// k-block k with the h fragment hb), the 4 partial tiles of a row group
// summed in LDS in k order, and the store.
template <int NKBW, class Step>
__device__ __forceinline__ void down_ks_mma(const ExpertLaunch& L, int blk, const float (&scd)[NKBW], unsigned char* lds,
                                            Step step) {
    typedef DownKsParts<NKBW> DP;
    constexpr size_t HS = DP::KW * 2 + 16;
    const int H = L.hidden, np = L.n_tokens;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int rg = wave >> 2, kq = wave & 3;
    const int g = lane >> 4, c = lane & 15;
    const int r0 = (blk * kDownKsGroups + rg) * kTileRows;
    unsigned char* hw = lds + (size_t)kq * (2 * kDownKsRows * HS);
    f32x4* red = reinterpret_cast<f32x4*>(lds + 4 * (2 * kDownKsRows * HS));  // [8][64]
    const size_t hrow = (size_t)min(c, np - 1);
    const unsigned char* lh = hw + hrow * HS + g * 64;
    const unsigned char* ll = hw + (kDownKsRows + hrow) * HS + g * 64;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < NKBW; ++k) {
        u32x4 hb[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            hb[j] = *reinterpret_cast<const u32x4*>(lh + k * (kKB * 2) + 16 * j);
            hb[4 + j] = *reinterpret_cast<const u32x4*>(ll + k * (kKB * 2) + 16 * j);
        }
        acc += scd[k] * step(k, hb);
    }
    red[wave * 64 + lane] = acc;
    __syncthreads();
    if (kq == 0 && c < np) {
        const f32x4* rr = red + rg * 4 * 64;
        const f32x4 sum = ((rr[lane] + rr[64 + lane]) + rr[128 + lane]) + rr[192 + lane];
        store_out4(L.y, L.y_f32, (size_t)c * H + r0 + 4 * g, sum, L.out_dtype);
    }
}

template <int NKBW>
__global__ __launch_bounds__(512) void k_down_ks(ExpertLaunch L) {
    extern __shared__ __attribute__((aligned(16))) unsigned char dk_lds[];
    // part sums first: older than the weight loads, so waiting for them
    // leaves the weights in flight
    DownKsParts<NKBW> P;
    down_ks_parts<NKBW>(L, P);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 wb[NKBW][2];
    down_ks_weights<NKBW>(down_ks_row<NKBW>(L, blockIdx.x), wb);
    __builtin_amdgcn_sched_barrier(0);
    float scd[NKBW];
    down_ks_scales<NKBW>(L, blockIdx.x, scd);
    down_ks_h<NKBW>(L, P, dk_lds);
    down_ks_mma<NKBW>(L, blockIdx.x, scd, dk_lds, [&](int k, const u32x4(&hb)[8]) { return down_step(wb[k], hb); });
}

// ---------------------------------------------------------------------------
// Grouped GEMM for items of up to 64 pairs (cx_grouped.h): gate/up over
// grid = inter/128 row tiles x items (one dimension, an item's tiles
// consecutive, so they spread over the XCDs), down over grid = (hidden/256,
// items).  Measured at config 3: the XCD-aware placement (all tiles of an item
// on one XCD, its x rows in one L2) streamed 2.5 % slower for the gate/up and
// 5 % slower for the down than the spread placement.  Both kernels are 8-wave
// workgroups at two waves per SIMD: one per CU.  C1: one-tile items stage
// their x rows a chunk at a time (hidden = 14 k-blocks x n only; 112 KB of
// LDS): 3.8 % faster on one-tile items, 1.3 % on a config-3-like plan.
template <int NKB, bool F16, bool SINGLE, bool C1>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void k_gu_grp(ExpertLaunch L) {
    extern __shared__ __attribute__((aligned(16))) unsigned char grp_lds[];
    const int n_tiles = L.inter / kGuGrpRows;
    grp_gate_up_tile<NKB, F16, SINGLE, C1>(L, blockIdx.x % n_tiles, blockIdx.x / n_tiles, grp_lds);
}

template <int NKB, bool SINGLE>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void k_dn_grp(ExpertLaunch L) {
    extern __shared__ __attribute__((aligned(16))) unsigned char grp_lds[];
    grp_down_tile<NKB, SINGLE>(L, blockIdx.x, blockIdx.y, grp_lds);
}

// ---------------------------------------------------------------------------
// Combine: y[t] = sum_k w_k * y_part[pair(t,k)]  (route order, fp32)
//               + y_part[pair(t, shared)]
// then cast (RNE).  One thread per 4 consecutive features.  A token's pair
// indices come in one round trip and every weight and partial row it needs
// (KC routes at a time, the shared expert's row with the first batch) in a
// second; a route the planner dropped (pair -1) contributes nothing.
__global__ __launch_bounds__(256) void k_combine(PlanPtrs plan, const float* __restrict__ y_part,
                                                 int n_tokens, int top_k, int hidden, void* y,
                                                 int out_dtype, float* y_f32) {
    constexpr int KC = 8;  // routes fetched per batch
    const int n4 = hidden / 4;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_tokens * n4) return;
    const int t = idx / n4;
    const int f = (idx - t * n4) * 4;
    const int* tp = plan.token_pairs + (size_t)t * (top_k + 1);
    const int ps = tp[top_k];
    float4 vs = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < top_k; k0 += KC) {
        int p[KC];
#pragma unroll
        for (int j = 0; j < KC; ++j) p[j] = k0 + j < top_k ? tp[k0 + j] : -1;
        float w[KC];
        float4 v[KC];
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const size_t q = p[j] >= 0 ? (size_t)p[j] : 0;
            w[j] = plan.pair_weight[q];
            v[j] = *reinterpret_cast<const float4*>(y_part + q * hidden + f);
        }
        if (k0 == 0 && ps >= 0) vs = *reinterpret_cast<const float4*>(y_part + (size_t)ps * hidden + f);
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            if (p[j] >= 0) {
                acc[0] += w[j] * v[j].x;
                acc[1] += w[j] * v[j].y;
                acc[2] += w[j] * v[j].z;
                acc[3] += w[j] * v[j].w;
            }
        }
    }
    if (ps >= 0) {
        if (top_k <= 0) vs = *reinterpret_cast<const float4*>(y_part + (size_t)ps * hidden + f);
        acc[0] += vs.x;
        acc[1] += vs.y;
        acc[2] += vs.z;
        acc[3] += vs.w;
    }
    uint16_t* yo = static_cast<uint16_t*>(y) + (size_t)t * hidden + f;
    const uint2 o = {cast_out(acc[0], out_dtype) | (cast_out(acc[1], out_dtype) << 16),
                     cast_out(acc[2], out_dtype) | (cast_out(acc[3], out_dtype) << 16)};
    *reinterpret_cast<uint2*>(yo) = o;
    if (y_f32 != nullptr) {
        *reinterpret_cast<float4*>(y_f32 + (size_t)t * hidden + f) = float4{acc[0], acc[1], acc[2], acc[3]};
    }
}

// Decode combine: the y_part row of (token t, route k) is S0 + t*K + k (S0 =
// T with a shared expert, whose rows are [0, T)), so the route weights, the
// pair table and the partial rows are all fetched at once (one round trip);
// a route dropped by the planner (pair -1) contributes nothing.  Same order
// as k_combine: route order, shared expert last.
__global__ __launch_bounds__(256) void k_combine_dec(const int* __restrict__ token_pairs,
                                                     const float* __restrict__ topk_w,
                                                     const float* __restrict__ y_part, int n_tokens,
                                                     int top_k, int has_shared, int hidden, void* y,
                                                     int out_dtype, float* y_f32) {
    constexpr int KC = 8;  // routes fetched per batch
    const int n4 = hidden / 4;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_tokens * n4) return;
    const int t = idx / n4;
    const int f = (idx - t * n4) * 4;
    const int s0 = has_shared ? n_tokens : 0;
    const int* tp = token_pairs + (size_t)t * (top_k + 1);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < top_k; k0 += KC) {
        int p[KC];
        float w[KC];
        float4 v[KC];
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const int k = min(k0 + j, top_k - 1);
            p[j] = k0 + j < top_k ? tp[k] : -1;
            w[j] = topk_w[(size_t)t * top_k + k];
            v[j] = *reinterpret_cast<const float4*>(y_part + ((size_t)s0 + (size_t)t * top_k + k) * hidden + f);
        }
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            if (p[j] >= 0) {
                acc[0] += w[j] * v[j].x;
                acc[1] += w[j] * v[j].y;
                acc[2] += w[j] * v[j].z;
                acc[3] += w[j] * v[j].w;
            }
        }
    }
    if (tp[top_k] >= 0) {
        const float4 v = *reinterpret_cast<const float4*>(y_part + (size_t)t * hidden + f);
        acc[0] += v.x;
        acc[1] += v.y;
        acc[2] += v.z;
        acc[3] += v.w;
    }
    store_out4(y, y_f32, (size_t)t * hidden + f, acc, out_dtype);
}

// ---------------------------------------------------------------------------
// Generic single-expert path (any shape / block size): one thread per output
// row, reference order.  Used for shapes the grouped kernels do not tile
// (e.g. the 4x8 / 1x1-block experts of the reference's control tests).
__device__ __forceinline__ float fp8_val(uint8_t b) {
    return __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(b), 0);
}

__device__ __forceinline__ float act_val(const void* x, size_t i, int dtype) {
    const uint16_t b = static_cast<const uint16_t*>(x)[i];
    if (dtype == CX_DTYPE_FP16) return static_cast<float>(__builtin_bit_cast(_Float16, b));
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__global__ void k_generic_gate_up(cx_expert_desc e, const void* x, int in_dtype, int n_tokens,
                                  float* h) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_tokens * e.inter) return;
    const int t = idx / e.inter, r = idx - t * e.inter;
    const int ncu = (e.hidden + e.up_cb - 1) / e.up_cb, ncg = (e.hidden + e.gate_cb - 1) / e.gate_cb;
    float up = 0.f, gate = 0.f;
    for (int k = 0; k < e.hidden; ++k) {
        const float xv = act_val(x, (size_t)t * e.hidden + k, in_dtype);
        const size_t wi = gu_elem_off(e.gu_layout, e.hidden, r, k);
        const float wu = fp8_val(e.w_up[wi]) * e.s_up[(r / e.up_rb) * ncu + k / e.up_cb];
        const float wg = fp8_val(e.w_gate[wi]) * e.s_gate[(r / e.gate_rb) * ncg + k / e.gate_cb];
        up = __fadd_rn(up, __fmul_rn(wu, xv));
        gate = __fadd_rn(gate, __fmul_rn(wg, xv));
    }
    h[idx] = (gate / (1.0f + expf(-gate))) * up;
}

__global__ void k_generic_down(cx_expert_desc e, const float* h, int n_tokens, void* y,
                               int out_dtype, float* y_f32) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_tokens * e.hidden) return;
    const int t = idx / e.hidden, r = idx - t * e.hidden;
    const int ncd = (e.inter + e.down_cb - 1) / e.down_cb;
    float sum = 0.f;
    for (int k = 0; k < e.inter; ++k) {
        const float w = fp8_val(e.w_down[(size_t)r * e.inter + k]) *
                        e.s_down[(r / e.down_rb) * ncd + k / e.down_cb];
        sum = __fadd_rn(sum, __fmul_rn(w, h[(size_t)t * e.inter + k]));
    }
    static_cast<uint16_t*>(y)[idx] = static_cast<uint16_t>(cast_out(sum, out_dtype));
    if (y_f32 != nullptr) y_f32[idx] = sum;
}

}  // namespace

bool fast_path_ok(const cx_expert_desc& e) {
    if (e.hidden <= 0 || e.inter <= 0) return false;
    if (e.hidden % (kTileRows * kWaves) != 0 || e.hidden % kKB != 0) return false;
    if (e.inter % kKB != 0 || e.hidden / kKB < kWaves) return false;
    const int rbs[3] = {e.up_rb, e.gate_rb, e.down_rb};
    const int cbs[3] = {e.up_cb, e.gate_cb, e.down_cb};
    for (int i = 0; i < 3; ++i) {
        if (rbs[i] <= 0 || rbs[i] % kTileRows != 0 || cbs[i] != kKB) return false;
    }
    return true;
}

namespace {

template <int NKB, int KS, int MAXT, bool F16>
void go_gate_up(const ExpertLaunch& L, dim3 grid, hipStream_t s) {
    constexpr int D = NKB < 4 ? NKB : 4;
    const dim3 block(64 * KS);
    const bool single = L.table == nullptr;
    if (MAXT == 1 && L.np_lds > 0) {
        const size_t lds = gate_up_lds_bytes(KS, 1, L.np_lds, L.hidden);
        if (single) cx_launch((k_gate_up_t<NKB, D, 1, F16, true, KS, true>), grid, block, lds, s, L);
        else cx_launch((k_gate_up_t<NKB, D, 1, F16, true, KS, false>), grid, block, lds, s, L);
    } else {
        const size_t lds = gate_up_lds_bytes(KS, MAXT, 0, L.hidden);
        if (single) cx_launch((k_gate_up_t<NKB, D, MAXT, F16, false, KS, true>), grid, block, lds, s, L);
        else cx_launch((k_gate_up_t<NKB, D, MAXT, F16, false, KS, false>), grid, block, lds, s, L);
    }
}

template <int MAXT, bool F16>
bool pick_gate_up(const ExpertLaunch& L, dim3 grid, hipStream_t s) {
    if (L.hidden % kKB != 0) return false;
    switch (L.hidden / kKB) {
        case 56: go_gate_up<14, 4, MAXT, F16>(L, grid, s); return true;
        case 4: go_gate_up<1, 4, MAXT, F16>(L, grid, s); return true;
        case 8: go_gate_up<2, 4, MAXT, F16>(L, grid, s); return true;
        default: return false;
    }
}

// Weight ring depth of the LDS-staged down kernel: 6 k-blocks (12 KB) in
// flight per wave keeps it within 128 registers (4 waves per SIMD, so a
// decode grid of 8 experts x 112 tiles is resident at once).
constexpr int kDownXlDepth = 6;

template <int NKB>
void go_down_item(const ExpertLaunch& L, dim3 grid, hipStream_t s) {
    const size_t lds = down_item_lds(L.inter);
    if (L.table == nullptr) cx_launch((k_down_item<NKB, kDownXlDepth, true>), grid, dim3(256), lds, s, L);
    else cx_launch((k_down_item<NKB, kDownXlDepth, false>), grid, dim3(256), lds, s, L);
}

template <int MAXT>
bool pick_down(const ExpertLaunch& L, dim3 grid, hipStream_t s) {
    if (MAXT == 1) {
        switch (L.inter / kKB) {
            case 4: go_down_item<4>(L, grid, s); return true;
            case 16: go_down_item<16>(L, grid, s); return true;
            default: return false;
        }
    }
    switch (L.inter / kKB) {
        case 4: cx_launch((k_down_t<4, 4, MAXT>), grid, dim3(256), 0, s, L); return true;
        case 16: cx_launch((k_down_t<16, 4, MAXT>), grid, dim3(256), 0, s, L); return true;
        default: return false;
    }
}

// The grouped GEMM serves items of up to 64 pairs when the device grants its
// LDS rings and the shape tiles evenly.
bool grp_ok(const ExpertLaunch& L) {
    return L.maxt == 4 && L.max_lds >= (int)grp_dn_lds() && L.inter % kGuGrpRows == 0 &&
           L.hidden % kDnGrpRows == 0 && L.hidden / kKB <= 64 && L.inter / kKB <= 64;
}

template <int NKB, bool F16, bool C1>
void go_gu_grp_c(const ExpertLaunch& L, dim3 grid, hipStream_t s) {
    const dim3 block(64 * kGuGrpWaves);
    const size_t lds = C1 ? grp_gu_c1_lds() : grp_gu_lds();
    if (L.table == nullptr) cx_launch((k_gu_grp<NKB, F16, true, C1>), grid, block, lds, s, L);
    else cx_launch((k_gu_grp<NKB, F16, false, C1>), grid, block, lds, s, L);
}

template <int NKB, bool F16>
void go_gu_grp(const ExpertLaunch& L, dim3 grid, hipStream_t s) {
    if constexpr (NKB % kGuChunk == 0) {
        if (L.max_lds >= (int)grp_gu_c1_lds()) {
            go_gu_grp_c<NKB, F16, true>(L, grid, s);
            return;
        }
    }
    go_gu_grp_c<NKB, F16, false>(L, grid, s);
}

bool pick_gu_grp(const ExpertLaunch& L, int items, hipStream_t s) {
    const dim3 grid((L.inter / kGuGrpRows) * items);
    const bool f16 = L.in_dtype == CX_DTYPE_FP16;
    switch (L.hidden / kKB) {
        case 56: f16 ? go_gu_grp<56, true>(L, grid, s) : go_gu_grp<56, false>(L, grid, s); return true;
        case 4: f16 ? go_gu_grp<4, true>(L, grid, s) : go_gu_grp<4, false>(L, grid, s); return true;
        case 8: f16 ? go_gu_grp<8, true>(L, grid, s) : go_gu_grp<8, false>(L, grid, s); return true;
        default: return false;
    }
}

template <int NKB>
void go_dn_grp(const ExpertLaunch& L, dim3 grid, hipStream_t s) {
    if (L.table == nullptr) cx_launch((k_dn_grp<NKB, true>), grid, dim3(512), grp_dn_lds(), s, L);
    else cx_launch((k_dn_grp<NKB, false>), grid, dim3(512), grp_dn_lds(), s, L);
}

bool pick_dn_grp(const ExpertLaunch& L, int items, hipStream_t s) {
    const dim3 grid(L.hidden / kDnGrpRows, items);
    switch (L.inter / kKB) {
        case 16: go_dn_grp<16>(L, grid, s); return true;
        case 4: go_dn_grp<4>(L, grid, s); return true;
        default: return false;
    }
}

}  // namespace

hipError_t launch_gate_up(const ExpertLaunch& L, hipStream_t s) {
    const int items = L.table != nullptr ? L.max_items + (L.gu_part != nullptr && L.maxt == 1 ? 1 : 0)
                                         : (L.n_tokens + kTileTok * L.maxt - 1) / (kTileTok * L.maxt);
    if (grp_ok(L) && pick_gu_grp(L, items, s)) return hipGetLastError();
    const dim3 grid(L.inter / kTileRows, items);
    const bool f16 = L.in_dtype == CX_DTYPE_FP16;
    bool done;
    if (L.maxt == 1) done = f16 ? pick_gate_up<1, true>(L, grid, s) : pick_gate_up<1, false>(L, grid, s);
    else done = f16 ? pick_gate_up<4, true>(L, grid, s) : pick_gate_up<4, false>(L, grid, s);
    if (!done) {
        if (L.maxt == 1) {
            if (f16) cx_launch((k_gate_up_rt<1, true>), grid, dim3(256), 0, s, L);
            else cx_launch((k_gate_up_rt<1, false>), grid, dim3(256), 0, s, L);
        } else {
            if (f16) cx_launch((k_gate_up_rt<4, true>), grid, dim3(256), 0, s, L);
            else cx_launch((k_gate_up_rt<4, false>), grid, dim3(256), 0, s, L);
        }
    }
    return hipGetLastError();
}

hipError_t launch_down(const ExpertLaunch& L, hipStream_t s) {
    const int items = L.table != nullptr ? L.max_items
                                         : (L.n_tokens + kTileTok * L.maxt - 1) / (kTileTok * L.maxt);
    if (grp_ok(L) && pick_dn_grp(L, items, s)) return hipGetLastError();
    const dim3 grid(L.hidden / (kTileRows * kWaves), items);
    const bool done = L.maxt == 1 ? pick_down<1>(L, grid, s) : pick_down<4>(L, grid, s);
    if (!done) {
        if (L.maxt == 1) cx_launch((k_down_rt<1>), grid, dim3(256), 0, s, L);
        else cx_launch((k_down_rt<4>), grid, dim3(256), 0, s, L);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Grouped GEMM for items of up to 128 pairs (cx_big.h).  Each ring stage is
// its own LDS array (static, one workgroup per CU), so the compiler's waits
// for the stage DMA do not cover the stages still in flight.
namespace {

template <int NKB, bool F16>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void k_gu_big(ExpertLaunch L) {
    __shared__ __attribute__((aligned(16))) unsigned char s0[kBigGuA + kBigGuB];
    __shared__ __attribute__((aligned(16))) unsigned char s1[kBigGuA + kBigGuB];
    __shared__ __attribute__((aligned(16))) unsigned char s2[kBigGuA + kBigGuB];
    __shared__ __attribute__((aligned(16))) unsigned char s3[kBigGuA + kBigGuB];
    unsigned char* const st[kBigGuRing] = {s0, s1, s2, s3};
    big_gate_up<NKB, F16>(L, st);
}

template <int NKB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void k_dn_big(ExpertLaunch L) {
    __shared__ __attribute__((aligned(16))) unsigned char s0[kBigDnA + 2 * kBigDnB];
    __shared__ __attribute__((aligned(16))) unsigned char s1[kBigDnA + 2 * kBigDnB];
    __shared__ __attribute__((aligned(16))) unsigned char s2[kBigDnA + 2 * kBigDnB];
    unsigned char* const st[kBigDnRing] = {s0, s1, s2};
    big_down<NKB>(L, st);
}

// grid: every (item, row tile) of the plan's bound, rounded up to whole XCD
// rows (big_tile maps the tiles that exist)
dim3 big_grid(int items, int row_tiles) { return dim3((items * row_tiles + 7) / 8 * 8); }

}  // namespace

bool big_shape_ok(int hidden, int inter, int in_dtype) {
    if (inter % kBigGuRows != 0 || hidden % kBigDnRows != 0) return false;
    const int nkg = hidden / kKB, nkd = inter / kKB;
    return (nkg == 56 || nkg == 16 || nkg == 8) && (nkd == 16 || nkd == 8 || nkd == 4) &&
           (in_dtype == CX_DTYPE_BF16 || in_dtype == CX_DTYPE_FP16);
}

bool big_ok(const ExpertLaunch& L) {
    return L.table != nullptr && big_shape_ok(L.hidden, L.inter, L.in_dtype);
}

hipError_t launch_gate_up_big(const ExpertLaunch& L, hipStream_t s) {
    if (!big_ok(L)) return hipErrorInvalidValue;
    const dim3 grid = big_grid(L.max_items, L.inter / kBigGuRows), block(512);
    const bool f16 = L.in_dtype == CX_DTYPE_FP16;
    switch (L.hidden / kKB) {
        case 56: f16 ? cx_launch((k_gu_big<56, true>), grid, block, 0, s, L) : cx_launch((k_gu_big<56, false>), grid, block, 0, s, L); break;
        case 16: f16 ? cx_launch((k_gu_big<16, true>), grid, block, 0, s, L) : cx_launch((k_gu_big<16, false>), grid, block, 0, s, L); break;
        default: f16 ? cx_launch((k_gu_big<8, true>), grid, block, 0, s, L) : cx_launch((k_gu_big<8, false>), grid, block, 0, s, L); break;
    }
    return hipGetLastError();
}

hipError_t launch_down_big(const ExpertLaunch& L, hipStream_t s) {
    if (!big_ok(L)) return hipErrorInvalidValue;
    const dim3 grid = big_grid(L.max_items, L.hidden / kBigDnRows), block(512);
    switch (L.inter / kKB) {
        case 16: cx_launch((k_dn_big<16>), grid, block, 0, s, L); break;
        case 8: cx_launch((k_dn_big<8>), grid, block, 0, s, L); break;
        default: cx_launch((k_dn_big<4>), grid, block, 0, s, L); break;
    }
    return hipGetLastError();
}

// Single mode at 1..4 tokens with 128-column k-blocks that split evenly into
// 2 k-parts (gate/up) and 4 k ranges (down).  The launchers also need
// L.gu_part (2 k-parts).
bool expert_small_ok(const ExpertLaunch& L) {
    if (L.table != nullptr || L.maxt != 1 || L.n_tokens < 1 || L.n_tokens > kDownKsRows) return false;
    if (L.hidden % (kDownKsGroups * kTileRows) != 0) return false;
    const int nkg = L.hidden / kKB, nkd = L.inter / kKB;
    return (nkg == 56 || nkg == 8 || nkg == 4) && (nkd == 16 || nkd == 4);
}

namespace {

template <int NKB, int KSA, bool F16>
void go_gate_up_kpart(const ExpertLaunch& L, hipStream_t s) {
    const dim3 grid(L.inter / kTileRows, 2), block(512);
    if (L.np_lds >= L.n_tokens) {
        cx_launch((k_gate_up_kpart<NKB, KSA, F16, true>), grid, block,
                  gate_up_lds_bytes(KSA, 1, L.np_lds, L.hidden), s, L);
    } else {
        cx_launch((k_gate_up_kpart<NKB, KSA, F16, false>), grid, block,
                  gate_up_lds_bytes(KSA, 1, 0, L.hidden), s, L);
    }
}

template <bool F16>
void pick_gate_up_kpart(const ExpertLaunch& L, hipStream_t s) {
    switch (L.hidden / kKB) {
        case 56: go_gate_up_kpart<4, 7, F16>(L, s); break;  // 2 x 7 waves x 4 k-blocks
        case 8: go_gate_up_kpart<1, 4, F16>(L, s); break;
        default: go_gate_up_kpart<1, 2, F16>(L, s); break;  // 4 k-blocks
    }
}

bool small_args_ok(const ExpertLaunch& L) {
    return expert_small_ok(L) && L.gu_part != nullptr && L.gu_kparts == 2;
}

}  // namespace

hipError_t launch_gate_up_kpart(const ExpertLaunch& L, hipStream_t s) {
    if (!small_args_ok(L)) return hipErrorInvalidValue;
    if (L.in_dtype == CX_DTYPE_FP16) pick_gate_up_kpart<true>(L, s);
    else pick_gate_up_kpart<false>(L, s);
    return hipGetLastError();
}

hipError_t launch_down_ks(const ExpertLaunch& L, hipStream_t s) {
    if (!small_args_ok(L)) return hipErrorInvalidValue;
    const dim3 grid(L.hidden / (kDownKsGroups * kTileRows)), block(512);
    if (L.inter / kKB == 16) cx_launch((k_down_ks<4>), grid, block, down_ks_lds(4), s, L);
    else cx_launch((k_down_ks<1>), grid, block, down_ks_lds(1), s, L);
    return hipGetLastError();
}

// Ring depth of the one-token down + combine: 8 k-blocks (16 KB) in flight
// per wave within 128 registers (two 8-wave workgroups per CU).
constexpr int kDc1Depth = 8;

size_t down_comb1_lds(int inter) {
    switch (inter / kKB) {
        case 16: return Dc1Geom<16>::kLds;
        case 8: return Dc1Geom<8>::kLds;
        case 4: return Dc1Geom<4>::kLds;
        default: return 0;
    }
}

bool down_comb1_ok(int hidden, int inter, int top_k, int max_lds) {
    const size_t lds = inter % kKB == 0 ? down_comb1_lds(inter) : 0;
    return lds > 0 && hidden % kTileRows == 0 && top_k >= 0 && top_k <= kDc1Waves &&
           (size_t)max_lds >= lds;
}

// Rows per one-token down workgroup.  Two workgroups share a CU, and the
// launch lasts as long as the CUs that stream the most rows: at hidden 7168
// on 256 CUs, 448 tiles of 16 rows put two on 24 of the 32 CUs of each XCD
// (32 rows) and one on the rest, while 512 tiles of 14 rows give every CU
// two (28 rows).  Measured: 448 and 384 tiles of 16 rows take the same time,
// 256 take 64 % of it.  14 is taken when it divides hidden and lowers the
// busiest CU's rows.
int down_comb1_rows(int hidden, int n_cu) {
    auto busiest = [&](int r) { const int n = hidden / r; return (n + n_cu - 1) / n_cu * r; };
    if (n_cu > 0 && hidden % 14 == 0 && busiest(14) < busiest(kTileRows)) return 14;
    return kTileRows;
}

hipError_t launch_down_comb1(const ExpertLaunch& L, const int* token_pairs, const float* topk_w,
                             int top_k, int n_cu, hipStream_t s) {
    if (L.table == nullptr || L.n_tokens != 1 || !down_comb1_ok(L.hidden, L.inter, top_k, L.max_lds))
        return hipErrorInvalidValue;
    const int rows = down_comb1_rows(L.hidden, n_cu);
    const dim3 grid(L.hidden / rows), block(64 * kDc1Waves);
    const size_t lds = down_comb1_lds(L.inter);
    switch (L.inter / kKB) {
        case 16: cx_launch((k_down_comb1<16, kDc1Depth>), grid, block, lds, s, L, token_pairs, topk_w, top_k, rows); break;
        case 8: cx_launch((k_down_comb1<8, kDc1Depth>), grid, block, lds, s, L, token_pairs, topk_w, top_k, rows); break;
        default: cx_launch((k_down_comb1<4, 4>), grid, block, lds, s, L, token_pairs, topk_w, top_k, rows); break;
    }
    return hipGetLastError();
}

hipError_t launch_combine(const PlanPtrs& plan, const float* y_part, int n_tokens, int top_k,
                          int hidden, void* y, int out_dtype, float* y_f32, hipStream_t s) {
    const int n = n_tokens * (hidden / 4);
    cx_launch(k_combine, dim3((n + 255) / 256), dim3(256), 0, s, plan, y_part,
                       n_tokens, top_k, hidden, y, out_dtype, y_f32);
    return hipGetLastError();
}

hipError_t launch_combine_dec(const PlanPtrs& plan, const float* topk_w, const float* y_part,
                              int n_tokens, int top_k, int has_shared, int hidden, void* y,
                              int out_dtype, float* y_f32, hipStream_t s) {
    const int n = n_tokens * (hidden / 4);
    cx_launch(k_combine_dec, dim3((n + 255) / 256), dim3(256), 0, s, plan.token_pairs, topk_w,
              y_part, n_tokens, top_k, has_shared, hidden, y, out_dtype, y_f32);
    return hipGetLastError();
}

hipError_t launch_generic_expert(const cx_expert_desc& e, const void* x, int in_dtype,
                                 int n_tokens, float* h_scratch, void* y, int out_dtype,
                                 float* y_f32, hipStream_t s) {
    const int n1 = n_tokens * e.inter, n2 = n_tokens * e.hidden;
    cx_launch(k_generic_gate_up, dim3((n1 + 127) / 128), dim3(128), 0, s, e, x,
                       in_dtype, n_tokens, h_scratch);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    cx_launch(k_generic_down, dim3((n2 + 127) / 128), dim3(128), 0, s, e, h_scratch,
                       n_tokens, y, out_dtype, y_f32);
    return hipGetLastError();
}

}  // namespace cx
