// cx_route.hip — DeepSeek-V3 router, the grouped-execution planners, and the
// decode-pipeline stages that run the shared expert beside them.
//
// Router semantics: route_token_real (server/moe_layer_runtime.py:232-408);
// the HF twin is MoEGate.forward (tmp/patched_modeling/
// modeling_deepseek_eager.py:428-540).  Logits accumulate exact products in
// fp64 and the whole selection runs in fp64, so the chosen expert sets equal
// the exact-math decision; ties break toward the lower index.
//
// Launch shapes
//  * cx_route / general path: k_route_logits (one workgroup per expert row
//    streams W_r once for up to 16 tokens; k_route_logits_mfma on the fp64
//    matrix cores from 32 tokens up), then k_route_select_small
//    (T <= 16, one workgroup) or k_route_select (4 tokens per workgroup),
//    then, for the grouped MoE, k_plan.
//  * decode pipeline (T <= 16, E <= 256):
//      stage 1  k_dec_logits        router logits
//      stage 2  k_dec_select_sgu    selection + planner (workgroup 0) |
//                                   shared expert gate/up tiles
//    or, with routes given (cx_moe_decode),
//      stage 2' k_dec_plan_sgu      planner (workgroup 0) | shared gate/up.
//    The selection and planner are a latency-bound single workgroup; the
//    shared expert's gate/up (29 MB of weights) streams from HBM on the
//    otherwise idle CUs meanwhile (its down projection joins the routed
//    experts' down launch).
#include <atomic>
#include <algorithm>

#include "cx_down.h"
#include "cx_gate_up.h"

namespace cx {
namespace {

constexpr int kRouteThreads = 256;
constexpr int kRouteTB = 16;        // tokens per row workgroup
constexpr int kMaxRouteExperts = 1024;
constexpr int kDecMaxExperts = 256;  // decode planner: one thread per expert
constexpr int kDecThreads = 1024;    // stage-2 workgroup: 16 selection waves
constexpr int kDecSplitMaxTokens = 8;  // the k-part split stage 2 has 8 selection waves

__device__ __forceinline__ bool better(double a, int ia, double b, int ib) {
    return a > b || (a == b && ia < ib);
}

// Raw 8-element chunk of bf16 (one dwordx4) or fp32 (two dwordx4) values,
// widened to fp64 at use (products of bf16 or fp32 values are exact in fp64).
template <bool F32>
struct Chunk8 {
    u32x4 a, b;
    __device__ __forceinline__ void load(const void* base, size_t elem) {
        if (F32) {
            const float* p = static_cast<const float*>(base) + elem;
            a = ld16(p);
            b = ld16(p + 4);
        } else {
            a = ld16(static_cast<const uint16_t*>(base) + elem);
        }
    }
    __device__ __forceinline__ double get(int i) const {
        if (F32) return static_cast<double>(__uint_as_float(i < 4 ? a[i] : b[i - 4]));
        const uint32_t w = a[i >> 1];
        return static_cast<double>(__uint_as_float((i & 1) ? (w & 0xFFFF0000u) : (w << 16)));
    }
};

// logits[t][e] for one expert row e = blockIdx.x and tokens [t0, t0+nt):
// thread i accumulates 8-element chunks i, i+256, ... in fp64, then a fixed
// shuffle tree per wave and a fixed-order sum over the 4 waves.  All W loads
// of a pass are issued before any FMA, and activations are fetched for 4
// tokens at a time (one L2 round trip per group of tokens).
template <bool XF32, bool WF32>
__device__ __forceinline__ void row_logits(const void* __restrict__ x, const void* __restrict__ w, int t0, int nt,
                           int hidden, int n_experts, double* __restrict__ logits,
                           double* red /* [4][kRouteTB] */) {
    const int e = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    double acc[kRouteTB];
#pragma unroll
    for (int t = 0; t < kRouteTB; ++t) acc[t] = 0.0;
    const int nchunk = hidden / 8;
    constexpr int G = 4;
    for (int c0 = 0; c0 < nchunk; c0 += G * kRouteThreads) {
        Chunk8<WF32> wc[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const int ci = c0 + j * kRouteThreads + tid;
            if (ci < nchunk) wc[j].load(w, (size_t)e * hidden + (size_t)ci * 8);
        }
#pragma unroll
        for (int tg = 0; tg < kRouteTB / 4; ++tg) {
            if (tg * 4 < nt) {
                Chunk8<XF32> xc[4][G];
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {
                    if (tg * 4 + tt < nt) {
#pragma unroll
                        for (int j = 0; j < G; ++j) {
                            const int ci = c0 + j * kRouteThreads + tid;
                            if (ci < nchunk)
                                xc[tt][j].load(x, (size_t)(t0 + tg * 4 + tt) * hidden + (size_t)ci * 8);
                        }
                    }
                }
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {
                    if (tg * 4 + tt < nt) {
#pragma unroll
                        for (int j = 0; j < G; ++j) {
                            const int ci = c0 + j * kRouteThreads + tid;
                            if (ci < nchunk) {
#pragma unroll
                                for (int i = 0; i < 8; ++i)
                                    acc[tg * 4 + tt] = fma(wc[j].get(i), xc[tt][j].get(i), acc[tg * 4 + tt]);
                            }
                        }
                    }
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < kRouteTB; ++t) {
        if (t < nt) {
            double v = acc[t];
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
            if (lane == 0) red[wave * kRouteTB + t] = v;
        }
    }
    __syncthreads();
    if (tid < nt) {
        const double v = ((red[tid] + red[kRouteTB + tid]) + red[2 * kRouteTB + tid]) +
                         red[3 * kRouteTB + tid];
        logits[(size_t)(t0 + tid) * n_experts + e] = v;
    }
}

// Decode form of row_logits: expert row e, tokens [t0, t0 + nt), nt <= 4,
// with the accumulators and the raw activation chunks of one pass held in
// few registers (the kernel shares its register budget with the shared
// expert's gate/up tiles).  bf16 weights: the product of two bf16 values is
// exact in fp32, so acc + (double)(w*x) rounds exactly like fma(w, x, acc)
// in fp64; fp32 weights use the fp64 fma.  Same fixed summation order.
__device__ __forceinline__ float bf16_at(u32x4 v, int i) {
    const uint32_t w = v[i >> 1];
    return __uint_as_float((i & 1) ? (w & 0xFFFF0000u) : (w << 16));
}

template <bool WF32, int NT>
__device__ __forceinline__ void row_logits4(const void* __restrict__ x, const void* __restrict__ w,
                                            int e, int t0, int nt, int hidden, int n_experts,
                                            double* __restrict__ logits,
                                            double* red /* [NT/64][4] */) {
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    const int nchunk = hidden / 8;
    constexpr int G = NT >= 512 ? 2 : 4;
    for (int c0 = 0; c0 < nchunk; c0 += G * NT) {
        u32x4 wr[G][WF32 ? 2 : 1];
        u32x4 xr[4][G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const int ci = c0 + j * NT + tid;
            if (ci < nchunk) {
                if (WF32) {
                    const float* p = static_cast<const float*>(w) + (size_t)e * hidden + (size_t)ci * 8;
                    wr[j][0] = ld16(p);
                    wr[j][WF32 ? 1 : 0] = ld16(p + 4);
                } else {
                    wr[j][0] = ld16(static_cast<const uint16_t*>(w) + (size_t)e * hidden + (size_t)ci * 8);
                }
            }
        }
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const int ci = c0 + j * NT + tid;
                if (tt < nt && ci < nchunk)
                    xr[tt][j] = ld16(static_cast<const uint16_t*>(x) + (size_t)(t0 + tt) * hidden + (size_t)ci * 8);
            }
        }
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const int ci = c0 + j * NT + tid;
                if (tt < nt && ci < nchunk) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const float wf = WF32 ? __uint_as_float(wr[j][WF32 ? (i >> 2) : 0][i & 3])
                                              : bf16_at(wr[j][0], i);
                        const float xf = bf16_at(xr[tt][j], i);
                        if (WF32) acc[tt] = fma(static_cast<double>(wf), static_cast<double>(xf), acc[tt]);
                        else acc[tt] = acc[tt] + static_cast<double>(wf * xf);
                    }
                }
                // bounded live ranges: one chunk's conversions at a time
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if (t < nt) {
            double v = acc[t];
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
            if (lane == 0) red[wave * 4 + t] = v;
        }
    }
    __syncthreads();
    if (tid < nt) {
        double v = red[tid];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) v += red[w2 * 4 + tid];
        logits[(size_t)(t0 + tid) * n_experts + e] = v;
    }
}

// Selection for one token by one wave.  c / taken are this wave's LDS
// scratch of n_experts entries (any expert count; the fallback).
__device__ __forceinline__ void select_token(const double* __restrict__ lrow, const float* __restrict__ bias,
                             const uint8_t* __restrict__ resident, int n_experts, int n_group,
                             int topk_group, int top_k, int norm, float scale,
                             int32_t* __restrict__ ids, float* __restrict__ wout, double* c,
                             double* s, uint8_t* gsel) {
    const int lane = threadIdx.x & 63;
    const int epg = n_experts / n_group;
    int nres = 0;
    for (int e = lane; e < n_experts; e += 64) {
        const double sg = 1.0 / (1.0 + exp(-lrow[e]));
        const bool res = resident == nullptr || resident[e] != 0;
        s[e] = res ? sg : 0.0;
        c[e] = res ? sg + static_cast<double>(bias[e]) : -INFINITY;
        nres += res ? 1 : 0;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) nres += __shfl_xor(nres, off, 64);
    __builtin_amdgcn_wave_barrier();
    // group score = sum of the top-2 choice scores of the group
    double gs = -INFINITY;
    if (lane < n_group) {
        int i1 = -1, i2 = -1;
        for (int j = lane * epg; j < (lane + 1) * epg; ++j) {
            if (i1 < 0 || better(c[j], j, c[i1], i1)) { i2 = i1; i1 = j; }
            else if (i2 < 0 || better(c[j], j, c[i2], i2)) { i2 = j; }
        }
        gs = epg >= 2 ? c[i1] + c[i2] : c[i1];
    }
    // keep topk_group groups: rank of each group among all groups
    int rank = 0;
    for (int g2 = 0; g2 < n_group; ++g2) {
        const double o = __shfl(gs, g2, 64);
        if (lane < n_group && g2 != lane && better(o, g2, gs, lane)) ++rank;
    }
    if (lane < n_group) gsel[lane] = rank < topk_group ? 1 : 0;
    __builtin_amdgcn_wave_barrier();
    // candidates outside the kept groups become -inf
    for (int e = lane; e < n_experts; e += 64)
        if (!gsel[e / epg]) c[e] = -INFINITY;
    __builtin_amdgcn_wave_barrier();
    const int k = min(top_k, nres);
    double wsum = 0.0;
    double wsel = 0.0;   // lane r keeps the weight of pick r
    int isel = -1;
    for (int r = 0; r < k; ++r) {
        double bv = -INFINITY;
        int bi = -1;
        for (int e = lane; e < n_experts; e += 64) {
            if (c[e] == c[e] && (bi < 0 || better(c[e], e, bv, bi))) {
                // taken experts are marked with NaN below
                bv = c[e];
                bi = e;
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const double ov = __shfl_xor(bv, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            if (oi >= 0 && (bi < 0 || better(ov, oi, bv, bi))) { bv = ov; bi = oi; }
        }
        if (lane == r) { isel = bi; wsel = s[bi]; }
        wsum += s[bi];
        if (lane == (bi & 63)) c[bi] = __builtin_nan("");
        __builtin_amdgcn_wave_barrier();
    }
    // normalise in pick order on every lane (same fixed order as the oracle)
    const double d = wsum + 1e-20;
    if (lane < top_k) {
        if (lane < k) {
            double v = wsel;
            if (norm && k > 1) v /= d;
            v *= static_cast<double>(scale);
            ids[lane] = isel;
            wout[lane] = static_cast<float>(v);
        } else {
            ids[lane] = -1;
            wout[lane] = 0.0f;
        }
    }
}

// ---------------------------------------------------------------------------
// Register-resident selection (one wave per token): lane l owns the EPL
// consecutive experts [l*EPL, (l+1)*EPL); a group of epg experts is a
// segment of LPG = epg/EPL lanes (a power of two <= 16, so a group never
// crosses a 16-lane DPP row).  Same decisions, tie rules and fixed
// summation order as select_token.  Cross-lane steps use DPP moves
// (row_shr, row_bcast) instead of ds_bpermute shuffles.
struct Top2 {
    double v1, v2;
    int i1, i2;
};

__device__ __forceinline__ Top2 merge2(Top2 a, Top2 b) {
    Top2 r;
    if (better(a.v1, a.i1, b.v1, b.i1)) {
        r.v1 = a.v1; r.i1 = a.i1;
        if (better(a.v2, a.i2, b.v1, b.i1)) { r.v2 = a.v2; r.i2 = a.i2; }
        else { r.v2 = b.v1; r.i2 = b.i1; }
    } else {
        r.v1 = b.v1; r.i1 = b.i1;
        if (better(a.v1, a.i1, b.v2, b.i2)) { r.v2 = a.v1; r.i2 = a.i1; }
        else { r.v2 = b.v2; r.i2 = b.i2; }
    }
    return r;
}

constexpr int kNoIdx = 0x7FFFFFFF;  // placeholder index: loses every tie

// DPP move of a lane's value from the lane selected by CTRL; lanes without a
// valid source (or masked by RM/BM) get their own value back.
template <int CTRL, int RM, int BM>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, RM, BM, false);
}

template <int CTRL, int RM, int BM>
__device__ __forceinline__ double dpp_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = dpp_i<CTRL, RM, BM>(static_cast<int>(b));
    const int hi = dpp_i<CTRL, RM, BM>(static_cast<int>(b >> 32));
    return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo));
}

template <int CTRL, int RM, int BM>
__device__ __forceinline__ void argmax_step(double& v, int& i) {
    const double ov = dpp_d<CTRL, RM, BM>(v);
    const int oi = dpp_i<CTRL, RM, BM>(i);
    if (better(ov, oi, v, i)) { v = ov; i = oi; }
}

// Arg-max (value desc, index asc) over the wave; the result is returned as
// wave-uniform values.  row_shr 1/2/4/8 reduce each 16-lane row into its lane
// 15, row_bcast:15 / row_bcast:31 fold the rows into lane 63.
__device__ __forceinline__ void wave_argmax(double& v, int& i) {
    argmax_step<0x111, 0xF, 0xF>(v, i);
    argmax_step<0x112, 0xF, 0xF>(v, i);
    argmax_step<0x114, 0xF, 0xF>(v, i);
    argmax_step<0x118, 0xF, 0xF>(v, i);
    argmax_step<0x142, 0xA, 0xF>(v, i);
    argmax_step<0x143, 0xC, 0xF>(v, i);
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane(static_cast<int>(b), 63);
    const int hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), 63);
    v = __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo));
    i = __builtin_amdgcn_readlane(i, 63);
}

// Segmented top-2 merge from the lane `s` below, kept only inside the group.
template <int CTRL>
__device__ __forceinline__ void top2_step(Top2& t, bool same_group) {
    Top2 o;
    o.v1 = dpp_d<CTRL, 0xF, 0xF>(t.v1);
    o.v2 = dpp_d<CTRL, 0xF, 0xF>(t.v2);
    o.i1 = dpp_i<CTRL, 0xF, 0xF>(t.i1);
    o.i2 = dpp_i<CTRL, 0xF, 0xF>(t.i2);
    if (same_group) t = merge2(t, o);
}

__device__ __forceinline__ double readlane_d(double v, int lane) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane(static_cast<int>(b), lane);
    const int hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), lane);
    return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo));
}

// Sigmoid score s and choice score c of one expert for one token, the
// reference's steps (moe_layer_runtime.py:323-341): s = sigmoid(logit),
// c = s + e_score_correction_bias; a non-resident expert gets c = -inf and
// s = 0.
__device__ __forceinline__ void expert_scores(double logit, float bias, bool res, double* s,
                                              double* c) {
    const double sg = 1.0 / (1.0 + exp(-logit));
    *s = res ? sg : 0.0;
    *c = res ? sg + static_cast<double>(bias) : -INFINITY;
}

// Inputs of one token's selection, held by its wave (EPL experts per lane),
// and the number of resident experts.
template <int EPL>
struct SelIn {
    double s[EPL], c[EPL];
    int nres;
};

template <int EPL>
__device__ __forceinline__ void sel_load(SelIn<EPL>& in, const double* __restrict__ lrow,
                                         const float* __restrict__ bias,
                                         const uint8_t* __restrict__ resident) {
    const int base = (threadIdx.x & 63) * EPL;
    in.nres = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const bool res = resident == nullptr || resident[base + i] != 0;
        expert_scores(lrow[base + i], bias[base + i], res, &in.s[i], &in.c[i]);
        in.nres += __popcll(__ballot(res));
    }
}

// From scores already in LDS (row of E doubles each) and the residency count.
template <int EPL>
__device__ __forceinline__ void sel_load_lds(SelIn<EPL>& in, const double* s_row, const double* c_row,
                                             int nres) {
    const int base = (threadIdx.x & 63) * EPL;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        in.s[i] = s_row[base + i];
        in.c[i] = c_row[base + i];
    }
    in.nres = nres;
}

// Lane r < kk holds pick r of the token (expert, final weight);
// kk = min(top_k, #resident).
struct SelOut {
    int isel;
    float w;
    int kk;
};

// Sigmoid scores, choice scores and the group stage (top-2 sum per group,
// topk_group groups kept; candidates of the other groups become -inf), exact
// in fp64.  Shared by the exact and the fast top-k stages.
template <int EPL>
struct SelState {
    double s[EPL], c[EPL];
    int nres;
};

template <int EPL>
__device__ __forceinline__ SelState<EPL> sel_groups(const SelIn<EPL>& in, int n_experts,
                                                    int n_group, int topk_group) {
    const int lane = threadIdx.x & 63;
    const int base = lane * EPL;
    const int epg = n_experts / n_group;
    const int lpg = epg / EPL;  // lanes per group: power of two <= 16 (host-checked)
    SelState<EPL> st;
    st.nres = in.nres;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        st.s[i] = in.s[i];
        st.c[i] = in.c[i];
    }
    // group score: top-2 sum over the group's lane segment, complete in the
    // segment's last lane
    Top2 t{-INFINITY, -INFINITY, kNoIdx, kNoIdx};
#pragma unroll
    for (int i = 0; i < EPL; ++i) t = merge2(t, Top2{st.c[i], -INFINITY, base + i, kNoIdx});
    const int sub = lane & (lpg - 1);
    if (lpg > 1) top2_step<0x111>(t, sub >= 1);
    if (lpg > 2) top2_step<0x112>(t, sub >= 2);
    if (lpg > 4) top2_step<0x114>(t, sub >= 4);
    if (lpg > 8) top2_step<0x118>(t, sub >= 8);
    const double gs_lane = epg >= 2 ? t.v1 + t.v2 : t.v1;
    const int grp = base / epg;
    // the full group scores sit in each segment's last lane: this lane's own
    // by one cross-lane read, the others as uniform values; rank this lane's
    // group among them
    const int src = grp * lpg + lpg - 1;
    const long long gb = __double_as_longlong(gs_lane);
    const int glo = __shfl(static_cast<int>(gb), src, 64), ghi = __shfl(static_cast<int>(gb >> 32), src, 64);
    const double my_gs = __longlong_as_double((static_cast<long long>(ghi) << 32) | static_cast<unsigned>(glo));
    int rank = 0;
    for (int g2 = 0; g2 < n_group; ++g2) {
        const double o = readlane_d(gs_lane, g2 * lpg + lpg - 1);
        if (g2 != grp && better(o, g2, my_gs, grp)) ++rank;
    }
    if (rank >= topk_group) {
#pragma unroll
        for (int i = 0; i < EPL; ++i) st.c[i] = -INFINITY;
    }
    return st;
}

template <int EPL>
__device__ __forceinline__ SelOut select_reg(const SelIn<EPL>& in, int n_experts, int n_group,
                                             int topk_group, int top_k, int norm, float scale) {
    const int lane = threadIdx.x & 63;
    const int base = lane * EPL;
    SelState<EPL> st = sel_groups<EPL>(in, n_experts, n_group, topk_group);
    double* s = st.s;
    double* c = st.c;
    const int nres = st.nres;
    const int k = min(top_k, nres);
    unsigned taken = 0;
    double wsum = 0.0, wsel = 0.0;
    int isel = -1;
    for (int r = 0; r < k; ++r) {
        double bv = -INFINITY;
        int bi = kNoIdx;
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            if (!((taken >> i) & 1u) && better(c[i], base + i, bv, bi)) {
                bv = c[i];
                bi = base + i;
            }
        }
        wave_argmax(bv, bi);
        // s of the pick lives in its owner lane
        const int owner = bi / EPL;
        double sv = 0.0;
#pragma unroll
        for (int i = 0; i < EPL; ++i)
            if (bi == base + i) sv = s[i];
        sv = readlane_d(sv, owner);
        if (owner == lane) taken |= 1u << (bi - base);
        if (lane == r) { isel = bi; wsel = sv; }
        wsum += sv;
    }
    // normalise in pick order on every lane (same fixed order as the oracle)
    const double d = wsum + 1e-20;
    double v = wsel;
    if (norm && k > 1) v /= d;
    v *= static_cast<double>(scale);
    return SelOut{isel, static_cast<float>(v), k};
}

// Fast top-k stage on 32-bit keys.  After the group stage (exact fp64, as in
// select_reg), each candidate's choice score is rounded to fp32 and mapped to
// a monotonic unsigned key; rounding to nearest is monotonic, so a strict key
// order is the fp64 order.  Each pick is a wave max of keys (DPP max chain,
// one instruction per step) and a ballot for the owner.  If any pick finds
// two candidates with its key (an fp32-level tie, or equal -inf scores), the
// function returns false and the caller runs the exact fp64 selection, so
// the decisions are always those of select_reg.
__device__ __forceinline__ uint32_t fkey(double c) {
    const uint32_t b = __float_as_uint(static_cast<float>(c));
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

template <int CTRL, int RM>
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v) {
    const uint32_t o = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), CTRL, RM, 0xF, false));
    return v > o ? v : o;
}

template <int EPL>
__device__ __forceinline__ bool select_fast(const SelIn<EPL>& in, int n_experts, int n_group,
                                            int topk_group, int top_k, int norm, float scale,
                                            SelOut* out) {
    const int lane = threadIdx.x & 63;
    const SelState<EPL> st = sel_groups<EPL>(in, n_experts, n_group, topk_group);
    const double* s = st.s;
    const int nres = st.nres;
    uint32_t key[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) key[i] = fkey(st.c[i]);
    const int k = min(top_k, nres);
    double wsum = 0.0, wsel = 0.0;
    int isel = -1;
    for (int r = 0; r < k; ++r) {
        uint32_t m = key[0];
#pragma unroll
        for (int i = 1; i < EPL; ++i) m = key[i] > m ? key[i] : m;
        m = dpp_max_u32<0x111, 0xF>(m);
        m = dpp_max_u32<0x112, 0xF>(m);
        m = dpp_max_u32<0x114, 0xF>(m);
        m = dpp_max_u32<0x118, 0xF>(m);
        m = dpp_max_u32<0x142, 0xA>(m);
        m = dpp_max_u32<0x143, 0xC>(m);
        const uint32_t M = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m), 63));
        int hits = 0, owner = -1, slot = 0;
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const unsigned long long b = __ballot(key[i] == M);
            hits += __popcll(b);
            if (b != 0ull) {
                owner = __builtin_ctzll(b);
                slot = i;
            }
        }
        if (hits != 1) return false;  // key tie: exact path decides
        const int bi = owner * EPL + slot;
        double sv = 0.0;
#pragma unroll
        for (int i = 0; i < EPL; ++i)
            if (i == slot) sv = s[i];
        sv = readlane_d(sv, owner);
        if (lane == owner) {
#pragma unroll
            for (int i = 0; i < EPL; ++i)
                if (i == slot) key[i] = 0u;  // taken: below every score key
        }
        if (lane == r) { isel = bi; wsel = sv; }
        wsum += sv;
    }
    const double d = wsum + 1e-20;
    double v = wsel;
    if (norm && k > 1) v /= d;
    v *= static_cast<double>(scale);
    *out = SelOut{isel, static_cast<float>(v), k};
    return true;
}

template <int EPL>
__device__ __forceinline__ SelOut select_any_reg(const SelIn<EPL>& in, int n_experts, int n_group,
                                                 int topk_group, int top_k, int norm, float scale) {
    SelOut o;
    if (!select_fast<EPL>(in, n_experts, n_group, topk_group, top_k, norm, scale, &o))
        o = select_reg<EPL>(in, n_experts, n_group, topk_group, top_k, norm, scale);
    return o;
}

__device__ __forceinline__ void write_sel(const SelOut& o, int top_k, int32_t* ids, float* wout) {
    const int lane = threadIdx.x & 63;
    if (lane < top_k) {
        ids[lane] = lane < o.kk ? o.isel : -1;
        wout[lane] = lane < o.kk ? o.w : 0.0f;
    }
}

template <int EPL>
__device__ __forceinline__ void select_token_reg(const double* lrow, const float* bias, const uint8_t* resident,
                                 int n_experts, int n_group, int topk_group, int top_k, int norm,
                                 float scale, int32_t* ids, float* wout) {
    SelIn<EPL> in;
    sel_load<EPL>(in, lrow, bias, resident);
    write_sel(select_any_reg<EPL>(in, n_experts, n_group, topk_group, top_k, norm, scale), top_k, ids,
              wout);
}

// Dispatch on experts per lane; fallback = the LDS version.
__device__ __forceinline__ void select_any(const double* lrow, const float* bias, const uint8_t* resident,
                           int n_experts, int n_group, int topk_group, int top_k, int norm,
                           float scale, int32_t* ids, float* wout, int epl, double* c, double* s,
                           uint8_t* gsel) {
    switch (epl) {
        case 1: select_token_reg<1>(lrow, bias, resident, n_experts, n_group, topk_group, top_k, norm, scale, ids, wout); return;
        case 2: select_token_reg<2>(lrow, bias, resident, n_experts, n_group, topk_group, top_k, norm, scale, ids, wout); return;
        case 4: select_token_reg<4>(lrow, bias, resident, n_experts, n_group, topk_group, top_k, norm, scale, ids, wout); return;
        case 8: select_token_reg<8>(lrow, bias, resident, n_experts, n_group, topk_group, top_k, norm, scale, ids, wout); return;
        default:
            select_token(lrow, bias, resident, n_experts, n_group, topk_group, top_k, norm, scale, ids, wout, c, s, gsel);
    }
}

// True when assignment i = (t, k) repeats an expert already listed earlier
// in token t's routes (the reference rejects such routes, validate_routes in
// server/moe_layer_runtime.py:84-98); the repeat is dropped and flagged.
__device__ __forceinline__ bool dup_route(const int32_t* ids, int i, int top_k) {
    const int t0 = (i / top_k) * top_k;
    for (int j = t0; j < i; ++j)
        if (ids[j] == ids[i]) return true;
    return false;
}

// ---------------------------------------------------------------------------
// General planner (one workgroup, any blockDim multiple of 64).  Counting
// sort of the (token, k) assignments by expert id; slots in ascending expert
// id, shared expert last with pairs [0, T); routed pairs from T; items of
// <= item_cap pairs, routed items first.  The order of pairs inside a slot
// only picks an MFMA column, which never changes a value, so the atomic
// cursor keeps the results deterministic.  LDS: 2*E + blockDim ints.
__device__ __forceinline__ int wave_incl_scan(int v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int a = __shfl_up(v, off, 64);
        if (lane >= off) v += a;
    }
    return v;
}

// Exclusive scan over the workgroup (blockDim a multiple of 64, at most
// 4096): a scan inside each wave, the waves' totals scanned by wave 0, three
// barriers in all.  tmp: >= 129 ints.
__device__ __forceinline__ int block_excl_scan(int v, int* tmp, int* total) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, nw = blockDim.x >> 6;
    const int incl = wave_incl_scan(v);
    if (lane == 63) tmp[wv] = incl;
    __syncthreads();
    if (wv == 0) {
        const int t = lane < nw ? tmp[lane] : 0;
        const int ti = wave_incl_scan(t);
        if (lane < nw) tmp[64 + lane] = ti - t;
        if (lane == 63) tmp[128] = ti;
    }
    __syncthreads();
    const int res = incl - v + tmp[64 + wv];
    *total = tmp[128];
    __syncthreads();
    return res;
}

__device__ __forceinline__ void plan_build(const int32_t* __restrict__ ids, const float* __restrict__ w,
                           int n_tokens, int top_k, const cx_expert_desc* table, int n_experts,
                           int has_shared, int item_cap, int max_items, const PlanPtrs& P,
                           int* err_flag, int* sm /* 2E + blockDim */) {
    __shared__ int s_err;
    int* cnt = sm;
    int* cur = sm + n_experts;
    int* scan = sm + 2 * n_experts;
    const int tid = threadIdx.x, nt = blockDim.x;
    if (tid == 0) s_err = 0;
    for (int e = tid; e < n_experts; e += nt) cnt[e] = 0;
    __syncthreads();
    const int n_assign = n_tokens * top_k;
    for (int i = tid; i < n_assign; i += nt) {
        const int e = ids[i];
        if (e < 0) continue;
        if (e >= n_experts) { atomicOr(&s_err, kErrBadExpertId); continue; }
        if (table[e].w_up == nullptr) { atomicOr(&s_err, kErrNotResident); continue; }
        if (dup_route(ids, i, top_k)) { atomicOr(&s_err, kErrDuplicateRoute); continue; }
        if (!route_weight_ok(w[i])) { atomicOr(&s_err, kErrBadWeight); continue; }
        atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    const bool shared = has_shared && table[n_experts].w_up != nullptr;
    const int s0 = shared ? n_tokens : 0;  // first routed pair
    const int chunk = (n_experts + nt - 1) / nt;
    const int e0 = min(tid * chunk, n_experts), e1 = min(e0 + chunk, n_experts);
    int my_pairs = 0, my_slots = 0;
    for (int e = e0; e < e1; ++e) {
        my_pairs += cnt[e];
        my_slots += cnt[e] > 0;
    }
    int tot_pairs = 0, tot_slots = 0;
    int pair_off = s0 + block_excl_scan(my_pairs, scan, &tot_pairs);
    int slot_off = block_excl_scan(my_slots, scan, &tot_slots);
    for (int e = e0; e < e1; ++e) {
        cur[e] = pair_off;
        if (cnt[e] > 0) {
            P.slot_expert[slot_off] = e;
            P.slot_pair_begin[slot_off] = pair_off;
            P.slot_pair_count[slot_off] = cnt[e];
            ++slot_off;
        }
        pair_off += cnt[e];
    }
    __syncthreads();
    for (int i = tid; i < n_assign; i += nt) {
        const int e = ids[i];
        const int t = i / top_k, k = i - t * top_k;
        int pos = -1;
        if (e >= 0 && e < n_experts && table[e].w_up != nullptr && !dup_route(ids, i, top_k) &&
            route_weight_ok(w[i])) {
            pos = atomicAdd(&cur[e], 1);
            P.pair_token[pos] = t;
            P.pair_weight[pos] = w[i];
        }
        P.token_pairs[(size_t)t * (top_k + 1) + k] = pos;
    }
    for (int t = tid; t < n_tokens; t += nt) {
        if (shared) {
            P.pair_token[t] = t;
            P.pair_weight[t] = 1.0f;
        }
        P.token_pairs[(size_t)t * (top_k + 1) + top_k] = shared ? t : -1;
    }
    if (shared && tid == 0) {
        P.slot_expert[tot_slots] = n_experts;
        P.slot_pair_begin[tot_slots] = 0;
        P.slot_pair_count[tot_slots] = n_tokens;
    }
    __syncthreads();
    const int n_slots = tot_slots + (shared ? 1 : 0);
    const int schunk = (n_slots + nt - 1) / nt;
    const int s0s = min(tid * schunk, n_slots), s1s = min(s0s + schunk, n_slots);
    int my_items = 0;
    for (int s = s0s; s < s1s; ++s) my_items += (P.slot_pair_count[s] + item_cap - 1) / item_cap;
    int tot_items = 0;
    int it = block_excl_scan(my_items, scan, &tot_items);
    for (int s = s0s; s < s1s; ++s) {
        const int pb = P.slot_pair_begin[s], pc = P.slot_pair_count[s];
        for (int o = 0; o < pc; o += item_cap) {
            if (it < max_items) {
                P.item_slot[it] = s;
                P.item_pair_begin[it] = pb + o;
                P.item_pair_count[it] = min(item_cap, pc - o);
            }
            ++it;
        }
    }
    // flat records for the expert kernels
    __syncthreads();
    for (int s = tid; s < n_slots; s += nt) {
        const cx_expert_desc& e = table[P.slot_expert[s]];
        P.slot_rec[s] = SlotRec{e.w_down, e.s_down, e.down_rb, 0};
    }
    for (int i = tid; i < min(tot_items, max_items); i += nt) {
        const cx_expert_desc& e = table[P.slot_expert[P.item_slot[i]]];
        const int pb = P.item_pair_begin[i], np = P.item_pair_count[i];
        const int t0 = P.pair_token[pb];
        const int t1 = np > 1 ? P.pair_token[pb + 1] : 0;
        const int t2 = np > 2 ? P.pair_token[pb + 2] : 0;
        const int t3 = np > 3 ? P.pair_token[pb + 3] : 0;
        P.item_rec[i] = ItemRec{e.w_up, e.w_gate, e.w_down, e.s_up, e.s_gate, e.s_down, pb, np,
                                e.up_rb, e.gate_rb, e.down_rb, e.gu_layout, {t0, t1, t2, t3}};
    }
    if (tid == 0) {
        const int shared_items = shared ? (n_tokens + item_cap - 1) / item_cap : 0;
        if (tot_items > max_items) s_err |= kErrPlanOverflow;
        P.hdr->n_slots = n_slots;
        P.hdr->n_items = min(tot_items, max_items);
        P.hdr->n_pairs = s0 + tot_pairs;
        P.hdr->n_routed_slots = tot_slots;
        P.hdr->n_routed_items = min(tot_items - shared_items, max_items);
        if (s_err) atomicOr(err_flag, s_err);
    }
}

constexpr int kPlanThreads = 1024;

// Staged planner: the same plan as plan_build with every input first copied
// into LDS in one round of independent loads (routes, layer table), so the
// passes that follow wait only on LDS and the block barriers.  Routes are
// held as 16-bit expert ids (clamped to [-1, E]; a route found invalid is
// set to -1 once every thread has checked its token's repeats), each
// thread keeping its routes' validity in a 64-bit mask: up to 64 routes per
// thread.  LDS layout: table[E+1] | ids16[n, even] | cnt[E] | cur[E] |
// scan[nt] | slot arrays (expert, first pair, count) [E+1] each.
constexpr int kPlanRoutesPerThread = 64;

size_t plan_staged_lds(int n_assign, int n_experts, int threads) {
    return sizeof(cx_expert_desc) * ((size_t)n_experts + 1) + 2 * (((size_t)n_assign + 1) & ~(size_t)1) +
           sizeof(int) * (2 * (size_t)n_experts + threads + 3 * ((size_t)n_experts + 1));
}

__device__ __forceinline__ void plan_build_staged(const int32_t* __restrict__ ids,
                                                  const float* __restrict__ w, int n_tokens,
                                                  int top_k, const cx_expert_desc* table,
                                                  int n_experts, int has_shared, int item_cap,
                                                  int max_items, const PlanPtrs& P, int* err_flag,
                                                  unsigned char* lds) {
    __shared__ int s_err;
    const int E = n_experts, n_assign = n_tokens * top_k;
    const int tid = threadIdx.x, nt = blockDim.x;
    cx_expert_desc* tab = reinterpret_cast<cx_expert_desc*>(lds);
    int16_t* sid = reinterpret_cast<int16_t*>(tab + E + 1);
    int* cnt = reinterpret_cast<int*>(sid + ((n_assign + 1) & ~1));
    int* cur = cnt + E;
    int* scan = cur + E;
    int* s_exp = scan + nt;
    int* s_pb = s_exp + E + 1;
    int* s_pc = s_pb + E + 1;
    // 1) inputs -> LDS, one round of independent loads
    {
        constexpr int kChunks = sizeof(cx_expert_desc) / 16;
        const u32x4* src = reinterpret_cast<const u32x4*>(table);
        u32x4* dst = reinterpret_cast<u32x4*>(tab);
        for (int i = tid; i < (E + 1) * kChunks; i += nt) dst[i] = ld16(src + i);
        for (int i = tid; i < n_assign; i += nt) sid[i] = (int16_t)max(-1, min(ldi(ids + i), E));
        for (int e = tid; e < E; e += nt) cnt[e] = 0;
        if (tid == 0) s_err = 0;
    }
    __syncthreads();
    // 2) validity (range, residency, repeats within the token) and counts;
    // then invalid routes -> -1
    uint64_t okm = 0;
    for (int i = tid, r = 0; i < n_assign; i += nt, ++r) {
        const int e = sid[i];
        if (e >= 0) {
            if (e >= E) atomicOr(&s_err, kErrBadExpertId);
            else if (tab[e].w_up == nullptr) atomicOr(&s_err, kErrNotResident);
            else {
                bool dup = false;
                for (int j = (i / top_k) * top_k; j < i; ++j) dup |= sid[j] == e;
                if (dup) atomicOr(&s_err, kErrDuplicateRoute);
                else if (!route_weight_ok(ldf(w + i))) atomicOr(&s_err, kErrBadWeight);
                else {
                    okm |= 1ull << r;
                    atomicAdd(&cnt[e], 1);
                }
            }
        }
    }
    __syncthreads();
    for (int i = tid, r = 0; i < n_assign; i += nt, ++r)
        if (!((okm >> r) & 1)) sid[i] = -1;
    __syncthreads();
    // 3) slots in ascending expert id (block scans over per-thread ranges)
    const bool shared = has_shared && tab[E].w_up != nullptr;
    const int s0 = shared ? n_tokens : 0;  // first routed pair
    const int chunk = (E + nt - 1) / nt;
    const int e0 = min(tid * chunk, E), e1 = min(e0 + chunk, E);
    int my_pairs = 0, my_slots = 0;
    for (int e = e0; e < e1; ++e) {
        my_pairs += cnt[e];
        my_slots += cnt[e] > 0;
    }
    int tot_pairs = 0, tot_slots = 0;
    int pair_off = s0 + block_excl_scan(my_pairs, scan, &tot_pairs);
    int slot_off = block_excl_scan(my_slots, scan, &tot_slots);
    for (int e = e0; e < e1; ++e) {
        cur[e] = pair_off;
        if (cnt[e] > 0) {
            s_exp[slot_off] = e;
            s_pb[slot_off] = pair_off;
            s_pc[slot_off] = cnt[e];
            ++slot_off;
        }
        pair_off += cnt[e];
    }
    if (shared && tid == 0) {
        s_exp[tot_slots] = E;
        s_pb[tot_slots] = 0;
        s_pc[tot_slots] = n_tokens;
    }
    __syncthreads();
    // 4) pairs (order inside a slot only picks an MFMA column)
    for (int i = tid; i < n_assign; i += nt) {
        const int t = i / top_k, k = i - t * top_k;
        int pos = -1;
        if (sid[i] >= 0) {
            pos = atomicAdd(&cur[sid[i]], 1);
            P.pair_token[pos] = t;
            P.pair_weight[pos] = w[i];
        }
        P.token_pairs[(size_t)t * (top_k + 1) + k] = pos;
    }
    for (int t = tid; t < n_tokens; t += nt) {
        if (shared) {
            P.pair_token[t] = t;
            P.pair_weight[t] = 1.0f;
        }
        P.token_pairs[(size_t)t * (top_k + 1) + top_k] = shared ? t : -1;
    }
    const int n_slots = tot_slots + (shared ? 1 : 0);
    for (int sl = tid; sl < n_slots; sl += nt) {
        P.slot_expert[sl] = s_exp[sl];
        P.slot_pair_begin[sl] = s_pb[sl];
        P.slot_pair_count[sl] = s_pc[sl];
        const cx_expert_desc& e = tab[s_exp[sl]];
        P.slot_rec[sl] = SlotRec{e.w_down, e.s_down, e.down_rb, 0};
    }
    // 5) items of <= item_cap pairs, routed first, shared last
    const int schunk = (n_slots + nt - 1) / nt;
    const int s0s = min(tid * schunk, n_slots), s1s = min(s0s + schunk, n_slots);
    int my_items = 0;
    for (int sl = s0s; sl < s1s; ++sl) my_items += (s_pc[sl] + item_cap - 1) / item_cap;
    int tot_items = 0;
    // (the scan's barriers also complete this block's pair_token writes)
    int it = block_excl_scan(my_items, scan, &tot_items);
    for (int sl = s0s; sl < s1s; ++sl) {
        const int pb = s_pb[sl], pc = s_pc[sl];
        const cx_expert_desc& e = tab[s_exp[sl]];
        for (int o = 0; o < pc; o += item_cap) {
            if (it < max_items) {
                const int np = min(item_cap, pc - o), q0 = pb + o;
                P.item_slot[it] = sl;
                P.item_pair_begin[it] = q0;
                P.item_pair_count[it] = np;
                const int t0 = P.pair_token[q0];
                const int t1 = np > 1 ? P.pair_token[q0 + 1] : 0;
                const int t2 = np > 2 ? P.pair_token[q0 + 2] : 0;
                const int t3 = np > 3 ? P.pair_token[q0 + 3] : 0;
                P.item_rec[it] = ItemRec{e.w_up, e.w_gate, e.w_down, e.s_up, e.s_gate, e.s_down,
                                         q0, np, e.up_rb, e.gate_rb, e.down_rb, e.gu_layout, {t0, t1, t2, t3}};
            }
            ++it;
        }
    }
    if (tid == 0) {
        const int shared_items = shared ? (n_tokens + item_cap - 1) / item_cap : 0;
        if (tot_items > max_items) s_err |= kErrPlanOverflow;
        P.hdr->n_slots = n_slots;
        P.hdr->n_items = min(tot_items, max_items);
        P.hdr->n_pairs = s0 + tot_pairs;
        P.hdr->n_routed_slots = tot_slots;
        P.hdr->n_routed_items = min(tot_items - shared_items, max_items);
        if (s_err) atomicOr(err_flag, s_err);
    }
}

__global__ __launch_bounds__(kPlanThreads) void k_plan_staged(const int32_t* __restrict__ ids,
                                                              const float* __restrict__ w,
                                                              int n_tokens, int top_k,
                                                              const cx_expert_desc* table,
                                                              int n_experts, int has_shared,
                                                              int item_cap, int max_items,
                                                              PlanPtrs P, int* err_flag) {
    extern __shared__ __attribute__((aligned(16))) unsigned char plds[];
    plan_build_staged(ids, w, n_tokens, top_k, table, n_experts, has_shared, item_cap, max_items,
                      P, err_flag, plds);
}

__global__ __launch_bounds__(kPlanThreads) void k_plan(const int32_t* __restrict__ ids,
                                                       const float* __restrict__ w, int n_tokens,
                                                       int top_k, const cx_expert_desc* table,
                                                       int n_experts, int has_shared, int item_cap,
                                                       int max_items, PlanPtrs P, int* err_flag) {
    extern __shared__ int sm[];
    plan_build(ids, w, n_tokens, top_k, table, n_experts, has_shared, item_cap, max_items, P,
               err_flag, sm);
}

// ---------------------------------------------------------------------------
// Decode planner (T <= 16 tokens, E <= 256 experts, one thread per expert).
// Input: the token x expert selection in LDS (bit e of mask[t] set when
// token t routes to expert e, with its weight wsel[t][e] and top-k position
// ksel[t][e]) and a copy of the layer table.  Output: the same plan layout
// as plan_build, deterministic by construction (no atomics on the order):
// slots in ascending expert id, a slot's pairs in ascending token order
// starting at T (pairs [0, T) are the shared expert's), one item per slot,
// the shared expert's slot and item last, and each pair's y_part row
// (pair_row: t for the shared expert, T + t*K + k for route k of token t).
// Every output cell is written exactly once, and every global input was
// fetched before the selection, so the planner itself only waits on LDS.
struct DecPlanLds {
    cx_expert_desc tab[kDecMaxExperts + 1];
    uint32_t mask[kTileTok][kDecMaxExperts / 32];
    float wsel[kTileTok][kDecMaxExperts];
    uint8_t ksel[kTileTok][kDecMaxExperts];
    int scan[16][2];
    int err;
    int nres_w[16];  // resident experts counted per wave (selection of the decode stage)
};

// Copies table entries [0, E] (entry E = shared expert, zeroed when absent)
// into LDS and clears the selection mask.
__device__ __forceinline__ void dec_plan_prologue(DecPlanLds& S, const cx_expert_desc* table,
                                                  int n_experts) {
    constexpr int kChunks = sizeof(cx_expert_desc) / 16;
    static_assert(sizeof(cx_expert_desc) % 16 == 0, "descriptor is copied in 16-byte chunks");
    const int n = (n_experts + 1) * kChunks;
    const u32x4* src = reinterpret_cast<const u32x4*>(table);
    u32x4* dst = reinterpret_cast<u32x4*>(S.tab);
    for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] = ld16(src + i);
    uint32_t* m = &S.mask[0][0];
    for (int i = threadIdx.x; i < kTileTok * (kDecMaxExperts / 32); i += blockDim.x) m[i] = 0u;
    if (threadIdx.x == 0) S.err = 0;
}

// Inclusive prefix sum over the 64 lanes of a wave by DPP row shifts and row
// broadcasts (no LDS round trips).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xF, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xF, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xF, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xF, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xA, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xC, 0xF, false));
    return v;
}

__device__ __forceinline__ void dec_plan_core(DecPlanLds& S, int T, int K, int E, int has_shared,
                                              const PlanPtrs& P, int* err_flag, int err) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    const int e = tid;
    int cnt = 0;
    if (e < E) {
        for (int t = 0; t < T; ++t) cnt += (S.mask[t][e >> 5] >> (e & 31)) & 1u;
        if (cnt > 0 && S.tab[e].w_up == nullptr) {  // routed to an expert the layer lacks
            err |= kErrNotResident;
            for (int t = 0; t < T; ++t)
                if ((S.mask[t][e >> 5] >> (e & 31)) & 1u)
                    P.token_pairs[(size_t)t * (K + 1) + S.ksel[t][e]] = -1;
            cnt = 0;
        }
    }
    // block-wide exclusive scan of (pairs, slots) in expert order, packed as
    // pairs | slots << 16 (pairs <= 16 * 64, slots <= 256)
    const uint32_t mine = static_cast<uint32_t>(cnt) | (cnt > 0 ? 0x10000u : 0u);
    const uint32_t incl = wave_incl_scan(mine);
    if (lane == 63) S.scan[wave][0] = static_cast<int>(incl);
    __syncthreads();
    uint32_t before = 0, total = 0;
    for (int w = 0; w < nw; ++w) {
        const uint32_t v = static_cast<uint32_t>(S.scan[w][0]);
        before += w < wave ? v : 0u;
        total += v;
    }
    const uint32_t excl = before + incl - mine;
    const int tp = static_cast<int>(total & 0xFFFFu), ts = static_cast<int>(total >> 16);
    const bool shared = has_shared && S.tab[E].w_up != nullptr;
    const int s0 = shared ? T : 0;
    if (cnt > 0) {
        const int first = s0 + static_cast<int>(excl & 0xFFFFu);
        const int slot = static_cast<int>(excl >> 16);
        const cx_expert_desc d = S.tab[e];
        P.slot_expert[slot] = e;
        P.slot_pair_begin[slot] = first;
        P.slot_pair_count[slot] = cnt;
        P.slot_rec[slot] = SlotRec{d.w_down, d.s_down, d.down_rb, 0};
        P.item_slot[slot] = slot;
        P.item_pair_begin[slot] = first;
        P.item_pair_count[slot] = cnt;
        int tk0 = 0, tk1 = 0, tk2 = 0, tk3 = 0;  // first 4 tokens (registers, not a
        int j = 0;                                // dynamically indexed array)
        for (int t = 0; t < T; ++t) {
            if ((S.mask[t][e >> 5] >> (e & 31)) & 1u) {
                tk0 = j == 0 ? t : tk0;
                tk1 = j == 1 ? t : tk1;
                tk2 = j == 2 ? t : tk2;
                tk3 = j == 3 ? t : tk3;
                const int q = first + j++;
                const int k = S.ksel[t][e];
                P.pair_token[q] = t;
                P.pair_weight[q] = S.wsel[t][e];
                P.pair_row[q] = s0 + t * K + k;
                P.token_pairs[(size_t)t * (K + 1) + k] = q;
            }
        }
        P.item_rec[slot] = ItemRec{d.w_up, d.w_gate, d.w_down, d.s_up, d.s_gate, d.s_down, first, cnt,
                                   d.up_rb, d.gate_rb, d.down_rb, d.gu_layout, {tk0, tk1, tk2, tk3}};
    }
    if (shared) {
        if (tid == 0) {
            const cx_expert_desc d = S.tab[E];
            P.slot_expert[ts] = E;
            P.slot_pair_begin[ts] = 0;
            P.slot_pair_count[ts] = T;
            P.slot_rec[ts] = SlotRec{d.w_down, d.s_down, d.down_rb, 0};
            P.item_slot[ts] = ts;
            P.item_pair_begin[ts] = 0;
            P.item_pair_count[ts] = T;
            P.item_rec[ts] = ItemRec{d.w_up, d.w_gate, d.w_down, d.s_up, d.s_gate, d.s_down, 0, T,
                                     d.up_rb, d.gate_rb, d.down_rb, d.gu_layout, {0, 1, 2, 3}};
        }
        if (tid < T) {
            P.pair_token[tid] = tid;
            P.pair_weight[tid] = 1.0f;
            P.pair_row[tid] = tid;
            P.token_pairs[(size_t)tid * (K + 1) + K] = tid;
        }
    } else if (tid < T) {
        P.token_pairs[(size_t)tid * (K + 1) + K] = -1;
    }
    if (err) atomicOr(&S.err, err);
    __syncthreads();
    if (tid == 0) {
        const int ns = ts + (shared ? 1 : 0);
        P.hdr->n_slots = ns;
        P.hdr->n_items = ns;
        P.hdr->n_pairs = s0 + tp;
        P.hdr->n_routed_slots = ts;
        P.hdr->n_routed_items = ts;
        if (S.err) atomicOr(err_flag, S.err);
    }
}

// ---------------------------------------------------------------------------
struct FusedArgs {
    const void* x;
    int x_dtype;
    const void* w;
    int w_dtype;
    const float* bias;
    const uint8_t* resident;
    int n_tokens, hidden, n_experts, n_group, topk_group, top_k, norm;
    float scale;
    double* logits;
    int32_t* ids;
    float* wout;
    int epl;               // experts per lane of the register selection, 0 = LDS fallback
    // planner
    const cx_expert_desc* table;
    int has_shared, item_cap, max_items;
    PlanPtrs plan;
    int* err_flag;
};

FusedArgs fused_args(const RouteArgs& R) {
    FusedArgs A{};
    A.x = R.x;
    A.x_dtype = R.x_dtype;
    A.w = R.w;
    A.w_dtype = R.w_dtype;
    A.bias = R.bias;
    A.resident = R.resident;
    A.n_tokens = R.n_tokens;
    A.hidden = R.hidden;
    A.n_experts = R.n_experts;
    A.n_group = R.n_group;
    A.topk_group = R.topk_group;
    A.top_k = R.top_k;
    A.norm = R.norm;
    A.scale = R.scale;
    A.logits = R.logits;
    A.ids = R.ids;
    A.wout = R.wout;
    if (R.plan != nullptr) {
        A.table = R.table;
        A.has_shared = R.has_shared;
        A.item_cap = R.item_cap;
        A.max_items = R.max_items;
        A.plan = *R.plan;
        A.err_flag = R.err_flag;
    }
    return A;
}

template <bool XF32, bool WF32>
__global__ __launch_bounds__(kRouteThreads) void k_route_logits(FusedArgs A) {
    __shared__ double red[4 * kRouteTB];
    const int t0 = blockIdx.y * kRouteTB;
    row_logits<XF32, WF32>(A.x, A.w, t0, min(kRouteTB, A.n_tokens - t0), A.hidden, A.n_experts,
                           A.logits, red);
}

// Router logits for many tokens on the fp64 matrix cores
// (v_mfma_f64_16x16x4_f64).  Workgroup tile = 16 experts x 32 tokens, the 8
// waves split K and their partial tiles are summed in LDS in a fixed order.
// Products of bf16 (or fp32) values are exact in fp64, so the logits equal
// the sequential fp64 sums of exact products up to fp64 summation order
// (relative 1e-15), far inside the 1e-12 margin below which a selection is
// treated as a tie.  MFMA operand layout: lane (i = lane % 16, g = lane / 16)
// holds A[i][g] and B[g][i]; here A = W rows (experts), B = x^T (tokens).
// The lane loads 8 consecutive k of its rows per 32-k chunk and feeds
// element s to MFMA step s, so step s covers k = k0 + 8g + s for all g.
// Chunks stream through a 4-deep register ring (L2 latency is the bound).
constexpr int kLgE = 16;       // experts per workgroup tile
constexpr int kLgT = 32;       // tokens per workgroup tile (two MFMA column tiles)
constexpr int kLgWaves = 8;    // K split
constexpr int kLgRing = 4;     // chunks in flight per wave
constexpr int kLgMinTokens = 64;  // below: too few tiles to fill the GPU

bool logits_mfma_ok(int n_tokens, int hidden) {
    return n_tokens >= kLgMinTokens && hidden % (kLgWaves * 32 * kLgRing) == 0;
}

// 8 elements (bf16: one dwordx4; fp32: two) widened to fp64 (exact).
template <bool F32>
struct Raw8 {
    u32x4 a, b;
    __device__ __forceinline__ void load(const void* base, size_t elem) {
        if (F32) {
            const float* p = static_cast<const float*>(base) + elem;
            a = ld16(p);
            b = ld16(p + 4);
        } else {
            a = ld16(static_cast<const uint16_t*>(base) + elem);
        }
    }
    __device__ __forceinline__ double get(int i) const {
        if (F32) return static_cast<double>(__uint_as_float(i < 4 ? a[i] : b[i - 4]));
        const uint32_t w = a[i >> 1];
        return static_cast<double>(__uint_as_float((i & 1) ? (w & 0xFFFF0000u) : (w << 16)));
    }
};

typedef double f64x4 __attribute__((ext_vector_type(4)));

template <bool XF32, bool WF32>
__global__ __launch_bounds__(64 * kLgWaves) void k_route_logits_mfma(FusedArgs A) {
    __shared__ double red[kLgWaves][2][4][64];
    const int E = A.n_experts, T = A.n_tokens, H = A.hidden;
    const int e0 = blockIdx.x * kLgE, t0 = blockIdx.y * kLgT;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int i = lane & 15, g = lane >> 4;
    const int kw = H / kLgWaves;  // k per wave, a multiple of 32 * kLgRing
    const size_t kb = (size_t)wave * kw + 8 * g;
    const size_t wr = (size_t)min(e0 + i, E - 1) * H + kb;
    const size_t xa = (size_t)min(t0 + i, T - 1) * H + kb;
    const size_t xb = (size_t)min(t0 + kTileTok + i, T - 1) * H + kb;
    f64x4 acc0 = {0.0, 0.0, 0.0, 0.0}, acc1 = {0.0, 0.0, 0.0, 0.0};
    Raw8<WF32> ra[kLgRing];
    Raw8<XF32> rb0[kLgRing], rb1[kLgRing];
    auto issue = [&](int c, int s) {
        ra[s].load(A.w, wr + (size_t)c * 32);
        rb0[s].load(A.x, xa + (size_t)c * 32);
        rb1[s].load(A.x, xb + (size_t)c * 32);
    };
    auto comp = [&](int s) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const double a = ra[s].get(e);
            acc0 = __builtin_amdgcn_mfma_f64_16x16x4f64(a, rb0[s].get(e), acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64(a, rb1[s].get(e), acc1, 0, 0, 0);
        }
    };
#pragma unroll
    for (int s = 0; s < kLgRing; ++s) {
        issue(s, s);
        __builtin_amdgcn_sched_barrier(0);
    }
    const int nch = kw / 32;
#pragma unroll 1
    for (int c = 0; c < nch - kLgRing; c += kLgRing) {
#pragma unroll
        for (int s = 0; s < kLgRing; ++s) {
            comp(s);
            __builtin_amdgcn_sched_barrier(0);
            issue(c + kLgRing + s, s);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int s = 0; s < kLgRing; ++s) comp(s);
    // the f64 16x16 result layout: lane (i, g) element r holds D[g + 4r][i]
    // (expert e0 + g + 4r, token t0 (+16) + i), unlike the 16-bit MFMAs'
    // D[4g + r][i]
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        red[wave][0][r][lane] = acc0[r];
        red[wave][1][r][lane] = acc1[r];
    }
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < 2 * 64) {
        const int tt = tid >> 6, l = tid & 63;
        const int t = t0 + tt * kTileTok + (l & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int e = e0 + (l >> 4) + 4 * r;
            double v = red[0][tt][r][l];
#pragma unroll
            for (int w = 1; w < kLgWaves; ++w) v += red[w][tt][r][l];
            if (t < T && e < E) A.logits[(size_t)t * E + e] = v;
        }
    }
}

// T <= 16, selection only: wave t selects token t (register path: all tokens
// in parallel; LDS fallback: 4 waves loop over the tokens).
__global__ __launch_bounds__(1024) void k_route_select_small(FusedArgs A) {
    extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    double* c = reinterpret_cast<double*>(dyn) + (size_t)wave * 2 * A.n_experts;
    double* s = c + A.n_experts;
    uint8_t* gsel = reinterpret_cast<uint8_t*>(reinterpret_cast<double*>(dyn) + 2 * (size_t)nw * A.n_experts) + wave * 64;
    for (int t = wave; t < A.n_tokens; t += nw) {
        select_any(A.logits + (size_t)t * A.n_experts, A.bias, A.resident, A.n_experts, A.n_group,
                   A.topk_group, A.top_k, A.norm, A.scale, A.ids + (size_t)t * A.top_k,
                   A.wout + (size_t)t * A.top_k, A.epl, c, s, gsel);
    }
}

// one wave per token, 4 tokens per workgroup
__global__ __launch_bounds__(kRouteThreads) void k_route_select(FusedArgs A) {
    extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
    const int wave = threadIdx.x >> 6;
    const int t = blockIdx.x * (kRouteThreads / 64) + wave;
    if (t >= A.n_tokens) return;
    double* c = reinterpret_cast<double*>(dyn) + (size_t)wave * 2 * A.n_experts;
    double* s = c + A.n_experts;
    uint8_t* gsel = reinterpret_cast<uint8_t*>(reinterpret_cast<double*>(dyn) + 8 * (size_t)A.n_experts) + wave * 64;
    select_any(A.logits + (size_t)t * A.n_experts, A.bias, A.resident, A.n_experts, A.n_group,
               A.topk_group, A.top_k, A.norm, A.scale, A.ids + (size_t)t * A.top_k,
               A.wout + (size_t)t * A.top_k, A.epl, c, s, gsel);
}

// ---------------------------------------------------------------------------
// Decode stage 1: router logits, block b = expert row b % E for tokens
// [4*(b/E), +4) (T <= 16).
template <bool WF32>
__global__ __launch_bounds__(kRouteThreads) void k_dec_logits(FusedArgs A) {
    __shared__ double red[4 * 4];
    const int e = blockIdx.x % A.n_experts, t0 = (blockIdx.x / A.n_experts) * 4;
    row_logits4<WF32, kRouteThreads>(A.x, A.w, e, t0, min(4, A.n_tokens - t0), A.hidden,
                                     A.n_experts, A.logits, red);
}

// Decode stage 2: workgroup 0 selects every token (wave t = token t,
// register path) and builds the plan; blocks 1.. run the shared expert's
// gate/up tiles (single mode, pairs [0, T)): KSA of the 16 waves split K, so
// the whole expert is in flight while the latency-bound selection runs.
// Every global input of workgroup 0 (logits, bias, resident mask, layer
// table) is requested before its first barrier.  LDS (dynamic) is shared by
// the two roles: the planner's DecPlanLds or the gate/up tile's reduction
// tile and staged activations.
// NTHR threads per workgroup (selection: one wave per token, so T <= NTHR/64);
// KP > 1: each shared-expert tile is split into KP k-parts over KP blocks
// (k-part sums finalised by the routed gate/up launch), so the expert's
// 29 MB spread over 2x the CUs (one CU sustains ~22 GB/s of these loads).
template <int EPL, int NKB, int KSA, bool XLDS, int NTHR = kDecThreads, int KP = 1>
__global__ __launch_bounds__(NTHR) void k_dec_select_sgu(FusedArgs A, ExpertLaunch SG) {
    extern __shared__ __attribute__((aligned(16))) unsigned char dlds[];
    if (blockIdx.x > 0) {
        // activations streamed from L2 ride the ring too: keep it 2 deep so
        // the block stays within 128 registers
        constexpr int D = NKB < (XLDS ? 4 : 2) ? NKB : (XLDS ? 4 : 2);
        const int b = blockIdx.x - 1;
        gate_up_tile<NKB, D, 1, false, XLDS, NTHR / 64, true, KSA, kTileRows, (KP > 1)>(
            SG, b / KP, 0, dlds, b % KP);
        return;
    }
    DecPlanLds& S = *reinterpret_cast<DecPlanLds*>(dlds);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int T = A.n_tokens, K = A.top_k, E = A.n_experts, TE = T * E;
    double* sS = reinterpret_cast<double*>(dlds + sizeof(DecPlanLds));  // [T][E]
    double* sC = sS + TE;                                               // [T][E]
    // 1) every global input at once: this thread's logits, bias and
    //    residency (<= 4 (token, expert) cells), the layer table
    constexpr int kCells = (NTHR / 64) * kDecMaxExperts / NTHR;  // T <= NTHR/64 tokens
    double lg[kCells];
    float bs[kCells];
    bool rs[kCells];
#pragma unroll
    for (int r = 0; r < kCells; ++r) {
        const int i = tid + r * NTHR, e = i % E;
        if (i < TE) {
            lg[r] = A.logits[i];
            bs[r] = A.bias[e];
            rs[r] = A.resident == nullptr || A.resident[e] != 0;
        }
    }
    dec_plan_prologue(S, A.table, E);
    // 2) scores of every (token, expert) cell, spread over all 16 waves
    int nres_part = 0;
#pragma unroll
    for (int r = 0; r < kCells; ++r) {
        const int i = tid + r * NTHR;
        if (i < TE) {
            expert_scores(lg[r], bs[r], rs[r], &sS[i], &sC[i]);
            nres_part += i < E && rs[r] ? 1 : 0;  // token 0's row counts each expert once
        }
    }
    const uint32_t nres_wave = wave_incl_scan(static_cast<uint32_t>(nres_part));
    if (lane == 63) S.nres_w[wave] = static_cast<int>(nres_wave);
    __syncthreads();
    // 3) selection: wave t = token t
    if (wave < T) {
        int nres = 0;
#pragma unroll
        for (int w = 0; w < NTHR / 64; ++w) nres += S.nres_w[w];
        SelIn<EPL> in;
        sel_load_lds<EPL>(in, sS + (size_t)wave * E, sC + (size_t)wave * E, nres);
        const SelOut o = select_any_reg<EPL>(in, E, A.n_group, A.topk_group, K, A.norm, A.scale);
        write_sel(o, K, A.ids + (size_t)wave * K, A.wout + (size_t)wave * K);
        if (lane < o.kk) {
            atomicOr(&S.mask[wave][o.isel >> 5], 1u << (o.isel & 31));
            S.wsel[wave][o.isel] = o.w;
            S.ksel[wave][o.isel] = static_cast<uint8_t>(lane);
        } else if (lane < K) {
            A.plan.token_pairs[(size_t)wave * (K + 1) + lane] = -1;
        }
    }
    __syncthreads();
    dec_plan_core(S, T, K, E, A.has_shared, A.plan, A.err_flag, 0);
}

// ---------------------------------------------------------------------------
// One-token decode with the selection inside the routed gate/up launch.
// The two-stage router (logits; selection + planner beside the shared gate/up)
// becomes: stage 1 = logits and scores beside the shared gate/up; stage 2 =
// the routed gate/up, in which every workgroup selects the token's experts
// itself.  A workgroup of the routed gate/up already waits two dependent
// memory round trips for its plan record before its first weight load; here
// it waits for the scores and its expert's descriptor instead, plus the
// selection's arithmetic, and the stage between them is gone.

// Stage 1.  Blocks [0, E): router row e's logit (exact fp64 products and a
// fixed-order sum, row_logits4) and its scores, s = sigmoid(logit) and
// c = s + bias (expert_scores, fp64), into sc[e] and sc[E + e].  Blocks E..:
// the shared expert's gate/up tiles as two k-parts (the split tiles of
// k_dec_select_sgu), finalised by stage 2.  8-wave blocks.
template <bool WF32, int NKB, int KSA, bool XLDS>
__global__ __launch_bounds__(512) void k_dec_logits_sgu(FusedArgs A, ExpertLaunch SG, double* sc) {
    extern __shared__ __attribute__((aligned(16))) unsigned char dlds[];
    const int E = A.n_experts;
    if ((int)blockIdx.x >= E) {
        constexpr int D = NKB < (XLDS ? 4 : 2) ? NKB : (XLDS ? 4 : 2);
        const int b = blockIdx.x - E;
        gate_up_tile<NKB, D, 1, false, XLDS, 8, true, KSA, kTileRows, true>(SG, b / 2, 0, dlds, b % 2);
        return;
    }
    const int e = blockIdx.x;
    row_logits4<WF32, 512>(A.x, A.w, e, 0, 1, A.hidden, E, A.logits, reinterpret_cast<double*>(dlds));
    if (threadIdx.x == 0) {  // the thread that stored the logit
        double sv, cv;
        expert_scores(A.logits[e], A.bias[e], true, &sv, &cv);
        sc[e] = sv;
        sc[E + e] = cv;
    }
}

// Selection of one token specialised to 256 experts in 8 groups of 32 (the
// DeepSeek-V3 router) and at most 8 picks, branch-free, for the one-token
// fused path.  Lane l holds the choice scores c of experts 4l..4l+3 (group
// l/8).  The decisions are select_reg's: a group's score is the sum of its
// two largest c (a sum over a multiset, so ties cannot change it); groups
// rank by score, then lower index; each pick is the largest remaining c,
// ties to the lower expert index (the lowest lane holding it, then its
// lowest slot).  Returns the picks' ids, wave-uniform.
constexpr int kSel256Experts = 256, kSel256Groups = 8, kSel256MaxPicks = 8;

struct Picks8 {
    int id[kSel256MaxPicks];
};

__device__ __forceinline__ double max_d(double a, double b) { return a > b ? a : b; }
__device__ __forceinline__ double min_d(double a, double b) { return a < b ? a : b; }

// (a, b) = the two largest of this lane's and lane CTRL's pairs
template <int CTRL>
__device__ __forceinline__ void top2_with(double& a, double& b) {
    const double oa = dpp_d<CTRL, 0xF, 0xF>(a), ob = dpp_d<CTRL, 0xF, 0xF>(b);
    const double na = max_d(a, oa);
    b = max_d(min_d(a, oa), max_d(b, ob));
    a = na;
}

// Group stage: keeps the topk_group best groups' scores and sets the
// others' to -inf.
__device__ __forceinline__ void groups256(double c[4], int topk_group) {
    const int lane = threadIdx.x & 63;
    // the group's two largest: this lane's four, then across its 8 lanes
    // (quad_perm [1,0,3,2], [2,3,0,1], then row_half_mirror: i <-> 7 - i)
    const double m01 = max_d(c[0], c[1]), n01 = min_d(c[0], c[1]);
    const double m23 = max_d(c[2], c[3]), n23 = min_d(c[2], c[3]);
    double a = max_d(m01, m23), b = max_d(min_d(m01, m23), max_d(n01, n23));
    top2_with<0xB1>(a, b);
    top2_with<0x4E>(a, b);
    top2_with<0x141>(a, b);
    const double gs = a + b;
    const int myg = lane >> 3;
    int grank = 0;
#pragma unroll
    for (int g = 0; g < kSel256Groups; ++g) {
        const double o = readlane_d(gs, 8 * g);
        grank += (o > gs || (o == gs && g < myg)) ? 1 : 0;
    }
    const bool keep = grank < topk_group;
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = keep ? c[i] : -INFINITY;
}

// Pick stage: the top_k largest remaining scores, in order.  The rounds run
// on 32-bit unsigned keys with the order of float(c) (rounding is monotonic,
// so the largest c holds the largest key): one DPP max per reduction step
// (bound_ctrl: a lane with no source reads 0, below every key) and the
// per-slot matches as ballots of the compares.  A round whose largest key is
// held by one entry alone is decided by it; otherwise (equal c, or c values
// closer than float resolution) the exact fp64 arg-max over the entries
// holding that key decides, ties to the lower expert index.  The same picks
// as a fp64 reduction per round, in about two thirds of its time.
template <int CTRL, int RM, int BM>
__device__ __forceinline__ uint32_t dpp_umax(uint32_t v) {
    const uint32_t o = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, RM, BM, true));
    return v > o ? v : o;
}

__device__ __forceinline__ uint32_t order_key(double c) {
    const uint32_t b = __float_as_uint(static_cast<float>(c));
    return b ^ ((b >> 31) ? 0xFFFFFFFFu : 0x80000000u);
}

__device__ __forceinline__ Picks8 picks256(const double c[4], int top_k) {
    const int lane = threadIdx.x & 63;
    uint32_t k[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = order_key(c[i]);
    Picks8 p;
#pragma unroll
    for (int r = 0; r < kSel256MaxPicks; ++r) {
        p.id[r] = -1;
        if (r < top_k) {
            uint32_t m = max(max(k[0], k[1]), max(k[2], k[3]));
            m = dpp_umax<0x111, 0xF, 0xF>(m);
            m = dpp_umax<0x112, 0xF, 0xF>(m);
            m = dpp_umax<0x114, 0xF, 0xF>(m);
            m = dpp_umax<0x118, 0xF, 0xF>(m);
            m = dpp_umax<0x142, 0xA, 0xF>(m);
            m = dpp_umax<0x143, 0xC, 0xF>(m);
            const uint32_t M = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m), 63));
            unsigned long long h[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) h[i] = __ballot(k[i] == M);
            const int n = __popcll(h[0]) + __popcll(h[1]) + __popcll(h[2]) + __popcll(h[3]);
            int pick = 0x7fffffff;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (h[i]) pick = min(pick, 4 * static_cast<int>(__builtin_ctzll(h[i])) + i);
            if (n != 1) {
                double v = -INFINITY;
                int vi = 0x7fffffff;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (k[q] == M && better(c[q], 4 * lane + q, v, vi)) {
                        v = c[q];
                        vi = 4 * lane + q;
                    }
                wave_argmax(v, vi);
                pick = vi;
            }
            // NaN scores (from NaN inputs) match no key: pick a valid id
            pick = pick >= 0 && pick < kSel256Experts ? pick : 0;
            p.id[r] = pick;
#pragma unroll
            for (int i = 0; i < 4; ++i) k[i] = 4 * lane + i == pick ? 0u : k[i];
        }
    }
    return p;
}

struct SelArgs {
    const double* sc;  // s [E] then c [E] of stage 1
    int n_experts, n_group, topk_group, top_k, norm, has_shared;
    float scale;
    int32_t* ids;      // [top_k] routes out (descending choice score)
    float* wout;       // [top_k]
};

// The routes (weights as select_reg forms them: s of the picks normalised
// by their sum in pick order, + 1e-20, then scaled) and the one-token plan
// the down + combine launch reads (down_comb1_tile): routed item i = pick i
// (descending choice score) owns pair s0 + i, the shared expert pair 0;
// token_pairs[k] = pair of route k (column top_k: the shared pair).  Lane
// r < top_k holds pick r.  The combine sums in route order, so the item
// order changes no output bit.
__device__ __forceinline__ void dec_sel_plan(const ExpertLaunch& L, const SelArgs& S, int isel,
                                             int s0) {
    const int lane = threadIdx.x & 63, K = S.top_k, rank = lane;
    const double sv = lane < K ? S.sc[isel] : 0.0;
    double wsum = 0.0;
    for (int r = 0; r < K; ++r) wsum += readlane_d(sv, r);
    double v = sv;
    if (S.norm && K > 1) v /= wsum + 1e-20;
    v *= static_cast<double>(S.scale);
    if (lane < K) {
        S.ids[lane] = isel;
        S.wout[lane] = static_cast<float>(v);
        L.plan.token_pairs[lane] = s0 + rank;
    }
    if (lane == K) L.plan.token_pairs[K] = s0 ? 0 : -1;
    if (lane < K || (s0 && lane == K)) {
        const bool routed = lane < K;
        const cx_expert_desc d = L.table[routed ? isel : S.n_experts];  // entry E: the shared expert
        L.plan.item_rec[routed ? rank : K] =
            ItemRec{d.w_up, d.w_gate, d.w_down, d.s_up, d.s_gate, d.s_down, routed ? s0 + rank : 0, 1,
                    d.up_rb, d.gate_rb, d.down_rb, d.gu_layout, {0, 0, 0, 0}};
    }
    if (lane == 0) {
        PlanHdr h{};
        h.n_slots = h.n_items = h.n_pairs = K + s0;
        h.n_routed_slots = h.n_routed_items = K;
        *L.plan.hdr = h;
    }
}

// Stage 2: grid (inter / 16 row tiles, top_k picks [+ 1]).  Wave 0 of every
// workgroup selects (select256 on stage 1's choice scores: the same inputs
// and code everywhere, so every workgroup finds the same picks) as far as
// pick blockIdx.y, whose expert it hands to the other waves through LDS
// (rows of early picks start streaming earlier); the workgroup then streams
// row tile blockIdx.x of that expert's gate and up (gate_up_tile_unit, x
// staged in LDS).  With a shared expert, the last grid row finalises its h
// from stage 1's k-part sums.
template <int NKB>
__global__ __launch_bounds__(256) void k_gate_up_sel(ExpertLaunch L, SelArgs S) {
    extern __shared__ __attribute__((aligned(16))) unsigned char gu_lds[];
    if (L.gu_part != nullptr && blockIdx.y == gridDim.y - 1) {
        shared_h_finalize(L, blockIdx.x);
        return;
    }
    __shared__ int s_expert;  // this workgroup's expert, or -1
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int item = blockIdx.y, K = S.top_k;
    const int s0 = S.has_shared ? 1 : 0;
    if (wave == 0) {
        double c[4];
        {
            const u32x4 v0 = ld16(S.sc + kSel256Experts + 4 * lane);
            const u32x4 v1 = ld16(S.sc + kSel256Experts + 4 * lane + 2);
            c[0] = __longlong_as_double((static_cast<long long>(v0[1]) << 32) | v0[0]);
            c[1] = __longlong_as_double((static_cast<long long>(v0[3]) << 32) | v0[2]);
            c[2] = __longlong_as_double((static_cast<long long>(v1[1]) << 32) | v1[0]);
            c[3] = __longlong_as_double((static_cast<long long>(v1[3]) << 32) | v1[2]);
        }
        groups256(c, S.topk_group);
        // grid row y takes pick y, so it needs picks 0..y only; the last
        // row's workgroup 0 has them all and writes the plan
        const Picks8 p = picks256(c, min(item + 1, K));
        int isel = -1;  // lane r <= item: pick r
#pragma unroll
        for (int r = 0; r < kSel256MaxPicks; ++r) isel = lane == r ? p.id[r] : isel;
        if (lane == 0) s_expert = item < K ? __builtin_amdgcn_readlane(isel, item) : -1;
        if (blockIdx.x == 0 && item == K - 1) dec_sel_plan(L, S, isel, s0);
    }
    __syncthreads();
    const int e = __builtin_amdgcn_readfirstlane(s_expert);
    if (e < 0) return;
    Unit u;
    u.e = ld_uniform(L.table + e);
    u.e.hidden = L.hidden;
    u.e.inter = L.inter;
    u.pb = s0 + item;
    u.np = 1;
#pragma unroll
    for (int q = 0; q < 4; ++q) u.tok[q] = 0;
    constexpr int D = NKB < 4 ? NKB : 4;
    gate_up_tile_unit<NKB, D, 1, false, true, 4, false>(L, blockIdx.x, u, gu_lds);
}

// Decode stage 1' (routes given): workgroup 0 validates the routes (range,
// repeats within a token: validate_routes, server/moe_layer_runtime.py:84-98)
// and builds the plan; blocks 1.. run the shared expert's gate/up tiles.
struct DecIdsArgs {
    const int32_t* ids;
    const float* w;
    int n_tokens, top_k, n_experts, has_shared;
    const cx_expert_desc* table;
    PlanPtrs plan;
    int* err_flag;
};

constexpr int kDecIdsPerThread = 4;  // T*K <= 16*64 assignments over 256 threads

template <int NKB, bool F16>
__global__ __launch_bounds__(kRouteThreads) void k_dec_plan_sgu(DecIdsArgs P, ExpertLaunch SG) {
    extern __shared__ __attribute__((aligned(16))) unsigned char dlds[];
    if (blockIdx.x > 0) {
        constexpr int D = NKB < 4 ? NKB : 4;
        gate_up_tile<NKB, D, 1, F16, false, 4, true>(SG, blockIdx.x - 1, 0, dlds);
        return;
    }
    DecPlanLds& S = *reinterpret_cast<DecPlanLds*>(dlds);
    int* rid = reinterpret_cast<int*>(dlds + sizeof(DecPlanLds));  // [16 * 64]
    const int tid = threadIdx.x;
    const int T = P.n_tokens, K = P.top_k, E = P.n_experts, n = T * K;
    int myid[kDecIdsPerThread];
    float myw[kDecIdsPerThread];
#pragma unroll
    for (int r = 0; r < kDecIdsPerThread; ++r) {
        const int i = tid + r * kRouteThreads;
        myid[r] = i < n ? P.ids[i] : -1;
        myw[r] = i < n ? P.w[i] : 0.0f;
    }
    dec_plan_prologue(S, P.table, E);
#pragma unroll
    for (int r = 0; r < kDecIdsPerThread; ++r) {
        const int i = tid + r * kRouteThreads;
        if (i < n) rid[i] = myid[r];
    }
    __syncthreads();
    int err = 0;
#pragma unroll
    for (int r = 0; r < kDecIdsPerThread; ++r) {
        const int i = tid + r * kRouteThreads;
        if (i >= n) continue;
        const int t = i / K, k = i - t * K, e = myid[r];
        bool ok = e >= 0;
        if (e >= E) {
            err |= kErrBadExpertId;
            ok = false;
        } else if (ok) {
            for (int j = t * K; j < i; ++j)
                if (rid[j] == e) { err |= kErrDuplicateRoute; ok = false; break; }
            if (ok && !route_weight_ok(myw[r])) {
                err |= kErrBadWeight;
                ok = false;
            }
        }
        if (ok) {
            atomicOr(&S.mask[t][e >> 5], 1u << (e & 31));
            S.wsel[t][e] = myw[r];
            S.ksel[t][e] = static_cast<uint8_t>(k);
        } else {
            P.plan.token_pairs[(size_t)t * (K + 1) + k] = -1;
        }
    }
    __syncthreads();
    dec_plan_core(S, T, K, E, P.has_shared, P.plan, P.err_flag, err);
}

// Experts per lane for the register selection (E = 64*EPL, groups made of a
// power-of-two number of whole lanes), or 0 for the LDS fallback.
int register_epl(int n_experts, int n_group) {
    if (n_experts % 64 != 0) return 0;
    const int epl = n_experts / 64;
    if (epl != 1 && epl != 2 && epl != 4 && epl != 8) return 0;
    const int epg = n_experts / n_group;
    if (epg % epl != 0) return 0;
    const int lpg = epg / epl;
    if ((lpg & (lpg - 1)) != 0 || lpg > 16 || n_group * lpg != 64) return 0;
    return epl;
}

size_t select_lds(int n_experts) {
    // 4 waves x (c, s) doubles + 4 x 64 group flags
    return (size_t)8 * n_experts * sizeof(double) + 4 * 64;
}

// Shared-expert gate/up tiling of stage 2 (16-wave blocks): k-blocks per
// active wave (NKB) and active waves (KSA) for hidden / 128 k-blocks.
template <int EPL, int XLDS>
void go_dec_select_h(const FusedArgs& A, const ExpertLaunch* sg, size_t lds, hipStream_t s) {
    ExpertLaunch none{};
    const ExpertLaunch& G = sg ? *sg : none;
    if (sg != nullptr && G.gu_part != nullptr) {  // k-part split: 8-wave blocks, T <= 8
        const dim3 grid(1 + 2 * (G.inter / kTileRows)), block(512);
        switch (A.hidden / kKB) {
            case 56: cx_launch((k_dec_select_sgu<EPL, 4, 7, XLDS, 512, 2>), grid, block, lds, s, A, G); break;
            case 8: cx_launch((k_dec_select_sgu<EPL, 1, 4, XLDS, 512, 2>), grid, block, lds, s, A, G); break;
            default: cx_launch((k_dec_select_sgu<EPL, 1, 2, XLDS, 512, 2>), grid, block, lds, s, A, G); break;
        }
        return;
    }
    const dim3 grid(1 + (sg ? G.inter / kTileRows : 0)), block(kDecThreads);
    switch (A.hidden / kKB) {
        case 56: cx_launch((k_dec_select_sgu<EPL, 4, 14, XLDS>), grid, block, lds, s, A, G); break;
        case 8: cx_launch((k_dec_select_sgu<EPL, 1, 8, XLDS>), grid, block, lds, s, A, G); break;
        default: cx_launch((k_dec_select_sgu<EPL, 1, 4, XLDS>), grid, block, lds, s, A, G); break;
    }
}

// Active waves of a shared-expert tile in stage 2 (k-part split: per part).
int dec_select_ksa(int hidden, bool split = false) {
    switch (hidden / kKB) {
        case 56: return split ? 7 : 14;
        case 8: return split ? 4 : 8;
        default: return split ? 2 : 4;
    }
}

template <int EPL>
void go_dec_select(const FusedArgs& A, const ExpertLaunch* sg, hipStream_t s) {
    const bool xl = sg != nullptr && sg->np_lds > 0;
    size_t lds = sizeof(DecPlanLds) + (size_t)2 * A.n_tokens * A.n_experts * sizeof(double);
    if (sg != nullptr)
        lds = std::max(lds, gate_up_lds_bytes(dec_select_ksa(A.hidden, sg->gu_part != nullptr), 1,
                                              xl ? sg->np_lds : 0, A.hidden));
    if (xl) go_dec_select_h<EPL, true>(A, sg, lds, s);
    else go_dec_select_h<EPL, false>(A, sg, lds, s);
}

template <int NKB>
void go_dec_plan(const DecIdsArgs& P, const ExpertLaunch* sg, hipStream_t s) {
    ExpertLaunch none{};
    const ExpertLaunch& G = sg ? *sg : none;
    const int grid = 1 + (sg ? G.inter / kTileRows : 0);
    size_t lds = sizeof(DecPlanLds) + sizeof(int) * kTileTok * 64;
    if (sg != nullptr) lds = std::max(lds, gate_up_lds_bytes(4, 1, 0, G.hidden));
    if (sg && G.in_dtype == CX_DTYPE_FP16)
        cx_launch((k_dec_plan_sgu<NKB, true>), dim3(grid), dim3(kRouteThreads), lds, s, P, G);
    else
        cx_launch((k_dec_plan_sgu<NKB, false>), dim3(grid), dim3(kRouteThreads), lds, s, P, G);
}

}  // namespace

bool dec_route_ok(int n_experts, int n_group) {
    const int epl = register_epl(n_experts, n_group);
    return n_experts <= kDecMaxExperts && (epl == 1 || epl == 2 || epl == 4);
}

int dec_sgu_np_lds(int hidden, int n_tokens, int max_lds) {
    if (hidden % 512 != 0 || n_tokens > 4) return 0;
    const int red = (int)gate_up_red_bytes(dec_select_ksa(hidden), 1);
    const int rows = (std::min(max_lds, 65536) - red) / (hidden * 2 + 16);
    return n_tokens <= rows ? n_tokens : 0;
}

bool dec_shared_split_ok(int hidden, int inter, int n_tokens) {
    return dec_shared_ok(hidden, inter) && n_tokens <= kDecSplitMaxTokens &&
           (hidden / kKB) % 2 == 0;
}

bool dec_shared_ok(int hidden, int inter) {
    const int nkh = hidden / kKB;
    if (hidden % kKB != 0 || (nkh != 56 && nkh != 8 && nkh != 4)) return false;
    return (inter == 2048 || inter == 512) && hidden % 64 == 0;
}

hipError_t launch_dec_logits(const RouteArgs& R, hipStream_t s) {
    if (R.n_tokens > kTileTok || R.x_dtype != CX_DTYPE_BF16) return hipErrorInvalidValue;
    const FusedArgs A = fused_args(R);
    const dim3 grid(R.n_experts * ((R.n_tokens + 3) / 4));
    if (R.w_dtype == CX_DTYPE_F32) cx_launch(k_dec_logits<true>, grid, dim3(kRouteThreads), 0, s, A);
    else cx_launch(k_dec_logits<false>, grid, dim3(kRouteThreads), 0, s, A);
    return hipGetLastError();
}

hipError_t launch_dec_select_sgu(const RouteArgs& R, const ExpertLaunch* sg, hipStream_t s) {
    if (R.plan == nullptr || R.n_tokens > kTileTok || !dec_route_ok(R.n_experts, R.n_group))
        return hipErrorInvalidValue;
    if (sg != nullptr && sg->gu_part != nullptr && R.n_tokens > kDecSplitMaxTokens)
        return hipErrorInvalidValue;
    const FusedArgs A = fused_args(R);
    switch (register_epl(R.n_experts, R.n_group)) {
        case 1: go_dec_select<1>(A, sg, s); break;
        case 2: go_dec_select<2>(A, sg, s); break;
        default: go_dec_select<4>(A, sg, s); break;
    }
    return hipGetLastError();
}

hipError_t launch_dec_plan_sgu(const int32_t* ids, const float* w, int n_tokens, int top_k,
                               const cx_expert_desc* table, int n_experts, int has_shared,
                               PlanPtrs plan, int* err_flag, const ExpertLaunch* sg,
                               hipStream_t s) {
    if (n_tokens > kTileTok || n_experts > kDecMaxExperts || top_k > 64) return hipErrorInvalidValue;
    DecIdsArgs P{ids, w, n_tokens, top_k, n_experts, has_shared, table, plan, err_flag};
    switch (sg ? sg->hidden / kKB : 4) {
        case 56: go_dec_plan<14>(P, sg, s); break;
        case 8: go_dec_plan<2>(P, sg, s); break;
        case 4: go_dec_plan<1>(P, sg, s); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool dec_fused_sel_ok(int n_experts, int n_group, int topk_group, int hidden, int top_k, int x_dtype) {
    const int nkb = hidden / kKB;
    return n_experts == kSel256Experts && n_group == kSel256Groups && topk_group >= 1 &&
           topk_group <= kSel256Groups && top_k >= 1 && top_k <= kSel256MaxPicks &&
           hidden % 512 == 0 && (nkb == 56 || nkb == 8) && x_dtype == CX_DTYPE_BF16;
}

hipError_t launch_dec_logits_sgu(const RouteArgs& R, const ExpertLaunch* sg, double* sc, hipStream_t s) {
    if (R.n_tokens != 1 || R.resident != nullptr || sc == nullptr ||
        !dec_fused_sel_ok(R.n_experts, R.n_group, R.topk_group, R.hidden, R.top_k, R.x_dtype))
        return hipErrorInvalidValue;
    if (sg != nullptr && (sg->gu_part == nullptr || sg->gu_kparts != 2)) return hipErrorInvalidValue;
    const FusedArgs A = fused_args(R);
    ExpertLaunch none{};
    const ExpertLaunch& G = sg ? *sg : none;
    const bool xl = sg != nullptr && sg->np_lds > 0;
    const bool big = R.hidden / kKB == 56;
    const size_t lds = std::max<size_t>(8 * 4 * sizeof(double),
                                        sg ? gate_up_lds_bytes(big ? 7 : 4, 1, xl ? sg->np_lds : 0, R.hidden) : 0);
    const dim3 grid(R.n_experts + (sg ? 2 * (sg->inter / kTileRows) : 0)), block(512);
    const bool wf = R.w_dtype == CX_DTYPE_F32;
#define CX_GO(WF, NKB, KSA, XL) cx_launch((k_dec_logits_sgu<WF, NKB, KSA, XL>), grid, block, lds, s, A, G, sc)
    if (big) {
        if (wf) { if (xl) CX_GO(true, 4, 7, true); else CX_GO(true, 4, 7, false); }
        else { if (xl) CX_GO(false, 4, 7, true); else CX_GO(false, 4, 7, false); }
    } else {
        if (wf) { if (xl) CX_GO(true, 1, 4, true); else CX_GO(true, 1, 4, false); }
        else { if (xl) CX_GO(false, 1, 4, true); else CX_GO(false, 1, 4, false); }
    }
#undef CX_GO
    return hipGetLastError();
}

hipError_t launch_gate_up_sel(const ExpertLaunch& L, const RouteArgs& R, const double* sc, hipStream_t s) {
    if (L.table == nullptr || L.n_tokens != 1 || L.np_lds < 1 || L.maxt != 1 || sc == nullptr ||
        !dec_fused_sel_ok(R.n_experts, R.n_group, R.topk_group, L.hidden, R.top_k, L.in_dtype))
        return hipErrorInvalidValue;
    SelArgs S{sc, R.n_experts, R.n_group, R.topk_group, R.top_k, R.norm, R.has_shared, R.scale, R.ids, R.wout};
    const dim3 grid(L.inter / kTileRows, R.top_k + (L.gu_part != nullptr ? 1 : 0)), block(256);
    const size_t lds = gate_up_lds_bytes(4, 1, L.np_lds, L.hidden);
    if (L.hidden / kKB == 56) cx_launch((k_gate_up_sel<14>), grid, block, lds, s, L, S);
    else cx_launch((k_gate_up_sel<2>), grid, block, lds, s, L, S);
    return hipGetLastError();
}

hipError_t launch_route(const RouteArgs& R, hipStream_t s) {
    FusedArgs A = fused_args(R);
    A.epl = register_epl(R.n_experts, R.n_group);
    const size_t sel = A.epl ? 0 : select_lds(R.n_experts);
    const bool xf = R.x_dtype == CX_DTYPE_F32, wf = R.w_dtype == CX_DTYPE_F32;
    if (logits_mfma_ok(R.n_tokens, R.hidden)) {
        // many tokens: fp64 MFMA tiles
        const dim3 lg((R.n_experts + kLgE - 1) / kLgE, (R.n_tokens + kLgT - 1) / kLgT);
        const dim3 blk(64 * kLgWaves);
        if (xf && wf) cx_launch((k_route_logits_mfma<true, true>), lg, blk, 0, s, A);
        else if (xf) cx_launch((k_route_logits_mfma<true, false>), lg, blk, 0, s, A);
        else if (wf) cx_launch((k_route_logits_mfma<false, true>), lg, blk, 0, s, A);
        else cx_launch((k_route_logits_mfma<false, false>), lg, blk, 0, s, A);
    } else {
        // few tokens: one workgroup per expert row streams W_r once
        const dim3 lg(R.n_experts, (R.n_tokens + kRouteTB - 1) / kRouteTB);
        if (xf && wf) cx_launch((k_route_logits<true, true>), lg, dim3(kRouteThreads), 0, s, A);
        else if (xf) cx_launch((k_route_logits<true, false>), lg, dim3(kRouteThreads), 0, s, A);
        else if (wf) cx_launch((k_route_logits<false, true>), lg, dim3(kRouteThreads), 0, s, A);
        else cx_launch((k_route_logits<false, false>), lg, dim3(kRouteThreads), 0, s, A);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (R.n_tokens <= kRouteTB) {
        // register path: one wave per token, all in parallel; fallback: 4 waves
        const int threads = A.epl ? 64 * R.n_tokens : kRouteThreads;
        const size_t lds = A.epl ? 0 : (size_t)2 * (threads / 64) * R.n_experts * sizeof(double) + (threads / 64) * 64;
        cx_launch(k_route_select_small, dim3(1), dim3(threads), lds, s, A);
    } else {
        cx_launch(k_route_select, dim3((R.n_tokens + 3) / 4), dim3(kRouteThreads), sel, s, A);
    }
    err = hipGetLastError();
    if (err != hipSuccess || R.plan == nullptr) return err;
    return launch_plan(R.ids, R.wout, R.n_tokens, R.top_k, R.table, R.n_experts, R.has_shared,
                       R.item_cap, R.max_items, *R.plan, R.err_flag, s);
}

// Dynamic LDS the current device grants one workgroup (queried once per device).
int plan_lds_limit() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return 65536;
    }
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) {
            (void)hipGetLastError();
            v = 65536;
        }
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

hipError_t launch_plan(const int32_t* ids, const float* w, int n_tokens, int top_k,
                       const cx_expert_desc* table, int n_experts, int has_shared, int item_cap,
                       int max_items, PlanPtrs plan, int* err_flag, hipStream_t s) {
    const int threads = n_tokens * top_k <= 512 ? 256 : kPlanThreads;
    const size_t staged = plan_staged_lds(n_tokens * top_k, n_experts, threads);
    if (n_experts < 32768 && n_tokens * top_k <= kPlanRoutesPerThread * threads &&
        staged <= (size_t)plan_lds_limit()) {
        cx_launch(k_plan_staged, dim3(1), dim3(threads), staged, s, ids, w, n_tokens, top_k,
                  table, n_experts, has_shared, item_cap, max_items, plan, err_flag);
        return hipGetLastError();
    }
    const size_t lds = sizeof(int) * (2 * (size_t)n_experts + threads);
    cx_launch(k_plan, dim3(1), dim3(threads), lds, s, ids, w, n_tokens, top_k, table,
              n_experts, has_shared, item_cap, max_items, plan, err_flag);
    return hipGetLastError();
}

int route_max_experts() { return kMaxRouteExperts; }

}  // namespace cx
