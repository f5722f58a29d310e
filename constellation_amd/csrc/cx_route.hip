// cx_route.hip — DeepSeek-V3 router and the grouped-execution planner.
//
// Router semantics: route_token_real (server/moe_layer_runtime.py:232-408);
// the HF twin is MoEGate.forward (tmp/patched_modeling/
// modeling_deepseek_eager.py:428-540).  Logits accumulate exact products in
// fp64 and the whole selection runs in fp64, so the chosen expert sets equal
// the exact-math decision; ties break toward the lower index.
//
// Launch shapes: k_route_logits (one workgroup per expert row streams W_r
// once for up to 16 tokens), then
//  * T <= 16: k_route_select_plan — one workgroup selects every token (one
//    wave per token) and, for cx_moe_layer, builds the grouped plan;
//  * T > 16: k_route_select (one wave per token), then k_plan.
#include "cx_internal.h"

namespace cx {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kRouteThreads = 256;
constexpr int kRouteTB = 16;        // tokens per row workgroup
constexpr int kMaxRouteExperts = 1024;

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
            a = *reinterpret_cast<const u32x4*>(p);
            b = *reinterpret_cast<const u32x4*>(p + 4);
        } else {
            a = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + elem);
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
__device__ void row_logits(const void* __restrict__ x, const void* __restrict__ w, int t0, int nt,
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
                    const int t = min(tg * 4 + tt, nt - 1);
#pragma unroll
                    for (int j = 0; j < G; ++j) {
                        const int ci = c0 + j * kRouteThreads + tid;
                        if (ci < nchunk) xc[tt][j].load(x, (size_t)(t0 + t) * hidden + (size_t)ci * 8);
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

// Selection for one token by one wave.  c / taken are this wave's LDS
// scratch of n_experts entries.
__device__ void select_token(const double* __restrict__ lrow, const float* __restrict__ bias,
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

// Register-resident selection (one wave per token): lane l owns the EPL
// consecutive experts [l*EPL, (l+1)*EPL); a group of epg experts is a
// segment of LPG = epg/EPL lanes (a power of two <= 16, so a group never
// crosses a 16-lane DPP row).  Same decisions, tie rules and fixed
// summation order as select_token.  Cross-lane steps use DPP moves
// (row_shr, row_bcast) instead of ds_bpermute shuffles, so one arg-max costs
// a few dozen VALU cycles rather than a chain of LDS-crossbar round trips.
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

template <int EPL>
__device__ void select_token_reg(const double* __restrict__ lrow, const float* __restrict__ bias,
                                 const uint8_t* __restrict__ resident, int n_experts, int n_group,
                                 int topk_group, int top_k, int norm, float scale,
                                 int32_t* __restrict__ ids, float* __restrict__ wout) {
    const int lane = threadIdx.x & 63;
    const int base = lane * EPL;
    const int epg = n_experts / n_group;
    const int lpg = epg / EPL;  // lanes per group: power of two <= 16 (host-checked)
    double s[EPL], c[EPL];
    int nres = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int e = base + i;
        const double sg = 1.0 / (1.0 + exp(-lrow[e]));
        const bool res = resident == nullptr || resident[e] != 0;
        s[i] = res ? sg : 0.0;
        c[i] = res ? sg + static_cast<double>(bias[e]) : -INFINITY;
        nres += __popcll(__ballot(res));
    }
    // group score: top-2 sum over the group's lane segment, complete in the
    // segment's last lane
    Top2 t{-INFINITY, -INFINITY, kNoIdx, kNoIdx};
#pragma unroll
    for (int i = 0; i < EPL; ++i) t = merge2(t, Top2{c[i], -INFINITY, base + i, kNoIdx});
    const int sub = lane & (lpg - 1);
    if (lpg > 1) top2_step<0x111>(t, sub >= 1);
    if (lpg > 2) top2_step<0x112>(t, sub >= 2);
    if (lpg > 4) top2_step<0x114>(t, sub >= 4);
    if (lpg > 8) top2_step<0x118>(t, sub >= 8);
    const double gs_lane = epg >= 2 ? t.v1 + t.v2 : t.v1;
    const int grp = base / epg;
    // the full group scores sit in each segment's last lane: read them all
    // (uniform lane index) and rank this lane's group among them
    int rank = 0;
    double my_gs = 0.0;
    for (int g2 = 0; g2 < n_group; ++g2) {
        const double o = readlane_d(gs_lane, g2 * lpg + lpg - 1);
        if (g2 == grp) my_gs = o;
    }
    for (int g2 = 0; g2 < n_group; ++g2) {
        const double o = readlane_d(gs_lane, g2 * lpg + lpg - 1);
        if (g2 != grp && better(o, g2, my_gs, grp)) ++rank;
    }
    if (rank >= topk_group) {
#pragma unroll
        for (int i = 0; i < EPL; ++i) c[i] = -INFINITY;
    }
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

// Dispatch on experts per lane; fallback = the LDS version.
__device__ void select_any(const double* lrow, const float* bias, const uint8_t* resident,
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
// Planner (one workgroup, any blockDim multiple of 64).  Counting sort of the
// (token, k) assignments by expert id; slots in ascending expert id, shared
// expert last; items of <= item_cap pairs.  The order of pairs inside a slot
// only picks an MFMA column, which never changes a value, so the atomic
// cursor keeps the results deterministic.  LDS: 2*E + blockDim ints.
__device__ int block_excl_scan(int v, int* tmp, int* total) {
    const int tid = threadIdx.x, n = blockDim.x;
    tmp[tid] = v;
    __syncthreads();
    for (int off = 1; off < n; off <<= 1) {
        const int a = tid >= off ? tmp[tid - off] : 0;
        __syncthreads();
        tmp[tid] += a;
        __syncthreads();
    }
    const int incl = tmp[tid];
    *total = tmp[n - 1];
    __syncthreads();
    return incl - v;
}

__device__ void plan_build(const int32_t* __restrict__ ids, const float* __restrict__ w,
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
        atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    const int chunk = (n_experts + nt - 1) / nt;
    const int e0 = min(tid * chunk, n_experts), e1 = min(e0 + chunk, n_experts);
    int my_pairs = 0, my_slots = 0;
    for (int e = e0; e < e1; ++e) {
        my_pairs += cnt[e];
        my_slots += cnt[e] > 0;
    }
    int tot_pairs = 0, tot_slots = 0;
    int pair_off = block_excl_scan(my_pairs, scan, &tot_pairs);
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
        if (e >= 0 && e < n_experts && table[e].w_up != nullptr && !dup_route(ids, i, top_k)) {
            pos = atomicAdd(&cur[e], 1);
            P.pair_token[pos] = t;
            P.pair_weight[pos] = w[i];
        }
        P.token_pairs[(size_t)t * (top_k + 1) + k] = pos;
    }
    const bool shared = has_shared && table[n_experts].w_up != nullptr;
    for (int t = tid; t < n_tokens; t += nt) {
        int pos = -1;
        if (shared) {
            pos = tot_pairs + t;
            P.pair_token[pos] = t;
            P.pair_weight[pos] = 1.0f;
        }
        P.token_pairs[(size_t)t * (top_k + 1) + top_k] = pos;
    }
    if (shared && tid == 0) {
        P.slot_expert[tot_slots] = n_experts;
        P.slot_pair_begin[tot_slots] = tot_pairs;
        P.slot_pair_count[tot_slots] = n_tokens;
    }
    __syncthreads();
    const int n_slots = tot_slots + (shared ? 1 : 0);
    const int schunk = (n_slots + nt - 1) / nt;
    const int s0 = min(tid * schunk, n_slots), s1 = min(s0 + schunk, n_slots);
    int my_items = 0;
    for (int s = s0; s < s1; ++s) my_items += (P.slot_pair_count[s] + item_cap - 1) / item_cap;
    int tot_items = 0;
    int it = block_excl_scan(my_items, scan, &tot_items);
    for (int s = s0; s < s1; ++s) {
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
        P.item_rec[i] = ItemRec{e.w_up, e.w_gate, e.w_down, e.s_up, e.s_gate, e.s_down,
                                P.item_pair_begin[i], P.item_pair_count[i], e.up_rb, e.gate_rb,
                                e.down_rb, 0};
    }
    // token-dense map for the decode down kernel: slot_tok_pair[s][t], t < 16
    if (P.slot_tok_pair != nullptr && n_tokens <= kTileTok) {
        __syncthreads();
        for (int i = tid; i < n_slots * kTileTok; i += nt) P.slot_tok_pair[i] = -1;
        __syncthreads();
        for (int s = tid; s < n_slots; s += nt) {
            const int pb = P.slot_pair_begin[s], pc = P.slot_pair_count[s];
            for (int q = 0; q < pc; ++q) P.slot_tok_pair[s * kTileTok + P.pair_token[pb + q]] = pb + q;
        }
    }
    if (tid == 0) {
        if (tot_items > max_items) s_err |= kErrPlanOverflow;
        P.hdr->n_slots = n_slots;
        P.hdr->n_items = min(tot_items, max_items);
        P.hdr->n_pairs = tot_pairs + (shared ? n_tokens : 0);
        if (s_err) atomicOr(err_flag, s_err);
    }
}

// Orders LDS traffic between lanes of one wave (compiler barrier; the LDS
// itself executes a wave's instructions in order).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Planner for n_tokens <= 16 run by ONE wave, no barriers and no atomics on
// global memory: same layout and order as plan_build (slots ascending by
// expert id, shared expert last, one item per slot since a slot holds <= 16
// pairs; pairs of a slot in assignment order).  Every output cell is written
// exactly once.  LDS: 3*E + 3*n_tokens*top_k ints.
__device__ void plan_wave(const int32_t* __restrict__ ids, const float* __restrict__ w,
                          int n_tokens, int top_k, const cx_expert_desc* table, int n_experts,
                          int has_shared, const PlanPtrs& P, int* err_flag, int* sm) {
    const int lane = threadIdx.x & 63;
    const int n_assign = n_tokens * top_k;
    int* cnt = sm;                      // [E] kept pairs per expert
    int* first = sm + n_experts;        // [E] first pair of the expert's slot
    int* slot_of = sm + 2 * n_experts;  // [E] slot index (where cnt > 0)
    int* eid = sm + 3 * n_experts;      // [n_assign] expert of a kept assignment, else -1
    int* pos = eid + n_assign;          // [n_assign] pair index or -1
    int err = 0;
    for (int e = lane; e < n_experts; e += 64) cnt[e] = 0;
    for (int i = lane; i < n_assign; i += 64) {
        int e = ids[i];
        if (e >= n_experts) { err |= kErrBadExpertId; e = -1; }
        else if (e >= 0 && table[e].w_up == nullptr) { err |= kErrNotResident; e = -1; }
        else if (e >= 0 && dup_route(ids, i, top_k)) { err |= kErrDuplicateRoute; e = -1; }
        eid[i] = e < 0 ? -1 : e;
    }
    wave_sync();
    for (int i = lane; i < n_assign; i += 64)
        if (eid[i] >= 0) atomicAdd(&cnt[eid[i]], 1);
    wave_sync();
    const int chunk = (n_experts + 63) / 64;
    const int e0 = min(lane * chunk, n_experts), e1 = min(e0 + chunk, n_experts);
    int mp = 0, ms = 0;
    for (int e = e0; e < e1; ++e) { mp += cnt[e]; ms += cnt[e] > 0; }
    int ip = mp, is = ms;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int a = __shfl_up(ip, off, 64), b = __shfl_up(is, off, 64);
        if (lane >= off) { ip += a; is += b; }
    }
    const int tot_pairs = __shfl(ip, 63, 64), tot_slots = __shfl(is, 63, 64);
    int po = ip - mp, so = is - ms;
    for (int e = e0; e < e1; ++e) {
        const int n = cnt[e];
        first[e] = po;
        slot_of[e] = so;
        if (n > 0) {
            const cx_expert_desc& d = table[e];
            P.slot_expert[so] = e;
            P.slot_pair_begin[so] = po;
            P.slot_pair_count[so] = n;
            P.slot_rec[so] = SlotRec{d.w_down, d.s_down, d.down_rb, 0};
            P.item_slot[so] = so;
            P.item_pair_begin[so] = po;
            P.item_pair_count[so] = n;
            P.item_rec[so] = ItemRec{d.w_up, d.w_gate, d.w_down, d.s_up, d.s_gate, d.s_down, po, n,
                                     d.up_rb, d.gate_rb, d.down_rb, 0};
            ++so;
        }
        po += n;
    }
    wave_sync();
    // pair position = first pair of the slot + earlier kept assignments of e
    for (int i = lane; i < n_assign; i += 64) {
        const int e = eid[i];
        const int t = i / top_k, k = i - t * top_k;
        int q = -1;
        if (e >= 0) {
            int before = 0;
            for (int j = 0; j < i; ++j) before += eid[j] == e;
            q = first[e] + before;
            P.pair_token[q] = t;
            P.pair_weight[q] = w[i];
        }
        pos[i] = q;
        P.token_pairs[(size_t)t * (top_k + 1) + k] = q;
    }
    wave_sync();
    // token-dense map: cell (s, t) = pair of token t in slot s, or -1
    for (int cell = lane; cell < tot_slots * kTileTok; cell += 64) {
        const int sl = cell / kTileTok, t = cell - sl * kTileTok;
        int q = -1;
        if (t < n_tokens) {
            for (int k = 0; k < top_k; ++k) {
                const int i = t * top_k + k;
                const int e = eid[i];
                if (e >= 0 && slot_of[e] == sl) q = pos[i];
            }
        }
        P.slot_tok_pair[cell] = q;
    }
    const bool shared = has_shared && table[n_experts].w_up != nullptr;
    const int n_slots = tot_slots + (shared ? 1 : 0);
    if (shared) {
        const cx_expert_desc& d = table[n_experts];
        if (lane == 0) {
            P.slot_expert[tot_slots] = n_experts;
            P.slot_pair_begin[tot_slots] = tot_pairs;
            P.slot_pair_count[tot_slots] = n_tokens;
            P.slot_rec[tot_slots] = SlotRec{d.w_down, d.s_down, d.down_rb, 0};
            P.item_slot[tot_slots] = tot_slots;
            P.item_pair_begin[tot_slots] = tot_pairs;
            P.item_pair_count[tot_slots] = n_tokens;
            P.item_rec[tot_slots] = ItemRec{d.w_up, d.w_gate, d.w_down, d.s_up, d.s_gate, d.s_down,
                                            tot_pairs, n_tokens, d.up_rb, d.gate_rb, d.down_rb, 0};
        }
        for (int t = lane; t < kTileTok; t += 64) {
            const int q = tot_pairs + t;
            if (t < n_tokens) {
                P.pair_token[q] = t;
                P.pair_weight[q] = 1.0f;
                P.token_pairs[(size_t)t * (top_k + 1) + top_k] = q;
            }
            P.slot_tok_pair[tot_slots * kTileTok + t] = t < n_tokens ? q : -1;
        }
    } else {
        for (int t = lane; t < n_tokens; t += 64) P.token_pairs[(size_t)t * (top_k + 1) + top_k] = -1;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) err |= __shfl_xor(err, off, 64);
    if (lane == 0) {
        P.hdr->n_slots = n_slots;
        P.hdr->n_items = n_slots;
        P.hdr->n_pairs = tot_pairs + (shared ? n_tokens : 0);
        if (err) atomicOr(err_flag, err);
    }
}

size_t plan_wave_lds(int n_experts, int n_tokens, int top_k) {
    return sizeof(int) * (3 * (size_t)n_experts + 2 * (size_t)n_tokens * top_k);
}

constexpr int kPlanThreads = 1024;

__global__ __launch_bounds__(64) void k_plan_wave(const int32_t* __restrict__ ids,
                                                  const float* __restrict__ w, int n_tokens,
                                                  int top_k, const cx_expert_desc* table,
                                                  int n_experts, int has_shared, PlanPtrs P,
                                                  int* err_flag) {
    extern __shared__ int smw[];
    plan_wave(ids, w, n_tokens, top_k, table, n_experts, has_shared, P, err_flag, smw);
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
    // optional planner
    int do_plan;
    const cx_expert_desc* table;
    int has_shared, item_cap, max_items;
    PlanPtrs plan;
    int* err_flag;
};

// T <= 16: selection of every token (wave t selects token t; with the
// register path all tokens run in parallel) and, for cx_moe_layer, the
// planner (one wave), in one workgroup after k_route_logits.  (A "last
// workgroup" fusion into the logits kernel needs a device-scope fence per
// workgroup, which on this multi-XCD part writes back L2 and costs far more
// than the kernel boundary.)
__global__ __launch_bounds__(1024) void k_route_select_plan(FusedArgs A) {
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
    if (A.do_plan) {
        __threadfence_block();
        __syncthreads();
        if (wave == 0)
            plan_wave(A.ids, A.wout, A.n_tokens, A.top_k, A.table, A.n_experts, A.has_shared,
                      A.plan, A.err_flag, reinterpret_cast<int*>(dyn));
    }
}

template <bool XF32, bool WF32>
__global__ __launch_bounds__(kRouteThreads) void k_route_logits(FusedArgs A) {
    __shared__ double red[4 * kRouteTB];
    const int t0 = blockIdx.y * kRouteTB;
    row_logits<XF32, WF32>(A.x, A.w, t0, min(kRouteTB, A.n_tokens - t0), A.hidden, A.n_experts,
                           A.logits, red);
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

}  // namespace

hipError_t launch_route(const RouteArgs& R, hipStream_t s) {
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
    A.do_plan = R.plan != nullptr;
    if (R.plan != nullptr) {
        A.table = R.table;
        A.has_shared = R.has_shared;
        A.item_cap = R.item_cap;
        A.max_items = R.max_items;
        A.plan = *R.plan;
        A.err_flag = R.err_flag;
    }
    A.epl = register_epl(R.n_experts, R.n_group);
    const size_t sel = A.epl ? 0 : select_lds(R.n_experts);
    const dim3 lg(R.n_experts, (R.n_tokens + kRouteTB - 1) / kRouteTB);
    const bool xf = R.x_dtype == CX_DTYPE_F32, wf = R.w_dtype == CX_DTYPE_F32;
    if (xf && wf) cx_launch((k_route_logits<true, true>), lg, dim3(kRouteThreads), 0, s, A);
    else if (xf) cx_launch((k_route_logits<true, false>), lg, dim3(kRouteThreads), 0, s, A);
    else if (wf) cx_launch((k_route_logits<false, true>), lg, dim3(kRouteThreads), 0, s, A);
    else cx_launch((k_route_logits<false, false>), lg, dim3(kRouteThreads), 0, s, A);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (R.n_tokens <= kRouteTB) {
        // register path: one wave per token, all in parallel; fallback: 4 waves
        const int threads = A.epl ? 64 * R.n_tokens : kRouteThreads;
        size_t lds = A.epl ? 0 : (size_t)2 * (threads / 64) * R.n_experts * sizeof(double) + (threads / 64) * 64;
        const size_t plan_lds = plan_wave_lds(R.n_experts, R.n_tokens, R.top_k);
        if (A.do_plan && plan_lds > lds) lds = plan_lds;
        cx_launch(k_route_select_plan, dim3(1), dim3(threads), lds, s, A);
        return hipGetLastError();
    }
    cx_launch(k_route_select, dim3((R.n_tokens + 3) / 4), dim3(kRouteThreads), sel, s, A);
    err = hipGetLastError();
    if (err != hipSuccess || R.plan == nullptr) return err;
    return launch_plan(R.ids, R.wout, R.n_tokens, R.top_k, R.table, R.n_experts, R.has_shared,
                       R.item_cap, R.max_items, *R.plan, R.err_flag, s);
}

hipError_t launch_plan(const int32_t* ids, const float* w, int n_tokens, int top_k,
                       const cx_expert_desc* table, int n_experts, int has_shared, int item_cap,
                       int max_items, PlanPtrs plan, int* err_flag, hipStream_t s) {
    if (n_tokens <= kTileTok && item_cap >= kTileTok && plan.slot_tok_pair != nullptr) {
        cx_launch(k_plan_wave, dim3(1), dim3(64), plan_wave_lds(n_experts, n_tokens, top_k),
                           s, ids, w, n_tokens, top_k, table, n_experts, has_shared, plan, err_flag);
        return hipGetLastError();
    }
    const int threads = n_tokens * top_k <= 512 ? 256 : kPlanThreads;
    const size_t lds = sizeof(int) * (2 * (size_t)n_experts + threads);
    cx_launch(k_plan, dim3(1), dim3(threads), lds, s, ids, w, n_tokens, top_k, table,
                       n_experts, has_shared, item_cap, max_items, plan, err_flag);
    return hipGetLastError();
}

int route_max_experts() { return kMaxRouteExperts; }

}  // namespace cx
