// cx_route.hip — DeepSeek-V3 router and the grouped-execution planner.
//
// Router semantics: route_token_real (server/moe_layer_runtime.py:232-408);
// the HF twin is MoEGate.forward (tmp/patched_modeling/
// modeling_deepseek_eager.py:428-540).  Logits accumulate exact products in
// fp64 and the whole selection runs in fp64, so the chosen expert sets equal
// the exact-math decision; ties break toward the lower index.
#include "cx_internal.h"

namespace cx {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bool better(double a, int ia, double b, int ib) {
    return a > b || (a == b && ia < ib);
}

// ---------------------------------------------------------------------------
// logits[t][e] = sum_k W[e][k] * x[t][k] in fp64.
// grid = (ceil(E/4), ceil(T/TB)), block = 256: one wave per expert row, TB
// tokens per workgroup.  Lane l accumulates 8-element chunks l, l+64, ...
// then a fixed xor-tree reduction: deterministic.
constexpr int kRouteTB = 8;

__device__ __forceinline__ void load8(const void* base, size_t elem, int dtype, double* v) {
    if (dtype == CX_DTYPE_F32) {
        const float* p = static_cast<const float*>(base) + elem;
        const u32x4 a = *reinterpret_cast<const u32x4*>(p);
        const u32x4 b = *reinterpret_cast<const u32x4*>(p + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = static_cast<double>(__uint_as_float(a[i]));
            v[4 + i] = static_cast<double>(__uint_as_float(b[i]));
        }
    } else {
        const u32x4 a = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + elem);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = static_cast<double>(__uint_as_float(a[i] << 16));
            v[2 * i + 1] = static_cast<double>(__uint_as_float(a[i] & 0xFFFF0000u));
        }
    }
}

__global__ __launch_bounds__(256) void k_route_logits(const void* __restrict__ x, int x_dtype,
                                                      const void* __restrict__ w, int w_dtype,
                                                      int n_tokens, int hidden, int n_experts,
                                                      double* __restrict__ logits) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = blockIdx.x * 4 + wave;
    if (e >= n_experts) return;
    const int t0 = blockIdx.y * kRouteTB;
    const int nt = min(kRouteTB, n_tokens - t0);
    double acc[kRouteTB];
#pragma unroll
    for (int t = 0; t < kRouteTB; ++t) acc[t] = 0.0;
    const int nchunk = hidden / 8;
    for (int ci = lane; ci < nchunk; ci += 64) {
        double wv[8];
        load8(w, (size_t)e * hidden + ci * 8, w_dtype, wv);
#pragma unroll
        for (int t = 0; t < kRouteTB; ++t) {
            if (t < nt) {
                double xv[8];
                load8(x, (size_t)(t0 + t) * hidden + ci * 8, x_dtype, xv);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[t] = fma(wv[i], xv[i], acc[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < kRouteTB; ++t) {
        double v = acc[t];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        if (lane == 0 && t < nt) logits[(size_t)(t0 + t) * n_experts + e] = v;
    }
}

// ---------------------------------------------------------------------------
// Selection, one workgroup per token, thread e = expert e (E <= 1024).
struct ArgMax {
    double v;
    int i;
};

__device__ ArgMax block_argmax(double v, int i, ArgMax* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const double ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(i, off, 64);
        if (oi >= 0 && (i < 0 || better(ov, oi, v, i))) { v = ov; i = oi; }
    }
    if (lane == 0) red[wave] = ArgMax{v, i};
    __syncthreads();
    ArgMax best = red[0];
    const int nw = (blockDim.x + 63) >> 6;
    for (int w = 1; w < nw; ++w) {
        const ArgMax o = red[w];
        if (o.i >= 0 && (best.i < 0 || better(o.v, o.i, best.v, best.i))) best = o;
    }
    __syncthreads();
    return best;
}

__global__ __launch_bounds__(1024) void k_route_select(const double* __restrict__ logits,
                                                       const float* __restrict__ bias,
                                                       const uint8_t* __restrict__ resident,
                                                       int n_experts, int n_group, int topk_group,
                                                       int top_k, int norm, float scale,
                                                       int32_t* __restrict__ ids,
                                                       float* __restrict__ wout) {
    __shared__ double s_c[1024];
    __shared__ double s_s[1024];
    __shared__ double s_gs[64];
    __shared__ int s_gsel[64];
    __shared__ int s_nres;
    __shared__ ArgMax s_red[16];
    __shared__ int s_ids[64];
    const int t = blockIdx.x, e = threadIdx.x;
    const int epg = n_experts / n_group;
    if (e == 0) s_nres = 0;
    __syncthreads();
    if (e < n_experts) {
        const double l = logits[(size_t)t * n_experts + e];
        const double sg = 1.0 / (1.0 + exp(-l));
        const bool res = resident == nullptr || resident[e] != 0;
        s_s[e] = res ? sg : 0.0;
        s_c[e] = res ? sg + static_cast<double>(bias[e]) : -INFINITY;
        if (res) atomicAdd(&s_nres, 1);
    }
    __syncthreads();
    if (e < n_group) {
        int i1 = -1, i2 = -1;
        for (int j = e * epg; j < (e + 1) * epg; ++j) {
            if (i1 < 0 || better(s_c[j], j, s_c[i1], i1)) { i2 = i1; i1 = j; }
            else if (i2 < 0 || better(s_c[j], j, s_c[i2], i2)) { i2 = j; }
        }
        s_gs[e] = epg >= 2 ? s_c[i1] + s_c[i2] : s_c[i1];
        s_gsel[e] = 0;
    }
    __syncthreads();
    if (e == 0) {
        for (int r = 0; r < topk_group; ++r) {
            int b = -1;
            for (int gi = 0; gi < n_group; ++gi)
                if (!s_gsel[gi] && (b < 0 || better(s_gs[gi], gi, s_gs[b], b))) b = gi;
            s_gsel[b] = 1;
        }
    }
    __syncthreads();
    double cand = -INFINITY;
    int ci = -1;
    if (e < n_experts) {
        cand = s_gsel[e / epg] ? s_c[e] : -INFINITY;
        ci = e;
    }
    const int k = min(top_k, s_nres);
    for (int r = 0; r < k; ++r) {
        const ArgMax b = block_argmax(cand, ci, s_red);
        if (e == 0) s_ids[r] = b.i;
        if (ci == b.i) ci = -1;  // taken
    }
    __syncthreads();
    if (e == 0) {
        double wsum = 0.0;
        double wv[64];
        for (int r = 0; r < k; ++r) {
            wv[r] = s_s[s_ids[r]];
            wsum += wv[r];
        }
        const double d = wsum + 1e-20;
        for (int r = 0; r < top_k; ++r) {
            if (r < k) {
                double v = wv[r];
                if (norm && k > 1) v /= d;
                v *= static_cast<double>(scale);
                ids[(size_t)t * top_k + r] = s_ids[r];
                wout[(size_t)t * top_k + r] = static_cast<float>(v);
            } else {
                ids[(size_t)t * top_k + r] = -1;
                wout[(size_t)t * top_k + r] = 0.0f;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Planner: one workgroup of 1024 threads.  Counting sort of the (token, k)
// assignments by expert id; slots in ascending expert id, shared expert last;
// items of <= item_cap pairs.  The position of a pair inside its slot only
// picks its MFMA column, which never changes its value, so the atomic
// cursor keeps results deterministic.
constexpr int kPlanThreads = 1024;

__device__ int block_excl_scan(int v, int* tmp, int* total) {
    const int tid = threadIdx.x;
    tmp[tid] = v;
    __syncthreads();
    for (int off = 1; off < kPlanThreads; off <<= 1) {
        const int a = tid >= off ? tmp[tid - off] : 0;
        __syncthreads();
        tmp[tid] += a;
        __syncthreads();
    }
    const int incl = tmp[tid];
    *total = tmp[kPlanThreads - 1];
    __syncthreads();
    return incl - v;
}

__global__ __launch_bounds__(kPlanThreads) void k_plan(const int32_t* __restrict__ ids,
                                                       const float* __restrict__ w, int n_tokens,
                                                       int top_k, const cx_expert_desc* table,
                                                       int n_experts, int has_shared, int item_cap,
                                                       int max_items, PlanPtrs P, int* err_flag) {
    extern __shared__ int sm[];
    int* cnt = sm;                    // [E]
    int* cur = sm + n_experts;        // [E]
    int* scan = sm + 2 * n_experts;   // [1024]
    __shared__ int s_err;
    const int tid = threadIdx.x;
    if (tid == 0) s_err = 0;
    for (int e = tid; e < n_experts; e += kPlanThreads) cnt[e] = 0;
    __syncthreads();
    const int n_assign = n_tokens * top_k;
    for (int i = tid; i < n_assign; i += kPlanThreads) {
        const int e = ids[i];
        if (e < 0) continue;
        if (e >= n_experts) { atomicOr(&s_err, kErrBadExpertId); continue; }
        if (table[e].w_up == nullptr) { atomicOr(&s_err, kErrNotResident); continue; }
        atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // Exclusive scans over experts (pairs, slots), chunked per thread.
    const int chunk = (n_experts + kPlanThreads - 1) / kPlanThreads;
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
    for (int i = tid; i < n_assign; i += kPlanThreads) {
        const int e = ids[i];
        const int t = i / top_k, k = i - t * top_k;
        int pos = -1;
        if (e >= 0 && e < n_experts && table[e].w_up != nullptr) {
            pos = atomicAdd(&cur[e], 1);
            P.pair_token[pos] = t;
            P.pair_weight[pos] = w[i];
        }
        P.token_pairs[(size_t)t * (top_k + 1) + k] = pos;
    }
    const bool shared = has_shared && table[n_experts].w_up != nullptr;
    for (int t = tid; t < n_tokens; t += kPlanThreads) {
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
    // Items: ceil(count / item_cap) per slot.
    const int schunk = (n_slots + kPlanThreads - 1) / kPlanThreads;
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
    if (tid == 0) {
        if (tot_items > max_items) s_err |= kErrPlanOverflow;
        P.hdr->n_slots = n_slots;
        P.hdr->n_items = min(tot_items, max_items);
        P.hdr->n_pairs = tot_pairs + (shared ? n_tokens : 0);
        if (s_err) atomicOr(err_flag, s_err);
    }
}

}  // namespace

hipError_t launch_route(const void* x, int x_dtype, const void* w, int w_dtype,
                        const float* bias, const uint8_t* resident, int n_tokens, int hidden,
                        int n_experts, int n_group, int topk_group, int top_k, int norm,
                        float scale, double* logits, int32_t* ids, float* wout, hipStream_t s) {
    const dim3 g1((n_experts + 3) / 4, (n_tokens + kRouteTB - 1) / kRouteTB);
    hipLaunchKernelGGL(k_route_logits, g1, dim3(256), 0, s, x, x_dtype, w, w_dtype, n_tokens,
                       hidden, n_experts, logits);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const int threads = ((n_experts + 63) / 64) * 64;
    hipLaunchKernelGGL(k_route_select, dim3(n_tokens), dim3(threads), 0, s, logits, bias,
                       resident, n_experts, n_group, topk_group, top_k, norm, scale, ids, wout);
    return hipGetLastError();
}

hipError_t launch_plan(const int32_t* ids, const float* w, int n_tokens, int top_k,
                       const cx_expert_desc* table, int n_experts, int has_shared, int item_cap,
                       int max_items, PlanPtrs plan, int* err_flag, hipStream_t s) {
    const size_t lds = sizeof(int) * (2 * (size_t)n_experts + kPlanThreads);
    hipLaunchKernelGGL(k_plan, dim3(1), dim3(kPlanThreads), lds, s, ids, w, n_tokens, top_k, table,
                       n_experts, has_shared, item_cap, max_items, plan, err_flag);
    return hipGetLastError();
}

}  // namespace cx
