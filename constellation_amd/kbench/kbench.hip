// cx_kbench — kernel-level measurements behind the design notes.  It compiles
// the library's kernels (cx_expert.hip) into a stand-alone program and times
// single launches with HIP events on synthetic experts placed as the HBM arena
// places them (back to back in 2 GiB chunks), so every figure it prints can be
// reproduced on one MI355X:
//
//   cx_kbench layout       grouped gate/up bytes of a config-3-like plan streamed
//                          bare (no compute) in the natural row-major order and in
//                          the tiled order a re-layout at upload would give
//   cx_kbench decode-down  one-token down projection: k_down_comb1 (down + combine
//                          in one launch) against k_down_item + k_combine_dec, and
//                          the down bytes streamed bare, row-major and as k-panels
//   cx_kbench placement    one-token gate/up and down launches with the experts
//                          packed into one buffer vs spread over 24 x 2 GiB chunks
//   cx_kbench decode-balance  one-token gate/up bytes streamed bare with tiles
//                          handed out statically or claimed from per-XCD counters,
//                          and k_down_comb1 over 256 / 384 / 448 / 512 tiles
//   cx_kbench grouped      the grouped prefill kernels on the config-3-like plan
//   cx_kbench grouped-down the plan's down bytes streamed bare in the grouped down
//                          kernel's shape, by tiles per workgroup and occupancy
//   cx_kbench fused1       one expert, one token: one launch split over inter (w_down
//                          as k-panels) + a reduce launch, against the two launches
//   cx_kbench decode-layout  one-token gate/up and down launch shapes streamed bare
//                          in natural rows and in 16-row x 128-column tiles, and
//                          k_gate_up_kpart / k_gate_up_t reading either gate/up layout
//   cx_kbench rates        per-CU rates the LDS-ring kernels are built on, in shader
//                          clocks (s_memtime): ds_read_b128 bytes per clock, bf16
//                          MFMA and fp8 -> 16-bit convert issue intervals, and
//                          whether independent converts overlap the MFMAs
//
// Bytes are synthetic (small finite fp8 codes, block scales 1e-3): the numbers
// are timings, not results.  Built by constellation_amd/build.py.
#include "cx_expert.hip"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

namespace cx {
LaunchTimer*& current_launch_timer() {
    static thread_local LaunchTimer* t = nullptr;
    return t;
}
}  // namespace cx

using namespace cx;

namespace {

#define KB_CHECK(x)                                                                      \
    do {                                                                                 \
        hipError_t e_ = (x);                                                             \
        if (e_ != hipSuccess) {                                                          \
            std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, \
                         __LINE__);                                                      \
            std::exit(1);                                                                \
        }                                                                                \
    } while (0)

constexpr int kH = 7168, kI = 2048;
constexpr size_t kMat = (size_t)kH * kI;
constexpr size_t kScaleBytes = 16 * 56 * 4;
constexpr size_t kExpert = 3 * kMat + 3 * kScaleBytes + 1024;  // as laid out in the arena
constexpr size_t kChunk = 2ull << 30;

__global__ void k_fill_bytes(uint32_t* p, size_t n, uint32_t salt) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        uint64_t z = (i + salt + 0x9E3779B97F4A7C15ull) * 0xBF58476D1CE4E5B9ull;
        z ^= z >> 31;
        z *= 0x94D049BB133111EBull;
        z ^= z >> 29;
        p[i] = (uint32_t)z & 0x3E3E3E3Eu;  // four finite fp8 codes of magnitude < 1
    }
}

__global__ void k_fill_f32(float* p, size_t n, float v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

// Synthetic experts: `spread` places them back to back in 24 chunks of 2 GiB
// (1152 experts, ~50 GB, as four resident layer copies occupy the arena);
// otherwise 48 experts in one 2.1 GB buffer.
struct Pool {
    std::vector<uint8_t*> chunks;
    std::vector<cx_expert_desc> d;
    explicit Pool(bool spread, int gu_layout = CX_LAYOUT_ROWS) {
        const int per_chunk = (int)(kChunk / kExpert);
        const int n_chunks = spread ? 24 : 1;
        const size_t bytes = spread ? kChunk : kExpert * 48;
        for (int c = 0; c < n_chunks; ++c) {
            uint8_t* p = nullptr;
            KB_CHECK(hipMalloc(&p, bytes));
            k_fill_bytes<<<4096, 256>>>((uint32_t*)p, bytes / 4, 1 + c);
            chunks.push_back(p);
        }
        const int n = spread ? n_chunks * per_chunk : 48;
        d.resize(n);
        for (int e = 0; e < n; ++e) {
            uint8_t* b = spread ? chunks[e / per_chunk] + (size_t)(e % per_chunk) * kExpert
                                : chunks[0] + (size_t)e * kExpert;
            cx_expert_desc& q = d[e];
            q.w_up = b;
            q.w_gate = b + kMat;
            q.w_down = b + 2 * kMat;
            float* s = (float*)(b + 3 * kMat);
            q.s_up = s;
            q.s_gate = s + 16 * 56;
            q.s_down = s + 2 * 16 * 56;
            k_fill_f32<<<16, 256>>>(s, 3 * 16 * 56, 1e-3f);
            q.hidden = kH;
            q.inter = kI;
            q.up_rb = q.up_cb = q.gate_rb = q.gate_cb = q.down_rb = q.down_cb = 128;
            q.gu_layout = gu_layout;
        }
        KB_CHECK(hipDeviceSynchronize());
    }
    ~Pool() {
        for (uint8_t* p : chunks) (void)hipFree(p);
    }
};

template <class T>
T* dev_copy(const std::vector<T>& v) {
    T* p = nullptr;
    KB_CHECK(hipMalloc(&p, std::max<size_t>(1, v.size()) * sizeof(T)));
    if (!v.empty()) KB_CHECK(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
    return p;
}

ItemRec item_of(const cx_expert_desc& q, int pb, int np) {
    return ItemRec{q.w_up, q.w_gate, q.w_down, q.s_up, q.s_gate, q.s_down, pb, np, 128, 128, 128, q.gu_layout, {0, 0, 0, 0}};
}

// Average single-launch time (us) of `n` launches issued back to back, each
// bracketed by its own start/stop events (the launcher's LaunchTimer).
template <class F>
double time_launches(int n, F fn) {
    for (int i = 0; i < 2; ++i) fn(i);
    KB_CHECK(hipDeviceSynchronize());
    std::vector<LaunchTimer> t(n);
    for (auto& x : t) {
        KB_CHECK(hipEventCreate(&x.start));
        KB_CHECK(hipEventCreate(&x.stop));
    }
    for (int i = 0; i < n; ++i) {
        current_launch_timer() = &t[i];
        fn(i);
    }
    current_launch_timer() = nullptr;
    KB_CHECK(hipDeviceSynchronize());
    double sum = 0;
    for (auto& x : t) {
        float ms = 0;
        KB_CHECK(hipEventElapsedTime(&ms, x.start, x.stop));
        sum += ms * 1e3;
        (void)hipEventDestroy(x.start);
        (void)hipEventDestroy(x.stop);
    }
    return sum / n;
}

void report(const char* what, double us, double bytes) {
    std::printf("  %-58s %9.2f us  %6.2f TB/s\n", what, us, bytes / us * 1e-6);
    std::fflush(stdout);
}

// ---------------------------------------------------------------------------
// One-token decode plans: 8 routed experts + the shared expert (pairs: shared
// 0, routed 1..8, as the decode planner numbers them).
struct DecodePlans {
    std::vector<PlanPtrs> plans;
    std::vector<cx_expert_desc> shared;
    float* topk_w = nullptr;
    uint16_t *x = nullptr, *h_hi = nullptr, *h_lo = nullptr, *y = nullptr;
    float* y_part = nullptr;
    DecodePlans(const Pool& pool, int n_plans, uint32_t seed) {
        std::mt19937 rng(seed);
        const int n_exp = (int)pool.d.size();
        for (int pi = 0; pi < n_plans; ++pi) {
            std::vector<int> pick;
            while ((int)pick.size() < 9) {
                const int e = rng() % n_exp;
                if (std::find(pick.begin(), pick.end(), e) == pick.end()) pick.push_back(e);
            }
            std::sort(pick.begin(), pick.begin() + 8);
            std::vector<ItemRec> rec;
            for (int i = 0; i < 8; ++i) rec.push_back(item_of(pool.d[pick[i]], 1 + i, 1));
            rec.push_back(item_of(pool.d[pick[8]], 0, 1));
            PlanPtrs P{};
            PlanHdr h{};
            h.n_slots = h.n_items = h.n_pairs = 9;
            h.n_routed_slots = h.n_routed_items = 8;
            P.hdr = dev_copy(std::vector<PlanHdr>{h});
            P.item_rec = dev_copy(rec);
            P.token_pairs = dev_copy(std::vector<int>{1, 2, 3, 4, 5, 6, 7, 8, 0});
            P.pair_row = dev_copy(std::vector<int>{0, 1, 2, 3, 4, 5, 6, 7, 8});
            plans.push_back(P);
            shared.push_back(pool.d[pick[8]]);
        }
        topk_w = dev_copy(std::vector<float>{0.3f, 0.25f, 0.2f, 0.4f, 0.35f, 0.3f, 0.4f, 0.3f});
        KB_CHECK(hipMalloc(&x, kH * 2));
        KB_CHECK(hipMalloc(&h_hi, 16 * kI * 2));
        KB_CHECK(hipMalloc(&h_lo, 16 * kI * 2));
        KB_CHECK(hipMalloc(&y, kH * 2));
        KB_CHECK(hipMalloc(&y_part, 16 * (size_t)kH * 4));
        k_fill_bytes<<<16, 256>>>((uint32_t*)x, kH / 2, 7);
        k_fill_bytes<<<64, 256>>>((uint32_t*)h_hi, 16 * kI / 2, 9);
        k_fill_bytes<<<64, 256>>>((uint32_t*)h_lo, 16 * kI / 2, 10);
        KB_CHECK(hipDeviceSynchronize());
    }
    ExpertLaunch launch(int pi, const cx_expert_desc* table, int max_lds) const {
        ExpertLaunch L{};
        L.table = table;
        L.plan = plans[pi % plans.size()];
        L.max_items = 8;
        L.n_tokens = 1;
        L.hidden = kH;
        L.inter = kI;
        L.maxt = 1;
        L.x = x;
        L.in_dtype = CX_DTYPE_BF16;
        L.h_hi = h_hi;
        L.h_lo = h_lo;
        L.y_part = y_part;
        L.y = y;
        L.out_dtype = CX_DTYPE_BF16;
        L.np_lds = 1;
        L.skip_shared = 1;
        L.max_lds = max_lds;
        return L;
    }
};

int max_lds() {
    int v = 0;
    KB_CHECK(hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, 0));
    return v;
}

int n_cu() {
    int v = 0;
    KB_CHECK(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, 0));
    return v;
}

// Bare stream of the one-token down's bytes (no compute): 9 matrices, the
// k_down_item shape (workgroup = one item x 64 rows, full-K waves) or the
// k_down_comb1 shape (workgroup = 16 rows x all items: wave w = item w's 16
// k-blocks then 2 k-blocks of the shared expert, one 8-deep ring).
struct DownPtrs {
    const uint8_t* m[9];
};

__device__ __forceinline__ uint32_t fold(const u32x4 (&w)[2]) {
    return w[0][0] + w[0][1] * 3u + w[0][2] * 5u + w[0][3] * 7u + w[1][0] * 11u + w[1][1] * 13u + w[1][2] + w[1][3];
}

// KP: the layout the matrices are read in; the bytes each lane loads are
// the same in all three (row r, k-block k, quarter g: 32 bytes as two
// 16-byte pieces p = 0, 1):
//   0  row-major [H][I]:               r * I + 128 k + 32 g + 16 p
//   1  32-column k-panels [I/32][H][32]: ((4k + g) * H + r) * 32 + 16 p
//      (a wave's 16 rows of one quarter are 512 contiguous bytes)
//   2  16-column k-panels [I/16][H][16]: ((8k + 2g + p) * H + r) * 16
//      (each 16-byte load instruction reads 8 whole 128-byte lines)
template <int KP>
__device__ __forceinline__ size_t down_off(size_t r, int k, int g, int p) {
    if (KP == 1) return ((size_t)(4 * k + g) * kH + r) * 32 + 16 * p;
    if (KP == 2) return ((size_t)(8 * k + 2 * g + p) * kH + r) * 16;
    return r * kI + (size_t)k * kKB + g * 32 + 16 * p;
}

template <int KP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_bare_down_item(DownPtrs P, uint32_t* sink) {
    constexpr int NKB = 16, D = 6;
    const int wave = wave_id(), lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const size_t r = (size_t)(blockIdx.x * 64 + wave * 16 + c);
    const uint8_t* m = P.m[blockIdx.y];
    u32x4 wb[D][2];
    uint32_t acc = 0;
#pragma unroll
    for (int s = 0; s < D; ++s) {
        wb[s][0] = ld16(m + down_off<KP>(r, s, g, 0));
        wb[s][1] = ld16(m + down_off<KP>(r, s, g, 1));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < NKB; ++k) {
        acc ^= fold(wb[k % D]);
        __builtin_amdgcn_sched_barrier(0);
        if (k + D < NKB) {
            wb[k % D][0] = ld16(m + down_off<KP>(r, k + D, g, 0));
            wb[k % D][1] = ld16(m + down_off<KP>(r, k + D, g, 1));
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if (acc == 0x12345678u) sink[threadIdx.x] = acc;
}

template <int KP>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void k_bare_down_rows(DownPtrs P, uint32_t* sink) {
    constexpr int NK = 18, D = 8;
    const int wave = wave_id(), lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const size_t r = (size_t)(blockIdx.x * 16 + c);
    auto at = [&](int k, int p) {
        return k < 16 ? P.m[wave] + down_off<KP>(r, k, g, p) : P.m[8] + down_off<KP>(r, 2 * wave + k - 16, g, p);
    };
    u32x4 wb[D][2];
    uint32_t acc = 0;
#pragma unroll
    for (int s = 0; s < D; ++s) {
        wb[s][0] = ld16(at(s, 0));
        wb[s][1] = ld16(at(s, 1));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < NK; ++k) {
        acc ^= fold(wb[k % D]);
        __builtin_amdgcn_sched_barrier(0);
        if (k + D < NK) {
            wb[k % D][0] = ld16(at(k + D, 0));
            wb[k % D][1] = ld16(at(k + D, 1));
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if (acc == 0x12345678u) sink[threadIdx.x] = acc;
}

int cmd_decode_down(int iters) {
    std::printf("decode-down: one token, 8 routed + shared expert, experts spread over 24 x 2 GiB\n");
    Pool pool(true);
    DecodePlans dp(pool, 16, 3);
    cx_expert_desc* table = dev_copy(pool.d);
    uint32_t* sink = nullptr;
    KB_CHECK(hipMalloc(&sink, 4096));
    const int lds = max_lds();
    const int cus = n_cu();
    const double down_bytes = 9.0 * (kMat + 56 * 16 * 4) + 2.0 * kH;
    std::mt19937 rng(11);
    std::vector<DownPtrs> sets(16);
    for (auto& s : sets)
        for (int j = 0; j < 9; ++j) s.m[j] = pool.d[rng() % pool.d.size()].w_down;
    for (int rep = 0; rep < 2; ++rep) {
        std::printf(" pass %d\n", rep + 1);
        report("bare stream, k_down_item shape (item x 64 rows)",
               time_launches(iters, [&](int i) {
                   cx_launch(k_bare_down_item<0>, dim3(112, 9), dim3(256), 0u, (hipStream_t)0, sets[i % 16], sink);
               }), 9.0 * kMat);
        report("  same bytes as 32-column k-panels",
               time_launches(iters, [&](int i) {
                   cx_launch(k_bare_down_item<1>, dim3(112, 9), dim3(256), 0u, (hipStream_t)0, sets[i % 16], sink);
               }), 9.0 * kMat);
        report("  same bytes as 16-column k-panels",
               time_launches(iters, [&](int i) {
                   cx_launch(k_bare_down_item<2>, dim3(112, 9), dim3(256), 0u, (hipStream_t)0, sets[i % 16], sink);
               }), 9.0 * kMat);
        report("bare stream, k_down_comb1 shape (16 rows x all items)",
               time_launches(iters, [&](int i) {
                   cx_launch(k_bare_down_rows<0>, dim3(kH / 16), dim3(512), 0u, (hipStream_t)0, sets[i % 16], sink);
               }), 9.0 * kMat);
        report("  same bytes as 32-column k-panels",
               time_launches(iters, [&](int i) {
                   cx_launch(k_bare_down_rows<1>, dim3(kH / 16), dim3(512), 0u, (hipStream_t)0, sets[i % 16], sink);
               }), 9.0 * kMat);
        report("  same bytes as 16-column k-panels",
               time_launches(iters, [&](int i) {
                   cx_launch(k_bare_down_rows<2>, dim3(kH / 16), dim3(512), 0u, (hipStream_t)0, sets[i % 16], sink);
               }), 9.0 * kMat);
        report("k_down_comb1 (down + combine)", time_launches(iters, [&](int i) {
                   ExpertLaunch L = dp.launch(i, table, lds);
                   L.skip_shared = 0;
                   L.max_items = 9;
                   KB_CHECK(launch_down_comb1(L, L.plan.token_pairs, dp.topk_w, 8, cus, 0));
               }), down_bytes);
        report("k_down_item (down, 9 items)", time_launches(iters, [&](int i) {
                   ExpertLaunch L = dp.launch(i, table, lds);
                   L.skip_shared = 0;
                   L.max_items = 9;
                   KB_CHECK(launch_down(L, 0));
               }), down_bytes);
        report("k_combine_dec (combine)", time_launches(iters, [&](int i) {
                   ExpertLaunch L = dp.launch(i, table, lds);
                   KB_CHECK(launch_combine_dec(L.plan, dp.topk_w, L.y_part, 1, 8, 1, kH, L.y, CX_DTYPE_BF16,
                                               nullptr, 0));
               }), 9.0 * kH * 4);
    }
    return 0;
}

int cmd_placement(int iters) {
    for (int spread = 0; spread < 2; ++spread) {
        Pool pool(spread == 1);
        std::printf("placement: %s (%zu experts)\n", spread ? "24 x 2 GiB chunks" : "one 2.1 GB buffer",
                    pool.d.size());
        DecodePlans dp(pool, 16, 3);
        cx_expert_desc* table = dev_copy(pool.d);
        const int lds = max_lds();
        const int cus = n_cu();
        const double gu_bytes = 8.0 * (2 * kMat + 2 * 16 * 56 * 4) + kH * 2;
        const double down_bytes = 9.0 * (kMat + 56 * 16 * 4) + 2.0 * kH;
        report("k_gate_up_t (8 routed experts)", time_launches(iters, [&](int i) {
                   KB_CHECK(launch_gate_up(dp.launch(i, table, lds), 0));
               }), gu_bytes);
        report("k_down_comb1 (8 routed + shared, combine)", time_launches(iters, [&](int i) {
                   ExpertLaunch L = dp.launch(i, table, lds);
                   L.skip_shared = 0;
                   L.max_items = 9;
                   KB_CHECK(launch_down_comb1(L, L.plan.token_pairs, dp.topk_w, 8, cus, 0));
               }), down_bytes);
        (void)hipFree(table);
    }
    return 0;
}

// ---------------------------------------------------------------------------
// Tile balance at one token.  A tile of the routed gate/up = 16 rows x full K
// of one expert's gate and up (4 waves x K/4, the k_gate_up_t shape), 8 x 128
// tiles.  The bare stream (no compute) hands tiles out three ways — MODE 0:
// workgroup b streams tiles b, b + grid, ...; MODE 1: per-XCD pools (tile
// 8j + x for pool x = b % 8, the dispatcher's round-robin XCD), first tile
// static, then claims from the pool's counter, requested before the current
// tile streams and read after it.  Claims only grow, so every workgroup
// exits and every tile is streamed once.
struct GuPtrs {
    const uint8_t* gate[8];
    const uint8_t* up[8];
};

__device__ __forceinline__ uint32_t bare_gu_tile(const GuPtrs& P, int t) {
    constexpr int NKB = 14, D = 4;
    const int e = t >> 7, rt = t & 127;
    const int wave = wave_id(), lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const size_t off = (size_t)(rt * 16 + c) * kH + (size_t)wave * NKB * kKB + g * 32;
    const uint8_t* pg = P.gate[e] + off;
    const uint8_t* pu = P.up[e] + off;
    u32x4 wg[D][2], wu[D][2];
    uint32_t acc = 0;
#pragma unroll
    for (int s = 0; s < D; ++s) {
        wg[s][0] = ld16(pg + s * kKB);
        wg[s][1] = ld16(pg + s * kKB + 16);
        wu[s][0] = ld16(pu + s * kKB);
        wu[s][1] = ld16(pu + s * kKB + 16);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < NKB; ++k) {
        acc ^= fold(wg[k % D]) + fold(wu[k % D]);
        __builtin_amdgcn_sched_barrier(0);
        if (k + D < NKB) {
            wg[k % D][0] = ld16(pg + (k + D) * kKB);
            wg[k % D][1] = ld16(pg + (k + D) * kKB + 16);
            wu[k % D][0] = ld16(pu + (k + D) * kKB);
            wu[k % D][1] = ld16(pu + (k + D) * kKB + 16);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    return acc;
}

template <int MODE>
__global__ __launch_bounds__(256) void k_bare_gu_tiles(GuPtrs P, uint32_t* sink, int* ctr) {
    constexpr int n_tiles = 8 * 128, pool = n_tiles / 8;
    __shared__ int next;
    uint32_t acc = 0;
    if (MODE == 0) {
        for (int t = blockIdx.x; t < n_tiles; t += gridDim.x) acc ^= bare_gu_tile(P, t);
    } else {
        const int x = blockIdx.x & 7, per = gridDim.x >> 3;
        int j = blockIdx.x >> 3;
        while (j < pool) {
            if (threadIdx.x == 0) next = atomicAdd(ctr + x * 32, 1) + per;
            acc ^= bare_gu_tile(P, j * 8 + x);
            __syncthreads();
            j = next;
            __syncthreads();
        }
    }
    if (acc == 0x12345678u) sink[threadIdx.x] = acc;
}

int cmd_decode_balance(int iters) {
    std::printf("decode-balance: one token, experts spread over 24 x 2 GiB\n");
    Pool pool(true);
    DecodePlans dp(pool, 16, 3);
    cx_expert_desc* table = dev_copy(pool.d);
    uint32_t* sink = nullptr;
    int* ctr = nullptr;
    KB_CHECK(hipMalloc(&sink, 4096));
    KB_CHECK(hipMalloc(&ctr, 8 * 32 * sizeof(int)));
    const int lds = max_lds();
    const double gu_bytes = 8.0 * 2 * kMat;
    std::mt19937 rng(13);
    std::vector<GuPtrs> sets(16);
    for (auto& s : sets)
        for (int j = 0; j < 8; ++j) {
            const cx_expert_desc& q = pool.d[rng() % pool.d.size()];
            s.gate[j] = q.w_gate;
            s.up[j] = q.w_up;
        }
    auto bare = [&](const char* what, int mode, int grid) {
        report(what, time_launches(iters, [&](int i) {
                   KB_CHECK(hipMemsetAsync(ctr, 0, 8 * 32 * sizeof(int), 0));
                   if (mode == 0)
                       cx_launch(k_bare_gu_tiles<0>, dim3(grid), dim3(256), 0u, (hipStream_t)0, sets[i % 16], sink, ctr);
                   else
                       cx_launch(k_bare_gu_tiles<1>, dim3(grid), dim3(256), 0u, (hipStream_t)0, sets[i % 16], sink, ctr);
               }), gu_bytes);
    };
    // k_down_comb1 over the first `grid` tiles of `rows` rows (the library
    // kernel; grids below hidden / rows leave the last rows unwritten)
    const double tile_bytes = 9.0 * 16 * kI;
    auto down = [&](const char* what, int grid, int rows) {
        report(what, time_launches(iters, [&](int i) {
                   ExpertLaunch L = dp.launch(i, table, lds);
                   L.skip_shared = 0;
                   L.max_items = 9;
                   cx_launch((k_down_comb1<16, kDc1Depth>), dim3(grid), dim3(64 * kDc1Waves),
                             (uint32_t)down_comb1_lds(kI), (hipStream_t)0, L, L.plan.token_pairs,
                             (const float*)dp.topk_w, 8, rows);
               }), tile_bytes / 16 * rows * grid);
    };
    for (int rep = 0; rep < 2; ++rep) {
        std::printf(" pass %d\n", rep + 1);
        report("k_gate_up_t (8 routed experts)", time_launches(iters, [&](int i) {
                   KB_CHECK(launch_gate_up(dp.launch(i, table, lds), 0));
               }), gu_bytes);
        bare("bare gate/up: static, 1024 workgroups x 1 tile", 0, 1024);
        bare("bare gate/up: static, 512 workgroups x 2 tiles", 0, 512);
        bare("bare gate/up: static, 256 workgroups x 4 tiles", 0, 256);
        bare("bare gate/up: per-XCD claims, 768 workgroups", 1, 768);
        bare("bare gate/up: per-XCD claims, 512 workgroups", 1, 512);
        bare("bare gate/up: per-XCD claims, 256 workgroups", 1, 256);
        down("k_down_comb1: first 256 tiles of 16 rows", 256, 16);
        down("k_down_comb1: first 384 tiles of 16 rows", 384, 16);
        down("k_down_comb1: 448 tiles of 16 rows (all rows)", kH / 16, 16);
        down("k_down_comb1: 512 tiles of 14 rows (all rows)", kH / 14, 14);
    }
    (void)hipFree(ctr);
    (void)hipFree(sink);
    (void)hipFree(table);
    return 0;
}

// ---------------------------------------------------------------------------
// Config-3-like prefill plan: 512 tokens, 256 routed experts whose pair counts
// follow 1 + 12 rank^-1.1 (sum 4096, max ~170), plus the shared expert's 512
// pairs; items of <= 64 pairs as the general planner cuts them.
struct PrefillPlan {
    ExpertLaunch L{};
    int n_items = 0, n_routed_items = 0;
    int tiles[5] = {0, 0, 0, 0, 0};
    PrefillPlan(const Pool& pool, uint32_t seed) {
        const int T = 512, E = 256, P = T * 8 + T;
        std::mt19937 rng(seed);
        std::vector<int> perm(E);
        for (int e = 0; e < E; ++e) perm[e] = e;
        std::shuffle(perm.begin(), perm.end(), rng);
        std::vector<double> wgt(E);
        double sum = 0;
        for (int r = 0; r < E; ++r) {
            wgt[perm[r]] = 1.0 + 12.0 * std::pow(r + 1, -1.1);
            sum += wgt[perm[r]];
        }
        std::vector<int> cnt(E);
        int tot = 0;
        for (int e = 0; e < E; ++e) {
            cnt[e] = std::max(1, (int)std::floor(4096 * wgt[e] / sum));
            tot += cnt[e];
        }
        for (int e = 0; tot < 4096; e = (e + 1) % E, ++tot) cnt[e]++;
        std::vector<int> pick;
        while ((int)pick.size() < E + 1) {
            const int e = rng() % pool.d.size();
            if (std::find(pick.begin(), pick.end(), e) == pick.end()) pick.push_back(e);
        }
        std::vector<ItemRec> items;
        std::vector<int> ptok(P);
        int p = T;
        for (int e = 0; e < E; ++e) {
            for (int o = 0; o < cnt[e]; o += 64) {
                const int np = std::min(64, cnt[e] - o);
                items.push_back(item_of(pool.d[pick[e]], p + o, np));
                tiles[(np + 15) / 16]++;
            }
            for (int j = 0; j < cnt[e]; ++j) ptok[p + j] = rng() % T;
            p += cnt[e];
        }
        n_routed_items = (int)items.size();
        for (int o = 0; o < T; o += 64) items.push_back(item_of(pool.d[pick[E]], o, 64));
        for (int t = 0; t < T; ++t) ptok[t] = t;
        n_items = (int)items.size();
        PlanHdr h{};
        h.n_slots = E + 1;
        h.n_items = n_items;
        h.n_pairs = P;
        h.n_routed_slots = E;
        h.n_routed_items = n_routed_items;
        PlanPtrs PP{};
        PP.hdr = dev_copy(std::vector<PlanHdr>{h});
        PP.item_rec = dev_copy(items);
        PP.pair_token = dev_copy(ptok);
        uint16_t *x = nullptr, *hh = nullptr, *hl = nullptr;
        float* yp = nullptr;
        KB_CHECK(hipMalloc(&x, (size_t)T * kH * 2));
        KB_CHECK(hipMalloc(&hh, (size_t)P * kI * 2));
        KB_CHECK(hipMalloc(&hl, (size_t)P * kI * 2));
        KB_CHECK(hipMalloc(&yp, (size_t)P * kH * 4));
        k_fill_bytes<<<1024, 256>>>((uint32_t*)x, (size_t)T * kH / 2, 7);
        k_fill_bytes<<<1024, 256>>>((uint32_t*)hh, (size_t)P * kI / 2, 9);
        k_fill_bytes<<<1024, 256>>>((uint32_t*)hl, (size_t)P * kI / 2, 10);
        L.table = dev_copy(pool.d);  // grouped mode (the grouped kernels read the plan's records)
        L.plan = PP;
        L.max_items = n_items;
        L.n_tokens = T;
        L.hidden = kH;
        L.inter = kI;
        L.maxt = 4;
        L.x = x;
        L.in_dtype = CX_DTYPE_BF16;
        L.h_hi = hh;
        L.h_lo = hl;
        L.y_part = yp;
        L.out_dtype = CX_DTYPE_BF16;
        L.max_lds = max_lds();
        KB_CHECK(hipDeviceSynchronize());
    }
};

// Bare streams over a prefill plan's gate/up bytes.  ORDER 0: the grouped
// kernel's pattern (128-row workgroups, wave = 16 rows x full K, row-major
// bytes); ORDER 1: 16-row workgroups, wave = 16 rows x K/4 (the decode
// gate/up's pattern); ORDER 2: 128-row workgroups, full-K waves, reading the
// same bytes in tiled order ([16-row group][k-block][16 rows x 128 B]
// contiguous), the order a re-layout at upload would store.
template <int ORDER>
__global__ __launch_bounds__(512) void k_bare_gu(ExpertLaunch L, uint32_t* sink) {
    constexpr int TILES = ORDER == 1 ? kI / 16 : kI / 128;
    const int tile = blockIdx.x % TILES, item = blockIdx.x / TILES;
    const int wave = wave_id(), lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    if (ORDER == 1 && wave >= 4) return;
    const ItemRec r = ld_uniform(L.plan.item_rec + item);
    constexpr int NKB = ORDER == 1 ? 14 : 56, D = 4;
    const int rg = ORDER == 1 ? tile : tile * 8 + wave;  // 16-row group
    const int kb0 = ORDER == 1 ? wave * 14 : 0;
    auto at = [&](const uint8_t* m, int k) -> const uint8_t* {
        if (ORDER == 2) return m + ((size_t)rg * 56 + k) * 2048 + (size_t)lane * 32;
        return m + (size_t)(rg * 16 + c) * kH + (size_t)(kb0 + k) * kKB + g * 32;
    };
    u32x4 wb[D][4];
    uint32_t acc = 0;
#pragma unroll
    for (int s = 0; s < D; ++s) {
        wb[s][0] = ld16(at(r.w_gate, s));
        wb[s][1] = ld16(at(r.w_gate, s) + 16);
        wb[s][2] = ld16(at(r.w_up, s));
        wb[s][3] = ld16(at(r.w_up, s) + 16);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll 4
    for (int k = 0; k < NKB; ++k) {
        const int s = k % D;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc ^= wb[s][j][0] + wb[s][j][1] * 3u + wb[s][j][2] * 5u + wb[s][j][3] * 7u;
        if (k + D < NKB) {
            __builtin_amdgcn_sched_barrier(0);
            wb[s][0] = ld16(at(r.w_gate, k + D));
            wb[s][1] = ld16(at(r.w_gate, k + D) + 16);
            wb[s][2] = ld16(at(r.w_up, k + D));
            wb[s][3] = ld16(at(r.w_up, k + D) + 16);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (acc == 0x12345678u) sink[threadIdx.x] = acc;
}

int cmd_layout(int iters) {
    Pool pool(true);
    std::vector<PrefillPlan> plans;
    for (int l = 0; l < 4; ++l) plans.emplace_back(pool, 5 + l);
    const PrefillPlan& p0 = plans[0];
    std::printf("layout: config-3-like plan, %d items (%d routed; column tiles 1:%d 2:%d 3:%d 4:%d), "
                "experts spread over 24 x 2 GiB\n",
                p0.n_items, p0.n_routed_items, p0.tiles[1], p0.tiles[2], p0.tiles[3], p0.tiles[4]);
    uint32_t* sink = nullptr;
    KB_CHECK(hipMalloc(&sink, 4096));
    const double bytes = 257.0 * 2 * kMat;
    for (int rep = 0; rep < 2; ++rep) {
        std::printf(" pass %d\n", rep + 1);
        report("natural order, 128-row workgroups, full-K waves", time_launches(iters, [&](int i) {
                   const PrefillPlan& p = plans[i % 4];
                   cx_launch(k_bare_gu<0>, dim3(16 * p.n_items), dim3(512), 0u, (hipStream_t)0, p.L, sink);
               }), bytes);
        report("natural order, 16-row workgroups, K/4 waves", time_launches(iters, [&](int i) {
                   const PrefillPlan& p = plans[i % 4];
                   cx_launch(k_bare_gu<1>, dim3(128 * p.n_items), dim3(256), 0u, (hipStream_t)0, p.L, sink);
               }), bytes);
        report("tiled order (re-layout at upload), 128-row workgroups", time_launches(iters, [&](int i) {
                   const PrefillPlan& p = plans[i % 4];
                   cx_launch(k_bare_gu<2>, dim3(16 * p.n_items), dim3(512), 0u, (hipStream_t)0, p.L, sink);
               }), bytes);
        report("k_gu_grp (the kernel, natural order)", time_launches(iters, [&](int i) {
                   KB_CHECK(launch_gate_up(plans[i % 4].L, 0));
               }), bytes + 512.0 * kH * 2);
    }
    return 0;
}

// Bare streams of a prefill plan's down bytes in the grouped down kernel's
// shape: 256-row workgroups (8 waves x 32 rows as two 16-row tiles), full-K
// waves (16 k-blocks), a 4-deep register ring, no compute.  Each workgroup
// takes M consecutive 256-row tiles of one item, the ring running on from
// one tile into the next (so a workgroup ramps up and drains once per M
// tiles).  Launched with 100 KB of dynamic LDS it runs one workgroup per CU,
// as the grouped down kernel does (242 VGPRs).
// ST: after its stream, each workgroup writes its 256 rows of every pair of
// the item into y_part (fp32, streamed stores), as the grouped down does.
template <int M, bool ST = false>
__global__ __launch_bounds__(512) void k_bare_dn(ExpertLaunch L, uint32_t* sink) {
    constexpr int NKB = 16, D = 4, WPI = kH / 256 / M;  // workgroups per item
    static_assert(kH % (256 * M) == 0, "tiles per workgroup divide the item's tiles");
    extern __shared__ uint32_t dyn_lds[];
    const int wg = blockIdx.x % WPI, item = blockIdx.x / WPI;
    const int wave = wave_id(), lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const ItemRec r = ld_uniform(L.plan.item_rec + item);
    auto at = [&](int k, int half) {
        const int t = wg * M + k / NKB;
        return r.w_down + (size_t)(t * 256 + wave * 32 + half * 16 + c) * kI + (size_t)(k % NKB) * kKB + g * 32;
    };
    u32x4 wb[D][4];
    uint32_t acc = 0;
#pragma unroll
    for (int s = 0; s < D; ++s) {
        wb[s][0] = ld16(at(s, 0));
        wb[s][1] = ld16(at(s, 0) + 16);
        wb[s][2] = ld16(at(s, 1));
        wb[s][3] = ld16(at(s, 1) + 16);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll 4
    for (int k = 0; k < M * NKB; ++k) {
        const int s = k % D;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc ^= wb[s][j][0] + wb[s][j][1] * 3u + wb[s][j][2] * 5u + wb[s][j][3] * 7u;
        if (k + D < M * NKB) {
            __builtin_amdgcn_sched_barrier(0);
            wb[s][0] = ld16(at(k + D, 0));
            wb[s][1] = ld16(at(k + D, 0) + 16);
            wb[s][2] = ld16(at(k + D, 1));
            wb[s][3] = ld16(at(k + D, 1) + 16);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (ST) {
        const f32x4 v = {(float)(acc & 0xff), 0.f, 0.f, 0.f};
        for (int t = 0; t < M; ++t)
            for (int q = c; q < r.np; q += 16)
                for (int a = 0; a < 2; ++a)
                    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(
                        L.y_part + (size_t)(r.pb + q) * kH + (wg * M + t) * 256 + wave * 32 + a * 16 + 4 * g));
    } else if (acc == 0x12345678u) {
        dyn_lds[threadIdx.x] = acc;
        sink[threadIdx.x] = dyn_lds[(threadIdx.x + 1) & 511];
    }
}

int cmd_grouped_down(int iters) {
    Pool pool(true);
    std::vector<PrefillPlan> plans;
    for (int l = 0; l < 4; ++l) plans.emplace_back(pool, 5 + l);
    std::printf("grouped-down: config-3-like plan, %d items, experts spread over 24 x 2 GiB\n", plans[0].n_items);
    uint32_t* sink = nullptr;
    KB_CHECK(hipMalloc(&sink, 4096));
    const double streamed = (double)plans[0].n_items * kMat;  // every item streams its expert's down matrix
    const double dn = 257.0 * kMat + 4608.0 * kH * 4;
    const uint32_t one_per_cu = 100u * 1024u;
    auto bare = [&](const char* what, auto kernel, int m, uint32_t lds) {
        report(what, time_launches(iters, [&](int i) {
                   const PrefillPlan& p = plans[i % 4];
                   cx_launch(kernel, dim3(kH / 256 / m * p.n_items), dim3(512), lds, (hipStream_t)0, p.L, sink);
               }), streamed);
    };
    for (int rep = 0; rep < 2; ++rep) {
        std::printf(" pass %d (bare lines: bytes streamed = items x down matrix)\n", rep + 1);
        bare("bare down, 1 tile per workgroup, occupancy free", k_bare_dn<1>, 1, 0u);
        bare("bare down, 1 tile per workgroup, 1 workgroup per CU", k_bare_dn<1>, 1, one_per_cu);
        bare("bare down, 2 tiles per workgroup, 1 workgroup per CU", k_bare_dn<2>, 2, one_per_cu);
        bare("bare down, 4 tiles per workgroup, 1 workgroup per CU", k_bare_dn<4>, 4, one_per_cu);
        bare("bare down, 7 tiles per workgroup, 1 workgroup per CU", k_bare_dn<7>, 7, one_per_cu);
        bare("bare down + the fp32 y_part stores, 1 tile per workgroup", k_bare_dn<1, true>, 1, one_per_cu);
        report("k_dn_grp (algorithmic bytes)", time_launches(iters, [&](int i) {
                   KB_CHECK(launch_down(plans[i % 4].L, 0));
               }), dn);
    }
    (void)hipFree(sink);
    return 0;
}

int cmd_grouped(int iters) {
    Pool pool(true);
    std::vector<PrefillPlan> plans;
    for (int l = 0; l < 4; ++l) plans.emplace_back(pool, 5 + l);
    std::printf("grouped: config-3-like plan, %d items, experts spread over 24 x 2 GiB\n", plans[0].n_items);
    const double gu = 257.0 * 2 * kMat + 512.0 * kH * 2;
    const double dn = 257.0 * kMat + 4608.0 * kH * 4;
    for (int rep = 0; rep < 2; ++rep) {
        report("k_gu_grp", time_launches(iters, [&](int i) { KB_CHECK(launch_gate_up(plans[i % 4].L, 0)); }), gu);
        report("k_dn_grp", time_launches(iters, [&](int i) { KB_CHECK(launch_down(plans[i % 4].L, 0)); }), dn);
    }
    return 0;
}


// ---------------------------------------------------------------------------
// rates: one workgroup per CU, every wave timing a fixed loop with s_memtime
// (the shader clock) between two barriers; the median over CUs is printed.
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_rate_lds(int iters, unsigned long long* clk, uint32_t* sink) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[65536];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < 65536 / 4; i += 64 * NW) reinterpret_cast<uint32_t*>(lds)[i] = i;
    __syncthreads();
    // 16 consecutive bytes per lane: one wave instruction reads 1 KB
    const uint32_t base = (uint32_t)(uintptr_t)lds + ((wave * 1024 + lane * 16) & 8191);
    u32x4 x = {0, 0, 0, 0};
    __syncthreads();
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
        u32x4 v0, v1, v2, v3, v4, v5, v6, v7;
        asm volatile(
            "ds_read_b128 %0, %8\n ds_read_b128 %1, %8 offset:8192\n ds_read_b128 %2, %8 offset:16384\n"
            "ds_read_b128 %3, %8 offset:24576\n ds_read_b128 %4, %8 offset:32768\n ds_read_b128 %5, %8 offset:40960\n"
            "ds_read_b128 %6, %8 offset:49152\n ds_read_b128 %7, %8 offset:57344\n s_waitcnt lgkmcnt(0)"
            : "=v"(v0), "=v"(v1), "=v"(v2), "=v"(v3), "=v"(v4), "=v"(v5), "=v"(v6), "=v"(v7)
            : "v"(base));
        x ^= v0 ^ v1 ^ v2 ^ v3 ^ v4 ^ v5 ^ v6 ^ v7;
    }
    __syncthreads();
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    if (tid == 0) clk[blockIdx.x] = t1 - t0;
    sink[blockIdx.x * 64 * NW + tid] = x[0] ^ x[1] ^ x[2] ^ x[3];
}

// NM independent bf16 MFMAs and NCVT independent fp8 -> bf16 converts per
// iteration (the converts' results do not feed the MFMAs)
template <int NW, int NM, int NCVT>
__global__ __launch_bounds__(64 * NW) void k_rate_valu(int iters, unsigned long long* clk, uint32_t* sink) {
    typedef Mma<false> M;
    const int tid = threadIdx.x;
    u32x4 ra, rb;
    for (int i = 0; i < 4; ++i) {
        ra[i] = 0x3f803f80u + tid;
        rb[i] = 0x3f003f00u + i;
    }
    const M::V a = M::bits(ra), b = M::bits(rb);
    f32x4 acc[8];
    for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    uint32_t src[16];
    for (int j = 0; j < 16; ++j) src[j] = 0x3c3c3c3cu + tid * 17 + j;
    __syncthreads();
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
        uint32_t r[16];
#pragma unroll
        for (int j = 0; j < (NM > NCVT ? NM : NCVT); ++j) {
            // the MFMA as written, so each accumulator stays in its own
            // registers across iterations (AGPRs at one wave per SIMD, where
            // the compiler otherwise rotates them through copies)
            if (j < NM) {
                if constexpr (NW <= 4)
                    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc[j]) : "v"(a), "v"(b));
                else
                    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc[j]) : "v"(a), "v"(b));
            }
            if (j < NCVT) asm volatile("v_cvt_scalef32_pk_bf16_fp8 %0, %1, %2" : "=v"(r[j]) : "v"(src[j]), "v"(1.0f));
        }
#pragma unroll
        for (int j = 0; j < NCVT; ++j) src[j] ^= r[j] & 1;
    }
    // the last MFMAs' results are read below: let them retire first
    asm volatile("s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7");
    __syncthreads();
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    float sum = 0.f;
    for (int j = 0; j < 8; ++j) sum += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
    uint32_t x = 0;
    for (int j = 0; j < 16; ++j) x ^= src[j];
    if (tid == 0) clk[blockIdx.x] = t1 - t0;
    sink[blockIdx.x * 64 * NW + tid] = __float_as_uint(sum) ^ x;
}

// ---------------------------------------------------------------------------
// Config 0 (one expert, one token) as one launch split over the inter
// dimension, against the library's two launches (k_gate_up_kpart +
// k_down_ks).  Workgroup b owns inter rows [8b, 8b + 8): it issues its gate
// and up rows (8 + 8 MFMA rows x 7168, K over 8 waves) and its down k-panel
// (w_down stored as 8-column panels [I/8][H][8], 7168 rows x 8 B, 56 KB
// contiguous) at once, forms h for its 8 rows in LDS, and writes the partial
// y_b = Wd[:, 8b:8b+8] . h_b for all 7168 rows (fp32); a second launch sums
// the 256 partials of each row in a fixed order.  FUSED_REDUCE = 0 times the
// first launch alone.  The w_down bytes are the pool's synthetic bytes read
// as panels (a re-layout would move them, not change the read pattern).
typedef float f32x2 __attribute__((ext_vector_type(2)));
constexpr int kF1Rows = 8;
constexpr int kF1Wg = kI / kF1Rows;  // 256

__global__ __launch_bounds__(512) void k_f1_expert(cx_expert_desc e, const uint16_t* x, float* ypart) {
    constexpr int NKW = 7;  // k-blocks per wave (56 / 8)
    __shared__ float red[8][16];
    __shared__ float hs[kF1Rows];
    typedef Mma<false> M;
    const int b = blockIdx.x, wave = wave_id(), lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const int r0 = b * kF1Rows;
    const uint8_t* pa = (c < 8 ? e.w_gate + (size_t)(r0 + c) * kH : e.w_up + (size_t)(r0 + c - 8) * kH) +
                        (size_t)wave * NKW * kKB + g * 32;
    u32x4 wa[NKW][2];
#pragma unroll
    for (int k = 0; k < NKW; ++k) {
        wa[k][0] = ld16(pa + k * kKB);
        wa[k][1] = ld16(pa + k * kKB + 16);
    }
    // down panel: this wave's 896 rows x 8 B, 16 B (two rows) per lane and load
    const uint8_t* pp = e.w_down + (size_t)b * kH * 8 + (size_t)wave * 896 * 8 + lane * 16;
    u32x4 wd[7];
#pragma unroll
    for (int j = 0; j < 7; ++j) wd[j] = ld16(pp + j * 1024);
    // x (column 0 of B): 32 contiguous bf16 per lane and k-block, zero elsewhere
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, kH * 2);
    u32x4 xb[NKW][4];
#pragma unroll
    for (int k = 0; k < NKW; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            xb[k][j] = bld16(xr, c == 0 ? (uint32_t)(((wave * NKW + k) * kKB + 32 * g + 8 * j) * 2) : kOob);
    __builtin_amdgcn_sched_barrier(0);
    const int rb = r0 / 128;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < NKW; ++k) {
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        f32x4 t = M::mma(M::cvt(wa[k][0][0], wa[k][0][1]), M::bits(xb[k][0]), zero);
        t = M::mma(M::cvt(wa[k][0][2], wa[k][0][3]), M::bits(xb[k][1]), t);
        t = M::mma(M::cvt(wa[k][1][0], wa[k][1][1]), M::bits(xb[k][2]), t);
        t = M::mma(M::cvt(wa[k][1][2], wa[k][1][3]), M::bits(xb[k][3]), t);
        const int kb = wave * NKW + k;
        const float sc = g < 2 ? ldsc(e.s_gate + rb * 56 + kb) : ldsc(e.s_up + rb * 56 + kb);
        acc += sc * t;
    }
    if (c == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][4 * g + i] = acc[i];
    }
    __syncthreads();
    if (wave == 0 && lane < kF1Rows) {
        float gs = 0.f, us = 0.f;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            gs += red[w][lane];
            us += red[w][8 + lane];
        }
        hs[lane] = (gs / (1.0f + expf(-gs))) * us;
    }
    __syncthreads();
    float h[kF1Rows];
#pragma unroll
    for (int i = 0; i < kF1Rows; ++i) h[i] = hs[i];
    const int kbd = r0 / 128;  // the slice's column block of w_down's scales
#pragma unroll
    for (int j = 0; j < 7; ++j) {
        const int R = wave * 896 + j * 128 + 2 * lane;
        const float sd = ldsc(e.s_down + (size_t)(wave * 7 + j) * 16 + kbd);
        float y2[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint32_t w0 = wd[j][2 * q], w1 = wd[j][2 * q + 1];
            const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(w0, false);
            const f32x2 bq = __builtin_amdgcn_cvt_pk_f32_fp8(w0, true);
            const f32x2 cq = __builtin_amdgcn_cvt_pk_f32_fp8(w1, false);
            const f32x2 dq = __builtin_amdgcn_cvt_pk_f32_fp8(w1, true);
            float sum = a[0] * h[0];
            sum += a[1] * h[1];
            sum += bq[0] * h[2];
            sum += bq[1] * h[3];
            sum += cq[0] * h[4];
            sum += cq[1] * h[5];
            sum += dq[0] * h[6];
            sum += dq[1] * h[7];
            y2[q] = sum * sd;
        }
        *reinterpret_cast<float2*>(ypart + (size_t)b * kH + R) = float2{y2[0], y2[1]};
    }
}

// y[r] = sum over the 256 partials in a fixed order: 16 groups of 16
// consecutive partials per thread, then the 16 group sums in group order.
__global__ __launch_bounds__(256) void k_f1_reduce(const float* ypart, uint16_t* y) {
    __shared__ float4 red[16][16];
    const int c4 = threadIdx.x & 15, grp = threadIdx.x >> 4;
    const int row = blockIdx.x * 64 + c4 * 4;
    float4 v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = *reinterpret_cast<const float4*>(ypart + (size_t)(grp * 16 + i) * kH + row);
    float4 s = v[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) s = float4{s.x + v[i].x, s.y + v[i].y, s.z + v[i].z, s.w + v[i].w};
    red[grp][c4] = s;
    __syncthreads();
    if (grp == 0) {
        float4 t = red[0][c4];
        for (int i = 1; i < 16; ++i) t = float4{t.x + red[i][c4].x, t.y + red[i][c4].y, t.z + red[i][c4].z, t.w + red[i][c4].w};
        const f32x4 tv = {t.x, t.y, t.z, t.w};
        store_out4(y, nullptr, (size_t)row, tv, CX_DTYPE_BF16);
    }
}

int cmd_fused1(int iters) {
    Pool pool(true);
    std::printf("fused1: one expert, one token, 64 experts rotated (24 x 2 GiB chunks)\n");
    const int lds = max_lds();
    uint16_t *x = nullptr, *y = nullptr;
    float *gu = nullptr, *yp = nullptr;
    KB_CHECK(hipMalloc(&x, kH * 2));
    KB_CHECK(hipMemset(x, 0x3c, kH * 2));
    KB_CHECK(hipMalloc(&y, kH * 2));
    KB_CHECK(hipMalloc(&gu, 2 * 2 * kI * 4));
    KB_CHECK(hipMalloc(&yp, (size_t)kF1Wg * kH * 4));
    const int n = std::min<int>(64, (int)pool.d.size());
    auto two = [&](int i) {
        ExpertLaunch L{};
        L.single = pool.d[(i * 17) % pool.d.size()];
        L.n_tokens = 1;
        L.hidden = kH;
        L.inter = kI;
        L.maxt = 1;
        L.x = x;
        L.in_dtype = CX_DTYPE_BF16;
        L.y = y;
        L.out_dtype = CX_DTYPE_BF16;
        L.np_lds = 1;
        L.max_lds = lds;
        L.gu_part = gu;
        L.gu_kparts = 2;
        return L;
    };
    const double bytes = 3.0 * kMat + 3 * 16 * 56 * 4 + 2 * kH * 2;
    for (int rep = 0; rep < 3; ++rep) {
        report("two launches: k_gate_up_kpart + k_down_ks", time_launches(iters, [&](int i) {
                   const ExpertLaunch L = two(i % n);
                   KB_CHECK(launch_gate_up_kpart(L, 0));
                   KB_CHECK(launch_down_ks(L, 0));
               }), bytes);
        report("  k_gate_up_kpart alone", time_launches(iters, [&](int i) {
                   KB_CHECK(launch_gate_up_kpart(two(i % n), 0));
               }), bytes * 2 / 3);
        report("split over inter: k_f1_expert + k_f1_reduce", time_launches(iters, [&](int i) {
                   const cx_expert_desc& e = pool.d[((i % n) * 17) % pool.d.size()];
                   cx_launch(k_f1_expert, dim3(kF1Wg), dim3(512), 0, (hipStream_t)0, e, (const uint16_t*)x, yp);
                   cx_launch(k_f1_reduce, dim3(kH / 64), dim3(256), 0, (hipStream_t)0, (const float*)yp, y);
               }), bytes);
        report("  k_f1_expert alone", time_launches(iters, [&](int i) {
                   const cx_expert_desc& e = pool.d[((i % n) * 17) % pool.d.size()];
                   cx_launch(k_f1_expert, dim3(kF1Wg), dim3(512), 0, (hipStream_t)0, e, (const uint16_t*)x, yp);
               }), bytes);
        report("  k_f1_reduce alone", time_launches(iters, [&](int) {
                   cx_launch(k_f1_reduce, dim3(kH / 64), dim3(256), 0, (hipStream_t)0, (const float*)yp, y);
               }), (double)kF1Wg * kH * 4);
    }
    (void)hipFree(x);
    (void)hipFree(y);
    (void)hipFree(gu);
    (void)hipFree(yp);
    return 0;
}

// ---------------------------------------------------------------------------
// Decode weight layouts.  Bare streams (no compute) of the one-token launch
// shapes, each reading the same bytes per lane in two orders: natural rows
// (lane = row c of a 16-row group, quarter g of a 128-byte k-block: 16 rows
// 128 B apart per k-step of 7168 or 2048 B) and tile-contiguous (the 16
// rows x 128 columns of one k-step are one 2 KB tile, lane l at 32 l: what
// CX_LAYOUT_TILE16 stores for gate/up).
template <bool TILED>
__device__ __forceinline__ size_t gu_bare_off(int rt, int kb, int lane, int cols) {
    return TILED ? ((size_t)rt * (cols / kKB) + kb) * 2048 + lane * 32
                 : (size_t)(rt * 16 + (lane & 15)) * cols + (size_t)kb * kKB + (lane >> 4) * 32;
}

// gate/up k-part shape (k_gate_up_kpart): 128 row tiles x 2 k-parts = 256
// workgroups of 8 waves, 7 active x 4 k-blocks of gate and up each.
template <bool TILED>
__global__ __launch_bounds__(512) void k_bare_kpart_gu(cx_expert_desc e, uint32_t* sink) {
    const int wave = wave_id(), lane = threadIdx.x & 63;
    if (wave >= 7) return;
    const int rt = blockIdx.x >> 1, kb0 = (blockIdx.x & 1) * 28 + wave * 4;
    u32x4 v[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const size_t off = gu_bare_off<TILED>(rt, kb0 + k, lane, kH);
        v[4 * k + 0] = ld16(e.w_gate + off);
        v[4 * k + 1] = ld16(e.w_gate + off + 16);
        v[4 * k + 2] = ld16(e.w_up + off);
        v[4 * k + 3] = ld16(e.w_up + off + 16);
    }
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc ^= v[i][0] + v[i][1] * 3u + v[i][2] * 5u + v[i][3] * 7u;
    if (acc == 0x12345678u) sink[threadIdx.x] = acc;
}

// down k-split shape (k_down_ks): 224 workgroups of 8 waves = 2 groups of 16
// rows x 4 k ranges of 4 k-blocks.
template <bool TILED>
__global__ __launch_bounds__(512) void k_bare_ks_dn(cx_expert_desc e, uint32_t* sink) {
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int rg = blockIdx.x * 2 + (wave >> 2), kr = wave & 3;
    u32x4 v[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const size_t off = gu_bare_off<TILED>(rg, kr * 4 + k, lane, kI);
        v[2 * k] = ld16(e.w_down + off);
        v[2 * k + 1] = ld16(e.w_down + off + 16);
    }
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc ^= v[i][0] + v[i][1] * 3u + v[i][2] * 5u + v[i][3] * 7u;
    if (acc == 0x12345678u) sink[threadIdx.x] = acc;
}

// one-token routed gate/up shape (k_gate_up_t, k_gate_up_sel): grid 128 row
// tiles x 8 experts, 4 waves x 14 k-blocks, a 4-deep register ring.
template <bool TILED>
__global__ __launch_bounds__(256) void k_bare_b1_gu(GuPtrs P, uint32_t* sink) {
    constexpr int NKB = 14, D = 4;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int rt = blockIdx.x, kb0 = wave * NKB;
    const uint8_t* pg = P.gate[blockIdx.y];
    const uint8_t* pu = P.up[blockIdx.y];
    u32x4 wb[D][4];
    uint32_t acc = 0;
#pragma unroll
    for (int s = 0; s < D; ++s) {
        const size_t off = gu_bare_off<TILED>(rt, kb0 + s, lane, kH);
        wb[s][0] = ld16(pg + off);
        wb[s][1] = ld16(pg + off + 16);
        wb[s][2] = ld16(pu + off);
        wb[s][3] = ld16(pu + off + 16);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < NKB; ++k) {
        const int s = k % D;
#pragma unroll
        for (int q = 0; q < 4; ++q) acc ^= wb[s][q][0] + wb[s][q][1] * 3u + wb[s][q][2] * 5u + wb[s][q][3] * 7u;
        __builtin_amdgcn_sched_barrier(0);
        if (k + D < NKB) {
            const size_t off = gu_bare_off<TILED>(rt, kb0 + k + D, lane, kH);
            wb[s][0] = ld16(pg + off);
            wb[s][1] = ld16(pg + off + 16);
            wb[s][2] = ld16(pu + off);
            wb[s][3] = ld16(pu + off + 16);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if (acc == 0x12345678u) sink[threadIdx.x] = acc;
}

int cmd_decode_layout(int iters) {
    Pool pool(true);
    const int n = std::min<int>(64, (int)pool.d.size());
    std::printf("decode-layout: one token, experts spread over 24 x 2 GiB (%d rotated for one expert)\n", n);
    uint32_t* sink = nullptr;
    KB_CHECK(hipMalloc(&sink, 4096));
    std::mt19937 rng(13);
    std::vector<GuPtrs> sets(16);
    for (auto& st : sets)
        for (int j = 0; j < 8; ++j) {
            const cx_expert_desc& q = pool.d[rng() % pool.d.size()];
            st.gate[j] = q.w_gate;
            st.up[j] = q.w_up;
        }
    auto one = [&](int i) { return pool.d[((i % n) * 17) % pool.d.size()]; };
    const int lds = max_lds();
    uint16_t *x = nullptr, *y = nullptr;
    float* gu = nullptr;
    KB_CHECK(hipMalloc(&x, kH * 2));
    KB_CHECK(hipMemset(x, 0x3c, kH * 2));
    KB_CHECK(hipMalloc(&y, kH * 2));
    KB_CHECK(hipMalloc(&gu, 2 * 2 * kI * 4));
    // the library's kernels read the layout from the descriptor; the bytes are
    // synthetic, so one buffer serves both readings
    auto expert_launch = [&](int i, int layout) {
        ExpertLaunch L{};
        L.single = one(i);
        L.single.gu_layout = layout;
        L.n_tokens = 1;
        L.hidden = kH;
        L.inter = kI;
        L.maxt = 1;
        L.x = x;
        L.in_dtype = CX_DTYPE_BF16;
        L.y = y;
        L.out_dtype = CX_DTYPE_BF16;
        L.np_lds = 1;
        L.max_lds = lds;
        L.gu_part = gu;
        L.gu_kparts = 2;
        return L;
    };
    DecodePlans dp_rows(pool, 16, 3);
    for (auto& q : pool.d) q.gu_layout = CX_LAYOUT_TILE16;
    DecodePlans dp_tiled(pool, 16, 3);
    cx_expert_desc* table = dev_copy(pool.d);
    const double b1_gu = 16.0 * kMat, kpart_gu = 2.0 * kMat;
    const double t_bytes = 8.0 * (2 * kMat + 2 * 16 * 56 * 4) + kH * 2;
    for (int rep = 0; rep < 3; ++rep) {
        std::printf(" pass %d\n", rep + 1);
        report("bare one-token routed gate/up shape, natural rows", time_launches(iters, [&](int i) {
                   cx_launch(k_bare_b1_gu<false>, dim3(128, 8), dim3(256), 0u, (hipStream_t)0, sets[i % 16], sink);
               }), b1_gu);
        report("bare one-token routed gate/up shape, tile-contiguous", time_launches(iters, [&](int i) {
                   cx_launch(k_bare_b1_gu<true>, dim3(128, 8), dim3(256), 0u, (hipStream_t)0, sets[i % 16], sink);
               }), b1_gu);
        report("bare gate/up k-part shape, natural rows", time_launches(iters, [&](int i) {
                   cx_launch(k_bare_kpart_gu<false>, dim3(256), dim3(512), 0u, (hipStream_t)0, one(i), sink);
               }), kpart_gu);
        report("bare gate/up k-part shape, tile-contiguous", time_launches(iters, [&](int i) {
                   cx_launch(k_bare_kpart_gu<true>, dim3(256), dim3(512), 0u, (hipStream_t)0, one(i), sink);
               }), kpart_gu);
        report("bare down k-split shape, natural rows", time_launches(iters, [&](int i) {
                   cx_launch(k_bare_ks_dn<false>, dim3(224), dim3(512), 0u, (hipStream_t)0, one(i), sink);
               }), 1.0 * kMat);
        report("bare down k-split shape, tile-contiguous", time_launches(iters, [&](int i) {
                   cx_launch(k_bare_ks_dn<true>, dim3(224), dim3(512), 0u, (hipStream_t)0, one(i), sink);
               }), 1.0 * kMat);
        for (int layout = 0; layout < 2; ++layout) {
            const char* tag = layout ? "CX_LAYOUT_TILE16" : "CX_LAYOUT_ROWS";
            char what[96];
            std::snprintf(what, sizeof what, "k_gate_up_kpart, %s", tag);
            report(what, time_launches(iters, [&](int i) {
                       KB_CHECK(launch_gate_up_kpart(expert_launch(i, layout), 0));
                   }), kpart_gu + 2 * 16 * 56 * 4 + kH * 2);
            std::snprintf(what, sizeof what, "k_gate_up_t (8 routed experts), %s", tag);
            const DecodePlans& dp = layout ? dp_tiled : dp_rows;
            report(what, time_launches(iters, [&](int i) {
                       KB_CHECK(launch_gate_up(dp.launch(i, table, lds), 0));
                   }), t_bytes);
        }
    }
    (void)hipFree(table);
    (void)hipFree(x);
    (void)hipFree(y);
    (void)hipFree(gu);
    (void)hipFree(sink);
    return 0;
}

int cmd_rates(int iters) {
    const int cus = n_cu();
    const int n = 2000 * std::max(1, iters / 30);
    unsigned long long* clk;
    uint32_t* sink;
    KB_CHECK(hipMalloc(&clk, sizeof(unsigned long long) * cus));
    KB_CHECK(hipMalloc(&sink, sizeof(uint32_t) * cus * 1024));
    hipEvent_t e0, e1;
    KB_CHECK(hipEventCreate(&e0));
    KB_CHECK(hipEventCreate(&e1));
    // second launch timed (the first warms up); median shader clocks over CUs
    auto run = [&](auto kern, int nw, double* ms) {
        for (int rep = 0; rep < 2; ++rep) {
            KB_CHECK(hipEventRecord(e0));
            hipLaunchKernelGGL(kern, dim3(cus), dim3(64 * nw), 0, 0, n, clk, sink);
            KB_CHECK(hipGetLastError());
            KB_CHECK(hipEventRecord(e1));
            KB_CHECK(hipEventSynchronize(e1));
        }
        float f;
        KB_CHECK(hipEventElapsedTime(&f, e0, e1));
        *ms = f;
        std::vector<unsigned long long> h(cus);
        KB_CHECK(hipMemcpy(h.data(), clk, sizeof(unsigned long long) * cus, hipMemcpyDeviceToHost));
        std::sort(h.begin(), h.end());
        return (double)h[cus / 2];
    };
    std::printf("%d CUs, %d loop iterations per wave; clocks are s_memtime (shader clock) counts\n", cus, n);
    double ms, c;
    c = run(k_rate_lds<4>, 4, &ms);
    std::printf("ds_read_b128, 4 waves/CU     %6.1f B per clock per CU  (%.3f ms, ~%.2f GHz)\n", 4.0 * n * 8 * 1024 / c, ms, c / (ms * 1e6));
    c = run(k_rate_lds<8>, 8, &ms);
    std::printf("ds_read_b128, 8 waves/CU     %6.1f B per clock per CU  (%.3f ms, ~%.2f GHz)\n", 8.0 * n * 8 * 1024 / c, ms, c / (ms * 1e6));
    c = run(k_rate_lds<16>, 16, &ms);
    std::printf("ds_read_b128, 16 waves/CU    %6.1f B per clock per CU  (%.3f ms, ~%.2f GHz)\n", 16.0 * n * 8 * 1024 / c, ms, c / (ms * 1e6));
    auto per = [&](double clks, int nw, int per_iter) { return clks / ((double)n * per_iter * nw / 4); };
    c = run(k_rate_valu<4, 8, 0>, 4, &ms);
    std::printf("bf16 MFMA 16x16x32, 1 wave/SIMD      %5.2f clocks per MFMA per SIMD\n", per(c, 4, 8));
    c = run(k_rate_valu<8, 8, 0>, 8, &ms);
    std::printf("bf16 MFMA 16x16x32, 2 waves/SIMD     %5.2f clocks per MFMA per SIMD  (%.0f TFLOP/s over the chip)\n", per(c, 8, 8),
                (double)cus * 4 * ((double)n * 8 * 2) * 16 * 16 * 32 * 2 / (ms * 1e-3) / 1e12);
    c = run(k_rate_valu<8, 0, 16>, 8, &ms);
    std::printf("fp8->bf16 pk convert, 2 waves/SIMD   %5.2f clocks per instruction per SIMD\n", per(c, 8, 16));
    c = run(k_rate_valu<4, 8, 4>, 4, &ms);
    std::printf("8 MFMA + 4 converts, 1 wave/SIMD     %5.2f clocks per MFMA per SIMD\n", per(c, 4, 8));
    c = run(k_rate_valu<4, 8, 8>, 4, &ms);
    std::printf("8 MFMA + 8 converts, 1 wave/SIMD     %5.2f clocks per MFMA per SIMD\n", per(c, 4, 8));
    c = run(k_rate_valu<8, 8, 4>, 8, &ms);
    std::printf("8 MFMA + 4 converts, 2 waves/SIMD    %5.2f clocks per MFMA per SIMD\n", per(c, 8, 8));
    c = run(k_rate_valu<8, 8, 8>, 8, &ms);
    std::printf("8 MFMA + 8 converts, 2 waves/SIMD    %5.2f clocks per MFMA per SIMD\n", per(c, 8, 8));
    KB_CHECK(hipFree(clk));
    KB_CHECK(hipFree(sink));
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    const char* cmd = argc > 1 ? argv[1] : "";
    const int iters = argc > 2 ? std::max(4, std::atoi(argv[2])) : 30;
    if (!std::strcmp(cmd, "layout")) return cmd_layout(std::min(iters, 12));
    if (!std::strcmp(cmd, "decode-down")) return cmd_decode_down(iters);
    if (!std::strcmp(cmd, "placement")) return cmd_placement(iters);
    if (!std::strcmp(cmd, "decode-balance")) return cmd_decode_balance(iters);
    if (!std::strcmp(cmd, "grouped")) return cmd_grouped(std::min(iters, 12));
    if (!std::strcmp(cmd, "grouped-down")) return cmd_grouped_down(std::min(iters, 12));
    if (!std::strcmp(cmd, "rates")) return cmd_rates(iters);
    if (!std::strcmp(cmd, "fused1")) return cmd_fused1(iters);
    if (!std::strcmp(cmd, "decode-layout")) return cmd_decode_layout(iters);
    std::fprintf(stderr, "usage: cx_kbench layout|decode-down|placement|decode-balance|grouped|grouped-down|"
                         "rates|fused1|decode-layout [launches]\n");
    return 2;
}
