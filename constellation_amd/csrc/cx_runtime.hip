// cx_runtime.hip — host side of the C ABI (include/cx_moe.h): per-device HBM
// arena, per-worker contexts with persistent scratch, argument checking,
// kernel sequencing.  No exceptions cross the ABI; every entry returns an
// int status and leaves a thread-local message for cx_last_error().
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "cx_internal.h"

using namespace cx;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define CX_HIP(call)                                                                   \
    do {                                                                               \
        hipError_t e_ = (call);                                                        \
        if (e_ != hipSuccess)                                                          \
            return fail(CX_EHIP, "%s failed: %s", #call, hipGetErrorString(e_));       \
    } while (0)

int set_device(int device) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n)
        return fail(CX_EINVAL, "invalid device %d (count %d)", device, n);
    CX_HIP(hipSetDevice(device));
    return CX_OK;
}

// Restores the calling thread's current device when it leaves scope, for
// entry points that may run on a caller's control thread (device probes,
// frees) and must not leave another device current there.
class DeviceRestore {
public:
    DeviceRestore() {
        if (hipGetDevice(&prev_) != hipSuccess) {
            (void)hipGetLastError();
            prev_ = -1;
        }
    }
    ~DeviceRestore() {
        if (prev_ >= 0) (void)hipSetDevice(prev_);
    }

private:
    int prev_ = -1;
};

size_t act_size(int dtype) { return dtype == CX_DTYPE_F32 ? 4 : 2; }
bool act16(int dtype) { return dtype == CX_DTYPE_FP16 || dtype == CX_DTYPE_BF16; }

// ---------------------------------------------------------------------------
// Per-device HBM arena: large hipMalloc chunks, first-fit sub-allocation with
// coalescing free lists.  Expert weights (44 MB each at DeepSeek shapes) sit
// back to back in 2 GiB chunks instead of six hipMallocs per expert.
constexpr size_t kAlign = 256;

struct Chunk {
    char* base = nullptr;
    size_t size = 0;
    std::map<size_t, size_t> free_ranges;  // offset -> length
};

struct Arena {
    std::mutex mu;
    std::vector<Chunk> chunks;
    std::unordered_map<void*, std::pair<size_t, size_t>> live;  // ptr -> (chunk, len)
    size_t used = 0, reserved = 0;
};

Arena& arena(int device) {
    static Arena arenas[64];
    return arenas[device & 63];
}

size_t chunk_bytes() {
    static size_t v = [] {
        const char* s = std::getenv("CX_ARENA_CHUNK_MB");
        size_t mb = s ? std::strtoull(s, nullptr, 10) : 2048;
        if (mb < 64) mb = 64;
        return mb << 20;
    }();
    return v;
}

int arena_alloc(int device, size_t bytes, void** out) {
    *out = nullptr;
    if (bytes == 0) bytes = kAlign;
    bytes = (bytes + kAlign - 1) / kAlign * kAlign;
    Arena& A = arena(device);
    std::lock_guard<std::mutex> lk(A.mu);
    for (size_t ci = 0; ci < A.chunks.size(); ++ci) {
        Chunk& ch = A.chunks[ci];
        for (auto it = ch.free_ranges.begin(); it != ch.free_ranges.end(); ++it) {
            if (it->second >= bytes) {
                const size_t off = it->first, len = it->second;
                ch.free_ranges.erase(it);
                if (len > bytes) ch.free_ranges[off + bytes] = len - bytes;
                void* p = ch.base + off;
                A.live[p] = {ci, bytes};
                A.used += bytes;
                *out = p;
                return CX_OK;
            }
        }
    }
    const size_t cb = std::max(chunk_bytes(), (bytes + (2u << 20) - 1) / (2u << 20) * (2u << 20));
    void* base = nullptr;
    if (hipMalloc(&base, cb) != hipSuccess || base == nullptr) {
        (void)hipGetLastError();
        return fail(CX_ENOMEM, "HBM arena: hipMalloc(%zu) failed (used %zu reserved %zu)", cb,
                    A.used, A.reserved);
    }
    Chunk ch;
    ch.base = static_cast<char*>(base);
    ch.size = cb;
    if (cb > bytes) ch.free_ranges[bytes] = cb - bytes;
    A.chunks.push_back(std::move(ch));
    A.reserved += cb;
    A.live[base] = {A.chunks.size() - 1, bytes};
    A.used += bytes;
    *out = base;
    return CX_OK;
}

// Returns a range to the free list.  When `in_use` the range may still be read
// by kernels queued on any stream of the device (a caller frees an expert while
// its worker thread computes), so the device is synchronised first, as
// hipFree/cudaFree do: the next upload can then overwrite the range safely.
int arena_free(int device, void* p, bool in_use = true) {
    if (p == nullptr) return CX_OK;
    Arena& A = arena(device);
    if (in_use) {
        {
            std::lock_guard<std::mutex> lk(A.mu);
            if (A.live.find(p) == A.live.end())
                return fail(CX_EINVAL, "cx_free_device: %p not allocated here", p);
        }
        DeviceRestore restore;
        int rc = set_device(device);
        if (rc) return rc;
        CX_HIP(hipDeviceSynchronize());
    }
    std::lock_guard<std::mutex> lk(A.mu);
    auto it = A.live.find(p);
    if (it == A.live.end()) return fail(CX_EINVAL, "cx_free_device: %p not allocated here", p);
    const size_t ci = it->second.first, len = it->second.second;
    A.live.erase(it);
    A.used -= len;
    Chunk& ch = A.chunks[ci];
    size_t off = static_cast<size_t>(static_cast<char*>(p) - ch.base);
    size_t l = len;
    auto nx = ch.free_ranges.lower_bound(off);
    if (nx != ch.free_ranges.end() && nx->first == off + l) {
        l += nx->second;
        ch.free_ranges.erase(nx);
    }
    auto pv = ch.free_ranges.lower_bound(off);
    if (pv != ch.free_ranges.begin()) {
        --pv;
        if (pv->first + pv->second == off) {
            off = pv->first;
            l += pv->second;
            ch.free_ranges.erase(pv);
        }
    }
    ch.free_ranges[off] = l;
    return CX_OK;
}

hipStream_t upload_stream(int device) {
    static std::mutex mu;
    static hipStream_t streams[64] = {};
    std::lock_guard<std::mutex> lk(mu);
    if (streams[device & 63] == nullptr) {
        (void)hipStreamCreateWithFlags(&streams[device & 63], hipStreamNonBlocking);
    }
    return streams[device & 63];
}

// ---------------------------------------------------------------------------
// Growable device buffer owned by a context.
struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
};

int ensure(DevBuf* b, size_t bytes, hipStream_t s) {
    if (b->bytes >= bytes && b->p != nullptr) return CX_OK;
    if (b->p != nullptr) {
        CX_HIP(hipStreamSynchronize(s));
        CX_HIP(hipFree(b->p));
        b->p = nullptr;
        b->bytes = 0;
    }
    const size_t want = std::max<size_t>(bytes, 4096);
    if (hipMalloc(&b->p, want) != hipSuccess) {
        (void)hipGetLastError();
        b->p = nullptr;
        return fail(CX_ENOMEM, "context scratch: hipMalloc(%zu) failed", want);
    }
    b->bytes = want;
    return CX_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
struct cx_ctx {
    int device = -1;
    hipStream_t own_stream = nullptr;  // for the host-buffer entry point
    int* err_flag = nullptr;           // device int: error bits of the device checks
    int max_lds = 65536;               // dynamic LDS budget per workgroup
    int n_cu = 0;                      // compute units (0: unknown)
    DevBuf plan_buf, hhi, hlo, ypart, logits, route_ids, route_w, hscratch;
    DevBuf gu_part;                    // shared expert's k-part gate/up sums (decode)
    DevBuf scores;                     // one-token router scores s, c [E][2] fp64 (decode)
    int route_T = 0, route_E = 0;      // shape of the fp64 logits of the last router call
    DevBuf dx, dy;                     // cx_expert_run_host staging (device)
    void* pin_x = nullptr;             // pinned host staging
    void* pin_y = nullptr;
    size_t pin_x_bytes = 0, pin_y_bytes = 0;
    // per-kernel HIP-event timing (cx_ctx_profile)
    bool prof = false;
    std::map<std::string, std::vector<std::pair<hipEvent_t, hipEvent_t>>> spans;
    std::map<std::string, std::pair<int, double>> totals;
};

namespace cx {
LaunchTimer*& current_launch_timer() {
    static thread_local LaunchTimer* t = nullptr;
    return t;
}
}  // namespace cx

struct cx_layer {
    int n_experts = 0;
    int has_shared = 0;
    int fast = 1;                      // every resident expert fits the grouped kernels
    int hidden = 0, inter = 0;
    cx_expert_desc* table = nullptr;   // device [n_experts + 1], entry n_experts = shared
    cx_expert_desc shared_desc{};      // host copy of the shared expert (when has_shared)
    std::vector<uint8_t> resident;     // host copy: entry i holds an expert
    int n_resident = 0;                // routed experts held
};

namespace {

// Times the kernels launched in its scope when profiling is on: the launches
// carry the events (cx_launch), so the span is first-kernel start to
// last-kernel end as the command processor stamps them.
class Span {
public:
    Span(cx_ctx* ctx, const char* name, hipStream_t s) : ctx_(ctx) {
        (void)s;
        if (ctx_ == nullptr || !ctx_->prof) return;
        if (hipEventCreate(&t_.start) != hipSuccess || hipEventCreate(&t_.stop) != hipSuccess) {
            (void)hipGetLastError();
            if (t_.start) (void)hipEventDestroy(t_.start);
            t_.start = t_.stop = nullptr;
            return;
        }
        name_ = name;
        prev_ = current_launch_timer();
        current_launch_timer() = &t_;
        active_ = true;
    }
    ~Span() {
        if (!active_) return;
        current_launch_timer() = prev_;
        if (t_.started) {
            ctx_->spans[name_].push_back({t_.start, t_.stop});
        } else {
            (void)hipEventDestroy(t_.start);
            (void)hipEventDestroy(t_.stop);
        }
    }

private:
    cx_ctx* ctx_;
    LaunchTimer t_;
    LaunchTimer* prev_ = nullptr;
    bool active_ = false;
    std::string name_;
};

void drain_spans(cx_ctx* ctx) {
    for (auto& kv : ctx->spans) {
        auto& tot = ctx->totals[kv.first];
        for (auto& ab : kv.second) {
            float ms = 0.f;
            if (hipEventSynchronize(ab.second) == hipSuccess &&
                hipEventElapsedTime(&ms, ab.first, ab.second) == hipSuccess) {
                tot.first += 1;
                tot.second += ms;
            }
            (void)hipEventDestroy(ab.first);
            (void)hipEventDestroy(ab.second);
        }
        kv.second.clear();
    }
}

struct PlanSizes {
    int max_slots, max_pairs, max_items, item_cap, maxt;
};

PlanSizes plan_sizes(int n_tokens, int top_k, int n_experts, int has_shared) {
    PlanSizes z;
    z.maxt = n_tokens <= kTileTok ? 1 : 4;
    z.item_cap = kTileTok * z.maxt;
    z.max_slots = std::min(n_tokens * top_k, n_experts) + has_shared;
    z.max_pairs = n_tokens * top_k + n_tokens * has_shared;
    z.max_items = z.max_slots + (z.max_pairs + z.item_cap - 1) / z.item_cap;
    return z;
}

// dense: a decode plan (dec_plan_core), which also fills pair_row; the
// general planner leaves it out.
int carve_plan(cx_ctx* ctx, const PlanSizes& z, int n_tokens, int top_k, bool dense,
               hipStream_t s, PlanPtrs* P) {
    const size_t recs = sizeof(ItemRec) * (size_t)z.max_items + sizeof(SlotRec) * (size_t)z.max_slots;
    const size_t ints = kPlanHdrInts + 3 * (size_t)z.max_slots + 3 * (size_t)z.max_items +
                        2 * (size_t)z.max_pairs + (size_t)n_tokens * (top_k + 1) +
                        (dense ? (size_t)z.max_pairs : 0);
    int rc = ensure(&ctx->plan_buf, recs + ints * 4 + 256, s);
    if (rc) return rc;
    char* raw = static_cast<char*>(ctx->plan_buf.p);
    P->item_rec = reinterpret_cast<ItemRec*>(raw);
    P->slot_rec = reinterpret_cast<SlotRec*>(raw + sizeof(ItemRec) * (size_t)z.max_items);
    int* base = reinterpret_cast<int*>(raw + recs);
    P->hdr = reinterpret_cast<PlanHdr*>(base);
    int* q = base + kPlanHdrInts;
    P->slot_expert = q; q += z.max_slots;
    P->slot_pair_begin = q; q += z.max_slots;
    P->slot_pair_count = q; q += z.max_slots;
    P->item_slot = q; q += z.max_items;
    P->item_pair_begin = q; q += z.max_items;
    P->item_pair_count = q; q += z.max_items;
    P->pair_token = q; q += z.max_pairs;
    P->pair_weight = reinterpret_cast<float*>(q); q += z.max_pairs;
    P->token_pairs = q; q += (size_t)n_tokens * (top_k + 1);
    P->pair_row = dense ? q : nullptr;
    return CX_OK;
}

int check_desc(const cx_expert_desc* e) {
    if (e == nullptr) return fail(CX_EINVAL, "expert descriptor is NULL");
    if (!e->w_up || !e->w_gate || !e->w_down || !e->s_up || !e->s_gate || !e->s_down)
        return fail(CX_EINVAL, "expert descriptor has a NULL buffer");
    if (e->hidden <= 0 || e->inter <= 0) return fail(CX_EINVAL, "expert dims must be > 0");
    const int b[6] = {e->up_rb, e->up_cb, e->gate_rb, e->gate_cb, e->down_rb, e->down_cb};
    for (int v : b)
        if (v <= 0) return fail(CX_EINVAL, "expert block sizes must be > 0");
    return CX_OK;
}

// Activation rows of one work item that fit the LDS budget next to the
// reduction tile (<= 16 KB); 0 when staging is not worth it or not possible.
int lds_rows(int max_lds, int hidden, int max_pairs_per_item) {
    if (hidden % 512 != 0) return 0;  // rows are copied in 1 KB wave chunks
    const int budget = std::min(max_lds, 65536) - 16384;
    const int rows = budget / (hidden * 2 + 16);
    return (max_pairs_per_item <= rows && max_pairs_per_item <= 4) ? max_pairs_per_item : 0;
}

int lds_rows(const cx_ctx* ctx, int hidden, int max_pairs_per_item) {
    return lds_rows(ctx->max_lds, hidden, max_pairs_per_item);
}

// ---------------------------------------------------------------------------
// One expert over n_tokens tokens (single mode: the tokens are the pairs, the
// down launch writes the output).  Shared by cx_expert_run (context scratch)
// and cx_expert_run_static (the library's static device scratch): plan_expert
// picks the path and states the scratch it needs, run_expert launches it.
enum ExpertPath { kPathGeneric, kPathSmall, kPathTiles };

struct ExpertPlan {
    ExpertLaunch L;
    int path;
    size_t h_f32_bytes;   // generic path: fp32 h [T, I]
    size_t h_plane_bytes; // tile path: each bf16 plane h_hi / h_lo [T, I]
    size_t gu_part_bytes; // small path: k-part gate/up sums [2][2][T][I] fp32
};

ExpertPlan plan_expert(const cx_expert_desc& e, const void* x, int in_dtype, int n_tokens,
                       void* y, int out_dtype, float* y_f32, int max_lds) {
    ExpertPlan P{};
    const size_t TI = (size_t)n_tokens * e.inter;
    if (!fast_path_ok(e)) {
        P.path = kPathGeneric;
        P.h_f32_bytes = TI * 4;
        return P;
    }
    ExpertLaunch& L = P.L;
    L.table = nullptr;
    L.single = e;
    L.n_tokens = n_tokens;
    L.hidden = e.hidden;
    L.inter = e.inter;
    L.maxt = n_tokens <= kTileTok ? 1 : 4;
    L.x = x;
    L.in_dtype = in_dtype;
    L.y = y;
    L.y_f32 = y_f32;
    L.out_dtype = out_dtype;
    L.np_lds = L.maxt == 1 ? lds_rows(max_lds, e.hidden, n_tokens) : 0;
    L.max_lds = max_lds;
    if (expert_small_ok(L)) {
        P.path = kPathSmall;
        P.gu_part_bytes = sizeof(float) * 2 * 2 * TI;
        L.gu_kparts = 2;
    } else {
        P.path = kPathTiles;
        P.h_plane_bytes = TI * 2;
    }
    return P;
}

// Launches a planned expert on `s`; the scratch pointers the path needs are
// set (h_f32 / h_hi + h_lo / gu_part).  ctx (nullable) only collects timing.
int run_expert(cx_ctx* ctx, ExpertPlan& P, const cx_expert_desc& e, const void* x, int in_dtype,
               int n_tokens, void* y, int out_dtype, float* y_f32, float* h_f32, uint16_t* h_hi,
               uint16_t* h_lo, float* gu_part, hipStream_t s) {
    if (P.path == kPathGeneric) {
        CX_HIP(launch_generic_expert(e, x, in_dtype, n_tokens, h_f32, y, out_dtype, y_f32, s));
        return CX_OK;
    }
    ExpertLaunch& L = P.L;
    if (P.path == kPathSmall) {
        L.gu_part = gu_part;
        {
            Span sp(ctx, "gate_up", s);
            CX_HIP(launch_gate_up_kpart(L, s));
        }
        Span sp(ctx, "down", s);
        CX_HIP(launch_down_ks(L, s));
        return CX_OK;
    }
    L.h_hi = h_hi;
    L.h_lo = h_lo;
    {
        Span sp(ctx, "gate_up", s);
        CX_HIP(launch_gate_up(L, s));
    }
    {
        Span sp(ctx, "down", s);
        CX_HIP(launch_down(L, s));
    }
    return CX_OK;
}

// ---------------------------------------------------------------------------
// Scratch of cx_expert_run_static: a file-scope device array.  Every GPU the
// library runs on holds its own copy, at its own address, until the process
// ends.  In host code `scratch` names a host-side stand-in, never device
// memory: static_scratch() looks up the device address once per device (with
// that device current) and every kernel argument uses that address.
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[CX_STATIC_SCRATCH_BYTES];

std::mutex g_static_mu;
unsigned char* g_static_ptr[kMaxDevices] = {};
int g_static_lds[kMaxDevices] = {};

// The calling thread's current device must be `device`.
int static_scratch(int device, unsigned char** ptr, int* max_lds) {
    std::lock_guard<std::mutex> lk(g_static_mu);
    if (g_static_ptr[device] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            return fail(CX_EHIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", device,
                        hipGetErrorString(e));
        }
        int lds = 0;
        if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device) !=
                hipSuccess ||
            lds <= 0) {
            (void)hipGetLastError();
            lds = 65536;
        }
        g_static_lds[device] = lds;
        g_static_ptr[device] = static_cast<unsigned char*>(p);
    }
    *ptr = g_static_ptr[device];
    *max_lds = g_static_lds[device];
    return CX_OK;
}

}  // namespace

namespace {

// The decode pipeline (T <= 16) serves this layer / router shape.
bool dec_path_ok(const cx_layer* layer, int top_k, const RouteArgs* route) {
    if (layer->n_experts > 256 || top_k > 64) return false;
    if (!dec_shared_ok(layer->hidden, layer->inter)) return false;
    return route == nullptr ||
           (route->x_dtype == CX_DTYPE_BF16 && dec_route_ok(route->n_experts, route->n_group));
}

// Decode pipeline for T <= 16 tokens (plan, h and y_part buffers ready):
//   router:  logits -> [select + plan | shared gate/up] -> routed gate/up
//            -> down (routed + shared items) -> combine
//   routes:  [plan | shared gate/up] -> routed gate/up
//            -> down (routed + shared items) -> combine
// The shared expert's gate/up streams beside the latency-bound selection
// and planner; the routed gate/up grid holds exactly the routed items (one
// resident round at 8 experts), and the down grid adds the shared item.  The
// combine sums in the reference's order: route order, shared expert last.
int moe_decode(cx_ctx* ctx, const cx_layer* layer, const void* x, int in_dtype, int n_tokens,
               const int32_t* ids, const float* w, int top_k, void* y, int out_dtype,
               float* y_f32, hipStream_t s, RouteArgs* route, const PlanSizes& z,
               const PlanPtrs& P) {
    const int T = n_tokens;
    const int np_lds = lds_rows(ctx, layer->hidden, T);
    ExpertLaunch SG{};
    SG.table = nullptr;
    SG.single = layer->shared_desc;
    SG.n_tokens = T;
    SG.hidden = layer->hidden;
    SG.inter = layer->inter;
    SG.maxt = 1;
    SG.x = x;
    SG.in_dtype = in_dtype;
    SG.h_hi = static_cast<uint16_t*>(ctx->hhi.p);  // shared pairs [0, T)
    SG.h_lo = static_cast<uint16_t*>(ctx->hlo.p);
    SG.y_part = static_cast<float*>(ctx->ypart.p);
    SG.np_lds = route != nullptr ? dec_sgu_np_lds(layer->hidden, T, ctx->max_lds) : 0;
    const ExpertLaunch* sg = layer->has_shared ? &SG : nullptr;
    // T <= 8 with the router: the shared gate/up tiles run as two k-parts
    // (twice the CUs); the routed gate/up launch finalises the shared h
    const bool split = route != nullptr && sg != nullptr &&
                       dec_shared_split_ok(layer->hidden, layer->inter, T);
    if (split) {
        int rc = ensure(&ctx->gu_part, sizeof(float) * 2 * 2 * (size_t)T * layer->inter, s);
        if (rc) return rc;
        SG.gu_part = static_cast<float*>(ctx->gu_part.p);
        SG.gu_kparts = 2;
    }
    const int routed_items = std::min(T * top_k, layer->n_experts);
    // One token with the router, no resident mask, every expert of the table
    // resident and the one-launch down + combine: the selection runs inside
    // the routed gate/up launch (each workgroup selects for itself), so the
    // stage between the logits and the routed gate/up is gone; the shared
    // expert's gate/up k-parts move beside the logits.
    const bool fused = route != nullptr && T == 1 && route->resident == nullptr &&
                       route->n_experts == layer->n_experts && route->top_k == top_k &&
                       layer->n_resident == layer->n_experts && np_lds > 0 &&
                       (sg == nullptr || split) &&
                       down_comb1_ok(layer->hidden, layer->inter, top_k, ctx->max_lds) &&
                       dec_fused_sel_ok(route->n_experts, route->n_group, route->topk_group,
                                        layer->hidden, top_k, route->x_dtype);
    double* sc = nullptr;
    if (fused) {
        int rc = ensure(&ctx->scores, sizeof(double) * 2 * (size_t)layer->n_experts, s);
        if (rc) return rc;
        sc = static_cast<double*>(ctx->scores.p);
    }
    if (route != nullptr) {
        route->plan = &P;
        route->table = layer->table;
        route->has_shared = layer->has_shared;
        route->item_cap = z.item_cap;
        route->max_items = z.max_items;
        route->err_flag = ctx->err_flag;
        if (fused) {
            Span sp(ctx, "route", s);
            CX_HIP(launch_dec_logits_sgu(*route, sg, sc, s));
        } else {
            {
                Span sp(ctx, "route", s);
                CX_HIP(launch_dec_logits(*route, s));
            }
            {
                Span sp(ctx, "plan", s);
                CX_HIP(launch_dec_select_sgu(*route, sg, s));
            }
        }
    } else {
        Span sp(ctx, "plan", s);
        CX_HIP(launch_dec_plan_sgu(ids, w, T, top_k, layer->table, layer->n_experts,
                                   layer->has_shared, P, ctx->err_flag, sg, s));
    }
    ExpertLaunch L{};
    L.table = layer->table;
    L.plan = P;
    L.max_items = routed_items;
    L.n_tokens = T;
    L.hidden = layer->hidden;
    L.inter = layer->inter;
    L.maxt = 1;
    L.x = x;
    L.in_dtype = in_dtype;
    L.h_hi = static_cast<uint16_t*>(ctx->hhi.p);
    L.h_lo = static_cast<uint16_t*>(ctx->hlo.p);
    L.y_part = static_cast<float*>(ctx->ypart.p);
    L.y = y;
    L.y_f32 = y_f32;
    L.out_dtype = out_dtype;
    L.np_lds = np_lds;
    L.skip_shared = 1;
    L.gu_part = SG.gu_part;
    L.gu_kparts = SG.gu_kparts;
    if (fused) {
        Span sp(ctx, "gate_up", s);
        CX_HIP(launch_gate_up_sel(L, *route, sc, s));
    } else if (L.max_items > 0 || L.gu_part != nullptr) {
        Span sp(ctx, "gate_up", s);
        CX_HIP(launch_gate_up(L, s));
    }
    L.gu_part = nullptr;
    // down: the routed items and the shared expert's item (last)
    L.skip_shared = 0;
    L.max_items = routed_items + layer->has_shared;
    L.max_lds = ctx->max_lds;
    const float* route_w = route != nullptr ? route->wout : w;
    if (T == 1 && down_comb1_ok(layer->hidden, layer->inter, top_k, ctx->max_lds)) {
        // one token: down of every item and the combine in one launch
        Span sp(ctx, "down", s);
        CX_HIP(launch_down_comb1(L, P.token_pairs, route_w, top_k, ctx->n_cu, s));
        return CX_OK;
    }
    if (L.max_items > 0) {
        Span sp(ctx, "down", s);
        CX_HIP(launch_down(L, s));
    }
    {
        Span sp(ctx, "combine", s);
        CX_HIP(launch_combine_dec(P, route_w, L.y_part, T, top_k,
                                  layer->has_shared, layer->hidden, y, out_dtype, y_f32, s));
    }
    return CX_OK;
}

// Routed-expert compute; when `route` is given, the router runs first on the
// same stream.  T <= 16 takes the decode pipeline where the shapes allow it;
// otherwise route -> plan -> grouped gate/up -> per-pair down -> combine.
// valid_routes: routes with an id >= 0 when the caller knows them on the
// host (the wire entry point), else -1.
int moe_run(cx_ctx* ctx, const cx_layer* layer, const void* x, int in_dtype, int n_tokens,
            const int32_t* ids, const float* w, int top_k, void* y, int out_dtype, float* y_f32,
            hipStream_t s, bool prefill, RouteArgs* route, int64_t valid_routes = -1) {
    if (!ctx || !layer) return fail(CX_EINVAL, "NULL context or layer");
    if (!act16(in_dtype) || !act16(out_dtype)) return fail(CX_EINVAL, "dtypes must be fp16/bf16");
    if (n_tokens <= 0 || top_k < 0 || top_k > 64) return fail(CX_EINVAL, "bad n_tokens/top_k");
    if (!x || !y || (top_k > 0 && (!ids || !w))) return fail(CX_EINVAL, "NULL buffer");
    if (!layer->fast)
        return fail(CX_EUNSUPPORTED, "layer experts do not fit the grouped kernels "
                                     "(need hidden%%64==0, dims%%128==0, 128-column blocks, "
                                     "row blocks multiple of 16)");
    int rc = set_device(ctx->device);
    if (rc) return rc;
    const bool dec = !prefill && n_tokens <= kTileTok && dec_path_ok(layer, top_k, route);
    PlanSizes z = plan_sizes(n_tokens, top_k, layer->n_experts, layer->has_shared);
    if (dec) z.max_items = z.max_slots;  // one item per slot (<= 16 pairs each)
    // Calls with at least kBigPairs pairs per resident routed expert on
    // average: the experts' weights serve hundreds of columns, so 128-pair
    // items through the LDS-ring GEMM instead of 64-pair items that each
    // re-stream them.  The pairs are counted on the host: exactly when the
    // caller knows its valid routes (the wire entry point), else as every
    // route slot, an upper bound — route tables masked to one node of
    // several (-1 for other nodes' experts) can then take the LDS-ring path
    // with mostly-padding tiles (correct, slower).
    const int64_t pairs = valid_routes >= 0 ? valid_routes : (int64_t)n_tokens * top_k;
    const bool big = !dec && big_shape_ok(layer->hidden, layer->inter, in_dtype) &&
                     pairs >= (int64_t)kBigPairs * std::max(1, layer->n_resident);
    if (big) {
        z.item_cap = kBigPairs;
        z.max_items = z.max_slots + (z.max_pairs + kBigPairs - 1) / kBigPairs;
    }
    if (z.max_pairs == 0) return fail(CX_EINVAL, "nothing to compute");
    PlanPtrs P;
    if ((rc = carve_plan(ctx, z, n_tokens, top_k, dec, s, &P))) return rc;
    const size_t H = layer->hidden, I = layer->inter;
    if ((rc = ensure(&ctx->hhi, (size_t)z.max_pairs * I * 2, s))) return rc;
    if ((rc = ensure(&ctx->hlo, (size_t)z.max_pairs * I * 2, s))) return rc;
    if ((rc = ensure(&ctx->ypart, (size_t)z.max_pairs * H * 4, s))) return rc;
    if (dec)
        return moe_decode(ctx, layer, x, in_dtype, n_tokens, ids, w, top_k, y, out_dtype, y_f32,
                          s, route, z, P);
    if (route != nullptr) {
        route->plan = &P;
        route->table = layer->table;
        route->has_shared = layer->has_shared;
        route->item_cap = z.item_cap;
        route->max_items = z.max_items;
        route->err_flag = ctx->err_flag;
        Span sp(ctx, "route", s);
        CX_HIP(launch_route(*route, s));
    } else {
        Span sp(ctx, "plan", s);
        CX_HIP(launch_plan(ids, w, n_tokens, top_k, layer->table, layer->n_experts,
                           layer->has_shared, z.item_cap, z.max_items, P, ctx->err_flag, s));
    }
    ExpertLaunch L{};
    L.table = layer->table;
    L.plan = P;
    L.max_items = z.max_items;
    L.n_tokens = n_tokens;
    L.hidden = layer->hidden;
    L.inter = layer->inter;
    L.maxt = z.maxt;
    L.x = x;
    L.in_dtype = in_dtype;
    L.h_hi = static_cast<uint16_t*>(ctx->hhi.p);
    L.h_lo = static_cast<uint16_t*>(ctx->hlo.p);
    L.y_part = static_cast<float*>(ctx->ypart.p);
    L.y = y;
    L.y_f32 = y_f32;
    L.out_dtype = out_dtype;
    L.np_lds = z.maxt == 1 ? lds_rows(ctx, layer->hidden, std::min(n_tokens, z.item_cap)) : 0;
    L.max_lds = ctx->max_lds;
    {
        Span sp(ctx, "gate_up", s);
        CX_HIP(big ? launch_gate_up_big(L, s) : launch_gate_up(L, s));
    }
    {
        Span sp(ctx, "down", s);
        CX_HIP(big ? launch_down_big(L, s) : launch_down(L, s));
    }
    {
        Span sp(ctx, "combine", s);
        CX_HIP(launch_combine(P, L.y_part, n_tokens, top_k, layer->hidden, y, out_dtype, y_f32, s));
    }
    return CX_OK;
}

int fill_route(cx_ctx* ctx, const void* x, int x_dtype, const void* w_router, int w_dtype,
               const float* bias, const uint8_t* resident, int n_tokens, int hidden,
               int n_experts, int n_group, int topk_group, int top_k, int norm,
               float scale, int32_t* ids, float* wout, hipStream_t s, RouteArgs* R) {
    if (!ctx) return fail(CX_EINVAL, "NULL context");
    if (!x || !w_router || !bias || !ids || !wout) return fail(CX_EINVAL, "NULL buffer");
    if ((x_dtype != CX_DTYPE_BF16 && x_dtype != CX_DTYPE_F32) ||
        (w_dtype != CX_DTYPE_BF16 && w_dtype != CX_DTYPE_F32))
        return fail(CX_EINVAL, "router x / weight dtype must be bf16 or fp32");
    if (n_tokens <= 0 || hidden <= 0 || hidden % 8 != 0)
        return fail(CX_EINVAL, "hidden must be a positive multiple of 8");
    if (n_experts <= 0 || n_experts > 512) return fail(CX_EINVAL, "n_experts must be 1..512");
    if (n_group <= 0 || n_group > 64 || n_experts % n_group != 0)
        return fail(CX_EINVAL, "num_experts=%d not divisible by n_group=%d", n_experts, n_group);
    if (topk_group <= 0 || topk_group > n_group)
        return fail(CX_EINVAL, "invalid topk_group=%d for n_group=%d", topk_group, n_group);
    if (top_k <= 0 || top_k > n_experts || top_k > 64)
        return fail(CX_EINVAL, "invalid top_k=%d for num_experts=%d", top_k, n_experts);
    int rc = set_device(ctx->device);
    if (rc) return rc;
    if ((rc = ensure(&ctx->logits, (size_t)n_tokens * n_experts * 8, s))) return rc;
    ctx->route_T = n_tokens;
    ctx->route_E = n_experts;
    *R = RouteArgs{};
    R->x = x;
    R->x_dtype = x_dtype;
    R->w = w_router;
    R->w_dtype = w_dtype;
    R->bias = bias;
    R->resident = resident;
    R->n_tokens = n_tokens;
    R->hidden = hidden;
    R->n_experts = n_experts;
    R->n_group = n_group;
    R->topk_group = topk_group;
    R->top_k = top_k;
    R->norm = norm;
    R->scale = scale;
    R->logits = static_cast<double*>(ctx->logits.p);
    R->ids = ids;
    R->wout = wout;
    return CX_OK;
}

}  // namespace

// ===========================================================================
// Whole-layer wire message helpers (MoeLayerRequest / MoeLayerResponse, cx_moe.h).
namespace {

struct LayerReq {
    cx_moe_layer_request_info info;
    const uint8_t* ids;  // int32 [n_routes], little-endian, unaligned
    const uint8_t* w;    // float [n_routes]
    const uint8_t* act;  // [T, H] 16-bit
    size_t n_routes, act_bytes;
};

bool rd32(const uint8_t* b, size_t n, size_t* off, uint32_t* v) {
    if (*off > n || n - *off < 4) return false;
    std::memcpy(v, b + *off, 4);
    *off += 4;
    return true;
}

// Exact-length decode (every field consumed, nothing trailing), as
// DecodeInferRequestBody (common/infer_codec.cc:22-43) requires.
int parse_layer_req(const uint8_t* body, size_t len, LayerReq* r) {
    if (!body) return fail(CX_EINVAL, "NULL request body");
    size_t off = 0;
    uint32_t f[8];
    for (int i = 0; i < 8; ++i)
        if (!rd32(body, len, &off, &f[i])) return fail(CX_EINVAL, "request body truncated in header");
    cx_moe_layer_request_info& h = r->info;
    h.layer_id = (int32_t)f[0];
    h.batch_size = (int32_t)f[1];
    h.hidden_dim = (int32_t)f[2];
    h.top_k = (int32_t)f[3];
    h.input_dtype = f[4];
    h.output_dtype = f[5];
    h.flags = f[6];
    const uint32_t n_routes = f[7];
    if (h.batch_size <= 0 || h.hidden_dim <= 0 || h.top_k < 0 || h.top_k > 64)
        return fail(CX_EINVAL, "bad batch_size/hidden_dim/top_k (%d, %d, %d)", h.batch_size,
                    h.hidden_dim, h.top_k);
    if (!act16((int)h.input_dtype) || !act16((int)h.output_dtype))
        return fail(CX_EINVAL, "activation dtypes must be fp16 (1) or bf16 (2)");
    if (h.flags & ~CX_MOE_LAYER_FLAG_SHARED) return fail(CX_EINVAL, "unknown flags 0x%x", h.flags);
    if ((uint64_t)n_routes != (uint64_t)h.batch_size * (uint64_t)h.top_k)
        return fail(CX_EINVAL, "n_routes %u != batch_size * top_k", n_routes);
    const uint64_t rb = (uint64_t)n_routes * 4;
    if (len - off < 2 * rb) return fail(CX_EINVAL, "request body truncated in routes");
    r->n_routes = n_routes;
    r->ids = body + off;
    r->w = body + off + rb;
    off += 2 * rb;
    uint32_t nb = 0;
    if (!rd32(body, len, &off, &nb)) return fail(CX_EINVAL, "request body truncated before activation");
    const uint64_t want = (uint64_t)h.batch_size * (uint64_t)h.hidden_dim * 2;
    if (nb != want) return fail(CX_EINVAL, "activation_nbytes %u != batch*hidden*2", nb);
    if (len - off != nb) return fail(CX_EINVAL, "request body length mismatch (trailing or missing bytes)");
    r->act = body + off;
    r->act_bytes = nb;
    return CX_OK;
}

size_t put32(uint8_t* b, size_t off, uint32_t v) {
    std::memcpy(b + off, &v, 4);
    return off + 4;
}

size_t write_layer_resp(uint8_t* resp, int status, const cx_moe_layer_request_info& h,
                        uint32_t nbytes) {
    size_t o = 0;
    o = put32(resp, o, (uint32_t)status);
    o = put32(resp, o, (uint32_t)h.batch_size);
    o = put32(resp, o, (uint32_t)h.hidden_dim);
    o = put32(resp, o, h.output_dtype);
    o = put32(resp, o, nbytes);
    return o + nbytes;  // body length: header + the output bytes that follow it
}

int pin_ensure(void** p, size_t* cap, size_t bytes) {
    if (*cap >= bytes) return CX_OK;
    if (*p) (void)hipHostFree(*p);
    *p = nullptr;
    *cap = 0;
    CX_HIP(hipHostMalloc(p, bytes, hipHostMallocDefault));
    *cap = bytes;
    return CX_OK;
}

}  // namespace

extern "C" {

const char* cx_last_error(void) { return g_err.c_str(); }
const char* cx_version(void) { return "constellation_amd cx_moe 0.1 (gfx950)"; }

int cx_device_count(int* count) {
    if (!count) return fail(CX_EINVAL, "NULL count");
    *count = 0;
    CX_HIP(hipGetDeviceCount(count));
    return CX_OK;
}

int cx_device_query(int device, cx_device_info* out) {
    if (!out) return fail(CX_EINVAL, "NULL out");
    std::memset(out, 0, sizeof(*out));
    DeviceRestore restore;  // the node probes from its control thread
    int rc = set_device(device);
    if (rc) return rc;
    hipDeviceProp_t prop;
    CX_HIP(hipGetDeviceProperties(&prop, device));
    std::snprintf(out->name, sizeof(out->name), "%s", prop.name);
    std::snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
    if (out->name[0] == '\0') {
        // the marketing name comes from libdrm's amdgpu.ids, which a host may
        // lack: name the device by its architecture instead
        const size_t n = std::strcspn(prop.gcnArchName, ":");
        std::snprintf(out->name, sizeof(out->name), "AMD %.*s", static_cast<int>(n), prop.gcnArchName);
    }
    out->total_mem_bytes = prop.totalGlobalMem;
    size_t fr = 0, tot = 0;
    CX_HIP(hipMemGetInfo(&fr, &tot));
    out->free_mem_bytes = fr;
    out->compute_units = prop.multiProcessorCount;
    uint32_t caps = 1u | 2u;  // kGpuCapFp16 | kGpuCapBf16 (common/types.h:76-77)
    if (std::strncmp(prop.gcnArchName, "gfx95", 5) == 0 || std::strncmp(prop.gcnArchName, "gfx94", 5) == 0)
        caps |= 4u;           // kGpuCapFp8
    out->capability_flags = caps;
    int xcc = 0;
    if (hipDeviceGetAttribute(&xcc, hipDeviceAttributeNumberOfXccs, device) != hipSuccess) {
        (void)hipGetLastError();
        xcc = 0;
    }
    out->num_xcds = xcc;
    return CX_OK;
}

int cx_upload_matrix(int device, const uint8_t* host_weight, uint64_t rows, uint64_t cols,
                     const float* host_scale, uint64_t scale_count, uint8_t** dev_weight,
                     float** dev_scale) {
    if (!dev_weight || !dev_scale) return fail(CX_EINVAL, "NULL output pointer");
    *dev_weight = nullptr;
    *dev_scale = nullptr;
    if (!host_weight || !host_scale || rows == 0 || cols == 0 || scale_count == 0)
        return fail(CX_EINVAL, "empty matrix or scales");
    int rc = set_device(device);
    if (rc) return rc;
    const size_t wbytes = rows * cols, sbytes = scale_count * 4;
    void *pw = nullptr, *ps = nullptr;
    if ((rc = arena_alloc(device, wbytes, &pw))) return rc;
    if ((rc = arena_alloc(device, sbytes, &ps))) {
        arena_free(device, pw, false);
        return rc;
    }
    hipStream_t s = upload_stream(device);
    hipError_t e = hipMemcpyAsync(pw, host_weight, wbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(ps, host_scale, sbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = launch_canonicalize_fp8(static_cast<uint8_t*>(pw), wbytes, s);
    // wait even after a failure: a copy queued before it may still write the blocks
    const hipError_t es = hipStreamSynchronize(s);
    if (e == hipSuccess) e = es;
    if (e != hipSuccess) {
        arena_free(device, pw, false);
        arena_free(device, ps, false);
        return fail(CX_EHIP, "upload failed: %s", hipGetErrorString(e));
    }
    *dev_weight = static_cast<uint8_t*>(pw);
    *dev_scale = static_cast<float*>(ps);
    return CX_OK;
}

int cx_upload_matrix_tiled(int device, const uint8_t* host_weight, uint64_t rows, uint64_t cols,
                           const float* host_scale, uint64_t scale_count, uint8_t** dev_weight,
                           float** dev_scale) {
    if (!dev_weight || !dev_scale) return fail(CX_EINVAL, "NULL output pointer");
    *dev_weight = nullptr;
    *dev_scale = nullptr;
    if (!host_weight || !host_scale || rows == 0 || cols == 0 || scale_count == 0)
        return fail(CX_EINVAL, "empty matrix or scales");
    if (!gu_tile16_ok(rows, cols) || rows > (1u << 30) || cols > (1u << 30))
        return fail(CX_EINVAL, "tiled upload needs rows %% 16 == 0 and cols %% 128 == 0 (got %llu x %llu)",
                    (unsigned long long)rows, (unsigned long long)cols);
    int rc = set_device(device);
    if (rc) return rc;
    const size_t wbytes = rows * cols, sbytes = scale_count * 4;
    void *pw = nullptr, *ps = nullptr, *stage = nullptr;
    if ((rc = arena_alloc(device, wbytes, &pw))) return rc;
    if ((rc = arena_alloc(device, sbytes, &ps))) {
        arena_free(device, pw, false);
        return rc;
    }
    // the wire bytes land in a second arena block first (freed before
    // returning), then one kernel re-tiles them into the expert's block
    if ((rc = arena_alloc(device, wbytes, &stage))) {
        arena_free(device, pw, false);
        arena_free(device, ps, false);
        return rc;
    }
    hipStream_t s = upload_stream(device);
    hipError_t e = hipMemcpyAsync(stage, host_weight, wbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(ps, host_scale, sbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = launch_tile16_fp8(static_cast<const uint8_t*>(stage), static_cast<uint8_t*>(pw), (int)rows,
                              (int)cols, s);
    // wait even after a failure: a copy queued before it may still write the stage block
    const hipError_t es = hipStreamSynchronize(s);
    if (e == hipSuccess) e = es;
    arena_free(device, stage, false);
    if (e != hipSuccess) {
        arena_free(device, pw, false);
        arena_free(device, ps, false);
        return fail(CX_EHIP, "tiled upload failed: %s", hipGetErrorString(e));
    }
    *dev_weight = static_cast<uint8_t*>(pw);
    *dev_scale = static_cast<float*>(ps);
    return CX_OK;
}

int cx_free_device(int device, void* dev_ptr) {
    if (device >= 64) return fail(CX_EINVAL, "bad device");
    if (device >= 0) return arena_free(device, dev_ptr);
    // device < 0: the caller does not track the owning device; find the arena
    // that holds the pointer (weights of one expert never span devices).
    if (dev_ptr == nullptr) return CX_OK;
    for (int d = 0; d < 64; ++d) {
        Arena& A = arena(d);
        {
            std::lock_guard<std::mutex> lk(A.mu);
            if (A.live.find(dev_ptr) == A.live.end()) continue;
        }
        return arena_free(d, dev_ptr);
    }
    return fail(CX_EINVAL, "cx_free_device: %p not allocated here", dev_ptr);
}

int cx_arena_stats(int device, uint64_t* used_bytes, uint64_t* reserved_bytes) {
    if (device < 0 || device >= 64) return fail(CX_EINVAL, "bad device");
    Arena& A = arena(device);
    std::lock_guard<std::mutex> lk(A.mu);
    if (used_bytes) *used_bytes = A.used;
    if (reserved_bytes) *reserved_bytes = A.reserved;
    return CX_OK;
}

int cx_ctx_create(int device, cx_ctx** out) {
    if (!out) return fail(CX_EINVAL, "NULL out");
    *out = nullptr;
    int rc = set_device(device);
    if (rc) return rc;
    cx_ctx* c = new (std::nothrow) cx_ctx();
    if (!c) return fail(CX_ENOMEM, "out of host memory");
    c->device = device;
    if (hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess ||
        hipMalloc(&c->err_flag, 2 * sizeof(int)) != hipSuccess ||
        hipMemset(c->err_flag, 0, 2 * sizeof(int)) != hipSuccess) {
        cx_ctx_destroy(c);
        return fail(CX_EHIP, "context init failed");
    }
    int lds = 0;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device) == hipSuccess &&
        lds > 0)
        c->max_lds = lds;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
        c->n_cu = cus;
    (void)hipGetLastError();
    *out = c;
    return CX_OK;
}

int cx_ctx_destroy(cx_ctx* c) {
    if (!c) return CX_OK;
    (void)hipSetDevice(c->device);
    (void)hipDeviceSynchronize();
    drain_spans(c);
    DevBuf* bufs[] = {&c->plan_buf, &c->hhi, &c->hlo, &c->ypart, &c->logits, &c->route_ids,
                      &c->route_w, &c->hscratch, &c->gu_part, &c->scores, &c->dx, &c->dy};
    for (DevBuf* b : bufs)
        if (b->p) (void)hipFree(b->p);
    if (c->err_flag) (void)hipFree(c->err_flag);
    if (c->pin_x) (void)hipHostFree(c->pin_x);
    if (c->pin_y) (void)hipHostFree(c->pin_y);
    if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
    delete c;
    return CX_OK;
}

int cx_ctx_sync(cx_ctx* ctx, void* stream) {
    if (!ctx) return fail(CX_EINVAL, "NULL context");
    int rc = set_device(ctx->device);
    if (rc) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int flag = 0;
    CX_HIP(hipMemcpyAsync(&flag, ctx->err_flag, sizeof(int), hipMemcpyDeviceToHost, s));
    CX_HIP(hipStreamSynchronize(s));
    if (flag != 0) {
        CX_HIP(hipMemsetAsync(ctx->err_flag, 0, sizeof(int), s));
        CX_HIP(hipStreamSynchronize(s));
        return fail(CX_EDEVICE, "device check failed (flags 0x%x:%s%s%s%s%s)", flag,
                    (flag & kErrBadExpertId) ? " expert id out of range" : "",
                    (flag & kErrNotResident) ? " expert not resident" : "",
                    (flag & kErrPlanOverflow) ? " plan overflow" : "",
                    (flag & kErrDuplicateRoute) ? " expert routed twice for one token" : "",
                    (flag & kErrBadWeight) ? " negative or non-finite route weight" : "");
    }
    return CX_OK;
}

int cx_ctx_profile(cx_ctx* ctx, int enable) {
    if (!ctx) return fail(CX_EINVAL, "NULL context");
    int rc = set_device(ctx->device);
    if (rc) return rc;
    drain_spans(ctx);
    if (enable) ctx->totals.clear();
    ctx->prof = enable != 0;
    return CX_OK;
}

int cx_ctx_profile_read(cx_ctx* ctx, const char* kernel, int* launches, double* total_ms) {
    if (!ctx || !kernel || !launches || !total_ms) return fail(CX_EINVAL, "NULL argument");
    int rc = set_device(ctx->device);
    if (rc) return rc;
    drain_spans(ctx);
    auto it = ctx->totals.find(kernel);
    *launches = it == ctx->totals.end() ? 0 : it->second.first;
    *total_ms = it == ctx->totals.end() ? 0.0 : it->second.second;
    return CX_OK;
}

int cx_expert_run(cx_ctx* ctx, const cx_expert_desc* expert, const void* x, int in_dtype,
                  int n_tokens, void* y, int out_dtype, float* y_f32, void* stream) {
    if (!ctx) return fail(CX_EINVAL, "NULL context");
    int rc = check_desc(expert);
    if (rc) return rc;
    if (!act16(in_dtype) || !act16(out_dtype)) return fail(CX_EINVAL, "dtypes must be fp16/bf16");
    if (n_tokens <= 0 || !x || !y) return fail(CX_EINVAL, "bad n_tokens or NULL buffer");
    if ((rc = set_device(ctx->device))) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    ExpertPlan P = plan_expert(*expert, x, in_dtype, n_tokens, y, out_dtype, y_f32, ctx->max_lds);
    if (P.h_f32_bytes && (rc = ensure(&ctx->hscratch, P.h_f32_bytes, s))) return rc;
    if (P.h_plane_bytes && ((rc = ensure(&ctx->hhi, P.h_plane_bytes, s)) ||
                            (rc = ensure(&ctx->hlo, P.h_plane_bytes, s))))
        return rc;
    if (P.gu_part_bytes && (rc = ensure(&ctx->gu_part, P.gu_part_bytes, s))) return rc;
    return run_expert(ctx, P, *expert, x, in_dtype, n_tokens, y, out_dtype, y_f32,
                      static_cast<float*>(ctx->hscratch.p), static_cast<uint16_t*>(ctx->hhi.p),
                      static_cast<uint16_t*>(ctx->hlo.p), static_cast<float*>(ctx->gu_part.p), s);
}

int cx_expert_run_static(int device, const cx_expert_desc* expert, const void* x, int in_dtype,
                         int n_tokens, void* y, int out_dtype, float* y_f32, void* stream) {
    int rc = check_desc(expert);
    if (rc) return rc;
    if (!act16(in_dtype) || !act16(out_dtype)) return fail(CX_EINVAL, "dtypes must be fp16/bf16");
    if (n_tokens <= 0 || !x || !y) return fail(CX_EINVAL, "bad n_tokens or NULL buffer");
    if (device < 0 || device >= kMaxDevices) return fail(CX_EINVAL, "invalid device %d", device);
    if ((rc = set_device(device))) return rc;
    unsigned char* base = nullptr;
    int max_lds = 0;
    if ((rc = static_scratch(device, &base, &max_lds))) return rc;
    ExpertPlan P = plan_expert(*expert, x, in_dtype, n_tokens, y, out_dtype, y_f32, max_lds);
    // one region per path: fp32 h, or h_hi then h_lo (256-B aligned), or the part sums
    const size_t lo_off = (P.h_plane_bytes + 255) & ~(size_t)255;
    const size_t need = std::max({P.h_f32_bytes, lo_off + P.h_plane_bytes, P.gu_part_bytes});
    if (need > CX_STATIC_SCRATCH_BYTES)
        return fail(CX_EINVAL,
                    "cx_expert_run_static: %d tokens x inter %d need %zu scratch bytes, "
                    "more than the static %d (use cx_expert_run)",
                    n_tokens, expert->inter, need, (int)CX_STATIC_SCRATCH_BYTES);
    return run_expert(nullptr, P, *expert, x, in_dtype, n_tokens, y, out_dtype, y_f32,
                      reinterpret_cast<float*>(base), reinterpret_cast<uint16_t*>(base),
                      reinterpret_cast<uint16_t*>(base + lo_off), reinterpret_cast<float*>(base),
                      static_cast<hipStream_t>(stream));
}

int cx_expert_run_host(cx_ctx* ctx, const cx_expert_desc* expert, const void* x_host,
                       size_t x_bytes, int in_dtype, int n_tokens, void* y_host, size_t y_bytes,
                       int out_dtype) {
    if (!ctx) return fail(CX_EINVAL, "NULL context");
    int rc = check_desc(expert);
    if (rc) return rc;
    if (!act16(in_dtype) || !act16(out_dtype)) return fail(CX_EINVAL, "dtypes must be fp16/bf16");
    if (n_tokens <= 0 || !x_host || !y_host) return fail(CX_EINVAL, "bad n_tokens or NULL buffer");
    const size_t elems = (size_t)n_tokens * expert->hidden;
    if (x_bytes != elems * act_size(in_dtype))
        return fail(CX_EINVAL, "activation bytes %zu != batch*hidden*%zu", x_bytes, act_size(in_dtype));
    if (y_bytes != elems * act_size(out_dtype))
        return fail(CX_EINVAL, "output bytes %zu != batch*hidden*%zu", y_bytes, act_size(out_dtype));
    if ((rc = set_device(ctx->device))) return rc;
    hipStream_t s = ctx->own_stream;
    if ((rc = ensure(&ctx->dx, x_bytes, s))) return rc;
    if ((rc = ensure(&ctx->dy, y_bytes, s))) return rc;
    if (ctx->pin_x_bytes < x_bytes) {
        if (ctx->pin_x) (void)hipHostFree(ctx->pin_x);
        ctx->pin_x = nullptr;
        ctx->pin_x_bytes = 0;
        CX_HIP(hipHostMalloc(&ctx->pin_x, x_bytes, hipHostMallocDefault));
        ctx->pin_x_bytes = x_bytes;
    }
    if (ctx->pin_y_bytes < y_bytes) {
        if (ctx->pin_y) (void)hipHostFree(ctx->pin_y);
        ctx->pin_y = nullptr;
        ctx->pin_y_bytes = 0;
        CX_HIP(hipHostMalloc(&ctx->pin_y, y_bytes, hipHostMallocDefault));
        ctx->pin_y_bytes = y_bytes;
    }
    std::memcpy(ctx->pin_x, x_host, x_bytes);
    CX_HIP(hipMemcpyAsync(ctx->dx.p, ctx->pin_x, x_bytes, hipMemcpyHostToDevice, s));
    if ((rc = cx_expert_run(ctx, expert, ctx->dx.p, in_dtype, n_tokens, ctx->dy.p, out_dtype,
                            nullptr, s)))
        return rc;
    CX_HIP(hipMemcpyAsync(ctx->pin_y, ctx->dy.p, y_bytes, hipMemcpyDeviceToHost, s));
    CX_HIP(hipStreamSynchronize(s));
    std::memcpy(y_host, ctx->pin_y, y_bytes);
    return CX_OK;
}

int cx_layer_create(cx_ctx* ctx, int n_experts, const cx_expert_desc* const* experts,
                    const cx_expert_desc* shared, cx_layer** out) {
    if (!ctx || !out) return fail(CX_EINVAL, "NULL argument");
    *out = nullptr;
    if (n_experts <= 0 || n_experts > 4096) return fail(CX_EINVAL, "n_experts must be 1..4096");
    int rc = set_device(ctx->device);
    if (rc) return rc;
    std::vector<cx_expert_desc> host(n_experts + 1);
    std::memset(host.data(), 0, sizeof(cx_expert_desc) * host.size());
    int H = 0, I = 0, fast = 1, any = 0;
    auto take = [&](const cx_expert_desc* e, cx_expert_desc* dst) -> int {
        int r = check_desc(e);
        if (r) return r;
        if (any && (e->hidden != H || e->inter != I))
            return fail(CX_EINVAL, "all experts of a layer must share hidden/inter dims");
        H = e->hidden;
        I = e->inter;
        any = 1;
        fast &= fast_path_ok(*e) ? 1 : 0;
        *dst = *e;
        return CX_OK;
    };
    for (int i = 0; i < n_experts; ++i)
        if (experts && experts[i] && (rc = take(experts[i], &host[i]))) return rc;
    if (shared && (rc = take(shared, &host[n_experts]))) return rc;
    if (!any) return fail(CX_EINVAL, "layer has no resident expert");
    cx_layer* L = new (std::nothrow) cx_layer();
    if (!L) return fail(CX_ENOMEM, "out of host memory");
    L->n_experts = n_experts;
    L->has_shared = shared ? 1 : 0;
    L->resident.assign(n_experts, 0);
    for (int i = 0; i < n_experts; ++i) L->resident[i] = (experts && experts[i]) ? 1 : 0;
    for (int i = 0; i < n_experts; ++i) L->n_resident += L->resident[i];
    L->shared_desc = host[n_experts];
    L->fast = fast;
    L->hidden = H;
    L->inter = I;
    if (hipMalloc(&L->table, sizeof(cx_expert_desc) * host.size()) != hipSuccess ||
        hipMemcpy(L->table, host.data(), sizeof(cx_expert_desc) * host.size(),
                  hipMemcpyHostToDevice) != hipSuccess) {
        if (L->table) (void)hipFree(L->table);
        delete L;
        return fail(CX_EHIP, "layer table upload failed");
    }
    *out = L;
    return CX_OK;
}

int cx_layer_destroy(cx_ctx* ctx, cx_layer* layer) {
    if (!layer) return CX_OK;
    if (ctx) (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();
    if (layer->table) (void)hipFree(layer->table);
    delete layer;
    return CX_OK;
}

int cx_route(cx_ctx* ctx, const void* x, int x_dtype, const void* w_router, int w_dtype,
             const float* bias, const uint8_t* resident, int n_tokens, int hidden, int n_experts,
             int n_group, int topk_group, int top_k, int norm_topk_prob,
             float routed_scaling_factor, int32_t* topk_ids, float* topk_w, void* stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    RouteArgs R{};
    int rc = fill_route(ctx, x, x_dtype, w_router, w_dtype, bias, resident, n_tokens, hidden,
                        n_experts, n_group, topk_group, top_k, norm_topk_prob,
                        routed_scaling_factor, topk_ids, topk_w, s, &R);
    if (rc) return rc;
    Span sp(ctx, "route", s);
    CX_HIP(launch_route(R, s));
    return CX_OK;
}

int cx_route_logits(cx_ctx* ctx, double* out, int n_tokens, int n_experts, void* stream) {
    if (!ctx || !out) return fail(CX_EINVAL, "NULL argument");
    if (ctx->route_T == 0 || n_tokens != ctx->route_T || n_experts != ctx->route_E)
        return fail(CX_EINVAL, "no router logits of shape [%d, %d] (last router call: [%d, %d])",
                    n_tokens, n_experts, ctx->route_T, ctx->route_E);
    int rc = set_device(ctx->device);
    if (rc) return rc;
    CX_HIP(hipMemcpyAsync(out, ctx->logits.p, (size_t)n_tokens * n_experts * sizeof(double),
                          hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)));
    return CX_OK;
}

int cx_moe_decode(cx_ctx* ctx, const cx_layer* layer, const void* x, int in_dtype, int n_tokens,
                  const int32_t* topk_ids, const float* topk_w, int top_k, void* y, int out_dtype,
                  float* y_f32, void* stream) {
    return moe_run(ctx, layer, x, in_dtype, n_tokens, topk_ids, topk_w, top_k, y, out_dtype,
                   y_f32, static_cast<hipStream_t>(stream), false, nullptr);
}

int cx_moe_prefill(cx_ctx* ctx, const cx_layer* layer, const void* x, int in_dtype, int n_tokens,
                   const int32_t* topk_ids, const float* topk_w, int top_k, void* y,
                   int out_dtype, float* y_f32, void* stream) {
    return moe_run(ctx, layer, x, in_dtype, n_tokens, topk_ids, topk_w, top_k, y, out_dtype,
                   y_f32, static_cast<hipStream_t>(stream), true, nullptr);
}

int cx_moe_layer(cx_ctx* ctx, const cx_layer* layer, const void* x, int in_dtype, int n_tokens,
                 const void* w_router, int w_dtype, const float* bias, const uint8_t* resident,
                 int n_group, int topk_group, int top_k, int norm_topk_prob,
                 float routed_scaling_factor, void* y, int out_dtype, float* y_f32,
                 int32_t* topk_ids, float* topk_w, void* stream) {
    if (!ctx || !layer) return fail(CX_EINVAL, "NULL context or layer");
    if (in_dtype != CX_DTYPE_BF16)
        return fail(CX_EINVAL, "cx_moe_layer routes bf16 activations (in_dtype must be bf16)");
    int rc = set_device(ctx->device);
    if (rc) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int32_t* ids = topk_ids;
    float* w = topk_w;
    if (!ids) {
        if ((rc = ensure(&ctx->route_ids, (size_t)n_tokens * top_k * 4, s))) return rc;
        ids = static_cast<int32_t*>(ctx->route_ids.p);
    }
    if (!w) {
        if ((rc = ensure(&ctx->route_w, (size_t)n_tokens * top_k * 4, s))) return rc;
        w = static_cast<float*>(ctx->route_w.p);
    }
    RouteArgs R{};
    if ((rc = fill_route(ctx, x, in_dtype, w_router, w_dtype, bias, resident, n_tokens,
                         layer->hidden, layer->n_experts, n_group, topk_group, top_k,
                         norm_topk_prob, routed_scaling_factor, ids, w, s, &R)))
        return rc;
    return moe_run(ctx, layer, x, in_dtype, n_tokens, ids, w, top_k, y, out_dtype, y_f32, s,
                   n_tokens > kTileTok, &R);
}

// ---------------------------------------------------------------------------
// Whole-layer wire message (MoeLayerRequest / MoeLayerResponse, cx_moe.h).


int cx_moe_layer_request_peek(const uint8_t* body, size_t body_len, cx_moe_layer_request_info* out) {
    if (!out) return fail(CX_EINVAL, "NULL output");
    LayerReq r;
    const int rc = parse_layer_req(body, body_len, &r);
    if (rc) return rc;
    *out = r.info;
    return CX_OK;
}

size_t cx_moe_layer_response_size(int batch_size, int hidden_dim) {
    if (batch_size <= 0 || hidden_dim <= 0) return 20;
    return 20 + (size_t)batch_size * (size_t)hidden_dim * 2;
}

int cx_moe_layer_request_run(cx_ctx* ctx, const cx_layer* layer, const uint8_t* body,
                             size_t body_len, uint8_t* resp, size_t resp_cap, size_t* resp_len) {
    if (!ctx || !layer || !resp || !resp_len) return fail(CX_EINVAL, "NULL argument");
    *resp_len = 0;
    LayerReq r;
    int rc = parse_layer_req(body, body_len, &r);
    if (rc) return rc;
    const cx_moe_layer_request_info& h = r.info;
    const int T = h.batch_size, H = h.hidden_dim, K = h.top_k;
    const size_t out_bytes = (size_t)T * H * 2;
    if (resp_cap < 20 + out_bytes) return fail(CX_EINVAL, "response buffer %zu < %zu", resp_cap, 20 + out_bytes);
    // request-level checks, mapped to the worker's status codes
    int status = 0;
    bool any_route = false;
    bool bad_weight = false;
    int64_t n_valid = 0;
    for (size_t i = 0; i < r.n_routes && status != 1; ++i) {
        int32_t id;
        float wt;
        std::memcpy(&id, r.ids + 4 * i, 4);
        std::memcpy(&wt, r.w + 4 * i, 4);
        if (id < 0) continue;
        any_route = true;
        ++n_valid;
        // validate_routes (server/moe_layer_runtime.py:96-97) rejects negative
        // weights; a non-finite one cannot be combined either
        if (!(wt >= 0.0f) || wt > 3.4028234663852886e38f) bad_weight = true;
        if (id >= layer->n_experts) status = 1;
        else if (!layer->resident[id] && status == 0) status = 2;
    }
    if (status == 0 && bad_weight) status = 4;
    const bool want_shared = (h.flags & CX_MOE_LAYER_FLAG_SHARED) != 0;
    if (status == 0 && want_shared && !layer->has_shared) status = 2;
    if (status == 0 && (H != layer->hidden || !layer->fast)) status = 4;
    if (status != 0) {
        *resp_len = write_layer_resp(resp, status, h, 0);
        return CX_OK;
    }
    if ((rc = set_device(ctx->device))) return rc;
    hipStream_t s = ctx->own_stream;
    if (!any_route && !want_shared) {  // nothing on this node: y = 0
        std::memset(resp + 20, 0, out_bytes);
        *resp_len = write_layer_resp(resp, 0, h, (uint32_t)out_bytes);
        return CX_OK;
    }
    // staging: [ids | weights | pad | activation], one copy each way
    const size_t rb = r.n_routes * 4;
    const size_t act_off = (2 * rb + 255) & ~(size_t)255;
    const size_t in_bytes = act_off + r.act_bytes;
    if ((rc = pin_ensure(&ctx->pin_x, &ctx->pin_x_bytes, in_bytes))) return rc;
    if ((rc = pin_ensure(&ctx->pin_y, &ctx->pin_y_bytes, out_bytes))) return rc;
    if ((rc = ensure(&ctx->dx, in_bytes, s))) return rc;
    if ((rc = ensure(&ctx->dy, out_bytes, s))) return rc;
    uint8_t* px = static_cast<uint8_t*>(ctx->pin_x);
    std::memcpy(px, r.ids, 2 * rb);
    std::memcpy(px + act_off, r.act, r.act_bytes);
    CX_HIP(hipMemcpyAsync(ctx->dx.p, px, in_bytes, hipMemcpyHostToDevice, s));
    uint8_t* dx = static_cast<uint8_t*>(ctx->dx.p);
    cx_layer view = *layer;  // the shared expert joins only when asked for
    view.has_shared = want_shared ? layer->has_shared : 0;
    rc = moe_run(ctx, &view, dx + act_off, (int)h.input_dtype, T,
                 K > 0 ? reinterpret_cast<const int32_t*>(dx) : nullptr,
                 K > 0 ? reinterpret_cast<const float*>(dx + rb) : nullptr, K, ctx->dy.p,
                 (int)h.output_dtype, nullptr, s, T > kTileTok, nullptr, n_valid);
    if (rc) {
        (void)hipStreamSynchronize(s);
        *resp_len = write_layer_resp(resp, 4, h, 0);
        return CX_OK;
    }
    CX_HIP(hipMemcpyAsync(ctx->pin_y, ctx->dy.p, out_bytes, hipMemcpyDeviceToHost, s));
    int flag = 0;
    CX_HIP(hipMemcpyAsync(&flag, ctx->err_flag, sizeof(int), hipMemcpyDeviceToHost, s));
    CX_HIP(hipStreamSynchronize(s));
    if (flag != 0) {  // a device check failed (e.g. a route listed twice for one token)
        CX_HIP(hipMemsetAsync(ctx->err_flag, 0, sizeof(int), s));
        CX_HIP(hipStreamSynchronize(s));
        *resp_len = write_layer_resp(resp, 4, h, 0);
        return CX_OK;
    }
    std::memcpy(resp + 20, ctx->pin_y, out_bytes);
    *resp_len = write_layer_resp(resp, 0, h, (uint32_t)out_bytes);
    return CX_OK;
}

int cx_gen_fp8_matrix(cx_ctx* ctx, uint64_t seed, uint64_t stream_id, int rows, int cols,
                      int row_block, int col_block, float std_dev, uint8_t* dev_weight,
                      float* dev_scale, void* stream) {
    if (!ctx || !dev_weight || !dev_scale) return fail(CX_EINVAL, "NULL argument");
    if (rows <= 0 || cols <= 0 || row_block <= 0 || col_block <= 0)
        return fail(CX_EINVAL, "bad matrix geometry");
    int rc = set_device(ctx->device);
    if (rc) return rc;
    CX_HIP(launch_gen_fp8(seed, stream_id, rows, cols, row_block, col_block, std_dev, dev_weight,
                          dev_scale, static_cast<hipStream_t>(stream)));
    return CX_OK;
}

int cx_gen_normal(cx_ctx* ctx, uint64_t seed, uint64_t stream_id, uint64_t count, float std_dev,
                  int dtype, void* dev_out, void* stream) {
    if (!ctx || !dev_out) return fail(CX_EINVAL, "NULL argument");
    if (dtype != CX_DTYPE_F32 && !act16(dtype)) return fail(CX_EINVAL, "bad dtype");
    int rc = set_device(ctx->device);
    if (rc) return rc;
    CX_HIP(launch_gen_normal(seed, stream_id, count, std_dev, dtype, dev_out,
                             static_cast<hipStream_t>(stream)));
    return CX_OK;
}

int cx_gen_expert(int device, uint64_t seed, uint64_t stream_base, int hidden, int inter,
                  int block, float std_dev, cx_expert_desc* out) {
    if (!out) return fail(CX_EINVAL, "NULL out");
    std::memset(out, 0, sizeof(*out));
    if (hidden <= 0 || inter <= 0 || block <= 0) return fail(CX_EINVAL, "bad expert geometry");
    int rc = set_device(device);
    if (rc) return rc;
    const size_t nsu = (size_t)((inter + block - 1) / block) * ((hidden + block - 1) / block);
    const size_t nsd = (size_t)((hidden + block - 1) / block) * ((inter + block - 1) / block);
    void* p[6] = {};
    const size_t sz[6] = {(size_t)inter * hidden, nsu * 4, (size_t)inter * hidden, nsu * 4,
                          (size_t)hidden * inter, nsd * 4};
    for (int i = 0; i < 6; ++i) {
        if ((rc = arena_alloc(device, sz[i], &p[i]))) {
            for (int j = 0; j < i; ++j) arena_free(device, p[j], false);
            return rc;
        }
    }
    hipStream_t s = upload_stream(device);
    // up and gate in 16-row tiles when the shape allows (as the node's upload stores them)
    const int gl = gu_tile16_ok(inter, hidden) ? CX_LAYOUT_TILE16 : CX_LAYOUT_ROWS;
    hipError_t e = launch_gen_fp8(seed, stream_base + 0, inter, hidden, block, block, std_dev,
                                  static_cast<uint8_t*>(p[0]), static_cast<float*>(p[1]), s, gl);
    if (e == hipSuccess)
        e = launch_gen_fp8(seed, stream_base + 1, inter, hidden, block, block, std_dev,
                           static_cast<uint8_t*>(p[2]), static_cast<float*>(p[3]), s, gl);
    if (e == hipSuccess)
        e = launch_gen_fp8(seed, stream_base + 2, hidden, inter, block, block, std_dev,
                           static_cast<uint8_t*>(p[4]), static_cast<float*>(p[5]), s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        for (int j = 0; j < 6; ++j) arena_free(device, p[j], false);
        return fail(CX_EHIP, "expert generation failed: %s", hipGetErrorString(e));
    }
    out->w_up = static_cast<uint8_t*>(p[0]);
    out->s_up = static_cast<float*>(p[1]);
    out->w_gate = static_cast<uint8_t*>(p[2]);
    out->s_gate = static_cast<float*>(p[3]);
    out->w_down = static_cast<uint8_t*>(p[4]);
    out->s_down = static_cast<float*>(p[5]);
    out->hidden = hidden;
    out->inter = inter;
    out->up_rb = out->up_cb = out->gate_rb = out->gate_cb = out->down_rb = out->down_cb = block;
    out->gu_layout = gl;
    return CX_OK;
}

int cx_free_expert(int device, cx_expert_desc* e) {
    if (!e) return fail(CX_EINVAL, "NULL expert");
    const void* p[6] = {e->w_up, e->s_up, e->w_gate, e->s_gate, e->w_down, e->s_down};
    int rc = CX_OK;
    for (const void* q : p) {
        if (q) {
            const int r = arena_free(device, const_cast<void*>(q));
            if (r) rc = r;
        }
    }
    std::memset(e, 0, sizeof(*e));
    return rc;
}

}  // extern "C"
