// Grouped GEMM for prefill items of up to 128 pairs, for calls with many
// tokens per expert.  There an expert's weights are reused by hundreds of
// token columns, so the MFMA rather than HBM bounds the work, and the
// register-streamed kernels of cx_grouped.h (weights read once per <= 64-pair
// item, x published per k-block) would re-read each expert's weights for
// every 64 pairs.  Here both operands go through an LDS ring:
//
//  * gate/up: workgroup = 128 inter rows of gate and of up x 128 pairs; a
//    stage is 64 k (half a 128-column scale block): 2 x 128 rows x 64 B of
//    fp8 weights and 128 pairs x 64 bf16/fp16 of x, 32 KB, four stages.
//  * down: workgroup = 256 hidden rows x 128 pairs; a stage is 256 rows x
//    64 B of fp8 weights and 128 pairs x 64 of h's hi and lo planes, 48 KB,
//    three stages.
//
// Operands are DMA'd global->LDS (16 B per lane) into XOR-swizzled rows so
// the fragment reads are free of bank conflicts; each stage buffer is its
// own LDS array, so the compiler's waits for the DMA stay per stage.  Waves:
// 4 row groups x 2 pair halves.  fp8 weights are converted exactly to
// bf16/fp16 for v_mfma_f32_16x16x32; each 128-column block's MFMA sums are
// kept apart and added into the accumulators scaled by that block's scale
// (RunDownReferenceV2 / RunExpertReferenceV2's dequantise-then-fp32 order
// per block, expert_reference_v2.cc:92-144).
#pragma once

#include "cx_gate_up.h"
#include "cx_grouped.h"

namespace cx {

constexpr int kBigGuRows = 128;  // inter rows (of gate and of up) per gate/up workgroup
constexpr int kBigDnRows = 256;  // hidden rows per down workgroup
constexpr int kBigK = 64;        // k per LDS stage
constexpr int kBigGuRing = 4;
constexpr int kBigDnRing = 3;
constexpr int kBigGuA = 2 * kBigGuRows * kBigK;  // 16 KB of weights per stage
constexpr int kBigGuB = kBigPairs * kBigK * 2;   // 16 KB of x per stage
constexpr int kBigDnA = kBigDnRows * kBigK;      // 16 KB of weights per stage
constexpr int kBigDnB = kBigPairs * kBigK * 2;   // 16 KB per h plane per stage

// Workgroup b runs on XCD b % 8 (round-robin dispatch).  Logical tile
// x * per + b / 8 runs on XCD x, per = ceil(n / 8) over the n tiles that
// exist, so every XCD takes one contiguous run: the row tiles of an item
// (sharing its x rows in that XCD's L2), then the expert's next item
// (sharing the weights).  -1 past the end.
__device__ __forceinline__ int big_tile(int n) {
    const int per = (n + 7) >> 3;
    const int b = blockIdx.x;
    const int t = (b & 7) * per + (b >> 3);
    return ((b >> 3) < per && t < n) ? t : -1;
}

// Logical tile -> (item, row tile): groups of kBigGroup consecutive items
// (an expert's items are consecutive in the plan) walk their row tiles
// together, so the workgroups that share a row tile's weights run side by
// side on one XCD and its L2 serves them one fetch.  false past the items.
constexpr int kBigGroup = 4;
__device__ __forceinline__ bool big_item_tile(int t, int n_items, int n_rt, int* item, int* tile) {
    const int span = kBigGroup * n_rt;
    const int g = t / span, r = t - g * span;
    const int in_group = min(kBigGroup, n_items - g * kBigGroup);
    *tile = r / in_group;
    *item = g * kBigGroup + (r - *tile * in_group);
    return *tile < n_rt;
}

// Fragment reads from the LDS ring.  As plain loads the compiler cannot tell
// which stage a pending global->LDS DMA writes and waits for all of them
// (vmcnt(0)) before reading any stage, draining the ring; as asm it inserts
// no wait, and big_lds_wait() waits for the reads (lgkmcnt(0)) with the
// fragments as operands, so no use of them moves above it.
__device__ __forceinline__ uint32_t big_lds_addr(const unsigned char* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)p;
}
// base + OFF through the instruction's offset field, so one base register
// serves every fragment of a stage
template <int OFF>
__device__ __forceinline__ u32x4 big_lds_read(uint32_t base) {
    static_assert(OFF >= 0 && OFF < 65536 && OFF % 16 == 0, "ds_read offset field");
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(base), "i"(OFF));
    return v;
}
template <int OFF, int STRIDE>
__device__ __forceinline__ void big_lds_read4(uint32_t base, u32x4 (&v)[4]) {
    v[0] = big_lds_read<OFF>(base);
    v[1] = big_lds_read<OFF + STRIDE>(base);
    v[2] = big_lds_read<OFF + 2 * STRIDE>(base);
    v[3] = big_lds_read<OFF + 3 * STRIDE>(base);
}
__device__ __forceinline__ void big_lds_wait(u32x4 (&a)[4], u32x4 (&b)[4]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]));
}
template <int N>
__device__ __forceinline__ void big_lds_wait(u32x4 (&v)[N]) {
    static_assert(N == 4 || N == 8, "fragment batch");
    if constexpr (N == 4)
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
    else
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]));
}

// The LDS ring: NS stages of LPS DMA loads per wave, RING buffers, stage s
// issued RING - 1 stages ahead into the buffer stage s - 1 used (free once
// every wave has passed stage s's barrier).  issue(stage, slot) and
// compute(stage, slot, half) get the buffer and the half of the 128-column
// block as compile-time values: the main loop runs whole turns of PER stages
// (a multiple of both RING and 2), the last turn is unrolled on its own.
template <int NS, int RING, int LPS, class Issue, class Compute>
__device__ __forceinline__ void big_ring(Issue& issue, Compute& compute) {
    constexpr int PER = RING % 2 == 0 ? RING : 2 * RING;
    // the main loop: whole turns of stages that all issue a later stage and
    // wait with RING - 2 stages in flight (no branch in its body)
    constexpr int NMAIN = NS >= RING ? (NS - RING + 1) / PER * PER : 0;
    static_assert(NS >= RING - 1 && RING >= 2 && RING <= 4, "ring shape");
#pragma unroll
    for (int s = 0; s < RING - 1; ++s) issue(s, s % RING);
    auto step = [&](int s, int i, int later, bool more) {
        // stage s has landed once only the later stages' loads are in flight
        if (later >= 2) vm_wait<2 * LPS>();
        else if (later == 1) vm_wait<LPS>();
        else vm_wait<0>();
        lds_dma_barrier();  // every wave's part of stage s; stage s - 1 consumed
        __builtin_amdgcn_sched_barrier(0);
        if (more) issue(s + RING - 1, (i + RING - 1) % RING);
        __builtin_amdgcn_sched_barrier(0);
        compute(s, i % RING, i & 1);
    };
    for (int s0 = 0; s0 < NMAIN; s0 += PER) {
#pragma unroll
        for (int i = 0; i < PER; ++i) step(s0 + i, i, RING - 2, true);
    }
#pragma unroll
    for (int i = 0; i < NS - NMAIN; ++i) {
        const int s = NMAIN + i;
        step(s, i, min(RING - 2, NS - 1 - s), s + RING - 1 < NS);
    }
}

// LDS row layouts (16-byte chunks XOR-swizzled by row; both keys measured
// free of bank conflicts for these fragment reads with SQ_LDS_BANK_CONFLICT,
// where plain rows cost 4-12 conflict cycles per ds_read_b128):
//  * weight rows of 64 B: chunk q of row r at chunk q ^ ((r >> 1) & 3);
//  * activation rows of 128 B (64 values): chunk q of row t at
//    q ^ (t & 7) ^ ((t >> 3) & 1).
// MFMA step j (0, 1) of a stage covers, in lane group g = lane / 16, the 8
// k values 16 g + 8 j ..: weight chunk g holds both steps' bytes, activation
// chunks 2 g + j.

// ---------------------------------------------------------------------------
// gate/up
template <int NKB, bool F16>
__device__ __forceinline__ void big_gate_up(const ExpertLaunch& L, unsigned char* const (&st)[kBigGuRing]) {
    typedef Mma<F16> M;
    typedef typename M::V V;
    constexpr int NS = 2 * NKB;  // stages
    static_assert(NKB <= 64 && NS >= kBigGuRing, "scale row one k-block per lane");
    const PlanHdr hd = ld_uniform(L.plan.hdr);
    const int n_items = L.skip_shared ? hd.n_routed_items : hd.n_items;
    const int n_rt = L.inter / kBigGuRows;
    const int t = big_tile(n_items * n_rt);
    if (t < 0) return;
    int item, tile;
    if (!big_item_tile(t, n_items, n_rt, &item, &tile)) return;
    Unit u;
    if (!resolve_unit<false>(L, item, kBigPairs, &u)) return;
    const int H = u.e.hidden, I = u.e.inter;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const int wr = wave & 3, wp = wave >> 2;  // 32-row group, 64-pair half
    const int r0 = tile * kBigGuRows;
    // DMA sources.  Weights: instruction i = 2 wave + m fills LDS rows
    // 16 i .. 16 i + 15 (gate rows 0..127, then up), lane -> row 16 i + lane / 4.
    const int gl = __builtin_amdgcn_readfirstlane(u.e.gu_layout);
    const uint8_t* asrc[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const int r = 16 * (2 * wave + m) + (lane >> 2);
        const int q = (lane & 3) ^ ((r >> 1) & 3);
        asrc[m] = (r < kBigGuRows ? u.e.w_gate : u.e.w_up) + gu_elem_off(gl, H, r0 + (r & (kBigGuRows - 1)), 16 * q);
    }
    // stage s (64 columns): s * 64 bytes row-major; in 16-row tiles, the
    // lower or upper half (quarters 0-1 or 2-3) of k-block s / 2
    auto a_stage = [&](int s) -> size_t {
        return gl == CX_LAYOUT_TILE16 ? (size_t)(s >> 1) * 2048 + (size_t)(s & 1) * 1024 : (size_t)s * kBigK;
    };
    // x: instruction i = 2 wave + m fills pairs 8 i .. 8 i + 7, lane -> pair
    // 8 i + lane / 8 (pairs past the item repeat its last row; not stored).
    const uint16_t* bsrc[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const int tp = 8 * (2 * wave + m) + (lane >> 3);
        const int q = (lane & 7) ^ (tp & 7) ^ ((tp >> 3) & 1);
        const int tok = ldi(L.plan.pair_token + u.pb + min(tp, u.np - 1));
        bsrc[m] = static_cast<const uint16_t*>(L.x) + (size_t)tok * H + 8 * q;
    }
    // scales: one lane per k-block, per 16-row tile of this wave
    float scg[2], scu[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const int row = r0 + wr * 32 + rt * 16;
        const int rbg = __builtin_amdgcn_readfirstlane(row / u.e.gate_rb);
        const int rbu = __builtin_amdgcn_readfirstlane(row / u.e.up_rb);
        scg[rt] = lane < NKB ? ldf(u.e.s_gate + (size_t)rbg * NKB + lane) : 0.f;
        scu[rt] = lane < NKB ? ldf(u.e.s_up + (size_t)rbu * NKB + lane) : 0.f;
    }
    auto issue = [&](int s, int slot) {
        unsigned char* sb = st[slot];
#pragma unroll
        for (int m = 0; m < 2; ++m)
            __builtin_amdgcn_global_load_lds(asrc[m] + a_stage(s), sb + (2 * wave + m) * 1024, 16, 0, 0);
#pragma unroll
        for (int m = 0; m < 2; ++m)
            __builtin_amdgcn_global_load_lds(bsrc[m] + (size_t)s * kBigK, sb + kBigGuA + (2 * wave + m) * 1024, 16, 0, 0);
    };
    const int aoff = c * kBigK + 16 * (g ^ ((c >> 1) & 3));
    int boff[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) boff[j] = c * 128 + 16 * ((2 * g + j) ^ (c & 7) ^ ((c >> 3) & 1));
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc[2][2][4], part[2][2][4];  // [gate/up][row tile][pair tile]
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) acc[m][rt][tt] = zero;
    // one stage: h = 0 first half of a k-block (fresh partial sums), 1 the
    // second (then scaled into the accumulators)
    auto compute = [&](int s, int slot, int h) {
        const uint32_t sb = big_lds_addr(st[slot]);
        u32x4 aw[4];  // [gate/up x row tile]: rows m * 128 + wr * 32 + rt * 16
        const uint32_t ab = sb + wr * 32 * kBigK + aoff;
        aw[0] = big_lds_read<0>(ab);
        aw[1] = big_lds_read<16 * kBigK>(ab);
        aw[2] = big_lds_read<kBigGuRows * kBigK>(ab);
        aw[3] = big_lds_read<(kBigGuRows + 16) * kBigK>(ab);
        u32x4 br[2][4];  // [step][pair tile]: pairs wp * 64 + tt * 16
        big_lds_read4<0, 16 * 128>(sb + kBigGuA + wp * 64 * 128 + boff[0], br[0]);
        big_lds_wait(aw, br[0]);
        // the second step's x fragments load under the first step's MFMAs
        big_lds_read4<0, 16 * 128>(sb + kBigGuA + wp * 64 * 128 + boff[1], br[1]);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            if (j == 1) big_lds_wait(br[1]);
            V bx[4];
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) bx[tt] = M::bits(br[j][tt]);
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const V a = M::cvt(aw[2 * m + rt][2 * j], aw[2 * m + rt][2 * j + 1]);
#pragma unroll
                    for (int tt = 0; tt < 4; ++tt)
                        part[m][rt][tt] = M::mma(a, bx[tt], (h == 0 && j == 0) ? zero : part[m][rt][tt]);
                }
        }
        if (h == 1) {
            const int kb = s >> 1;
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const float sg = lane_scale(scg[rt], kb), su = lane_scale(scu[rt], kb);
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {
                    acc[0][rt][tt] += sg * part[0][rt][tt];
                    acc[1][rt][tt] += su * part[1][rt][tt];
                    // keep the scaled add here: left free, the compiler
                    // defers it and holds two blocks' partial sums
                    asm volatile("" : "+v"(acc[0][rt][tt]), "+v"(acc[1][rt][tt]));
                }
            }
        }
    };
    big_ring<NS, kBigGuRing, 4>(issue, compute);
    // SiLU(gate) * up -> h as bf16 hi + lo, per pair
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        const int q = wp * 64 + tt * 16 + c;
        if (q >= u.np) continue;
        const size_t p = (size_t)(u.pb + q);
        const float wf = L.fold_weight ? L.plan.pair_weight[p] : 1.0f;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int row = r0 + wr * 32 + rt * 16 + 4 * g;
            uint32_t hi[4], lo[4];
            float hv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float gate = acc[0][rt][tt][i], up = acc[1][rt][tt][i];
                const float hh = (gate / (1.0f + expf(-gate))) * up;
                hv[i] = hh;
                const float hw = hh * wf;
                hi[i] = bf16_rne(hw);
                lo[i] = bf16_rne(hw - __uint_as_float(hi[i] << 16));
            }
            *reinterpret_cast<uint2*>(L.h_hi + p * I + row) = uint2{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
            *reinterpret_cast<uint2*>(L.h_lo + p * I + row) = uint2{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
            if (L.h_f32 != nullptr)
                *reinterpret_cast<float4*>(L.h_f32 + p * I + row) = float4{hv[0], hv[1], hv[2], hv[3]};
        }
    }
}

// ---------------------------------------------------------------------------
// down: y_part[pair] = Wd . h, h as hi + lo planes (both MFMA'd against the
// same converted weights)
template <int NKB>
__device__ __forceinline__ void big_down(const ExpertLaunch& L, unsigned char* const (&st)[kBigDnRing]) {
    typedef Mma<false> M;
    typedef M::V V;
    constexpr int NS = 2 * NKB;
    static_assert(NKB <= 64 && NS >= kBigDnRing, "scale row one k-block per lane");
    const PlanHdr hd = ld_uniform(L.plan.hdr);
    const int n_items = L.skip_shared ? hd.n_routed_items : hd.n_items;
    const int n_rt = L.hidden / kBigDnRows;
    const int t = big_tile(n_items * n_rt);
    if (t < 0) return;
    int item, tile;
    if (!big_item_tile(t, n_items, n_rt, &item, &tile)) return;
    Unit u;
    if (!resolve_unit<false>(L, item, kBigPairs, &u)) return;
    const int H = u.e.hidden, I = u.e.inter;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const int wr = wave & 3, wp = wave >> 2;  // 64-row group, 64-pair half
    const int r0 = tile * kBigDnRows;
    const uint8_t* asrc[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const int r = 16 * (2 * wave + m) + (lane >> 2);
        const int q = (lane & 3) ^ ((r >> 1) & 3);
        asrc[m] = u.e.w_down + (size_t)(r0 + r) * I + 16 * q;
    }
    // h: instruction i = 4 wave + m (0..31): plane i / 16, pairs 8 (i % 16) ..
    const uint16_t* bsrc[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int i = 4 * wave + m;
        const int tp = 8 * (i & 15) + (lane >> 3);
        const int q = (lane & 7) ^ (tp & 7) ^ ((tp >> 3) & 1);
        bsrc[m] = ((i >> 4) ? L.h_lo : L.h_hi) + (size_t)(u.pb + min(tp, u.np - 1)) * I + 8 * q;
    }
    float scd[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
        const int rb = __builtin_amdgcn_readfirstlane((r0 + wr * 64 + rt * 16) / u.e.down_rb);
        scd[rt] = lane < NKB ? ldf(u.e.s_down + (size_t)rb * NKB + lane) : 0.f;
    }
    auto issue = [&](int s, int slot) {
        unsigned char* sb = st[slot];
#pragma unroll
        for (int m = 0; m < 2; ++m)
            __builtin_amdgcn_global_load_lds(asrc[m] + (size_t)s * kBigK, sb + (2 * wave + m) * 1024, 16, 0, 0);
#pragma unroll
        for (int m = 0; m < 4; ++m)
            __builtin_amdgcn_global_load_lds(bsrc[m] + (size_t)s * kBigK, sb + kBigDnA + (4 * wave + m) * 1024, 16, 0, 0);
    };
    const int aoff = c * kBigK + 16 * (g ^ ((c >> 1) & 3));
    int boff[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) boff[j] = c * 128 + 16 * ((2 * g + j) ^ (c & 7) ^ ((c >> 3) & 1));
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc[4][4], part[4][4];  // [row tile][pair tile]
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc[rt][tt] = zero;
    auto compute = [&](int s, int slot, int h) {
        const uint32_t sb = big_lds_addr(st[slot]);
        u32x4 aw[4];  // rows wr * 64 + rt * 16
        big_lds_read4<0, 16 * kBigK>(sb + wr * 64 * kBigK + aoff, aw);
        // four batches of x fragments: (step j, plane pl) = (0,hi) (0,lo)
        // (1,hi) (1,lo), each loading under the previous batch's MFMAs
        const uint32_t bb[2] = {sb + kBigDnA + wp * 64 * 128 + boff[0], sb + kBigDnA + wp * 64 * 128 + boff[1]};
        u32x4 br[2][4];
        big_lds_read4<0, 16 * 128>(bb[0], br[0]);
        big_lds_wait(aw, br[0]);
        V a[4];
#pragma unroll
        for (int bt = 0; bt < 4; ++bt) {
            const int j = bt >> 1;
            __builtin_amdgcn_sched_barrier(0);
            if (bt + 1 < 4) {
                const int jn = (bt + 1) >> 1;
                if (((bt + 1) & 1) == 0) big_lds_read4<0, 16 * 128>(bb[jn], br[(bt + 1) & 1]);
                else big_lds_read4<kBigDnB, 16 * 128>(bb[jn], br[(bt + 1) & 1]);
            }
            if ((bt & 1) == 0) {
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) a[rt] = M::cvt(aw[rt][2 * j], aw[rt][2 * j + 1]);
            }
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
#pragma unroll
                for (int tt = 0; tt < 4; ++tt)
                    part[rt][tt] = M::mma(a[rt], M::bits(br[bt & 1][tt]), (h == 0 && bt == 0) ? zero : part[rt][tt]);
            __builtin_amdgcn_sched_barrier(0);
            if (bt + 1 < 4) big_lds_wait(br[(bt + 1) & 1]);
        }
        if (h == 1) {
            const int kb = s >> 1;
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const float sd = lane_scale(scd[rt], kb);
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {
                    acc[rt][tt] += sd * part[rt][tt];
                    asm volatile("" : "+v"(acc[rt][tt]));
                }
            }
        }
    };
    big_ring<NS, kBigDnRing, 6>(issue, compute);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        const int q = wp * 64 + tt * 16 + c;
        if (q >= u.np) continue;
        const size_t p = (size_t)(u.pb + q);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            const int row = r0 + wr * 64 + rt * 16 + 4 * g;
            const f32x4 v = acc[rt][tt];
            *reinterpret_cast<float4*>(L.y_part + p * H + row) = float4{v[0], v[1], v[2], v[3]};
        }
    }
}

}  // namespace cx
