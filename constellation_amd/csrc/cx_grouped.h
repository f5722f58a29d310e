// cx_grouped.h — the grouped fp8 expert MLP for work items of up to 64
// pairs (prefill chunks and large decode batches): gate/up + SiLU and the
// down projection as two MFMA GEMM kernels over (row tile, item).
// Semantics: RunFusedUpGateReferenceV2 / RunDownReferenceV2
// (expert_node_v2/backend/expert_reference_v2.cc:11-144) per expert,
// dequantise-then-fp32, h kept to 16 significant bits (bf16 hi + lo).
//
// Why this shape.  The activations of an item (x rows for gate/up, h rows for
// down) are shared by every weight row of the tile, so they go through LDS.
// For each 128-column k-block, the workgroup's waves each load a share of
// the item's activation block into registers (gate/up: 512 B per wave;
// down: 1 KB per wave and h plane), whole pairs' 256-byte rows or halves
// of them, so that every load instruction reads whole 128-byte lines (a
// share cut along the MFMA fragments instead touched twice to four times
// as many lines and measured 5-8 % slower).  They issue
// it together with that k-block's weights, D k-blocks ahead, in the same
// register ring.  Just before the k-block is used, each lane writes its
// piece where the MFMA fragments read it, in one of two LDS slots, and a
// barrier publishes them.  Every vector load
// in the loop is an ordinary load of the same kind, so the in-order vmcnt
// wait that makes a k-block's weights usable also covers its activations.
// The compiler keeps exact waits across the rolled loop.  Direct
// global->LDS loads would instead mark the counter out of order and drain
// it at every loop header.
//
#pragma once

#include "cx_gate_up.h"

namespace cx {

constexpr int kGrpTiles = 4;                         // 16-pair column tiles per item
constexpr int kGrpPairs = kTileTok * kGrpTiles;      // 64 pairs per item
constexpr size_t kPiece = 1024;                      // one wave load (64 x 16 B)
constexpr size_t kActBlk = 4 * kPiece;               // 16 pairs x 128 k x 16 bit

// gate/up: 8 waves x 16 rows of gate and of up, D-deep register ring; two
// LDS slots of kGrpTiles activation blocks.  Each wave loads two pairs'
// rows (8 B per lane) of every column tile per k-block, so one activation
// block serves 128 weight rows.
constexpr int kGuGrpWaves = 8;
constexpr int kGuGrpRows = kTileRows * kGuGrpWaves;  // 128
constexpr int kGuGrpD = 4;
constexpr size_t grp_gu_lds() { return (size_t)2 * kGrpTiles * kActBlk; }  // 32 KB

// down: 8 waves x 32 rows (two 16-row MFMA tiles sharing each B fragment);
// h enters as two planes (hi, lo), so a slot holds 2 x kGrpTiles blocks.
constexpr int kDnGrpWaves = 8;
constexpr int kDnGrpRows = kDnGrpWaves * 2 * kTileRows;  // 256
constexpr int kDnGrpD = 4;
constexpr size_t grp_dn_lds() { return (size_t)2 * 2 * kGrpTiles * kActBlk; }  // 64 KB

// Barrier after this wave's LDS writes: the writes complete (lgkmcnt), no
// wait on vector memory loads (a release fence on all memory would drain
// the weight ring).
__device__ __forceinline__ void lds_write_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) const u32x2 global_u32x2;
__device__ __forceinline__ u32x2 ld8(const void* p) { return *(global_u32x2*)(p); }

// Scale of k-block k of the lane-distributed scale row `v` (lane l holds
// k-block l).
__device__ __forceinline__ float lane_scale(float v, int k) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
}

// Wait for the stage issued W stages back (W = stages issued after it, each
// of PS loads): a compile-time count for s_waitcnt.
template <int PS>
__device__ __forceinline__ void wait_stages(int later) {
    if (later >= 3) vm_wait<3 * PS>();
    else if (later == 2) vm_wait<2 * PS>();
    else if (later == 1) vm_wait<PS>();
    else vm_wait<0>();
}

// The streaming loop shared by both kernels: a prologue of D stages, then
// NKB steps of [wait for stage k; publish its activations; compute k; issue
// stage k + D].  The steady part runs as a rolled loop of D-step bodies so
// every ring index and LDS slot (k % D, k % 2) is a compile-time constant.
// `issue(k, s)`, `publish(s, slot)` and `compute(k, s, slot)` are the
// kernel's stage actions; `ready()` runs once the first stage has landed.
template <int NKB, int D, int PS, class Issue, class Publish, class Compute, class Ready>
__device__ __forceinline__ void grp_stream(Issue&& issue, Publish&& publish, Compute&& compute,
                                           Ready&& ready) {
    static_assert(D % 2 == 0 || NKB <= D, "LDS slot k % 2 must be fixed per ring stage");
    static_assert((D - 1) * PS < 64, "vmcnt range");
    // the prologue keeps stage order (the loop's waits assume it)
#pragma unroll
    for (int k = 0; k < D && k < NKB; ++k) {
        issue(k, k);
        __builtin_amdgcn_sched_barrier(0);
    }
    // stage 0 and every older load (the kernel's per-tile setup loads) have
    // landed here; `ready` pins those values so that no later wait is
    // computed for them (a loop-carried wait on them would drain the ring)
    if (NKB > D) vm_wait<(D - 1) * PS>();
    else vm_wait<0>();
    ready();
    constexpr int NST = NKB > D ? NKB - D : 0;  // steps that issue a stage
    constexpr int NCH = NST / D;
    int k0 = 0;
#pragma unroll 1
    for (int ch = 0; ch < NCH; ++ch, k0 += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            vm_wait<(D - 1) * PS>();
            publish(i, i & 1);
            lds_write_barrier();
            compute(k0 + i, i, i & 1);
            __builtin_amdgcn_sched_barrier(0);
            issue(k0 + i + D, i);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int i = 0; i < NST % D; ++i) {
        const int k = NCH * D + i;
        __builtin_amdgcn_sched_barrier(0);
        vm_wait<(D - 1) * PS>();
        publish(k % D, k & 1);
        lds_write_barrier();
        compute(k, k % D, k & 1);
        __builtin_amdgcn_sched_barrier(0);
        issue(k + D, k % D);
        __builtin_amdgcn_sched_barrier(0);
    }
    constexpr int NTAIL = NKB < D ? NKB : D;
#pragma unroll
    for (int i = 0; i < NTAIL; ++i) {
        const int k = NST + i;
        // keep each step's conversions below its own wait
        __builtin_amdgcn_sched_barrier(0);
        wait_stages<PS>(NTAIL - 1 - i);
        publish(k % D, k & 1);
        lds_write_barrier();
        compute(k, k % D, k & 1);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// ---------------------------------------------------------------------------
// gate/up.  NKB = hidden / 128 k-blocks (<= 64), NT = 16-pair column tiles
// of this item (1..4, a compile-time branch per item).
template <int NKB, int NT, bool F16, bool SINGLE, int GL>
__device__ __forceinline__ void grp_gate_up_item(const ExpertLaunch& L, const Unit& u, int tile,
                                                 unsigned char* lds) {
    typedef Mma<F16> M;
    typedef typename M::V V;
    // short K (test shapes): a 2-deep ring keeps the steady-state loop a
    // loop (a single-trip loop is flattened and the schedule then spills)
    constexpr int D = NKB >= 12 ? kGuGrpD : 2;
    constexpr int PS = 4 + NT;  // loads per stage per wave
    constexpr size_t SLOT = (size_t)kGrpTiles * kActBlk;
    static_assert(NKB <= 64, "scale row held one k-block per lane");
    const int H = u.e.hidden, I = u.e.inter;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const int r0 = tile * kGuGrpRows + wave * kTileRows;
    constexpr int KW = GL == CX_LAYOUT_TILE16 ? 2048 : kKB;  // weight bytes between k-blocks
    const size_t roff = gu_piece_off(GL, H, r0 + c, 0, g);
    const uint8_t* pg = u.e.w_gate + roff;
    const uint8_t* pu = u.e.w_up + roff;
    const int rbg = __builtin_amdgcn_readfirstlane(r0 / u.e.gate_rb);
    const int rbu = __builtin_amdgcn_readfirstlane(r0 / u.e.up_rb);
    float scg_v = lane < NKB ? ldf(u.e.s_gate + (size_t)rbg * NKB + lane) : 0.f;
    float scu_v = lane < NKB ? ldf(u.e.s_up + (size_t)rbu * NKB + lane) : 0.f;
    // activations of a column tile and k-block: 16 pairs x 128 elements.
    // Wave w loads pairs 2w and 2w + 1 whole (256 B each), so each load
    // instruction reads 4 whole 128-byte lines; lane l takes pair xp,
    // elements xe .. +4, and publishes them where the MFMA fragment of
    // (pair xp, k = 32 g + 8 j) is read from: piece j, lane (g, xp), half.
    // (These writes land 16 lanes on 2-4 LDS bank groups; an XOR swizzle of
    // the slots that spread them measured no faster, so the fragment reads
    // keep their plain lane order.)
    static_assert(kGuGrpWaves * 2 == kTileTok, "two pairs per wave cover a column tile");
    const int xp = 2 * wave + (lane >> 5), xe = 4 * (lane & 31);
    const size_t xdst = (size_t)((xe & 31) >> 3) * kPiece + (size_t)((xe >> 5) * 16 + xp) * 16 + 8 * ((xe & 7) >> 2);
    const uint16_t* xs[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
        const int q = min(tt * kTileTok + xp, u.np - 1);
        const int tok = SINGLE ? u.pb + q : ldi(L.plan.pair_token + u.pb + q);
        xs[tt] = static_cast<const uint16_t*>(L.x) + (size_t)tok * H + xe;
    }
    u32x4 wb[D][4];
    u32x2 xr[D][NT];
    f32x4 accg[NT], accu[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
        accg[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
        accu[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    auto issue = [&](int k, int s) {
        wb[s][0] = ld16(pg + (size_t)k * KW);
        wb[s][1] = ld16(pg + (size_t)k * KW + 16);
        wb[s][2] = ld16(pu + (size_t)k * KW);
        wb[s][3] = ld16(pu + (size_t)k * KW + 16);
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) xr[s][tt] = ld8(xs[tt] + (size_t)k * kKB);
    };
    auto publish = [&](int s, int slot) {
        unsigned char* dst = lds + (size_t)slot * SLOT + xdst;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) *reinterpret_cast<u32x2*>(dst + tt * kActBlk) = xr[s][tt];
    };
    auto compute = [&](int k, int s, int slot) {
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        const float sgk = lane_scale(scg_v, k), suk = lane_scale(scu_v, k);
        V ag[4], au[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            ag[j] = M::cvt(wb[s][j >> 1][(j & 1) * 2], wb[s][j >> 1][(j & 1) * 2 + 1]);
            au[j] = M::cvt(wb[s][2 + (j >> 1)][(j & 1) * 2], wb[s][2 + (j >> 1)][(j & 1) * 2 + 1]);
        }
        const unsigned char* src = lds + (size_t)slot * SLOT + lane * 16;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            V bx[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                bx[j] = M::bits(*reinterpret_cast<const u32x4*>(src + tt * kActBlk + j * kPiece));
            f32x4 tg = M::mma(ag[0], bx[0], zero);
            f32x4 tu = M::mma(au[0], bx[0], zero);
#pragma unroll
            for (int j = 1; j < 4; ++j) {
                tg = M::mma(ag[j], bx[j], tg);
                tu = M::mma(au[j], bx[j], tu);
            }
            accg[tt] += sgk * tg;
            accu[tt] += suk * tu;
        }
    };
    grp_stream<NKB, D, PS>(issue, publish, compute,
                           [&] { asm volatile("" : "+v"(scg_v), "+v"(scu_v)); });
    // epilogue: h = SiLU(gate) * up as bf16 hi + lo (route weight folded in
    // when the caller combines by plain sums)
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
        const int q = tt * kTileTok + c;
        if (q < u.np) {
            const size_t p = (size_t)(u.pb + q);
            const float wf = !SINGLE && L.fold_weight ? L.plan.pair_weight[p] : 1.0f;
            const int row = r0 + 4 * g;
            uint32_t hi[4], lo[4];
            float hv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float gate = accg[tt][i], up = accu[tt][i];
                const float h = (gate / (1.0f + expf(-gate))) * up;
                hv[i] = h;
                const float hw = h * wf;
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

// gate/up of a one-tile item (<= 16 pairs) with the x rows staged in LDS a
// chunk of kGuChunk k-blocks at a time (two chunk buffers): the next chunk is
// loaded into registers while the current one is consumed and published with
// one barrier per chunk, so the k-block steps issue weight loads only.  The
// whole K loop is unrolled (every load is an ordinary register load, so the
// compiler's waits stay exact).  LDS: grp_gu_c1_lds().
constexpr int kGuChunk = 14;
constexpr size_t kGuChunkBytes = (size_t)kGuChunk * kActBlk;  // 56 KB
constexpr size_t grp_gu_c1_lds() { return 2 * kGuChunkBytes; }

template <int NKB, bool F16, bool SINGLE, int GL, int D = kGuGrpD>
__device__ __forceinline__ void grp_gate_up_item_c1(const ExpertLaunch& L, const Unit& u, int tile,
                                                    unsigned char* lds) {
    typedef Mma<F16> M;
    typedef typename M::V V;
    static_assert(NKB % kGuChunk == 0 && NKB <= 64, "whole chunks; scale row one k-block per lane");
    static_assert(kGuGrpWaves == 8, "chunk loader: 512 threads x 7 pieces = 14 k-blocks");
    constexpr int NCH = NKB / kGuChunk, XL = kGuChunk / 2;  // x loads per thread and chunk
    const int H = u.e.hidden, I = u.e.inter;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const int r0 = tile * kGuGrpRows + wave * kTileRows;
    constexpr int KW = GL == CX_LAYOUT_TILE16 ? 2048 : kKB;  // weight bytes between k-blocks
    const size_t roff = gu_piece_off(GL, H, r0 + c, 0, g);
    const uint8_t* pg = u.e.w_gate + roff;
    const uint8_t* pu = u.e.w_up + roff;
    const int rbg = __builtin_amdgcn_readfirstlane(r0 / u.e.gate_rb);
    const int rbu = __builtin_amdgcn_readfirstlane(r0 / u.e.up_rb);
    float scg_v = lane < NKB ? ldf(u.e.s_gate + (size_t)rbg * NKB + lane) : 0.f;
    float scu_v = lane < NKB ? ldf(u.e.s_up + (size_t)rbu * NKB + lane) : 0.f;
    // chunk loader: wave w carries pairs 4 (w % 4) .. +4 whole (256 B each,
    // one 1 KB load instruction = 8 whole 128-byte lines) of k-blocks
    // w / 4 + 2i (i < 7) of the chunk; lane l takes pair xp, elements
    // xe .. +8, published where the MFMA fragment of (pair xp,
    // k = 32 g + 8 j) is read from: piece j, lane (g, xp)
    const int xp = 4 * (wave & 3) + (lane >> 4), xe = 8 * (lane & 15);
    const int q = min(xp, u.np - 1);
    const int tok = SINGLE ? u.pb + q : ldi(L.plan.pair_token + u.pb + q);
    const int kq = wave >> 2;
    const uint16_t* xs = static_cast<const uint16_t*>(L.x) + (size_t)tok * H + xe;
    unsigned char* xdst = lds + (size_t)((xe & 31) >> 3) * kPiece + (size_t)((xe >> 5) * 16 + xp) * 16;
    u32x4 xr[XL];
    // chunk loads from a base advanced per chunk (kept opaque so the offsets
    // stay immediates instead of one precomputed address per load)
    const uint16_t* xb = xs + (size_t)kq * kKB;
    auto load_chunk = [&](int ch) {
        if (ch > 0) {
            xb += (size_t)kGuChunk * kKB;
            asm volatile("" : "+v"(xb));
        }
#pragma unroll
        for (int i = 0; i < XL; ++i) xr[i] = ld16(xb + (size_t)(2 * i) * kKB);
    };
    auto store_chunk = [&](int ch) {
        unsigned char* dst = xdst + (size_t)(ch & 1) * kGuChunkBytes;
#pragma unroll
        for (int i = 0; i < XL; ++i) *reinterpret_cast<u32x4*>(dst + (size_t)(kq + 2 * i) * kActBlk) = xr[i];
    };
    u32x4 wb[D][4];
    // weight loads relative to the current chunk's base (kb = first k-block)
    const uint8_t* pgb = pg;
    const uint8_t* pub = pu;
    auto issue = [&](int k, int kb) {
        const int st = k % D;
        const size_t o = (size_t)(k - kb) * KW;
        wb[st][0] = ld16(pgb + o);
        wb[st][1] = ld16(pgb + o + 16);
        wb[st][2] = ld16(pub + o);
        wb[st][3] = ld16(pub + o + 16);
    };
    // chunk 0 first, then the weight prologue, then chunk 0 into LDS and
    // chunk 1 behind the weights
    load_chunk(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < D && k < NKB; ++k) {
        issue(k, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
    store_chunk(0);
    if (NCH > 1) load_chunk(1);
    asm volatile("" : "+v"(scg_v), "+v"(scu_v));
    lds_write_barrier();
    __builtin_amdgcn_sched_barrier(0);
    f32x4 accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        const unsigned char* src = lds + (size_t)(ch & 1) * kGuChunkBytes + lane * 16;
        if (ch > 0) {
            pgb += (size_t)kGuChunk * KW;
            pub += (size_t)kGuChunk * KW;
            asm volatile("" : "+v"(pgb), "+v"(pub));
        }
#pragma unroll
        for (int kk = 0; kk < kGuChunk; ++kk) {
            const int k = ch * kGuChunk + kk, st = k % D;
            const float sgk = lane_scale(scg_v, k), suk = lane_scale(scu_v, k);
            V ag[4], au[4], bx[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                ag[j] = M::cvt(wb[st][j >> 1][(j & 1) * 2], wb[st][j >> 1][(j & 1) * 2 + 1]);
                au[j] = M::cvt(wb[st][2 + (j >> 1)][(j & 1) * 2], wb[st][2 + (j >> 1)][(j & 1) * 2 + 1]);
                bx[j] = M::bits(*reinterpret_cast<const u32x4*>(src + (size_t)kk * kActBlk + j * kPiece));
            }
            f32x4 tg = M::mma(ag[0], bx[0], zero);
            f32x4 tu = M::mma(au[0], bx[0], zero);
#pragma unroll
            for (int j = 1; j < 4; ++j) {
                tg = M::mma(ag[j], bx[j], tg);
                tu = M::mma(au[j], bx[j], tu);
            }
            accg += sgk * tg;
            accu += suk * tu;
            // keep the scaled accumulate at this step (left free, the
            // compiler defers it and holds every step's product)
            asm volatile("" : "+v"(accg), "+v"(accu));
            __builtin_amdgcn_sched_barrier(0);
            if (k + D < NKB) issue(k + D, ch * kGuChunk);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (ch + 1 < NCH) {
            // chunk ch + 1 into the buffer chunk ch - 1 used (every wave has
            // passed the barrier after its last read), chunk ch + 2 behind
            store_chunk(ch + 1);
            if (ch + 2 < NCH) load_chunk(ch + 2);
            lds_write_barrier();
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (c < u.np) {
        const size_t p = (size_t)(u.pb + c);
        const float wf = !SINGLE && L.fold_weight ? L.plan.pair_weight[p] : 1.0f;
        const int row = r0 + 4 * g;
        uint32_t hi[4], lo[4];
        float hv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float gate = accg[i], up = accu[i];
            const float h = (gate / (1.0f + expf(-gate))) * up;
            hv[i] = h;
            const float hw = h * wf;
            hi[i] = bf16_rne(hw);
            lo[i] = bf16_rne(hw - __uint_as_float(hi[i] << 16));
        }
        *reinterpret_cast<uint2*>(L.h_hi + p * I + row) = uint2{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
        *reinterpret_cast<uint2*>(L.h_lo + p * I + row) = uint2{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
        if (L.h_f32 != nullptr)
            *reinterpret_cast<float4*>(L.h_f32 + p * I + row) = float4{hv[0], hv[1], hv[2], hv[3]};
    }
}

// C1: one-tile items take the chunked path (needs grp_gu_c1_lds() of LDS).
template <int NKB, bool F16, bool SINGLE, bool C1, int GL>
__device__ __forceinline__ void grp_gate_up_unit(const ExpertLaunch& L, const Unit& u, int tile,
                                                 unsigned char* lds) {
    const int nt = (u.np + kTileTok - 1) / kTileTok;  // uniform: one branch per item
    if constexpr (C1) {
        if (nt == 1) {
            grp_gate_up_item_c1<NKB, F16, SINGLE, GL>(L, u, tile, lds);
            return;
        }
    }
    if (nt == 1) grp_gate_up_item<NKB, 1, F16, SINGLE, GL>(L, u, tile, lds);
    else if (nt == 2) grp_gate_up_item<NKB, 2, F16, SINGLE, GL>(L, u, tile, lds);
    else if (nt == 3) grp_gate_up_item<NKB, 3, F16, SINGLE, GL>(L, u, tile, lds);
    else grp_gate_up_item<NKB, 4, F16, SINGLE, GL>(L, u, tile, lds);
}

template <int NKB, bool F16, bool SINGLE, bool C1 = false>
__device__ __forceinline__ void grp_gate_up_tile(const ExpertLaunch& L, int tile, int item,
                                                 unsigned char* lds) {
    Unit u;
    if (!resolve_unit<SINGLE>(L, item, kGrpPairs, &u)) return;
    if (u.e.gu_layout == CX_LAYOUT_TILE16) grp_gate_up_unit<NKB, F16, SINGLE, C1, CX_LAYOUT_TILE16>(L, u, tile, lds);
    else grp_gate_up_unit<NKB, F16, SINGLE, C1, CX_LAYOUT_ROWS>(L, u, tile, lds);
}

// ---------------------------------------------------------------------------
// down.  NKB = inter / 128 k-blocks (<= 64).  Each wave owns 32 rows of Wd
// (two MFMA row tiles) and reads each h fragment once for both.
template <int NKB, int NT, bool SINGLE>
__device__ __forceinline__ void grp_down_item(const ExpertLaunch& L, const Unit& u, int tile,
                                              unsigned char* lds) {
    typedef Mma<false> M;
    typedef M::V V;
    constexpr int D = NKB >= 8 ? kDnGrpD : 2;
    constexpr int PS = 4 + NT;
    constexpr size_t PLANE = (size_t)kGrpTiles * kActBlk;
    constexpr size_t SLOT = 2 * PLANE;
    static_assert(NKB <= 64, "scale row held one k-block per lane");
    const int H = u.e.hidden, I = u.e.inter;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const int rw = tile * kDnGrpRows + wave * (2 * kTileRows);
    const uint8_t* pd = u.e.w_down + (size_t)(rw + c) * I + g * 32;
    const size_t pd1 = (size_t)kTileRows * I;  // second row tile
    const int rb0 = __builtin_amdgcn_readfirstlane(rw / u.e.down_rb);
    const int rb1 = __builtin_amdgcn_readfirstlane((rw + kTileRows) / u.e.down_rb);
    float sd0_v = lane < NKB ? ldf(u.e.s_down + (size_t)rb0 * NKB + lane) : 0.f;
    float sd1_v = lane < NKB ? ldf(u.e.s_down + (size_t)rb1 * NKB + lane) : 0.f;
    // h of a column tile and k-block: 16 pairs x 128 elements per plane.
    // Wave w loads plane w / 4 (hi, lo), quarter j = w % 4: pairs
    // 8 (j >> 1) .. +8, elements 64 (j & 1) .. +64 of each, so each load
    // instruction reads 8 whole 128-byte lines; lane l takes pair hp,
    // elements hk0 .. +8, and publishes them where the MFMA fragment of
    // (pair hp, k = 32 g + 8 j) is read from: piece (hk0 % 32) / 8, lane
    // (hk0 / 32, hp).
    static_assert(kDnGrpWaves == 8, "h loader: 2 planes x 4 quarters of 8 pairs x 64 elements");
    const int plane = wave >> 2, pj = wave & 3;
    const int hp = 8 * (pj >> 1) + (lane >> 3);
    const int hk0 = 64 * (pj & 1) + 8 * (lane & 7);
    const size_t hdst = (size_t)plane * PLANE + (size_t)((hk0 & 31) >> 3) * kPiece +
                        (size_t)((hk0 >> 5) * 16 + hp) * 16;
    const uint16_t* hs[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
        const int q = min(tt * kTileTok + hp, u.np - 1);
        hs[tt] = (plane ? L.h_lo : L.h_hi) + (size_t)(u.pb + q) * I + hk0;
    }
    u32x4 wb[D][4];
    u32x4 hr[D][NT];
    f32x4 acc[2][NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
        acc[0][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc[1][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    auto issue = [&](int k, int s) {
        wb[s][0] = ld16(pd + (size_t)k * kKB);
        wb[s][1] = ld16(pd + (size_t)k * kKB + 16);
        wb[s][2] = ld16(pd + pd1 + (size_t)k * kKB);
        wb[s][3] = ld16(pd + pd1 + (size_t)k * kKB + 16);
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) hr[s][tt] = ld16(hs[tt] + (size_t)k * kKB);
    };
    auto publish = [&](int s, int slot) {
        unsigned char* dst = lds + (size_t)slot * SLOT + hdst;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) *reinterpret_cast<u32x4*>(dst + tt * kActBlk) = hr[s][tt];
    };
    auto compute = [&](int k, int s, int slot) {
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        const float s0 = lane_scale(sd0_v, k), s1 = lane_scale(sd1_v, k);
        V a0[4], a1[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a0[j] = M::cvt(wb[s][j >> 1][(j & 1) * 2], wb[s][j >> 1][(j & 1) * 2 + 1]);
            a1[j] = M::cvt(wb[s][2 + (j >> 1)][(j & 1) * 2], wb[s][2 + (j >> 1)][(j & 1) * 2 + 1]);
        }
        const unsigned char* src = lds + (size_t)slot * SLOT + lane * 16;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            V bh[4], bl[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                bh[j] = M::bits(*reinterpret_cast<const u32x4*>(src + tt * kActBlk + j * kPiece));
                bl[j] = M::bits(*reinterpret_cast<const u32x4*>(src + PLANE + tt * kActBlk + j * kPiece));
            }
            f32x4 t0 = M::mma(a0[0], bh[0], zero);
            f32x4 t1 = M::mma(a1[0], bh[0], zero);
            t0 = M::mma(a0[0], bl[0], t0);
            t1 = M::mma(a1[0], bl[0], t1);
#pragma unroll
            for (int j = 1; j < 4; ++j) {
                t0 = M::mma(a0[j], bh[j], t0);
                t1 = M::mma(a1[j], bh[j], t1);
                t0 = M::mma(a0[j], bl[j], t0);
                t1 = M::mma(a1[j], bl[j], t1);
            }
            acc[0][tt] += s0 * t0;
            acc[1][tt] += s1 * t1;
        }
    };
    grp_stream<NKB, D, PS>(issue, publish, compute,
                           [&] { asm volatile("" : "+v"(sd0_v), "+v"(sd1_v)); });
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        const int row = rw + a * kTileRows + 4 * g;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            const int q = tt * kTileTok + c;
            if (q < u.np) {
                const size_t p = (size_t)(u.pb + q);
                const f32x4 v = acc[a][tt];
                // y_part is read once, by the combine launch: streamed stores
                if (SINGLE) store_out4(L.y, L.y_f32, p * H + row, v, L.out_dtype);
                else __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(L.y_part + p * H + row));
            }
        }
    }
}

template <int NKB, bool SINGLE>
__device__ __forceinline__ void grp_down_tile(const ExpertLaunch& L, int tile, int item,
                                              unsigned char* lds) {
    Unit u;
    if (!resolve_unit<SINGLE>(L, item, kGrpPairs, &u)) return;
    const int nt = (u.np + kTileTok - 1) / kTileTok;
    if (nt == 1) grp_down_item<NKB, 1, SINGLE>(L, u, tile, lds);
    else if (nt == 2) grp_down_item<NKB, 2, SINGLE>(L, u, tile, lds);
    else if (nt == 3) grp_down_item<NKB, 3, SINGLE>(L, u, tile, lds);
    else grp_down_item<NKB, 4, SINGLE>(L, u, tile, lds);
}

}  // namespace cx
