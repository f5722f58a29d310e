// cx_device.h — device-side helpers shared by the gfx950 kernels: fp8
// conversion, MFMA wrappers, typed global / buffer loads, rounding, DPP moves.
#pragma once

#include "cx_internal.h"

namespace cx {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 8 fp8-e4m3 bytes (two dwords) -> 8 bf16 / fp16, exact (e4m3 fits both).
__device__ __forceinline__ bf16x8 cvt8_bf16(uint32_t w0, uint32_t w1) {
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ __forceinline__ f16x8 cvt8_f16(uint32_t w0, uint32_t w1) {
    const f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false);
    const f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true);
    const f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false);
    const f16x2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true);
    return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// v_mfma_f32_16x16x32_{bf16,f16}: A = 16 weight rows x 32 k, B = 32 k x 16
// columns (tokens or pairs), fp32 accumulate.
template <bool F16>
struct Mma;

template <>
struct Mma<false> {
    typedef bf16x8 V;
    static __device__ __forceinline__ V cvt(uint32_t a, uint32_t b) { return cvt8_bf16(a, b); }
    static __device__ __forceinline__ V bits(u32x4 v) { return __builtin_bit_cast(V, v); }
    static __device__ __forceinline__ f32x4 mma(V a, V b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mma<true> {
    typedef f16x8 V;
    static __device__ __forceinline__ V cvt(uint32_t a, uint32_t b) { return cvt8_f16(a, b); }
    static __device__ __forceinline__ V bits(u32x4 v) { return __builtin_bit_cast(V, v); }
    static __device__ __forceinline__ f32x4 mma(V a, V b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

// 16-byte load from global memory.  The explicit global address space keeps
// the compiler from emitting FLAT loads (which also count against lgkmcnt,
// so any LDS access would drain the whole weight-prefetch ring).
typedef __attribute__((address_space(1))) const u32x4 global_u32x4;
__device__ __forceinline__ u32x4 ld16(const void* p) { return *(global_u32x4*)(p); }

__device__ __forceinline__ float ldf(const float* p) {
    return *(__attribute__((address_space(1))) const float*)(p);
}

// Load through the constant address space: with a wave-uniform address the
// compiler emits a scalar load (s_load) into an SGPR.  Read-only data only.
__device__ __forceinline__ float ldsc(const float* p) {
    return *(__attribute__((address_space(4))) const float*)(p);
}

// Whole-record load through the constant address space (scalar loads when
// the address is wave-uniform), for records written by an earlier kernel.
template <class T>
__device__ __forceinline__ T ld_uniform(const T* p) {
    static_assert(sizeof(T) % 4 == 0, "record of whole dwords");
    struct Raw {
        uint32_t w[sizeof(T) / 4];
    };
#if defined(__HIP_DEVICE_COMPILE__)
    Raw r;
    const __attribute__((address_space(4))) uint32_t* q =
        (const __attribute__((address_space(4))) uint32_t*)(p);
#pragma unroll
    for (unsigned i = 0; i < sizeof(T) / 4; ++i) r.w[i] = q[i];
    return __builtin_bit_cast(T, r);
#else
    return *p;  // host pass only parses device code
#endif
}

__device__ __forceinline__ int ldi(const int* p) {
    return *(__attribute__((address_space(1))) const int*)(p);
}

// Raw buffer resource over [base, base + bytes): a load whose offset lies
// beyond `bytes` returns zero without touching memory, which masks absent
// MFMA columns for free (no branch, no traffic).
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

__device__ __forceinline__ u32x4 bld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt bits [3:0] and [15:14]; expcnt
// and lgkmcnt left at "no wait").  For waits the compiler cannot see, such as
// LDS written by direct global->LDS loads that are older than N loads still
// in flight.
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier after LDS filled by direct global->LDS loads whose
// arrival each wave has already waited for (vm_wait).  A release fence would
// wait for every outstanding load (LDS DMA counts as a load), so only the
// acquire side is fenced: LDS reads cannot move above the barrier.  Not for
// LDS written by ordinary stores (use __syncthreads).
__device__ __forceinline__ void lds_dma_barrier() {
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Wave index as a scalar (uniform) value, so address arithmetic that depends
// on it stays in SGPRs and uniform loads become scalar loads.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// fp32 -> bf16 bits, round to nearest even (finite inputs; NaN kept quiet).
__device__ __forceinline__ uint32_t bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ uint32_t f16_rne(float f) {
    const _Float16 h = static_cast<_Float16>(f);  // v_cvt_f16_f32: RNE
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h));
}

__device__ __forceinline__ uint32_t cast_out(float f, int out_dtype) {
    return out_dtype == CX_DTYPE_FP16 ? f16_rne(f) : bf16_rne(f);
}

// Writes 4 consecutive outputs (16-bit out dtype, optional fp32 copy).
__device__ __forceinline__ void store_out4(void* y, float* y_f32, size_t idx, f32x4 v,
                                           int out_dtype) {
    uint16_t* yo = static_cast<uint16_t*>(y) + idx;
    *reinterpret_cast<uint2*>(yo) = uint2{cast_out(v[0], out_dtype) | (cast_out(v[1], out_dtype) << 16),
                                          cast_out(v[2], out_dtype) | (cast_out(v[3], out_dtype) << 16)};
    if (y_f32 != nullptr) *reinterpret_cast<float4*>(y_f32 + idx) = float4{v[0], v[1], v[2], v[3]};
}

// The first n (<= 4) of four consecutive output rows, one element at a time
// (idx need not be a multiple of 4).
__device__ __forceinline__ void store_out_n(void* y, float* y_f32, size_t idx, f32x4 v, int n,
                                            int out_dtype) {
    uint16_t* yo = static_cast<uint16_t*>(y) + idx;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (i < n) {
            yo[i] = (uint16_t)cast_out(v[i], out_dtype);
            if (y_f32 != nullptr) y_f32[idx + i] = v[i];
        }
    }
}

}  // namespace cx
