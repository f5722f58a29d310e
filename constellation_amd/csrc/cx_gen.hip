// cx_gen.hip — synthetic expert / activation generator and upload helpers.
//
// The generator definition (also restated independently by the CPU checker;
// tests require bit equality):
//   r  = mix(mix(seed ^ mix(stream)) + idx)           splitmix64 finaliser
//   u1 = ((r >> 40) + 1) * 2^-24,  u2 = ((r >> 16) & 0xFFFFFF) * 2^-24
//   N  = sqrt(-2 ln u1) * cos(2 pi u2)                 Box-Muller
// ln / sqrt / cos are fixed sequences of IEEE fp32 operations (Taylor
// polynomials with explicit fma, Newton steps), compiled without
// contraction, so the bits do not depend on the device math library.
// Block quantisation: scale = max(amax / 448, 1e-12) (correctly rounded
// divide), q = e4m3fn round-to-nearest-even of v / scale, saturating at 448.
#include "cx_internal.h"

#pragma clang fp contract(off)

namespace cx {
namespace {

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Per-(seed, stream) base of the counter hash; the device adds the index.
uint64_t mix64_host(uint64_t seed, uint64_t stream) { return mix64(seed ^ mix64(stream)); }

__device__ __forceinline__ float det_log(float u) {
    const uint32_t b = __float_as_uint(u);
    int e = (int)(b >> 23) - 127;
    float m = __uint_as_float((b & 0x7FFFFFu) | 0x3F800000u);
    if (m > 0x1.6a09e6p+0f) {
        m = __fmul_rn(m, 0.5f);
        e += 1;
    }
    const float f = __fsub_rn(m, 1.0f);
    float p = -0x1.24924ap-4f;
    p = __builtin_fmaf(p, f, 0x1.3b13b2p-4f);
    p = __builtin_fmaf(p, f, -0x1.555556p-4f);
    p = __builtin_fmaf(p, f, 0x1.745d18p-4f);
    p = __builtin_fmaf(p, f, -0x1.99999ap-4f);
    p = __builtin_fmaf(p, f, 0x1.c71c72p-4f);
    p = __builtin_fmaf(p, f, -0x1.0p-3f);
    p = __builtin_fmaf(p, f, 0x1.24924ap-3f);
    p = __builtin_fmaf(p, f, -0x1.555556p-3f);
    p = __builtin_fmaf(p, f, 0x1.99999ap-3f);
    p = __builtin_fmaf(p, f, -0x1.0p-2f);
    p = __builtin_fmaf(p, f, 0x1.555556p-2f);
    p = __builtin_fmaf(p, f, -0x1.0p-1f);
    p = __builtin_fmaf(p, f, 1.0f);
    p = __fmul_rn(p, f);
    return __builtin_fmaf((float)e, 0x1.62e430p-1f, p);
}

__device__ __forceinline__ float det_sqrt(float v) {
    if (!(v > 0.0f)) return 0.0f;
    float y = __uint_as_float(0x5f3759dfu - (__float_as_uint(v) >> 1));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float t = __fmul_rn(v, y);
        t = __fmul_rn(t, y);
        t = __builtin_fmaf(-0.5f, t, 1.5f);
        y = __fmul_rn(y, t);
    }
    return __fmul_rn(v, y);
}

__device__ __forceinline__ float det_cos2pi(float u) {
    const float v = __fsub_rn(u, 0.5f);
    float a = fabsf(v);
    float sgn = -1.0f;
    if (a > 0.25f) {
        a = __fsub_rn(0.5f, a);
        sgn = 1.0f;
    }
    const float w = __fmul_rn(a, a);
    float p = -0x1.2a0c5ap-5f;
    p = __builtin_fmaf(p, w, 0x1.20c62cp-2f);
    p = __builtin_fmaf(p, w, -0x1.b6e250p+0f);
    p = __builtin_fmaf(p, w, 0x1.f9d38ap+2f);
    p = __builtin_fmaf(p, w, -0x1.a6d1f2p+4f);
    p = __builtin_fmaf(p, w, 0x1.e1f506p+5f);
    p = __builtin_fmaf(p, w, -0x1.55d3c8p+6f);
    p = __builtin_fmaf(p, w, 0x1.03c1f0p+6f);
    p = __builtin_fmaf(p, w, -0x1.3bd3ccp+4f);
    p = __builtin_fmaf(p, w, 1.0f);
    return __fmul_rn(sgn, p);
}

__device__ __forceinline__ float gen_normal(uint64_t base, uint64_t idx) {
    const uint64_t r = mix64(base + idx);
    const float u1 = __fmul_rn((float)((uint32_t)(r >> 40) + 1u), 0x1.0p-24f);
    const float u2 = __fmul_rn((float)((uint32_t)(r >> 16) & 0xFFFFFFu), 0x1.0p-24f);
    const float l = det_log(u1);
    return __fmul_rn(det_sqrt(__fmul_rn(-2.0f, l)), det_cos2pi(u2));
}

__device__ __forceinline__ uint8_t fp8_encode(float v) {
    const uint32_t bits = __float_as_uint(v);
    const uint32_t sign = (bits >> 24) & 0x80u;
    const uint32_t abits = bits & 0x7FFFFFFFu;
    if (abits > 0x7F800000u) return (uint8_t)(sign | 0x7Fu);
    if (abits >= 0x43E00000u) return (uint8_t)(sign | 0x7Eu);
    if (abits < 0x3C800000u) {
        const float q = rintf(__fmul_rn(__uint_as_float(abits), 512.0f));
        return (uint8_t)(sign | (uint32_t)q);
    }
    int e = (int)(abits >> 23) - 127;
    const uint32_t mant = (abits & 0x7FFFFFu) | 0x800000u;
    uint32_t q = mant >> 20;
    const uint32_t rem = mant & 0xFFFFFu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) q++;
    if (q == 16u) {
        q = 8u;
        e++;
    }
    if (e > 8 || (e == 8 && q > 14u)) return (uint8_t)(sign | 0x7Eu);
    return (uint8_t)(sign | ((uint32_t)(e + 7) << 3) | (q - 8u));
}

__device__ __forceinline__ uint16_t bf16_rne_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__global__ void k_gen_normal(uint64_t base, uint64_t count, float std_dev, int dtype, void* out) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
        const float v = __fmul_rn(std_dev, gen_normal(base, i));
        if (dtype == CX_DTYPE_F32) {
            static_cast<float*>(out)[i] = v;
        } else if (dtype == CX_DTYPE_FP16) {
            const _Float16 h = static_cast<_Float16>(v);
            static_cast<uint16_t*>(out)[i] = __builtin_bit_cast(uint16_t, h);
        } else {
            static_cast<uint16_t*>(out)[i] = bf16_rne_bits(v);
        }
    }
}

// One workgroup per scale block: pass 1 finds amax, pass 2 quantises.
__global__ __launch_bounds__(256) void k_gen_fp8(uint64_t base, int rows, int cols, int rb,
                                                 int cb, float std_dev, uint8_t* q, float* scale,
                                                 int layout) {
    const int ncb = (cols + cb - 1) / cb;
    const int br = blockIdx.x / ncb, bc = blockIdx.x - br * ncb;
    const int r0 = br * rb, c0 = bc * cb;
    const int nr = min(rb, rows - r0), nc = min(cb, cols - c0);
    const int n = nr * nc;
    float amax = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int r = r0 + i / nc, c = c0 + i % nc;
        const float v = __fmul_rn(std_dev, gen_normal(base, (uint64_t)r * cols + c));
        amax = fmaxf(amax, fabsf(v));
    }
    __shared__ float red[256];
    red[threadIdx.x] = amax;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + off]);
        __syncthreads();
    }
    float s = __fdiv_rn(red[0], 448.0f);
    if (s < 1e-12f) s = 1e-12f;
    if (threadIdx.x == 0) scale[blockIdx.x] = s;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int r = r0 + i / nc, c = c0 + i % nc;
        const float v = __fmul_rn(std_dev, gen_normal(base, (uint64_t)r * cols + c));
        q[gu_elem_off(layout, cols, r, c)] = fp8_encode(__fdiv_rn(v, s));
    }
}

// 0x7F / 0xFF (OCP NaN) -> 0x7E / 0xFE: both pairs decode to +-448 in the
// reference's table (backend/fp8_lut_v2.cc:61).
__global__ void k_canonicalize(uint8_t* p, uint64_t n) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint8_t b = p[i];
        if ((b & 0x7Fu) == 0x7Fu) p[i] = (uint8_t)(b - 1u);
    }
}

// Row-major fp8 bytes -> CX_LAYOUT_TILE16, with the 0x7F/0xFF
// canonicalisation of k_canonicalize: one thread per 32-byte piece.
__global__ __launch_bounds__(256) void k_tile16_fp8(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                    int rows, int cols) {
    const int ppr = cols / 32;  // pieces per row
    const uint64_t n = (uint64_t)rows * ppr;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const int r = (int)(i / ppr), p = (int)(i - (uint64_t)r * ppr);
        typedef uint32_t w4 __attribute__((ext_vector_type(4)));
        const uint8_t* a = src + (size_t)r * cols + (size_t)p * 32;
        w4 v[2] = {*reinterpret_cast<const w4*>(a), *reinterpret_cast<const w4*>(a + 16)};
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t x = v[h][w];
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    if (((x >> (8 * b)) & 0x7Fu) == 0x7Fu) x -= 1u << (8 * b);
                v[h][w] = x;
            }
        uint8_t* d = dst + gu_piece_off(CX_LAYOUT_TILE16, cols, r, p >> 2, p & 3);
        *reinterpret_cast<w4*>(d) = v[0];
        *reinterpret_cast<w4*>(d + 16) = v[1];
    }
}

}  // namespace

hipError_t launch_tile16_fp8(const uint8_t* src, uint8_t* dst, int rows, int cols, hipStream_t s) {
    if (!gu_tile16_ok(rows, cols)) return hipErrorInvalidValue;
    uint64_t blocks = ((uint64_t)rows * (cols / 32) + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) return hipSuccess;
    cx_launch(k_tile16_fp8, dim3((unsigned)blocks), dim3(256), 0, s, src, dst, rows, cols);
    return hipGetLastError();
}

hipError_t launch_gen_normal(uint64_t seed, uint64_t stream_id, uint64_t count, float std_dev,
                             int dtype, void* out, hipStream_t s) {
    const uint64_t base = mix64_host(seed, stream_id);
    uint64_t blocks = (count + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) return hipSuccess;
    cx_launch(k_gen_normal, dim3((unsigned)blocks), dim3(256), 0, s, base, count, std_dev,
                       dtype, out);
    return hipGetLastError();
}

hipError_t launch_gen_fp8(uint64_t seed, uint64_t stream_id, int rows, int cols, int rb, int cb,
                          float std_dev, uint8_t* q, float* scale, hipStream_t s, int layout) {
    if (layout == CX_LAYOUT_TILE16 && !gu_tile16_ok(rows, cols)) return hipErrorInvalidValue;
    const uint64_t base = mix64_host(seed, stream_id);
    const int nblk = ((rows + rb - 1) / rb) * ((cols + cb - 1) / cb);
    cx_launch(k_gen_fp8, dim3(nblk), dim3(256), 0, s, base, rows, cols, rb, cb, std_dev,
                       q, scale, layout);
    return hipGetLastError();
}

hipError_t launch_canonicalize_fp8(uint8_t* p, uint64_t n, hipStream_t s) {
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) return hipSuccess;
    cx_launch(k_canonicalize, dim3((unsigned)blocks), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

}  // namespace cx
