/*
 * cx_oracle.c — CPU restatement of the reference's MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (constellation_amd/,
 * include/) links, loads or calls this file.  Only tests/, the smoke() check
 * of __graft_entry__.py and the cpu_baseline leg of bench.py use it, and only
 * as the checker / CPU baseline, never as the thing measured or shipped.
 *
 * Every function names the reference file:line it restates.  How each one is
 * pinned (golden vectors from the reference's own C++ compiled into
 * oracle/_ref, closed forms, torch, brute force) is listed in the test that
 * pins it (tests/test_oracle_*.py).
 *
 * Build: gcc -O2 -fopenmp -ffp-contract=off (oracle/Makefile).  Contraction
 * is off so every a*b+c below rounds twice, exactly as written.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define CXO_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------- */
/* fp8 e4m3fn decode with the reference quirk: exp==15 && mant==7 (0x7F/0xFF)
 * decodes to +-448 instead of NaN.  backend/fp8_lut_v2.cc:47-66. */
CXO_API float cxo_fp8_decode(uint8_t v) {
    const int sign = (v >> 7) & 1;
    const int e = (v >> 3) & 0xF;
    const int m = v & 7;
    const float s = sign ? -1.0f : 1.0f;
    if (e == 0) {
        if (m == 0) return s * 0.0f;
        return s * ldexpf((float)m / 8.0f, -6);
    }
    if (e == 15 && m == 7) return s * 448.0f;
    return s * ldexpf(1.0f + (float)m / 8.0f, e - 7);
}

/* fp32 -> e4m3fn, round-to-nearest-even, saturating to +-448 (0x7E/0xFE).
 * Quantiser of the synthetic experts (quantised per 128x128 block,
 * scale = amax/448), equal to torch.to(float8_e4m3fn) for
 * |v| <= 448.  Written on the bit pattern so CPU and GPU agree exactly. */
CXO_API uint8_t cxo_fp8_encode(float v) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    const uint8_t sign = (uint8_t)((bits >> 24) & 0x80);
    const uint32_t abits = bits & 0x7FFFFFFFu;
    if (abits > 0x7F800000u) return (uint8_t)(sign | 0x7F);     /* NaN */
    if (abits >= 0x43E00000u) return (uint8_t)(sign | 0x7E);    /* >= 448 */
    if (abits < 0x3C800000u) {                                    /* < 2^-6 */
        float a;
        memcpy(&a, &abits, 4);
        const float q = nearbyintf(a * 512.0f);                   /* quantum 2^-9 */
        return (uint8_t)(sign | (uint8_t)q);                      /* q==8 -> 0x08 */
    }
    int e = (int)(abits >> 23) - 127;                              /* -6..8 */
    uint32_t mant = (abits & 0x7FFFFFu) | 0x800000u;
    uint32_t q = mant >> 20;                                       /* 8..15 */
    const uint32_t rem = mant & 0xFFFFFu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) q++;
    if (q == 16u) { q = 8u; e++; }
    if (e > 8 || (e == 8 && q > 14u)) return (uint8_t)(sign | 0x7E);
    return (uint8_t)(sign | (uint8_t)(((uint32_t)(e + 7) << 3) | (q - 8u)));
}

/* ------------------------------------------------------------------------- */
/* Activation codecs, backend/activation_codec_v2.h:8-114.
 * Decoders are exact.  The reference encoders round half-up on the raw bits
 * (bf16: bits + 0x8000, :83-88; fp16: + 0x1000 then >> 13, :49-81); the RNE
 * encoders are what the HIP kernels use. */
CXO_API float cxo_bf16_decode(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

CXO_API uint16_t cxo_bf16_encode_ref(float x) {
    uint32_t bits;
    memcpy(&bits, &x, 4);
    bits += 0x00008000u;
    return (uint16_t)(bits >> 16);
}

CXO_API uint16_t cxo_bf16_encode_rne(float x) {
    uint32_t bits;
    memcpy(&bits, &x, 4);
    if ((bits & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((bits >> 16) | 0x40);
    bits += 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

CXO_API float cxo_fp16_decode(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t f = h & 0x3FFu;
    uint32_t out;
    if (e == 0) {
        if (f == 0) {
            out = sign;
        } else {
            int ex = -14;
            while ((f & 0x400u) == 0) { f <<= 1; ex--; }
            out = sign | ((uint32_t)(ex + 127) << 23) | ((f & 0x3FFu) << 13);
        }
    } else if (e == 0x1F) {
        out = sign | 0x7F800000u | (f << 13);
    } else {
        out = sign | ((e + 112u) << 23) | (f << 13);
    }
    float r;
    memcpy(&r, &out, 4);
    return r;
}

CXO_API uint16_t cxo_fp16_encode_ref(float x) {
    uint32_t bits;
    memcpy(&bits, &x, 4);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    int e = (int)((bits >> 23) & 0xFFu) - 127 + 15;
    uint32_t mant = bits & 0x7FFFFFu;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant = (mant | 0x800000u) >> (1 - e);
        return (uint16_t)(sign | ((mant + 0x1000u) >> 13));
    }
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    uint32_t hm = (mant + 0x1000u) >> 13;
    if (hm == 0x400u) {
        hm = 0;
        e++;
        if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | hm);
}

CXO_API uint16_t cxo_fp16_encode_rne(float x) {
    uint32_t bits;
    memcpy(&bits, &x, 4);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const uint32_t abits = bits & 0x7FFFFFFFu;
    if (abits > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);   /* NaN */
    if (abits >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  /* >= 65520 -> inf */
    if (abits < 0x38800000u) {                                      /* < 2^-14 */
        float a;
        memcpy(&a, &abits, 4);
        return (uint16_t)(sign | (uint16_t)nearbyintf(a * 16777216.0f));
    }
    const uint32_t mant = abits & 0x7FFFFFu;
    uint32_t q = (((abits >> 23) - 112u) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* ------------------------------------------------------------------------- */
/* Synthetic-data generator (defined by this build; the reference has none for
 * these shapes).  The HIP library implements the same definition
 * (constellation_amd/csrc/cx_gen.hip); tests assert the two agree bit for bit.
 *   r   = mix(mix(seed ^ mix(stream)) + idx)          splitmix64 finaliser
 *   u1  = ((r >> 40) + 1) * 2^-24   in (0,1]
 *   u2  = ((r >> 16) & 0xFFFFFF) * 2^-24  in [0,1)
 *   N   = sqrt(-2 ln u1) * cos(2 pi u2)               Box-Muller
 * ln, sqrt and cos are fixed polynomial / Newton sequences of IEEE fp32
 * operations, so both sides produce identical bits. */
static uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

CXO_API uint64_t cxo_rand64(uint64_t seed, uint64_t stream, uint64_t idx) {
    return mix64(mix64(seed ^ mix64(stream)) + idx);
}

static float f_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_from_f(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* ln(u), u in (0,1]: u = m*2^e with m in [sqrt(.5), sqrt(2)), ln(1+f) Taylor
 * series to f^14 (|f| <= 0.415). */
static float det_log(float u) {
    uint32_t b = bits_from_f(u);
    int e = (int)(b >> 23) - 127;
    float m = f_from_bits((b & 0x7FFFFFu) | 0x3F800000u);
    if (m > 0x1.6a09e6p+0f) { m = m * 0.5f; e += 1; }
    const float f = m - 1.0f;
    float p = -0x1.24924ap-4f;
    p = fmaf(p, f, 0x1.3b13b2p-4f);
    p = fmaf(p, f, -0x1.555556p-4f);
    p = fmaf(p, f, 0x1.745d18p-4f);
    p = fmaf(p, f, -0x1.99999ap-4f);
    p = fmaf(p, f, 0x1.c71c72p-4f);
    p = fmaf(p, f, -0x1.0p-3f);
    p = fmaf(p, f, 0x1.24924ap-3f);
    p = fmaf(p, f, -0x1.555556p-3f);
    p = fmaf(p, f, 0x1.99999ap-3f);
    p = fmaf(p, f, -0x1.0p-2f);
    p = fmaf(p, f, 0x1.555556p-2f);
    p = fmaf(p, f, -0x1.0p-1f);
    p = fmaf(p, f, 1.0f);
    p = p * f;
    return fmaf((float)e, 0x1.62e430p-1f, p);
}

/* sqrt(v), v >= 0: bit-trick reciprocal-sqrt seed, 4 Newton steps. */
static float det_sqrt(float v) {
    if (!(v > 0.0f)) return 0.0f;
    float y = f_from_bits(0x5f3759dfu - (bits_from_f(v) >> 1));
    for (int i = 0; i < 4; ++i) {
        float t = v * y;
        t = t * y;
        t = fmaf(-0.5f, t, 1.5f);
        y = y * t;
    }
    return v * y;
}

/* cos(2 pi u), u in [0,1): fold to a in [0, 1/4], Taylor series in a^2. */
static float det_cos2pi(float u) {
    float v = u - 0.5f;                 /* cos(2pi u) = -cos(2pi v) */
    float a = fabsf(v);
    float sgn = -1.0f;
    if (a > 0.25f) { a = 0.5f - a; sgn = 1.0f; }
    const float w = a * a;
    float p = -0x1.2a0c5ap-5f;
    p = fmaf(p, w, 0x1.20c62cp-2f);
    p = fmaf(p, w, -0x1.b6e250p+0f);
    p = fmaf(p, w, 0x1.f9d38ap+2f);
    p = fmaf(p, w, -0x1.a6d1f2p+4f);
    p = fmaf(p, w, 0x1.e1f506p+5f);
    p = fmaf(p, w, -0x1.55d3c8p+6f);
    p = fmaf(p, w, 0x1.03c1f0p+6f);
    p = fmaf(p, w, -0x1.3bd3ccp+4f);
    p = fmaf(p, w, 1.0f);
    return sgn * p;
}

CXO_API float cxo_normal(uint64_t seed, uint64_t stream, uint64_t idx) {
    const uint64_t r = cxo_rand64(seed, stream, idx);
    const float u1 = (float)((uint32_t)(r >> 40) + 1u) * 0x1.0p-24f;
    const float u2 = (float)((uint32_t)(r >> 16) & 0xFFFFFFu) * 0x1.0p-24f;
    const float l = det_log(u1);
    return det_sqrt(-2.0f * l) * det_cos2pi(u2);
}

CXO_API void cxo_gen_normal_f32(uint64_t seed, uint64_t stream, uint64_t n,
                                float std_dev, float* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = std_dev * cxo_normal(seed, stream, i);
}

CXO_API void cxo_gen_normal_bf16(uint64_t seed, uint64_t stream, uint64_t n,
                                 float std_dev, uint16_t* out) {
    for (uint64_t i = 0; i < n; ++i)
        out[i] = cxo_bf16_encode_rne(std_dev * cxo_normal(seed, stream, i));
}

CXO_API void cxo_gen_normal_fp16(uint64_t seed, uint64_t stream, uint64_t n,
                                 float std_dev, uint16_t* out) {
    for (uint64_t i = 0; i < n; ++i)
        out[i] = cxo_fp16_encode_rne(std_dev * cxo_normal(seed, stream, i));
}

/* Block-quantised fp8 matrix: element (r,c) = std*N(seed,stream,r*cols+c);
 * per block scale = max(amax/448, 1e-12); q = encode(v/scale). */
CXO_API void cxo_gen_fp8_matrix(uint64_t seed, uint64_t stream, int rows, int cols,
                                int rb, int cb, float std_dev,
                                uint8_t* q, float* scale) {
    const int nrb = (rows + rb - 1) / rb, ncb = (cols + cb - 1) / cb;
#pragma omp parallel for schedule(static)
    for (int br = 0; br < nrb; ++br) {
        for (int bc = 0; bc < ncb; ++bc) {
            const int r1 = (br + 1) * rb < rows ? (br + 1) * rb : rows;
            const int c1 = (bc + 1) * cb < cols ? (bc + 1) * cb : cols;
            float amax = 0.0f;
            for (int r = br * rb; r < r1; ++r)
                for (int c = bc * cb; c < c1; ++c) {
                    const float v = std_dev * cxo_normal(seed, stream, (uint64_t)r * cols + c);
                    const float a = fabsf(v);
                    if (a > amax) amax = a;
                }
            float s = amax / 448.0f;
            if (s < 1e-12f) s = 1e-12f;
            scale[br * ncb + bc] = s;
            for (int r = br * rb; r < r1; ++r)
                for (int c = bc * cb; c < c1; ++c) {
                    const float v = std_dev * cxo_normal(seed, stream, (uint64_t)r * cols + c);
                    q[(size_t)r * cols + c] = cxo_fp8_encode(v / s);
                }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Expert MLP, dequantise-then-fp32, in the reference's accumulation order:
 * RunFusedUpGateReferenceV2 (backend/expert_reference_v2.cc:11-90):
 *   for k: w = lut[b]*scale; sum += w*x   (one rounding each), up and gate;
 *   h = (gate/(1+exp(-gate))) * up
 * RunDownReferenceV2 (:92-144): y = sum_k (lut[b]*scale)*h[k].
 * x is already decoded to fp32 (DecodeActivationToFloatV2 is exact); y is
 * returned pre-cast.  Rows are independent, so the row loop is parallel;
 * each row's sum keeps the sequential order. */
/* x [n_tokens][len] -> blocks of tb tokens, k-major: out[(b*len + k)*tb + t]
 * (zeros for the padding tokens of the last block). */
static float* cxo_token_blocks(const float* x, int n_tokens, int len, int tb) {
    const int nb = (n_tokens + tb - 1) / tb;
    float* out = (float*)calloc((size_t)nb * len * tb, sizeof(float));
    if (!out) return NULL;
    for (int t = 0; t < n_tokens; ++t) {
        const int b = t / tb, tt = t % tb;
        for (int k = 0; k < len; ++k) out[((size_t)b * len + k) * tb + tt] = x[(size_t)t * len + k];
    }
    return out;
}

/* Gate/up rows [r0, r1) for token block b (TB tokens, k-major xk): h of the
 * block's real tokens into h [T][inter] and hb (k-major, as the down reads). */
static inline __attribute__((always_inline)) void cxo_gu_row(
    const uint8_t* wu, const float* su_r, const uint8_t* wg, const float* sg_r, const float* lut,
    int hidden, int inter, int up_cb, int gate_cb, const float* xk, int r, int b, int n_tokens,
    float* h, float* hb, const int TB) {
    const size_t base = (size_t)r * hidden;
    float up[16], gate[16];
    for (int t = 0; t < TB; ++t) up[t] = gate[t] = 0.0f;
    int k = 0;
    while (k < hidden) {
        const int ku = (k / up_cb + 1) * up_cb, kg = (k / gate_cb + 1) * gate_cb;
        const int kend = ku < kg ? (ku < hidden ? ku : hidden) : (kg < hidden ? kg : hidden);
        const float s_u = su_r[k / up_cb], s_g = sg_r[k / gate_cb];
        for (; k < kend; ++k) {
            const float wuv = lut[wu[base + k]] * s_u;
            const float wgv = lut[wg[base + k]] * s_g;
            const float* xv = xk + (size_t)k * TB;
            for (int t = 0; t < TB; ++t) {
                const float pu = wuv * xv[t];
                const float pg = wgv * xv[t];
                up[t] = up[t] + pu;
                gate[t] = gate[t] + pg;
            }
        }
    }
    for (int t = 0; t < TB && b * TB + t < n_tokens; ++t) {
        const float silu = gate[t] / (1.0f + expf(-gate[t]));
        const float hv = silu * up[t];
        h[(size_t)(b * TB + t) * inter + r] = hv;
        hb[((size_t)b * inter + r) * TB + t] = hv;
    }
}

static inline __attribute__((always_inline)) void cxo_down_row(
    const uint8_t* wd, const float* sd_r, const float* lut, int hidden, int inter, int down_cb,
    const float* hk, int r, int b, int n_tokens, float* y, const int TB) {
    const size_t base = (size_t)r * inter;
    float sum[16];
    for (int t = 0; t < TB; ++t) sum[t] = 0.0f;
    int k = 0;
    while (k < inter) {
        const int kd = (k / down_cb + 1) * down_cb;
        const int kend = kd < inter ? kd : inter;
        const float s_d = sd_r[k / down_cb];
        for (; k < kend; ++k) {
            const float w = lut[wd[base + k]] * s_d;
            const float* hv = hk + (size_t)k * TB;
            for (int t = 0; t < TB; ++t) {
                const float pr = w * hv[t];
                sum[t] = sum[t] + pr;
            }
        }
    }
    for (int t = 0; t < TB && b * TB + t < n_tokens; ++t) y[(size_t)(b * TB + t) * hidden + r] = sum[t];
}

CXO_API void cxo_expert_ref(const uint8_t* wu, const float* su,
                            const uint8_t* wg, const float* sg,
                            const uint8_t* wd, const float* sd,
                            int hidden, int inter,
                            int up_rb, int up_cb, int gate_rb, int gate_cb,
                            int down_rb, int down_cb,
                            const float* x, int n_tokens, float* h, float* y) {
    /* Each (token, row) value is the reference's sequence of fp32 operations
     * (w = lut[b]*scale, p = w*x[k], sum = sum + p, k ascending); the loops
     * only decode each weight once per block of tokens and read each column
     * block's scale once, which changes no rounding. */
    float lut[256];
    for (int i = 0; i < 256; ++i) lut[i] = cxo_fp8_decode((uint8_t)i);
    const int up_ncb = (hidden + up_cb - 1) / up_cb;
    const int gate_ncb = (hidden + gate_cb - 1) / gate_cb;
    const int down_ncb = (inter + down_cb - 1) / down_cb;
    const int tb = n_tokens >= 16 ? 16 : n_tokens >= 4 ? 4 : 1;
    const int nb = (n_tokens + tb - 1) / tb;
    float* xb = cxo_token_blocks(x, n_tokens, hidden, tb);
    float* hb = (float*)calloc((size_t)nb * inter * tb, sizeof(float));
    if (!xb || !hb) {
        free(xb);
        free(hb);
        return;
    }
#pragma omp parallel for schedule(static)
    for (int r = 0; r < inter; ++r) {
        const float* su_r = su + (size_t)(r / up_rb) * up_ncb;
        const float* sg_r = sg + (size_t)(r / gate_rb) * gate_ncb;
        for (int b = 0; b < nb; ++b) {
            const float* xk = xb + (size_t)b * hidden * tb;
            if (tb == 16)
                cxo_gu_row(wu, su_r, wg, sg_r, lut, hidden, inter, up_cb, gate_cb, xk, r, b, n_tokens, h, hb, 16);
            else if (tb == 4)
                cxo_gu_row(wu, su_r, wg, sg_r, lut, hidden, inter, up_cb, gate_cb, xk, r, b, n_tokens, h, hb, 4);
            else
                cxo_gu_row(wu, su_r, wg, sg_r, lut, hidden, inter, up_cb, gate_cb, xk, r, b, n_tokens, h, hb, 1);
        }
    }
#pragma omp parallel for schedule(static)
    for (int r = 0; r < hidden; ++r) {
        const float* sd_r = sd + (size_t)(r / down_rb) * down_ncb;
        for (int b = 0; b < nb; ++b) {
            const float* hk = hb + (size_t)b * inter * tb;
            if (tb == 16) cxo_down_row(wd, sd_r, lut, hidden, inter, down_cb, hk, r, b, n_tokens, y, 16);
            else if (tb == 4) cxo_down_row(wd, sd_r, lut, hidden, inter, down_cb, hk, r, b, n_tokens, y, 4);
            else cxo_down_row(wd, sd_r, lut, hidden, inter, down_cb, hk, r, b, n_tokens, y, 1);
        }
    }
    free(xb);
    free(hb);
}

/* ------------------------------------------------------------------------- */
/* The reference CPU expert path, restated: RunExpertCpuV2
 * (backend/cpu/backend_cpu_v2.cc:196-267) -> RunFusedUpGateCpuV2
 * (backend/cpu/fused_up_gate_cpu_v2.cc:12-178) -> RunDownCpuV2
 * (backend/cpu/down_cpu_v2.cc:10-119): x decoded to fp32 first; OpenMP
 * static over rows; per column block the scale is loaded once; four partial
 * sums over k&3, combined (s0+s1)+(s2+s3); output encoded with the
 * reference's half-up encoders.  dtype: 1 fp16, 2 bf16.  Single block size
 * pair per matrix as in the reference (up and gate col blocks must match). */
CXO_API int cxo_expert_cpu_baseline(const uint8_t* wu, const float* su,
                                    const uint8_t* wg, const float* sg,
                                    const uint8_t* wd, const float* sd,
                                    int hidden, int inter, int rb, int cb,
                                    const uint16_t* x, int in_dtype,
                                    uint16_t* y, int out_dtype,
                                    float* h_scratch, float* x_scratch,
                                    int n_threads) {
    if ((in_dtype != 1 && in_dtype != 2) || (out_dtype != 1 && out_dtype != 2)) return -1;
    if (n_threads <= 0) n_threads = 1;
    float lut[256];
    for (int i = 0; i < 256; ++i) lut[i] = cxo_fp8_decode((uint8_t)i);
    for (int k = 0; k < hidden; ++k)
        x_scratch[k] = in_dtype == 1 ? cxo_fp16_decode(x[k]) : cxo_bf16_decode(x[k]);
    const int up_ncb = (hidden + cb - 1) / cb;
#pragma omp parallel for schedule(static) num_threads(n_threads)
    for (int r = 0; r < inter; ++r) {
        const size_t base = (size_t)r * hidden;
        float u[4] = {0, 0, 0, 0}, g[4] = {0, 0, 0, 0};
        for (int k0 = 0; k0 < hidden; k0 += cb) {
            const int k1 = k0 + cb < hidden ? k0 + cb : hidden;
            const float us = su[(r / rb) * up_ncb + k0 / cb];
            const float gs = sg[(r / rb) * up_ncb + k0 / cb];
            for (int k = k0; k < k1; ++k) {
                const int lane = (k - k0) & 3;
                const float pu = (lut[wu[base + k]] * us) * x_scratch[k];
                const float pg = (lut[wg[base + k]] * gs) * x_scratch[k];
                u[lane] = u[lane] + pu;
                g[lane] = g[lane] + pg;
            }
        }
        const float up = (u[0] + u[1]) + (u[2] + u[3]);
        const float gate = (g[0] + g[1]) + (g[2] + g[3]);
        h_scratch[r] = (gate / (1.0f + expf(-gate))) * up;
    }
    const int down_ncb = (inter + cb - 1) / cb;
#pragma omp parallel for schedule(static) num_threads(n_threads)
    for (int r = 0; r < hidden; ++r) {
        const size_t base = (size_t)r * inter;
        float s4[4] = {0, 0, 0, 0};
        for (int k0 = 0; k0 < inter; k0 += cb) {
            const int k1 = k0 + cb < inter ? k0 + cb : inter;
            const float sc = sd[(r / rb) * down_ncb + k0 / cb];
            for (int k = k0; k < k1; ++k) {
                const int lane = (k - k0) & 3;
                const float p = (lut[wd[base + k]] * sc) * h_scratch[k];
                s4[lane] = s4[lane] + p;
            }
        }
        const float sum = (s4[0] + s4[1]) + (s4[2] + s4[3]);
        y[r] = out_dtype == 1 ? cxo_fp16_encode_ref(sum) : cxo_bf16_encode_ref(sum);
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* DeepSeek-V3 router in float64, route_token_real
 * (server/moe_layer_runtime.py:321-381):
 *   logits = W.x; s = sigmoid; c = s + bias, -inf where not resident;
 *   s = 0 where not resident (:340-341); group score = top-2 sum of c
 *   (:343-345); keep topk_group groups (:347-361); top min(top_k,#resident)
 *   of c inside them (:363-371); w = s[idx] (:373); normalise with +1e-20
 *   when norm and k>1 (:376-378); w *= scale (:381).
 * Ties break toward the lower index (torch.topk leaves it unspecified).
 * ids are written in descending choice order; returns the number chosen.
 * margins[0] = (kth - (k+1)th) choice score among kept candidates (inf if
 * none), margins[1] = (topk_group-th - next) group score (inf if all kept).
 * Products of fp32 values are exact in fp64, so only the sum order differs
 * from exact math. */
static int better(double a, int ia, double b, int ib) {
    return a > b || (a == b && ia < ib);
}

CXO_API int cxo_route(const float* x, const float* w, const float* bias,
                      const uint8_t* resident, int hidden, int n_experts,
                      int n_group, int topk_group, int top_k, int norm,
                      double scale, int* ids, double* wout, double* margins,
                      double* logits_out) {
    if (n_experts <= 0 || n_group <= 0 || n_experts % n_group != 0) return -1;
    if (topk_group <= 0 || topk_group > n_group || top_k <= 0 || top_k > n_experts) return -1;
    if (n_experts > 4096) return -1;
    const int epg = n_experts / n_group;
    double c[4096], s[4096], gs[512];
    int n_res = 0;
    for (int e = 0; e < n_experts; ++e) {
        double acc = 0.0;
        for (int k = 0; k < hidden; ++k) acc += (double)w[(size_t)e * hidden + k] * (double)x[k];
        if (logits_out) logits_out[e] = acc;
        const double sg = 1.0 / (1.0 + exp(-acc));
        const int res = resident ? resident[e] != 0 : 1;
        n_res += res;
        s[e] = res ? sg : 0.0;
        c[e] = res ? sg + (double)bias[e] : -INFINITY;
    }
    if (n_res == 0) return -2;
    for (int g = 0; g < n_group; ++g) {
        int i1 = -1, i2 = -1;
        for (int j = g * epg; j < (g + 1) * epg; ++j) {
            if (i1 < 0 || better(c[j], j, c[i1], i1)) { i2 = i1; i1 = j; }
            else if (i2 < 0 || better(c[j], j, c[i2], i2)) { i2 = j; }
        }
        gs[g] = epg >= 2 ? c[i1] + c[i2] : c[i1];
    }
    int gsel[512];
    int gtaken[512] = {0};
    for (int r = 0; r < topk_group; ++r) {
        int b = -1;
        for (int g = 0; g < n_group; ++g)
            if (!gtaken[g] && (b < 0 || better(gs[g], g, gs[b], b))) b = g;
        gtaken[b] = 1;
        gsel[r] = b;
    }
    if (margins) {
        margins[1] = INFINITY;
        if (topk_group < n_group) {
            int b = -1;
            for (int g = 0; g < n_group; ++g)
                if (!gtaken[g] && (b < 0 || better(gs[g], g, gs[b], b))) b = g;
            margins[1] = gs[gsel[topk_group - 1]] - gs[b];
        }
    }
    double cand[4096];
    for (int e = 0; e < n_experts; ++e) cand[e] = gtaken[e / epg] ? c[e] : -INFINITY;
    const int k = top_k < n_res ? top_k : n_res;
    int taken[4096];
    memset(taken, 0, sizeof(int) * (size_t)n_experts);
    double wsum = 0.0;
    for (int r = 0; r < k; ++r) {
        int b = -1;
        for (int e = 0; e < n_experts; ++e)
            if (!taken[e] && (b < 0 || better(cand[e], e, cand[b], b))) b = e;
        taken[b] = 1;
        ids[r] = b;
        wout[r] = s[b];
        wsum += s[b];
    }
    if (margins) {
        margins[0] = INFINITY;
        int b = -1;
        for (int e = 0; e < n_experts; ++e)
            if (!taken[e] && (b < 0 || better(cand[e], e, cand[b], b))) b = e;
        if (b >= 0) margins[0] = cand[ids[k - 1]] - cand[b];
    }
    if (norm && k > 1) {
        const double d = wsum + 1e-20;
        for (int r = 0; r < k; ++r) wout[r] /= d;
    }
    for (int r = 0; r < k; ++r) wout[r] *= scale;
    return k;
}
