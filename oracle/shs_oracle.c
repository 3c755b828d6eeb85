/*
 * shs_oracle.c — CPU restatement of llm-shield's Shieldstral prefill arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP path is compared against and
 * the CPU baseline ("port") timed by bench.py. The product library never links it.
 * Built with -ffp-contract=off so that every fused multiply-add below is an
 * explicit fmaf() where the reference fuses, and nothing else is fused.
 *
 * Pinning (what checks each function independently of this file; tests/ names):
 *   ora_half_to_float        all 65 536 patterns vs numpy float16 (test_oracle_golden)
 *   ora_dequantize           gguf-package fixture, quantized + synthetic blocks, bit-exact
 *   ora_quantize             replay of the gguf fixture generator's rng: reproduces the
 *                            fixture's quantized bytes exactly (Q4_0/Q4_1/Q5_0/Q5_1/Q8_0)
 *   ora_quantize_activations closed-form invariants (round trip ≤ 1.05/254 of block max,
 *                            zero block, ties to even) + numpy restatement on random data
 *   ora_block_sums           numpy int64 brute force, exact
 *   ora_matmul*              float64 closed form within 1e-5; exact-rational emulation of
 *                            the fused epilogue on small shapes (bit-exact); batch
 *                            invariance and row-subset identity (bit-exact)
 *   ora_rmsnorm/swiglu/softmax/dot4/add_scaled4   float64 closed forms at 1e-5/1e-6
 *   ora_rope_*               closed forms: identity at 0, norm preserved, adjacent pairs,
 *                            YaRN mscale = 1 when apply_scale is off, ramp endpoints
 *   ora_forward              stage by stage against a numpy float64 restatement, each
 *                            stage fed this oracle's captured input, ≤ 1e-5 relative per
 *                            stage, for query/KV head counts 4/1, 4/2, 8/2, 8/4, 6/3, 32/8
 *                            (GQA mapping and per-head KV layout), after a cached prefix,
 *                            and with YaRN + the query temperature engaged; the KV snapshot
 *                            equals the captured k/v rows; end to end on a 4/1 model within
 *                            2e-3 (int8 code flips compound across layers there); prefix-
 *                            cache bit identity
 *   ora_score                closed form
 *   ora_expf                 < 1 ulp of float64 exp: measured over all 2.24e9 floats in
 *                            (-104, 89] (worst 0.99999997 ulp), tested on every 257th;
 *                            exact at 0; the overflow, underflow and NaN edges
 * Parity unpinned at the ulp level against .NET: exp/sigmoid (ora_expf here, the
 * vectorized polynomial of System.Numerics.Tensors there), cos/sin/pow (glibc here, the
 * .NET runtime's CRT calls there), and the order of the horizontal Vector<float>.Sum
 * (taken to be pairwise, ((0+1)+(2+3))+((4+5)+(6+7))) and of TensorPrimitives.Sum
 * (taken to be 8 strided lanes, pairwise-summed, then the tail in order).
 */
#include "shs_oracle.h"

#include <float.h>
#include <stdint.h>
#include <stdio.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 32

/* ------------------------------------------------------------- fp16 */

/* Exact fp16 → fp32 for every bit pattern, NaNs quieted
 * (IntegerGemm.HalfToSingle, IntegerGemm.cs:235-245; (float)Half). */
float ora_half_to_float(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* fp32 → fp16, round to nearest even, overflow to infinity (numpy astype(float16),
 * System.Half explicit conversion). */
uint16_t ora_float_to_half(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u | ((ax >> 13) & 0x3FFu) : 0));
    if (ax >= 0x477FF000u) /* ≥ 65520 rounds to inf */
        return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) { /* result subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t man = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126 - e; /* 14..24 */
        uint32_t half_bits = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (half_bits & 1))) half_bits++;
        return (uint16_t)(sign | half_bits);
    }
    uint32_t e = (ax >> 23) - 112;
    uint32_t man = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)(sign | h);
}

static inline float rd_half(const uint8_t* p) { return ora_half_to_float((uint16_t)(p[0] | (p[1] << 8))); }
static inline void wr_half(uint8_t* p, float f) { uint16_t h = ora_float_to_half(f); p[0] = (uint8_t)h; p[1] = (uint8_t)(h >> 8); }
static inline uint32_t rd_u32(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }

/* --------------------------------------------------- block geometry / decode */

/* GgmlTypeInfo.TypeSize (GgmlType.cs:67-106) for the 32-element legacy types. */
int ora_type_size(int type)
{
    switch (type) {
    case ORA_Q4_0: return 18;
    case ORA_Q4_1: return 20;
    case ORA_Q5_0: return 22;
    case ORA_Q5_1: return 24;
    case ORA_Q8_0: return 34;
    case ORA_F32: return 4 * QK;
    case ORA_F16: return 2 * QK;
    default: return -1;
    }
}

int64_t ora_row_bytes(int type, int64_t cols)
{
    int ts = ora_type_size(type);
    if (ts < 0 || cols % QK) return -1;
    return cols / QK * ts;
}

/* Dequantizer.Q4_0/Q4_1/Q5_0/Q5_1/Q8_0 (Dequantizer.cs:127-213). */
int ora_dequantize(int type, const uint8_t* src, float* dst, int64_t n)
{
    if (n % QK) return -1;
    for (int64_t b = 0; b < n / QK; b++, dst += QK) {
        switch (type) {
        case ORA_Q4_0: {
            const uint8_t* p = src + b * 18;
            float d = rd_half(p);
            for (int j = 0; j < 16; j++) {
                dst[j] = d * (float)((p[2 + j] & 0x0F) - 8);
                dst[16 + j] = d * (float)((p[2 + j] >> 4) - 8);
            }
            break;
        }
        case ORA_Q4_1: {
            const uint8_t* p = src + b * 20;
            float d = rd_half(p), m = rd_half(p + 2);
            for (int j = 0; j < 16; j++) {
                dst[j] = d * (float)(p[4 + j] & 0x0F) + m;
                dst[16 + j] = d * (float)(p[4 + j] >> 4) + m;
            }
            break;
        }
        case ORA_Q5_0: {
            const uint8_t* p = src + b * 22;
            float d = rd_half(p);
            uint32_t qh = rd_u32(p + 2);
            for (int j = 0; j < 16; j++) {
                int lo = (p[6 + j] & 0x0F) | (int)(((qh >> j) & 1u) << 4);
                int hi = (p[6 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
                dst[j] = d * (float)(lo - 16);
                dst[16 + j] = d * (float)(hi - 16);
            }
            break;
        }
        case ORA_Q5_1: {
            const uint8_t* p = src + b * 24;
            float d = rd_half(p), m = rd_half(p + 2);
            uint32_t qh = rd_u32(p + 4);
            for (int j = 0; j < 16; j++) {
                int lo = (p[8 + j] & 0x0F) | (int)(((qh >> j) & 1u) << 4);
                int hi = (p[8 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
                dst[j] = d * (float)lo + m;
                dst[16 + j] = d * (float)hi + m;
            }
            break;
        }
        case ORA_Q8_0: {
            const uint8_t* p = src + b * 34;
            float d = rd_half(p);
            for (int j = 0; j < 32; j++) dst[j] = (float)(int8_t)p[2 + j] * d;
            break;
        }
        default:
            return -1;
        }
    }
    return 0;
}

/* First element of largest magnitude, sign kept (numpy abs().argmax + take). */
static float signed_absmax(const float* x)
{
    float amax = 0.0f, v = 0.0f;
    for (int j = 0; j < QK; j++)
        if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); v = x[j]; }
    return v;
}

/* gguf-py's 0.5-biased truncation of (x·id + bias) evaluated in float64 and then
 * rounded to float32 before the truncation (np.trunc(..., dtype=float32)). */
static int trunc_biased64(float x, float id, double bias, int hi)
{
    double t = (double)x * (double)id;
    t = t + bias;
    float tf = truncf((float)t);
    int q = (int)tf;
    if (q < 0) q = 0;
    if (q > hi) q = hi;
    return q;
}

static int trunc_biased32(float x, float min, float id, int hi)
{
    float a = x - min;
    a = a * id;
    a = a + 0.5f;
    int q = (int)truncf(a);
    if (q < 0) q = 0;
    if (q > hi) q = hi;
    return q;
}

/* Round half away from zero as gguf's np_roundf. */
static float roundf_away(float n)
{
    float a = fabsf(n);
    float fl = floorf(a);
    float b = fl + floorf(2.0f * (a - fl));
    return n < 0 ? -b : b;
}

/* The ggml legacy-block quantizers as published by gguf-py (quants.py): used only to
 * build synthetic weights; the GPU and this oracle then consume the same bytes. */
int ora_quantize(int type, const float* src, uint8_t* dst, int64_t n)
{
    if (n % QK) return -1;
    for (int64_t b = 0; b < n / QK; b++) {
        const float* x = src + b * QK;
        int q[QK];
        switch (type) {
        case ORA_Q4_0: {
            uint8_t* p = dst + b * 18;
            float mx = signed_absmax(x);
            float d = mx / -8.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            for (int j = 0; j < QK; j++) q[j] = trunc_biased64(x[j], id, 8.5, 15);
            wr_half(p, d);
            for (int j = 0; j < 16; j++) p[2 + j] = (uint8_t)(q[j] | (q[16 + j] << 4));
            break;
        }
        case ORA_Q5_0: {
            uint8_t* p = dst + b * 22;
            float mx = signed_absmax(x);
            float d = mx / -16.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint32_t qh = 0;
            for (int j = 0; j < QK; j++) {
                q[j] = trunc_biased64(x[j], id, 16.5, 31);
                qh |= (uint32_t)((q[j] >> 4) & 1) << j;
            }
            wr_half(p, d);
            for (int k = 0; k < 4; k++) p[2 + k] = (uint8_t)(qh >> (8 * k));
            for (int j = 0; j < 16; j++) p[6 + j] = (uint8_t)((q[j] & 0x0F) | ((q[16 + j] & 0x0F) << 4));
            break;
        }
        case ORA_Q4_1:
        case ORA_Q5_1: {
            int five = type == ORA_Q5_1;
            uint8_t* p = dst + b * (five ? 24 : 20);
            float mx = x[0], mn = x[0];
            for (int j = 1; j < QK; j++) { if (x[j] > mx) mx = x[j]; if (x[j] < mn) mn = x[j]; }
            float d = (mx - mn) / (five ? 31.0f : 15.0f);
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint32_t qh = 0;
            for (int j = 0; j < QK; j++) {
                q[j] = trunc_biased32(x[j], mn, id, five ? 31 : 15);
                qh |= (uint32_t)((q[j] >> 4) & 1) << j;
            }
            wr_half(p, d);
            wr_half(p + 2, mn);
            uint8_t* qs = p + 4;
            if (five) {
                for (int k = 0; k < 4; k++) p[4 + k] = (uint8_t)(qh >> (8 * k));
                qs = p + 8;
            }
            for (int j = 0; j < 16; j++) qs[j] = (uint8_t)((q[j] & 0x0F) | ((q[16 + j] & 0x0F) << 4));
            break;
        }
        case ORA_Q8_0: {
            uint8_t* p = dst + b * 34;
            float amax = 0.0f;
            for (int j = 0; j < QK; j++) if (fabsf(x[j]) > amax) amax = fabsf(x[j]);
            float d = amax / 127.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            wr_half(p, d);
            for (int j = 0; j < QK; j++) p[2 + j] = (uint8_t)(int8_t)roundf_away(x[j] * id);
            break;
        }
        default:
            return -1;
        }
    }
    return 0;
}

/* ------------------------------------------------ activation quantization */

/* IntegerGemm.QuantizeActivations (IntegerGemm.cs:97-138): per 32 values
 * d = max|x|/127 (fp32, IEEE division), inv = d ≠ 0 ? 1/d : 0, q = RNE(x·inv)
 * (vcvtps2dq under the default rounding mode), s = Σq. */
/* vcvtps2dq, which Avx.ConvertToVector256Int32 is: round to nearest even (the default
 * MXCSR mode); NaN and anything outside the int32 range give 0x80000000. */
static inline int32_t cvtps2dq(float v)
{
    float r = nearbyintf(v);
    if (!(r >= -2147483648.0f && r < 2147483648.0f)) return INT32_MIN;
    return (int32_t)r;
}

/* IntegerGemm.QuantizeActivations (IntegerGemm.cs:97-138): max|x| per block, d = max/127,
 * inverse = 1/d (0 for an all-zero block), q = vcvtps2dq(x·inverse). The codes are the
 * int32 values packed with signed saturation (vpackssdw, vpacksswb) to [-128, 127]; the
 * block sum is the int32 sum of the unsaturated values, wrapping like Vector256<int> adds.
 * |q| <= 127 for every finite block whose inverse is finite; a block max below 3.7e-37
 * makes d so small that 1/d overflows to +inf, and then every value converts to
 * 0x80000000 (code -128). */
void ora_quantize_activations(const float* x, int64_t n, int8_t* q, float* d, int32_t* s)
{
    for (int64_t b = 0; b < n / QK; b++) {
        const float* xb = x + b * QK;
        float mx = 0.0f;
        for (int j = 0; j < QK; j++) mx = fmaxf(mx, fabsf(xb[j]));
        float dd = mx / 127.0f;
        float inv = dd != 0.0f ? 1.0f / dd : 0.0f;
        uint32_t sum = 0;
        for (int j = 0; j < QK; j++) {
            int32_t qi = cvtps2dq(xb[j] * inv);
            q[b * QK + j] = (int8_t)(qi < -128 ? -128 : qi > 127 ? 127 : qi);
            sum += (uint32_t)qi;
        }
        d[b] = dd;
        s[b] = (int32_t)sum;
    }
}

/* (int)float as .NET 9+ converts on every platform: saturating, NaN to 0. */
static inline int32_t dotnet_float_to_int(float v)
{
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

/* IntegerDot.QuantizeActivations (IntegerDot.cs:60-98): same d and inverse, but the
 * value rounds half away from zero, clamps to ±127, and the stored scale is fp16. */
void ora_quantize_activations_q8(const float* x, int64_t n, int8_t* q, float* d, int32_t* s)
{
    for (int64_t b = 0; b < n / QK; b++) {
        const float* xb = x + b * QK;
        float mx = 0.0f;
        for (int j = 0; j < QK; j++) { float a = fabsf(xb[j]); if (a > mx) mx = a; }
        float dd = mx / 127.0f;
        float inv = dd != 0.0f ? 1.0f / dd : 0.0f;
        int32_t sum = 0;
        for (int j = 0; j < QK; j++) {
            float v = xb[j] * inv;
            int qi = dotnet_float_to_int(roundf(v)); /* C roundf: half away from zero */
            if (qi < -127) qi = -127;
            if (qi > 127) qi = 127;
            q[b * QK + j] = (int8_t)qi;
            sum += qi;
        }
        d[b] = ora_half_to_float(ora_float_to_half(dd));
        s[b] = sum;
    }
}

/* ------------------------------------------------------------------ GEMM */

/* Unpacks one weight row to signed integer weights w = u − z (IntegerGemm.cs:75-81,
 * 258-329) plus per-block fp32 scale and offset (0 for the zero-point types). */
static int unpack_row(int type, const uint8_t* row, int blocks, int8_t* w, float* scale, float* offset)
{
    for (int b = 0; b < blocks; b++) {
        int8_t* wb = w + b * QK;
        switch (type) {
        case ORA_Q4_0: {
            const uint8_t* p = row + b * 18;
            scale[b] = rd_half(p); offset[b] = 0.0f;
            for (int j = 0; j < 16; j++) { wb[j] = (int8_t)((p[2 + j] & 0x0F) - 8); wb[16 + j] = (int8_t)((p[2 + j] >> 4) - 8); }
            break;
        }
        case ORA_Q4_1: {
            const uint8_t* p = row + b * 20;
            scale[b] = rd_half(p); offset[b] = rd_half(p + 2);
            for (int j = 0; j < 16; j++) { wb[j] = (int8_t)(p[4 + j] & 0x0F); wb[16 + j] = (int8_t)(p[4 + j] >> 4); }
            break;
        }
        case ORA_Q5_0: {
            const uint8_t* p = row + b * 22;
            uint32_t qh = rd_u32(p + 2);
            scale[b] = rd_half(p); offset[b] = 0.0f;
            for (int j = 0; j < 16; j++) {
                wb[j] = (int8_t)(((p[6 + j] & 0x0F) | (int)(((qh >> j) & 1u) << 4)) - 16);
                wb[16 + j] = (int8_t)(((p[6 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4)) - 16);
            }
            break;
        }
        case ORA_Q5_1: {
            const uint8_t* p = row + b * 24;
            uint32_t qh = rd_u32(p + 4);
            scale[b] = rd_half(p); offset[b] = rd_half(p + 2);
            for (int j = 0; j < 16; j++) {
                wb[j] = (int8_t)((p[8 + j] & 0x0F) | (int)(((qh >> j) & 1u) << 4));
                wb[16 + j] = (int8_t)((p[8 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4));
            }
            break;
        }
        case ORA_Q8_0: {
            const uint8_t* p = row + b * 34;
            scale[b] = rd_half(p); offset[b] = 0.0f;
            for (int j = 0; j < QK; j++) wb[j] = (int8_t)p[2 + j];
            break;
        }
        default:
            return -1;
        }
    }
    return 0;
}

static int has_offset(int type) { return type == ORA_Q4_1 || type == ORA_Q5_1; }

/* IntegerGemm.ZeroPoint (IntegerGemm.cs:75-81): the unsigned payload u = w + z. */
static int zero_point(int type)
{
    return type == ORA_Q4_0 ? 8 : type == ORA_Q5_0 ? 16 : type == ORA_Q8_0 ? 128 : 0;
}

/* The block sum as IntegerGemm forms it (IntegerGemm.cs:384-397): −z·Σa + Σ u·a in int32,
 * with Σa the quantizer's block sum (sum) and a the saturated codes. u·a products and
 * their sums are exact; the whole is taken modulo 2^32 like the vector adds. For every
 * block whose codes did not saturate, Σa equals Σ codes and this is Σ (u − z)·a. */
static inline int32_t block_dot(const int8_t* w, const int8_t* q, int z, int32_t sum)
{
    int32_t acc = 0, codes = 0;
    for (int k = 0; k < QK; k++) {
        acc += (int32_t)w[k] * (int32_t)q[k];
        codes += q[k];
    }
    /* Σ u·a = Σ (w + z)·a = acc + z·Σ codes */
    return (int32_t)((uint32_t)acc + (uint32_t)z * (uint32_t)codes - (uint32_t)z * (uint32_t)sum);
}

int ora_block_sums(int type, const uint8_t* w, int rows, int cols,
                   const int8_t* q, const int32_t* s, int tokens, int32_t* out)
{
    if (cols % QK) return -1;
    int z = zero_point(type);
    int blocks = cols / QK;
    int64_t rb = ora_row_bytes(type, cols);
    if (rb < 0) return -1;
    int8_t* wr = (int8_t*)malloc((size_t)cols);
    float* sc = (float*)malloc(sizeof(float) * (size_t)blocks);
    float* of = (float*)malloc(sizeof(float) * (size_t)blocks);
    int rc = 0;
    for (int r = 0; r < rows && rc == 0; r++) {
        rc = unpack_row(type, w + (int64_t)r * rb, blocks, wr, sc, of);
        for (int t = 0; t < tokens; t++)
            for (int b = 0; b < blocks; b++)
                out[((int64_t)t * rows + r) * blocks + b] =
                    block_dot(wr + b * QK, q + (int64_t)t * cols + b * QK, z, s[(int64_t)t * blocks + b]);
    }
    free(wr); free(sc); free(of);
    return rc;
}

/* The per-output epilogue of IntegerGemm.Multiply4/Multiply1 (IntegerGemm.cs:376-418,
 * 434-457): acc starts at 0; for b in order, acc = fma(float(I_b), RN(d_w·d_a), acc),
 * then for the offset types acc = fma(m_w, RN(d_a·float(Σq)), acc). */
int ora_matmul_q(int type, const uint8_t* w, int rows, int cols,
                 const int8_t* q, const float* d, const int32_t* s, int tokens,
                 const int32_t* row_ids, int n_ids, float* y, int threads)
{
    if (cols % QK) return -1;
    int blocks = cols / QK;
    int64_t rb = ora_row_bytes(type, cols);
    if (rb < 0) return -1;
    int out_rows = row_ids ? n_ids : rows;
    int off = has_offset(type), z = zero_point(type);
    int bad = 0;
    if (row_ids)
        for (int i = 0; i < n_ids; i++) if (row_ids[i] < 0 || row_ids[i] >= rows) bad = 1;
    if (bad) return -2;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
#endif
    {
        int8_t* wr = (int8_t*)malloc((size_t)cols);
        float* sc = (float*)malloc(sizeof(float) * (size_t)blocks);
        float* of = (float*)malloc(sizeof(float) * (size_t)blocks);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 8)
#endif
        for (int i = 0; i < out_rows; i++) {
            int r = row_ids ? row_ids[i] : i;
            unpack_row(type, w + (int64_t)r * rb, blocks, wr, sc, of);
            for (int t = 0; t < tokens; t++) {
                const int8_t* qt = q + (int64_t)t * cols;
                const float* dt = d + (int64_t)t * blocks;
                const int32_t* st = s + (int64_t)t * blocks;
                float acc = 0.0f;
                for (int b = 0; b < blocks; b++) {
                    int32_t I = block_dot(wr + b * QK, qt + b * QK, z, st[b]);
                    float scale = sc[b] * dt[b];
                    acc = fmaf((float)I, scale, acc);
                    if (off) acc = fmaf(of[b], dt[b] * (float)st[b], acc);
                }
                y[(int64_t)t * out_rows + i] = acc;
            }
        }
        free(wr); free(sc); free(of);
    }
    return 0;
}

int ora_matmul(int type, const uint8_t* w, int rows, int cols, const float* x, int tokens,
               const int32_t* row_ids, int n_ids, float* y, int semantics, int threads)
{
    if (cols % QK) return -1;
    int blocks = cols / QK;
    int8_t* q = (int8_t*)malloc((size_t)tokens * cols);
    float* d = (float*)malloc(sizeof(float) * (size_t)tokens * blocks);
    int32_t* s = (int32_t*)malloc(sizeof(int32_t) * (size_t)tokens * blocks);
    for (int t = 0; t < tokens; t++) {
        if (semantics == 1)
            ora_quantize_activations_q8(x + (int64_t)t * cols, cols, q + (int64_t)t * cols, d + (int64_t)t * blocks, s + (int64_t)t * blocks);
        else
            ora_quantize_activations(x + (int64_t)t * cols, cols, q + (int64_t)t * cols, d + (int64_t)t * blocks, s + (int64_t)t * blocks);
    }
    int rc = ora_matmul_q(type, w, rows, cols, q, d, s, tokens, row_ids, n_ids, y, threads);
    free(q); free(d); free(s);
    return rc;
}

int ora_gather_rows(int type, const uint8_t* table, int rows, int cols,
                    const int32_t* ids, int n, float* out)
{
    int64_t rb = ora_row_bytes(type, cols);
    if (rb < 0) return -1;
    for (int i = 0; i < n; i++) {
        if (ids[i] < 0 || ids[i] >= rows) return -2;
        if (type == ORA_F32) memcpy(out + (int64_t)i * cols, table + (int64_t)ids[i] * rb, (size_t)rb);
        else ora_dequantize(type, table + (int64_t)ids[i] * rb, out + (int64_t)i * cols, cols);
    }
    return 0;
}

/* ------------------------------------------------------------ elementwise */

/* Vector256<float>.Sum: Sum(lower128) + Sum(upper128), each pairwise. */
static inline float vsum8(const float a[8])
{
    return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
}

/* Kernels.RmsNorm (Kernels.cs:26-61) with Vector<float>.Count = 8: two interleaved
 * 8-lane float accumulators of x², summed to double; s = 1/sqrt((float)(Σ/n)+eps);
 * y = (x·s)·w. */
void ora_rmsnorm(const float* x, const float* w, float eps, int n, float* y)
{
    const int W = 8;
    double sum = 0.0;
    int i = 0;
    if (n >= 2 * W) {
        float even[8] = {0}, odd[8] = {0};
        for (; i + 2 * W <= n; i += 2 * W)
            for (int l = 0; l < W; l++) {
                float a = x[i + l], b = x[i + W + l];
                even[l] = even[l] + a * a;
                odd[l] = odd[l] + b * b;
            }
        sum = (double)vsum8(even) + (double)vsum8(odd);
    }
    for (; i < n; i++) sum += (double)x[i] * (double)x[i];
    float scale = 1.0f / sqrtf((float)(sum / n) + eps);
    for (i = 0; i < n; i++) y[i] = x[i] * scale * w[i];
}

/* e^x for TensorPrimitives.Exp/Sigmoid (Kernels.cs:88,120). The reference's vectorized
 * exp is a polynomial of its own; this restatement fixes one: Cody–Waite reduction
 * x = n·ln2 + r with ln2 split into a 16-bit head (so n·head is exact) and a tail,
 * the degree-7 Taylor polynomial of e^r in Horner form with fused multiply-adds, and
 * an exact scaling by 2^n. Every step is an IEEE single operation, so any
 * implementation that performs the same steps returns the same bits. < 1 ulp. */
float ora_expf(float x)
{
    if (x != x) return x;
    if (!(x > -104.0f)) return 0.0f;
    if (x > 0x1.62e42ep+6f) return INFINITY;         /* ln(FLT_MAX) rounded down */
    const float log2e = 0x1.715476p+0f;                /* RN(1/ln 2) */
    const float ln2_hi = 0x1.62e400p-1f;               /* ln 2 to 16 significant bits */
    const float ln2_lo = 0x1.7f7d1cp-20f;              /* RN(ln 2 − ln2_hi) */
    float n = nearbyintf(x * log2e);
    float r = fmaf(-n, ln2_hi, x);
    r = fmaf(-n, ln2_lo, r);
    float p = 0x1.a01a02p-13f;                         /* 1/7! */
    p = fmaf(p, r, 0x1.6c16c2p-10f);                   /* 1/6! */
    p = fmaf(p, r, 0x1.111112p-7f);                    /* 1/5! */
    p = fmaf(p, r, 0x1.555556p-5f);                    /* 1/4! */
    p = fmaf(p, r, 0x1.555556p-3f);                    /* 1/3! */
    p = fmaf(p, r, 0x1p-1f);
    p = fmaf(p, r, 0x1p+0f);
    p = fmaf(p, r, 0x1p+0f);
    return ldexpf(p, (int)n);
}

/* ora_expf over an array (lets a test sweep millions of arguments in one call). */
void ora_expf_n(const float* x, int64_t n, float* y)
{
    for (int64_t i = 0; i < n; i++) y[i] = ora_expf(x[i]);
}

/* Kernels.SwiGlu (Kernels.cs:83-90): up ← g·u; dst ← sigmoid(g); dst ← dst·up. */
void ora_swiglu(const float* gate, float* up, float* dst, int64_t n)
{
    for (int64_t i = 0; i < n; i++) {
        float g = gate[i];
        float gu = g * up[i];
        up[i] = gu;
        float sg = 1.0f / (1.0f + ora_expf(-g));
        dst[i] = sg * gu;
    }
}

/* Kernels.Softmax (Kernels.cs:103-122): max-shift, exp, divide by the sum; a row whose
 * max is not finite becomes uniform. */
void ora_softmax(float* x, int n)
{
    if (n == 0) return;
    float mx = x[0];
    for (int i = 1; i < n; i++) if (x[i] > mx || isnan(x[i])) mx = x[i];
    if (!isfinite(mx)) {
        for (int i = 0; i < n; i++) x[i] = 1.0f / (float)n;
        return;
    }
    float lanes[8] = {0};
    int i = 0;
    for (; i < n; i++) x[i] = ora_expf(x[i] - mx);
    for (i = 0; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) lanes[l] += x[i + l];
    float sum = vsum8(lanes);
    for (; i < n; i++) sum += x[i];
    for (i = 0; i < n; i++) x[i] = x[i] / sum;
}

/* Kernels.Dot4 (Kernels.cs:157-186): four 8-lane fused chains against one shared operand. */
void ora_dot4(const float* s, const float* a0, const float* a1, const float* a2,
              const float* a3, int n, float* r)
{
    float acc[4][8] = {{0}};
    const float* a[4] = {a0, a1, a2, a3};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int k = 0; k < 4; k++)
            for (int l = 0; l < 8; l++) acc[k][l] = fmaf(a[k][i + l], s[i + l], acc[k][l]);
    for (int k = 0; k < 4; k++) r[k] = vsum8(acc[k]);
    for (; i < n; i++)
        for (int k = 0; k < 4; k++) r[k] += a[k][i] * s[i];
}

/* Kernels.AddScaled4 (Kernels.cs:193-220): d_k = fma(src, w_k, d_k). */
void ora_add_scaled4(const float* src, float* d0, float* d1, float* d2, float* d3,
                     const float w[4], int n)
{
    float* d[4] = {d0, d1, d2, d3};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int k = 0; k < 4; k++)
            for (int l = 0; l < 8; l++) d[k][i + l] = fmaf(src[i + l], w[k], d[k][i + l]);
    for (; i < n; i++)
        for (int k = 0; k < 4; k++) d[k][i] += src[i] * w[k];
}

/* --------------------------------------------------------------- RoPE */

static float mscale_of(float scale, float m) { return scale <= 1.0f ? 1.0f : 0.1f * m * logf(scale) + 1.0f; }

/* Rope ctor, ComputeMagnitudeScale and YarnCorrectionDims (Rope.cs:33-106). */
void ora_rope_freqs(const ora_config* c, float* freqs, float* mscale)
{
    int dim = c->rope_dim, half = dim / 2;
    float freq_scale = 1.0f / c->rope_scale;
    if (!c->yarn_active) {
        for (int i = 0; i < half; i++)
            freqs[i] = freq_scale / powf(c->rope_theta, 2.0f * (float)i / (float)dim);
        *mscale = c->rope_attn_factor;
        return;
    }
    float low, high;
    if (c->yarn_beta_fast == 0.0f && c->yarn_beta_slow == 0.0f) {
        low = FLT_MAX;
        high = (float)dim / 2.0f - 1.0f;
    } else {
        const float PI = 3.14159265358979323846f;
        float cf = (float)dim * logf((float)c->rope_orig_ctx / (c->yarn_beta_fast * 2.0f * PI)) / (2.0f * logf(c->rope_theta));
        float cs = (float)dim * logf((float)c->rope_orig_ctx / (c->yarn_beta_slow * 2.0f * PI)) / (2.0f * logf(c->rope_theta));
        low = fmaxf(0.0f, floorf(cf));
        high = fminf((float)dim / 2.0f - 1.0f, ceilf(cs));
    }
    for (int i = 0; i < half; i++) {
        float extrapolated = 1.0f / powf(c->rope_theta, 2.0f * (float)i / (float)dim);
        float interpolated = freq_scale * extrapolated;
        float y = ((float)i - low) / fmaxf(0.001f, high - low);
        float cl = y < 0.0f ? 0.0f : (y > 1.0f ? 1.0f : y);
        float mix = (1.0f - cl) * c->yarn_ext_factor;
        freqs[i] = interpolated * (1.0f - mix) + extrapolated * mix;
    }
    float factor = c->rope_scale;
    float ms = c->yarn_mscale != 0.0f ? c->yarn_mscale : 1.0f;
    float ratio = c->yarn_mscale_all_dim != 0.0f
        ? mscale_of(factor, ms) / mscale_of(factor, c->yarn_mscale_all_dim)
        : mscale_of(factor, 1.0f);
    *mscale = ratio * c->rope_attn_factor;
}

/* Rope.Apply (Rope.cs:112-135): adjacent pairs, cos/sin of position·freq, times mscale. */
void ora_rope_apply(const float* freqs, float mscale, int rope_dim,
                    float* data, int heads, int head_dim, int position)
{
    int half = rope_dim / 2;
    float cs[512], sn[512];
    for (int i = 0; i < half; i++) {
        float theta = (float)position * freqs[i];
        cs[i] = cosf(theta) * mscale;
        sn[i] = sinf(theta) * mscale;
    }
    for (int h = 0; h < heads; h++) {
        float* hd = data + (int64_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            float x0 = hd[2 * i], x1 = hd[2 * i + 1];
            float a = x0 * cs[i], b = x1 * sn[i];
            float c = x0 * sn[i], e = x1 * cs[i];
            hd[2 * i] = a - b;
            hd[2 * i + 1] = c + e;
        }
    }
}

/* ------------------------------------------------------------------ model */

static void capture(ora_capture_fn fn, void* user, const char* name, const float* p, int r, int c)
{
    if (fn) fn(name, p, r, c, user);
}

static void matmul_into(int type, const uint8_t* w, int rows, int cols, const float* x, int tokens,
                        float* y, int threads)
{
    ora_matmul(type, w, rows, cols, x, tokens, NULL, 0, y, 0, threads);
}

/* MinistralModel.AttendGroup (MinistralModel.cs:372-440) for all kv heads and tokens. */
static void attention(const ora_config* c, const ora_kv* kv, int layer, const float* q, float* ctx,
                      int seq, int start, int threads)
{
    int heads = c->n_head, kvh = c->n_kv_head, hd = c->head_dim;
    int group = heads / kvh, qdim = heads * hd;
    int cache_len = start + seq;
    float scale = 1.0f / sqrtf((float)hd);
    int64_t per_head = (int64_t)kv->cap * hd;
    const float* kl = kv->k + (int64_t)layer * kvh * per_head;
    const float* vl = kv->v + (int64_t)layer * kvh * per_head;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
#endif
    {
        float* scores = (float*)malloc(sizeof(float) * 4 * (size_t)cache_len);
        float* spill = (float*)malloc(sizeof(float) * (size_t)hd);
#ifdef _OPENMP
#pragma omp for collapse(2) schedule(dynamic, 1)
#endif
        for (int g = 0; g < kvh; g++)
            for (int t = 0; t < seq; t++) {
                const float* keys = kl + (int64_t)g * per_head;
                const float* vals = vl + (int64_t)g * per_head;
                int limit = start + t + 1;
                const float* qrow = q + (int64_t)t * qdim;
                float* crow = ctx + (int64_t)t * qdim;
                for (int g0 = 0; g0 < group; g0 += 4) {
                    int live = group - g0 < 4 ? group - g0 : 4;
                    int first = g * group + g0;
                    const float* qh[4];
                    float* ch[4];
                    for (int k = 0; k < 4; k++) {
                        qh[k] = qrow + (int64_t)(first + (k < live ? k : 0)) * hd;
                        ch[k] = k < live ? crow + (int64_t)(first + k) * hd : spill;
                    }
                    float* sc[4] = {scores, scores + cache_len, scores + 2 * cache_len, scores + 3 * cache_len};
                    for (int p = 0; p < limit; p++) {
                        float r[4];
                        ora_dot4(keys + (int64_t)p * hd, qh[0], qh[1], qh[2], qh[3], hd, r);
                        for (int k = 0; k < 4; k++) sc[k][p] = r[k] * scale;
                    }
                    for (int k = 0; k < 4; k++) ora_softmax(sc[k], limit);
                    for (int k = 0; k < 4; k++) memset(ch[k], 0, sizeof(float) * (size_t)hd);
                    for (int p = 0; p < limit; p++) {
                        float wts[4] = {sc[0][p], sc[1][p], sc[2][p], sc[3][p]};
                        if (wts[0] == 0.0f && wts[1] == 0.0f && wts[2] == 0.0f && wts[3] == 0.0f) continue;
                        ora_add_scaled4(vals + (int64_t)p * hd, ch[0], ch[1], ch[2], ch[3], wts, hd);
                    }
                }
            }
        free(scores);
        free(spill);
    }
}

/* One pass of the layer loop body (MinistralModel.cs:216-237) over h[n][hidden] in
 * place, keys/values written at cache positions start..start+n-1. */
static void layer_forward(const ora_model* m, ora_kv* kv, int l, float* h, int n, int start,
                          const float* freqs, float mscale, ora_capture_fn cap, void* user, int threads)
{
    const ora_config* c = &m->cfg;
    int hidden = c->hidden, ff = c->ffn, hd = c->head_dim;
    int qdim = c->n_head * hd, kvdim = c->n_kv_head * hd;
    int64_t per_head = (int64_t)kv->cap * hd;
    float* norm = (float*)malloc(sizeof(float) * (size_t)n * hidden);
    float* blk = (float*)malloc(sizeof(float) * (size_t)n * hidden);
    float* qb = (float*)malloc(sizeof(float) * (size_t)n * qdim);
    float* ctx = (float*)malloc(sizeof(float) * (size_t)n * qdim);
    float* kvb = (float*)malloc(sizeof(float) * (size_t)n * kvdim);
    float* g = (float*)malloc(sizeof(float) * (size_t)n * ff);
    float* u = (float*)malloc(sizeof(float) * (size_t)n * ff);
    char name[64];
    const ora_layer* L = &m->layers[l];
    for (int t = 0; t < n; t++)
        ora_rmsnorm(h + (int64_t)t * hidden, L->attn_norm, c->eps, hidden, norm + (int64_t)t * hidden);
    snprintf(name, sizeof name, "blk.%d.attn_norm", l); capture(cap, user, name, norm, n, hidden);

    /* AttentionAsync (MinistralModel.cs:282-354) */
    matmul_into(L->type_q, L->q, qdim, hidden, norm, n, qb, threads);
    for (int t = 0; t < n; t++) {
        int pos = start + t;
        float* row = qb + (int64_t)t * qdim;
        ora_rope_apply(freqs, mscale, c->rope_dim, row, c->n_head, hd, pos);
        if (c->rope_orig_ctx > 0 && c->attn_temperature != 0.0f) {
            float interval = floorf((float)pos / (float)c->rope_orig_ctx);
            if (interval != 0.0f) {
                float sc = 1.0f + c->attn_temperature * logf(1.0f + interval);
                for (int i = 0; i < qdim; i++) row[i] = row[i] * sc;
            }
        }
    }
    snprintf(name, sizeof name, "blk.%d.q_rope", l); capture(cap, user, name, qb, n, qdim);

    matmul_into(L->type_k, L->k, kvdim, hidden, norm, n, kvb, threads);
    for (int t = 0; t < n; t++) {
        float* row = kvb + (int64_t)t * kvdim;
        ora_rope_apply(freqs, mscale, c->rope_dim, row, c->n_kv_head, hd, start + t);
        for (int kh = 0; kh < c->n_kv_head; kh++)
            memcpy(kv->k + ((int64_t)l * c->n_kv_head + kh) * per_head + (int64_t)(start + t) * hd,
                   row + (int64_t)kh * hd, sizeof(float) * (size_t)hd);
    }
    snprintf(name, sizeof name, "blk.%d.k_rope", l); capture(cap, user, name, kvb, n, kvdim);

    matmul_into(L->type_v, L->v, kvdim, hidden, norm, n, kvb, threads);
    for (int t = 0; t < n; t++)
        for (int kh = 0; kh < c->n_kv_head; kh++)
            memcpy(kv->v + ((int64_t)l * c->n_kv_head + kh) * per_head + (int64_t)(start + t) * hd,
                   kvb + (int64_t)t * kvdim + (int64_t)kh * hd, sizeof(float) * (size_t)hd);
    snprintf(name, sizeof name, "blk.%d.v", l); capture(cap, user, name, kvb, n, kvdim);

    attention(c, kv, l, qb, ctx, n, start, threads);
    snprintf(name, sizeof name, "blk.%d.attn_weighted", l); capture(cap, user, name, ctx, n, qdim);
    matmul_into(L->type_o, L->o, hidden, qdim, ctx, n, blk, threads);
    snprintf(name, sizeof name, "blk.%d.attn_out", l); capture(cap, user, name, blk, n, hidden);

    for (int64_t i = 0; i < (int64_t)n * hidden; i++) h[i] = h[i] + blk[i];
    snprintf(name, sizeof name, "blk.%d.post_attn", l); capture(cap, user, name, h, n, hidden);

    for (int t = 0; t < n; t++)
        ora_rmsnorm(h + (int64_t)t * hidden, L->ffn_norm, c->eps, hidden, norm + (int64_t)t * hidden);
    snprintf(name, sizeof name, "blk.%d.ffn_norm", l); capture(cap, user, name, norm, n, hidden);

    matmul_into(L->type_gate, L->gate, ff, hidden, norm, n, g, threads);
    matmul_into(L->type_up, L->up, ff, hidden, norm, n, u, threads);
    ora_swiglu(g, u, g, (int64_t)n * ff);
    matmul_into(L->type_down, L->down, hidden, ff, g, n, blk, threads);
    snprintf(name, sizeof name, "blk.%d.ffn_out", l); capture(cap, user, name, blk, n, hidden);

    for (int64_t i = 0; i < (int64_t)n * hidden; i++) h[i] = h[i] + blk[i];
    snprintf(name, sizeof name, "blk.%d.output", l); capture(cap, user, name, h, n, hidden);
    free(norm); free(blk); free(qb); free(ctx); free(kvb); free(g); free(u);
}

int ora_forward(const ora_model* m, ora_kv* kv, const int32_t* tokens, int n,
                int head_mode, const int32_t* vocab_ids, int n_ids, float* logits,
                ora_capture_fn cap, void* user, int threads)
{
    const ora_config* c = &m->cfg;
    if (n <= 0) return -1;
    int start = kv->len;
    if (start + n > kv->cap) return -3;
    int hidden = c->hidden;
    float* h = (float*)malloc(sizeof(float) * (size_t)n * hidden);
    float* norm = (float*)malloc(sizeof(float) * (size_t)hidden);
    float freqs[512], mscale;
    int rc = 0;
    ora_rope_freqs(c, freqs, &mscale);

    if (ora_gather_rows(m->embd_type, m->token_embd, c->vocab, hidden, tokens, n, h)) { rc = -2; goto done; }
    capture(cap, user, "embeddings", h, n, hidden);
    for (int l = 0; l < c->n_layer; l++)
        layer_forward(m, kv, l, h, n, start, freqs, mscale, cap, user, threads);
    kv->len = start + n;
    if (head_mode == 0) goto done;

    ora_rmsnorm(h + (int64_t)(n - 1) * hidden, m->output_norm, c->eps, hidden, norm);
    capture(cap, user, "final_norm", norm, 1, hidden);
    if (head_mode == 1) {
        rc = ora_matmul(m->embd_type, m->token_embd, c->vocab, hidden, norm, 1, vocab_ids, n_ids, logits, 0, threads);
    } else {
        rc = ora_matmul(m->embd_type, m->token_embd, c->vocab, hidden, norm, 1, NULL, 0, logits, 0, threads);
        capture(cap, user, "logits", logits, 1, c->vocab);
    }
done:
    free(h); free(norm);
    return rc;
}

int ora_layer_forward(const ora_model* m, ora_kv* kv, int layer, const float* x, int n, float* y, int threads)
{
    if (n <= 0 || layer < 0 || layer >= m->cfg.n_layer || n > kv->cap) return -1;
    float freqs[512], mscale;
    ora_rope_freqs(&m->cfg, freqs, &mscale);
    memcpy(y, x, sizeof(float) * (size_t)n * m->cfg.hidden);
    layer_forward(m, kv, layer, y, n, 0, freqs, mscale, NULL, NULL, threads);
    return 0;
}

/* ShieldstralModerator.Score (ShieldstralModerator.cs:348-364). */
void ora_score(const float* logits, int n_yes, int n_no, float* score, float* yes, float* no)
{
    float y = -INFINITY, n = -INFINITY;
    for (int i = 0; i < n_yes; i++) if (logits[i] > y) y = logits[i];
    for (int i = 0; i < n_no; i++) if (logits[n_yes + i] > n) n = logits[n_yes + i];
    float mx = fmaxf(y, n);
    float ey = expf(y - mx), en = expf(n - mx);
    *score = ey / (ey + en);
    *yes = y;
    *no = n;
}
