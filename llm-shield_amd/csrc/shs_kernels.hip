// gfx950 kernels of the Shieldstral prefill path. Device layouts: shs_kernels.h.
//
// Numerics follow the reference bit for bit where it is integer or a single IEEE op:
// activation quantization (IntegerGemm.cs:97-138), the exact int32 block sums and the
// serial per-block epilogue acc = fma(float(I_b), RN(d_w·d_a), acc) (IntegerGemm.cs:
// 376-418), RMSNorm's accumulation order (Kernels.cs:26-61) and RoPE's rotation
// (Rope.cs:112-135). The file is compiled with -ffp-contract=off; every fma is explicit.
#include "shs_kernels.h"
#include <atomic>
#include <algorithm>
#include <mutex>
#include <type_traits>

#include <math.h>

namespace shs {

// A kernel's dynamic LDS beyond 64 KB must be allowed with hipFuncSetAttribute, which HIP keeps
// per device. One LdsLimit per kernel remembers the largest size allowed on each device, so the
// call is made once per size increase; handles on several host threads may launch at once (a
// lock-free check, then the raise under a mutex, always to the largest size asked so far).
struct LdsLimit {
    static constexpr int MAX_DEVICES = 16;
    std::atomic<size_t> allowed[MAX_DEVICES] = {};
    std::mutex mu;
    hipError_t raise(const void* fn, size_t bytes)
    {
        if (bytes <= (64u << 10)) return hipSuccess;
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        std::atomic<size_t>* a = dev >= 0 && dev < MAX_DEVICES ? &allowed[dev] : nullptr;
        if (a && a->load(std::memory_order_acquire) >= bytes) return hipSuccess;
        std::lock_guard<std::mutex> lock(mu);
        const size_t target = a ? std::max(bytes, a->load(std::memory_order_relaxed)) : bytes;
        e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)target);
        if (e == hipSuccess && a) a->store(target, std::memory_order_release);
        return e;
    }
};

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef float v4f __attribute__((ext_vector_type(4)));

int qs_bytes(int type) { return type == SHS_TYPE_Q8_0 ? 32 : 16; }
bool type_supported(int t) { return t == 2 || t == 3 || t == 6 || t == 7 || t == 8; }
bool type_has_offset(int t) { return t == 3 || t == 7; }
bool type_has_qh(int t) { return t == 6 || t == 7; }

// Exact fp16 → fp32 for every bit pattern (IntegerGemm.HalfToSingle, IntegerGemm.cs:235-245).
__device__ inline float half_bits_to_float(uint32_t h)
{
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0u);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    return __uint_as_float(bits);
}

// fp32 → fp16 → fp32 with round-to-nearest-even (the Half cast of IntegerDot.cs:82).
__device__ inline float round_to_half(float f)
{
    return (float)(_Float16)f;
}

template <int TYPE> struct BlockFmt;
template <> struct BlockFmt<SHS_TYPE_Q4_0> { static constexpr int TS = 18, QS = 2, QH = -1, M = -1; };
template <> struct BlockFmt<SHS_TYPE_Q4_1> { static constexpr int TS = 20, QS = 4, QH = -1, M = 2; };
template <> struct BlockFmt<SHS_TYPE_Q5_0> { static constexpr int TS = 22, QS = 6, QH = 2, M = -1; };
template <> struct BlockFmt<SHS_TYPE_Q5_1> { static constexpr int TS = 24, QS = 8, QH = 4, M = 2; };
template <> struct BlockFmt<SHS_TYPE_Q8_0> { static constexpr int TS = 34, QS = 2, QH = -1, M = -1; };

// Position p of a stored 32-byte block → quant element index: [0..7, 16..23, 8..15, 24..31].
__host__ __device__ inline int perm_elem(int p) { return p < 8 ? p : p < 16 ? p + 8 : p < 24 ? p - 8 : p; }

// ------------------------------------------------------------------ repack

template <int TYPE>
__global__ void k_repack(const uint8_t* __restrict__ native, int row0, int nrows, int B,
                         uint8_t* __restrict__ qs, uint32_t* __restrict__ qh, float* __restrict__ d,
                         float* __restrict__ m)
{
    typedef BlockFmt<TYPE> F;
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)nrows * B) return;
    int rr = (int)(idx / B), b = (int)(idx % B);
    int r = row0 + rr;
    const uint8_t* blk = native + idx * F::TS;
    int64_t rec = (int64_t)(r >> 5) * B + b;
    int ri = r & 31;
    d[rec * 32 + ri] = half_bits_to_float(blk[0] | (blk[1] << 8));
    if (F::M >= 0) m[rec * 32 + ri] = half_bits_to_float(blk[F::M] | (blk[F::M + 1] << 8));
    if (F::QH >= 0)
        qh[rec * 32 + ri] = (uint32_t)blk[F::QH] | ((uint32_t)blk[F::QH + 1] << 8) |
                            ((uint32_t)blk[F::QH + 2] << 16) | ((uint32_t)blk[F::QH + 3] << 24);
    if (TYPE == SHS_TYPE_Q8_0) {
        uint8_t* dst = qs + rec * 1024 + ri * 32;
        for (int p = 0; p < 32; p++) dst[p] = blk[F::QS + perm_elem(p)];
    } else {
        uint8_t* dst = qs + rec * 512 + ri * 16;
        for (int p = 0; p < 16; p++) dst[p] = blk[F::QS + p];
    }
}

hipError_t launch_repack(const DevMatrix& w, const uint8_t* native, int row0, int nrows, hipStream_t s)
{
    int64_t n = (int64_t)nrows * w.blocks;
    dim3 grid((unsigned)((n + 255) / 256)), block(256);
    switch (w.type) {
    case SHS_TYPE_Q4_0: hipLaunchKernelGGL(k_repack<SHS_TYPE_Q4_0>, grid, block, 0, s, native, row0, nrows, w.blocks, w.qs, w.qh, w.d, w.m); break;
    case SHS_TYPE_Q4_1: hipLaunchKernelGGL(k_repack<SHS_TYPE_Q4_1>, grid, block, 0, s, native, row0, nrows, w.blocks, w.qs, w.qh, w.d, w.m); break;
    case SHS_TYPE_Q5_0: hipLaunchKernelGGL(k_repack<SHS_TYPE_Q5_0>, grid, block, 0, s, native, row0, nrows, w.blocks, w.qs, w.qh, w.d, w.m); break;
    case SHS_TYPE_Q5_1: hipLaunchKernelGGL(k_repack<SHS_TYPE_Q5_1>, grid, block, 0, s, native, row0, nrows, w.blocks, w.qs, w.qh, w.d, w.m); break;
    case SHS_TYPE_Q8_0: hipLaunchKernelGGL(k_repack<SHS_TYPE_Q8_0>, grid, block, 0, s, native, row0, nrows, w.blocks, w.qs, w.qh, w.d, w.m); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------- activation quantization

// fp16 bit pattern of a small integer (|v| ≤ 2048: exact).
__device__ __forceinline__ uint32_t half_bits(int v)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)v);
}

// The B column of the conversion MFMA for a block with code sum Σq (|Σq| ≤ 32·127):
// fp16 (−6144, −hi, −lo, 0) with Σq = 64·hi + lo, 0 ≤ lo < 64, so |hi| ≤ 64 — every
// entry an exact fp16 integer. Against the A row (2048, 64z, z, 0) it sums to
// −(1.5·2^23 + z·Σq).
// vcvtps2dq, the conversion IntegerGemm.QuantizeActivations uses: round to nearest even;
// NaN and values outside the int32 range give 0x80000000 (v_cvt_i32_f32 alone would
// saturate instead).
__device__ __forceinline__ int cvt_rne_x86(float v)
{
    const float r = __builtin_rintf(v);
    return __builtin_fabsf(r) < 2147483648.0f ? (int)r : (int)0x80000000;
}

// The code a converted value packs to (vpackssdw + vpacksswb: signed saturation).
__device__ __forceinline__ uint32_t code_byte(int q)
{
    return (uint32_t)(min(127, max(-128, q)) & 0xFF);
}

// Σq as the zero-point correction takes it, modulo 2^31: a block whose 1/d overflowed has
// converted values of 0x80000000, and z·2^31 ≡ 0 (mod 2^32) for every even zero point z,
// so IntegerGemm's −z·Σq + Σ u·q is unchanged. What is left lies within ±32·127.
__device__ __forceinline__ int correction_sum(int sum)
{
    return (sum > 4096 || sum < -4096) ? (sum ^ (int)0x80000000) : sum;
}

__device__ __forceinline__ uint2 conversion_operand(int sum)
{
    sum = correction_sum(sum);
    const int hi = sum >> 6, lo = sum - 64 * hi;
    return make_uint2(half_bits(-6144) | (half_bits(-hi) << 16), half_bits(-lo));
}

// Byte offset of element group 4·l8..4·l8+3 of (token t, block b) in the code array: half
// h = (l8 >> 1) & 1 holds elements [8h..8h+7, 16+8h..16+8h+7] of each token.
__device__ __forceinline__ int64_t act_code_offset(const ActQ8& a, int t, int b, int l8)
{
    const int h = (l8 >> 1) & 1;
    const int idx = 4 * (l8 & 1) + 8 * (l8 >> 2);
    return ((((int64_t)(t >> 5) * a.B + b) * 2 + h) * 32 + (t & 31)) * 16 + idx;
}

// Lane exchanges on the DPP path (an operand modifier of a VALU instruction, no LDS round
// trip as __shfl takes), for reductions over aligned lane groups: quad_perm [1,0,3,2] swaps
// neighbours (xor 1), [2,3,0,1] swaps pairs (xor 2), row_half_mirror maps lane i of an
// 8-lane group to 7 − i and row_mirror lane i of a 16-lane row to 15 − i. After the two quad
// steps of a reduction every lane of a quad holds the same value, so the mirrors then pair
// quads like xor 4 and xor 8 would.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}

__device__ __forceinline__ float readlane_f(float v, int lane)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// max over the 64 lanes of a wave (NaN lanes are ignored, as fmaxf does), in every lane
__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

__device__ __forceinline__ int wave_or(int v)
{
    v |= dpp_i<DPP_XOR1>(v);
    v |= dpp_i<DPP_XOR2>(v);
    v |= dpp_i<DPP_HALF_MIRROR>(v);
    v |= dpp_i<DPP_MIRROR>(v);
    return __builtin_amdgcn_readlane(v, 0) | __builtin_amdgcn_readlane(v, 16) | __builtin_amdgcn_readlane(v, 32) |
           __builtin_amdgcn_readlane(v, 48);
}

// vsum8's ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)) of an aligned 8-lane group holding a_t in
// lane t, in every lane of the group (each addition is commutative, so the lanes agree)
__device__ __forceinline__ float vsum8_lanes(float v)
{
    v = v + dpp_f<DPP_XOR1>(v);
    v = v + dpp_f<DPP_XOR2>(v);
    return v + dpp_f<DPP_HALF_MIRROR>(v);
}

// One 32-value block: IntegerGemm.QuantizeActivations (semantics 0: d = max|x|/127,
// q = RNE(x·(1/d)), IntegerGemm.cs:97-138) or IntegerDot.QuantizeActivations (1: q rounded
// half away from zero and clamped to ±127, d rounded to fp16, IntegerDot.cs:60-98); d and
// 1/d are IEEE (correctly rounded division is on for this file), d = 0 gives q = 0. Also
// float(Σq) and d·Σq, the offset types' second epilogue factor. The 8 lanes of an aligned
// lane group (l8 = lane % 8) hold elements 4·l8 .. 4·l8+3; max and Σq are exact in any
// order, so the group reductions are order-free. Each lane stores its 4 int8 codes.
// The quantization of one block, without its stores: the lane's 4 codes packed in a word,
// the block's d (as stored) and Σq (both the same in every lane of the group).
struct QBlock {
    uint32_t w;
    float d;
    int sum;
};

__device__ __forceinline__ QBlock quant_block8_values(float4 v, int semantics)
{
    float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    mx = fmaxf(mx, dpp_f<DPP_XOR1>(mx));
    mx = fmaxf(mx, dpp_f<DPP_XOR2>(mx));
    mx = fmaxf(mx, dpp_f<DPP_HALF_MIRROR>(mx));
    const float d = mx / 127.0f;
    const float inv = d != 0.0f ? 1.0f / d : 0.0f;
    int q0, q1, q2, q3;
    float dd;
    if (semantics == 0) {
        q0 = cvt_rne_x86(v.x * inv);
        q1 = cvt_rne_x86(v.y * inv);
        q2 = cvt_rne_x86(v.z * inv);
        q3 = cvt_rne_x86(v.w * inv);
        dd = d;
    } else {
        q0 = min(127, max(-127, (int)roundf(v.x * inv)));
        q1 = min(127, max(-127, (int)roundf(v.y * inv)));
        q2 = min(127, max(-127, (int)roundf(v.z * inv)));
        q3 = min(127, max(-127, (int)roundf(v.w * inv)));
        dd = round_to_half(d);
    }
    int sum = (q0 + q1) + (q2 + q3);
    sum += dpp_i<DPP_XOR1>(sum);
    sum += dpp_i<DPP_XOR2>(sum);
    sum += dpp_i<DPP_HALF_MIRROR>(sum);
    const uint32_t w = code_byte(q0) | (code_byte(q1) << 8) | (code_byte(q2) << 16) | (code_byte(q3) << 24);
    return QBlock{w, dd, sum};
}

__device__ __forceinline__ void quant_block8(float4 v, int l8, const ActQ8& a, int t, int b, int semantics)
{
    const QBlock qb = quant_block8_values(v, semantics);
    *reinterpret_cast<uint32_t*>(a.q + act_code_offset(a, t, b, l8)) = qb.w;
    if (l8 == 0) {
        a.d[(int64_t)b * a.Tpad + t] = qb.d;
        a.cv[(int64_t)b * a.Tpad + t] = conversion_operand(qb.sum);
        a.ds[(int64_t)b * a.Tpad + t] = qb.d * (float)qb.sum;
    }
}

__device__ __forceinline__ void zero_block8(int l8, const ActQ8& a, int t, int b)
{
    *reinterpret_cast<uint32_t*>(a.q + act_code_offset(a, t, b, l8)) = 0u;
    if (l8 == 0) {
        a.d[(int64_t)b * a.Tpad + t] = 0.0f;
        a.cv[(int64_t)b * a.Tpad + t] = conversion_operand(0);
        a.ds[(int64_t)b * a.Tpad + t] = 0.0f;
    }
}

// IntegerGemm.QuantizeActivations over x[T × K] (semantics 0) or IntegerDot's variant (1):
// 8 lanes per 32-block, blocks of a token row adjacent across lane groups (coalesced).
__global__ __launch_bounds__(256) void k_quant_act(const float* __restrict__ x, int ldx, ActQ8 a, int semantics,
                                                   bool vec)
{
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t g = idx >> 3;
    const int l8 = (int)(idx & 7);
    if (g >= (int64_t)a.Tpad * a.B) return;
    const int b = (int)(g % a.B), t = (int)(g / a.B);
    if (t >= a.T) {
        zero_block8(l8, a, t, b);
        return;
    }
    const float* src = x + (int64_t)t * ldx + 32 * b + 4 * l8;
    const float4 v = vec ? *reinterpret_cast<const float4*>(src) : make_float4(src[0], src[1], src[2], src[3]);
    quant_block8(v, l8, a, t, b, semantics);
}

hipError_t launch_quant_act(const float* x, int ldx, const ActQ8& a, int semantics, hipStream_t s)
{
    const int64_t n = (int64_t)a.Tpad * a.B * 8;
    const bool vec = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && ((ldx & 3) == 0);
    hipLaunchKernelGGL(k_quant_act, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, ldx, a, semantics, vec);
    return hipGetLastError();
}

// ------------------------------------------------------- RMSNorm + quantize

__device__ inline float vsum8(const float* a)
{
    return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
}

// A work-group barrier that waits only for this wave's LDS operations, whatever else is
// outstanding: global loads in flight (a caller's prefetched weights) stay in flight. The
// fence of __syncthreads() also waits for every vector-memory operation once the wave has
// generic (flat) accesses outstanding. Only LDS data may be handed between waves across it.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Kernels.RmsNorm (Kernels.cs:26-61) in its own order — 16 running float sums of x²
// (8 "even" lanes, 8 "odd" lanes of Vector<float>), each pairwise-summed and widened to
// double — followed by y = (x·s)·w, handed 4 elements at a time to `sink(v, l8, b)` (the
// lanes l8 = 0..7 of an aligned group hold block b's elements 4·l8 .. 4·l8+3): token row xr,
// by a whole block of 256 threads. LDS: sx holds 2n floats (the row, then its squares),
// part 16 floats and s_scale one. The next use of sx must be preceded by a barrier.
// `issue()` runs right after the row's loads are issued and before they are used: loads it
// issues stay in flight through the normalization (global loads complete in issue order, and
// its barriers wait for the LDS only).
template <class Sink, class Issue>
__device__ __forceinline__ void rmsnorm_rows(const float* __restrict__ xr, const float* __restrict__ w, float eps,
                                             int n, float* sx, float* part, float* s_scale, Sink&& sink,
                                             Issue&& issue)
{
    const int tid = threadIdx.x;
    float* sq = sx + n;
    // the gains this thread's 8-lane group applies (blocks tid/8 + 32i, 4 elements each),
    // loaded now so their latency overlaps the row's
    constexpr int WPRE = 4;
    float4 wpre[WPRE];
    const int l8 = tid & 7;
#pragma unroll
    for (int i = 0; i < WPRE; i++) {
        const int b = (tid >> 3) + (256 >> 3) * i;
        wpre[i] = b < n / 32 ? *reinterpret_cast<const float4*>(w + 32 * b + 4 * l8) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (((reinterpret_cast<uintptr_t>(xr) & 15) == 0) && (n & 3) == 0 && n >= 4) {
        // float4 row copy: a thread's first RPRE loads issued together (unconditionally, a
        // load past the row re-reading its last float4, so no branch separates them), then
        // issue(), then the copies and the squares x·x (rounded, as the reference's running
        // sums add them); a longer row's remaining float4s load and store one by one
        constexpr int RPRE = 4;
        float4 rv[RPRE];
#pragma unroll
        for (int k = 0; k < RPRE; k++) {
            const int i = tid + 256 * k;
            rv[k] = reinterpret_cast<const float4*>(xr)[i < n / 4 ? i : n / 4 - 1];
        }
        asm volatile("" ::: "memory");
        issue();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < RPRE; k++) {
            const int i = tid + 256 * k;
            if (i < n / 4) {
                const float4 v = rv[k];
                reinterpret_cast<float4*>(sx)[i] = v;
                reinterpret_cast<float4*>(sq)[i] = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
            }
        }
        for (int i = tid + 256 * RPRE; i < n / 4; i += 256) {
            const float4 v = reinterpret_cast<const float4*>(xr)[i];
            reinterpret_cast<float4*>(sx)[i] = v;
            reinterpret_cast<float4*>(sq)[i] = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
        }
    } else {
        issue();
        for (int i = tid; i < n; i += 256) {
            const float v = xr[i];
            sx[i] = v;
            sq[i] = v * v;
        }
    }
    lds_barrier();
    if (tid < 16) {
        // lane tid's running sum over elements tid + 16k in order; the reads of 16 steps are
        // issued together into one of two register sets, the next 16 (kept ahead by an empty
        // asm that takes acc) before the current 16 adds, which stay one chain
        float acc = 0.0f;
        const int nk = n / 16;
        const int kfull = nk & ~15;
        int k = 0;
        float va[16], vb[16];
#define SHS_SQ_LOAD(V, K0)                                                        \
    {                                                                             \
        _Pragma("unroll") for (int q = 0; q < 16; q++) V[q] = sq[((K0) + q) * 16 + tid]; \
        asm volatile("" : "+v"(acc)::"memory");                                   \
    }
#define SHS_SQ_RUN(V)                                                             \
    {                                                                             \
        _Pragma("unroll") for (int q = 0; q < 16; q++) acc = acc + V[q];          \
        asm volatile("" : "+v"(acc)::"memory");                                   \
    }
        if (kfull > 0) {
            SHS_SQ_LOAD(va, 0);
            for (; k + 32 <= kfull; k += 32) {
                SHS_SQ_LOAD(vb, k + 16);
                SHS_SQ_RUN(va);
                SHS_SQ_LOAD(va, k + 48 <= kfull ? k + 32 : k);  // past the last group: unused
                SHS_SQ_RUN(vb);
            }
            if (k < kfull) {
                SHS_SQ_RUN(va);
                k += 16;
            }
        }
#undef SHS_SQ_LOAD
#undef SHS_SQ_RUN
        for (; k < nk; k++) acc = acc + sq[k * 16 + tid];
        part[tid] = acc;
    }
    lds_barrier();
    if (tid == 0) {
        double sum = 0.0;
        int i = 0;
        if (n >= 16) {
            sum = (double)vsum8(part) + (double)vsum8(part + 8);
            i = n / 16 * 16;
        }
        for (; i < n; i++) sum += (double)sx[i] * (double)sx[i];
        *s_scale = 1.0f / sqrtf((float)(sum / n) + eps);
    }
    lds_barrier();
    const float sc = *s_scale;
    int i = 0;
    for (int b = tid >> 3; b < n / 32; b += 256 >> 3, i++) {  // uniform per 8-lane group
        const int e = 32 * b + 4 * l8;
        const float4 xv = *reinterpret_cast<const float4*>(sx + e);
        float4 wv;
        if (i < WPRE) {
            // (a register array read with a runtime index would go to scratch: select instead)
            wv = i == 0 ? wpre[0] : i == 1 ? wpre[1] : i == 2 ? wpre[2] : wpre[3];
        } else {
            wv = *reinterpret_cast<const float4*>(w + e);
        }
        float4 v;
        v.x = (xv.x * sc) * wv.x;
        v.y = (xv.y * sc) * wv.y;
        v.z = (xv.z * sc) * wv.z;
        v.w = (xv.w * sc) * wv.w;
        sink(v, l8, b);
    }
}

// RMSNorm + quantization of one token row per 256 threads, ROWS rows per block (padding
// tokens get zero codes): Kernels.RmsNorm's arithmetic as rmsnorm_rows states it, laid out for
// a whole row at once. Four rows per block where their LDS fits, rather than one: the
// launch's cost grows with its work-group count (1024 one-row blocks took 14.1 µs, 256
// four-row blocks 12.4 µs, same bits).
//  * The row's float4s are loaded once; x goes to the LDS row-major and x·x transposed as
//    sq[s][k] = x²[s + 16k] (rows padded to a multiple of 4 floats plus 4, so the 16 chain
//    lanes' float4 reads fall in distinct banks).
//  * Lane s < 16 runs running sum s over k = 0, 1, … in order, reading 4 steps per LDS load,
//    16 steps ahead of its adds.
//  * Thread p = 2b + h quantizes half h of block b: elements 8h..8h+7 and 16+8h..16+8h+7,
//    exactly the 16 code bytes the GEMM's lane half h multiplies, written as one 16-byte
//    store. The block's max and Σq combine over the lane pair (exact in any order), then
//    d = max/127, 1/d and the codes follow IntegerGemm.QuantizeActivations as quant_block8.
constexpr int RMS_SQ_PAD = 4;
__device__ __forceinline__ int rms_sq_ld(int n) { return (((n >> 4) + 3) & ~3) + RMS_SQ_PAD; }

template <int ROWS>
__global__ __launch_bounds__(256 * ROWS) void k_rmsnorm_quant(const float* __restrict__ x, int ldx,
                                                              const float* __restrict__ w, float eps, int n,
                                                              ActQ8 a, float* __restrict__ y_opt)
{
    extern __shared__ float sx_all[];  // per row: the row, then the transposed squares
    __shared__ float part_all[ROWS][16];
    __shared__ float s_scale_all[ROWS];
    const int rr = threadIdx.x >> 8, tid = threadIdx.x & 255;  // row of the block, thread of the row
    const int t = blockIdx.x * ROWS + rr;
    // a padding row's threads write zero codes and skip the work, but meet every barrier
    const bool live = t < a.T;
    if (!live) {
        for (int b = tid >> 3; b < a.B; b += 256 >> 3) zero_block8(tid & 7, a, t, b);
    }
    const int nk = n >> 4, ld = rms_sq_ld(n), npair = n >> 4;
    float* sx = sx_all + (int64_t)rr * (n + 16 * ld);
    float* part = part_all[rr];
    float& s_scale = s_scale_all[rr];
    float* sq = sx + n;
    const float* xr = x + (int64_t)(live ? t : 0) * ldx;
    // the gains of this thread's first pair, loaded now so their latency overlaps the row's
    float4 wpre[4];
    if (live && tid < npair) {
        const float* wp = w + 32 * (tid >> 1) + 8 * (tid & 1);
        wpre[0] = *reinterpret_cast<const float4*>(wp);
        wpre[1] = *reinterpret_cast<const float4*>(wp + 4);
        wpre[2] = *reinterpret_cast<const float4*>(wp + 16);
        wpre[3] = *reinterpret_cast<const float4*>(wp + 20);
    }
    const bool vec = ((reinterpret_cast<uintptr_t>(xr) & 15) == 0) && (ldx & 3) == 0;
    for (int i = tid; live && i < n / 4; i += 256) {
        const float4 v = vec ? reinterpret_cast<const float4*>(xr)[i]
                             : make_float4(xr[4 * i], xr[4 * i + 1], xr[4 * i + 2], xr[4 * i + 3]);
        reinterpret_cast<float4*>(sx)[i] = v;
        // elements 4i + c: running sum s = 4(i & 3) + c, step k = i >> 2
        float* d = sq + 4 * (i & 3) * ld + (i >> 2);
        d[0] = v.x * v.x;
        d[ld] = v.y * v.y;
        d[2 * ld] = v.z * v.z;
        d[3 * ld] = v.w * v.w;
    }
    lds_barrier();
    if (live && tid < 16) {
        const float* row = sq + tid * ld;
        float acc = 0.0f;
        int k = 0;
        // 16 steps per group: the next group's four float4 reads are issued before the
        // current group's 16 adds, which stay one chain in order
        const int kfull = nk & ~15;
        if (kfull > 0) {
            float4 ca[4], cb[4];
#pragma unroll
            for (int q = 0; q < 4; q++) ca[q] = reinterpret_cast<const float4*>(row)[q];
            for (; k < kfull; k += 16) {
                const int kn = k + 16 < kfull ? k + 16 : k;  // past the last group: reread, unused
#pragma unroll
                for (int q = 0; q < 4; q++) cb[q] = reinterpret_cast<const float4*>(row + kn)[q];
                asm volatile("" : "+v"(acc)::"memory");
#pragma unroll
                for (int q = 0; q < 4; q++) acc = ((((acc + ca[q].x) + ca[q].y) + ca[q].z) + ca[q].w);
                asm volatile("" : "+v"(acc)::"memory");
#pragma unroll
                for (int q = 0; q < 4; q++) ca[q] = cb[q];
            }
        }
        for (; k < nk; k++) acc = acc + row[k];
        part[tid] = acc;
    }
    lds_barrier();
    if (live && tid == 0) {
        double sum = 0.0;
        int i = 0;
        if (n >= 16) {
            sum = (double)vsum8(part) + (double)vsum8(part + 8);
            i = n / 16 * 16;
        }
        for (; i < n; i++) sum += (double)sx[i] * (double)sx[i];
        s_scale = 1.0f / sqrtf((float)(sum / n) + eps);
    }
    lds_barrier();
    const float sc = s_scale;
    float* y_row = y_opt ? y_opt + (int64_t)t * n : nullptr;
    for (int p = tid; live && p < npair; p += 256) {
        const int b = p >> 1, h = p & 1;
        const int e0 = 32 * b + 8 * h;
        float4 wv[4];
        if (p == tid) {
            wv[0] = wpre[0], wv[1] = wpre[1], wv[2] = wpre[2], wv[3] = wpre[3];
        } else {
            wv[0] = *reinterpret_cast<const float4*>(w + e0);
            wv[1] = *reinterpret_cast<const float4*>(w + e0 + 4);
            wv[2] = *reinterpret_cast<const float4*>(w + e0 + 16);
            wv[3] = *reinterpret_cast<const float4*>(w + e0 + 20);
        }
        float v[16];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4 xv = *reinterpret_cast<const float4*>(sx + e0 + 4 * (g & 1) + 16 * (g >> 1));
            v[4 * g] = (xv.x * sc) * wv[g].x;
            v[4 * g + 1] = (xv.y * sc) * wv[g].y;
            v[4 * g + 2] = (xv.z * sc) * wv[g].z;
            v[4 * g + 3] = (xv.w * sc) * wv[g].w;
        }
        if (y_row) {
#pragma unroll
            for (int g = 0; g < 4; g++)
                *reinterpret_cast<float4*>(y_row + e0 + 4 * (g & 1) + 16 * (g >> 1)) =
                    make_float4(v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]);
        }
        // fmaxf drops NaN operands, so a block's max is NaN only when all 32 values are
        // (as the 8-lane reduction of quant_block8 gives it)
        float mx = fabsf(v[0]);
#pragma unroll
        for (int r = 1; r < 16; r++) mx = fmaxf(mx, fabsf(v[r]));
        mx = fmaxf(mx, dpp_f<DPP_XOR1>(mx));
        const float d = mx / 127.0f;
        const float inv = d != 0.0f ? 1.0f / d : 0.0f;
        int q[16];
        uint32_t usum = 0;  // modulo 2^32, like the reference's int32 sums of wrapped codes
#pragma unroll
        for (int r = 0; r < 16; r++) {
            q[r] = cvt_rne_x86(v[r] * inv);
            usum += (uint32_t)q[r];
        }
        const int sum = (int)(usum + (uint32_t)dpp_i<DPP_XOR1>((int)usum));
        uint4 c;
        c.x = code_byte(q[0]) | (code_byte(q[1]) << 8) | (code_byte(q[2]) << 16) | (code_byte(q[3]) << 24);
        c.y = code_byte(q[4]) | (code_byte(q[5]) << 8) | (code_byte(q[6]) << 16) | (code_byte(q[7]) << 24);
        c.z = code_byte(q[8]) | (code_byte(q[9]) << 8) | (code_byte(q[10]) << 16) | (code_byte(q[11]) << 24);
        c.w = code_byte(q[12]) | (code_byte(q[13]) << 8) | (code_byte(q[14]) << 16) | (code_byte(q[15]) << 24);
        *reinterpret_cast<uint4*>(a.q + ((((int64_t)(t >> 5) * a.B + b) * 2 + h) * 32 + (t & 31)) * 16) = c;
        if (h == 0) {
            a.d[(int64_t)b * a.Tpad + t] = d;
            a.cv[(int64_t)b * a.Tpad + t] = conversion_operand(sum);
            a.ds[(int64_t)b * a.Tpad + t] = d * (float)sum;
        }
    }
}

template <int ROWS>
static hipError_t rmsnorm_launch(const float* x, int ldx, const float* w, float eps, int n, const ActQ8& a,
                                 float* y_opt, hipStream_t s, size_t lds_row)
{
    const size_t lds = ROWS * lds_row;
    static LdsLimit limit;
    hipError_t e = limit.raise(reinterpret_cast<const void*>(k_rmsnorm_quant<ROWS>), lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_rmsnorm_quant<ROWS>, dim3(a.Tpad / ROWS), dim3(256 * ROWS), lds, s, x, ldx, w, eps, n, a,
                       y_opt);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_quant(const float* x, int ldx, const float* w, float eps, int n, const ActQ8& a,
                                float* y_opt, hipStream_t s)
{
    if (n % 32 != 0) return hipErrorInvalidValue;
    const size_t lds_row = sizeof(float) * ((size_t)n + 16 * (size_t)((((n >> 4) + 3) & ~3) + RMS_SQ_PAD));
    // four rows per block while they fit the 160 KB of LDS (hidden sizes up to ≈4900), else one
    if (4 * lds_row <= 160 * 1024 && a.Tpad % 4 == 0) return rmsnorm_launch<4>(x, ldx, w, eps, n, a, y_opt, s, lds_row);
    return rmsnorm_launch<1>(x, ldx, w, eps, n, a, y_opt, s, lds_row);
}

__device__ __forceinline__ float det_expf(float x);

// ------------------------------------------------------- SwiGLU + quantize

// Kernels.SwiGlu (Kernels.cs:83-90): gu = g·u, s = 1/(1+e^−g), y = s·gu; then the
// 32-block quantization of y for the down projection. gu rows hold [gate | up]. 8 lanes per
// block, 4 consecutive features per lane, blocks of a token adjacent across lane groups.
__global__ __launch_bounds__(256) void k_swiglu_quant(const float* __restrict__ gu, int ldgu, int ffn, ActQ8 a,
                                                      float* __restrict__ y_opt)
{
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t g = idx >> 3;
    const int l8 = (int)(idx & 7);
    if (g >= (int64_t)a.Tpad * a.B) return;
    const int b = (int)(g % a.B), t = (int)(g / a.B);
    if (t >= a.T) {
        zero_block8(l8, a, t, b);
        return;
    }
    const int f = 32 * b + 4 * l8;
    const float4 gv = *reinterpret_cast<const float4*>(gu + (int64_t)t * ldgu + f);
    const float4 uv = *reinterpret_cast<const float4*>(gu + (int64_t)t * ldgu + ffn + f);
    float4 v;
    v.x = (1.0f / (1.0f + det_expf(-gv.x))) * (gv.x * uv.x);
    v.y = (1.0f / (1.0f + det_expf(-gv.y))) * (gv.y * uv.y);
    v.z = (1.0f / (1.0f + det_expf(-gv.z))) * (gv.z * uv.z);
    v.w = (1.0f / (1.0f + det_expf(-gv.w))) * (gv.w * uv.w);
    if (y_opt) *reinterpret_cast<float4*>(y_opt + (int64_t)t * ffn + f) = v;
    quant_block8(v, l8, a, t, b, 0);
}

hipError_t launch_swiglu_quant(const float* gu, int ldgu, int ffn, const ActQ8& a, float* y_opt, hipStream_t s)
{
    const int64_t n = (int64_t)a.Tpad * a.B * 8;
    hipLaunchKernelGGL(k_swiglu_quant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, gu, ldgu, ffn, a, y_opt);
    return hipGetLastError();
}

// ------------------------------------------------------------------- GEMM

// Four 4-bit fifth-bit flags → 0x10 in the byte of each set bit.
__device__ inline uint32_t expand_bits4(uint32_t x4)
{
    return ((__umul24(x4, 0x00204081u)) & 0x01010101u) << 4;
}

template <int TYPE> struct ZeroPoint {
    static constexpr int z = TYPE == SHS_TYPE_Q4_0 ? 8 : TYPE == SHS_TYPE_Q5_0 ? 16 : 0;  // IntegerGemm.cs:75-81
};

// Lane half h's 16 weight codes of one row's block as the int8 MFMA's A operand, in the
// activation order [8h..8h+7, 16+8h..16+8h+7]: the unsigned codes u (nibble, plus the fifth
// bit for Q5) — their zero point is applied through the activation sums, like the
// reference's −z·Σa — or the stored signed bytes for Q8_0. q0/q1 are qs bytes 8h..8h+7
// (Q4/Q5); for Q8_0, q0..q3 are the lane's 16 stored bytes.
template <int TYPE>
__device__ __forceinline__ v4i weights_i8(uint32_t q0, uint32_t q1, uint32_t q2, uint32_t q3, uint32_t qh, int h)
{
    if (TYPE == SHS_TYPE_Q8_0) return v4i{(int)q0, (int)q1, (int)q2, (int)q3};
    uint32_t e0 = q0 & 0x0F0F0F0Fu, e1 = q1 & 0x0F0F0F0Fu;
    uint32_t e2 = (q0 >> 4) & 0x0F0F0F0Fu, e3 = (q1 >> 4) & 0x0F0F0F0Fu;
    if (TYPE == SHS_TYPE_Q5_0 || TYPE == SHS_TYPE_Q5_1) {
        const uint32_t sh = 8u * h;
        e0 |= expand_bits4((qh >> sh) & 0xFu);
        e1 |= expand_bits4((qh >> (sh + 4)) & 0xFu);
        e2 |= expand_bits4((qh >> (sh + 16)) & 0xFu);
        e3 |= expand_bits4((qh >> (sh + 20)) & 0xFu);
    }
    return v4i{(int)e0, (int)e1, (int)e2, (int)e3};
}

template <int TYPE>
__device__ __forceinline__ v4i load_weight_i8(const uint8_t* __restrict__ wqs, const uint32_t* __restrict__ wqh,
                                              int64_t rec, int ri, int h)
{
    if (TYPE == SHS_TYPE_Q8_0) {
        const uint4 q = *reinterpret_cast<const uint4*>(wqs + rec * 1024 + ri * 32 + h * 16);
        return weights_i8<TYPE>(q.x, q.y, q.z, q.w, 0u, h);
    }
    const uint2 q = *reinterpret_cast<const uint2*>(wqs + rec * 512 + ri * 16 + h * 8);
    const uint32_t qh = (TYPE == SHS_TYPE_Q5_0 || TYPE == SHS_TYPE_Q5_1) ? wqh[rec * 32 + ri] : 0u;
    return weights_i8<TYPE>(q.x, q.y, 0u, 0u, qh, h);
}

// The integer MFMA accumulates Σu·q onto the bit pattern of 1.5·2^23, which read as fp32 is
// 1.5·2^23 + Σu·q exactly while |Σu·q| < 2^22 (|Σu·q| ≤ 32·128·127 for every type).
constexpr int MAGIC_BITS = 0x4B400000;

// The pattern in 16 registers, built once per kernel: the empty asm hides the constant from
// the compiler, which would otherwise rebuild it before every MFMA that reads it.
__device__ __forceinline__ v16i magic16()
{
    v16i m;
#pragma unroll
    for (int r = 0; r < 16; r++) m[r] = MAGIC_BITS;
    asm volatile("" : "+v"(m));
    return m;
}

// Position of work-group L of `total` in an order where each XCD (work-groups are dealt to
// the 8 XCDs round-robin) runs one contiguous range of row groups, so its L2 holds its own
// slice of the weights.
__device__ __forceinline__ int xcd_order(int L, int total)
{
    const int q = total >> 3, r = total & 7, x = L & 7, slot = L >> 3;
    return x < r ? x * (q + 1) + slot : r * (q + 1) + (x - r) * q + slot;
}

// ---- asynchronous global → LDS copies (global_load_lds), issued through inline asm so the
// compiler's own wait insertion (which would wait for every copy before any LDS read) stays
// out of the pipeline; the kernel waits for them itself with vmcnt. lds is the wave-uniform
// LDS byte address of the wave's destination: lane i's bytes land at lds + i·size.
// m0 (the copy's LDS base) is reserved: clang warns about naming it as a clobber; nothing
// else in these kernels keeps a value in m0 across the copies.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_copy16(const void* g, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void lds_copy4(const void* g, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
// The same copies addressed as a scalar base plus a per-lane 32-bit offset (the saddr
// form): no vector instruction forms the address. The masked form copies only the lanes of
// `mask` (exec is saved and restored inside the one asm statement).
__device__ __forceinline__ void lds_copy16_s(const void* sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
                 : "memory", "m0");
}
__device__ __forceinline__ void lds_copy16_s_masked(const void* sbase, uint32_t voff, uint32_t lds, uint64_t mask)
{
    uint64_t save;
    asm volatile("s_mov_b64 %0, exec\n\ts_mov_b64 exec, %4\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %1, %2\n\ts_mov_b64 exec, %0"
                 : "=&s"(save)
                 : "v"(voff), "s"(sbase), "s"(lds), "s"(mask)
                 : "memory", "m0");
}
__device__ __forceinline__ void lds_copy4_s(const void* sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
// A pointer every lane of the wave holds, moved into scalar registers (the saddr operand).
__device__ __forceinline__ const void* wave_uniform(const void* p)
{
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ uint32_t lds_addr(const void* p)
{
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)p);
}

// Wait until at most N of this wave's global → LDS copies are outstanding (they complete in
// order), then meet the work-group at a barrier.
template <int N>
__device__ __forceinline__ void wait_copies_barrier()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// The GEMM y = x·Wᵀ by 32-row × 32-token tiles, block by block in the reference order.
//  * Integer block sums: one v_mfma_i32_32x32x32_i8 per (tile, block) on the unsigned weight
//    codes and the int8 activation codes, accumulated onto the magic bit pattern above:
//    F = 1.5·2^23 + Σu·q as fp32.
//  * Conversion and zero point: one v_mfma_f32_32x32x8_f16 per (tile, block) with C = F,
//    A row (2048, 64z, z, 0) and the activation's B column (−6144, −⌊Σq/64⌋,
//    −(Σq mod 64), 0): I = F − 1.5·2^23 − z·Σq = Σ(u−z)·q. Every product and partial sum
//    is an integer below 2^24, so I is exact whatever the MFMA's summation order.
//  * Scale RN(d_w·d_a): one v_mfma_f32_32x32x1_2b_f32 per two tiles, fma(d_w, d_a, 0).
//  * Epilogue on the VALU: acc = fma(I_b, S_b, acc) (+ fma(m_w, RN(d_a·Σq), acc) for the
//    offset types) — IntegerGemm.Multiply4/Multiply1 per output, bit for bit
//    (IntegerGemm.cs:371-473).
// The two integer MFMA steps run on the matrix cores beside the VALU epilogue; the fp32
// scale step and the epilogue share the VALU's issue slots.
// A work-group is 4 waves, one 32-row tile each, over TT 32-token tiles; the scale step pairs
// the two token tiles (TT = 2) or two consecutive blocks (TT = 1). The K loop runs over stages
// of BPS blocks through a ring of NS LDS slots filled by global → LDS copies NS − 1 stages
// ahead, so memory latency hides behind NS − 1 stages of arithmetic; one barrier per stage.
// Two-tile work-groups take stages of 2 blocks in 4 slots; single-tile work-groups, whose
// slots are half as large, take stages of 4 blocks in 3 slots when the block count allows
// (half the barriers and copy groups per block, the same LDS as 4 two-tile slots).
// A slot holds the stage's activation codes and per-token operands (d_a, the conversion
// column, d_a·Σq; shared by the 4 waves) and each wave's weight bytes and per-row factors
// (d_w, fifth bits, m_w). D[i][j] (row i, token j) sits in lane j + 32·(i%8/4), register
// 4·(i/8) + i%4.
template <int TYPE, int TT, int BPS>
struct GemmSlot {
    static_assert((TT == 2 && BPS == 2) || (TT == 1 && (BPS == 2 || BPS == 4)), "stage shape");
    static constexpr bool OFF = (TYPE == SHS_TYPE_Q4_1 || TYPE == SHS_TYPE_Q5_1);
    static constexpr bool QH = (TYPE == SHS_TYPE_Q5_0 || TYPE == SHS_TYPE_Q5_1);
    static constexpr bool Q8 = (TYPE == SHS_TYPE_Q8_0);
    static constexpr int ACT = BPS * TT * 1024;  // [tile][block] 1 KB code chunks
    // per-token operands, [block][TT·32 tokens] each: conversion columns (8 B), then d_a and
    // d_a·Σq (4 B) — two copies of 1 KB (one of two masked halves at TT = 1, BPS = 2)
    static constexpr int CV = BPS * TT * 32 * 8;
    static constexpr int DA = BPS * TT * 32 * 4;
    static constexpr int FACT = CV + 2 * DA;
    static constexpr bool HALF_FACT = FACT == 1024;          // operand copies of half a wave each
    static constexpr int W = (Q8 ? 1024 : 512) * BPS;        // per wave: [block][32 rows][QSB]
    static constexpr int WX1 = 128 * BPS;                    // per wave and array: [block][32 rows] f32
    static constexpr int WX = WX1 * (1 + QH + OFF);          // d_w [, qh] [, m_w]
    static constexpr int BYTES = ACT + FACT + 4 * (W + WX);
    static constexpr int NSH_REAL = BPS * TT + 2;            // shared copies per stage: codes, then 2 of operands
    static constexpr int SHARED = (NSH_REAL + 3) / 4;        // per wave (the last waves may repeat one)
    static constexpr int OWN = W / 1024 + (1 + QH + OFF) * BPS / 2;  // each wave's own copies per stage
    static constexpr int PER_STAGE = SHARED + OWN;
    static constexpr int NS = BPS == 4 ? 3 : 4;              // ring depth
};

// The down projection's input block (one 32-feature tile × token j) held as the MFMA D
// layout: lane j + 32h has features 8g + 4h + i in y[4g + i]. Quantized exactly like
// quant_block8 (semantics 0: d = max|y|/127, q = RNE(y·(1/d))), the max and Σq reduced over
// the lane pair; codes, d, the conversion column and d·Σq written at token t, block b.
__device__ __forceinline__ void quant_block_pair(const float* y, int h, const ActQ8& o, int t, int b)
{
    float mx = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; r++) mx = fmaxf(mx, fabsf(y[r]));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float d = mx / 127.0f;
    const float inv = d != 0.0f ? 1.0f / d : 0.0f;
    int q[16];
    int sum = 0;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        q[r] = cvt_rne_x86(y[r] * inv);
        sum += q[r];
    }
    sum += __shfl_xor(sum, 32);
    // feature 8g + 4h + i sits in half g & 1 at index 4h + i + 8·(g >> 1)
    int8_t* base = o.q + (((int64_t)(t >> 5) * o.B + b) * 2 * 32 + (t & 31)) * 16;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const uint32_t w = code_byte(q[4 * g]) | (code_byte(q[4 * g + 1]) << 8) | (code_byte(q[4 * g + 2]) << 16) |
                           (code_byte(q[4 * g + 3]) << 24);
        *reinterpret_cast<uint32_t*>(base + (g & 1) * 512 + 4 * h + 8 * (g >> 1)) = w;
    }
    if (h == 0) {
        o.d[(int64_t)b * o.Tpad + t] = d;
        o.cv[(int64_t)b * o.Tpad + t] = conversion_operand(sum);
        o.ds[(int64_t)b * o.Tpad + t] = d * (float)sum;
    }
}

// Work-groups per CU the LDS ring admits (at most 3, the register budget's target): Q8_0's
// two-tile ring (≈61 KB) admits 2.
template <int TYPE, int TT, int BPS>
constexpr int gemm_wg_per_cu()
{
    typedef GemmSlot<TYPE, TT, BPS> L;
    return 3 * L::NS * L::BYTES <= 160 * 1024 ? 3 : 2;
}

template <int TYPE, int TT, int MODE, int BPS>
__global__ __launch_bounds__(256, (gemm_wg_per_cu<TYPE, TT, BPS>())) void k_gemm(const uint8_t* __restrict__ wqs, const uint32_t* __restrict__ wqh,
                                                 const float* __restrict__ wd, const float* __restrict__ wm,
                                                 int ntiles, int B, ActQ8 a, float* __restrict__ y, int ldy, int N,
                                                 int n_tg, ActQ8 ao, int n_ft, RopeArgs ra)
{
    typedef GemmSlot<TYPE, TT, BPS> L;
    constexpr bool OFF = L::OFF, QH = L::QH, Q8 = L::Q8;
    constexpr int NS = L::NS;
    constexpr int Z = ZeroPoint<TYPE>::z;
    __shared__ __align__(16) uint8_t ring[NS * L::BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31, h = lane >> 5;
    const int R = xcd_order(blockIdx.x, gridDim.x);
    // token groups fastest (an XCD's work-groups share a few row groups' weights in its L2);
    // the one-round q|k|v launch measured faster with row groups fastest
    const int n_rg = gridDim.x / n_tg;
    const int rg = MODE == GEMM_QKV ? R % n_rg : R / n_tg;
    const int tg = MODE == GEMM_QKV ? R / n_rg : R - rg * n_tg;
    // GEMM_SWIGLU: waves 0/1 take gate/up of feature tile 2·rg, waves 2/3 of 2·rg + 1
    const int ft = 2 * rg + (wave >> 1);
    const int rt = MODE == GEMM_SWIGLU ? (wave & 1) * n_ft + ft : rg * 4 + wave;
    const bool active = MODE == GEMM_SWIGLU ? ft < n_ft : rt < ntiles;
    const int rtl = active ? rt : ntiles - 1;  // inactive waves copy a valid tile (their share of the stage)
    const int ntt = a.Tpad >> 5;
    const int tt0 = tg * TT;
    // (BPS = 4 is launched only for block counts that are a multiple of 4)
    const int nstages = (B + BPS - 1) / BPS;

    // ---- the copy plan. Every copy of a stage is a scalar base that advances by a fixed
    // stride per stage plus a per-lane 32-bit offset fixed for the kernel, so issuing a stage
    // costs no vector instructions and no branches. The activation arrays share one
    // allocation (codes, d_a, d_a·Σq, conversion columns: act_q8_view) and are addressed
    // from the codes' base.
    const uint8_t* const abase = reinterpret_cast<const uint8_t*>(a.q);
    const int64_t ld = (int64_t)a.Tpad;
    const uint8_t* sh_base[L::SHARED];
    int64_t sh_stride[L::SHARED];
    uint32_t sh_voff[L::SHARED], sh_lds[L::SHARED];
    uint64_t sh_mask[L::SHARED];
#pragma unroll
    for (int k = 0; k < L::SHARED; k++) {
        int i = wave + 4 * k;
        if (i >= L::NSH_REAL) i = 0;  // padding: repeat copy 0 (same bytes, same place)
        if (i < BPS * TT) {
            // activation codes of (tile u, block bb): 64 lanes × 16 B
            const int u = i / BPS, bb = i % BPS;
            const int tile = tt0 + u < ntt ? tt0 + u : ntt - 1;
            sh_base[k] = abase + ((int64_t)tile * B + bb) * 1024;
            sh_stride[k] = BPS * 1024;
            sh_voff[k] = lane * 16;
            sh_lds[k] = i * 1024;
            sh_mask[k] = ~0ull;
        } else {
            // per-token operands, [block][TT·32 tokens] each in the slot: conversion columns
            // (8 B), d_a, d_a·Σq (4 B; d_a again when there is no offset term). Copy f = 0
            // brings the columns, f = 1 the two float arrays; each fills 64 lanes × 16 B, or,
            // when the region is 1 KB (TT = 1, BPS = 2), one half of it (the other lanes
            // masked off)
            const int f = i - BPS * TT;
            const int P = !L::HALF_FACT ? f * 1024 + lane * 16 : lane * 16;  // byte in the operand region
            int e;
            const uint8_t* arr;
            if (P < L::CV) {
                e = P / 8, arr = reinterpret_cast<const uint8_t*>(a.cv);
            } else if (P < L::CV + L::DA) {
                e = (P - L::CV) / 4, arr = reinterpret_cast<const uint8_t*>(a.d);
            } else {
                e = (P - L::CV - L::DA) / 4, arr = reinterpret_cast<const uint8_t*>(OFF ? a.ds : a.d);
            }
            const int esize = f == 0 ? 8 : 4;
            const int bb = e / (TT * 32);
            int tok = e % (TT * 32);
            if ((tok >> 5) >= ntt - tt0) tok &= 31;  // a token tile past the end rereads tile tt0
            sh_base[k] = abase;
            sh_stride[k] = BPS * ld * esize;
            sh_voff[k] = (uint32_t)(arr - abase) + (uint32_t)(((int64_t)bb * ld + tt0 * 32 + tok) * esize);
            sh_lds[k] = BPS * TT * 1024 + (!L::HALF_FACT ? f * 1024 : 0);
            sh_mask[k] = !L::HALF_FACT ? ~0ull : (f == 0 ? 0x00000000FFFFFFFFull : 0xFFFFFFFF00000000ull);
        }
    }
    const uint32_t w_voff = Q8 ? lane * 16 : h * 512 + j * 16;
    const uint32_t x_voff = (h * 32 + j) * 4;
    const uint32_t ring_lds = lds_addr(ring);

    // ---- issue the copies of stage sidx into ring slot `slot`
    auto issue_fast = [&](int sidx, int slot) {
        const uint32_t slot_lds = ring_lds + slot * L::BYTES;
#pragma unroll
        for (int k = 0; k < L::SHARED; k++) {
            if (L::HALF_FACT)
                lds_copy16_s_masked(sh_base[k] + sidx * sh_stride[k], sh_voff[k], slot_lds + sh_lds[k], sh_mask[k]);
            else
                lds_copy16_s(sh_base[k] + sidx * sh_stride[k], sh_voff[k], slot_lds + sh_lds[k]);
        }
        // own copies: weight bytes of the stage's BPS blocks and the per-row factors
        // (d_w [, qh] [, m_w]), two blocks per copy (one for Q8_0's bytes)
        const uint32_t wlds = slot_lds + L::ACT + L::FACT + wave * L::W;
        const uint32_t xlds = slot_lds + L::ACT + L::FACT + 4 * L::W + wave * L::WX;
        const int64_t rb = (int64_t)rtl * B + BPS * sidx;  // first block of the stage in the tile's records
        if constexpr (Q8) {
#pragma unroll
            for (int c = 0; c < BPS; c++) lds_copy16_s(wqs + (rb + c) * 1024, w_voff, wlds + c * 1024);
        } else {
#pragma unroll
            for (int c = 0; c < BPS / 2; c++) lds_copy16_s(wqs + (rb + 2 * c) * 512, w_voff, wlds + c * 1024);
        }
#pragma unroll
        for (int c = 0; c < BPS / 2; c++) {
            lds_copy4_s(wd + (rb + 2 * c) * 32, x_voff, xlds + c * 256);
            if (QH) lds_copy4_s(wqh + (rb + 2 * c) * 32, x_voff, xlds + L::WX1 + c * 256);
            if (OFF) lds_copy4_s(wm + (rb + 2 * c) * 32, x_voff, xlds + L::WX1 * (1 + QH) + c * 256);
        }
    };
    // The last stage of an odd block count: its second block does not exist, and each copy
    // rereads block B−1 in its place (per-lane 64-bit addresses; runs once per kernel).
    // (only two-block stages have one: four-block stages are launched for whole stages only)
    auto issue_last_odd = [&](int sidx, int slot) {
        if constexpr (BPS == 2) {
            uint8_t* base = ring + slot * L::BYTES;
            const int blk = B - 1;
            // the lane index laundered here, so that nothing below is hoisted out of this rare
            // path and kept live (in registers) across the K loop
            int lane = threadIdx.x & 63;
            asm volatile("" : "+v"(lane));
            const int j = lane & 31;
    #pragma unroll
            for (int k = 0; k < L::SHARED; k++) {
                int i = wave + 4 * k;
                if (i >= L::NSH_REAL) i = 0;
                if (i < 2 * TT) {
                    const int u = i >> 1;
                    const int tile = tt0 + u < ntt ? tt0 + u : ntt - 1;
                    lds_copy16(a.q + ((int64_t)tile * B + blk) * 1024 + lane * 16, lds_addr(base + i * 1024));
                } else {
                    const int f = i - 2 * TT;
                    const int P = TT == 2 ? f * 1024 + lane * 16 : lane * 16;
                    const bool mine = TT == 2 || (f == 0) == (lane < 32);
                    int e;
                    const uint8_t* arr;
                    if (P < L::CV) {
                        e = P / 8, arr = reinterpret_cast<const uint8_t*>(a.cv);
                    } else if (P < L::CV + L::DA) {
                        e = (P - L::CV) / 4, arr = reinterpret_cast<const uint8_t*>(a.d);
                    } else {
                        e = (P - L::CV - L::DA) / 4, arr = reinterpret_cast<const uint8_t*>(OFF ? a.ds : a.d);
                    }
                    const int esize = f == 0 ? 8 : 4;
                    int tok = e % (TT * 32);
                    if ((tok >> 5) >= ntt - tt0) tok &= 31;
                    if (mine)
                        lds_copy16(arr + ((int64_t)blk * ld + tt0 * 32 + tok) * esize,
                                   lds_addr(base + 2 * TT * 1024 + (TT == 2 ? f * 1024 : 0)));
                }
            }
            uint8_t* wbase = base + L::ACT + L::FACT + wave * L::W;
            uint8_t* xbase = base + L::ACT + L::FACT + 4 * L::W + wave * L::WX;
            if constexpr (Q8) {
    #pragma unroll
                for (int bb = 0; bb < 2; bb++)
                    lds_copy16(wqs + ((int64_t)rtl * B + blk) * 1024 + lane * 16, lds_addr(wbase + bb * 1024));
            } else {
                lds_copy16(wqs + ((int64_t)rtl * B + blk) * 512 + j * 16, lds_addr(wbase));
            }
            const int64_t rec = ((int64_t)rtl * B + blk) * 32 + j;
            lds_copy4(wd + rec, lds_addr(xbase));
            if (QH) lds_copy4(wqh + rec, lds_addr(xbase + 256));
            if (OFF) lds_copy4(wm + rec, lds_addr(xbase + 256 * (1 + QH)));
        }
    };
    auto issue = [&](int sidx, int slot) {
        if constexpr (BPS == 4) {
            issue_fast(sidx, slot);
        } else {
            if (2 * sidx + 1 < B) issue_fast(sidx, slot);
            else issue_last_odd(sidx, slot);
        }
    };

    v16f acc[TT];
#pragma unroll
    for (int u = 0; u < TT; u++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[u][r] = 0.0f;
    v32f zero32;
#pragma unroll
    for (int r = 0; r < 32; r++) zero32[r] = 0.0f;
    const v16i magic = magic16();
    // A rows of the conversion MFMA: (2048, 64z, z, 0) in lane half 0, zeros in half 1
    v4h acv;
#pragma unroll
    for (int k = 0; k < 4; k++) acv[k] = (_Float16)0.0f;
    if (h == 0) {
        acv[0] = (_Float16)2048.0f;
        acv[1] = (_Float16)(float)(64 * Z);
        acv[2] = (_Float16)(float)Z;
    }

    // exact block sums of (token tile u, block bb) from the slot
    auto block_sums = [&](const uint8_t* base, v4i w, int u, int bb) -> v16f {
        const v4i q = *reinterpret_cast<const v4i*>(base + (u * BPS + bb) * 1024 + h * 512 + j * 16);
        const v16i F = __builtin_amdgcn_mfma_i32_32x32x32_i8(w, q, magic, 0, 0, 0);
        const v4h c = *reinterpret_cast<const v4h*>(base + L::ACT + (bb * TT * 32 + u * 32 + j) * 8);
        return __builtin_amdgcn_mfma_f32_32x32x8f16(acv, c, __builtin_bit_cast(v16f, F), 0, 0, 0);
    };

    // m_w·RN(d_a·Σq) of block bb on token tile u (offset types)
    auto offset_term = [&](const uint8_t* base, int bb, int u, bool valid) {
        const float* dsa = reinterpret_cast<const float*>(base + L::ACT + L::CV + L::DA);
        float dsv = dsa[bb * TT * 32 + u * 32 + j];
        dsv = valid ? dsv : 0.0f;
        const float4* m4p = reinterpret_cast<const float4*>(base + L::ACT + L::FACT + 4 * L::W + wave * L::WX +
                                                            L::WX1 * (1 + QH));
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4 m4 = m4p[bb * 8 + 2 * g + h];
            acc[u][4 * g] = fmaf(m4.x, dsv, acc[u][4 * g]);
            acc[u][4 * g + 1] = fmaf(m4.y, dsv, acc[u][4 * g + 1]);
            acc[u][4 * g + 2] = fmaf(m4.z, dsv, acc[u][4 * g + 2]);
            acc[u][4 * g + 3] = fmaf(m4.w, dsv, acc[u][4 * g + 3]);
        }
    };

    // Weight codes of block bb for lane (row j, half h), from the slot.
    auto weights = [&](const uint8_t* base, int bb) -> v4i {
        const uint8_t* wb = base + L::ACT + L::FACT + wave * L::W;
        if constexpr (Q8) {
            const uint4 q = *reinterpret_cast<const uint4*>(wb + bb * 1024 + j * 32 + h * 16);
            return weights_i8<TYPE>(q.x, q.y, q.z, q.w, 0u, h);
        } else {
            const uint2 q = *reinterpret_cast<const uint2*>(wb + bb * 512 + j * 16 + h * 8);
            uint32_t qh = 0u;
            if (QH)
                qh = reinterpret_cast<const uint32_t*>(base + L::ACT + L::FACT + 4 * L::W + wave * L::WX + L::WX1)[bb * 32 + j];
            return weights_i8<TYPE>(q.x, q.y, 0u, 0u, qh, h);
        }
    };

    for (int p = 0; p < NS - 1 && p < nstages; p++) issue(p, p);
    // Stage sidx lives in ring slot sidx % NS; the loop below runs whole rounds of the ring
    // with the slot a compile-time constant, so every LDS address is a fixed offset.
    // STEADY: a stage at least NS stages before the end, whose wait and copy issue need no
    // checks (the stage it issues is a whole one, never the odd last).
    auto stage = [&](int sidx, auto slot_c, auto steady_c) {
        constexpr int SLOT = decltype(slot_c)::value;
        if constexpr (decltype(steady_c)::value) {
            wait_copies_barrier<(NS - 2) * L::PER_STAGE>();
            issue_fast(sidx + NS - 1, (SLOT + NS - 1) % NS);
        } else {
            // stages issued after this one: NS − 2 in the steady state, fewer at the end
            const int ahead = nstages - 1 - sidx;
            if (ahead >= NS - 2) wait_copies_barrier<(NS - 2) * L::PER_STAGE>();
            else if (NS == 4 && ahead == 1) wait_copies_barrier<L::PER_STAGE>();
            else wait_copies_barrier<0>();
            if (sidx + NS - 1 < nstages) issue(sidx + NS - 1, (SLOT + NS - 1) % NS);
        }
        if (!active) return;
        const uint8_t* base = ring + SLOT * L::BYTES;
        const float* da_s = reinterpret_cast<const float*>(base + L::ACT + L::CV);
        const float* dw_s = reinterpret_cast<const float*>(base + L::ACT + L::FACT + 4 * L::W + wave * L::WX);
        // A block past B (odd B, last stage) holds copies of block B−1: its d_w is taken as 0,
        // so S = 0 and fma(I, 0, acc) leaves acc unchanged (acc is never −0), and the loop body
        // needs no branch.
        const bool valid1 = BPS == 4 || decltype(steady_c)::value || 2 * sidx + 1 < B;
        if constexpr (TT == 2) {
#pragma unroll
            for (int bb = 0; bb < 2; bb++) {
                const bool valid = bb == 0 || valid1;
                const float da = da_s[bb * 64 + lane];
                float dw = dw_s[bb * 32 + j];
                dw = valid ? dw : 0.0f;
                const v32f S = __builtin_amdgcn_mfma_f32_32x32x1f32(dw, da, zero32, 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                const v4i w = weights(base, bb);
                const v16f G0 = block_sums(base, w, 0, bb);
                const v16f G1 = block_sums(base, w, 1, bb);
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    acc[0][r] = fmaf(G0[r], S[r], acc[0][r]);
                    acc[1][r] = fmaf(G1[r], S[16 + r], acc[1][r]);
                }
                if (OFF) {
                    offset_term(base, bb, 0, valid);
                    offset_term(base, bb, 1, valid);
                }
            }
        } else {
            // the scale step of blocks 2p and 2p + 1: lane half h holds block 2p + h
#pragma unroll
            for (int p = 0; p < BPS / 2; p++) {
                const float da = da_s[(2 * p + h) * 32 + j];
                float dw = dw_s[(2 * p + h) * 32 + j];
                dw = (h == 0 || valid1) ? dw : 0.0f;
                const v32f S = __builtin_amdgcn_mfma_f32_32x32x1f32(dw, da, zero32, 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                const v16f G0 = block_sums(base, weights(base, 2 * p), 0, 2 * p);
                const v16f G1 = block_sums(base, weights(base, 2 * p + 1), 0, 2 * p + 1);
#pragma unroll
                for (int r = 0; r < 16; r++) acc[0][r] = fmaf(G0[r], S[r], acc[0][r]);
                if (OFF) offset_term(base, 2 * p, 0, true);
#pragma unroll
                for (int r = 0; r < 16; r++) acc[0][r] = fmaf(G1[r], S[16 + r], acc[0][r]);
                if (OFF) offset_term(base, 2 * p + 1, 0, valid1);
            }
        }
    };
    typedef std::integral_constant<int, 0> S0;
    typedef std::integral_constant<int, 1> S1;
    typedef std::integral_constant<int, 2> S2;
    typedef std::integral_constant<int, 3> S3;
    typedef std::true_type ST;
    typedef std::false_type CK;
    // stages that hold BPS real blocks (all but an odd last one)
    const int nfull = B / BPS;
    int sidx = 0;
    // Whole rounds of the ring whose every stage is steady (the round's last stage issues
    // stage sidx + 2·NS − 2, which must be a whole one), then the checked stages.
    if constexpr (NS == 4) {
        for (; sidx + 2 * NS - 1 <= nfull; sidx += NS) {
            stage(sidx, S0(), ST());
            stage(sidx + 1, S1(), ST());
            stage(sidx + 2, S2(), ST());
            stage(sidx + 3, S3(), ST());
        }
        for (; sidx + NS <= nstages; sidx += NS) {
            stage(sidx, S0(), CK());
            stage(sidx + 1, S1(), CK());
            stage(sidx + 2, S2(), CK());
            stage(sidx + 3, S3(), CK());
        }
        if (sidx < nstages) stage(sidx, S0(), CK());
        if (sidx + 1 < nstages) stage(sidx + 1, S1(), CK());
        if (sidx + 2 < nstages) stage(sidx + 2, S2(), CK());
    } else {
        static_assert(NS == 3, "rings of three or four slots");
        for (; sidx + 2 * NS - 1 <= nfull; sidx += NS) {
            stage(sidx, S0(), ST());
            stage(sidx + 1, S1(), ST());
            stage(sidx + 2, S2(), ST());
        }
        for (; sidx + NS <= nstages; sidx += NS) {
            stage(sidx, S0(), CK());
            stage(sidx + 1, S1(), CK());
            stage(sidx + 2, S2(), CK());
        }
        if (sidx < nstages) stage(sidx, S0(), CK());
        if (sidx + 1 < nstages) stage(sidx + 1, S1(), CK());
    }
    const int nv = ntt - tt0 < TT ? ntt - tt0 : TT;
    if constexpr (MODE == GEMM_SWIGLU) {
        // Exchange the accumulators through the (now idle) ring: X[wave][u][r][lane]; then
        // (feature tile 2·rg + p, token tile u) goes to wave 2p + u (waves 0..2·TT−1):
        // y = sigmoid(g)·(g·u) as Kernels.SwiGlu (Kernels.cs:83-90) forms it, then quantized.
        float* X = reinterpret_cast<float*>(ring);
        __syncthreads();
#pragma unroll
        for (int u = 0; u < TT; u++)
#pragma unroll
            for (int r = 0; r < 16; r++) X[((wave * TT + u) * 16 + r) * 64 + lane] = acc[u][r];
        __syncthreads();
        const int p = wave >> 1, u = wave & 1;
        const int fti = 2 * rg + p;
        if (u >= nv || fti >= n_ft) return;
        float yv[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float g = X[(((2 * p) * TT + u) * 16 + r) * 64 + lane];
            const float v = X[(((2 * p + 1) * TT + u) * 16 + r) * 64 + lane];
            yv[r] = (1.0f / (1.0f + det_expf(-g))) * (g * v);
        }
        quant_block_pair(yv, h, ao, (tt0 + u) * 32 + j, fti);
        return;
    }
    // q|k|v stages its output tiles through the ring, which is free once every wave (active
    // or not) has left the K loop
    if constexpr (MODE == GEMM_QKV) __syncthreads();
    if (!active) return;
    if constexpr (MODE == GEMM_QKV) {
        // Rope.Apply on adjacent pairs (x0, x1) → (x0c − x1s, x0s + x1c), unfused, then the
        // query position scale (MinistralModel.cs:442-482); StoreKeys/StoreValues put k and v
        // at the token's cache slot. A tile lies inside one head (hd is a multiple of 32).
        // The tile goes through this wave's part of the ring as [token][32 features]; read back
        // as 8 lanes per token (4 features each), the rotation's table reads and the stores
        // below each touch 8 token rows per instruction, the stores in whole 128-byte rows.
        constexpr int XLD = 36;  // floats per staged token row: rows start 4 banks apart
        static_assert(NS * L::BYTES >= 4 * TT * 32 * XLD * 4, "the ring holds the staged tiles");
        float* X = reinterpret_cast<float*>(ring) + wave * TT * 32 * XLD;
        const int hrow = rt * 32 / ra.hd, e0 = rt * 32 % ra.hd;
        const bool rot = hrow < ra.n_head + ra.n_kv, query = hrow < ra.n_head;
#pragma unroll
        for (int u = 0; u < TT; u++) {
#pragma unroll
            for (int g = 0; g < 4; g++)
                *reinterpret_cast<float4*>(X + (u * 32 + j) * XLD + 8 * g + 4 * h) =
                    make_float4(acc[u][4 * g], acc[u][4 * g + 1], acc[u][4 * g + 2], acc[u][4 * g + 3]);
        }
        // this wave's rows are in the LDS (only this wave reads them)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int c4 = 4 * (lane & 7);
        const int pi0 = (e0 + c4) / 2;  // this lane's two pairs of the head: pi0, pi0 + 1
#pragma unroll
        for (int u = 0; u < TT; u++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = (lane >> 3) + 8 * i;
                const int token = (tt0 + u) * 32 + r;
                if (u >= nv || token >= a.T) continue;
                const float4 x = *reinterpret_cast<const float4*>(X + (u * 32 + r) * XLD + c4);
                float v[4] = {x.x, x.y, x.z, x.w};
                if (rot || query) {
                    const int p = ra.pos[token];
                    if (rot) {
#pragma unroll
                        for (int k = 0; k < 2; k++) {
                            const int pi = pi0 + k;
                            if (pi < ra.half) {
                                const float c = ra.ct[(int64_t)p * ra.half + pi], sn = ra.st[(int64_t)p * ra.half + pi];
                                const float x0 = v[2 * k], x1 = v[2 * k + 1];
                                const float a0 = x0 * c, b0 = x1 * sn;
                                const float e1 = x0 * sn, f1 = x1 * c;
                                v[2 * k] = a0 - b0;
                                v[2 * k + 1] = e1 + f1;
                            }
                        }
                    }
                    if (query) {
                        const float qs = ra.qscale[p];
                        if (qs != 1.0f) {
#pragma unroll
                            for (int k = 0; k < 4; k++) v[k] = v[k] * qs;
                        }
                    }
                }
                const float4 vo = make_float4(v[0], v[1], v[2], v[3]);
                float* dst;
                if (query)
                    dst = y + (int64_t)token * ldy + rt * 32 + c4;
                else if (rot)
                    dst = ra.kc + ((int64_t)(hrow - ra.n_head) * ra.cap + ra.slot0 + token) * ra.hd + e0 + c4;
                else
                    dst = ra.vc + ((int64_t)(hrow - ra.n_head - ra.n_kv) * ra.cap + ra.slot0 + token) * ra.hd + e0 + c4;
                *reinterpret_cast<float4*>(dst) = vo;
            }
        }
        return;
    }

    const bool vec = ((ldy & 3) == 0) && ((reinterpret_cast<uintptr_t>(y) & 15) == 0);
#pragma unroll
    for (int u = 0; u < TT; u++) {
        const int token = (tt0 + u) * 32 + j;
        if (u >= nv || token >= a.T) continue;
        float* yr = y + (int64_t)token * ldy;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int row = rt * 32 + 8 * g + 4 * h;
            if (vec && row + 3 < N) {
                float4* pp = reinterpret_cast<float4*>(yr + row);
                float4 v = make_float4(acc[u][4 * g], acc[u][4 * g + 1], acc[u][4 * g + 2], acc[u][4 * g + 3]);
                if (MODE == GEMM_ADD) {
                    float4 o = *pp;
                    v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
                }
                *pp = v;
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    if (row + k < N) {
                        float v = acc[u][4 * g + k];
                        if (MODE == GEMM_ADD) v = yr[row + k] + v;
                        yr[row + k] = v;
                    }
                }
            }
        }
    }
}

static hipError_t launch_gemm_narrow(const DevMatrix& w, const ActQ8& a, float* y, int ldy, int mode, hipStream_t s,
                                     const ActQ8& ao, int n_ft, const RopeArgs& ra, const NormIn& nin);

template <int TYPE, int TT, int MODE>
static hipError_t gemm_launch(const DevMatrix& w, const ActQ8& a, float* y, int ldy, hipStream_t s,
                              const ActQ8& ao = ActQ8(), int n_ft = 0, const RopeArgs& ra = RopeArgs())
{
    const int n_rg = MODE == GEMM_SWIGLU ? (n_ft + 1) / 2 : (w.tiles + 3) / 4;
    const int n_tg = ((a.Tpad >> 5) + TT - 1) / TT;
    dim3 grid((unsigned)(n_rg * n_tg)), block(256);
    if constexpr (TYPE == SHS_TYPE_Q4_0 && TT == 1) {
        if (gemm_stage_blocks(w, TT) == 4) {
            hipLaunchKernelGGL((k_gemm<TYPE, 1, MODE, 4>), grid, block, 0, s, w.qs, w.qh, w.d, w.m, w.tiles, w.blocks,
                               a, y, ldy, w.rows, n_tg, ao, n_ft, ra);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((k_gemm<TYPE, TT, MODE, 2>), grid, block, 0, s, w.qs, w.qh, w.d, w.m, w.tiles, w.blocks, a, y,
                       ldy, w.rows, n_tg, ao, n_ft, ra);
    return hipGetLastError();
}

// Resident blocks of k_gemm<TYPE, TT, MODE, BPS> on the whole device (blocks per CU × CUs),
// asked of the runtime once per instantiation and device.
template <int TYPE, int TT, int MODE, int BPS>
static int gemm_slots()
{
    static std::atomic<int> cached[64] = {};  // threads that race store the same value
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int slots = cached[dev].load(std::memory_order_relaxed);
    if (slots == 0) {
        int per_cu = 0, n_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_gemm<TYPE, TT, MODE, BPS>, 256, 0) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        slots = per_cu * n_cu;
        cached[dev].store(slots, std::memory_order_relaxed);
    }
    return slots;
}

// Token tiles per work-group: 2 when its work-groups fill their last round of resident
// slots to ≥ 90 % or at least as well as single tiles would (two tiles decode each weight
// block once for 64 tokens), else 1.
template <int TYPE, int MODE>
static int gemm_tt_of(const DevMatrix& w, const ActQ8& a)
{
    const int ntt = a.Tpad >> 5, rg = (w.tiles + 3) / 4;
    auto fill = [&](int tt, int slots) {
        const int64_t blocks = (int64_t)rg * ((ntt + tt - 1) / tt);
        if (slots <= 0) return 0.0;
        const int64_t rounds = (blocks + slots - 1) / slots;
        return (double)blocks / (double)(rounds * slots);
    };
    if (ntt < 2) return 1;
    const double f2 = fill(2, gemm_slots<TYPE, 2, MODE, 2>());
    int slots1 = 0;
    if constexpr (TYPE == SHS_TYPE_Q4_0) slots1 = gemm_stage_blocks(w, 1) == 4 ? gemm_slots<TYPE, 1, MODE, 4>() : 0;
    if (slots1 == 0) slots1 = gemm_slots<TYPE, 1, MODE, 2>();
    if (f2 >= 0.9 || f2 >= fill(1, slots1)) return 2;
    return 1;
}

template <int TYPE, int MODE>
static hipError_t gemm_mode(const DevMatrix& w, const ActQ8& a, float* y, int ldy, hipStream_t s)
{
    if (gemm_tt_of<TYPE, MODE>(w, a) == 2) return gemm_launch<TYPE, 2, MODE>(w, a, y, ldy, s);
    return gemm_launch<TYPE, 1, MODE>(w, a, y, ldy, s);
}

template <int TYPE>
static hipError_t gemm_type(const DevMatrix& w, const ActQ8& a, float* y, int ldy, int mode, hipStream_t s)
{
    return mode == GEMM_ADD ? gemm_mode<TYPE, GEMM_ADD>(w, a, y, ldy, s) : gemm_mode<TYPE, GEMM_STORE>(w, a, y, ldy, s);
}

template <int TYPE>
static hipError_t gemm_swiglu_type(const DevMatrix& w, const ActQ8& a, int n_ft, const ActQ8& ao, hipStream_t s)
{
    if (gemm_tt_of<TYPE, GEMM_SWIGLU>(w, a) == 2) return gemm_launch<TYPE, 2, GEMM_SWIGLU>(w, a, nullptr, 0, s, ao, n_ft);
    return gemm_launch<TYPE, 1, GEMM_SWIGLU>(w, a, nullptr, 0, s, ao, n_ft);
}

template <int TYPE>
static hipError_t gemm_qkv_type(const DevMatrix& w, const ActQ8& a, float* y, int ldy, const RopeArgs& ra, hipStream_t s)
{
    if (gemm_tt_of<TYPE, GEMM_QKV>(w, a) == 2) return gemm_launch<TYPE, 2, GEMM_QKV>(w, a, y, ldy, s, ActQ8(), 0, ra);
    return gemm_launch<TYPE, 1, GEMM_QKV>(w, a, y, ldy, s, ActQ8(), 0, ra);
}

template <int TYPE>
static int gemm_tt_type(const DevMatrix& w, const ActQ8& a, int mode)
{
    if (mode == GEMM_QKV) return gemm_tt_of<TYPE, GEMM_QKV>(w, a);
    if (mode == GEMM_SWIGLU) return gemm_tt_of<TYPE, GEMM_SWIGLU>(w, a);
    return mode == GEMM_ADD ? gemm_tt_of<TYPE, GEMM_ADD>(w, a) : gemm_tt_of<TYPE, GEMM_STORE>(w, a);
}

int gemm_token_tiles(const DevMatrix& w, const ActQ8& a, int mode)
{
    switch (w.type) {
    case SHS_TYPE_Q4_0: return gemm_tt_type<SHS_TYPE_Q4_0>(w, a, mode);
    case SHS_TYPE_Q4_1: return gemm_tt_type<SHS_TYPE_Q4_1>(w, a, mode);
    case SHS_TYPE_Q5_0: return gemm_tt_type<SHS_TYPE_Q5_0>(w, a, mode);
    case SHS_TYPE_Q5_1: return gemm_tt_type<SHS_TYPE_Q5_1>(w, a, mode);
    case SHS_TYPE_Q8_0: return gemm_tt_type<SHS_TYPE_Q8_0>(w, a, mode);
    default: return 0;
    }
}

hipError_t launch_gemm_swiglu(const DevMatrix& w, const ActQ8& a, int n_ft, const ActQ8& out, hipStream_t s,
                              const NormIn* norm)
{
    if (w.tiles != 2 * n_ft || out.B != n_ft || out.Tpad != a.Tpad) return hipErrorInvalidValue;
    if (norm) {
        if (gemm_narrow_tokens(w, a, GEMM_SWIGLU, true) == 0) return hipErrorInvalidValue;
        return launch_gemm_narrow(w, a, nullptr, 0, GEMM_SWIGLU, s, out, n_ft, RopeArgs(), *norm);
    }
    if (gemm_narrow_tokens(w, a, GEMM_SWIGLU) > 0)
        return launch_gemm_narrow(w, a, nullptr, 0, GEMM_SWIGLU, s, out, n_ft, RopeArgs(), NormIn());
    switch (w.type) {
    case SHS_TYPE_Q4_0: return gemm_swiglu_type<SHS_TYPE_Q4_0>(w, a, n_ft, out, s);
    case SHS_TYPE_Q4_1: return gemm_swiglu_type<SHS_TYPE_Q4_1>(w, a, n_ft, out, s);
    case SHS_TYPE_Q5_0: return gemm_swiglu_type<SHS_TYPE_Q5_0>(w, a, n_ft, out, s);
    case SHS_TYPE_Q5_1: return gemm_swiglu_type<SHS_TYPE_Q5_1>(w, a, n_ft, out, s);
    case SHS_TYPE_Q8_0: return gemm_swiglu_type<SHS_TYPE_Q8_0>(w, a, n_ft, out, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm_qkv(const DevMatrix& w, const ActQ8& a, float* y, int ldy, const RopeArgs& ra, hipStream_t s,
                           const NormIn* norm)
{
    if (ra.hd % 32 != 0 || w.rows != (ra.n_head + 2 * ra.n_kv) * ra.hd || (ldy & 3) != 0 ||
        (reinterpret_cast<uintptr_t>(y) & 15) != 0)
        return hipErrorInvalidValue;
    if (norm) {
        if (gemm_narrow_tokens(w, a, GEMM_QKV, true) == 0) return hipErrorInvalidValue;
        return launch_gemm_narrow(w, a, y, ldy, GEMM_QKV, s, ActQ8(), 0, ra, *norm);
    }
    if (gemm_narrow_tokens(w, a, GEMM_QKV) > 0)
        return launch_gemm_narrow(w, a, y, ldy, GEMM_QKV, s, ActQ8(), 0, ra, NormIn());
    switch (w.type) {
    case SHS_TYPE_Q4_0: return gemm_qkv_type<SHS_TYPE_Q4_0>(w, a, y, ldy, ra, s);
    case SHS_TYPE_Q4_1: return gemm_qkv_type<SHS_TYPE_Q4_1>(w, a, y, ldy, ra, s);
    case SHS_TYPE_Q5_0: return gemm_qkv_type<SHS_TYPE_Q5_0>(w, a, y, ldy, ra, s);
    case SHS_TYPE_Q5_1: return gemm_qkv_type<SHS_TYPE_Q5_1>(w, a, y, ldy, ra, s);
    case SHS_TYPE_Q8_0: return gemm_qkv_type<SHS_TYPE_Q8_0>(w, a, y, ldy, ra, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm(const DevMatrix& w, const ActQ8& a, float* y, int ldy, int mode, hipStream_t s)
{
    if ((mode == GEMM_STORE || mode == GEMM_ADD) && gemm_narrow_tokens(w, a, mode) > 0)
        return launch_gemm_narrow(w, a, y, ldy, mode, s, ActQ8(), 0, RopeArgs(), NormIn());
    switch (w.type) {
    case SHS_TYPE_Q4_0: return gemm_type<SHS_TYPE_Q4_0>(w, a, y, ldy, mode, s);
    case SHS_TYPE_Q4_1: return gemm_type<SHS_TYPE_Q4_1>(w, a, y, ldy, mode, s);
    case SHS_TYPE_Q5_0: return gemm_type<SHS_TYPE_Q5_0>(w, a, y, ldy, mode, s);
    case SHS_TYPE_Q5_1: return gemm_type<SHS_TYPE_Q5_1>(w, a, y, ldy, mode, s);
    case SHS_TYPE_Q8_0: return gemm_type<SHS_TYPE_Q8_0>(w, a, y, ldy, mode, s);
    default: return hipErrorInvalidValue;
    }
}

// The GEMM's exact block sums, out[t][r][b], through the same two MFMA steps (integer sum
// onto the magic pattern, then conversion with the zero point) — parity instrumentation.
template <int TYPE>
__global__ __launch_bounds__(256) void k_gemm_sums(const uint8_t* __restrict__ wqs, const uint32_t* __restrict__ wqh,
                                                   int ntiles, int B, ActQ8 a, int32_t* __restrict__ out, int N)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 31, h = lane >> 5;
    const int rt = blockIdx.x * 4 + wave;
    if (rt >= ntiles) return;
    const int tile = blockIdx.y;
    const int token = tile * 32 + j;
    constexpr int Z = ZeroPoint<TYPE>::z;
    const uint4* aq = reinterpret_cast<const uint4*>(a.q);
    const v16i magic = magic16();
    v4h acv;
    for (int k = 0; k < 4; k++) acv[k] = (_Float16)0.0f;
    if (h == 0) {
        acv[0] = (_Float16)2048.0f;
        acv[1] = (_Float16)(float)(64 * Z);
        acv[2] = (_Float16)(float)Z;
    }
    for (int b = 0; b < B; ++b) {
        const v4i w = load_weight_i8<TYPE>(wqs, wqh, (int64_t)rt * B + b, j, h);
        const v4i q = __builtin_bit_cast(v4i, aq[((int64_t)tile * B + b) * 64 + h * 32 + j]);
        const v16i F = __builtin_amdgcn_mfma_i32_32x32x32_i8(w, q, magic, 0, 0, 0);
        const v4h c = __builtin_bit_cast(v4h, a.cv[(int64_t)b * a.Tpad + token]);
        const v16f G = __builtin_amdgcn_mfma_f32_32x32x8f16(acv, c, __builtin_bit_cast(v16f, F), 0, 0, 0);
        if (token < a.T)
            for (int r = 0; r < 16; r++) {
                const int row = rt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < N) out[((int64_t)token * N + row) * B + b] = (int32_t)G[r];
            }
    }
}

hipError_t launch_gemm_block_sums(const DevMatrix& w, const ActQ8& a, int32_t* out, hipStream_t s)
{
    dim3 grid((unsigned)((w.tiles + 3) / 4), (unsigned)(a.Tpad >> 5)), block(256);
    switch (w.type) {
    case SHS_TYPE_Q4_0: hipLaunchKernelGGL(k_gemm_sums<SHS_TYPE_Q4_0>, grid, block, 0, s, w.qs, w.qh, w.tiles, w.blocks, a, out, w.rows); break;
    case SHS_TYPE_Q4_1: hipLaunchKernelGGL(k_gemm_sums<SHS_TYPE_Q4_1>, grid, block, 0, s, w.qs, w.qh, w.tiles, w.blocks, a, out, w.rows); break;
    case SHS_TYPE_Q5_0: hipLaunchKernelGGL(k_gemm_sums<SHS_TYPE_Q5_0>, grid, block, 0, s, w.qs, w.qh, w.tiles, w.blocks, a, out, w.rows); break;
    case SHS_TYPE_Q5_1: hipLaunchKernelGGL(k_gemm_sums<SHS_TYPE_Q5_1>, grid, block, 0, s, w.qs, w.qh, w.tiles, w.blocks, a, out, w.rows); break;
    case SHS_TYPE_Q8_0: hipLaunchKernelGGL(k_gemm_sums<SHS_TYPE_Q8_0>, grid, block, 0, s, w.qs, w.qh, w.tiles, w.blocks, a, out, w.rows); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------------ GEMV (selected rows)

// Weight element e (0..31) of one row's block as a signed integer (u − z, or u).
template <int TYPE>
__device__ __forceinline__ int weight_elem(const uint8_t* q, uint32_t qh, int e)
{
    if (TYPE == SHS_TYPE_Q8_0) return (int)(int8_t)q[e];
    const int j = e & 15;
    int u = e < 16 ? (q[j] & 0x0F) : (q[j] >> 4);
    if (TYPE == SHS_TYPE_Q5_0 || TYPE == SHS_TYPE_Q5_1) u |= (int)(((qh >> e) & 1u) << 4);
    return TYPE == SHS_TYPE_Q4_0 ? u - 8 : TYPE == SHS_TYPE_Q5_0 ? u - 16 : u;
}

// One wave per (token, selected row). The lanes form the exact integer block sums and the
// scales of all blocks in parallel; lane 0 then runs the serial epilogue over the blocks in
// order — the GEMM's arithmetic, so every value equals the corresponding entry of the full
// product bit for bit (QuantMatMul.ForwardRowsAsync, QuantMatMul.cs:98-110).
template <int TYPE>
__global__ __launch_bounds__(64) void k_gemv_rows(const uint8_t* __restrict__ wqs, const uint32_t* __restrict__ wqh,
                                                  const float* __restrict__ wd, const float* __restrict__ wm, int B,
                                                  const int32_t* __restrict__ ids, int n_ids, ActQ8 a,
                                                  float* __restrict__ y)
{
    constexpr bool OFF = (TYPE == SHS_TYPE_Q4_1 || TYPE == SHS_TYPE_Q5_1);
    extern __shared__ float sh[];  // I_b as float (exact), RN(d_w·d_a), then m_w and d_a·Σq for the offset types
    float* sI = sh;
    float* sS = sh + B;
    float* sM = sh + 2 * B;
    float* sD = sh + 3 * B;
    const int i = blockIdx.x % n_ids, t = blockIdx.x / n_ids;
    const int r = ids[i];
    const int ri = r & 31;
    for (int b = threadIdx.x; b < B; b += 64) {
        const int64_t rec = (int64_t)(r >> 5) * B + b;
        // code position p (half p/16, index p%16) holds element perm_elem(p)
        const int8_t* act = a.q + (((int64_t)(t >> 5) * B + b) * 2 * 32 + (t & 31)) * 16;
        int I = 0;
        if (TYPE == SHS_TYPE_Q8_0) {
            const uint8_t* q = wqs + rec * 1024 + ri * 32;  // stored in the same element order
            for (int p = 0; p < 32; p++) I += (int)(int8_t)q[p] * (int)act[(p >> 4) * 512 + (p & 15)];
        } else {
            const uint8_t* q = wqs + rec * 512 + ri * 16;
            const uint32_t qh = (TYPE == SHS_TYPE_Q5_0 || TYPE == SHS_TYPE_Q5_1) ? wqh[rec * 32 + ri] : 0u;
            for (int p = 0; p < 32; p++)
                I += weight_elem<TYPE>(q, qh, perm_elem(p)) * (int)act[(p >> 4) * 512 + (p & 15)];
        }
        sI[b] = (float)I;
        sS[b] = wd[rec * 32 + ri] * a.d[(int64_t)b * a.Tpad + t];
        if (OFF) {
            sM[b] = wm[rec * 32 + ri];
            sD[b] = a.ds[(int64_t)b * a.Tpad + t];
        }
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    float acc = 0.0f;
    for (int b = 0; b < B; ++b) {
        acc = fmaf(sI[b], sS[b], acc);
        if (OFF) acc = fmaf(sM[b], sD[b], acc);
    }
    y[(int64_t)t * n_ids + i] = acc;
}

hipError_t launch_gemv_rows(const DevMatrix& w, const ActQ8& a, const int32_t* ids, int n_ids, float* y,
                            hipStream_t s)
{
    const int64_t n = (int64_t)a.T * n_ids;
    if (n <= 0) return hipSuccess;
    dim3 grid((unsigned)n), block(64);
    const size_t shm = sizeof(float) * 4 * (size_t)w.blocks;
    switch (w.type) {
    case SHS_TYPE_Q4_0: hipLaunchKernelGGL(k_gemv_rows<SHS_TYPE_Q4_0>, grid, block, shm, s, w.qs, w.qh, w.d, w.m, w.blocks, ids, n_ids, a, y); break;
    case SHS_TYPE_Q4_1: hipLaunchKernelGGL(k_gemv_rows<SHS_TYPE_Q4_1>, grid, block, shm, s, w.qs, w.qh, w.d, w.m, w.blocks, ids, n_ids, a, y); break;
    case SHS_TYPE_Q5_0: hipLaunchKernelGGL(k_gemv_rows<SHS_TYPE_Q5_0>, grid, block, shm, s, w.qs, w.qh, w.d, w.m, w.blocks, ids, n_ids, a, y); break;
    case SHS_TYPE_Q5_1: hipLaunchKernelGGL(k_gemv_rows<SHS_TYPE_Q5_1>, grid, block, shm, s, w.qs, w.qh, w.d, w.m, w.blocks, ids, n_ids, a, y); break;
    case SHS_TYPE_Q8_0: hipLaunchKernelGGL(k_gemv_rows<SHS_TYPE_Q8_0>, grid, block, shm, s, w.qs, w.qh, w.d, w.m, w.blocks, ids, n_ids, a, y); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------- narrow GEMM (decode, T ≤ 4)

// Rows per work-group (R): 8 for the smaller layer projections (many work-groups for a few MB
// of weights), 16 from 16k rows and for the fused q|k|v (whose work-groups each normalize the
// hidden row first: half as many of them measured ≈1 µs faster), 32 from 64k rows (the
// vocabulary head: one tile per work-group, its activation staging spread over 4× the
// weights); the fused gate|up takes a gate tile and its up tile (64 rows), so a work-group
// owns whole 32-feature blocks.
static int narrow_rows(const DevMatrix& w, int mode)
{
    if (mode == GEMM_SWIGLU) return 64;
    return w.rows >= 65536 ? 32 : (w.rows >= 16384 || mode == GEMM_QKV) ? 16 : 8;
}

// Row-blocks per batch and thread: 8 when a thread owns many blocks (64-row work-groups).
__host__ __device__ constexpr int narrow_nb(int R) { return R >= 64 ? 8 : 4; }

// Bytes of dynamic LDS k_gemm_narrow<.., R> needs for B blocks and nt tokens: the activation
// codes, then per (token, row, block) the pair (I, RN(d_w·d_a)), then m_w per (row, block)
// for the offset types, then Σa, d_a and RN(d_a·Σa) per (token, block).
static size_t narrow_lds_bytes(int R, int B, int nt, bool off)
{
    const size_t pb = (size_t)B + 1;
    return 32 * (size_t)nt * B + 8 * (size_t)nt * R * pb + (off ? 4 * (size_t)R * pb : 0) + 4 * (size_t)nt * B * 3;
}

// One batch of a thread's row-blocks: blocks b0 + j·(256/R), j < NB, clamped to the last
// block (a clamped load re-reads a line the work-group already has).
template <int TYPE, int NB>
struct NarrowBatch {
    uint4 q[NB], q8[NB];
    uint32_t qh[NB];
    float dw[NB], mw[NB];
};

template <int TYPE, int R, int NB>
__device__ __forceinline__ void narrow_load(NarrowBatch<TYPE, NB>& nb, const uint8_t* __restrict__ wqs,
                                            const uint32_t* __restrict__ wqh, const float* __restrict__ wd,
                                            const float* __restrict__ wm, int64_t rec0, int ri, int b0, int B)
{
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int64_t rec = rec0 + min(b0 + j * (256 / R), B - 1);
        if (TYPE == SHS_TYPE_Q8_0) {
            nb.q[j] = *reinterpret_cast<const uint4*>(wqs + rec * 1024 + ri * 32);
            nb.q8[j] = *reinterpret_cast<const uint4*>(wqs + rec * 1024 + ri * 32 + 16);
        } else {
            nb.q[j] = *reinterpret_cast<const uint4*>(wqs + rec * 512 + ri * 16);
        }
        if (TYPE == SHS_TYPE_Q5_0 || TYPE == SHS_TYPE_Q5_1) nb.qh[j] = wqh[rec * 32 + ri];
        nb.dw[j] = wd[rec * 32 + ri];
        if (TYPE == SHS_TYPE_Q4_1 || TYPE == SHS_TYPE_Q5_1) nb.mw[j] = wm[rec * 32 + ri];
    }
}

// y = x·Wᵀ for NT ≤ 4 tokens: single-token decode and the full-vocabulary head at the last
// position. At this width the weights are streamed once from HBM and the int8 MFMA's
// 32-token tiles would be mostly padding, so a work-group takes R rows × all blocks:
// - the first batch of weight loads is issued, then the activation codes, d_a, Σa (from the
//   conversion column) and RN(d_a·Σa) are staged in the LDS under its latency;
// - phase 1: thread (row r = tid % R, blocks b ≡ tid / R mod 256/R, NB per batch, the next
//   batch loading while this one computes) forms the exact block sums I = Σu·a − z·Σa of
//   every token with v_dot4 and the scale RN(d_w·d_a) into the LDS;
// - phase 2: lane (t, r) runs the reference's chain acc = fma(I_b, RN(d_w·d_a), acc)
//   [then fma(m_w, RN(d_a·Σa), acc) for the offset types] over b in order
//   (IntegerGemm.cs:384-397) — k_gemm's arithmetic, so an output does not depend on the
//   path that computed it;
// - the epilogue by mode, as k_gemm's: 0 store, 1 add into y; 3 (q|k|v) RoPE on adjacent
//   row pairs (neighbouring lanes), the query position scale, q into y and k, v into the KV
//   cache; 2 (gate|up, work-group = gate tile f and up tile f) SwiGLU of each feature, then
//   the 32-feature block quantized into the down projection's codes `ao`.
// The grid is a multiple of 8 and work-group g of the logical order runs on XCD g / (grid/8):
// the work-groups of a 32-row tile share its d (and qh, m) lines in one L2.
template <int TYPE, int NT, int MODE, int R>
__global__ __launch_bounds__(256) void k_gemm_narrow(const uint8_t* __restrict__ wqs, const uint32_t* __restrict__ wqh,
                                                     const float* __restrict__ wd, const float* __restrict__ wm,
                                                     int rows, int B, int n_wg, ActQ8 a, float* __restrict__ y, int ldy,
                                                     ActQ8 ao, int n_ft, RopeArgs ra, NormIn nin)
{
    constexpr bool OFF = TYPE == SHS_TYPE_Q4_1 || TYPE == SHS_TYPE_Q5_1;
    constexpr bool Q8 = TYPE == SHS_TYPE_Q8_0;
    constexpr int Z = ZeroPoint<TYPE>::z;
    constexpr int BS = 256 / R;  // block stride between a thread's row-blocks
    constexpr int NB = narrow_nb(R);
    static_assert(MODE != GEMM_SWIGLU || R == 64, "the gate|up epilogue pairs a gate tile with its up tile");
    const int g = (int)(blockIdx.x & 7) * (int)(gridDim.x >> 3) + (int)(blockIdx.x >> 3);
    if (g >= n_wg) return;
    extern __shared__ uint4 nw_lds[];
    const int PB = B + 1;  // odd float2 stride: the chain lanes read different banks
    uint4* sA = nw_lds;                                              // [NT][B][2 halves] codes
    float2* sP = reinterpret_cast<float2*>(sA + NT * B * 2);         // [NT][R][PB] (I, RN(d_w·d_a))
    float* sM = reinterpret_cast<float*>(sP + NT * R * PB);          // [R][PB] m_w
    int* sSum = reinterpret_cast<int*>(sM + (OFF ? R * PB : 0));     // [NT][B] Σa
    float* sDa = reinterpret_cast<float*>(sSum + NT * B);            // [NT][B] d_a
    float* sDs = sDa + NT * B;                                       // [NT][B] RN(d_a·Σa)
    const int tid = threadIdx.x;
    const int r = tid % R, bl = tid / R;
    // the work-group's local row r: gate row 32g + r or up row 32(n_ft + g) + r − 32 (mode 2),
    // else row gR + r (< tiles·32: n_wg covers the padded rows exactly)
    auto global_row = [&](int lr) {
        return MODE == GEMM_SWIGLU ? (lr < 32 ? 32 * g + lr : 32 * (n_ft + g) + lr - 32) : g * R + lr;
    };
    const int row = global_row(r);
    const int64_t rec0 = (int64_t)(row >> 5) * B;
    const int ri = row & 31;

    // The first batch of weight loads is issued before the input is staged, or, when the
    // work-group normalizes the hidden row itself, right after the row's loads: the RMSNorm
    // then runs while the batch is in flight (its barriers wait for the LDS only).
    // (only the q|k|v and gate|up launches normalize their own input; the other modes are
    // compiled without that path)
    constexpr bool NORM_MODE = MODE == GEMM_QKV || MODE == GEMM_SWIGLU;
    const bool norm_in = NORM_MODE && nin.x != nullptr;
    NarrowBatch<TYPE, NB> cur, nxt;
    if (!norm_in) narrow_load<TYPE, R, NB>(cur, wqs, wqh, wd, wm, rec0, ri, bl, B);

    // the staged input: codes, d_a and Σa of the NT tokens from the activation buffers
    auto stage_codes = [&] {
        for (int i = tid; i < NT * B * 2; i += 256) {
            const int t = i / (2 * B), rem = i - t * 2 * B, b = rem >> 1, h = rem & 1;
            sA[i] = *reinterpret_cast<const uint4*>(a.q + (((int64_t)(t >> 5) * B + b) * 64 + (t & 31)) * 16 + h * 512);
        }
        for (int i = tid; i < NT * B; i += 256) {
            const int t = i / B, b = i - t * B;
            const int64_t k = (int64_t)b * a.Tpad + t;
            sDa[i] = a.d[k];
            if (OFF) sDs[i] = a.ds[k];
            if (Z != 0) {
                // the conversion column holds fp16 (−6144, −hi, −lo, 0) with Σa = 64·hi + lo
                const uint2 cv = a.cv[k];
                const int hi = (int)(float)__builtin_bit_cast(_Float16, (uint16_t)(cv.x >> 16));
                const int lo = (int)(float)__builtin_bit_cast(_Float16, (uint16_t)(cv.y & 0xFFFFu));
                sSum[i] = -(64 * hi + lo);
            }
        }
        __syncthreads();
    };
    if constexpr (NORM_MODE) {
        if (norm_in) {
            // the codes formed here from the hidden rows: Kernels.RmsNorm, then the 32-block
            // quantization, into the arrays the staged codes would fill (the row's scratch follows)
            // (offset from the LDS base, so the pointer keeps the LDS address space)
            const int nsx_off = (int)(reinterpret_cast<const char*>(sDs + NT * B) - reinterpret_cast<const char*>(nw_lds));
            float* nsx = reinterpret_cast<float*>(reinterpret_cast<char*>(nw_lds) + ((nsx_off + 15) & ~15));
            uint8_t* sAb = reinterpret_cast<uint8_t*>(sA);
            const int K = 32 * B;
            for (int t = 0; t < NT; ++t) {
                rmsnorm_rows(nin.x + (int64_t)t * nin.ldx, nin.w, nin.eps, K, nsx, nsx + 2 * K, nsx + 2 * K + 16,
                             [&](float4 v, int l8, int b) {
                                 const QBlock qb = quant_block8_values(v, 0);
                                 // element group 4·l8 .. +3 sits in half (l8 >> 1) & 1 (the act_code_offset order)
                                 const int hf = (l8 >> 1) & 1, idx = 4 * (l8 & 1) + 8 * (l8 >> 2);
                                 *reinterpret_cast<uint32_t*>(sAb + ((t * B + b) * 2 + hf) * 16 + idx) = qb.w;
                                 if (l8 == 0) {
                                     sDa[t * B + b] = qb.d;
                                     sSum[t * B + b] = correction_sum(qb.sum);
                                     sDs[t * B + b] = qb.d * (float)qb.sum;
                                 }
                             },
                             [&] {
                                 if (t == 0) narrow_load<TYPE, R, NB>(cur, wqs, wqh, wd, wm, rec0, ri, bl, B);
                             });
                lds_barrier();
            }
        } else {
            stage_codes();
        }
    } else {
        stage_codes();
    }

    // batches of NB·BS blocks; the next batch is prefetched only when there is one
    const int n_batch = (B + NB * BS - 1) / (NB * BS);
    for (int bt = 0; bt < n_batch; bt++) {
        const int b0 = bl + bt * NB * BS;
        if (bt + 1 < n_batch) narrow_load<TYPE, R, NB>(nxt, wqs, wqh, wd, wm, rec0, ri, b0 + NB * BS, B);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int b = b0 + j * BS;
            if (b < B) {
                const v4i w0 = Q8 ? v4i{(int)cur.q[j].x, (int)cur.q[j].y, (int)cur.q[j].z, (int)cur.q[j].w}
                                  : weights_i8<TYPE>(cur.q[j].x, cur.q[j].y, 0u, 0u, cur.qh[j], 0);
                const v4i w1 = Q8 ? v4i{(int)cur.q8[j].x, (int)cur.q8[j].y, (int)cur.q8[j].z, (int)cur.q8[j].w}
                                  : weights_i8<TYPE>(cur.q[j].z, cur.q[j].w, 0u, 0u, cur.qh[j], 1);
                if (OFF) sM[r * PB + b] = cur.mw[j];
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const uint4 a0 = sA[(t * B + b) * 2], a1 = sA[(t * B + b) * 2 + 1];
                    int s = 0;
                    s = __builtin_amdgcn_sdot4(w0[0], (int)a0.x, s, false);
                    s = __builtin_amdgcn_sdot4(w0[1], (int)a0.y, s, false);
                    s = __builtin_amdgcn_sdot4(w0[2], (int)a0.z, s, false);
                    s = __builtin_amdgcn_sdot4(w0[3], (int)a0.w, s, false);
                    s = __builtin_amdgcn_sdot4(w1[0], (int)a1.x, s, false);
                    s = __builtin_amdgcn_sdot4(w1[1], (int)a1.y, s, false);
                    s = __builtin_amdgcn_sdot4(w1[2], (int)a1.z, s, false);
                    s = __builtin_amdgcn_sdot4(w1[3], (int)a1.w, s, false);
                    if (Z != 0) s -= Z * sSum[t * B + b];
                    sP[(t * R + r) * PB + b] = make_float2((float)s, cur.dw[j] * sDa[t * B + b]);
                }
            }
        }
        if (bt + 1 < n_batch) cur = nxt;
    }
    __syncthreads();

    const bool chain = tid < NT * R;
    const int t = tid / R, rr = tid % R;  // chain lane (token, local row)
    float acc = 0.0f;
    if (chain) {
        const float2* p = sP + (t * R + rr) * PB;
        const float* pm = sM + rr * PB;
        const float* pd = sDs + t * B;
        // The chain's operands are read 16 steps at a time into two alternating register sets:
        // the next 16 steps' reads are issued (kept ahead by an empty asm that takes acc) before the
        // current 16 FMAs run, so the LDS latency is paid about once instead of once per 16
        // steps.
        const int bfull = B & ~15;
        float2 va[16], vb[16];
        float ma[16], da[16], mb[16], db[16];
#define SHS_CHAIN_LOAD(V, M, D, B0)                            \
    _Pragma("unroll") for (int k = 0; k < 16; k++)             \
    {                                                          \
        V[k] = p[(B0) + k];                                    \
        if (OFF) {                                             \
            M[k] = pm[(B0) + k];                               \
            D[k] = pd[(B0) + k];                               \
        }                                                      \
    }                                                          \
    asm volatile("" : "+v"(acc)::"memory");
#define SHS_CHAIN_RUN(V, M, D)                                 \
    _Pragma("unroll") for (int k = 0; k < 16; k++)             \
    {                                                          \
        acc = fmaf(V[k].x, V[k].y, acc);                       \
        if (OFF) acc = fmaf(M[k], D[k], acc);                  \
    }
        int b = 0;
        if (bfull > 0) SHS_CHAIN_LOAD(va, ma, da, 0);
        for (; b + 32 <= bfull; b += 32) {
            SHS_CHAIN_LOAD(vb, mb, db, b + 16);
            SHS_CHAIN_RUN(va, ma, da);
            // (no round after the next: the current one again, unused, from a uniform base)
            SHS_CHAIN_LOAD(va, ma, da, b + 48 <= bfull ? b + 32 : b);
            SHS_CHAIN_RUN(vb, mb, db);
        }
        if (b < bfull) {
            SHS_CHAIN_RUN(va, ma, da);
            b += 16;
        }
#undef SHS_CHAIN_LOAD
#undef SHS_CHAIN_RUN
        for (; b < B; ++b) {
            const float2 v = p[b];
            acc = fmaf(v.x, v.y, acc);
            if (OFF) acc = fmaf(pm[b], pd[b], acc);
        }
    }

    if (MODE == GEMM_STORE || MODE == GEMM_ADD) {
        const int orow = global_row(rr);
        if (chain && orow < rows) {
            float* dst = y + (int64_t)t * ldy + orow;
            *dst = MODE == GEMM_ADD ? *dst + acc : acc;
        }
    } else if (MODE == GEMM_QKV) {
        // Rope.Apply on the pair (2i, 2i+1) of a head (Rope.cs:112-135): the pair's rows are
        // neighbouring chain lanes (R and the head size are even); every chain lane takes part
        // in the exchange, whole quads of the first wave
        const float other = dpp_f<DPP_XOR1>(acc);
        const int orow = global_row(rr);
        if (chain && orow < rows) {
            const int hh = orow / ra.hd, d = orow - hh * ra.hd, i = d >> 1;
            const int p = ra.pos[t];
            float v = acc;
            if (hh < ra.n_head + ra.n_kv && i < ra.half) {
                const float c = ra.ct[(int64_t)p * ra.half + i], s = ra.st[(int64_t)p * ra.half + i];
                const float x0 = (d & 1) ? other : acc, x1 = (d & 1) ? acc : other;
                v = (d & 1) ? x0 * s + x1 * c : x0 * c - x1 * s;
            }
            if (hh < ra.n_head) {
                const float qs = ra.qscale[p];
                if (qs != 1.0f) v = v * qs;  // ApplyPositionScale (MinistralModel.cs:476-482)
                y[(int64_t)t * ldy + orow] = v;
            } else if (hh < ra.n_head + ra.n_kv) {
                ra.kc[((int64_t)(hh - ra.n_head) * ra.cap + ra.slot0 + t) * ra.hd + d] = v;
            } else {
                ra.vc[((int64_t)(hh - ra.n_head - ra.n_kv) * ra.cap + ra.slot0 + t) * ra.hd + d] = v;
            }
        }
    } else {  // GEMM_SWIGLU
        // Kernels.SwiGlu (Kernels.cs:83-90): y = sigmoid(g)·(g·u) per feature, then the block's
        // quantization (8 lanes per token, 4 features each)
        float* sOut = reinterpret_cast<float*>(sA);  // the codes are no longer read
        if (chain) sOut[t * 64 + rr] = acc;
        __syncthreads();
        if (tid < 8 * NT) {
            const int tq = tid >> 3, l8 = tid & 7;
            const float* go = sOut + tq * 64 + 4 * l8;
            const float* uo = go + 32;
            float4 v;
            v.x = (1.0f / (1.0f + det_expf(-go[0]))) * (go[0] * uo[0]);
            v.y = (1.0f / (1.0f + det_expf(-go[1]))) * (go[1] * uo[1]);
            v.z = (1.0f / (1.0f + det_expf(-go[2]))) * (go[2] * uo[2]);
            v.w = (1.0f / (1.0f + det_expf(-go[3]))) * (go[3] * uo[3]);
            quant_block8(v, l8, ao, tq, g, 0);
        }
    }
}

// LDS for a work-group that forms its own codes (NormIn): one hidden row and its squares,
// then the 16 running sums and the scale
static size_t narrow_norm_lds_bytes(int B) { return sizeof(float) * (2 * 32 * (size_t)B + 17) + 16; }

template <int TYPE, int NT, int MODE, int R>
static hipError_t narrow_launch(const DevMatrix& w, const ActQ8& a, float* y, int ldy, hipStream_t s,
                                const ActQ8& ao, int n_ft, const RopeArgs& ra, const NormIn& nin)
{
    constexpr bool OFF = TYPE == SHS_TYPE_Q4_1 || TYPE == SHS_TYPE_Q5_1;
    const int n_wg = MODE == GEMM_SWIGLU ? n_ft : w.tiles * (32 / R);
    const size_t shm = narrow_lds_bytes(R, w.blocks, NT, OFF) + (nin.x ? narrow_norm_lds_bytes(w.blocks) : 0);
    static LdsLimit limit;
    hipError_t e = limit.raise(reinterpret_cast<const void*>(k_gemm_narrow<TYPE, NT, MODE, R>), shm);
    if (e != hipSuccess) return e;
    dim3 grid((unsigned)((n_wg + 7) / 8 * 8)), block(256);
    hipLaunchKernelGGL((k_gemm_narrow<TYPE, NT, MODE, R>), grid, block, shm, s, w.qs, w.qh, w.d, w.m, w.rows,
                       w.blocks, n_wg, a, y, ldy, ao, n_ft, ra, nin);
    return hipGetLastError();
}

template <int TYPE, int NT, int MODE>
static hipError_t narrow_rows_launch(const DevMatrix& w, const ActQ8& a, float* y, int ldy, hipStream_t s,
                                     const ActQ8& ao, int n_ft, const RopeArgs& ra, const NormIn& nin)
{
    if constexpr (MODE == GEMM_SWIGLU) {
        return narrow_launch<TYPE, NT, MODE, 64>(w, a, y, ldy, s, ao, n_ft, ra, nin);
    } else {
        switch (narrow_rows(w, MODE)) {
        case 32: return narrow_launch<TYPE, NT, MODE, 32>(w, a, y, ldy, s, ao, n_ft, ra, nin);
        case 16: return narrow_launch<TYPE, NT, MODE, 16>(w, a, y, ldy, s, ao, n_ft, ra, nin);
        default: return narrow_launch<TYPE, NT, MODE, 8>(w, a, y, ldy, s, ao, n_ft, ra, nin);
        }
    }
}

template <int TYPE, int MODE>
static hipError_t narrow_mode(const DevMatrix& w, const ActQ8& a, float* y, int ldy, hipStream_t s,
                              const ActQ8& ao, int n_ft, const RopeArgs& ra, const NormIn& nin)
{
    switch (a.T) {
    case 1: return narrow_rows_launch<TYPE, 1, MODE>(w, a, y, ldy, s, ao, n_ft, ra, nin);
    case 2: return narrow_rows_launch<TYPE, 2, MODE>(w, a, y, ldy, s, ao, n_ft, ra, nin);
    case 3: return narrow_rows_launch<TYPE, 3, MODE>(w, a, y, ldy, s, ao, n_ft, ra, nin);
    default: return narrow_rows_launch<TYPE, 4, MODE>(w, a, y, ldy, s, ao, n_ft, ra, nin);
    }
}

template <int TYPE>
static hipError_t narrow_type(const DevMatrix& w, const ActQ8& a, float* y, int ldy, int mode, hipStream_t s,
                              const ActQ8& ao, int n_ft, const RopeArgs& ra, const NormIn& nin)
{
    switch (mode) {
    case GEMM_ADD: return narrow_mode<TYPE, GEMM_ADD>(w, a, y, ldy, s, ao, n_ft, ra, nin);
    case GEMM_SWIGLU: return narrow_mode<TYPE, GEMM_SWIGLU>(w, a, y, ldy, s, ao, n_ft, ra, nin);
    case GEMM_QKV: return narrow_mode<TYPE, GEMM_QKV>(w, a, y, ldy, s, ao, n_ft, ra, nin);
    default: return narrow_mode<TYPE, GEMM_STORE>(w, a, y, ldy, s, ao, n_ft, ra, nin);
    }
}

static hipError_t launch_gemm_narrow(const DevMatrix& w, const ActQ8& a, float* y, int ldy, int mode, hipStream_t s,
                                     const ActQ8& ao, int n_ft, const RopeArgs& ra, const NormIn& nin)
{
    switch (w.type) {
    case SHS_TYPE_Q4_0: return narrow_type<SHS_TYPE_Q4_0>(w, a, y, ldy, mode, s, ao, n_ft, ra, nin);
    case SHS_TYPE_Q4_1: return narrow_type<SHS_TYPE_Q4_1>(w, a, y, ldy, mode, s, ao, n_ft, ra, nin);
    case SHS_TYPE_Q5_0: return narrow_type<SHS_TYPE_Q5_0>(w, a, y, ldy, mode, s, ao, n_ft, ra, nin);
    case SHS_TYPE_Q5_1: return narrow_type<SHS_TYPE_Q5_1>(w, a, y, ldy, mode, s, ao, n_ft, ra, nin);
    case SHS_TYPE_Q8_0: return narrow_type<SHS_TYPE_Q8_0>(w, a, y, ldy, mode, s, ao, n_ft, ra, nin);
    default: return hipErrorInvalidValue;
    }
}

int gemm_narrow_tokens(const DevMatrix& w, const ActQ8& a, int mode, bool with_norm)
{
    if (a.T < 1 || a.T > NARROW_MAX_T || !type_supported(w.type)) return 0;
    const bool off = type_has_offset(w.type);
    const size_t lds = narrow_lds_bytes(narrow_rows(w, mode), w.blocks, a.T, off) +
                       (with_norm ? narrow_norm_lds_bytes(w.blocks) : 0);
    return lds <= (160u << 10) ? a.T : 0;
}

// -------------------------------------------------------- embedding gather

// QuantMatMul.GatherRows → Dequantizer (QuantMatMul.cs:534-545, Dequantizer.cs:127-213),
// read from the repacked table: one thread per (token, block).
template <int TYPE>
__global__ void k_embed(const uint8_t* __restrict__ wqs, const uint32_t* __restrict__ wqh, const float* __restrict__ wd,
                        const float* __restrict__ wm, int B, const int32_t* __restrict__ ids, int n,
                        float* __restrict__ h, int ldh)
{
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)n * B) return;
    const int b = (int)(idx % B), t = (int)(idx / B);
    const int r = ids[t], ri = r & 31;
    const int64_t rec = (int64_t)(r >> 5) * B + b;
    const float d = wd[rec * 32 + ri];
    float* out = h + (int64_t)t * ldh + 32 * b;
    if (TYPE == SHS_TYPE_Q8_0) {
        const int8_t* q = reinterpret_cast<const int8_t*>(wqs + rec * 1024 + ri * 32);
        for (int p = 0; p < 32; p++) out[perm_elem(p)] = (float)q[p] * d;
        return;
    }
    const uint8_t* q = wqs + rec * 512 + ri * 16;
    const uint32_t qh = (TYPE == SHS_TYPE_Q5_0 || TYPE == SHS_TYPE_Q5_1) ? wqh[rec * 32 + ri] : 0u;
    const float m = (TYPE == SHS_TYPE_Q4_1 || TYPE == SHS_TYPE_Q5_1) ? wm[rec * 32 + ri] : 0.0f;
    for (int jj = 0; jj < 16; jj++) {
        int lo = q[jj] & 0x0F, hi = q[jj] >> 4;
        if (TYPE == SHS_TYPE_Q5_0 || TYPE == SHS_TYPE_Q5_1) {
            lo |= (int)(((qh >> jj) & 1u) << 4);
            hi |= (int)(((qh >> (jj + 16)) & 1u) << 4);
        }
        if (TYPE == SHS_TYPE_Q4_0) { out[jj] = d * (float)(lo - 8); out[16 + jj] = d * (float)(hi - 8); }
        else if (TYPE == SHS_TYPE_Q5_0) { out[jj] = d * (float)(lo - 16); out[16 + jj] = d * (float)(hi - 16); }
        else { float a0 = d * (float)lo; float a1 = d * (float)hi; out[jj] = a0 + m; out[16 + jj] = a1 + m; }
    }
}

hipError_t launch_embed(const DevMatrix& w, const int32_t* ids, int n, float* h, int ldh, hipStream_t s)
{
    int64_t cnt = (int64_t)n * w.blocks;
    dim3 grid((unsigned)((cnt + 255) / 256)), block(256);
    switch (w.type) {
    case SHS_TYPE_Q4_0: hipLaunchKernelGGL(k_embed<SHS_TYPE_Q4_0>, grid, block, 0, s, w.qs, w.qh, w.d, w.m, w.blocks, ids, n, h, ldh); break;
    case SHS_TYPE_Q4_1: hipLaunchKernelGGL(k_embed<SHS_TYPE_Q4_1>, grid, block, 0, s, w.qs, w.qh, w.d, w.m, w.blocks, ids, n, h, ldh); break;
    case SHS_TYPE_Q5_0: hipLaunchKernelGGL(k_embed<SHS_TYPE_Q5_0>, grid, block, 0, s, w.qs, w.qh, w.d, w.m, w.blocks, ids, n, h, ldh); break;
    case SHS_TYPE_Q5_1: hipLaunchKernelGGL(k_embed<SHS_TYPE_Q5_1>, grid, block, 0, s, w.qs, w.qh, w.d, w.m, w.blocks, ids, n, h, ldh); break;
    case SHS_TYPE_Q8_0: hipLaunchKernelGGL(k_embed<SHS_TYPE_Q8_0>, grid, block, 0, s, w.qs, w.qh, w.d, w.m, w.blocks, ids, n, h, ldh); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------ RoPE + KV store

// Rope.Apply on adjacent pairs (Rope.cs:112-135) with host-computed cos/sin tables,
// ApplyPositionScale on queries (MinistralModel.cs:476-482), and StoreKeys/StoreValues
// (MinistralModel.cs:452-469). One wave per (token, head) of [q heads | k heads | v heads].
__global__ __launch_bounds__(64) void k_rope_store(float* __restrict__ qkv, int ld, int n_head, int n_kv, int hd,
                                                   const int32_t* __restrict__ pos, const float* __restrict__ ct,
                                                   const float* __restrict__ st, const float* __restrict__ qscale,
                                                   int half, float* __restrict__ kc, float* __restrict__ vc, int cap,
                                                   int slot0)
{
    const int t = blockIdx.x, hh = blockIdx.y, tid = threadIdx.x;
    const int p = pos[t];
    float* row = qkv + (int64_t)t * ld;
    if (hh < n_head + n_kv) {
        float* x = row + (int64_t)hh * hd;
        const float* c = ct + (int64_t)p * half;
        const float* s = st + (int64_t)p * half;
        for (int i = tid; i < half; i += 64) {
            float x0 = x[2 * i], x1 = x[2 * i + 1];
            float a = x0 * c[i], bb = x1 * s[i];
            float e = x0 * s[i], f = x1 * c[i];
            x[2 * i] = a - bb;
            x[2 * i + 1] = e + f;
        }
        if (hh < n_head) {
            const float qs = qscale[p];
            if (qs != 1.0f) {
                __syncthreads();
                for (int i = tid; i < hd; i += 64) x[i] = x[i] * qs;
            }
        } else {
            __syncthreads();
            const int kh = hh - n_head;
            float* dst = kc + ((int64_t)kh * cap + slot0 + t) * hd;
            for (int i = tid; i < hd; i += 64) dst[i] = x[i];
        }
    } else {
        const int kh = hh - n_head - n_kv;
        const float* x = row + (int64_t)(n_head + n_kv + kh) * hd;
        float* dst = vc + ((int64_t)kh * cap + slot0 + t) * hd;
        for (int i = tid; i < hd; i += 64) dst[i] = x[i];
    }
}

hipError_t launch_rope_store(float* qkv, int ldqkv, int T, int n_head, int n_kv, int hd, const int32_t* pos,
                             const float* ct, const float* st, const float* qscale, int half, float* kc, float* vc,
                             int cap, int slot0, hipStream_t s)
{
    hipLaunchKernelGGL(k_rope_store, dim3(T, n_head + 2 * n_kv), dim3(64), 0, s, qkv, ldqkv, n_head, n_kv, hd, pos, ct, st,
                       qscale, half, kc, vc, cap, slot0);
    return hipGetLastError();
}

// ------------------------------------------------------------------ attention

// e^x as a fixed sequence of IEEE single operations (Cody–Waite reduction with a
// 16-bit head of ln 2, the degree-7 Taylor polynomial of e^r in fused Horner form,
// exact scaling by 2^n), so that any implementation performing the same steps — the
// CPU restatement included — returns the same bits. ≤ 1 ulp against float64 exp.
// NaN returns x, x ≤ −104 returns 0 and x above ln(FLT_MAX) returns +inf; those cases
// are selected after the arithmetic rather than branched around, so a wave whose lanes
// disagree runs one straight sequence.
__device__ __forceinline__ float det_expf(float x)
{
    const float n = __builtin_rintf(x * 0x1.715476p+0f);
    float r = fmaf(-n, 0x1.62e400p-1f, x);
    r = fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0x1p-1f);
    p = fmaf(p, r, 0x1p+0f);
    p = fmaf(p, r, 0x1p+0f);
    // n is in [−150, 128] wherever the result is used; the clamp keeps the conversion
    // defined for the selected-away cases
    float y = ldexpf(p, (int)fminf(fmaxf(n, -256.0f), 256.0f));
    y = x > 0x1.62e42ep+6f ? INFINITY : y;
    y = x > -104.0f ? y : 0.0f;
    return x != x ? x : y;
}

// det_expf for x ≤ 0 that is not NaN (a softmax's s − max): the same operations, and the
// same result, without the tests only a NaN or a positive argument needs.
__device__ __forceinline__ float det_expf_nonpos(float x)
{
    const float n = __builtin_rintf(x * 0x1.715476p+0f);
    float r = fmaf(-n, 0x1.62e400p-1f, x);
    r = fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0x1p-1f);
    p = fmaf(p, r, 0x1p+0f);
    p = fmaf(p, r, 0x1p+0f);
    const float y = ldexpf(p, (int)fmaxf(n, -256.0f));
    return x > -104.0f ? y : 0.0f;
}

// Causal GQA attention in MinistralModel.AttendGroup's floating-point order
// (MinistralModel.cs:372-440, Kernels.cs:103-220), bit for bit:
//  * score = (Σ over 8 lanes of a 16-step FMA chain q[l+8m]·k[l+8m], summed pairwise)·scale
//    — Kernels.Dot4 with Vector<float>.Count = 8;
//  * softmax: max, e = exp(s − max), Σe over 8 strided lanes (pairwise) then the tail in
//    order, w = e / Σe; a row whose max is not finite becomes uniform (e = 1, Σe = n);
//  * ctx[d] = fma(v[p][d], w[p], ctx[d]) for p = 0, 1, 2, … — Kernels.AddScaled4.
// v_mfma_f32_32x32x2f32 computes fma(a1, b1, fma(a0, b0, c)) per element, so each
// instruction is two consecutive steps of those FMA chains for a 32×32 tile.
// Three kernels, each parallel over what its step allows:
//  1. scores: one block per (item, chunk of ≤ 4 key tiles, KV head), a wave per query head;
//     each 32×32 score tile goes to the scratch with its per-row max;
//  2. softmax: one block per (item, query head): Σe in order, then w = e / Σe over the scores;
//  3. values: one block per (item, 64-dimension half, KV head): the ordered FMA chain of w·v
//     over the keys.
// A score tile is stored in the MFMA's D layout with its rows permuted: lane j + 32h,
// register r holds query j and key 2r + h of the tile (the A operand's row i carries key
// kap(i) = 8(i/8) + 2(i%4) + (i%8)/4), so the value step feeds register c of both lane
// halves to the MFMA as the key pair (2c, 2c+1).
constexpr int ATT_HD = 128;

__device__ __forceinline__ int att_tiles(const AttnItem& it) { return (it.pos0 + it.q_count + 31) >> 5; }

// Key-major K tile, rows padded by 4 floats: the 16 lanes of one 16-byte read phase hold
// 16 different keys, whose rows start 4 banks apart.
constexpr int ATT_KROW = ATT_HD + 4;

__device__ __forceinline__ void attn_scores_work(const AttnChunk ch, int kvh, const float* __restrict__ q, int ldq,
                                                 const float* __restrict__ kc, int cap,
                                                 const AttnItem* __restrict__ items, int n_head, int n_kv, float scale,
                                                 float* __restrict__ scratch, float* __restrict__ pm,
                                                 float (*Ks)[32 * ATT_KROW])
{
    constexpr int KROW = ATT_KROW;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int j = lane & 31, h = lane >> 5;
    const AttnItem it = items[ch.item];
    const int group = n_head / n_kv;
    const bool active = wave < group;
    const int head = active ? kvh * group + wave : kvh * group;
    const float* kb = kc + ((int64_t)kvh * cap + it.key_start) * ATT_HD;
    const int n_keys = it.pos0 + it.q_count;
    const int64_t tile0 = it.s_off / 1024 + (int64_t)(kvh * 4 + wave) * att_tiles(it);
    const bool qvalid = active && j < it.q_count;
    const int nq = it.pos0 + j + 1;  // keys this query attends to

    // B operands: step s of chain l needs q[l + 16s + 8h]; qv[s] holds l = 0..7.
    float4 qv[8][2];
    {
        const float* qrow = q + (int64_t)(it.q_start + (qvalid ? j : 0)) * ldq + head * ATT_HD + 8 * h;
#pragma unroll
        for (int s = 0; s < 8; s++)
#pragma unroll
            for (int x = 0; x < 2; x++)
                qv[s][x] = qvalid ? *reinterpret_cast<const float4*>(qrow + 16 * s + 4 * x) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // A operands: row i of the A tile carries key kap(i), so D row i holds key kap(i).
    const int kap = 8 * (j >> 3) + 2 * (j & 3) + ((j >> 2) & 1);

    float4 kr[4];  // next K tile: thread tid holds key e >> 5, elements 4(e & 31) .. +3 for e = tid + 256i
    auto kload = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = tid + 256 * i;
            const int kidx = kt * 32 + (e >> 5);
            kr[i] = kidx < n_keys ? *reinterpret_cast<const float4*>(kb + (int64_t)kidx * ATT_HD + 4 * (e & 31))
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto kstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = tid + 256 * i;
            *reinterpret_cast<float4*>(&Ks[buf][(e >> 5) * KROW + 4 * (e & 31)]) = kr[i];
        }
    };
    // K tiles double-buffered, one barrier per tile: tile u + 1 is written into the other
    // buffer after tile u's MFMAs (its last readers, tile u − 1, finished before the previous
    // barrier), and its global load was issued a tile earlier.
    kload(ch.kt0);
    kstore(0);
    if (ch.nkt > 1) kload(ch.kt0 + 1);
    __syncthreads();
    for (int u = 0; u < ch.nkt; ++u) {
        const int kt = ch.kt0 + u;
        const float* krow = Ks[u & 1] + kap * KROW + 8 * h;
        v16f c[8];
        if (active) {
            // The 8 chains advance together: step s is 8 independent MFMAs.
#pragma unroll
            for (int l = 0; l < 8; l++)
#pragma unroll
                for (int r = 0; r < 16; r++) c[l][r] = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const float4 k0 = *reinterpret_cast<const float4*>(krow + 16 * s);
                const float4 k1 = *reinterpret_cast<const float4*>(krow + 16 * s + 4);
                c[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(k0.x, qv[s][0].x, c[0], 0, 0, 0);
                c[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(k0.y, qv[s][0].y, c[1], 0, 0, 0);
                c[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(k0.z, qv[s][0].z, c[2], 0, 0, 0);
                c[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(k0.w, qv[s][0].w, c[3], 0, 0, 0);
                c[4] = __builtin_amdgcn_mfma_f32_32x32x2f32(k1.x, qv[s][1].x, c[4], 0, 0, 0);
                c[5] = __builtin_amdgcn_mfma_f32_32x32x2f32(k1.y, qv[s][1].y, c[5], 0, 0, 0);
                c[6] = __builtin_amdgcn_mfma_f32_32x32x2f32(k1.z, qv[s][1].z, c[6], 0, 0, 0);
                c[7] = __builtin_amdgcn_mfma_f32_32x32x2f32(k1.w, qv[s][1].w, c[7], 0, 0, 0);
            }
        }
        if (u + 1 < ch.nkt) kstore((u + 1) & 1);
        if (u + 2 < ch.nkt) kload(kt + 2);
        if (active) {
            float sc[16];
            float mx = -INFINITY;
            bool nan = false;
            // A tile below every row's first masked key (pos0 + 1) needs no mask: rows past
            // q_count are never read back, whatever their maximum.
            const bool full = (kt + 1) * 32 <= it.pos0 + 1;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                // vsum8 of the chains, then the scale
                const float a = (c[0][r] + c[1][r]) + (c[2][r] + c[3][r]);
                const float b = (c[4][r] + c[5][r]) + (c[6][r] + c[7][r]);
                sc[r] = (a + b) * scale;
                const int key = kt * 32 + 2 * r + h;
                const bool valid = full || (qvalid && key < nq);  // selects, not branches
                mx = valid ? fmaxf(mx, sc[r]) : mx;
                nan = nan || (valid && sc[r] != sc[r]);
            }
            // tile layout [query j][residue t][k] for key t + 8k: register r holds key 2r + h,
            // so residue 2m + h is (sc[m], sc[m+4], sc[m+8], sc[m+12])
            float* out = scratch + (tile0 + kt) * 1024 + j * 32 + h * 4;
#pragma unroll
            for (int m = 0; m < 4; m++)
                *reinterpret_cast<float4*>(out + 8 * m) = make_float4(sc[m], sc[m + 4], sc[m + 8], sc[m + 12]);
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            nan = nan || __shfl_xor((int)nan, 32);
            if (h == 0) pm[(tile0 + kt) * 32 + j] = nan ? __builtin_nanf("") : mx;
        }
        __syncthreads();
    }
}

// w = e / Σe, correctly rounded, from rcp = RN(1/Σe): q = RN(e·rcp) is within one ulp of
// e/Σe, the residual e − q·Σe is exact in one FMA, and RN(q + residual·rcp) is then the
// correctly rounded quotient (Markstein's theorem) as long as nothing underflows. With
// 1 ≤ Σe ≤ 2^24 that holds for e ≥ 2^-100 and for e = 0; a lane holding any e in (0, 2^-100)
// divides outright.
template <int N>
__device__ __forceinline__ void softmax_divide(const float* e, float* w, float total, float rcp)
{
    bool tiny = false;
#pragma unroll
    for (int c = 0; c < N; c++) {
        tiny = tiny || (__float_as_uint(e[c]) - 1u) < 0x0D7FFFFFu;  // 0 < e < 2^-100
        const float q = e[c] * rcp;
        const float r = fmaf(-q, total, e[c]);
        w[c] = fmaf(r, rcp, q);
    }
    if (tiny) {
#pragma unroll
        for (int c = 0; c < N; c++) w[c] = e[c] / total;
    }
}

// One block per (item, query head); 8 lanes per query row, lane t owning residue t of the
// row's keys — exactly Kernels.Softmax's Vector<float> lane t, summed in key order.
__device__ __forceinline__ void attn_softmax_work(int idx, int head, const AttnItem* __restrict__ items, int n_head,
                                                  int n_kv, float* __restrict__ scratch, const float* __restrict__ pm)
{
    const int tid = threadIdx.x;
    const int j = tid >> 3, t = tid & 7;  // query row j of the item, residue t
    const AttnItem it = items[idx];
    const int group = n_head / n_kv;
    const int kvh = head / group, wave = head % group;  // the score kernel's (KV head, wave)
    const int n_kt = att_tiles(it);
    const int64_t tile0 = it.s_off / 1024 + (int64_t)(kvh * 4 + wave) * n_kt;
    const bool qvalid = j < it.q_count;
    const int nq = it.pos0 + j + 1;
    const int n8 = nq & ~7;

    float mx = -INFINITY;
    bool nan = false;
    for (int kt = t; kt < n_kt; kt += 8) {
        const float v = pm[(tile0 + kt) * 32 + j];
        mx = fmaxf(mx, v);
        nan = nan || v != v;
    }
    mx = fmaxf(mx, dpp_f<DPP_XOR1>(mx));
    mx = fmaxf(mx, dpp_f<DPP_XOR2>(mx));
    mx = fmaxf(mx, dpp_f<DPP_HALF_MIRROR>(mx));
    {
        int nn = nan ? 1 : 0;
        nn |= dpp_i<DPP_XOR1>(nn);
        nn |= dpp_i<DPP_XOR2>(nn);
        nn |= dpp_i<DPP_HALF_MIRROR>(nn);
        nan = nn != 0;
    }
    const bool uniform = nan || !(fabsf(mx) <= 3.402823466e38f);  // Kernels.Softmax: a non-finite max

    // Keys t + 8k (k = 0..3) of a tile are the float4 at [query j][residue t].
    const int64_t rec = (int64_t)j * 32 + t * 4;
    auto expo = [&](float sc, int key) {
        const float ex = uniform ? 1.0f : det_expf(sc - mx);
        return key < nq ? ex : 0.0f;
    };
    float lane_sum = 0.0f, tail_e = 0.0f;
    // Tiles are read in batches of 4 (16 values per lane), the next batch in flight.
    constexpr int NB = 4;
    float sv[NB * 4], nx[NB * 4];
    auto load = [&](int kt0, float* dst) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const float4 v = kt0 + b < n_kt ? *reinterpret_cast<const float4*>(scratch + (tile0 + kt0 + b) * 1024 + rec)
                                            : make_float4(0.f, 0.f, 0.f, 0.f);
            dst[4 * b] = v.x;
            dst[4 * b + 1] = v.y;
            dst[4 * b + 2] = v.z;
            dst[4 * b + 3] = v.w;
        }
    };
    // pass 1: Σe in Kernels.Softmax's order
    if (qvalid) load(0, nx);
    for (int kt0 = 0; qvalid && kt0 < n_kt; kt0 += NB) {
#pragma unroll
        for (int i = 0; i < NB * 4; i++) sv[i] = nx[i];
        if (kt0 + NB < n_kt) load(kt0 + NB, nx);
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int key = (kt0 + b) * 32 + t + 8 * k;
                const float e = expo(sv[4 * b + k], key);
                lane_sum = key < n8 ? lane_sum + e : lane_sum;
                tail_e = key >= n8 && key < nq ? e : tail_e;
            }
    }
    // vsum8: ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)); addition is commutative, so each lane
    // forms its pair with its xor partner.
    float total = vsum8_lanes(lane_sum);
    // the tail keys n8 .. nq−1 in order; lane k holds key n8 + k
#pragma unroll
    for (int k = 0; k < 7; k++) {
        const float e = __shfl(tail_e, k, 8);
        if (n8 + k < nq) total = total + e;
    }
    // pass 2: w = e / Σe over the scores (e recomputed: the exponential is deterministic),
    // written over them; keys outside the row get w = 0
    const float rcp = 1.0f / total;
    if (qvalid) load(0, nx);
    for (int kt0 = 0; qvalid && kt0 < n_kt; kt0 += NB) {
#pragma unroll
        for (int i = 0; i < NB * 4; i++) sv[i] = nx[i];
        if (kt0 + NB < n_kt) load(kt0 + NB, nx);
        float e[NB * 4], w[NB * 4];
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int k = 0; k < 4; k++) e[4 * b + k] = expo(sv[4 * b + k], (kt0 + b) * 32 + t + 8 * k);
        softmax_divide<NB * 4>(e, w, total, rcp);
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (kt0 + b >= n_kt) break;
            *reinterpret_cast<float4*>(scratch + (tile0 + kt0 + b) * 1024 + rec) =
                make_float4(w[4 * b], w[4 * b + 1], w[4 * b + 2], w[4 * b + 3]);
        }
    }
}

// ctx for NSL consecutive 32-dimension slices (starting at slice NSL·dt) of the 4 query
// heads of KV head kvh over item idx: one wave per head, the V slices staged in LDS per key
// tile and shared by the waves; each output is one ordered FMA chain over the keys
// (Kernels.AddScaled4: ctx = fma(v, w, ctx) in key order), two keys per MFMA step.
constexpr int ATT_PV_NSL = 2;
__device__ __forceinline__ void attn_pv_work(int idx, int dt, int kvh, const float* __restrict__ vc, int cap,
                                             const AttnItem* __restrict__ items, int n_head, int n_kv,
                                             const float* __restrict__ scratch, float* __restrict__ ctx, int ldc,
                                             const ActQ8& ao, float (*Vs)[32 * 32 * ATT_PV_NSL])
{
    constexpr int NSL = ATT_PV_NSL, DW = 32 * NSL;  // dimensions per work item
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int j = lane & 31, h = lane >> 5;
    const AttnItem it = items[idx];
    const int group = n_head / n_kv;
    const bool active = wave < group;
    const int head = active ? kvh * group + wave : kvh * group;
    const int n_keys = it.pos0 + it.q_count;
    const int n_kt = att_tiles(it);
    const int64_t tile0 = it.s_off / 1024 + (int64_t)(kvh * 4 + wave) * n_kt;
    const bool qvalid = active && j < it.q_count;
    const float* vb = vc + ((int64_t)kvh * cap + it.key_start) * ATT_HD + DW * dt;

    const int vkey = tid >> 3, vd = 4 * NSL * (tid & 7);  // thread tid stages key vkey, dimensions vd .. vd+4·NSL−1
    v16f o[NSL];
#pragma unroll
    for (int sl = 0; sl < NSL; sl++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[sl][r] = 0.0f;
    // Two tiles in flight: tile kt's weights and V slices load while tile kt − 2 is multiplied.
    struct Stage {
        float4 w[4];    // this lane's weights: float4 m holds keys 2m + h + 8k, k = 0..3
        float4 v[NSL];  // the V elements this thread stages
    };
    // weights of query j, key 2c + h: residue 2m + h (m = c & 3), k = c >> 2 of the tile's
    // [query][residue][k] layout — one float4 per m
    auto load = [&](int kt, Stage& st) {
        const int kidx = kt * 32 + vkey;
#pragma unroll
        for (int x = 0; x < NSL; x++)
            st.v[x] = kidx < n_keys ? *reinterpret_cast<const float4*>(vb + (int64_t)kidx * ATT_HD + vd + 4 * x)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
        const float* in = scratch + (tile0 + kt) * 1024 + j * 32 + h * 4;
#pragma unroll
        for (int m = 0; m < 4; m++)
            st.w[m] = active ? *reinterpret_cast<const float4*>(in + 8 * m) : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    auto step = [&](int kt, Stage& st) {
        const int buf = kt & 1;
#pragma unroll
        for (int x = 0; x < NSL; x++) *reinterpret_cast<float4*>(&Vs[buf][vkey * DW + vd + 4 * x]) = st.v[x];
        float w[16];
#pragma unroll
        for (int m = 0; m < 4; m++) {
            w[m] = st.w[m].x; w[m + 4] = st.w[m].y; w[m + 8] = st.w[m].z; w[m + 12] = st.w[m].w;
        }
        __syncthreads();
        if (kt + 2 < n_kt) load(kt + 2, st);
        if (active) {
#pragma unroll
            for (int c = 0; c < 16; c++)
#pragma unroll
                for (int sl = 0; sl < NSL; sl++)
                    o[sl] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[buf][(2 * c + h) * DW + 32 * sl + j], w[c], o[sl], 0,
                                                                 0, 0);
        }
    };
    Stage s0, s1;
    if (n_kt > 0) load(0, s0);
    if (n_kt > 1) load(1, s1);
    for (int kt = 0; kt < n_kt; kt += 2) {
        step(kt, s0);
        if (kt + 1 < n_kt) step(kt + 1, s1);
    }
    if (ao.q) {
        // The o projection's quantization of ctx, fused: each slice is one 32-dimension block
        // of query j, in the layout quant_block_pair takes. Rows past the item's queries are
        // not written (they belong to the next item, or are padding the GEMM never stores).
        if (!active) return;
        const bool valid = j < it.q_count;
#pragma unroll
        for (int sl = 0; sl < NSL; sl++) {
            float y[16];
#pragma unroll
            for (int r = 0; r < 16; r++) y[r] = o[sl][r];
            // both lanes of a pair share the query, so they agree on `valid`
            if (valid) quant_block_pair(y, h, ao, it.q_start + j, (head * ATT_HD + DW * dt + 32 * sl) / 32);
        }
        return;
    }
    if (!qvalid) return;
    float* outp = ctx + (int64_t)(it.q_start + j) * ldc + head * ATT_HD + DW * dt;
#pragma unroll
    for (int sl = 0; sl < NSL; sl++)
#pragma unroll
        for (int g = 0; g < 4; g++)
            *reinterpret_cast<float4*>(outp + 32 * sl + 8 * g + 4 * h) =
                make_float4(o[sl][4 * g], o[sl][4 * g + 1], o[sl][4 * g + 2], o[sl][4 * g + 3]);
}

// Scores, softmax and values of one (item, query head) in one block of eight waves, the
// item's scores kept in the LDS between the phases (MinistralModel.AttendGroup,
// MinistralModel.cs:372-440, in the floating-point order stated above):
//  * scores: the block's 32 query rows go to the LDS once, as the operands each chain step
//    reads; wave w computes whole 32×32 tiles w, w + 8, … — the eight Dot4 chains on
//    v_mfma_f32_32x32x2f32 as in attn_scores_work, its K operands loaded from global memory
//    three chain steps ahead into a register ring (a K row is read once per block, and the
//    phase has no barrier). vsum8, the scale and the row maxima (NaN-propagating, so a NaN
//    score reaches the softmax as a NaN maximum) follow in registers; the tile goes into
//    the LDS in the softmax layout;
//  * softmax: thread (p, j, t) owns residue t of query row j in half p of the tiles, as in
//    attn_softmax_work: both halves form e in place, half 0 runs the Σe chain in
//    Kernels.Softmax's order over its tiles as it goes and then over half 1's, and both
//    halves form w = e / Σe in place;
//  * values: wave w < 4 runs the ordered FMA chain of 32-dimension slice w over all keys,
//    its V elements loaded from global memory two tiles ahead (each load issued in the
//    shadow of the MFMA that last reads its register), its weights from the LDS one tile
//    ahead; no barrier either.
// LDS: kt_cap score tiles of 1024 floats, [query j][slot][k] with residue t in slot
// t ^ (j & 7) (conflict-free float4 writes, 2-way float4 reads), then the eight waves'
// 32 row maxima, the 32 row sums and the query operands. Blocks map to (KV-head group, head
// in group) so that the group's heads — which read the same K and V rows — share an XCD and
// start together: block b runs group 8·(b >> 5) + (b & 7) (groups longest first) and head
// (b >> 3) & 3 of it.
constexpr int ATT_THREADS = 512;  // eight waves: two per SIMD in the score and softmax phases
constexpr int ATT_RMAX = (ATT_THREADS / 64) * 32;  // floats of the row maxima after the score tiles
constexpr int ATT_QLDS = 32 * ATT_HD;              // floats of the query rows after the maxima and Σe

__device__ __forceinline__ int att_swz(int j, int t) { return j * 32 + ((t ^ (j & 7)) << 2); }

// The value phase: slice `wave` (32 dimensions) of head `head`, the weights read from the
// block's LDS score tiles S. Lane (j, h) feeds V[key 2c + h][32·wave + j] as the A operand
// and w[j][2c + h] as the B operand of step c of a tile, so each v_mfma_f32_32x32x2f32 is
// two consecutive keys of every chain ctx[j][d] = fma(v, w, ctx[j][d]).
template <bool SPILL>
__device__ __forceinline__ void attn_values_stream(const float* __restrict__ vc, int cap, const AttnItem& it, int kvh,
                                                   int head, int n_kt, int n_keys, const float* S,
                                                   const float* __restrict__ G, int kt_lds,
                                                   float* __restrict__ ctx, int ldc, const ActQ8& ao)
{
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int j = lane & 31, h = lane >> 5;
    const bool vwave = wave < ATT_HD / 32;  // waves 0..3 each run one 32-dimension slice
    const float* vbase = vc + ((int64_t)kvh * cap + it.key_start) * ATT_HD;
    const int voff = h * (ATT_HD * 4) + (32 * (wave & 3) + j) * 4;  // bytes
    struct VOps {
        float a[16];  // V of key 2c + h, dimension 32·wave + j
    };
    struct WOps {
        float w[16];  // weights of query j, key 2c + h
    };
    // One buffer resource per tile, whose range ends at the item's last key: rows past it
    // (and tiles past the last) read as 0 without touching memory. Their weights are 0 as
    // well, and fma(0, 0, ctx) is ctx (ctx starts at +0 and a sum that starts at +0 is never
    // −0), as for the in-range keys a query does not see.
    auto vload = [&](int kt, VOps& op) {
        const int rows = n_keys - kt * 32;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(vbase + (int64_t)kt * 32 * ATT_HD), 0, rows > 0 ? rows * (ATT_HD * 4) : 0, 0x00020000);
#pragma unroll
        for (int c = 0; c < 16; c++)
            op.a[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, voff + c * (2 * ATT_HD * 4), 0, 0));
    };
    auto wread = [&](int kt, WOps& op) {
        // residue 2m + h (m = c & 3), k = c >> 2 of the tile's rows; past the last tile the
        // last is read again, unused. Tiles from kt_lds on live in the block's spill region.
        const int k = min(kt, n_kt - 1);
        float4 v[4];
        if (!SPILL || k < kt_lds) {
#pragma unroll
            for (int m = 0; m < 4; m++) v[m] = *reinterpret_cast<const float4*>(S + k * 1024 + att_swz(j, 2 * m + h));
        } else {
#pragma unroll
            for (int m = 0; m < 4; m++)
                v[m] = *reinterpret_cast<const float4*>(G + (int64_t)k * 1024 + att_swz(j, 2 * m + h));
        }
#pragma unroll
        for (int m = 0; m < 4; m++) {
            op.w[m] = v[m].x;
            op.w[m + 4] = v[m].y;
            op.w[m + 8] = v[m].z;
            op.w[m + 12] = v[m].w;
        }
    };
    v16f o;
#pragma unroll
    for (int r = 0; r < 16; r++) o[r] = 0.0f;
    VOps va, vb;
    WOps wa, wb;
    if (vwave) {
        vload(0, va);
        vload(1, vb);
    }
    __syncthreads();  // every w is written
    if (!vwave) return;
    wread(0, wa);
    // iteration kt: `cur` holds V(kt) (V(kt + 1) in flight), `w` tile kt's weights; it reads
    // tile kt + 1's weights, then issues tile kt's 16 MFMAs, loading V(kt + 2) into `cur`
    auto step = [&](int kt, VOps& cur, WOps& w, WOps& wn) {
        wread(kt + 1, wn);
        const int rows = n_keys - (kt + 2) * 32;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(vbase + (int64_t)(kt + 2) * 32 * ATT_HD), 0, rows > 0 ? rows * (ATT_HD * 4) : 0,
            0x00020000);
        __builtin_amdgcn_sched_barrier(0);
        // V(kt + 2) into `cur`, each load issued in the shadow of the MFMA that last reads its
        // register (16 loads issued back to back would hold up the next tile's first MFMA)
#pragma unroll
        for (int c = 0; c < 16; c++) {
            o = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.a[c], w.w[c], o, 0, 0, 0);
            cur.a[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, voff + c * (2 * ATT_HD * 4), 0, 0));
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    int kt = 0;
    for (; kt + 1 < n_kt; kt += 2) {
        step(kt, va, wa, wb);
        step(kt + 1, vb, wb, wa);
    }
    if (kt < n_kt) step(kt, va, wa, wb);
    if (ao.q) {
        // The o projection's quantization of ctx, fused: the slice is one 32-dimension block
        // of query j, in the layout quant_block_pair takes. Rows past the item's queries are
        // not written (they belong to the next item, or are padding the GEMM never stores).
        if (j < it.q_count) {
            float y[16];
#pragma unroll
            for (int r = 0; r < 16; r++) y[r] = o[r];
            quant_block_pair(y, h, ao, it.q_start + j, (head * ATT_HD + 32 * wave) / 32);
        }
        return;
    }
    if (j >= it.q_count) return;
    float* outp = ctx + (int64_t)(it.q_start + j) * ldc + head * ATT_HD + 32 * wave;
#pragma unroll
    for (int gq = 0; gq < 4; gq++)
        *reinterpret_cast<float4*>(outp + 8 * gq + 4 * h) = make_float4(o[4 * gq], o[4 * gq + 1], o[4 * gq + 2], o[4 * gq + 3]);
}

// SPILL = false: every item fits the LDS tiles (kt_cap ≥ its key tiles), and the kernel has no
// spill path at all; SPILL = true: items past kt_cap keep their later tiles in `spill`.
template <bool SPILL>
__global__ __launch_bounds__(ATT_THREADS, 1) void k_attn_fused(const float* __restrict__ q, int ldq,
                                                              const float* __restrict__ kc,
                                                              const float* __restrict__ vc, int cap,
                                                              const AttnItem* __restrict__ items, int n_items,
                                                              int n_head, int n_kv, float scale,
                                                              float* __restrict__ ctx, int ldc, ActQ8 ao, int kt_cap,
                                                              float* __restrict__ spill)
{
    extern __shared__ float4 att_lds4[];
    float* S = reinterpret_cast<float*>(att_lds4);
    float* rmax = S + (int64_t)kt_cap * 1024;  // [wave][query row] maxima of the score phase
    float* tot = rmax + ATT_RMAX;               // [query row] Σe
    float* qlds = tot + 32;                     // [step][half][query][8] query operands
    const int tid = threadIdx.x;
    const int b = blockIdx.x;
    const int g = 8 * (b >> 5) + (b & 7), hg = (b >> 3) & 3;
    const int group = n_head / n_kv;
    if (g >= n_items * n_kv || hg >= group) return;  // the whole block leaves
    const int idx = n_items - 1 - g / n_kv, kvh = g % n_kv;
    const int head = kvh * group + hg;
    const AttnItem it = items[idx];
    const int n_kt = att_tiles(it);
    const int n_keys = it.pos0 + it.q_count;
    // Tiles 0 .. kt_cap − 1 live in the LDS; an item with more keeps tiles kt_cap .. n_kt − 1 in
    // its scratch region for this head (the region the three-kernel path uses), read back by
    // this block only, after the barriers that order its phases.
    float* G = SPILL ? spill + it.s_off + (int64_t)(kvh * 4 + hg) * n_kt * 1024 : nullptr;

    // ---- scores
    {
        const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int j = lane & 31, h = lane >> 5;
        const bool q_ok = j < it.q_count;
        const int nq = it.pos0 + j + 1;  // keys query j attends to
        const float* kb = kc + ((int64_t)kvh * cap + it.key_start) * ATT_HD + 8 * h;
        // A operands: row i of the A tile carries key kap(i), so D row i holds key kap(i),
        // and register r of lane half h holds key 2r + h
        const int kap = 8 * (j >> 3) + 2 * (j & 3) + ((j >> 2) & 1);
        // B operands: step s of chain l needs q[l + 16s + 8h], l = 0..7 — the block's 32
        // query rows go to the LDS once, as [s][h][query][l] (zeros past the item's queries)
        for (int f = tid; f < 32 * ATT_HD / 4; f += ATT_THREADS) {
            const int jq = f >> 5, d0 = (f & 31) * 4;
            v4f v = {0.f, 0.f, 0.f, 0.f};
            if (jq < it.q_count)
                v = *reinterpret_cast<const v4f*>(q + (int64_t)(it.q_start + jq) * ldq + head * ATT_HD + d0);
            *reinterpret_cast<v4f*>(qlds + (((d0 >> 4) * 2 + ((d0 >> 3) & 1)) * 32 + jq) * 8 + (d0 & 7)) = v;
        }
        const v4f* qop = reinterpret_cast<const v4f*>(qlds + (h * 32 + j) * 8);  // step s at qop[s * 128]
        // K operands of step s of tile kt: k[l + 16s + 8h] of key kap, l = 0..7; rows past
        // the item's last key read that key (their scores are masked)
        auto kload = [&](int kt, int s, v4f (&k)[2]) {
            const float* src = kb + (int64_t)min(kt * 32 + kap, n_keys - 1) * ATT_HD + 16 * s;
            k[0] = *reinterpret_cast<const v4f*>(src);
            k[1] = *reinterpret_cast<const v4f*>(src + 4);
        };
        constexpr int NW = ATT_THREADS / 64;
        const int n_mine = n_kt > wave ? (n_kt - wave + NW - 1) / NW : 0;  // tiles wave, wave + NW, ...
        const int last = wave + NW * (n_mine > 0 ? n_mine - 1 : 0);
        float mx = -INFINITY;
        v4f kr[4][2];  // ring: step g of the wave's step sequence in slot g & 3, loaded 3 steps ahead
        if (n_mine > 0) {
            kload(wave, 0, kr[0]);
            kload(wave, 1, kr[1]);
            kload(wave, 2, kr[2]);
        }
        __syncthreads();  // the query operands are in the LDS
        for (int u = 0; u < n_mine; u++) {
            const int kt = wave + NW * u;
            const int ktn = min(kt + NW, last);  // the wave's next tile; its last tile repeats
            v16f c[8];
#pragma unroll
            for (int s = 0; s < 8; s++) {
                if (s < 5) kload(kt, s + 3, kr[(s + 3) & 3]);
                else kload(ktn, s - 5, kr[(s + 3) & 3]);
                const v4f q0 = qop[s * 128], q1 = qop[s * 128 + 1];
                // the loads go out before this step's MFMAs
                __builtin_amdgcn_sched_barrier(0);
                const v4f k0 = kr[s & 3][0], k1 = kr[s & 3][1];
                const v16f z = {};
                // the 8 chains advance together: step s is 8 independent MFMAs
                c[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(k0.x, q0.x, s ? c[0] : z, 0, 0, 0);
                c[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(k0.y, q0.y, s ? c[1] : z, 0, 0, 0);
                c[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(k0.z, q0.z, s ? c[2] : z, 0, 0, 0);
                c[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(k0.w, q0.w, s ? c[3] : z, 0, 0, 0);
                c[4] = __builtin_amdgcn_mfma_f32_32x32x2f32(k1.x, q1.x, s ? c[4] : z, 0, 0, 0);
                c[5] = __builtin_amdgcn_mfma_f32_32x32x2f32(k1.y, q1.y, s ? c[5] : z, 0, 0, 0);
                c[6] = __builtin_amdgcn_mfma_f32_32x32x2f32(k1.z, q1.z, s ? c[6] : z, 0, 0, 0);
                c[7] = __builtin_amdgcn_mfma_f32_32x32x2f32(k1.w, q1.w, s ? c[7] : z, 0, 0, 0);
            }
            float sc[16];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                // vsum8 of the chains, then the scale
                const float a = (c[0][r] + c[1][r]) + (c[2][r] + c[3][r]);
                const float bsum = (c[4][r] + c[5][r]) + (c[6][r] + c[7][r]);
                sc[r] = (a + bsum) * scale;
            }
            // residue 2m + h of query j is (sc[m], sc[m+4], sc[m+8], sc[m+12])
            if (!SPILL || kt < kt_cap) {
                float* out = S + kt * 1024;
#pragma unroll
                for (int m = 0; m < 4; m++)
                    *reinterpret_cast<float4*>(out + att_swz(j, 2 * m + h)) =
                        make_float4(sc[m], sc[m + 4], sc[m + 8], sc[m + 12]);
            } else {
                float* out = G + (int64_t)kt * 1024;
#pragma unroll
                for (int m = 0; m < 4; m++)
                    *reinterpret_cast<float4*>(out + att_swz(j, 2 * m + h)) =
                        make_float4(sc[m], sc[m + 4], sc[m + 8], sc[m + 12]);
            }
            if ((kt + 1) * 32 <= it.pos0 + 1) {
                // below every row's first masked key; rows past q_count are never read back
#pragma unroll
                for (int r = 0; r < 16; r += 2)
                    mx = __builtin_elementwise_maximum(mx, __builtin_elementwise_maximum(sc[r], sc[r + 1]));
            } else {
#pragma unroll
                for (int r = 0; r < 16; r++)
                    mx = __builtin_elementwise_maximum(mx, q_ok && kt * 32 + 2 * r + h < nq ? sc[r] : -INFINITY);
            }
        }
        // the ring's loads past the wave's last tile are still in flight
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, 32));
        if (h == 0) rmax[wave * 32 + j] = mx;
        __syncthreads();  // every score and maximum is written
    }

    // ---- softmax: thread (p, j, t) owns residue t of query row j in half p of the tiles.
    // Both halves form e in place, half 0 running the Σe chain of Kernels.Softmax's order
    // over its own tiles as it goes; then half 0 continues the chain over half 1's tiles;
    // then both halves form w = e / Σe in place.
    {
        const int p = tid >> 8, r = tid & 255;
        const int j = r >> 3, t = r & 7;
        const bool qvalid = j < it.q_count;
        const int nq = it.pos0 + j + 1;
        const int n8 = nq & ~7;
        float mx = rmax[j];
#pragma unroll
        for (int w = 1; w < ATT_THREADS / 64; w++) mx = __builtin_elementwise_maximum(mx, rmax[w * 32 + j]);
        const bool nan = mx != mx;
        const bool uniform = nan || !(fabsf(mx) <= 3.402823466e38f);
        const int sw = att_swz(j, t);
        const int full_kt = ((it.pos0 + 1) & ~7) >> 5;
        const bool fast = !__any(qvalid && uniform);
        const int kh = n_kt >> 1;  // tiles [0, kh) in half 0, [kh, n_kt) in half 1
        const int k0 = p ? kh : 0, k1 = p ? n_kt : kh;
        constexpr int NB = 4;
        // Σe: lane t sums its residue's keys below n8 in key order, the 8 lanes pairwise,
        // then the keys n8 .. nq − 1 in order. Below full_kt every key is below n8.
        float lane_sum = 0.0f, tail_e = 0.0f;
        auto chain = [&](int kt, const float (&e)[4]) {
            if (kt < full_kt) {
#pragma unroll
                for (int k = 0; k < 4; k++) lane_sum = lane_sum + e[k];
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int key = kt * 32 + t + 8 * k;
                    lane_sum = key < n8 ? lane_sum + e[k] : lane_sum;
                    tail_e = key >= n8 && key < nq ? e[k] : tail_e;
                }
            }
        };
        // this thread's float4 of tile kt: in the LDS below kt_cap, else in the spill region.
        // A batch of NB tiles all in the LDS takes the LDS-only form of each loop below.
        auto ldt = [&](int kt) -> float4 {
            if (kt < kt_cap) return *reinterpret_cast<const float4*>(S + kt * 1024 + sw);
            return *reinterpret_cast<const float4*>(G + (int64_t)kt * 1024 + sw);
        };
        auto stt = [&](int kt, float4 v) {
            if (kt < kt_cap) *reinterpret_cast<float4*>(S + kt * 1024 + sw) = v;
            else *reinterpret_cast<float4*>(G + (int64_t)kt * 1024 + sw) = v;
        };
        auto e_batch = [&](int kt0, auto lds_only) {
            float4 sv[NB];
#pragma unroll
            for (int qq = 0; qq < NB; qq++) {
                const int kt = kt0 + qq < k1 ? kt0 + qq : kt0;
                if constexpr (decltype(lds_only)::value) sv[qq] = *reinterpret_cast<const float4*>(S + kt * 1024 + sw);
                else sv[qq] = ldt(kt);
            }
#pragma unroll
            for (int qq = 0; qq < NB; qq++) {
                if (kt0 + qq >= k1) break;
                const float sc[4] = {sv[qq].x, sv[qq].y, sv[qq].z, sv[qq].w};
                float e[4];
                if (fast && kt0 + qq < full_kt) {
#pragma unroll
                    for (int k = 0; k < 4; k++) e[k] = det_expf_nonpos(sc[k] - mx);
                } else {
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const int key = (kt0 + qq) * 32 + t + 8 * k;
                        const float ex = uniform ? 1.0f : det_expf(sc[k] - mx);
                        e[k] = qvalid && key < nq ? ex : 0.0f;
                    }
                }
                const float4 ev = make_float4(e[0], e[1], e[2], e[3]);
                if constexpr (decltype(lds_only)::value) *reinterpret_cast<float4*>(S + (kt0 + qq) * 1024 + sw) = ev;
                else stt(kt0 + qq, ev);
                if (p == 0) chain(kt0 + qq, e);
            }
        };
        for (int kt0 = k0; kt0 < k1; kt0 += NB) {
            if constexpr (!SPILL) e_batch(kt0, std::true_type());
            else if (kt0 + NB <= kt_cap) e_batch(kt0, std::true_type());
            else e_batch(kt0, std::false_type());
        }
        __syncthreads();  // every e is written
        if (p == 0) {
            auto sum_batch = [&](int kt0, auto lds_only) {
                float4 ev[NB];
#pragma unroll
                for (int qq = 0; qq < NB; qq++) {
                    const int kt = kt0 + qq < n_kt ? kt0 + qq : kt0;
                    if constexpr (decltype(lds_only)::value) ev[qq] = *reinterpret_cast<const float4*>(S + kt * 1024 + sw);
                    else ev[qq] = ldt(kt);
                }
#pragma unroll
                for (int qq = 0; qq < NB; qq++) {
                    if (kt0 + qq >= n_kt) break;
                    const float e[4] = {ev[qq].x, ev[qq].y, ev[qq].z, ev[qq].w};
                    chain(kt0 + qq, e);
                }
            };
            for (int kt0 = kh; kt0 < n_kt; kt0 += NB) {
                if constexpr (!SPILL) sum_batch(kt0, std::true_type());
                else if (kt0 + NB <= kt_cap) sum_batch(kt0, std::true_type());
                else sum_batch(kt0, std::false_type());
            }
            float total = vsum8_lanes(lane_sum);
#pragma unroll
            for (int k = 0; k < 7; k++) {
                const float e = __shfl(tail_e, k, 8);
                if (n8 + k < nq) total = total + e;
            }
            if (t == 0) tot[j] = total;
        }
        __syncthreads();  // every Σe is written
        if (qvalid) {
            const float total = tot[j];
            const float rcp = 1.0f / total;
            auto div_batch = [&](int kt0, auto lds_only) {
                float e[16], w[16];
#pragma unroll
                for (int qq = 0; qq < 4; qq++) {
                    const int kt = kt0 + qq < k1 ? kt0 + qq : kt0;  // past the end: reread, not written
                    float4 v;
                    if constexpr (decltype(lds_only)::value) v = *reinterpret_cast<const float4*>(S + kt * 1024 + sw);
                    else v = ldt(kt);
                    e[4 * qq] = v.x;
                    e[4 * qq + 1] = v.y;
                    e[4 * qq + 2] = v.z;
                    e[4 * qq + 3] = v.w;
                }
                softmax_divide<16>(e, w, total, rcp);
#pragma unroll
                for (int qq = 0; qq < 4; qq++) {
                    if (kt0 + qq >= k1) continue;
                    const float4 wv = make_float4(w[4 * qq], w[4 * qq + 1], w[4 * qq + 2], w[4 * qq + 3]);
                    if constexpr (decltype(lds_only)::value) *reinterpret_cast<float4*>(S + (kt0 + qq) * 1024 + sw) = wv;
                    else stt(kt0 + qq, wv);
                }
            };
            for (int kt0 = k0; kt0 < k1; kt0 += 4) {
                if constexpr (!SPILL) div_batch(kt0, std::true_type());
                else if (kt0 + 4 <= kt_cap) div_batch(kt0, std::true_type());
                else div_batch(kt0, std::false_type());
            }
        }
    }
    attn_values_stream<SPILL>(vc, cap, it, kvh, head, n_kt, n_keys, S, G, kt_cap, ctx, ldc, ao);
}

// The softmax and value kernels of the three-kernel path take their work longest first
// from a counter, one item per block at a time (greedy longest-processing-time order), so
// that the causal triangle's long rows spread over all CUs whatever the hardware's block
// placement. Every block leaves its loop once the counter passes the work count.
__device__ __forceinline__ int next_work(int* counter, int* slot)
{
    __syncthreads();  // the block is done with the previous item (and its LDS)
    if (threadIdx.x == 0) *slot = atomicAdd(counter, 1);
    __syncthreads();
    return *slot;
}

__global__ __launch_bounds__(256, 2) void k_attn_scores(const float* __restrict__ q, int ldq, const float* __restrict__ kc,
                                                        int cap, const AttnItem* __restrict__ items,
                                                        const AttnChunk* __restrict__ chunks, int n_chunks, int n_head,
                                                        int n_kv, float scale, float* __restrict__ scratch,
                                                        float* __restrict__ pm)
{
    // one block per (chunk, KV head); the chunks come longest first, and the hardware hands
    // out blocks in order, so the causal triangle's long rows start first
    __shared__ float Ks[2][32 * ATT_KROW];
    const int w = blockIdx.x;
    attn_scores_work(chunks[w / n_kv], w % n_kv, q, ldq, kc, cap, items, n_head, n_kv, scale, scratch, pm, Ks);
}

__global__ __launch_bounds__(256) void k_attn_softmax(const AttnItem* __restrict__ items, int n_items, int n_head,
                                                      int n_kv, float* __restrict__ scratch, const float* __restrict__ pm,
                                                      int* __restrict__ counter)
{
    __shared__ int slot;
    for (;;) {
        const int w = next_work(counter, &slot);
        if (w >= n_items * n_head) break;
        attn_softmax_work(n_items - 1 - w / n_head, w % n_head, items, n_head, n_kv, scratch, pm);
    }
}

__global__ __launch_bounds__(256) void k_attn_pv(const float* __restrict__ vc, int cap, const AttnItem* __restrict__ items,
                                                 int n_items, int n_head, int n_kv, const float* __restrict__ scratch,
                                                 float* __restrict__ ctx, int ldc, ActQ8 ao, int* __restrict__ counter)
{
    __shared__ float Vs[2][32 * 32 * ATT_PV_NSL];  // [key][dimension within the slices]
    __shared__ int slot;
    constexpr int NDT = 4 / ATT_PV_NSL;  // work items per (item, KV head)
    for (;;) {
        const int w = next_work(counter, &slot);
        if (w >= n_items * NDT * n_kv) break;
        const int per = NDT * n_kv;
        attn_pv_work(n_items - 1 - w / per, (w % per) / n_kv, (w % per) % n_kv, vc, cap, items, n_head, n_kv, scratch,
                     ctx, ldc, ao, Vs);
    }
}

static dim3 attn_blocks(int n_work, int per_cu, int n_cu)
{
    return dim3((unsigned)(n_work < per_cu * n_cu ? n_work : per_cu * n_cu));
}

int attn_score_slots(int n_cu)
{
    static std::atomic<int> cached{0};  // the same on every gfx950 device; racing threads store the same value
    int per_cu = cached.load(std::memory_order_relaxed);
    if (per_cu == 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_attn_scores, 256, 0) != hipSuccess || per_cu <= 0)
            per_cu = 2;
        cached.store(per_cu, std::memory_order_relaxed);
    }
    return per_cu * n_cu;
}

hipError_t launch_attn_scores(const float* q, int ldq, const float* kc, int cap, const AttnItem* items,
                              const AttnChunk* chunks, int n_chunks, int n_head, int n_kv, int head_dim, float scale,
                              float* scratch, float* pm, hipStream_t s)
{
    if (head_dim != ATT_HD || n_head % n_kv != 0 || n_head / n_kv > 4) return hipErrorInvalidValue;
    if (n_chunks <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_attn_scores, dim3((unsigned)(n_chunks * n_kv)), dim3(256), 0, s, q, ldq, kc, cap, items,
                       chunks, n_chunks, n_head, n_kv, scale, scratch, pm);
    return hipGetLastError();
}

hipError_t launch_attn_softmax(const AttnItem* items, int n_items, int n_head, int n_kv, float* scratch, const float* pm,
                               int* counters, int n_cu, hipStream_t s)
{
    if (n_items <= 0) return hipSuccess;
    hipError_t e = launch_fill_zero(reinterpret_cast<float*>(counters), 2, s);  // its and launch_attn_pv's counter
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_softmax, attn_blocks(n_items * n_head, 8, n_cu), dim3(256), 0, s, items, n_items, n_head,
                       n_kv, scratch, pm, counters);
    return hipGetLastError();
}

hipError_t launch_attn_pv(const float* vc, int cap, const AttnItem* items, int n_items, int n_head, int n_kv,
                          const float* scratch, float* ctx, int ldc, const ActQ8* codes, int* counters, int n_cu,
                          hipStream_t s)
{
    if (n_items <= 0) return hipSuccess;
    if (codes && (codes->B != n_head * ATT_HD / 32 || !codes->q)) return hipErrorInvalidValue;
    const ActQ8 ao = codes ? *codes : ActQ8();
    hipLaunchKernelGGL(k_attn_pv, attn_blocks(n_items * (4 / ATT_PV_NSL) * n_kv, 5, n_cu), dim3(256), 0, s, vc, cap,
                       items, n_items, n_head, n_kv, scratch, ctx, ldc, ao, counters + 1);
    return hipGetLastError();
}

int attn_fused_kt_limit(int max_lds_bytes)
{
    const int kt = (max_lds_bytes - (ATT_RMAX + 32 + ATT_QLDS) * (int)sizeof(float)) / (1024 * (int)sizeof(float));
    return kt > 0 ? kt : 0;
}

hipError_t launch_attn_fused(const float* q, int ldq, const float* kc, const float* vc, int cap, const AttnItem* items,
                             int n_items, int n_head, int n_kv, int head_dim, float scale, float* ctx, int ldc,
                             const ActQ8* codes, int kt_cap, float* spill, hipStream_t s)
{
    if (n_items <= 0) return hipSuccess;
    if (head_dim != ATT_HD || n_head % n_kv != 0 || n_head / n_kv > 4 || kt_cap <= 0) return hipErrorInvalidValue;
    if (codes && (codes->B != n_head * ATT_HD / 32 || !codes->q)) return hipErrorInvalidValue;
    const ActQ8 ao = codes ? *codes : ActQ8();
    const size_t lds = ((size_t)kt_cap * 1024 + ATT_RMAX + 32 + ATT_QLDS) * sizeof(float);
    static LdsLimit limit_lds, limit_spill;
    const int n_groups = n_items * n_kv;
    const unsigned grid = (unsigned)(((n_groups + 7) / 8) * 32);
    hipError_t e;
    if (spill) {
        if ((e = limit_spill.raise(reinterpret_cast<const void*>(k_attn_fused<true>), lds)) != hipSuccess) return e;
        hipLaunchKernelGGL(k_attn_fused<true>, dim3(grid), dim3(ATT_THREADS), lds, s, q, ldq, kc, vc, cap, items, n_items,
                           n_head, n_kv, scale, ctx, ldc, ao, kt_cap, spill);
    } else {
        if ((e = limit_lds.raise(reinterpret_cast<const void*>(k_attn_fused<false>), lds)) != hipSuccess) return e;
        hipLaunchKernelGGL(k_attn_fused<false>, dim3(grid), dim3(ATT_THREADS), lds, s, q, ldq, kc, vc, cap, items, n_items,
                           n_head, n_kv, scale, ctx, ldc, ao, kt_cap, nullptr);
    }
    return hipGetLastError();
}

// ------------------------------------------------------ attention at decode width

// Items of at most ATT_DEC_MAX_Q queries (single-token decode, a few tokens per sequence)
// skip the 32-query tiles above, which would be almost all padding. At this width the cost
// is memory latency, so the work is spread over many blocks with all their loads issued up
// front, in two kernels:
//  1. k_attn_dec_scores, one block per (item, KV head, 64-key chunk): the chunk's K rows
//     (coalesced) and the group's q rows go to the LDS; lane i of a key's 4 lanes runs Dot4's
//     chains 2i and 2i+1, c_l = fma(k[l+8m], q[l+8m], c_l) for m = 0..15, the 4 lanes add
//     pairwise in vsum8's order and the scale follows (MinistralModel.cs:392-405,
//     Kernels.cs:103-122); every query head of the group and every query of the item;
//  2. k_attn_dec_pv, one block per (item, query head, 32-dimension slice): the slice of V is
//     loaded while the block forms the softmax of the head's scores — max; e = exp(s − max)
//     (1 when the max is not finite); Σe over 8 lanes of residues in key order, pairwise,
//     then the tail in order; w = e / Σe correctly rounded (Kernels.cs:157-200) — then lane
//     (query, dimension) runs ctx = fma(v, w, ctx) over the keys in order (Kernels.AddScaled4).
//     A slice is one 32-dimension block of the o projection's input, quantized in place when
//     codes are given.
// Scores go to the item's scratch region as [head][query][ld_k], ld_k = keys rounded up to 4.
constexpr int DEC_KT = 64;             // keys per score block
constexpr int DEC_KROW = ATT_HD + 8;   // padded K row: 8 consecutive keys start 8 banks apart
constexpr int DEC_VCH = 256;           // keys per staged V chunk

__device__ __forceinline__ int dec_ld_k(const AttnItem& it) { return (it.pos0 + it.q_count + 3) & ~3; }

__global__ __launch_bounds__(256) void k_attn_dec_scores(const float* __restrict__ q, int ldq,
                                                         const float* __restrict__ kc, int cap,
                                                         const AttnItem* __restrict__ items, int n_head, int n_kv,
                                                         int n_chunks, float scale, float* __restrict__ scratch)
{
    const int G = n_head / n_kv;
    const int b = blockIdx.x;
    const int idx = b / (n_kv * n_chunks), r = b % (n_kv * n_chunks);
    const int kvh = r / n_chunks, ch = r % n_chunks;
    const AttnItem it = items[idx];
    const int qc = it.q_count, nk = it.pos0 + qc;
    if (ch * DEC_KT >= nk) return;
    extern __shared__ float dsk[];
    float* sK = dsk;                      // [DEC_KT][DEC_KROW]
    float* sQ = dsk + DEC_KT * DEC_KROW;  // [G·qc][128]
    const int tid = threadIdx.x;
    const float* kb = kc + ((int64_t)kvh * cap + it.key_start) * ATT_HD;
    // K rows ch·64 .. +63: float4 e = tid + 256j is key e / 32, columns 4(e % 32) .. +3
    v4f kr[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int e = tid + 256 * j;
        const int key = min(ch * DEC_KT + (e >> 5), nk - 1);
        kr[j] = *reinterpret_cast<const v4f*>(kb + (int64_t)key * ATT_HD + 4 * (e & 31));
    }
    for (int i = tid; i < G * qc * (ATT_HD / 4); i += 256) {
        const int hq = i / (ATT_HD / 4), u = i % (ATT_HD / 4);
        const int hg = hq / qc, qi = hq % qc;
        reinterpret_cast<v4f*>(sQ)[i] = *reinterpret_cast<const v4f*>(
            q + (int64_t)(it.q_start + qi) * ldq + (kvh * G + hg) * ATT_HD + 4 * u);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int e = tid + 256 * j;
        *reinterpret_cast<v4f*>(sK + (e >> 5) * DEC_KROW + 4 * (e & 31)) = kr[j];
    }
    __syncthreads();
    const int kk = tid >> 2, ci = tid & 3;
    const int key = ch * DEC_KT + kk;
    const int ld_k = dec_ld_k(it);
    const float2* krow = reinterpret_cast<const float2*>(sK + kk * DEC_KROW + 2 * ci);
    for (int hq = 0; hq < G * qc; hq++) {
        const int hg = hq / qc, qi = hq % qc;
        const float2* qrow = reinterpret_cast<const float2*>(sQ + hq * ATT_HD + 2 * ci);
        float c0 = 0.0f, c1 = 0.0f;
#pragma unroll
        for (int m = 0; m < 16; m++) {
            const float2 kv = krow[4 * m], qv = qrow[4 * m];
            c0 = fmaf(kv.x, qv.x, c0);
            c1 = fmaf(kv.y, qv.y, c1);
        }
        // vsum8: ((c0+c1)+(c2+c3))+((c4+c5)+(c6+c7)); lane i holds c_2i + c_2i+1
        float p = c0 + c1;
        p = p + dpp_f<DPP_XOR1>(p);
        p = p + dpp_f<DPP_XOR2>(p);
        if (ci == 0 && key <= it.pos0 + qi)
            scratch[it.s_off + ((int64_t)(kvh * G + hg) * qc + qi) * ld_k + key] = p * scale;
    }
}

__global__ __launch_bounds__(256) void k_attn_dec_pv(const float* __restrict__ vc, int cap,
                                                     const AttnItem* __restrict__ items, int n_head, int n_kv,
                                                     int ld_s, int max_qc, const float* __restrict__ scratch,
                                                     float* __restrict__ ctx, int ldc, ActQ8 ao)
{
    constexpr int NSL = ATT_HD / 32;
    const int G = n_head / n_kv;
    const int b = blockIdx.x;
    const int idx = b / (n_head * NSL), r = b % (n_head * NSL);
    const int head = r / NSL, sl = r % NSL;
    const int kvh = head / G;
    const AttnItem it = items[idx];
    const int qc = it.q_count, nk = it.pos0 + qc;
    const int ld_k = dec_ld_k(it);
    extern __shared__ float dpv[];
    float* sW = dpv;                          // [qc][ld_s] scores → e → w
    float* sV = dpv + max_qc * ld_s;          // [DEC_VCH][32]
    float* sR = sV + DEC_VCH * 32;            // per query: max, uniform flag, Σe, pad
    float* sC = sR + 4 * ATT_DEC_MAX_Q;       // [qc][32]
    __shared__ float wred[4][ATT_DEC_MAX_Q];
    __shared__ int wnan[4][ATT_DEC_MAX_Q];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* vb = vc + ((int64_t)kvh * cap + it.key_start) * ATT_HD + 32 * sl;

    // V chunk c: float4 e = tid + 256j is key e / 8, dimensions 4(e % 8) .. +3 of the slice
    v4f vr[8];
    auto vload = [&](int c) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int e = tid + 256 * j;
            const int key = min(c * DEC_VCH + (e >> 3), nk - 1);
            vr[j] = *reinterpret_cast<const v4f*>(vb + (int64_t)key * ATT_HD + 4 * (e & 7));
        }
    };
    vload(0);

    const float* sc = scratch + it.s_off + (int64_t)head * qc * ld_k;
    for (int qi = 0; qi < qc; qi++)
        for (int key = tid; key < ld_s; key += 256)
            sW[qi * ld_s + key] = key <= it.pos0 + qi ? sc[(int64_t)qi * ld_k + key] : 0.0f;
    __syncthreads();

    // row maxima (NaN noted: Kernels.Softmax then weighs every key equally)
    for (int qi = 0; qi < qc; qi++) {
        const int nq = it.pos0 + qi + 1;
        float mx = -INFINITY;
        int nan = 0;
        for (int key = tid; key < nq; key += 256) {
            const float v = sW[qi * ld_s + key];
            mx = fmaxf(mx, v);
            nan |= v != v;
        }
        mx = wave_max(mx);
        nan = wave_or(nan);
        if (lane == 0) {
            wred[wave][qi] = mx;
            wnan[wave][qi] = nan;
        }
    }
    __syncthreads();
    if (tid < qc) {
        const float mx = fmaxf(fmaxf(wred[0][tid], wred[1][tid]), fmaxf(wred[2][tid], wred[3][tid]));
        const int nan = wnan[0][tid] | wnan[1][tid] | wnan[2][tid] | wnan[3][tid];
        sR[4 * tid] = mx;
        sR[4 * tid + 1] = (nan || !(fabsf(mx) <= 3.402823466e38f)) ? 1.0f : 0.0f;
    }
    __syncthreads();

    // e in place (keys of the row only; the rest stay 0)
    for (int qi = 0; qi < qc; qi++) {
        const float mx = sR[4 * qi];
        const bool uniform = sR[4 * qi + 1] != 0.0f;
        for (int key = tid; key <= it.pos0 + qi; key += 256)
            sW[qi * ld_s + key] = uniform ? 1.0f : det_expf(sW[qi * ld_s + key] - mx);
    }
    __syncthreads();

    // Σe: lane t of the 8-lane group of query qi sums residue t up to n8 in key order
    if (tid < 8 * qc) {
        const int qi = tid >> 3, t = tid & 7;
        const int nq = it.pos0 + qi + 1, n8 = nq & ~7;
        const float* e = sW + qi * ld_s;
        float part = 0.0f;
        int key = t;
        for (; key + 56 < n8; key += 64) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = e[key + 8 * k];
#pragma unroll
            for (int k = 0; k < 8; k++) part = part + v[k];
        }
        for (; key < n8; key += 8) part = part + e[key];
        float total = vsum8_lanes(part);
        // the tail keys n8 .. nq − 1 in order (at most 7; read together, slots past nq are 0)
        float tl[7];
#pragma unroll
        for (int k = 0; k < 7; k++) tl[k] = e[n8 + k];
#pragma unroll
        for (int k = 0; k < 7; k++) total = n8 + k < nq ? total + tl[k] : total;
        if (t == 0) sR[4 * qi + 2] = total;
    }
    __syncthreads();

    // w = e / Σe over the row's keys (the zeros past it stay), and the first V chunk into the LDS
    for (int qi = 0; qi < qc; qi++) {
        const float total = sR[4 * qi + 2];
        for (int key = tid; key <= it.pos0 + qi; key += 256) sW[qi * ld_s + key] = sW[qi * ld_s + key] / total;
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int e = tid + 256 * j;
        *reinterpret_cast<v4f*>(sV + (e >> 3) * 32 + 4 * (e & 7)) = vr[j];
    }

    // values: lane (qi, d) runs the ordered chain over the keys; V staged per 256-key chunk.
    // Steps past a query's last key have v = 0 and w = 0, so fma leaves ctx unchanged (ctx
    // is never −0: it starts at +0 and a sum that cancels rounds to +0).
    const int n_ch = (nk + DEC_VCH - 1) / DEC_VCH;
    const int qi = tid >> 5, d = tid & 31;
    const bool chain = tid < 32 * qc;
    const int nq = it.pos0 + (chain ? qi : 0) + 1;
    const float* w = sW + (chain ? qi : 0) * ld_s;
    float acc = 0.0f;
    for (int c = 0; c < n_ch; c++) {
        if (c > 0) {
            __syncthreads();  // the previous chunk's readers are done
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int e = tid + 256 * j;
                *reinterpret_cast<v4f*>(sV + (e >> 3) * 32 + 4 * (e & 7)) = vr[j];
            }
        }
        __syncthreads();
        if (c + 1 < n_ch) vload(c + 1);
        if (chain) {
            const int k0 = c * DEC_VCH, k1 = min(k0 + DEC_VCH, nq);
            // 16 steps at a time: weights as four float4 reads, then the chain; the chunk's rows
            // are all staged (clamped past the last key), and only the last group masks its
            // steps past k1
            auto group = [&](int key, bool masked) {
                float v[16];
                float4 w4[4];
#pragma unroll
                for (int g = 0; g < 4; g++) w4[g] = *reinterpret_cast<const float4*>(w + key + 4 * g);
#pragma unroll
                for (int k = 0; k < 16; k++) v[k] = sV[(key - k0 + k) * 32 + d];
                if (masked) {
#pragma unroll
                    for (int k = 0; k < 16; k++) v[k] = key + k < k1 ? v[k] : 0.0f;
                }
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    acc = fmaf(v[4 * g], w4[g].x, acc);
                    acc = fmaf(v[4 * g + 1], w4[g].y, acc);
                    acc = fmaf(v[4 * g + 2], w4[g].z, acc);
                    acc = fmaf(v[4 * g + 3], w4[g].w, acc);
                }
            };
            // Full groups alternate between two register sets: the next group's reads are
            // issued (kept ahead by an empty asm that takes acc) before the current group's
            // FMAs, so the LDS latency is paid about once per chunk.
            const int kfull = k0 + ((k1 - k0) & ~15);
            int key = k0;
            float va[16], vb[16];
            float4 wa[4], wb[4];
#define SHS_DEC_LOAD(V, W, KEY)                                                        \
    {                                                                                  \
        _Pragma("unroll") for (int g = 0; g < 4; g++) W[g] =                           \
            *reinterpret_cast<const float4*>(w + (KEY) + 4 * g);                      \
        _Pragma("unroll") for (int k = 0; k < 16; k++) V[k] = sV[((KEY) - k0 + k) * 32 + d]; \
        asm volatile("" : "+v"(acc)::"memory");                                        \
    }
#define SHS_DEC_RUN(V, W)                                                              \
    _Pragma("unroll") for (int g = 0; g < 4; g++)                                      \
    {                                                                                  \
        acc = fmaf(V[4 * g], W[g].x, acc);                                             \
        acc = fmaf(V[4 * g + 1], W[g].y, acc);                                         \
        acc = fmaf(V[4 * g + 2], W[g].z, acc);                                         \
        acc = fmaf(V[4 * g + 3], W[g].w, acc);                                         \
    }
            if (key < kfull) SHS_DEC_LOAD(va, wa, key);
            for (; key + 32 <= kfull; key += 32) {
                SHS_DEC_LOAD(vb, wb, key + 16);
                SHS_DEC_RUN(va, wa);
                // (no group after the next: the current one again, unused)
                SHS_DEC_LOAD(va, wa, key + 48 <= kfull ? key + 32 : key);
                SHS_DEC_RUN(vb, wb);
            }
            if (key < kfull) {
                SHS_DEC_RUN(va, wa);
                key += 16;
            }
#undef SHS_DEC_LOAD
#undef SHS_DEC_RUN
            if (key < k1) group(key, true);
        }
    }
    if (!ao.q) {
        if (chain) ctx[(int64_t)(it.q_start + qi) * ldc + head * ATT_HD + 32 * sl + d] = acc;
        return;
    }
    if (chain) sC[tid] = acc;
    __syncthreads();
    // the o projection's codes: 8 lanes per query, 4 dimensions each
    if (tid < 8 * qc) {
        const int q8 = tid >> 3, l8 = tid & 7;
        const float4 v = *reinterpret_cast<const float4*>(sC + q8 * 32 + 4 * l8);
        quant_block8(v, l8, ao, it.q_start + q8, (head * ATT_HD + 32 * sl) / 32, 0);
    }
}

static size_t dec_scores_lds(int G, int max_qc)
{
    return sizeof(float) * ((size_t)DEC_KT * DEC_KROW + (size_t)G * max_qc * ATT_HD);
}

static size_t dec_pv_lds(int max_qc, int ld_s)
{
    return sizeof(float) * ((size_t)max_qc * ld_s + (size_t)DEC_VCH * 32 + 4 * ATT_DEC_MAX_Q + (size_t)max_qc * 32);
}

int attn_decode_max_keys(int max_qc, int max_lds_bytes)
{
    if (max_qc < 1 || max_qc > ATT_DEC_MAX_Q) return 0;
    const int64_t room = (int64_t)max_lds_bytes - (int64_t)dec_pv_lds(max_qc, 0) - 1024;
    // a row's stride is the key count rounded up by at most 15
    const int64_t keys = room / (int64_t)sizeof(float) / max_qc - 15;
    return keys > 0 ? (int)keys : 0;
}

hipError_t launch_attn_decode(const float* q, int ldq, const float* kc, const float* vc, int cap, const AttnItem* items,
                              int n_items, int n_head, int n_kv, int head_dim, float scale, int max_qc, int max_keys,
                              float* scratch, float* ctx, int ldc, const ActQ8* codes, hipStream_t s)
{
    if (head_dim != ATT_HD || n_kv <= 0 || n_head % n_kv != 0 || n_head / n_kv > 4 || max_qc < 1 ||
        max_qc > ATT_DEC_MAX_Q)
        return hipErrorInvalidValue;
    if (n_items <= 0) return hipSuccess;
    const int G = n_head / n_kv;
    const int n_chunks = (max_keys + DEC_KT - 1) / DEC_KT;
    const size_t shs = dec_scores_lds(G, max_qc);
    static LdsLimit scores_limit, pv_limit;
    hipError_t e = scores_limit.raise(reinterpret_cast<const void*>(k_attn_dec_scores), shs);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_dec_scores, dim3((unsigned)(n_items * n_kv * n_chunks)), dim3(256), shs, s, q, ldq, kc,
                       cap, items, n_head, n_kv, n_chunks, scale, scratch);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int ld_s = (max_keys + 15) & ~15;  // the value loop reads weights 16 at a time
    const size_t shp = dec_pv_lds(max_qc, ld_s);
    e = pv_limit.raise(reinterpret_cast<const void*>(k_attn_dec_pv), shp);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_dec_pv, dim3((unsigned)(n_items * n_head * (ATT_HD / 32))), dim3(256), shp, s, vc, cap,
                       items, n_head, n_kv, ld_s, max_qc, scratch, ctx, ldc, codes ? *codes : ActQ8());
    return hipGetLastError();
}

__global__ void k_expf(const float* __restrict__ x, int n, float* __restrict__ y)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = det_expf(x[i]);
}

hipError_t launch_expf(const float* x, int n, float* y, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_expf, dim3((n + 255) / 256), dim3(256), 0, s, x, n, y);
    return hipGetLastError();
}

// ------------------------------------------------------------------ utilities

__global__ void k_copy_rows(const float* __restrict__ src, int lds, float* __restrict__ dst, int ldd, int rows, int cols)
{
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * cols) return;
    int r = (int)(idx / cols), c = (int)(idx % cols);
    dst[(int64_t)r * ldd + c] = src[(int64_t)r * lds + c];
}

hipError_t launch_copy_rows(const float* src, int lds, float* dst, int ldd, int rows, int cols, hipStream_t s)
{
    int64_t n = (int64_t)rows * cols;
    hipLaunchKernelGGL(k_copy_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, lds, dst, ldd, rows, cols);
    return hipGetLastError();
}

__global__ void k_fill_zero(float* p, size_t n)
{
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < n) p[idx] = 0.0f;
}

hipError_t launch_fill_zero(float* p, size_t n, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

// Kernels.Add (Kernels.cs:64): a ← a + b.
__global__ void k_add_inplace(float* __restrict__ a, const float* __restrict__ b, size_t n)
{
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < n) a[idx] = a[idx] + b[idx];
}

hipError_t launch_add_inplace(float* a, const float* b, size_t n, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_add_inplace, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a, b, n);
    return hipGetLastError();
}

__global__ void k_gather_rows(const float* __restrict__ src, int lds, const int32_t* __restrict__ rows, int n, int cols,
                              float* __restrict__ dst, int ldd)
{
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)n * cols) return;
    int r = (int)(idx / cols), c = (int)(idx % cols);
    dst[(int64_t)r * ldd + c] = src[(int64_t)rows[r] * lds + c];
}

hipError_t launch_gather_rows(const float* src, int lds, const int32_t* rows, int n, int cols, float* dst, int ldd,
                              hipStream_t s)
{
    int64_t cnt = (int64_t)n * cols;
    if (cnt == 0) return hipSuccess;
    hipLaunchKernelGGL(k_gather_rows, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, s, src, lds, rows, n, cols, dst, ldd);
    return hipGetLastError();
}

// ------------------------------------------------------ synthetic weights

__device__ inline uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Two standard normals (Box–Muller) from counter c of stream (seed, tensor).
__device__ inline void normal_pair(uint64_t seed, uint64_t tensor, uint64_t c, float* z0, float* z1)
{
    uint64_t u = mix64(seed ^ mix64((tensor << 40) ^ c));
    float u1 = (float)((u >> 40) + 1) * (1.0f / 16777216.0f);
    float u2 = (float)(u & 0xFFFFFFu) * (1.0f / 16777216.0f);
    float r = sqrtf(-2.0f * logf(u1));
    float a = 6.283185307179586f * u2;
    *z0 = r * cosf(a);
    *z1 = r * sinf(a);
}

__device__ inline void wr_half(uint8_t* p, float f)
{
    _Float16 h = (_Float16)f;
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    p[0] = (uint8_t)b;
    p[1] = (uint8_t)(b >> 8);
}

// ggml block quantizers (gguf-py quants.py rules) for one 32-value block.
__device__ void quantize_block(int type, const float* x, uint8_t* p)
{
    int q[32];
    if (type == SHS_TYPE_Q4_0 || type == SHS_TYPE_Q5_0) {
        const bool five = type == SHS_TYPE_Q5_0;
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 32; j++)
            if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); mx = x[j]; }
        float d = mx / (five ? -16.0f : -8.0f);
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t qh = 0;
        for (int j = 0; j < 32; j++) {
            double t = (double)x[j] * (double)id;
            t = t + (five ? 16.5 : 8.5);
            int v = (int)truncf((float)t);
            v = v < 0 ? 0 : (v > (five ? 31 : 15) ? (five ? 31 : 15) : v);
            q[j] = v;
            qh |= (uint32_t)((v >> 4) & 1) << j;
        }
        wr_half(p, d);
        uint8_t* qs = p + 2;
        if (five) {
            for (int k = 0; k < 4; k++) p[2 + k] = (uint8_t)(qh >> (8 * k));
            qs = p + 6;
        }
        for (int j = 0; j < 16; j++) qs[j] = (uint8_t)((q[j] & 0x0F) | ((q[16 + j] & 0x0F) << 4));
    } else if (type == SHS_TYPE_Q4_1 || type == SHS_TYPE_Q5_1) {
        const bool five = type == SHS_TYPE_Q5_1;
        float mx = x[0], mn = x[0];
        for (int j = 1; j < 32; j++) { mx = fmaxf(mx, x[j]); mn = fminf(mn, x[j]); }
        float d = (mx - mn) / (five ? 31.0f : 15.0f);
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t qh = 0;
        for (int j = 0; j < 32; j++) {
            float a = x[j] - mn;
            a = a * id;
            a = a + 0.5f;
            int v = (int)truncf(a);
            v = v < 0 ? 0 : (v > (five ? 31 : 15) ? (five ? 31 : 15) : v);
            q[j] = v;
            qh |= (uint32_t)((v >> 4) & 1) << j;
        }
        wr_half(p, d);
        wr_half(p + 2, mn);
        uint8_t* qs = p + 4;
        if (five) {
            for (int k = 0; k < 4; k++) p[4 + k] = (uint8_t)(qh >> (8 * k));
            qs = p + 8;
        }
        for (int j = 0; j < 16; j++) qs[j] = (uint8_t)((q[j] & 0x0F) | ((q[16 + j] & 0x0F) << 4));
    } else {  // Q8_0
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr_half(p, d);
        for (int j = 0; j < 32; j++) {
            float v = x[j] * id;
            float a = fabsf(v), fl = floorf(a);
            float r = fl + floorf(2.0f * (a - fl));
            p[2 + j] = (uint8_t)(int8_t)(v < 0.0f ? -r : r);
        }
    }
}

__global__ void k_synth_native(int type, int ts, uint64_t seed, uint64_t tensor, int rows, int B, float mean, float std,
                               uint8_t* __restrict__ native)
{
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * B) return;
    float x[32];
    for (int i = 0; i < 16; i++) {
        float z0, z1;
        normal_pair(seed, tensor, (uint64_t)idx * 16 + i, &z0, &z1);
        x[2 * i] = mean + std * z0;
        x[2 * i + 1] = mean + std * z1;
    }
    quantize_block(type, x, native + idx * ts);
}

hipError_t launch_synth_native(int type, uint64_t seed, uint64_t tensor, int rows, int cols, float mean, float std,
                               uint8_t* native, hipStream_t s)
{
    int ts = type == SHS_TYPE_Q4_0 ? 18 : type == SHS_TYPE_Q4_1 ? 20 : type == SHS_TYPE_Q5_0 ? 22
           : type == SHS_TYPE_Q5_1 ? 24 : type == SHS_TYPE_Q8_0 ? 34 : -1;
    if (ts < 0 || cols % 32) return hipErrorInvalidValue;
    int B = cols / 32;
    int64_t n = (int64_t)rows * B;
    hipLaunchKernelGGL(k_synth_native, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, type, ts, seed, tensor, rows, B,
                       mean, std, native);
    return hipGetLastError();
}

__global__ void k_synth_f32(uint64_t seed, uint64_t tensor, int64_t n, float mean, float std, float* __restrict__ out)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (2 * i >= n) return;
    float z0, z1;
    normal_pair(seed, tensor, (uint64_t)i, &z0, &z1);
    out[2 * i] = mean + std * z0;
    if (2 * i + 1 < n) out[2 * i + 1] = mean + std * z1;
}

hipError_t launch_synth_f32(uint64_t seed, uint64_t tensor, int64_t n, float mean, float std, float* out, hipStream_t s)
{
    int64_t pairs = (n + 1) / 2;
    hipLaunchKernelGGL(k_synth_f32, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, s, seed, tensor, n, mean, std, out);
    return hipGetLastError();
}

// -------------------------------------------------------- unpack (inverse)

template <int TYPE>
__global__ void k_unpack_native(const uint8_t* __restrict__ qs, const uint32_t* __restrict__ qh,
                                const float* __restrict__ d, const float* __restrict__ m, int row0, int nrows, int B,
                                uint8_t* __restrict__ native)
{
    typedef BlockFmt<TYPE> F;
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)nrows * B) return;
    int rr = (int)(idx / B), b = (int)(idx % B);
    int r = row0 + rr;
    uint8_t* blk = native + idx * F::TS;
    int64_t rec = (int64_t)(r >> 5) * B + b;
    int ri = r & 31;
    wr_half(blk, d[rec * 32 + ri]);
    if (F::M >= 0) wr_half(blk + F::M, m[rec * 32 + ri]);
    if (F::QH >= 0) {
        uint32_t v = qh[rec * 32 + ri];
        for (int k = 0; k < 4; k++) blk[F::QH + k] = (uint8_t)(v >> (8 * k));
    }
    if (TYPE == SHS_TYPE_Q8_0) {
        const uint8_t* src = qs + rec * 1024 + ri * 32;
        for (int p = 0; p < 32; p++) blk[F::QS + perm_elem(p)] = src[p];
    } else {
        const uint8_t* src = qs + rec * 512 + ri * 16;
        for (int p = 0; p < 16; p++) blk[F::QS + p] = src[p];
    }
}

hipError_t launch_unpack_native(const DevMatrix& w, int row0, int nrows, uint8_t* native, hipStream_t s)
{
    int64_t n = (int64_t)nrows * w.blocks;
    dim3 grid((unsigned)((n + 255) / 256)), block(256);
    switch (w.type) {
    case SHS_TYPE_Q4_0: hipLaunchKernelGGL(k_unpack_native<SHS_TYPE_Q4_0>, grid, block, 0, s, w.qs, w.qh, w.d, w.m, row0, nrows, w.blocks, native); break;
    case SHS_TYPE_Q4_1: hipLaunchKernelGGL(k_unpack_native<SHS_TYPE_Q4_1>, grid, block, 0, s, w.qs, w.qh, w.d, w.m, row0, nrows, w.blocks, native); break;
    case SHS_TYPE_Q5_0: hipLaunchKernelGGL(k_unpack_native<SHS_TYPE_Q5_0>, grid, block, 0, s, w.qs, w.qh, w.d, w.m, row0, nrows, w.blocks, native); break;
    case SHS_TYPE_Q5_1: hipLaunchKernelGGL(k_unpack_native<SHS_TYPE_Q5_1>, grid, block, 0, s, w.qs, w.qh, w.d, w.m, row0, nrows, w.blocks, native); break;
    case SHS_TYPE_Q8_0: hipLaunchKernelGGL(k_unpack_native<SHS_TYPE_Q8_0>, grid, block, 0, s, w.qs, w.qh, w.d, w.m, row0, nrows, w.blocks, native); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------- fixed scratch (no allocation)

// The activation codes of shs_matmul_device_noalloc. Its host-side name is a stand-in, not
// a device address: kernels get the address noalloc_scratch() looks up.
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

hipError_t noalloc_scratch(int device, uint8_t** out)
{
    static std::mutex mu;
    static uint8_t* addr[64] = {};
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[device]) {
        hipError_t e = hipSetDevice(device);
        if (e != hipSuccess) return e;
        void* p = nullptr;
        if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return e;
        addr[device] = static_cast<uint8_t*>(p);
    }
    *out = addr[device];
    return hipSuccess;
}

}  // namespace shs
