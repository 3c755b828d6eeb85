// Instruction-issue probes for the GEMM's and the attention's design choices on gfx950: how
// many cycles each MFMA form and the fp32 VALU FMA take per wave, and which of them overlap when one wave issues
// them together. Built as its own library (libshs_probe.so) beside the product; bench.py
// --isa-probe runs every pattern and prints the table. Nothing here touches memory except
// the one result record per wave (and a sink store that never executes).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

enum {
    P_I8 = 0,         // 4 independent v_mfma_i32_32x32x32_i8 chains
    P_F16X8,          // 4 independent v_mfma_f32_32x32x8_f16 chains
    P_F16X16,         // 4 independent v_mfma_f32_32x32x16_f16 chains
    P_F32_1_2B,       // 2 v_mfma_f32_32x32x1_2b_f32 with C = 0 (the GEMM's scale form)
    P_F32X2,          // 2 independent v_mfma_f32_32x32x2_f32 chains (the attention's form)
    P_FMA,            // 32 independent v_fma_f32 chains
    P_I8_FMA,         // 2 int8 MFMAs + 32 independent FMAs
    P_F16_FMA,        // 2 fp16 (x8) MFMAs + 32 independent FMAs
    P_F32_FMA,        // 1 fp32 1_2b MFMA + 32 independent FMAs
    P_GEMM_BLOCK,     // one block of the GEMM's K loop on two token tiles: scale MFMA, 2 int8,
                      // 2 fp16 conversions, 32 FMAs that read their results
    P_F32X2_CHAIN,    // 4 v_mfma_f32_32x32x2_f32 on one accumulator (the attention's value chain)
    P_F32X2_FMA,      // 1 v_mfma_f32_32x32x2_f32 + 16 independent FMAs (the score phase's mix)
    P_COUNT
};

__device__ __forceinline__ void keep(v16f& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void keep(v16i& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void keep(v32f& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void keep(float& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void keep(v4h& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void keep(v8h& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void keep(v4i& x) { asm volatile("" : "+v"(x)); }

template <int P>
__global__ __launch_bounds__(768) void k_probe(int iters, uint64_t* out, float* sink, int never)
{
    const int lane = threadIdx.x & 63;
    const float fl = (float)lane * 0.001f;
    v4i a4, b4;
    for (int k = 0; k < 4; k++) a4[k] = 0x01010101 * (lane & 3), b4[k] = 0x02020202 * (k + 1);
    v4h ah, bh;
    v8h ah8, bh8;
    for (int k = 0; k < 4; k++) ah[k] = (_Float16)(0.5f * k), bh[k] = (_Float16)(0.25f * k);
    for (int k = 0; k < 8; k++) ah8[k] = (_Float16)(0.5f * k), bh8[k] = (_Float16)(0.25f * k);
    v16i ci[4];
    v16f cf[4];
    v32f z32, c32[2];
    for (int r = 0; r < 16; r++)
        for (int k = 0; k < 4; k++) ci[k][r] = r + k, cf[k][r] = fl + r;
    for (int r = 0; r < 32; r++) z32[r] = 0.0f, c32[0][r] = fl, c32[1][r] = fl + 1.0f;
    float x[32];
    for (int k = 0; k < 32; k++) x[k] = fl + k;
    float fa = 1.0000001f + fl * 1e-6f, fb = 1e-7f;
    keep(fa);
    keep(fb);
    keep(a4);
    keep(b4);
    keep(ah);
    keep(bh);
    keep(ah8);
    keep(bh8);
    v16i magic = ci[2];
    keep(magic);

    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; it++) {
        if constexpr (P == P_I8) {
#pragma unroll
            for (int k = 0; k < 4; k++) ci[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a4, b4, ci[k], 0, 0, 0);
        } else if constexpr (P == P_F16X8) {
#pragma unroll
            for (int k = 0; k < 4; k++) cf[k] = __builtin_amdgcn_mfma_f32_32x32x8f16(ah, bh, cf[k], 0, 0, 0);
        } else if constexpr (P == P_F16X16) {
#pragma unroll
            for (int k = 0; k < 4; k++) cf[k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah8, bh8, cf[k], 0, 0, 0);
        } else if constexpr (P == P_F32_1_2B) {
#pragma unroll
            for (int k = 0; k < 2; k++) {
                keep(fa);
                c32[k] = __builtin_amdgcn_mfma_f32_32x32x1f32(fa, fb, z32, 0, 0, 0);
                keep(c32[k]);
            }
        } else if constexpr (P == P_F32X2) {
#pragma unroll
            for (int k = 0; k < 2; k++) cf[k] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa, fb, cf[k], 0, 0, 0);
        } else if constexpr (P == P_FMA) {
#pragma unroll
            for (int k = 0; k < 32; k++) x[k] = fmaf(x[k], fa, fb);
        } else if constexpr (P == P_I8_FMA) {
#pragma unroll
            for (int k = 0; k < 2; k++) ci[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a4, b4, ci[k], 0, 0, 0);
#pragma unroll
            for (int k = 0; k < 32; k++) x[k] = fmaf(x[k], fa, fb);
        } else if constexpr (P == P_F16_FMA) {
#pragma unroll
            for (int k = 0; k < 2; k++) cf[k] = __builtin_amdgcn_mfma_f32_32x32x8f16(ah, bh, cf[k], 0, 0, 0);
#pragma unroll
            for (int k = 0; k < 32; k++) x[k] = fmaf(x[k], fa, fb);
        } else if constexpr (P == P_F32_FMA) {
            keep(fa);
            c32[0] = __builtin_amdgcn_mfma_f32_32x32x1f32(fa, fb, z32, 0, 0, 0);
            keep(c32[0]);
#pragma unroll
            for (int k = 0; k < 32; k++) x[k] = fmaf(x[k], fa, fb);
        } else if constexpr (P == P_GEMM_BLOCK) {
            keep(fa);
            const v32f S = __builtin_amdgcn_mfma_f32_32x32x1f32(fa, fb, z32, 0, 0, 0);
            const v16i F0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a4, b4, magic, 0, 0, 0);
            const v16i F1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b4, a4, magic, 0, 0, 0);
            const v16f G0 = __builtin_amdgcn_mfma_f32_32x32x8f16(ah, bh, __builtin_bit_cast(v16f, F0), 0, 0, 0);
            const v16f G1 = __builtin_amdgcn_mfma_f32_32x32x8f16(ah, bh, __builtin_bit_cast(v16f, F1), 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                cf[0][r] = fmaf(G0[r], S[r], cf[0][r]);
                cf[1][r] = fmaf(G1[r], S[16 + r], cf[1][r]);
            }
            keep(cf[0]);
            keep(cf[1]);
        } else if constexpr (P == P_F32X2_CHAIN) {
#pragma unroll
            for (int k = 0; k < 4; k++) cf[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa, fb, cf[0], 0, 0, 0);
        } else if constexpr (P == P_F32X2_FMA) {
            cf[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa, fb, cf[0], 0, 0, 0);
#pragma unroll
            for (int k = 0; k < 16; k++) x[k] = fmaf(x[k], fa, fb);
        }
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) {
        const int w = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
        out[4 * w] = t0;
        out[4 * w + 1] = t1;
        out[4 * w + 2] = r0;
        out[4 * w + 3] = r1;
    }
    if (never) {
        // keeps every result live; `never` is 0 on every launch
        float s = 0.0f;
        for (int k = 0; k < 4; k++)
            for (int r = 0; r < 16; r++) s += (float)ci[k][r] + cf[k][r];
        for (int k = 0; k < 2; k++)
            for (int r = 0; r < 32; r++) s += c32[k][r];
        for (int k = 0; k < 32; k++) s += x[k];
        sink[threadIdx.x] = s;
    }
}

template <int P>
hipError_t launch(int blocks, int waves, int iters, uint64_t* out, float* sink)
{
    hipLaunchKernelGGL(k_probe<P>, dim3(blocks), dim3(64 * waves), 0, 0, iters, out, sink, 0);
    return hipGetLastError();
}

hipError_t launch_pattern(int p, int blocks, int waves, int iters, uint64_t* out, float* sink)
{
    switch (p) {
    case P_I8: return launch<P_I8>(blocks, waves, iters, out, sink);
    case P_F16X8: return launch<P_F16X8>(blocks, waves, iters, out, sink);
    case P_F16X16: return launch<P_F16X16>(blocks, waves, iters, out, sink);
    case P_F32_1_2B: return launch<P_F32_1_2B>(blocks, waves, iters, out, sink);
    case P_F32X2: return launch<P_F32X2>(blocks, waves, iters, out, sink);
    case P_FMA: return launch<P_FMA>(blocks, waves, iters, out, sink);
    case P_I8_FMA: return launch<P_I8_FMA>(blocks, waves, iters, out, sink);
    case P_F16_FMA: return launch<P_F16_FMA>(blocks, waves, iters, out, sink);
    case P_F32_FMA: return launch<P_F32_FMA>(blocks, waves, iters, out, sink);
    case P_GEMM_BLOCK: return launch<P_GEMM_BLOCK>(blocks, waves, iters, out, sink);
    case P_F32X2_CHAIN: return launch<P_F32X2_CHAIN>(blocks, waves, iters, out, sink);
    case P_F32X2_FMA: return launch<P_F32X2_FMA>(blocks, waves, iters, out, sink);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

extern "C" {

int shs_probe_count(void) { return P_COUNT; }

// Runs pattern p on `blocks` work-groups of `waves` waves (4 waves = one per SIMD of a CU,
// 12 = three per SIMD) for `iters` iterations. Per work-group, the span from its first wave's
// start to its last wave's end, in shader-clock cycles, divided by the iterations each SIMD
// ran (iters · waves / 4): `simd_cycles_per_iter`, averaged over work-groups; `clock_mhz` from
// the same spans on the 100 MHz real-time counter. Returns 0, or the HIP error code.
int shs_probe_run(int p, int blocks, int waves, int iters, double* simd_cycles_per_iter, double* clock_mhz)
{
    if (p < 0 || p >= P_COUNT || blocks < 1 || blocks > 4096 || waves < 1 || waves > 12 || (waves & 3) != 0 ||
        iters < 1)
        return (int)hipErrorInvalidValue;
    const int nw = blocks * waves;
    uint64_t* out = nullptr;
    float* sink = nullptr;
    hipError_t e = hipMalloc(&out, sizeof(uint64_t) * 4 * nw);
    if (e == hipSuccess) e = hipMalloc(&sink, sizeof(float) * 64 * waves);
    if (e == hipSuccess) e = launch_pattern(p, blocks, waves, 8, out, sink);  // warm-up
    if (e == hipSuccess) e = launch_pattern(p, blocks, waves, iters, out, sink);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    uint64_t* host = (uint64_t*)malloc(sizeof(uint64_t) * 4 * nw);
    if (e == hipSuccess && !host) e = hipErrorOutOfMemory;
    if (e == hipSuccess) e = hipMemcpy(host, out, sizeof(uint64_t) * 4 * nw, hipMemcpyDeviceToHost);
    if (e == hipSuccess) {
        double c = 0.0, r = 0.0;
        for (int b = 0; b < blocks; b++) {
            uint64_t t0 = ~0ull, t1 = 0, r0 = ~0ull, r1 = 0;
            for (int w = b * waves; w < (b + 1) * waves; w++) {
                t0 = host[4 * w] < t0 ? host[4 * w] : t0;
                t1 = host[4 * w + 1] > t1 ? host[4 * w + 1] : t1;
                r0 = host[4 * w + 2] < r0 ? host[4 * w + 2] : r0;
                r1 = host[4 * w + 3] > r1 ? host[4 * w + 3] : r1;
            }
            c += (double)(t1 - t0);
            r += (double)(r1 - r0);
        }
        *simd_cycles_per_iter = c / blocks / ((double)iters * waves / 4);
        *clock_mhz = r > 0 ? c / r * 100.0 : 0.0;
    }
    free(host);
    if (out) (void)hipFree(out);
    if (sink) (void)hipFree(sink);
    return (int)e;
}

}  // extern "C"
