// probe.hip -- what the matrix cores of this part sustain on the prefill
// GEMM's instruction, for the measurement of the prefill roofline.
//
// MI355X's published dense MXFP4 rate (10.1 PFLOP/s) is 256 CUs x 4 SIMDs x
// one V_MFMA_SCALE_F32_32X32X64_F8F6F4 (FP4 x FP4) every 32 cycles at
// 2.4 GHz. Under a sustained MFMA load the part lowers its shader clock, and
// by how much depends on the operand values: the same instruction stream on
// random E2M1 codes holds a lower clock than on constant codes. This kernel
// issues scaled FP4 MFMAs back to back on every SIMD (two waves per SIMD, a
// workgroup of eight waves per CU, independent accumulators, operands
// rotating over four register sets so that consecutive instructions see
// different codes) and records, per wave, the shader clock counter
// (s_memtime) and the constant-rate wall clock (s_memrealtime) around the
// loop: the rate it reaches and the clock it holds are the ceiling a GEMM on
// these operands can approach, against which the prefill kernels are read.
#include "mx4_device.h"
#include "mx4_kernels.h"

namespace mx4 {

namespace {

constexpr int kProbeWaves = 8;  // two per SIMD

__device__ __forceinline__ uint32_t probe_mix(uint32_t x) {
    // a 32-bit finalizer (xorshift-multiply) for the random operand codes
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// SHAPE 0: 32x32x64 (8 accumulators of 16 floats per wave); 1: 16x16x128
// (16 accumulators of 4 floats). `iters` is a multiple of 4.
template <int SHAPE>
__global__ __launch_bounds__(64 * kProbeWaves) void mfma_ceiling_kernel(uint32_t iters, uint32_t random,
                                                                       uint64_t* __restrict__ clocks,
                                                                       float* __restrict__ sink) {
    constexpr int NACC = SHAPE == 0 ? 8 : 16;
    using Acc = typename std::conditional<SHAPE == 0, f32x16, f32x4>::type;
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t gw = blockIdx.x * kProbeWaves + threadIdx.x / 64;
    i32x8 a[4], b[4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // an FP4 operand is the first four registers; the rest stay zero
            const uint32_t ha = probe_mix((gw * 64 + lane) * 64 + s * 8 + j);
            const uint32_t hb = probe_mix(ha ^ 0x9e3779b9u);
            a[s][j] = j < 4 ? (int)(random ? ha : 0x22222222u) : 0;
            b[s][j] = j < 4 ? (int)(random ? hb : 0x22222222u) : 0;
        }
    Acc acc[NACC];
#pragma unroll
    for (int i = 0; i < NACC; ++i) acc[i] = Acc{};
    const uint64_t c0 = clock64(), w0 = wall_clock64();
    for (uint32_t it = 0; it < iters; it += 4) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < NACC; ++i) {
                if constexpr (SHAPE == 0)
                    acc[i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[i % 4], b[(i / 2 + r) % 4], acc[i], 4,
                                                                            4, 0, 127, 0, 127);
                else
                    acc[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[i % 4], b[(i / 2 + r) % 4], acc[i],
                                                                             4, 4, 0, 127, 0, 127);
            }
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NACC; ++i)
#pragma unroll
        for (int v = 0; v < (SHAPE == 0 ? 16 : 4); ++v) s += acc[i][v];
    const uint64_t c1 = clock64(), w1 = wall_clock64();
    sink[blockIdx.x * 64 * kProbeWaves + threadIdx.x] = s;  // keeps the MFMAs
    if (lane == 0) {
        clocks[4 * gw + 0] = c0;
        clocks[4 * gw + 1] = c1;
        clocks[4 * gw + 2] = w0;
        clocks[4 * gw + 3] = w1;
    }
}

}  // namespace

uint32_t mfma_ceiling_waves(uint32_t grid) { return grid * kProbeWaves; }

double mfma_ceiling_flops(int shape, uint32_t iters, uint32_t grid) {
    const double per = shape == 0 ? 2.0 * 32 * 32 * 64 : 2.0 * 16 * 16 * 128;
    const double nacc = shape == 0 ? 8 : 16;
    return per * nacc * (double)iters * (double)mfma_ceiling_waves(grid);
}

hipError_t launch_mfma_ceiling(int shape, uint32_t iters, bool random, uint32_t grid, uint64_t* clocks, float* sink,
                               hipStream_t s) {
    if ((shape != 0 && shape != 1) || iters % 4 != 0 || grid == 0) return hipErrorInvalidValue;
    if (shape == 0)
        hipLaunchKernelGGL(mfma_ceiling_kernel<0>, dim3(grid), dim3(64 * kProbeWaves), 0, s, iters, (uint32_t)random,
                           clocks, sink);
    else
        hipLaunchKernelGGL(mfma_ceiling_kernel<1>, dim3(grid), dim3(64 * kProbeWaves), 0, s, iters, (uint32_t)random,
                           clocks, sink);
    return hipGetLastError();
}

}  // namespace mx4
