// probe.hip -- what the matrix cores of this part sustain on the instructions
// of the matrix-core kernels, for the measurement of their rooflines.
//
// MI355X's published dense rates (MXFP4 10.1, FP8 5.0, bf16 2.5 PFLOP/s) are
// 256 CUs x 4 SIMDs x the instructions' issue rates at 2.4 GHz. Under a
// sustained MFMA load the part lowers its shader clock, and by how much
// depends on the operand values: the same instruction stream on random codes
// holds a lower clock than on constant codes. This kernel issues one kind of
// MFMA back to back on every SIMD (two waves per SIMD, a workgroup of eight
// waves per CU, independent accumulators, operands rotating over four
// register sets so that consecutive instructions see different codes) and
// records, per wave, the shader clock counter (s_memtime) and the
// constant-rate wall clock (s_memrealtime) around the loop: the rate it
// reaches and the clock it holds are the ceiling a kernel built on that
// instruction and operand statistics can approach. Shapes: 0 the block-scaled
// 32x32x64 FP4 x FP4 (MXFP4 prefill), 1 its 16x16x128 form, 2 the block-scaled
// 32x32x64 FP8 x FP4 (MX-FP8 prefill), 3 the bf16 32x32x16 (exact GEMM).
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

// Accumulators per wave and flops per instruction of each shape.
__host__ __device__ constexpr int probe_nacc(int shape) { return shape == 1 ? 16 : 8; }
__host__ __device__ constexpr double probe_flops(int shape) {
    return shape == 1 ? 2.0 * 16 * 16 * 128 : shape == 3 ? 2.0 * 32 * 32 * 16 : 2.0 * 32 * 32 * 64;
}

// Random operand words: FP4 codes are any nibbles; E4M3 bytes keep bit 3 of
// each nibble clear (never the NaN pattern); bf16 halves keep |v| < 2.
template <int SHAPE>
__device__ __forceinline__ uint32_t probe_word(uint32_t h, bool a_side) {
    if constexpr (SHAPE == 2) return a_side ? (h & 0x77777777u) : h;
    if constexpr (SHAPE == 3) return h & 0xbfffbfffu;
    return h;
}

// `iters` is a multiple of 4.
template <int SHAPE>
__global__ __launch_bounds__(64 * kProbeWaves) void mfma_ceiling_kernel(uint32_t iters, uint32_t random,
                                                                       uint64_t* __restrict__ clocks,
                                                                       float* __restrict__ sink) {
    constexpr int NACC = probe_nacc(SHAPE);
    using Acc = typename std::conditional<SHAPE == 1, f32x4, f32x16>::type;
    // registers each operand uses: FP4 four, E4M3 eight, bf16 four
    constexpr int AW = SHAPE == 2 ? 8 : 4;
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t gw = blockIdx.x * kProbeWaves + threadIdx.x / 64;
    const uint32_t fixed = SHAPE == 3 ? 0x3f803f80u : 0x22222222u;  // bf16 1.0 pairs / small codes
    i32x8 a[4], b[4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t ha = probe_mix((gw * 64 + lane) * 64 + s * 8 + j);
            const uint32_t hb = probe_mix(ha ^ 0x9e3779b9u);
            a[s][j] = j < AW ? (int)(random ? probe_word<SHAPE>(ha, true) : fixed) : 0;
            b[s][j] = j < 4 ? (int)(random ? probe_word<SHAPE>(hb, false) : fixed) : 0;
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
                const i32x8& av = a[i % 4];
                const i32x8& bv = b[(i / 2 + r) % 4];
                if constexpr (SHAPE == 0)
                    acc[i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc[i], 4, 4, 0, 127, 0, 127);
                else if constexpr (SHAPE == 1)
                    acc[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc[i], 4, 4, 0, 127, 0, 127);
                else if constexpr (SHAPE == 2)
                    acc[i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc[i], 0, 4, 0, 127, 0, 127);
                else
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, u32x4{(uint32_t)av[0], (uint32_t)av[1], (uint32_t)av[2], (uint32_t)av[3]}),
                        __builtin_bit_cast(bf16x8, u32x4{(uint32_t)bv[0], (uint32_t)bv[1], (uint32_t)bv[2], (uint32_t)bv[3]}),
                        acc[i], 0, 0, 0);
            }
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NACC; ++i)
#pragma unroll
        for (int v = 0; v < (SHAPE == 1 ? 4 : 16); ++v) s += acc[i][v];
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
    return probe_flops(shape) * probe_nacc(shape) * (double)iters * (double)mfma_ceiling_waves(grid);
}

hipError_t launch_mfma_ceiling(int shape, uint32_t iters, bool random, uint32_t grid, uint64_t* clocks, float* sink,
                               hipStream_t s) {
    if (shape < 0 || shape > 3 || iters % 4 != 0 || grid == 0) return hipErrorInvalidValue;
    const dim3 g(grid), b(64 * kProbeWaves);
    switch (shape) {
        case 0: hipLaunchKernelGGL(mfma_ceiling_kernel<0>, g, b, 0, s, iters, (uint32_t)random, clocks, sink); break;
        case 1: hipLaunchKernelGGL(mfma_ceiling_kernel<1>, g, b, 0, s, iters, (uint32_t)random, clocks, sink); break;
        case 2: hipLaunchKernelGGL(mfma_ceiling_kernel<2>, g, b, 0, s, iters, (uint32_t)random, clocks, sink); break;
        default: hipLaunchKernelGGL(mfma_ceiling_kernel<3>, g, b, 0, s, iters, (uint32_t)random, clocks, sink); break;
    }
    return hipGetLastError();
}

}  // namespace mx4
