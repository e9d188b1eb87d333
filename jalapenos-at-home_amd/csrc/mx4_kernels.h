// mx4_kernels.h -- host-side launchers of the gfx950 kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mx4 {

// y[m, n] = x[m, k] . dequant(W[n, k])^T on one stream.
struct GemvGroup;
struct GemvArgs {
    const uint8_t* packed;  // [n][k/2]
    const uint8_t* scales;  // [n][k/32]
    const void* x;          // [m][k] f32 or bf16
    float* y;               // [m][n]
    uint32_t m, n, k;
    bool x_bf16;
    hipStream_t stream;
    // The few-token GEMV and the skinny kernel: when set, one launch over the
    // group's weights (all of width k, sharing x; y[s] is [m][n[s]]) instead
    // of packed / scales / y / n, each weight's rows a run of whole row-sets
    // or 16-row tiles of the launch.
    const GemvGroup* group = nullptr;
};

bool gemv_m1_supported(uint32_t k);
hipError_t launch_gemv_m1(const GemvArgs& a, int cus);

// M == 1 over up to 4 weights of width k sharing one x (q|k|v, gate|up).
struct GemvGroup {
    const uint8_t* packed[4];
    const uint8_t* scales[4];
    float* y[4];
    uint32_t n[4];
    uint32_t count, k;
    const void* x;
    bool x_bf16;
    hipStream_t stream;
};
// Kernel configuration of the M == 1 GEMV: waves per team (the team splits a
// row's K), rows per team per iteration, teams in the grid (0: one row-set each).
struct M1Config {
    int wg = 0, r = 0;      // waves per team, rows per team
    int tpw = 0;            // teams per workgroup (x staged in LDS when > 1)
    uint32_t grid = 0;      // teams in the launch (0: one row-set each)
};
hipError_t launch_gemv_m1_group(const GemvGroup& g, int cus, const M1Config* forced);
// 2 <= m <= 4 tokens with bf16 activations: the M == 1 weight stream with
// every decoded weight multiplied into all token rows (exact, like skinny).
bool gemv_mt_supported(uint32_t m, uint32_t k, bool x_bf16);
// teams / tpw (teams per workgroup): 0 = the default launch shape.
hipError_t launch_gemv_mt(const GemvArgs& a, int cus, uint32_t teams = 0, uint32_t tpw = 0);
hipError_t launch_gemv_generic(const GemvArgs& a);
// M = 1 projection + greedy argmax epilogue (a.y may be null); hipErrorNotSupported
// for configurations without the epilogue instance. partial: max_partials keys.
hipError_t launch_gemv_m1_argmax(const GemvArgs& a, uint64_t* partial, uint32_t max_partials, uint32_t* idx,
                                 int cus);
// Embedding rows (engine/src/lib.rs:222-227, engine/src/gpu.metal:43-55): out
// [count][cols] bf16 = decoded row ids[t] truncated to bf16; MXFP4 (packed,
// scales) or bf16 (bf16 != null) table; ids >= rows give zero rows.
hipError_t launch_embed(const uint8_t* packed, const uint8_t* scales, const uint16_t* bf16, const uint32_t* ids,
                        uint32_t count, uint32_t rows, uint32_t cols, uint16_t* out, hipStream_t s);

// Exact skinny path (1 <= m <= 32) on bf16 MFMA with decoded weights.
bool skinny_supported(uint32_t m, uint32_t k);
// Device scratch of the split-K launches (bf16 x; K = 12288 from 17 tokens,
// K = 4096 from 17 tokens on 1024-row weights (four ways) and, two ways,
// from 20 tokens on ring-length weights only (gate/up; q/o at K = 4096 run
// unsplit), when the partial tiles fit): part_tiles partial tiles of 1 KiB and
// count_tiles arrival counts, which must be zero before the first launch and
// are left at zero by every launch. Launches that share it must be ordered
// (one stream). With no scratch, or too little, the kernel runs unsplit.
struct SkinnyScratch {
    float* part = nullptr;
    uint32_t* count = nullptr;
    uint32_t part_tiles = 0, count_tiles = 0;
};
hipError_t launch_skinny(const GemvArgs& a, int cus, const SkinnyScratch& sc);

// Exact GEMM on bf16 MFMA for more than 32 token rows (gemm.hip): K % 128 == 0,
// scale bytes 2..252. GemmConfig picks an instance: waves along M x N and 32x32
// MFMA tiles per wave along M x N (all zero: the default for the shape), and
// the number of K slices across workgroups (ks <= 1: none). A split writes
// ks * m * n f32 partials to `part` (part_bytes of device scratch, shared with
// the other split launches of the stream) and adds them in slice order.
struct GemmConfig {
    int wm = 0, wn = 0, tm = 0, tn = 0, ks = 0;
};
bool gemm_exact_supported(uint32_t m, uint32_t n, uint32_t k, bool x_bf16);
hipError_t launch_gemm_exact(const GemvArgs& a, int cus, const GemmConfig* forced, float* part, uint64_t part_bytes);

// bf16 weights [n][k] (engine/src/lib.rs:255, None arm), any m, f32 accumulation.
hipError_t launch_bf16_matmul(const uint16_t* w, const void* x, bool x_bf16, float* y, uint32_t m, uint32_t n,
                              uint32_t k, hipStream_t s);

// Block-scaled MFMA prefill on requantized activations. Both operands are in
// the fragment-native layout of prefill.hip (launch_to_fragments, or the
// quantizers' fragment output).
// Up to kMaxPrefillGroup weights of the same K that share the activations
// (q|k|v, gate|up) run as one launch: segment s owns the workgroup columns
// from its own first tile on, each with its own weight and output.
constexpr uint32_t kMaxPrefillGroup = 4;
struct PrefillArgs {
    const uint8_t* wf[kMaxPrefillGroup];   // weight codes, fragment-native, rows padded to 32
    const uint8_t* wsf[kMaxPrefillGroup];  // weight scales, fragment-native
    float* y[kMaxPrefillGroup];            // [m][n[s]]
    uint32_t n[kMaxPrefillGroup];          // rows of each weight
    uint32_t count;                        // weights in the group, 1..kMaxPrefillGroup
    const uint8_t* xf;                     // requantized activations: fp4 or fp8 fragments
    const uint8_t* xsf;                    // activation scales, fragment-native
    uint32_t m, k;
    bool fp8;                              // activations are MX-FP8 (E4M3) instead of MXFP4
    hipStream_t stream;
    // 0: the default for the shape; else the workgroup tile (rows, columns)
    // and K split inside it of a compiled instance (hipErrorNotSupported if none)
    uint32_t tile_m = 0, tile_n = 0, split_k = 0;
};
bool prefill_supported(uint32_t m, uint32_t n, uint32_t k);
hipError_t launch_prefill(const PrefillArgs& a, int cus);
// Sizes of the fragment-native copies of a rows x k operand (rows padded to 32).
uint64_t fragment_bytes(uint32_t rows, uint32_t k, bool fp8);
uint64_t fragment_scale_bytes(uint32_t rows, uint32_t k);
// Row-major codes [rows][k/2] (fp4) or [rows][k] (fp8) + scales [rows][k/32]
// -> fragment-native copies.
hipError_t launch_to_fragments(const uint8_t* codes, const uint8_t* scales, uint32_t rows, uint32_t k, bool fp8,
                               uint8_t* codes_f, uint8_t* scales_f, hipStream_t s);

// quantize_mxfp4.py:18-39 on device: rows x cols (cols % 32 == 0) f32/bf16 ->
// packed [rows][cols/2] + scales [rows][cols/32]. Non-finite input sets *bad.
hipError_t launch_quantize_mxfp4(const void* in, bool in_bf16, uint64_t rows, uint32_t cols,
                                 uint8_t* packed, uint8_t* scales, uint32_t* bad, hipStream_t s);
// MX-FP8 (E4M3): codes [rows][cols] + scales [rows][cols/32]
hipError_t launch_quantize_fp8(const void* in, bool in_bf16, uint64_t rows, uint32_t cols,
                               uint8_t* codes, uint8_t* scales, uint32_t* bad, hipStream_t s);
// The same two rules writing the fragment-native layout of prefill.hip
// (cols % 256 == 0); rows past `rows` in the last group of 32 are written as zeros.
hipError_t launch_quantize_fragments(const void* in, bool in_bf16, uint32_t rows, uint32_t cols, bool fp8,
                                     uint8_t* codes_f, uint8_t* scales_f, uint32_t* bad, hipStream_t s);
// engine/src/mxfp4.rs:35-49 on device: packed/scales -> f32 [elements]
hipError_t launch_dequantize(const uint8_t* packed, const uint8_t* scales, uint64_t elements,
                             float* out, hipStream_t s);
// engine/src/model.rs:288-296 per row; `partial` holds max_partials keys of
// scratch for rows split over several blocks.
hipError_t launch_argmax_rows(const float* x, uint32_t rows, uint32_t width, uint32_t* out, uint64_t* partial,
                              uint32_t max_partials, int cus, hipStream_t s);
// Row r's index from the keys partial[r * count .. + count) (0 when all are 0).
hipError_t launch_argmax_reduce(const uint64_t* partial, uint32_t rows, uint32_t count, uint32_t* out,
                                hipStream_t s);
// Synthetic inputs (SplitMix64 -> Box-Muller -> sigma -> f32 -> bf16)
hipError_t launch_synth_bf16(uint64_t seed, double sigma, uint64_t start, uint64_t count,
                             uint16_t* out, hipStream_t s);
hipError_t launch_synth_weight(uint64_t seed, double sigma, uint32_t rows, uint32_t cols,
                               uint8_t* packed, uint8_t* scales, hipStream_t s);
// Smallest scale byte of a resident weight (flags subnormal-scale blocks)
hipError_t launch_min_max_scale(const uint8_t* scales, uint64_t count, uint32_t* out2,
                                hipStream_t s);
// Hardware-converter table for the exhaustive decode check: out[s*16 + c]
hipError_t launch_decode_table(int mode, float* out, hipStream_t s);
// Matrix-core ceiling probe (probe.hip): back-to-back scaled FP4 MFMAs
// (shape 0: 32x32x64, 1: 16x16x128) on `grid` workgroups of eight waves;
// clocks[4 w ..] = shader clock and wall clock at the start and end of wave
// w's loop; sink[grid * 512] keeps the results.
uint32_t mfma_ceiling_waves(uint32_t grid);
double mfma_ceiling_flops(int shape, uint32_t iters, uint32_t grid);
hipError_t launch_mfma_ceiling(int shape, uint32_t iters, bool random, uint32_t grid, uint64_t* clocks, float* sink,
                               hipStream_t s);

}  // namespace mx4
