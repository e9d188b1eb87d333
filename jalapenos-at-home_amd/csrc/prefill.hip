// prefill.hip -- prefill GEMM (many token rows) on CDNA4 block-scaled MFMA:
// y[m, n] = sum_k xq[m, k] * w(n, k) with V_MFMA_SCALE_F32_32X32X64_F8F6F4.
//
// The reference runs prefill on a 16x16 FP32 tiled kernel that decodes each
// weight element into threadgroup memory (project_mxfp4,
// engine/src/matmul.metal:65-97). Here the weights stay in their MXFP4 form all
// the way into the matrix core: operand B is the packed E2M1 nibbles exactly as
// stored (element 2j in the low nibble of byte j, which is also the operand's
// element order) with the E8M0 byte of each 32-element block as the lane's B
// scale. Operand A is the activations after per-32 requantization (MXFP4 by the
// same rule as the weights, python/quantize_mxfp4.py:18-39, or MX-FP8 E4M3),
// with their E8M0 bytes as A scales. Products of FP4/FP8 values with power-of-
// two scales are exact; the matrix core accumulates in f32.
//
// Operand layout (32x32x64), established by in-bounds probes and pinned by the
// identity tests: for FP4, lane l holds row (l % 32) of A (column of B) and the
// 32 K values [32 (l / 32), +32) of the 64 -- one MX block; for FP8 A, lane
// group h = l / 32 holds K [16h, 16h + 16) and [32 + 16h, +16). Either way the
// scale byte of lane group h applies to K block h. C: lane l holds column
// l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4 of accumulator register v.
//
// Tiling: a 256-thread workgroup computes a 128 x 128 output tile as 2 x 2
// waves of 64 x 64 (2 x 2 MFMA tiles each). K advances in stages of 256: each
// stage's A and B tiles (128 rows x 128 bytes of FP4, or 256 bytes of FP8) and
// their scales are loaded with 128-byte contiguous row segments into registers,
// written to padded LDS, and consumed while the next stage is in flight.
#include "mx4_device.h"
#include "mx4_kernels.h"

namespace mx4 {

namespace {

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// See skinny.hip: drain the matrix pipe before accumulators are read after a branch.
__device__ __forceinline__ void mfma_drain() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    __builtin_amdgcn_sched_barrier(0);
}

constexpr int BM = 128, BN = 128, KS = 256;   // tile rows, cols, K per stage
constexpr int kFmtFp8 = 0, kFmtFp4 = 4;        // MFMA operand format codes (cbsz / blgp)

template <bool A_FP8>
struct Cfg {
    static constexpr uint32_t a_row = A_FP8 ? KS : KS / 2;  // bytes of A per row per stage
    static constexpr uint32_t b_row = KS / 2;
    static constexpr uint32_t a_pitch = a_row + 16;          // LDS row pitch (bank spread)
    static constexpr uint32_t b_pitch = b_row + 16;
    static constexpr uint32_t a_bytes = BM * a_pitch;
    static constexpr uint32_t b_bytes = BN * b_pitch;
    static constexpr uint32_t a_loads = BM * a_row / (256 * 16);  // 16-byte loads per thread
    static constexpr uint32_t b_loads = BN * b_row / (256 * 16);
};

template <bool A_FP8>
__global__ __launch_bounds__(256) void prefill_kernel(const uint8_t* __restrict__ wq, const uint8_t* __restrict__ ws,
                                                      const uint8_t* __restrict__ xq, const uint8_t* __restrict__ xs,
                                                      float* __restrict__ y, uint32_t m, uint32_t n, uint32_t k) {
    using C = Cfg<A_FP8>;
    const uint32_t t = threadIdx.x, lane = t % 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t / 64);
    const uint32_t wm = wave / 2, wn = wave % 2;  // wave position in the 2 x 2 grid
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const uint32_t stages = k / KS;
    const uint32_t a_rowbytes = A_FP8 ? k : k / 2, b_rowbytes = k / 2, sblk = k / 32;

    // bounded views: rows past m or n read as zeros
    const uint32_t arows = m - m0 < (uint32_t)BM ? m - m0 : (uint32_t)BM;
    const uint32_t brows = n - n0 < (uint32_t)BN ? n - n0 : (uint32_t)BN;
    const __amdgpu_buffer_rsrc_t ar = rsrc(xq + (size_t)m0 * a_rowbytes, arows * a_rowbytes);
    const __amdgpu_buffer_rsrc_t br = rsrc(wq + (size_t)n0 * b_rowbytes, brows * b_rowbytes);
    const __amdgpu_buffer_rsrc_t asr = rsrc(xs + (size_t)m0 * sblk, arows * sblk);
    const __amdgpu_buffer_rsrc_t bsr = rsrc(ws + (size_t)n0 * sblk, brows * sblk);

    __shared__ __attribute__((aligned(16))) uint8_t lds_a[2][C::a_bytes];
    __shared__ __attribute__((aligned(16))) uint8_t lds_b[2][C::b_bytes];
    __shared__ uint32_t lds_as[2][BM * (KS / 32) / 4];  // scale bytes, [row][8 blocks]
    __shared__ uint32_t lds_bs[2][BN * (KS / 32) / 4];

    // global -> register staging: thread t covers 16-byte pieces of the tile
    struct Stage {
        u32x4 a[C::a_loads];
        u32x4 b[C::b_loads];
        uint32_t as, bs;
    };
    constexpr uint32_t a_pieces = C::a_row / 16, b_pieces = C::b_row / 16;
    auto gload = [&](uint32_t s, Stage& st) {
        const uint32_t aoff = s * C::a_row, boff = s * C::b_row, soff = s * (KS / 32);
#pragma unroll
        for (uint32_t i = 0; i < C::a_loads; ++i) {
            const uint32_t p = t + 256 * i, row = p / a_pieces, piece = p % a_pieces;
            st.a[i] = __builtin_amdgcn_raw_buffer_load_b128(ar, row * a_rowbytes + aoff + 16 * piece, 0, 0);
        }
#pragma unroll
        for (uint32_t i = 0; i < C::b_loads; ++i) {
            const uint32_t p = t + 256 * i, row = p / b_pieces, piece = p % b_pieces;
            st.b[i] = __builtin_amdgcn_raw_buffer_load_b128(br, row * b_rowbytes + boff + 16 * piece, 0, 2);
        }
        // 8 scale bytes per row per stage: thread t takes row t / 2, half t % 2
        st.as = __builtin_amdgcn_raw_buffer_load_b32(asr, (t / 2) * sblk + soff + 4 * (t % 2), 0, 0);
        st.bs = __builtin_amdgcn_raw_buffer_load_b32(bsr, (t / 2) * sblk + soff + 4 * (t % 2), 0, 0);
    };
    auto lstore = [&](uint32_t buf, const Stage& st) {
#pragma unroll
        for (uint32_t i = 0; i < C::a_loads; ++i) {
            const uint32_t p = t + 256 * i, row = p / a_pieces, piece = p % a_pieces;
            *reinterpret_cast<u32x4*>(&lds_a[buf][row * C::a_pitch + 16 * piece]) = st.a[i];
        }
#pragma unroll
        for (uint32_t i = 0; i < C::b_loads; ++i) {
            const uint32_t p = t + 256 * i, row = p / b_pieces, piece = p % b_pieces;
            *reinterpret_cast<u32x4*>(&lds_b[buf][row * C::b_pitch + 16 * piece]) = st.b[i];
        }
        lds_as[buf][t] = st.as;
        lds_bs[buf][t] = st.bs;
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const uint32_t r32 = lane % 32, h = lane / 32;
    auto compute = [&](uint32_t buf) {
        const uint8_t* la = lds_a[buf];
        const uint8_t* lb = lds_b[buf];
        const uint8_t* las = reinterpret_cast<const uint8_t*>(lds_as[buf]);
        const uint8_t* lbs = reinterpret_cast<const uint8_t*>(lds_bs[buf]);
#pragma unroll
        for (uint32_t ks = 0; ks < KS / 64; ++ks) {
            i32x8 af[2], bf[2];
            int32_t sa[2], sb[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t row = wm * 64 + i * 32 + r32;
                if constexpr (A_FP8) {
                    // 8-bit operands interleave the K halves: lane group h holds K
                    // [16h, 16h + 16) in registers 0-3 and [32 + 16h, +16) in 4-7;
                    // the scale of K block b still comes from lane group b.
                    const uint8_t* p = la + row * C::a_pitch + ks * 64 + h * 16;
                    const u32x4 lo = *reinterpret_cast<const u32x4*>(p);
                    const u32x4 hi = *reinterpret_cast<const u32x4*>(p + 32);
                    af[i] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
                } else {
                    const u32x4 v = *reinterpret_cast<const u32x4*>(la + row * C::a_pitch + ks * 32 + h * 16);
                    af[i] = i32x8{(int)v[0], (int)v[1], (int)v[2], (int)v[3], 0, 0, 0, 0};
                }
                sa[i] = las[row * 8 + ks * 2 + h];
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t row = wn * 64 + j * 32 + r32;
                const u32x4 v = *reinterpret_cast<const u32x4*>(lb + row * C::b_pitch + ks * 32 + h * 16);
                bf[j] = i32x8{(int)v[0], (int)v[1], (int)v[2], (int)v[3], 0, 0, 0, 0};
                sb[j] = lbs[row * 8 + ks * 2 + h];
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        af[i], bf[j], acc[i][j], A_FP8 ? kFmtFp8 : kFmtFp4, kFmtFp4, 0, sa[i], 0, sb[j]);
        }
    };

    Stage st;
    gload(0, st);
    lstore(0, st);
    __syncthreads();
    for (uint32_t s = 0; s < stages; ++s) {
        const uint32_t buf = s & 1;
        const bool more = s + 1 < stages;
        if (more) gload(s + 1, st);
        compute(buf);
        if (more) lstore(buf ^ 1, st);
        __syncthreads();
    }
    mfma_drain();

    // write the 64 x 64 wave tile
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t col = n0 + wn * 64 + j * 32 + r32;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t row = m0 + wm * 64 + i * 32 + 8 * (v / 4) + 4 * h + (v % 4);
                if (row < m && col < n) y[(size_t)row * n + col] = acc[i][j][v];
            }
        }
}

}  // namespace

bool prefill_supported(uint32_t m, uint32_t n, uint32_t k) {
    return m >= 1 && n >= 1 && k % KS == 0 && k >= KS && (uint64_t)n * (k / 2) < (1ull << 31) &&
           (uint64_t)m * k < (1ull << 31);
}

hipError_t launch_prefill(const PrefillArgs& a, int) {
    if (!prefill_supported(a.m, a.n, a.k)) return hipErrorNotSupported;
    dim3 grid((a.n + BN - 1) / BN, (a.m + BM - 1) / BM);
    if (a.fp8)
        hipLaunchKernelGGL(prefill_kernel<true>, grid, dim3(256), 0, a.stream, a.packed, a.scales, a.xq, a.xs, a.y,
                           a.m, a.n, a.k);
    else
        hipLaunchKernelGGL(prefill_kernel<false>, grid, dim3(256), 0, a.stream, a.packed, a.scales, a.xq, a.xs, a.y,
                           a.m, a.n, a.k);
    return hipGetLastError();
}

}  // namespace mx4
