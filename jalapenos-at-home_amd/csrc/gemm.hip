// gemm.hip -- exact matrix-core GEMM for more than 32 token rows:
// y[m, r] = sum_k x[m, k] * w(r, k), f32 accumulation of exact products.
//
// The reference sends every projection with M > 32 token rows (and, through
// its per-call bridge, every M > 1) to a tiled FP32 GEMM that decodes the
// weights into threadgroup tiles (project_mxfp4, engine/src/matmul.metal:65-97;
// dispatch engine/src/gpu.rs:510-514, engine/src/metal.m:103-105). Here the
// multiply-accumulate runs on gfx950's V_MFMA_F32_32X32X16_BF16 while the
// weights stay 4-bit in HBM, in the stored row-major layout:
//  * a workgroup owns a BM x BN output tile (token rows x weight rows) and
//    walks K in stages of 128. Each stage's activations (BM rows x 256 bytes
//    of bf16) and weights (BN rows x 64 packed bytes + 4 scale bytes) are
//    loaded straight into LDS (direct-to-LDS buffer loads, whole rows per
//    instruction) into a ring of D stages, D - 1 of them in flight while one
//    is computed (one barrier per stage);
//  * a wave owns TM x TN 32x32 MFMA tiles. Lane l (row l % 32, half h = l / 32)
//    takes elements [64h, 64h + 64) of the stage for both operands; k-step s
//    of the stage contracts elements [64h + 8s, +8). The contraction is over
//    K, so this order, shared by A and B, changes nothing in the result;
//  * a weight lane reads its row's 32 packed bytes once per stage and decodes
//    8 elements per k-step with the hardware E2M1 converter, the E8M0 scale
//    folded in (exact in bf16 for scale bytes 2..252, which the dispatcher
//    guarantees);
//  * bf16 activations are exact operands; f32 activations are split into three
//    bf16 terms hi + mid + lo (24 significant bits), three MFMAs each, so every
//    product is exact and only the f32 summation order differs from the
//    reference's sequential loop (engine/src/lib.rs:240-266);
//  * every global load goes through a buffer resource: token rows >= M and
//    weight rows >= N read as zeros without touching memory, and their outputs
//    are not stored.
#include <type_traits>
#include "mx4_device.h"
#include "mx4_kernels.h"

namespace mx4 {

namespace {

// Three bf16 terms of eight f32 values, hi + mid + lo = x exactly
// (split3_bf16: non-finite values stay in hi).
__device__ __forceinline__ void split3x8(const f32x4 a, const f32x4 b, bf16x8& hi, bf16x8& mid, bf16x8& lo) {
    const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        __bf16 h, md, l;
        split3_bf16(v[e], h, md, l);
        hi[e] = h;
        mid[e] = md;
        lo[e] = l;
    }
}

// Eight weights of one lane at one k-step: packed word `word` (elements
// [8s, 8s + 8) of the lane's 64), block scale 2^(s - 127) folded in.
__device__ __forceinline__ bf16x8 decode8(uint32_t word, float sc) {
    const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 0);
    const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 1);
    const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 2);
    const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 3);
    bf16x8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

// Wait states after the last MFMAs before their accumulators are read (the
// compiler has placed such reads after a branch without them on gfx950).
__device__ __forceinline__ void mfma_drain() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7");
    __builtin_amdgcn_sched_barrier(0);
}

constexpr int kBK = 128;  // K elements per stage

// Stage layout in LDS (no padding): activations BM rows x A_CPR 16-byte slots,
// packed weights BN rows x 4 slots, then BN scale words. Slots are written by
// direct-to-LDS buffer loads, lane l of a load instruction at slot base + l,
// so the layout is chosen through which global chunk each lane loads: chunk c
// of row r sits in slot c ^ (r % 16) of an activation row and c ^ ((r / 4) % 4)
// of a weight row. The MFMA-operand reads (32 rows, one logical chunk) then
// spread over all LDS banks.
template <bool XBF16, int WM, int WN, int TM, int TN, int D>
struct Geometry {
    static constexpr int NW = WM * WN, NT = 64 * NW;
    static constexpr int BM = 32 * TM * WM, BN = 32 * TN * WN;
    static constexpr int XB = XBF16 ? 2 : 4;              // bytes per activation element
    static constexpr int A_CPR = kBK * XB / 16;           // 16-byte chunks per activation row
    static constexpr int A_BYTES = BM * A_CPR * 16, B_BYTES = BN * 4 * 16, S_BYTES = BN * 4;
    static constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;
    static constexpr int A_INSTR = BM * A_CPR / NT;       // 64-lane loads per wave per stage
    static constexpr int B_INSTR = BN * 4 / NT;
    static constexpr int S_ROWS = BN / NW;                // scale words per wave per stage
    static constexpr int LPS = A_INSTR + B_INSTR + 1;     // vector memory instructions per stage
    static_assert(BM * A_CPR % NT == 0 && BN * 4 % NT == 0 && BN % NW == 0 && S_ROWS <= 64, "stage split");
    static_assert(D >= 2 && D <= 4 && (D - 2) * LPS <= 63, "vmcnt range");
    static_assert(D * STAGE <= 160 * 1024, "the stages must fit the LDS");
};

// Up to four weights of one width sharing x (q|k|v, gate|up at more than 32
// token rows) in one launch: weight s owns the column tiles [tile0[s],
// tile0[s + 1]) of the grid; a workgroup picks its weight with uniform
// selects. Passed as the trailing argument, so the leading scalars keep
// arriving preloaded; NoGemmSegs stands there for one weight. No K split.
struct NoGemmSegs {};
struct GemmSegs {
    const uint8_t* packed[4];
    const uint8_t* scales[4];
    float* y[4];
    uint32_t n[4];
    uint32_t tile0[4];
    uint32_t count;
};

template <bool XBF16, int WM, int WN, int TM, int TN, int D, class SG = NoGemmSegs>
__global__ __launch_bounds__(64 * WM * WN) void gemm_exact_kernel(const uint8_t* __restrict__ packed,
                                                                  const uint8_t* __restrict__ scales,
                                                                  const void* __restrict__ x, float* __restrict__ y,
                                                                  uint32_t m, uint32_t n, uint32_t k,
                                                                  uint32_t tiles_n, uint32_t tiles,
                                                                  uint32_t kslice, float* __restrict__ part,
                                                                  const SG group) {
    using G = Geometry<XBF16, WM, WN, TM, TN, D>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[D * G::STAGE];
    const uint32_t lane = threadIdx.x % 64, h = lane / 32, r32 = lane % 32;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t wm = wave / WN, wn = wave % WN;
    // K split: workgroup b takes tile b % tiles over K slice b / tiles and
    // writes its partial tile to part[slice][m][n] (summed afterwards in slice order)
    const uint32_t slice = blockIdx.x / tiles, tile = blockIdx.x % tiles;
    uint32_t tn = tile % tiles_n;
    const uint32_t tm = tile / tiles_n;
    if constexpr (std::is_same_v<SG, GemmSegs>) {
        // the column tile's weight, and the tile within it
        uint32_t t0 = 0;
        packed = group.packed[0];
        scales = group.scales[0];
        y = group.y[0];
        n = group.n[0];
#pragma unroll
        for (int q = 1; q < 4; ++q) {
            const bool in = q < (int)group.count && tn >= group.tile0[q];
            packed = in ? group.packed[q] : packed;
            scales = in ? group.scales[q] : scales;
            y = in ? group.y[q] : y;
            n = in ? group.n[q] : n;
            t0 = in ? group.tile0[q] : t0;
        }
        tn -= t0;
    }
    const uint32_t row0 = tm * G::BM, col0 = tn * G::BN;
    const uint32_t k0 = slice * kslice, stages = kslice / kBK;
    if (part) y = part + (size_t)slice * m * n;

    const __amdgpu_buffer_rsrc_t xr = rsrc(x, m * k * G::XB);
    const __amdgpu_buffer_rsrc_t pr = rsrc(packed, n * (k / 2));
    const __amdgpu_buffer_rsrc_t sr = rsrc(scales, n * (k / 32));

    // this lane's global offsets (stage 0) of its loads; LDS slot p = (q NW + wave) 64 + lane
    uint32_t a_goff[G::A_INSTR], b_goff[G::B_INSTR];
#pragma unroll
    for (int q = 0; q < G::A_INSTR; ++q) {
        const uint32_t p = (q * G::NW + wave) * 64 + lane, row = p / G::A_CPR, c = (p % G::A_CPR) ^ (row % 16);
        a_goff[q] = (row0 + row) * k * G::XB + k0 * G::XB + c * 16;
    }
#pragma unroll
    for (int q = 0; q < G::B_INSTR; ++q) {
        const uint32_t p = (q * G::NW + wave) * 64 + lane, row = p / 4, c = (p % 4) ^ ((row >> 2) & 3);
        b_goff[q] = (col0 + row) * (k / 2) + k0 / 2 + c * 16;
    }
    const uint32_t s_row = wave * G::S_ROWS + lane;
    const uint32_t s_goff = (col0 + s_row) * (k / 32) + k0 / 32;

    auto issue = [&](uint32_t st, uint32_t slot) {
        uint8_t* base = lds + slot * G::STAGE;
#pragma unroll
        for (int q = 0; q < G::A_INSTR; ++q)
            load_lds16(xr, (lds_ptr)(base + (q * G::NW + wave) * 1024), a_goff[q] + st * kBK * G::XB);
#pragma unroll
        for (int q = 0; q < G::B_INSTR; ++q)
            load_lds16(pr, (lds_ptr)(base + G::A_BYTES + (q * G::NW + wave) * 1024), b_goff[q] + st * (kBK / 2));
        // the wave's S_ROWS scale words; lanes past them stay inactive, so they
        // write nothing into the next wave's words (the instruction still
        // counts once in vmcnt: lane 0 is always active)
        if (lane < (uint32_t)G::S_ROWS)
            load_lds4(sr, (lds_ptr)(base + G::A_BYTES + G::B_BYTES + wave * G::S_ROWS * 4), s_goff + st * (kBK / 32));
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    auto compute = [&](uint32_t slot) {
        const uint8_t* base = lds + slot * G::STAGE;
        u32x4 wq[TN][2];
        uint32_t sw[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t r = (wn * TN + j) * 32 + r32, f = (r >> 2) & 3;
            const uint8_t* bp = base + G::A_BYTES + r * 64;
            wq[j][0] = *reinterpret_cast<const u32x4*>(bp + ((2 * h) ^ f) * 16);
            wq[j][1] = *reinterpret_cast<const u32x4*>(bp + ((2 * h + 1) ^ f) * 16);
            sw[j] = *reinterpret_cast<const uint32_t*>(base + G::A_BYTES + G::B_BYTES + r * 4);
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            bf16x8 b[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                // elements [64h + 8s, +8) lie in block 2h + s / 4 of the stage
                const uint32_t sb = (sw[j] >> (8 * (2 * h + s / 4))) & 0xffu;
                b[j] = decode8(wq[j][s / 4][s % 4], __uint_as_float(sb << 23));
            }
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const uint32_t r = (wm * TM + i) * 32 + r32, sw16 = r % 16;
                const uint8_t* ap = base + r * (G::A_CPR * 16);
                if constexpr (XBF16) {
                    const uint32_t c = (8 * h + s) ^ sw16;
                    const bf16x8 a = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(ap + c * 16));
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b[j], acc[i][j], 0, 0, 0);
                } else {
                    const uint32_t c0 = (16 * h + 2 * s) ^ sw16, c1 = (16 * h + 2 * s + 1) ^ sw16;
                    const f32x4 v0 = __builtin_bit_cast(f32x4, *reinterpret_cast<const u32x4*>(ap + c0 * 16));
                    const f32x4 v1 = __builtin_bit_cast(f32x4, *reinterpret_cast<const u32x4*>(ap + c1 * 16));
                    bf16x8 hi, mid, lo;
                    split3x8(v0, v1, hi, mid, lo);
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hi, b[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(mid, b[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo, b[j], acc[i][j], 0, 0, 0);
                    }
                }
            }
        }
    };

    // D-stage ring: stages st + 1 .. st + D - 2 stay in flight while stage st
    // is computed; stage st + D - 1 is issued into the slot stage st - 1 used,
    // after the barrier that ends every wave's reads of it
#pragma unroll
    for (int p = 0; p < D - 1; ++p)
        if ((uint32_t)p < stages) issue(p, p);
    for (uint32_t st = 0; st < stages; ++st) {
        const uint32_t ahead = stages - 1 - st;  // stages issued after st, at most D - 2
        if (ahead >= (uint32_t)(D - 2)) wait_vm<(D - 2) * G::LPS>();
        else if (D > 3 && ahead == 1) wait_vm<(D > 3 ? 1 : 0) * G::LPS>();
        else wait_vm<0>();
        lds_barrier();
        if (st + D - 1 < stages) issue(st + D - 1, (st + D - 1) % D);
        compute(st % D);
    }
    mfma_drain();

    // D[i][j] of a 32x32 tile: lane l holds column l % 32 and, in register r,
    // row 8 (r / 4) + 4 (l / 32) + r % 4
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t col = col0 + (wn * TN + j) * 32 + r32;
            if (col >= n) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = row0 + (wm * TM + i) * 32 + 8 * (r / 4) + 4 * h + r % 4;
                if (row < m) y[(size_t)row * n + col] = acc[i][j][r];
            }
        }
}

// y = sum over the slices of part[s] (count floats each), in slice order.
__global__ __launch_bounds__(256) void split_sum_kernel(const float* __restrict__ part, uint32_t ks, uint32_t count,
                                                        float* __restrict__ y) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (count % 4 == 0) {
        if (4 * i >= count) return;
        f32x4 a = *reinterpret_cast<const f32x4*>(part + 4 * i);
        for (uint32_t s = 1; s < ks; ++s) a += *reinterpret_cast<const f32x4*>(part + (size_t)s * count + 4 * i);
        *reinterpret_cast<f32x4*>(y + 4 * i) = a;
    } else {
        if (i >= count) return;
        float a = part[i];
        for (uint32_t s = 1; s < ks; ++s) a += part[(size_t)s * count + i];
        y[i] = a;
    }
}

template <bool XBF16, int WM, int WN, int TM, int TN>
hipError_t go(const GemvArgs& a, uint32_t ks, float* part) {
    // deepest ring that fits: 3 stages of a 128 x 128 bf16 tile (121.5 KiB)
    constexpr int D3 = Geometry<XBF16, WM, WN, TM, TN, 2>::STAGE * 3 <= 160 * 1024 ? 3 : 2;
    constexpr int D = (Geometry<XBF16, WM, WN, TM, TN, 2>::STAGE * 4 <= 160 * 1024 &&
                       2 * Geometry<XBF16, WM, WN, TM, TN, 2>::LPS <= 63) ? 4 : D3;
    using G = Geometry<XBF16, WM, WN, TM, TN, D>;
    const uint32_t tiles_m = (a.m + G::BM - 1) / G::BM;
    if (a.group) {
        // each weight of the group a run of column tiles; no K split
        if (ks > 1) return hipErrorNotSupported;
        GemmSegs sg{};
        uint32_t tiles_n = 0;
        sg.count = a.group->count;
        for (uint32_t s = 0; s < sg.count; ++s) {
            sg.packed[s] = a.group->packed[s];
            sg.scales[s] = a.group->scales[s];
            sg.y[s] = a.group->y[s];
            sg.n[s] = a.group->n[s];
            sg.tile0[s] = tiles_n;
            tiles_n += (sg.n[s] + G::BN - 1) / G::BN;
        }
        const uint32_t tiles = tiles_n * tiles_m;
        hipLaunchKernelGGL((gemm_exact_kernel<XBF16, WM, WN, TM, TN, D, GemmSegs>), dim3(tiles), dim3(G::NT), 0,
                           a.stream, nullptr, nullptr, a.x, nullptr, a.m, 0u, a.k, tiles_n, tiles, a.k, nullptr, sg);
        return hipGetLastError();
    }
    const uint32_t tiles_n = (a.n + G::BN - 1) / G::BN;
    const uint32_t tiles = tiles_n * tiles_m;
    if (ks < 1) ks = 1;
    hipLaunchKernelGGL((gemm_exact_kernel<XBF16, WM, WN, TM, TN, D>), dim3(tiles * ks), dim3(G::NT), 0, a.stream,
                       a.packed, a.scales, a.x, a.y, a.m, a.n, a.k, tiles_n, tiles, a.k / ks, ks > 1 ? part : nullptr,
                       NoGemmSegs{});
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || ks == 1) return e;
    const uint32_t count = a.m * a.n, threads = count % 4 == 0 ? count / 4 : count;
    hipLaunchKernelGGL(split_sum_kernel, dim3((threads + 255) / 256), dim3(256), 0, a.stream, part, ks, count, a.y);
    return hipGetLastError();
}

template <bool XBF16>
hipError_t dispatch(const GemvArgs& a, const GemmConfig& c, float* part) {
    // instances: (waves along M x along N, MFMA tiles per wave along M x N)
    const uint32_t ks = c.ks < 1 ? 1u : (uint32_t)c.ks;
    if (c.wm == 2 && c.wn == 2 && c.tm == 2 && c.tn == 3) return go<XBF16, 2, 2, 2, 3>(a, ks, part);
    if (c.wm == 2 && c.wn == 2 && c.tm == 2 && c.tn == 2) return go<XBF16, 2, 2, 2, 2>(a, ks, part);
    if (c.wm == 2 && c.wn == 2 && c.tm == 2 && c.tn == 1) return go<XBF16, 2, 2, 2, 1>(a, ks, part);
    if (c.wm == 2 && c.wn == 2 && c.tm == 1 && c.tn == 2) return go<XBF16, 2, 2, 1, 2>(a, ks, part);
    if (c.wm == 4 && c.wn == 1 && c.tm == 1 && c.tn == 2) return go<XBF16, 4, 1, 1, 2>(a, ks, part);
    if (c.wm == 2 && c.wn == 2 && c.tm == 1 && c.tn == 1) return go<XBF16, 2, 2, 1, 1>(a, ks, part);
    if (c.wm == 1 && c.wn == 4 && c.tm == 2 && c.tn == 2) return go<XBF16, 1, 4, 2, 2>(a, ks, part);
    if (c.wm == 1 && c.wn == 4 && c.tm == 2 && c.tn == 1) return go<XBF16, 1, 4, 2, 1>(a, ks, part);
    if (c.wm == 1 && c.wn == 4 && c.tm == 1 && c.tn == 2) return go<XBF16, 1, 4, 1, 2>(a, ks, part);
    if (c.wm == 1 && c.wn == 4 && c.tm == 1 && c.tn == 1) return go<XBF16, 1, 4, 1, 1>(a, ks, part);
    // a 128 x 256 tile of f32 activations would leave room for one stage only
    if constexpr (XBF16)
        if (c.wm == 2 && c.wn == 4 && c.tm == 2 && c.tn == 2) return go<XBF16, 2, 4, 2, 2>(a, ks, part);
    if (c.wm == 2 && c.wn == 4 && c.tm == 1 && c.tn == 2) return go<XBF16, 2, 4, 1, 2>(a, ks, part);
    return hipErrorNotSupported;
}

}  // namespace

bool gemm_exact_supported(uint32_t m, uint32_t n, uint32_t k, bool x_bf16) {
    // 32-bit buffer offsets over x and the packed weights
    const uint64_t xb = (uint64_t)m * k * (x_bf16 ? 2 : 4);
    return m >= 1 && n >= 1 && k % kBK == 0 && k >= kBK && xb + 256 * k * 4 < (1ull << 31) &&
           (uint64_t)(n + 256) * (k / 2) < (1ull << 31);
}

// The few-token-row K split (a grid short of the CUs) takes at most 4 MiB of
// partials, the range its picks were measured in.
constexpr uint64_t kFewRowsSplitBytes = 4ull << 20;

hipError_t launch_gemm_exact(const GemvArgs& a, int cus, const GemmConfig* forced, float* part, uint64_t part_bytes) {
    if (a.group) {
        // a group: every weight supported, no explicit configuration
        if (forced && forced->wm) return hipErrorNotSupported;
        if (a.group->count < 1 || a.group->count > 4) return hipErrorNotSupported;
        for (uint32_t s = 0; s < a.group->count; ++s)
            if (!gemm_exact_supported(a.m, a.group->n[s], a.k, a.x_bf16)) return hipErrorNotSupported;
    } else if (!gemm_exact_supported(a.m, a.n, a.k, a.x_bf16)) {
        return hipErrorNotSupported;
    }
    // column tiles of width bn over the weight (or over each weight of a group)
    auto col_tiles = [&](uint32_t bn) -> uint64_t {
        if (!a.group) return (a.n + bn - 1) / bn;
        uint64_t t = 0;
        for (uint32_t s = 0; s < a.group->count; ++s) t += (a.group->n[s] + bn - 1) / bn;
        return t;
    };
    GemmConfig c;
    if (forced && forced->wm) {
        c = *forced;
        // an explicit K split: whole stages per slice and partials within the scratch
        if (c.ks > 1 && (a.k % ((uint32_t)c.ks * kBK) != 0 || !part ||
                         (uint64_t)c.ks * a.m * a.n * 4 > part_bytes))
            return hipErrorNotSupported;
    } else {
        // The tile with the least estimated time: whole rounds of workgroups
        // (one per CU) times the time one round of that tile takes. The round
        // times (µs at K = 4096, bf16 x) are from a sweep of every instance on
        // the Qwen3-8B q, gate and down weights at M = 64..2048 on MI355X
        // (cold weights); with them the pick was the fastest instance, or
        // within 2% of it, at every M of the sweep: gate at M = 384 / 768 /
        // 1536 128 x 192 (47 / 90 / 145 us, where the largest tile whose grid
        // reaches three quarters of the CUs takes 64 / 102 / 157 us), at 2048
        // 128 x 256 (176 us); q and down at M = 512 64 x 128 (23 / 64 us).
        // The larger tiles re-read fewer operand bytes per flop, the smaller
        // ones leave fewer CUs idle in the last round.
        struct Cand { int wm, wn, tm, tn, bm, bn; double round_us; };
        const Cand cands[] = {{2, 4, 2, 2, 128, 256, 50.0}, {2, 2, 2, 3, 128, 192, 46.0},
                              {1, 4, 2, 2, 64, 256, 33.5},  {2, 2, 2, 2, 128, 128, 34.5},
                              {1, 4, 2, 1, 64, 128, 22.0},  {2, 2, 1, 1, 64, 64, 16.5}};
        const uint64_t nc = (uint64_t)(cus > 0 ? cus : 256);
        const uint64_t want = nc * 3 / 4;
        const Cand* best = nullptr;
        double best_t = 0.0;
        for (const Cand& cd : cands) {
            if (!a.x_bf16 && cd.wn == 4 && cd.wm == 2) continue;  // no f32 instance of 128 x 256
            const uint64_t tiles = (uint64_t)((a.m + cd.bm - 1) / cd.bm) * col_tiles(cd.bn);
            const double t = (double)((tiles + nc - 1) / nc) * cd.round_us;
            if (!best || t < best_t) {
                best = &cd;
                best_t = t;
            }
        }
        // f32 activations, and bf16 ones on wide K (K >= 8192): the largest
        // tile whose workgroups, with K cut into 1-4 slices of whole stages,
        // make one round of at least three quarters of the CUs (the most
        // workgroups among equal tiles). Measured on the 8B q / gate / down
        // weights at 64..1024 rows (cold): f32 q at 256 / 512 rows 63.9 /
        // 113.0 -> 44.2 / 75.8 us, gate at 128 / 256 113.3 / 131.7 -> 53.2 /
        // 90.9, down at 256 / 512 184 / 329 -> 107 / 201; bf16 down at 384 /
        // 512 / 1024 60.7 / 66.0 / 101.7 -> 47.5 / 54.1 / 93.3. bf16 at K =
        // 4096 keeps the round-time pick (its splits measured slower there).
        if (!a.x_bf16 || a.k >= 8192) {
            const Cand* sel = nullptr;
            uint32_t sel_ks = 0;
            uint64_t sel_area = 0, sel_wgs = 0;
            for (const Cand& cd : cands) {
                if (!a.x_bf16 && cd.wn == 4 && cd.wm == 2) continue;
                const uint64_t tiles = (uint64_t)((a.m + cd.bm - 1) / cd.bm) * col_tiles(cd.bn);
                for (uint32_t ks = 1; ks <= 4; ++ks) {
                    if (a.k % (ks * kBK) != 0) continue;
                    if (ks > 1 && (a.group || !part || (uint64_t)ks * a.m * a.n * 4 > part_bytes)) continue;
                    const uint64_t wgs = tiles * ks, area = (uint64_t)cd.bm * cd.bn;
                    if (wgs > nc || wgs < want) continue;
                    if (!sel || area > sel_area || (area == sel_area && wgs > sel_wgs)) {
                        sel = &cd;
                        sel_ks = ks;
                        sel_area = area;
                        sel_wgs = wgs;
                    }
                }
            }
            if (sel) {
                c.wm = sel->wm; c.wn = sel->wn; c.tm = sel->tm; c.tn = sel->tn;
                c.ks = (int)sel_ks;
                if (a.group) return a.x_bf16 ? dispatch<true>(a, c, nullptr) : dispatch<false>(a, c, nullptr);
                return a.x_bf16 ? dispatch<true>(a, c, part) : dispatch<false>(a, c, part);
            }
        }
        const Cand pick = *best;
        c.wm = pick.wm; c.wn = pick.wn; c.tm = pick.tm; c.tn = pick.tn;
        // A grid still short of the CUs (few token rows): split K across up to
        // four workgroups per tile, each slice whole stages, when the partials
        // fit the scratch; a second small kernel adds them in slice order.
        const uint64_t tiles = (uint64_t)((a.m + pick.bm - 1) / pick.bm) * col_tiles(pick.bn);
        c.ks = 1;
        // a group runs unsplit even when its tiles leave CUs idle: one round
        // of them beats its weights' separate launches, split or not (8B
        // q|k|v at 64 token rows: 96 tiles)
        if (a.group) return a.x_bf16 ? dispatch<true>(a, c, nullptr) : dispatch<false>(a, c, nullptr);
        for (uint32_t ks = 4; ks >= 2 && tiles < want; --ks) {
            if (a.k % (ks * kBK) == 0 && part && (uint64_t)ks * a.m * a.n * 4 <= kFewRowsSplitBytes) {
                c.ks = (int)ks;
                break;
            }
        }
    }
    return a.x_bf16 ? dispatch<true>(a, c, part) : dispatch<false>(a, c, part);
}

}  // namespace mx4
