// skinny.hip -- exact skinny kernel for a few tokens (speculative verify,
// 2 <= M <= 32): y[m, r] = sum_k x[m, k] * w(r, k) on bf16 matrix cores.
//
// The reference runs these shapes on project_rows{4,8,12}_mxfp4
// (engine/src/gpu.metal:277-322, dispatch engine/src/gpu.rs:484-509): FP32
// FMA, one weight read per chunk of 4/8/12 tokens. On gfx950 a VALU dot2 per
// token would be VALU-bound from M = 4 on, so the multiply-accumulate moves to
// V_MFMA_F32_16X16X32_BF16 while the weights stay 4-bit in HBM:
//  * each lane converts its 16 packed bytes (one MX block of one weight row)
//    with the hardware E2M1 converter, the E8M0 scale folded in -- exact in
//    bf16 for scale bytes 2..252, which the dispatcher guarantees;
//  * MFMA operand B is 16 weight rows x 32 K, operand A 16 tokens x 32 K.
//    Within a 128-element K chunk, lane group g (= lane / 16) holds block
//    4c + g and MFMA t takes elements [8t, 8t + 8) of it, for A and B alike;
//    the contraction is over K, so any K order shared by A and B is exact;
//  * bf16 activations are exact operands. f32 activations are split into
//    three bf16 terms hi + mid + lo (24 significant bits), three MFMAs each;
//  * a persistent workgroup of TW waves splits K (unit p of wave w is the U
//    adjacent chunks from (p TW + w) U on, so a wave reads whole 128-byte
//    lines of each row; its activation fragments stay in registers for the
//    whole kernel), walks 16-row weight tiles with the next ones prefetched,
//    and reduces its TW partial tiles through LDS;
//  * loads go through buffer resources: token rows >= M and weight rows >= N
//    read as zeros without touching memory;
//  * split K (KS > 1, rows too wide for a workgroup's activations to stay
//    resident): KS workgroups share a tile, each over one K slice with its
//    slice's activations resident, and the last of them to finish adds the KS
//    partial tiles in slice order;
//  * up to 16 bf16 tokens at K = 12288 (XLM, NP): the activations are loaded
//    into LDS by the workgroup -- all of K up to 5 tokens, one K half or
//    third at a time above -- and each unit's operand fragments read from
//    there, instead of every unit loading its 16-token fragments from the L2.
#include <type_traits>

#include "mx4_device.h"
#include "mx4_kernels.h"

namespace mx4 {

namespace {


constexpr int kNT = 2;  // streamed once: do not keep in the caches

// Eight bf16 weights: elements [8t, 8t + 8) of a lane's block (dword t of
// its 16 packed bytes), scale folded into the converter.
__device__ __forceinline__ bf16x8 weights8(uint32_t word, float sc) {
    bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 0);
    bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 1);
    bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 2);
    bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 3);
    bf16x8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// The 4U scale bytes of a unit's U adjacent chunks in one row, one load per
// lane (the four lanes of a row read the same bytes): byte 4q + g of the run
// is lane group g's block of chunk q.
template <int U>
__device__ __forceinline__ void load_scale_run(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t (&out)[U]) {
    if constexpr (U == 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
    } else if constexpr (U == 3) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, off, 0, 0);
        out[0] = v[0]; out[1] = v[1]; out[2] = v[2];
    } else if constexpr (U == 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        out[0] = v[0]; out[1] = v[1];
    } else {
        static_assert(U == 1, "1 to 4 chunks per unit");
        out[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    }
}

// Wait states after an MFMA chain whose accumulators are read next. The
// compiler can place a v_accvgpr_read of an XDL result right after a branch
// without the wait states the result needs (seen with ROCm 7.2 on gfx950: the
// last two MFMAs of a chain were lost), so the chain is drained explicitly;
// 24 wait states cover the longest 16x16 XDL op.
__device__ __forceinline__ void mfma_drain() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    __builtin_amdgcn_sched_barrier(0);
}

// f32 -> three bf16 terms with x = hi + mid + lo exactly (split3_bf16:
// non-finite values stay in hi).
__device__ __forceinline__ void split3(const f32x4 a, const f32x4 b, bf16x8& hi, bf16x8& mid, bf16x8& lo) {
    const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        __bf16 h, m, l;
        split3_bf16(v[e], h, m, l);
        hi[e] = h;
        mid[e] = m;
        lo[e] = l;
    }
}

// Persistent kernel, K = 128 * U * NU * TW * KS exactly. Workgroup b covers
// K slice b % KS (128 U NU TW elements); unit p of its wave w is the U
// adjacent 128-element chunks from (p TW + w) U on within the slice, in every
// weight row. The workgroup walks 16-row weight tiles (tile, tile +
// grid, ...); each tile is NU units per wave. A unit's weights (16 rows x U
// blocks per lane group), scales and activation fragments are loaded one unit
// ahead of the MFMAs, or, with one unit per tile, two tiles ahead. After a
// tile's last unit the TW partial 16x16 tiles are summed through LDS
// (double-buffered: one barrier per tile).
// The weights of a launch. One weight (OneTiles, built in the kernel from its
// leading scalar arguments, which arrive preloaded in SGPRs: a by-value
// struct argument would end the preloaded run), or up to four of one width
// sharing x (TileSegs, the trailing argument: weight s owns the 16-row tiles
// [first[s], first[s + 1]) of the launch; q|k|v or gate|up of a few-token
// verify step in one launch; NoTiles stands there for one weight). A tile's
// weight is picked with uniform selects, as in the GEMV.
struct NoTiles {};
struct TileSeg {
    const uint8_t* packed;
    const uint8_t* scales;
    float* y;
    uint32_t n, first;
};
struct OneTiles {
    const uint8_t* packed;
    const uint8_t* scales;
    float* y;
    uint32_t n;
};
struct TileSegs {
    const uint8_t* packed[4];
    const uint8_t* scales[4];
    float* y[4];
    uint32_t n[4];
    uint32_t first[4];
    uint32_t count;
};
__device__ __forceinline__ TileSeg pick_tiles(const OneTiles& o, uint32_t) {
    return TileSeg{o.packed, o.scales, o.y, o.n, 0u};
}
__device__ __forceinline__ TileSeg pick_tiles(const TileSegs& sg, uint32_t tile) {
    TileSeg s{sg.packed[0], sg.scales[0], sg.y[0], sg.n[0], 0u};
#pragma unroll
    for (int q = 1; q < 4; ++q) {
        const bool in = q < (int)sg.count && tile >= sg.first[q];
        s.packed = in ? sg.packed[q] : s.packed;
        s.scales = in ? sg.scales[q] : s.scales;
        s.y = in ? sg.y[q] : s.y;
        s.n = in ? sg.n[q] : s.n;
        s.first = in ? sg.first[q] : s.first;
    }
    return s;
}

template <bool XBF16, int MT, int U, int NU, int TW, bool RESX, int KS, int XLM = 0, int NP = 1, class SG = NoTiles>
__global__ __launch_bounds__(64 * TW) void skinny_kernel(const uint8_t* __restrict__ packed,
                                                         const uint8_t* __restrict__ scales,
                                                         const void* __restrict__ x, float* __restrict__ y,
                                                         uint32_t m, uint32_t n, uint32_t tiles,
                                                         float* __restrict__ part, uint32_t* __restrict__ count,
                                                         const SG group) {
    const auto sg = [&]() {
        if constexpr (std::is_same_v<SG, TileSegs>) return group;
        else return OneTiles{packed, scales, y, n};
    }();
    constexpr uint32_t ks = 128 * U * NU * TW;  // K of one slice
    constexpr uint32_t k = ks * KS;
    constexpr uint32_t row_bytes = k / 2, nblk = k / 32;
    constexpr int XQ = XBF16 ? 4 : 8;  // 16-byte activation loads per chunk and token tile
    // the wave index is uniform; saying so keeps chunk indices and buffer
    // resources in scalar registers (otherwise every load becomes a waterfall loop)
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t col = lane % 16, g = lane / 16;
    // the slice's first MX block in a row (KS divides the grid: uniform)
    const uint32_t slice = KS > 1 ? blockIdx.x % KS : 0u;
    const uint32_t kb = slice * (ks / 32);
    const __amdgpu_buffer_rsrc_t empty = rsrc(x, 0);
    const __amdgpu_buffer_rsrc_t xr = rsrc(x, m * k * (XBF16 ? 2u : 4u));
    // XLM > 0 (bf16 x, m <= XLM, rows too wide for registers): the token rows
    // live in LDS, XS bytes apart (16 bytes of padding put the 16 token rows
    // of an operand read in different bank groups), and each unit's
    // activation fragments are read from there instead of from the L2 -- a
    // unit's global loads are then its weights and scales only. With NP > 1
    // passes LDS holds one K slice of them at a time (units s NU / NP to
    // (s + 1) NU / NP cover slice s), loaded by the whole workgroup between
    // two barriers when its first unit comes up.
    static_assert(NP == 1 || (XLM > 0 && KS == 1 && NU % NP == 0), "passes over K slices need whole units");
    constexpr uint32_t KP = k / NP;  // K elements of one pass
    constexpr uint32_t XS = KP * 2 + 16;
    constexpr int UPP = NU / NP;     // units per pass
    __shared__ __attribute__((aligned(16))) uint8_t xl[XLM > 0 ? XLM * XS : 16];
    // The slice goes in by direct-to-LDS loads, one 1 KiB piece of a token
    // row per wave instruction, all in flight at once; the wave then waits
    // for its own (the caller's barrier follows). Through registers, each
    // thread's load had to land before its LDS write, one memory latency per
    // 16 bytes.
    static_assert(XLM == 0 || (KP * 2) % 1024 == 0, "a pass's row slice is whole 1 KiB pieces");
    auto fill = [&](uint32_t pass) {
        constexpr uint32_t ppr = KP * 2 / 1024;  // pieces per row
        const uint32_t pieces = (m < (uint32_t)XLM ? m : (uint32_t)XLM) * ppr;
        for (uint32_t pc = wave; pc < pieces; pc += TW) {
            const uint32_t r = pc / ppr, o = pc % ppr;
            load_lds16(xr, (lds_ptr)(xl + r * XS + 1024 * o), r * k * 2 + pass * KP * 2 + 1024 * o + 16 * lane);
        }
        wait_vm<0>();
    };
    if constexpr (XLM > 0) {
        static_assert(XBF16 && MT == 1 && !RESX, "LDS-resident activations: bf16, one token tile");
        fill(0);
        __syncthreads();
    }
    struct Unit {
        u32x4 w[U];
        uint32_t s[U];  // scale-byte runs: chunk q's byte for lane group g is byte g of s[q]
        u32x4 xa[RESX ? 1 : MT][RESX ? 1 : U][RESX ? 1 : XQ];
    };
    // RESX: a wave's K chunks are the same for every tile, so its activation
    // fragments for all of them are loaded once, here, instead of with every
    // tile's weights (for the lm_head that halves the bytes the kernel reads).
    // A chunk of a token tile is 16 token rows x 256 bytes (4 MX blocks of
    // bf16). The MFMA wants lane (col, g) to hold row col's block g as four
    // 16-byte pieces; loaded that way, every instruction touches 64 cache
    // lines for 16 bytes each. Instead instruction c loads rows 4c .. 4c + 3
    // whole (lane l: row 4c + l / 16, piece l % 16, 8 full lines per
    // instruction), and settle_x() moves each chunk into the MFMA layout
    // through the wave's own 4 KiB of LDS, after the first tiles' weight
    // loads are out (so only these loads are waited for). Slot 16 t + (s ^ t)
    // holds piece s of row t: the writes and the reads of any 8 consecutive
    // lanes fall in 8 different 16-byte bank groups.
    static_assert(!RESX || XBF16, "resident activations are bf16");
    u32x4 xres[RESX ? NU : 1][RESX ? U : 1][RESX ? MT : 1][RESX ? XQ : 1];
    __shared__ u32x4 xt[RESX ? TW : 1][RESX ? 256 : 1];
    if constexpr (RESX) {
#pragma unroll
        for (int p = 0; p < NU; ++p)
#pragma unroll
            for (int q = 0; q < U; ++q) {
                const uint32_t b0 = kb + 4 * ((p * TW + wave) * U + q);  // the chunk's first block
#pragma unroll
                for (int j = 0; j < MT; ++j)
#pragma unroll
                    for (int c = 0; c < XQ; ++c) {
                        const uint32_t off = ((16 * j + 4 * c + lane / 16) * k + 32 * b0) * 2 + 16 * (lane % 16);
                        xres[p][q][j][c] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
                    }
            }
    }
    auto settle_x = [&]() {
        if constexpr (RESX) {
#pragma unroll
            for (int p = 0; p < NU; ++p)
#pragma unroll
                for (int q = 0; q < U; ++q)
#pragma unroll
                    for (int j = 0; j < MT; ++j) {
#pragma unroll
                        for (int c = 0; c < XQ; ++c) {
                            const uint32_t t = 4 * c + lane / 16;
                            xt[wave][16 * t + ((lane % 16) ^ t)] = xres[p][q][j][c];
                        }
#pragma unroll
                        for (int c = 0; c < XQ; ++c) xres[p][q][j][c] = xt[wave][16 * col + ((4 * g + c) ^ col)];
                    }
        }
    };
    // TRANS (two or four chunks per unit): a unit's 16 rows x 64U bytes are
    // loaded as 16/U rows per instruction, 64U contiguous bytes each (whole
    // cache lines instead of one half line per row: half the memory requests),
    // then passed through the wave's own LDS stage into the MFMA layout. Load i
    // holds rows (16/U) i + j, block b of the unit at lane (4U) j + b. Its stage
    // slot is swizzled so that the writes and the reads of any 8 consecutive
    // lanes fall in 8 different 16-byte bank groups:
    //   U = 4: 64 i + 16 j + (b + 2 j + (i & 1)) % 16
    //   U = 2: 64 i + 8 j + (b + (j & ~1)) % 8
    constexpr bool TRANS = U == 2 || U == 4;
    constexpr uint32_t RPL = 16 / U, BPR = 4 * U;  // rows per load, blocks per row of a unit
    __shared__ u32x4 stage[TRANS ? TW : 1][TRANS ? 64 * U : 1];
    auto swz = [](uint32_t i, uint32_t j, uint32_t b) -> uint32_t {
        if constexpr (U == 4) return 64 * i + 16 * j + ((b + 2 * j + (i & 1)) & 15);
        else return 64 * i + 8 * j + ((b + (j & ~1u)) & 7);
    };
    // chunk q of unit `unit`: its activation fragments from the LDS slice
    // now loaded (the unit lies in slice unit / UPP)
    auto read_xq = [&](uint32_t unit, int q, Unit& out) {
        // token rows >= m: zeros, the address in row 0 (the dispatcher keeps m <= XLM)
        const bool live = col < m;
        const uint32_t blk = kb + 4 * ((unit * TW + wave) * U + q) + g - (NP > 1 ? (unit / UPP) * (KP / 32) : 0u);
        const uint8_t* src = xl + (live ? col : 0u) * XS + 64 * blk;
#pragma unroll
        for (int c = 0; c < XQ; ++c) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(src + 16 * c);
            out.xa[0][q][c] = live ? v : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto read_x = [&](uint32_t unit, Unit& out) {
#pragma unroll
        for (int q = 0; q < U; ++q) read_xq(unit, q, out);
    };
    auto load = [&](uint32_t tile, uint32_t unit, Unit& out, bool xnow = true) {
        const bool valid = tile < tiles;
        const TileSeg sw = pick_tiles(sg, tile);
        const uint32_t row0 = valid ? (tile - sw.first) * 16 : 0;
        const uint32_t rows = valid ? (sw.n - row0 < 16u ? sw.n - row0 : 16u) : 0;
        const __amdgpu_buffer_rsrc_t wr = valid ? rsrc(sw.packed + (size_t)row0 * row_bytes, rows * row_bytes) : empty;
        const __amdgpu_buffer_rsrc_t sr = valid ? rsrc(sw.scales + (size_t)row0 * nblk, rows * nblk) : empty;
        const __amdgpu_buffer_rsrc_t xq = valid ? xr : empty;
        load_scale_run<U>(sr, col * nblk + kb + 4 * (unit * TW + wave) * U, out.s);
        const uint32_t span = 16 * kb + 64 * (unit * TW + wave) * U;  // the unit's first byte in a row
#pragma unroll
        for (int q = 0; q < U; ++q) {
            const uint32_t blk = kb + 4 * ((unit * TW + wave) * U + q) + g;
            if constexpr (TRANS)
                out.w[q] = __builtin_amdgcn_raw_buffer_load_b128(wr, (RPL * q + lane / BPR) * row_bytes + span + 16 * (lane % BPR),
                                                                 0, kNT);
            else
                out.w[q] = __builtin_amdgcn_raw_buffer_load_b128(wr, col * row_bytes + 16 * blk, 0, kNT);
            if constexpr (RESX) continue;
            if constexpr (XLM > 0 && NP == 1) {
                // token row col of the operand; rows >= m are zeros (the
                // address stays in row 0, the value is not used)
                const bool live = col < m;
                const uint8_t* src = xl + (live ? col : 0u) * XS + 64 * blk;
#pragma unroll
                for (int c = 0; c < XQ; ++c) {
                    const u32x4 v = *reinterpret_cast<const u32x4*>(src + 16 * c);
                    out.xa[0][q][c] = live ? v : u32x4{0u, 0u, 0u, 0u};
                }
                continue;
            }
            if constexpr (XLM > 0) {
                if (xnow) read_xq(unit, q, out);
                continue;
            }
#pragma unroll
            for (int j = 0; j < MT; ++j) {
                const uint32_t off = ((16 * j + col) * k + 32 * blk) * (XBF16 ? 2u : 4u);
#pragma unroll
                for (int c = 0; c < XQ; ++c) out.xa[j][q][c] = __builtin_amdgcn_raw_buffer_load_b128(xq, off + 16 * c, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    f32x4 acc[MT];
    auto zero = [&]() {
#pragma unroll
        for (int j = 0; j < MT; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    };
    // unit `p` (compile-time) of the current tile
    auto compute = [&](const Unit& cur, int p) {
        auto xa = [&](int j, int q, int c) -> u32x4 {
            if constexpr (RESX) return xres[p][q][j][c];
            else return cur.xa[j][q][c];
        };
        u32x4 wq[U];
        if constexpr (TRANS) {
#pragma unroll
            for (int i = 0; i < U; ++i) stage[wave][swz(i, lane / BPR, lane % BPR)] = cur.w[i];
#pragma unroll
            for (int q = 0; q < U; ++q) wq[q] = stage[wave][swz(col / RPL, col % RPL, 4 * q + g)];
        } else {
#pragma unroll
            for (int q = 0; q < U; ++q) wq[q] = cur.w[q];
        }
#pragma unroll
        for (int q = 0; q < U; ++q) {
            const float sc = __uint_as_float(((cur.s[q] >> (8 * g)) & 0xffu) << 23);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bf16x8 b = weights8(wq[q][t], sc);
#pragma unroll
                for (int j = 0; j < MT; ++j) {
                    if constexpr (XBF16) {
                        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xa(j, q, t)), b, acc[j], 0, 0, 0);
                    } else {
                        bf16x8 hi, mid, lo;
                        split3(__builtin_bit_cast(f32x4, xa(j, q, 2 * t)), __builtin_bit_cast(f32x4, xa(j, q, 2 * t + 1)),
                               hi, mid, lo);
                        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, b, acc[j], 0, 0, 0);
                        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mid, b, acc[j], 0, 0, 0);
                        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, b, acc[j], 0, 0, 0);
                    }
                }
            }
        }
        mfma_drain();
    };

    // The hand-over of the waves' sums alternates between two buffers, so a
    // fast wave's next tile cannot overwrite sums a slow one still reads. With
    // K slices (NP > 1) every tile after the first opens with a workgroup
    // barrier before its first slice, after every wave's reads of the last
    // tile's sums: one buffer serves, and the 8 KiB it frees lets 16 tokens
    // run in thirds of K.
    constexpr uint32_t RB = NP > 1 ? 1 : 2;
    __shared__ f32x4 red[RB][TW][MT][64];
    uint32_t parity = 0;
    // Split K: partials are stored and loaded with device scope (SC1), so
    // they are not kept in the per-XCD L2s; the fences below order them.
    constexpr int kDeviceScope = 0x10;
    auto write_y = [&](uint32_t tile, uint32_t j, const f32x4& sum) {
        const TileSeg sw = pick_tiles(sg, tile);
        const uint32_t row = (tile - sw.first) * 16 + col;
        if (row < sw.n) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t tok = 16 * j + 4 * g + r;
                if (tok < m) sw.y[(size_t)tok * sw.n + row] = sum[r];
            }
        }
    };
    auto reduce_write = [&](uint32_t tile) {
#pragma unroll
        for (int j = 0; j < MT; ++j) red[parity][wave][j][lane] = acc[j];
        __syncthreads();
        if constexpr (KS > 1) {
            // wave 0 stores the slice's partial tile, part[tile][slice][j];
            // the tiles are counted after the tile loop
            if (wave == 0) {
                const __amdgpu_buffer_rsrc_t pr = rsrc(part + (size_t)tile * KS * MT * 256, KS * MT * 1024);
#pragma unroll
                for (int j = 0; j < MT; ++j) {
                    f32x4 sum = red[parity][0][j][lane];
#pragma unroll
                    for (int w = 1; w < TW; ++w) sum += red[parity][w][j][lane];
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sum), pr,
                                                           ((slice * MT + j) * 64 + lane) * 16, 0, kDeviceScope);
                }
            }
            parity = (parity + 1) % RB;
            zero();
            return;
        }
        // The tile's 256 MT sums, spread over 4 MT waves (a single wave
        // summing the whole tile kept the other seven waiting at the next
        // barrier): wave (j, g) owns the 16 rows x 4 tokens of lane group g
        // of token tile j, lane (col, r) = (lane / 4, lane % 4) one of them,
        // added over the waves in wave order as before, so the same bits.
        // The reads are consecutive floats of the hand-over; each store
        // instruction writes four 64-byte runs of rows.
        const float* rf = reinterpret_cast<const float*>(&red[parity][0][0][0]);
        for (uint32_t v = wave; v < 4u * MT; v += TW) {
            const uint32_t j = v / 4, gg = v % 4, c = lane / 4, r = lane % 4;
            const uint32_t at = (j * 64 + 16 * gg + c) * 4 + r;  // float index within one wave's hand-over
            float sum = rf[at];
#pragma unroll
            for (int w = 1; w < TW; ++w) sum += rf[w * MT * 256 + at];
            const TileSeg sw = pick_tiles(sg, tile);
            const uint32_t row = (tile - sw.first) * 16 + c, tok = 16 * j + 4 * gg + r;
            if (row < sw.n && tok < m) sw.y[(size_t)tok * sw.n + row] = sum;
        }
        parity = (parity + 1) % RB;
        zero();
    };

    // The units of a tile are unrolled (their index, and so their activation
    // fragments, known at compile time); each unit's weights are loaded while
    // the previous one computes, the next tile's first unit during the last.
    uint32_t tile = blockIdx.x / KS;
    if (tile >= tiles) return;
    zero();
    const uint32_t stride = gridDim.x / KS;  // tiles past the end load zeros and use nothing
    if constexpr (RESX && NU == 1) {
        // A tile is one unit: the next D - 1 tiles' weights are in flight
        // while one computes (D buffers, rotated by unrolling). The compiler's
        // wait counts are exact inside the unrolled body but conservative at
        // the loop head, where it waits for all but the newest tile; two
        // rounds of D steps per loop turn make that one step in 2 D.
        constexpr int D = 3;
        Unit u[D];
#pragma unroll
        for (int d = 0; d + 1 < D; ++d) load(tile + d * stride, 0, u[d]);
        settle_x();
        auto step = [&](uint32_t cur, auto slot) {
            constexpr int S = decltype(slot)::value % D;
            load(cur + (D - 1) * stride, 0, u[(S + D - 1) % D]);
            compute(u[S], 0);
            reduce_write(cur);
        };
        auto turn = [&](auto first) -> bool {
            constexpr int F = decltype(first)::value;
            step(tile, std::integral_constant<int, F + 0>{});
            if ((tile += stride) >= tiles) return true;
            step(tile, std::integral_constant<int, F + 1>{});
            if ((tile += stride) >= tiles) return true;
            if constexpr (D >= 3) {
                step(tile, std::integral_constant<int, F + 2>{});
                if ((tile += stride) >= tiles) return true;
            }
            if constexpr (D >= 4) {
                step(tile, std::integral_constant<int, F + 3>{});
                if ((tile += stride) >= tiles) return true;
            }
            return false;
        };
        for (;;) {
            if (turn(std::integral_constant<int, 0>{})) break;
            if (turn(std::integral_constant<int, D>{})) break;
        }
    } else {
        // Units ping-pong through two buffers, unit p of a tile in u[p % 2]
        // (NU is even or 1 only with the ring above).
        static_assert(NU % 2 == 0, "an odd unit count needs the copy-free rotation");
        Unit u[2];
        load(tile, 0, u[0]);
        settle_x();
        if constexpr (NP == 1) {
            for (;;) {
                const uint32_t next = tile + stride;
#pragma unroll
                for (int p = 0; p < NU; ++p) {
                    if (p + 1 < NU)
                        load(tile, (uint32_t)(p + 1), u[(p + 1) % 2]);
                    else
                        load(next, 0, u[(p + 1) % 2]);
                    compute(u[p % 2], p);
                }
                reduce_write(tile);
                if (next >= tiles) break;
                tile = next;
            }
        } else {
        bool first = true;
        for (;;) {
            const uint32_t next = tile + stride;
#pragma unroll
            for (int p = 0; p < NU; ++p) {
                if constexpr (NP > 1) {
                    // the first unit of a pass after the first: its slice
                    // replaces the previous one once every wave is done with it
                    if (p % UPP == 0 && (p > 0 || !first)) {
                        __syncthreads();
                        fill((uint32_t)(p / UPP));
                        __syncthreads();
                        read_x((uint32_t)p, u[p % 2]);
                    }
                }
                // the next unit's activations wait for its slice when it opens a pass
                const bool xnow = NP == 1 || (p + 1) % UPP != 0;
                if (p + 1 < NU)
                    load(tile, (uint32_t)(p + 1), u[(p + 1) % 2], xnow);
                else
                    load(next, 0, u[(p + 1) % 2], xnow);
                compute(u[p % 2], p);
            }
            reduce_write(tile);
            first = false;
            if (next >= tiles) break;
            tile = next;
        }
        }
    }
    if constexpr (KS > 1) {
        // Wave 0 counts its tiles once, after its last partial store (one
        // release per workgroup, not per tile). Lane i counts the workgroup's
        // i-th tile; the last of a tile's KS workgroups to count it reads the
        // KS partials, adds them in slice order, writes y and re-arms the
        // count for the next launch. No wave waits for another workgroup.
        //
        // Ordering (HIP memory model, agent scope): the release fence makes
        // this wave's partial stores visible device-wide before its counts
        // increment; a wave that reads KS - 1 from a count runs an acquire
        // fence before it loads the partials, so it sees every slice's
        // stores. Only a workgroup that finishes some tile pays the acquire
        // (on gfx950 it invalidates this XCD's L2; the release writes back
        // the L2's dirty lines): together about 2 us per launch.
        if (wave != 0) return;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const uint32_t first = blockIdx.x / KS;
        const uint32_t mine = (tiles - first + stride - 1) / stride;  // <= 64, checked at launch
        uint32_t before = 0;
        if (lane < mine)
            before = __hip_atomic_fetch_add(count + first + lane * stride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t last = __ballot(lane < mine && before == KS - 1);
        if (last != 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        for (uint32_t i = 0; i < mine; ++i) {
            if (!((last >> i) & 1)) continue;
            const uint32_t t = first + i * stride;
            const __amdgpu_buffer_rsrc_t pr = rsrc(part + (size_t)t * KS * MT * 256, KS * MT * 1024);
            u32x4 v[KS][MT];
#pragma unroll
            for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
                for (int j = 0; j < MT; ++j)
                    v[s2][j] = __builtin_amdgcn_raw_buffer_load_b128(pr, ((s2 * MT + j) * 64 + lane) * 16, 0, kDeviceScope);
#pragma unroll
            for (int j = 0; j < MT; ++j) {
                f32x4 sum = __builtin_bit_cast(f32x4, v[0][j]);
#pragma unroll
                for (int s2 = 1; s2 < KS; ++s2) sum += __builtin_bit_cast(f32x4, v[s2][j]);
                write_y(t, j, sum);
            }
            if (lane == 0) __hip_atomic_store(count + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// 16-row tiles of a launch: one weight's, or those of every weight of a group
// (each weight starts a tile of its own).
uint32_t tiles_of(const GemvArgs& a) {
    if (!a.group) return (a.n + 15) / 16;
    uint32_t t = 0;
    for (uint32_t s = 0; s < a.group->count; ++s) t += (a.group->n[s] + 15) / 16;
    return t;
}

template <bool XBF16, int MT, int U, int NU, int TW, bool RESX, int KS = 1, int XLM = 0, int NP = 1>
hipError_t go(const GemvArgs& a, int cus, const SkinnyScratch& sc = {}) {
    const uint32_t tiles = tiles_of(a);
    // two workgroups of TW waves per CU; with one unit per tile, eight waves
    // per CU (two per SIMD: the three buffers need more than the 128 VGPRs of
    // four waves per SIMD). With split K, one workgroup per CU and KS of them
    // per tile: consecutive workgroups take the KS slices of one tile, so each
    // XCD (every eighth workgroup) keeps one slice of the activations in its L2.
    uint32_t grid = KS > 1 ? (uint32_t)cus / KS : (uint32_t)cus * ((RESX && NU == 1) ? 8u / TW : 2u);
    if (grid > tiles) grid = tiles;
    if (grid == 0) grid = 1;
    const uint32_t per = (tiles + grid - 1) / grid;
    grid = (tiles + per - 1) / per;
    if (a.group) {
        TileSegs sg{};
        sg.count = a.group->count;
        for (uint32_t s = 0, t = 0; s < sg.count; ++s) {
            sg.packed[s] = a.group->packed[s];
            sg.scales[s] = a.group->scales[s];
            sg.y[s] = a.group->y[s];
            sg.n[s] = a.group->n[s];
            sg.first[s] = t;
            t += (sg.n[s] + 15) / 16;
        }
        hipLaunchKernelGGL((skinny_kernel<XBF16, MT, U, NU, TW, RESX, KS, XLM, NP, TileSegs>), dim3(grid * KS),
                           dim3(64 * TW), 0, a.stream, nullptr, nullptr, a.x, nullptr, a.m, 0u, tiles, sc.part,
                           sc.count, sg);
    } else {
        hipLaunchKernelGGL((skinny_kernel<XBF16, MT, U, NU, TW, RESX, KS, XLM, NP, NoTiles>), dim3(grid * KS),
                           dim3(64 * TW), 0, a.stream, a.packed, a.scales, a.x, a.y, a.m, a.n, tiles, sc.part,
                           sc.count, NoTiles{});
    }
    return hipGetLastError();
}

// Split K needs KS * MT partial tiles and one count per 16-row tile, and
// counts a workgroup's tiles with one lane each (at most 64 tiles per
// workgroup; the launch puts cus / KS workgroups on each slice).
bool split_fits(const GemvArgs& a, int cus, const SkinnyScratch& sc, uint32_t ks, uint32_t mt) {
    const uint64_t tiles = tiles_of(a);
    uint64_t grid = (uint64_t)cus / ks;
    if (grid > tiles) grid = tiles;
    if (grid == 0) grid = 1;
    return sc.part && sc.count && tiles * ks * mt <= sc.part_tiles && tiles <= sc.count_tiles &&
           (tiles + grid - 1) / grid <= 64;
}

// The three-tile ring (bf16 activations, K 2048 or 4096) pays from two tiles
// per workgroup at eight waves per CU (K = 2048 runs 4-wave workgroups).
bool tile_ring(const GemvArgs& a, int cus) {
    const uint32_t tiles = tiles_of(a);
    const uint32_t waves = (uint32_t)(cus > 0 ? cus : 256) * 8u;
    const uint32_t tw = a.k == 2048 ? 4u : 8u;
    return a.x_bf16 && (a.k == 2048 || a.k == 4096) && tiles >= 2 * waves / tw;
}

// Chunks per unit: two for bf16 activations and one token tile, one otherwise,
// so that two units (the one computed and the one in flight) fit the registers.
// With resident activations and at least two tiles per workgroup of the ring
// launch (8 waves per CU), a tile is one unit and three tiles stream through
// the ring: gate/up at 8 tokens 14.3 -> 10.4 us, lm_head 91 -> 86 us. Weights
// with fewer tiles (each workgroup one tile or two) keep two units per tile,
// which measured 0.3-0.8 us faster there.
template <bool XBF16, int MT>
hipError_t go_k(const GemvArgs& a, int cus, const SkinnyScratch& sc) {
    constexpr int U = (XBF16 && MT == 1) ? 2 : 1;
    constexpr int TW = 8;
    // bf16 activations of up to 16 tokens stay resident in registers for K up
    // to 6144 (at most 6 chunks per wave: 96 VGPRs)
    constexpr bool R = XBF16 && MT == 1;
    const bool ring = R && tile_ring(a, cus);
    switch (a.k) {
        case 2048:
            if constexpr (R) if (ring) return go<XBF16, MT, 4, 1, 4, R>(a, cus);
            return go<XBF16, MT, U, 16 / (U * 4), 4, R>(a, cus);
        case 4096:
            if constexpr (R) if (ring) return go<XBF16, MT, 4, 1, TW, R>(a, cus);
            // 17-32 bf16 tokens: split K, four ways (4-wave workgroups) when
            // that gives each CU one tile, two chunks per wave, activations
            // resident: 8B k at 32 tokens 11.7 -> 9.1 us (6.5 us before the
            // agent-scope fences of the arrival count, which cost about 2 us
            // per launch). Two ways (8 waves) from 20 tokens on only for the
            // ring-length weights that launch_skinny sends here (gate/up): on
            // q/o the fenced split measured slower than unsplit (12.9 against
            // 12.0 us at 32 tokens).
            if constexpr (XBF16 && MT == 2) {
                if (4 * tiles_of(a) <= (uint32_t)cus && split_fits(a, cus, sc, 4, MT))
                    return go<XBF16, MT, 2, 1, 4, true, 4>(a, cus, sc);
                if (a.m >= 20 && tile_ring(a, cus) && split_fits(a, cus, sc, 2, MT))
                    return go<XBF16, MT, 2, 1, 8, true, 2>(a, cus, sc);
            }
            return go<XBF16, MT, U, 4 / U, TW, R>(a, cus);
        case 6144:  // (a one-unit tile of 6 chunks would spill)
            return go<XBF16, MT, R ? 3 : U, R ? 2 : 6 / U, TW, R>(a, cus);
        // wider rows keep the per-tile activation loads: resident in registers
        // they need 16 or 12 waves per workgroup and measured slower (down)
        case 8192: return go<XBF16, MT, U, 8 / U, TW, false>(a, cus);
        case 12288:
            // bf16 activations of one token tile (up to 16 tokens) in LDS
            // beside the kernel's 32 KiB of stage and reduction buffers (24
            // KiB with K slices: one reduction buffer): all of K up to 5
            // tokens (5 x 24 KiB), one K half at a time up to 10, one third up
            // to 16 (sixths at 16 with two reduction buffers: 11.2 -> 10.1
            // us in thirds). 8B down at 3 / 4 / 5
            // tokens 10.0 / 10.3 / 10.3 -> 7.7-8.0 / 8.0-8.3 / 8.3-8.7 us, at
            // 6 / 8 / 10 / 11 tokens 11.0 / 12.4 / 13.2 / 13.8 -> 9.4 / 10.2 /
            // 10.9 / 11.6 us against the per-unit activation loads, and at 12
            // / 14 / 16 tokens 14.3 / 14.2 / 14.5 -> 12.4 / 13.0 / 13.8 us
            // against the split-K form (repetitions on two machines).
            if constexpr (XBF16 && MT == 1) {
                if (a.m <= 5) return go<XBF16, 1, U, 12 / U, TW, false, 1, 5>(a, cus);
                if (a.m <= 10) return go<XBF16, 1, U, 12 / U, TW, false, 1, 10, 2>(a, cus);
                return go<XBF16, 1, U, 12 / U, TW, false, 1, 16, 3>(a, cus);
            }
            // bf16 x, two token tiles (17-32 tokens): four workgroups per
            // tile, each over a 3072-wide K slice with its activations resident
            // and the three-tile ring, so that every workgroup reads a quarter
            // of x instead of all of it (6 waves of four chunks; 8B down at 32
            // tokens 32.7 -> 18.6 us with the agent-scope fences of the
            // arrival count, about 2 us per launch; three-chunk units, with
            // half-line loads, measured 0.8-1.4 us slower)
            if constexpr (XBF16 && MT == 2)
                if (split_fits(a, cus, sc, 4, MT)) return go<XBF16, MT, 4, 1, 6, true, 4>(a, cus, sc);
            return go<XBF16, MT, U, 12 / U, TW, false>(a, cus);
        default: return hipErrorNotSupported;
    }
}

}  // namespace

bool skinny_supported(uint32_t m, uint32_t k) {
    // the Qwen3 widths; M within two 16-token tiles
    const bool kk = k == 2048 || k == 4096 || k == 6144 || k == 8192 || k == 12288;
    return m >= 1 && m <= 32 && kk;
}

// More than 16 tokens on weights long enough for the tile ring run as two
// launches of 16 and m - 16 token rows: the one-token-tile kernel keeps its
// activations resident and streams through the ring, which two token tiles
// per launch cannot afford in registers (lm_head at 17-32 tokens: 256-357 us
// in one launch, 115-125 in two; gate 29-40 -> 18-20 us). Shorter weights
// measured faster in one launch with two token tiles. From 20 tokens on at
// K = 4096, one split-K launch beats the two where its partials fit (8B gate
// at 20 / 32 tokens: 18.3 / 20.2 -> 16.1 / 16.9 us).
hipError_t launch_skinny(const GemvArgs& a, int cus, const SkinnyScratch& sc) {
    if (!skinny_supported(a.m, a.k)) return hipErrorNotSupported;
    if (a.group) {
        if (a.group->count < 1 || a.group->count > 4) return hipErrorNotSupported;
        for (uint32_t s = 0; s < a.group->count; ++s)
            if (a.group->n[s] == 0) return hipErrorNotSupported;
    }
    auto one = [&](const GemvArgs& b) { return b.x_bf16 ? go_k<true, 1>(b, cus, sc) : go_k<false, 1>(b, cus, sc); };
    if (a.m <= 16) return one(a);
    if (!tile_ring(a, cus)) return a.x_bf16 ? go_k<true, 2>(a, cus, sc) : go_k<false, 2>(a, cus, sc);
    // K = 4096 from 20 tokens on, when the partial tiles fit (8B gate/up, not
    // the lm_head): one two-way split-K launch reads the weights once
    if (a.x_bf16 && a.k == 4096 && a.m >= 20 && split_fits(a, cus, sc, 2, 2)) return go_k<true, 2>(a, cus, sc);
    GemvArgs lo = a, hi = a;
    lo.m = 16;
    hi.m = a.m - 16;
    hi.x = static_cast<const uint8_t*>(a.x) + (size_t)16 * a.k * (a.x_bf16 ? 2 : 4);
    hi.y = a.y + (size_t)16 * a.n;
    GemvGroup hg{};
    if (a.group) {
        // every weight's outputs from token row 16 on
        hg = *a.group;
        for (uint32_t s = 0; s < hg.count; ++s) hg.y[s] = a.group->y[s] + (size_t)16 * a.group->n[s];
        hi.group = &hg;
    }
    const hipError_t e = one(lo);
    return e != hipSuccess ? e : one(hi);
}

}  // namespace mx4
