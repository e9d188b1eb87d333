// gemv.hip -- exact MXFP4 x activation kernels for decode (M = 1) and the
// generic exact fallback (any M, any K % 32 == 0).
//
// Computes y[m, r] = sum_k x[m, k] * w(r, k), the product of
// engine/src/lib.rs:240-266, with w decoded from packed E2M1 + E8M0 per 32
// (engine/src/mxfp4.rs:27-33). Like the reference's fastest Metal kernel
// (project_token_blocks, engine/src/gpu.metal:324-356) the E8M0 scale is
// factored out of each 32-element block: the block's 32 products are summed
// with exact E2M1 levels, then multiplied once by 2^(s-127).
//
// gemv_m1 design (gfx950, HBM-bound):
//  * a team of WG waves owns R weight rows at a time; its 64*WG lanes split
//    each row's K/32 blocks, lane t taking blocks t + 64*WG*j (j < BPL), so
//    every 128-bit load instruction reads 1 KiB of contiguous packed bytes;
//  * the lane's activations for its BPL blocks are loaded once into VGPRs and
//    reused for every row the persistent team visits;
//  * the next row-set's loads are issued before the current one is reduced
//    (register double-buffering), keeping R*BPL KiB in flight per wave;
//  * E2M1 -> bf16/f32 by the hardware converter, bf16 dot2 (or f32 FMA)
//    accumulation, wave reduction through lane shuffles, cross-wave through LDS.
#include <type_traits>
#include "mx4_device.h"
#include "mx4_kernels.h"

namespace mx4 {

template <bool XBF16, int BPL>
struct LaneX;

template <int BPL>
struct LaneX<true, BPL> {
    uint32_t p[BPL][16];  // bf16 pairs, element order
    __device__ __forceinline__ void load(const void* xv, uint32_t blk0, uint32_t stride) {
        const uint8_t* x = static_cast<const uint8_t*>(xv);
#pragma unroll
        for (int j = 0; j < BPL; ++j) {
            const uint8_t* src = x + (size_t)(blk0 + j * stride) * 64;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                u32x4 v = load_u32x4(src + 16 * q);
                p[j][4 * q + 0] = v[0];
                p[j][4 * q + 1] = v[1];
                p[j][4 * q + 2] = v[2];
                p[j][4 * q + 3] = v[3];
            }
        }
    }
    // the same blocks from a copy of x staged in LDS
    __device__ __forceinline__ void load_lds(const uint8_t* xl, uint32_t blk0, uint32_t stride) {
#pragma unroll
        for (int j = 0; j < BPL; ++j) {
            const uint8_t* src = xl + (size_t)(blk0 + j * stride) * 64;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(src + 16 * q);
                p[j][4 * q + 0] = v[0];
                p[j][4 * q + 1] = v[1];
                p[j][4 * q + 2] = v[2];
                p[j][4 * q + 3] = v[3];
            }
        }
    }
    __device__ __forceinline__ float dot(int j, const u32x4 w) const { return block_dot_bf16(w, p[j]); }
};

template <int BPL>
struct LaneX<false, BPL> {
    float f[BPL][32];
    __device__ __forceinline__ void load(const void* xv, uint32_t blk0, uint32_t stride) {
        const float* x = static_cast<const float*>(xv);
#pragma unroll
        for (int j = 0; j < BPL; ++j) {
            const float* src = x + (size_t)(blk0 + j * stride) * 32;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                f32x4 v = *reinterpret_cast<const f32x4*>(src + 4 * q);
                f[j][4 * q + 0] = v[0];
                f[j][4 * q + 1] = v[1];
                f[j][4 * q + 2] = v[2];
                f[j][4 * q + 3] = v[3];
            }
        }
    }
    __device__ __forceinline__ void load_lds(const uint8_t* xl, uint32_t blk0, uint32_t stride) {
#pragma unroll
        for (int j = 0; j < BPL; ++j) {
            const float* src = reinterpret_cast<const float*>(xl) + (size_t)(blk0 + j * stride) * 32;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(src + 4 * q);
                f[j][4 * q + 0] = v[0];
                f[j][4 * q + 1] = v[1];
                f[j][4 * q + 2] = v[2];
                f[j][4 * q + 3] = v[3];
            }
        }
    }
    __device__ __forceinline__ float dot(int j, const u32x4 w) const { return block_dot_f32(w, f[j]); }
};

// Up to kMaxSegs weights of the same width K that share one activation row
// (q|k|v, gate|up) run as one launch: segment s owns rowsets
// [first[s], first[s+1]) of the flattened row space.
constexpr int kMaxSegs = 4;
struct Segs {
    const uint8_t* packed[kMaxSegs];
    const uint8_t* scales[kMaxSegs];
    float* y[kMaxSegs];
    uint32_t n[kMaxSegs];
    uint32_t first[kMaxSegs + 1];
    uint32_t count;
    uint32_t rowsets;  // first[count], passed directly so no argument load depends on another
    uint64_t* am_partial;  // greedy-argmax epilogue: one key per workgroup (unused otherwise)
};

// Sum R per-lane values over the 64 lanes of a wave in log2(64) exchange
// stages. In the first log2(R) stages each lane keeps half of its values and
// sends the other half to its partner, so the R totals cost 63 + R - 1
// additions instead of R * 63. The exchanges stay in the VALU: DPP
// row_half_mirror (partner l ^ 7), quad permutations (l ^ 1, l ^ 2) and
// row_ror:8 (l ^ 8) within rows of 16 lanes, then v_permlane16_swap (l ^ 16)
// and v_permlane32_swap (l ^ 32). The half-mirror stage goes first: it flips
// lane bits 0-2 together, which is a valid butterfly partner only while no
// earlier stage has made lanes differ in bits 0-1. The halving stages select
// by lane bits 2, 0, 1 in that order, so lane l ends with the total of row
// reduced_row_of_lane<R>(l).
template <int CTRL>
__device__ __forceinline__ float dpp_partner(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int CTRL, int R>
__device__ __forceinline__ void dpp_stage(float (&v)[R], int& n, bool upper) {
    if (n > 1) {
        const int half = n / 2;
#pragma unroll
        for (int i = 0; i < R / 2; ++i) {
            if (i < half) {
                const float send = upper ? v[i] : v[i + half];
                const float keep = upper ? v[i + half] : v[i];
                v[i] = keep + dpp_partner<CTRL>(send);
            }
        }
        n = half;
    } else {
        v[0] += dpp_partner<CTRL>(v[0]);
    }
}

// Exchange across rows (SWAP = 16) or half-waves (SWAP = 32). After
// permlane*_swap(a, b) lane l holds {own a, partner's a} if it is the lower
// partner and {partner's b, own b} if it is the upper one, so the sum of the
// pair is keep + partner's send in both cases.
template <int SWAP>
__device__ __forceinline__ float swap_sum(float lower_keeps, float upper_keeps) {
    const auto p = SWAP == 16
                       ? __builtin_amdgcn_permlane16_swap(__float_as_uint(lower_keeps), __float_as_uint(upper_keeps), false, false)
                       : __builtin_amdgcn_permlane32_swap(__float_as_uint(lower_keeps), __float_as_uint(upper_keeps), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

template <int SWAP, int R>
__device__ __forceinline__ void swap_stage(float (&v)[R], int& n) {
    if (n > 1) {
        const int half = n / 2;
#pragma unroll
        for (int i = 0; i < R / 2; ++i)
            if (i < half) v[i] = swap_sum<SWAP>(v[i], v[i + half]);
        n = half;
    } else {
        v[0] = swap_sum<SWAP>(v[0], v[0]);
    }
}

constexpr int kDppHalfMirror = 0x141, kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppRowRor8 = 0x128;

template <int R>
__device__ __forceinline__ float wave_reduce_rows(float (&v)[R], uint32_t lane) {
    int n = R;
    dpp_stage<kDppHalfMirror, R>(v, n, (lane & 4) != 0);
    dpp_stage<kDppQuadXor1, R>(v, n, (lane & 1) != 0);
    dpp_stage<kDppQuadXor2, R>(v, n, (lane & 2) != 0);
    dpp_stage<kDppRowRor8, R>(v, n, (lane & 8) != 0);
    swap_stage<16, R>(v, n);
    swap_stage<32, R>(v, n);
    return v[0];
}

// Row whose total lane `lane` holds after wave_reduce_rows<R> (R <= 8): the
// halving stages take the upper half when lane bit 2, then 0, then 1 is set.
template <int R>
__device__ __forceinline__ uint32_t reduced_row_of_lane(uint32_t lane) {
    static_assert(R == 1 || R == 2 || R == 4 || R == 8, "rows per team");
    uint32_t row = 0;
    if constexpr (R >= 2) row += (lane & 4) ? R / 2 : 0;
    if constexpr (R >= 4) row += (lane & 1) ? R / 4 : 0;
    if constexpr (R >= 8) row += (lane & 2) ? 1 : 0;
    return row;
}

// One lane per row writes its total: lane bits outside the row-select bits are zero.
template <int R>
__device__ __forceinline__ bool row_writer(uint32_t lane) {
    constexpr uint32_t row_bits = R >= 8 ? 7u : R == 4 ? 5u : R == 2 ? 4u : 0u;
    return (lane & ~row_bits) == 0;
}


constexpr int kNonTemporal = 2;  // streamed once per pass: do not keep in the caches

template <bool XBF16, int BPL, int R>
struct RowSet {
    u32x4 w[R][BPL];
    uint32_t s[R][BPL];
};

// One segment's fields, selected from the table with uniform conditional
// moves (a dynamic index into the by-value table would become scalar loads
// from the argument segment, with waits in the middle of the stream).
struct Seg {
    const uint8_t* packed;
    const uint8_t* scales;
    float* y;
    uint32_t n, first;
};

__device__ __forceinline__ Seg pick_seg(const Segs& sg, uint32_t rs) {
    Seg s{sg.packed[0], sg.scales[0], sg.y[0], sg.n[0], sg.first[0]};
#pragma unroll
    for (int q = 1; q < kMaxSegs; ++q) {
        const bool in = q < (int)sg.count && rs >= sg.first[q];
        s.packed = in ? sg.packed[q] : s.packed;
        s.scales = in ? sg.scales[q] : s.scales;
        s.y = in ? sg.y[q] : s.y;
        s.n = in ? sg.n[q] : s.n;
        s.first = in ? sg.first[q] : s.first;
    }
    return s;
}

// Issue the loads of one row-set. A row-set index past the end gets
// zero-sized buffer resources: its loads return zeros without touching memory,
// so the prefetch can be issued unconditionally. (A prefetch under a branch
// makes the compiler's wait-count merge fall back to waiting for every load,
// the prefetch included, which serialises streaming and compute.)
template <bool XBF16, int WG, int BPL, int R>
__device__ __forceinline__ void load_rowset_in(const Seg& sgm, uint32_t rs, uint32_t rowsets, uint32_t t,
                                               uint32_t row_bytes, uint32_t nblk, RowSet<XBF16, BPL, R>& out) {
    const bool valid = rs < rowsets;
    const uint32_t row0 = valid ? (rs - sgm.first) * R : 0;
    uint32_t rows = sgm.n - row0 < (uint32_t)R ? sgm.n - row0 : (uint32_t)R;
    rows = valid ? rows : 0;
    const __amdgpu_buffer_rsrc_t wr = rsrc(sgm.packed + (size_t)row0 * row_bytes, rows * row_bytes);
    const __amdgpu_buffer_rsrc_t sr = rsrc(sgm.scales + (size_t)row0 * nblk, rows * nblk);
#pragma unroll
    for (int i = 0; i < R; ++i) {
#pragma unroll
        for (int j = 0; j < BPL; ++j) {
            const uint32_t b = t + j * 64 * WG;
            out.w[i][j] = __builtin_amdgcn_raw_buffer_load_b128(wr, 16 * b, i * row_bytes, kNonTemporal);
            out.s[i][j] = __builtin_amdgcn_raw_buffer_load_b8(sr, b, i * nblk, 0);
        }
    }
    // keep the stream ahead of the arithmetic that follows
    __builtin_amdgcn_sched_barrier(0);
}

// One weight: the segment of a single-weight launch of the few-token GEMV,
// built in the kernel from its leading scalar arguments (which arrive
// preloaded in SGPRs, so the first weight load waits for no scalar memory
// round trip; a by-value struct argument ends the preloaded run). A group
// launch passes its table as the trailing argument; NoSegs stands there for
// one weight.
struct NoSegs {};
struct OneSeg {
    const uint8_t* packed;
    const uint8_t* scales;
    float* y;
    uint32_t n;
};

__device__ __forceinline__ Seg pick_seg(const OneSeg& o, uint32_t) { return Seg{o.packed, o.scales, o.y, o.n, 0u}; }

template <bool XBF16, int WG, int BPL, int R, class SG>
__device__ __forceinline__ void load_rowset(const SG& sg, uint32_t rs, uint32_t rowsets, uint32_t t,
                                            uint32_t row_bytes, uint32_t nblk, RowSet<XBF16, BPL, R>& out) {
    load_rowset_in<XBF16, WG, BPL, R>(pick_seg(sg, rs), rs, rowsets, t, row_bytes, nblk, out);
}

// Sum over one row's blocks owned by this lane. The E8M0 scale is folded into
// the hardware converter (level * 2^(s-127) is exact in bf16/f32 for scale
// bytes 2..254, which the dispatcher guarantees), so each 32-element block costs
// 16 conversions and 16 bf16 dot2 (or 32 f32 FMA) and one shift.
template <bool XBF16, int BPL>
__device__ __forceinline__ float row_dot(const LaneX<XBF16, BPL>& xr, const u32x4 (&w)[BPL], const uint32_t (&s)[BPL]) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
        const float sc = __uint_as_float(s[j] << 23);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            if constexpr (XBF16) {
                acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j][d], sc, 0),
                                                      as_bf16x2(xr.p[j][4 * d + 0]), acc, false);
                acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j][d], sc, 1),
                                                      as_bf16x2(xr.p[j][4 * d + 1]), acc, false);
                acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j][d], sc, 2),
                                                      as_bf16x2(xr.p[j][4 * d + 2]), acc, false);
                acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j][d], sc, 3),
                                                      as_bf16x2(xr.p[j][4 * d + 3]), acc, false);
            } else {
                f32x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[j][d], sc, 0);
                f32x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[j][d], sc, 1);
                f32x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[j][d], sc, 2);
                f32x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[j][d], sc, 3);
                acc = __builtin_fmaf(xr.f[j][8 * d + 0], v0.x, acc);
                acc = __builtin_fmaf(xr.f[j][8 * d + 1], v0.y, acc);
                acc = __builtin_fmaf(xr.f[j][8 * d + 2], v1.x, acc);
                acc = __builtin_fmaf(xr.f[j][8 * d + 3], v1.y, acc);
                acc = __builtin_fmaf(xr.f[j][8 * d + 4], v2.x, acc);
                acc = __builtin_fmaf(xr.f[j][8 * d + 5], v2.y, acc);
                acc = __builtin_fmaf(xr.f[j][8 * d + 6], v3.x, acc);
                acc = __builtin_fmaf(xr.f[j][8 * d + 7], v3.y, acc);
            }
        }
    }
    return acc;
}

template <bool XBF16, int WG, int BPL, int R, bool AM>
__device__ __forceinline__ void finish_rowset(const Segs& sg, uint32_t rs, const LaneX<XBF16, BPL>& xr,
                                              const RowSet<XBF16, BPL, R>& cur, uint32_t t,
                                              float (*red)[WG][R], uint32_t& parity, uint64_t& best) {
    const uint32_t wave = t / 64, lane = t % 64;
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = row_dot<XBF16, BPL>(xr, cur.w[i], cur.s[i]);
    const Seg sgm = pick_seg(sg, rs);
    const uint32_t row0 = (rs - sgm.first) * R;
    const uint32_t n = sgm.n;
    float* y = sgm.y;
    const float total = wave_reduce_rows<R>(acc, lane);
    const uint32_t myrow = reduced_row_of_lane<R>(lane);
    const bool writer = row_writer<R>(lane);
    if constexpr (WG == 1) {
        if (writer && row0 + myrow < n) {
            if constexpr (AM) {
                if (y) y[row0 + myrow] = total;
                best = max_u64(best, argmax_key(total, row0 + myrow));
            } else {
                y[row0 + myrow] = total;
            }
        }
    } else {
        if (writer) red[parity][wave][myrow] = total;
        __syncthreads();
        if (t < (uint32_t)R) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < WG; ++w) v += red[parity][w][t];
            if (row0 + t < n) {
                if constexpr (AM) {
                    if (y) y[row0 + t] = v;
                    best = max_u64(best, argmax_key(v, row0 + t));
                } else {
                    y[row0 + t] = v;
                }
            }
        }
        parity ^= 1;
    }
}

// A workgroup holds `tpw` independent teams of 64 WG threads. With more
// than one, x is staged once per workgroup in LDS and every team reads its
// blocks from there: each workgroup loads the whole activation row, so fewer,
// larger workgroups cut that L2 traffic (for o at K = 4096 it matched the
// weight bytes with one team per workgroup). Dynamic LDS: x (k elements), then
// the cross-wave partial sums [tpw][2][WG][R].
//
// HEAD0: the launcher guarantees every team's first row-set lies in segment 0
// (grid * tpw <= first[1]), so the first load needs only segment 0's weight
// and scale pointers and row count, taken from `early`; `late(early)` then
// supplies the whole table, fetched while that load is in flight.
struct AllEarly {
    __device__ const Segs& operator()(const Segs& early) const { return early; }
};

template <bool XBF16, int WG, int BPL, int R, bool AM, bool HEAD0 = false, class Late = AllEarly>
__device__ __forceinline__ void gemv_m1_body(const Segs& early, const void* __restrict__ x, uint32_t k, uint32_t tpw,
                                             uint32_t grid, Late late = {}) {
    constexpr uint32_t T = 64 * WG;  // threads per team
    const uint32_t team = __builtin_amdgcn_readfirstlane(threadIdx.x / T);
    const uint32_t t = threadIdx.x % T;
    const uint32_t row_bytes = k / 2;
    const uint32_t nblk = k / 32;
    const uint32_t rowsets = early.rowsets;
    const uint32_t stride = grid * tpw;
    const uint32_t first = blockIdx.x * tpw;  // the workgroup's first team visits the most row-sets
    uint32_t rs = first + team;               // the host launches at most `rowsets` teams per row-set turn

    // Every kernel argument is needed before the first load. Pinning them in
    // SGPRs here makes the compiler fetch them in one scalar round trip
    // (otherwise it splits the fetch and waits twice before the first weight
    // load); the weight stream is issued first, the activations right behind.
    RowSet<XBF16, BPL, R> a, b;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t xbytes = k * (XBF16 ? 2 : 4);
    // K = 64 WG BPL blocks of 32. When several teams share one LDS copy of x,
    // x is fetched first from K = 6144 on (12 KiB of bf16 x per workgroup)
    // and for one-row teams: its direct-to-LDS loads go out before the first
    // row-set's, so that waiting for them (loads return in order) does not
    // also wait for the weights, and the second row-set is issued once x is
    // in, not once the first one is (8B down 7.10 -> 6.43 us; q, o 3.62 ->
    // 3.52 us and k, v 2.54 -> 2.29 us with four one-row teams sharing x).
    // With two-row teams at K = 4096 (gate, gate|up, lm_head) the same order
    // measured 0.05-0.13 us slower, so there x follows the weights.
    constexpr bool XFIRST = WG * BPL >= 3 || R == 1;
    if (XFIRST && tpw > 1) {
        const __amdgpu_buffer_rsrc_t xres = rsrc(x, xbytes);
        const uint32_t lane = threadIdx.x % 64, wave0 = threadIdx.x - lane;
        for (uint32_t c0 = wave0; c0 < xbytes / 16; c0 += tpw * T)
            load_lds16(xres, (lds_ptr)(smem + 16 * c0), 16 * (c0 + lane));
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (HEAD0) {
        asm volatile("" ::"s"(early.packed[0]), "s"(early.scales[0]), "s"(early.n[0]), "s"(x), "s"(k), "s"(rowsets),
                     "s"(tpw));
        __builtin_amdgcn_sched_barrier(0);
        load_rowset_in<XBF16, WG, BPL, R>(Seg{early.packed[0], early.scales[0], nullptr, early.n[0], 0u}, rs, rowsets,
                                          t, row_bytes, nblk, a);
    } else {
#pragma unroll
        for (int q = 0; q < kMaxSegs; ++q)
            asm volatile("" ::"s"(early.packed[q]), "s"(early.scales[q]), "s"(early.y[q]), "s"(early.n[q]),
                         "s"(early.first[q]));
        asm volatile("" ::"s"(x), "s"(early.count), "s"(k), "s"(tpw));
        __builtin_amdgcn_sched_barrier(0);
        load_rowset<XBF16, WG, BPL, R>(early, rs, rowsets, t, row_bytes, nblk, a);
    }
    const Segs sg = late(early);
    LaneX<XBF16, BPL> xr;
    // the host sizes dynamic LDS as (tpw > 1 ? x : nothing) + tpw * 2 * WG * R floats
    float(*red)[WG][R] = reinterpret_cast<float(*)[WG][R]>(smem + (tpw > 1 ? xbytes : 0)) + 2 * team;
    if (tpw == 1) {
        xr.load(x, t, T);
    } else if constexpr (XFIRST) {
        // x's loads were issued before the first row-set's 2 R BPL loads
        wait_vm<2 * R * BPL>();
        __syncthreads();
        xr.load_lds(smem, t, T);
    } else {
        const uint8_t* xg = static_cast<const uint8_t*>(x);
        for (uint32_t c = threadIdx.x; c < xbytes / 16; c += tpw * T)
            *reinterpret_cast<u32x4*>(smem + 16 * c) = load_u32x4(xg + 16 * c);
        __syncthreads();
        xr.load_lds(smem, t, T);
    }

    uint32_t parity = 0;
    uint64_t best = 0;  // greedy-argmax key of the rows this thread finished
    // ping-pong: the next row-set streams in while the current one is reduced.
    // Every team of the workgroup runs as many turns as the first one (the
    // cross-wave reduction has a workgroup barrier); a team past the end
    // loads zeros and writes nothing.
    for (uint32_t rf = first;;) {
        uint32_t nxt = rs + stride;
        load_rowset<XBF16, WG, BPL, R>(sg, nxt, rowsets, t, row_bytes, nblk, b);
        finish_rowset<XBF16, WG, BPL, R, AM>(sg, rs, xr, a, t, red, parity, best);
        rf += stride;
        if (rf >= rowsets) break;
        rs = nxt;
        nxt = rs + stride;
        load_rowset<XBF16, WG, BPL, R>(sg, nxt, rowsets, t, row_bytes, nblk, a);
        finish_rowset<XBF16, WG, BPL, R, AM>(sg, rs, xr, b, t, red, parity, best);
        rf += stride;
        if (rf >= rowsets) break;
        rs = nxt;
    }
    if constexpr (AM) {
        // the workgroup's best key -> am_partial[blockIdx.x]
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const uint32_t lo = __shfl_xor((uint32_t)best, off, kWave), hi = __shfl_xor((uint32_t)(best >> 32), off, kWave);
            best = max_u64(best, ((uint64_t)hi << 32) | lo);
        }
        __shared__ uint64_t wbest[8];
        if (threadIdx.x % 64 == 0) wbest[threadIdx.x / 64] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t m = 0;
            for (uint32_t w = 0; w < tpw * WG; ++w) m = max_u64(m, wbest[w]);
            sg.am_partial[blockIdx.x] = m;
        }
    }
}

// The launchers pass the teams per workgroup (`tpw`) and the grid size as
// arguments: blockDim.x and gridDim.x are read from the dispatch's hidden
// arguments, the workgroup size by a vector load whose address depends on a
// scalar load, two memory round trips that would otherwise stand before the
// first weight load.
//
// A group of up to four weights (their table passed by value).
template <bool XBF16, int WG, int BPL, int R, bool AM>
__global__ __launch_bounds__(512) void gemv_m1_kernel(Segs sg, const void* __restrict__ x, uint32_t k, uint32_t tpw,
                                                      uint32_t grid) {
    gemv_m1_body<XBF16, WG, BPL, R, AM>(sg, x, k, tpw, grid);
}

// A group whose teams all start in segment 0: what the first load needs --
// segment 0's weight and scale pointers and row count, x, k, the row-set
// count and the launch shape -- comes first, as scalars that kernel argument
// preloading places in SGPRs; the by-value table behind them is read from the
// argument segment only for later row-sets and the stores.
//
// The table is read through the kernel argument segment pointer, laundered
// after the first load is issued: a by-value argument's loads are placed at
// kernel entry, where the compiler would wait for them (the register it
// reuses from an 8-dword fetch) before the first weight load. Explicit
// arguments are laid out in order at their natural alignment, as the members
// of HeadArgs are.
struct HeadArgs {
    const uint8_t* packed0;
    const uint8_t* scales0;
    const void* x;
    uint32_t n0, k, rowsets, tpw, grid;
    Segs tail;
};

using KernargSegs = const __attribute__((address_space(4))) Segs;

struct HeadTail {
    __device__ Segs operator()(const Segs& early) const {
        uint64_t kp = reinterpret_cast<uint64_t>(__builtin_amdgcn_kernarg_segment_ptr());
        asm volatile("" : "+s"(kp));
        KernargSegs* tail = reinterpret_cast<KernargSegs*>(kp + offsetof(HeadArgs, tail));
        Segs sg;
#pragma unroll
        for (int q = 0; q < kMaxSegs; ++q) {
            sg.packed[q] = tail->packed[q];
            sg.scales[q] = tail->scales[q];
            sg.y[q] = tail->y[q];
            sg.n[q] = tail->n[q];
            sg.first[q] = tail->first[q];
        }
        sg.first[kMaxSegs] = tail->first[kMaxSegs];
        sg.count = tail->count;
        sg.am_partial = nullptr;
        sg.packed[0] = early.packed[0];
        sg.scales[0] = early.scales[0];
        sg.n[0] = early.n[0];
        sg.rowsets = early.rowsets;
        return sg;
    }
};

template <bool XBF16, int WG, int BPL, int R>
__global__ __launch_bounds__(512) void gemv_m1_head_kernel(const uint8_t* __restrict__ packed0,
                                                           const uint8_t* __restrict__ scales0,
                                                           const void* __restrict__ x, uint32_t n0, uint32_t k,
                                                           uint32_t rowsets, uint32_t tpw, uint32_t grid, Segs tail) {
    (void)tail;  // read through the argument segment by HeadTail
    Segs early{};
    early.packed[0] = packed0;
    early.scales[0] = scales0;
    early.n[0] = n0;
    early.rowsets = rowsets;
    gemv_m1_body<XBF16, WG, BPL, R, false, true>(early, x, k, tpw, grid, HeadTail{});
}

// One weight, every argument a plain scalar: this file is built with kernel
// argument preloading, so on entry the ones the first loads need already sit
// in SGPRs and the first weight load issues without a memory round trip (a
// by-value table cannot be preloaded; y and am_partial, needed only at the
// first store, come last and may be fetched).
template <bool XBF16, int WG, int BPL, int R, bool AM>
__global__ __launch_bounds__(512) void gemv_m1_one_kernel(const uint8_t* __restrict__ packed,
                                                          const uint8_t* __restrict__ scales,
                                                          const void* __restrict__ x, uint32_t n, uint32_t k,
                                                          uint32_t rowsets, uint32_t tpw, uint32_t grid,
                                                          float* __restrict__ y, uint64_t* __restrict__ am_partial) {
    Segs sg;
#pragma unroll
    for (int q = 0; q < kMaxSegs; ++q) {
        sg.packed[q] = packed;
        sg.scales[q] = scales;
        sg.y[q] = y;
        sg.n[q] = n;
        sg.first[q + 1] = rowsets;
    }
    sg.first[0] = 0;
    sg.count = 1;
    sg.rowsets = rowsets;
    sg.am_partial = am_partial;
    gemv_m1_body<XBF16, WG, BPL, R, AM>(sg, x, k, tpw, grid);
}

// A few tokens (speculative verify, 2 <= m <= MT, bf16 activations): the
// M = 1 weight stream -- each lane's 16-byte blocks of R rows, 1 KiB contiguous
// per wave load instruction, the next row-set in flight while the current one
// is reduced -- with every converted weight pair multiplied into all MT token
// rows, so the weights are read once for all of them. A team (one workgroup)
// of WG waves splits each row's K; each lane keeps the x blocks of every token
// in registers (token slots >= m hold zeros and write nothing). The R * MT
// per-lane sums go through the same butterfly as the M = 1 kernel, then (for
// WG > 1) through LDS.
template <int BPL, int MT>
__device__ __forceinline__ void rows_dot_mt(const LaneX<true, BPL> (&xr)[MT], const u32x4 (&w)[BPL],
                                            const uint32_t (&s)[BPL], float* acc) {
#pragma unroll
    for (int tok = 0; tok < MT; ++tok) acc[tok] = 0.0f;
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
        const float sc = __uint_as_float(s[j] << 23);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const bf16x2 w0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j][d], sc, 0);
            const bf16x2 w1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j][d], sc, 1);
            const bf16x2 w2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j][d], sc, 2);
            const bf16x2 w3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j][d], sc, 3);
#pragma unroll
            for (int tok = 0; tok < MT; ++tok) {
                float a = acc[tok];
                a = __builtin_amdgcn_fdot2_f32_bf16(w0, as_bf16x2(xr[tok].p[j][4 * d + 0]), a, false);
                a = __builtin_amdgcn_fdot2_f32_bf16(w1, as_bf16x2(xr[tok].p[j][4 * d + 1]), a, false);
                a = __builtin_amdgcn_fdot2_f32_bf16(w2, as_bf16x2(xr[tok].p[j][4 * d + 2]), a, false);
                a = __builtin_amdgcn_fdot2_f32_bf16(w3, as_bf16x2(xr[tok].p[j][4 * d + 3]), a, false);
                acc[tok] = a;
            }
        }
    }
}

// SHARED: several teams per workgroup share one LDS copy of the token rows
// (tpw > 1); otherwise each team loads its own into registers (tpw == 1).
// SG: NoSegs (one weight: packed, scales, n, y) or Segs (a group: each
// weight a run of row-sets; packed, scales, n and y unused).
template <int WG, int BPL, int R, int MT, bool SHARED, class SG>
__global__ __launch_bounds__(512) void gemv_mt_kernel(const uint8_t* __restrict__ packed,
                                                      const uint8_t* __restrict__ scales,
                                                      const void* __restrict__ x, uint32_t m, uint32_t n,
                                                      uint32_t rowsets, uint32_t tpw, uint32_t grid,
                                                      float* __restrict__ y, const SG group) {
    const auto sg = [&]() {
        if constexpr (std::is_same_v<SG, Segs>) return group;
        else return OneSeg{packed, scales, y, n};
    }();
    constexpr int RM = R * MT;
    static_assert(RM == 2 || RM == 4 || RM == 8, "rows x tokens per team");
    constexpr uint32_t T = 64 * WG;
    constexpr uint32_t nblk = 64 * WG * BPL, k = 32 * nblk, row_bytes = k / 2, xbytes = MT * k * 2;
    const uint32_t team = __builtin_amdgcn_readfirstlane(threadIdx.x / T);
    const uint32_t t = threadIdx.x % T, lane = t % 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t / 64);
    const uint32_t stride = grid * tpw;
    const uint32_t first = blockIdx.x * tpw;  // the workgroup's first team visits the most row-sets
    uint32_t rs = first + team;
    RowSet<true, BPL, R> a, b;
    // Dynamic LDS: the MT token rows of x when several teams share the
    // workgroup (loaded once, then each lane copies its blocks to registers),
    // then the cross-wave partial sums [tpw][2][WG][RM].
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    if constexpr (SHARED) {
        // The token rows' direct-to-LDS loads go out before the first
        // row-set's, so that waiting for them (loads return in order) does not
        // also wait for the weights: the second row-set is issued once x is
        // in (8B down / gate at 2 tokens 8.5 / 7.8 -> 7.0 / 7.2 us). Token
        // rows >= m lie past the resource and read as zeros; xbytes / 16 is a
        // multiple of 64, so every turn of the loop is whole waves.
        const uint32_t live = (m < (uint32_t)MT ? m : (uint32_t)MT) * k * 2;
        const __amdgpu_buffer_rsrc_t xres = rsrc(x, live);
        const uint32_t wave0 = threadIdx.x - threadIdx.x % 64;
        for (uint32_t c0 = wave0; c0 < xbytes / 16; c0 += tpw * T)
            load_lds16(xres, (lds_ptr)(smem + 16 * c0), 16 * (c0 + lane));
        __builtin_amdgcn_sched_barrier(0);
    }
    load_rowset<true, WG, BPL, R>(sg, rs, rowsets, t, row_bytes, nblk, a);
    float(*red)[WG][RM] = reinterpret_cast<float(*)[WG][RM]>(smem + (tpw > 1 ? xbytes : 0)) + 2 * team;
    LaneX<true, BPL> xr[MT];
    const uint8_t* xb = static_cast<const uint8_t*>(x);
    if constexpr (SHARED) {
        // the first row-set's 2 R BPL loads were issued after x's
        wait_vm<2 * R * BPL>();
        __syncthreads();
#pragma unroll
        for (int tok = 0; tok < MT; ++tok) xr[tok].load_lds(smem + (size_t)tok * k * 2, t, T);
    } else if (tpw > 1) {
        // (the launcher sends shared copies to the SHARED instances)
        const uint32_t live = (m < (uint32_t)MT ? m : (uint32_t)MT) * k * 2;
        for (uint32_t c = threadIdx.x; c < xbytes / 16; c += tpw * T)
            *reinterpret_cast<u32x4*>(smem + 16 * c) = 16 * c < live ? load_u32x4(xb + 16 * c) : u32x4{0u, 0u, 0u, 0u};
        __syncthreads();
#pragma unroll
        for (int tok = 0; tok < MT; ++tok) xr[tok].load_lds(smem + (size_t)tok * k * 2, t, T);
    } else {
        // each team's own copy, behind the first row-set
#pragma unroll
        for (int tok = 0; tok < MT; ++tok) {
            if ((uint32_t)tok < m) {
                xr[tok].load(xb + (size_t)tok * k * 2, t, T);
            } else {
#pragma unroll
                for (int j = 0; j < BPL; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) xr[tok].p[j][e] = 0u;
            }
        }
    }
    uint32_t parity = 0;
    auto finish = [&](uint32_t set, const RowSet<true, BPL, R>& cur) {
        float acc[RM];
#pragma unroll
        for (int i = 0; i < R; ++i) rows_dot_mt<BPL, MT>(xr, cur.w[i], cur.s[i], acc + i * MT);
        // the row-set's weight; past its n for a team beyond the last
        // row-set, so nothing is written
        const Seg sgm = pick_seg(sg, set);
        const uint32_t row0 = (set - sgm.first) * R, n = sgm.n;
        float* const y = sgm.y;
        const float total = wave_reduce_rows<RM>(acc, lane);
        const uint32_t idx = reduced_row_of_lane<RM>(lane);
        if constexpr (WG == 1) {
            const uint32_t row = row0 + idx / MT, tok = idx % MT;
            if (row_writer<RM>(lane) && row < n && tok < m) y[(size_t)tok * n + row] = total;
        } else {
            if (row_writer<RM>(lane)) red[parity][wave][idx] = total;
            __syncthreads();
            if (t < (uint32_t)RM) {
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < WG; ++w) v += red[parity][w][t];
                const uint32_t row = row0 + t / MT, tok = t % MT;
                if (row < n && tok < m) y[(size_t)tok * n + row] = v;
            }
            parity ^= 1;
        }
    };
    // Every team of the workgroup runs as many turns as the first one (the
    // cross-wave reduction has a workgroup barrier); a team past the end loads
    // zeros and writes nothing.
    for (uint32_t rf = first;;) {
        uint32_t nxt = rs + stride;
        load_rowset<true, WG, BPL, R>(sg, nxt, rowsets, t, row_bytes, nblk, b);
        finish(rs, a);
        rf += stride;
        if (rf >= rowsets) break;
        rs = nxt;
        nxt = rs + stride;
        load_rowset<true, WG, BPL, R>(sg, nxt, rowsets, t, row_bytes, nblk, a);
        finish(rs, b);
        rf += stride;
        if (rf >= rowsets) break;
        rs = nxt;
    }
}

// Generic exact kernel: any M (tokens processed MT at a time), any K % 32 == 0,
// any scale byte. Every element is decoded exactly as engine/src/mxfp4.rs:27-33
// does (level * 2^(s-127): subnormal for small bytes, inf for large levels at
// bytes 253/254) and multiplied with its activation, so inf/NaN and subnormal
// weights behave like the reference's sequential loop; only the summation
// order differs. One wave per weight row; lanes stride over the row's blocks.
template <bool XBF16, int MT>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const uint8_t* __restrict__ packed,
                                                           const uint8_t* __restrict__ scales,
                                                           const void* __restrict__ xv,
                                                           float* __restrict__ y, uint32_t m,
                                                           uint32_t n, uint32_t k) {
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t row = blockIdx.x * 4 + threadIdx.x / 64;
    const uint32_t m0 = blockIdx.y * MT;
    if (row >= n) return;
    const uint32_t nblk = k / 32;
    const uint8_t* prow = packed + (size_t)row * (k / 2);
    const uint8_t* srow = scales + (size_t)row * nblk;
    float acc[MT];
#pragma unroll
    for (int q = 0; q < MT; ++q) acc[q] = 0.0f;
    for (uint32_t b = lane; b < nblk; b += 64) {
        const u32x4 w = load_u32x4(prow + 16 * (size_t)b);
        const float sc = e8m0_to_f32(srow[b]);
        float wv[32];
#pragma unroll
        for (int e = 0; e < 32; ++e) wv[e] = level_of((w[e / 8] >> (4 * (e % 8))) & 15u) * sc;
#pragma unroll
        for (int q = 0; q < MT; ++q) {
            const uint32_t tok = m0 + q < m ? m0 + q : m - 1;
            if constexpr (XBF16) {
                const uint8_t* src = static_cast<const uint8_t*>(xv) + ((size_t)tok * k + (size_t)b * 32) * 2;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const u32x4 v = load_u32x4(src + 16 * c);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        acc[q] = __builtin_fmaf(bf16_bits_to_f32(v[e] & 0xffffu), wv[8 * c + 2 * e], acc[q]);
                        acc[q] = __builtin_fmaf(bf16_bits_to_f32(v[e] >> 16), wv[8 * c + 2 * e + 1], acc[q]);
                    }
                }
            } else {
                const float* src = static_cast<const float*>(xv) + (size_t)tok * k + (size_t)b * 32;
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const f32x4 v = *reinterpret_cast<const f32x4*>(src + 4 * c);
                    acc[q] = __builtin_fmaf(v[0], wv[4 * c + 0], acc[q]);
                    acc[q] = __builtin_fmaf(v[1], wv[4 * c + 1], acc[q]);
                    acc[q] = __builtin_fmaf(v[2], wv[4 * c + 2], acc[q]);
                    acc[q] = __builtin_fmaf(v[3], wv[4 * c + 3], acc[q]);
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < MT; ++q) {
        const float v = wave_sum(acc[q]);
        if (lane == 0 && m0 + q < m) y[(size_t)(m0 + q) * n + row] = v;
    }
}

// ------------------------------------------------------------------ launchers

template <bool XBF16, int WG, int BPL, int R>
static hipError_t go_m1(const Segs& sg, const void* x, uint32_t k, uint32_t grid, int tpw, hipStream_t st) {
    const size_t lds = (tpw > 1 ? (size_t)k * (XBF16 ? 2 : 4) : 0) + (size_t)tpw * 2 * WG * R * sizeof(float);
    if (sg.count == 1)
        hipLaunchKernelGGL((gemv_m1_one_kernel<XBF16, WG, BPL, R, false>), dim3(grid), dim3(64 * WG * tpw), lds, st,
                           sg.packed[0], sg.scales[0], x, sg.n[0], k, sg.rowsets, (uint32_t)tpw, grid, sg.y[0],
                           (uint64_t*)nullptr);
    else if ((uint64_t)grid * tpw <= sg.first[1])
        hipLaunchKernelGGL((gemv_m1_head_kernel<XBF16, WG, BPL, R>), dim3(grid), dim3(64 * WG * tpw), lds, st,
                           sg.packed[0], sg.scales[0], x, sg.n[0], k, sg.rowsets, (uint32_t)tpw, grid, sg);
    else
        hipLaunchKernelGGL((gemv_m1_kernel<XBF16, WG, BPL, R, false>), dim3(grid), dim3(64 * WG * tpw), lds, st, sg,
                           x, k, (uint32_t)tpw, grid);
    return hipGetLastError();
}

// Rows per team allowed for a blocks-per-lane count: R * BPL <= 8 keeps the
// double-buffered weights within 64 VGPRs.
template <bool XBF16, int WG, int BPL>
static hipError_t go_r(const Segs& sg, const void* x, uint32_t k, uint32_t grid, int r, int tpw, hipStream_t st) {
    switch (r) {
        case 1: return go_m1<XBF16, WG, BPL, 1>(sg, x, k, grid, tpw, st);
        case 2: if constexpr (BPL <= 4) return go_m1<XBF16, WG, BPL, 2>(sg, x, k, grid, tpw, st); break;
        case 4: if constexpr (BPL <= 2) return go_m1<XBF16, WG, BPL, 4>(sg, x, k, grid, tpw, st); break;
        case 8: if constexpr (BPL <= 1) return go_m1<XBF16, WG, BPL, 8>(sg, x, k, grid, tpw, st); break;
        default: break;
    }
    return hipErrorNotSupported;
}

template <bool XBF16>
static hipError_t go_cfg(const Segs& sg, const void* x, uint32_t k, uint32_t grid, int wg, int bpl, int r, int tpw,
                         hipStream_t st) {
#define MX4_M1_CASE(W, B) \
    if (wg == W && bpl == B) return go_r<XBF16, W, B>(sg, x, k, grid, r, tpw, st);
    MX4_M1_CASE(1, 1) MX4_M1_CASE(1, 2) MX4_M1_CASE(2, 1) MX4_M1_CASE(1, 3) MX4_M1_CASE(3, 1)
    MX4_M1_CASE(1, 4) MX4_M1_CASE(2, 2) MX4_M1_CASE(4, 1) MX4_M1_CASE(1, 6) MX4_M1_CASE(2, 3)
    MX4_M1_CASE(3, 2) MX4_M1_CASE(6, 1)
#undef MX4_M1_CASE
    return hipErrorNotSupported;
}

bool gemv_m1_supported(uint32_t k) {
    const uint32_t nblk = k / 32;
    return k % 32 == 0 && (nblk == 64 || nblk == 128 || nblk == 192 || nblk == 256 || nblk == 384);
}

// Default configuration, from sweeps on MI355X over the launches of the Qwen3
// 1.7B and 8B decode steps (q|k|v and gate|up grouped, cold weights, recorded
// passes). One wave per team for K <= 4096 (1-2 blocks per lane), several
// teams per workgroup for the wide matrices (two-wave teams for the
// vocabulary-sized lm_head); for long K multi-wave teams and few workgroups,
// because every workgroup loads the whole activation row (24 KiB at K =
// 12288): at 12288 four 2-wave teams share one LDS copy of it. Grids are in
// teams per CU.
static void default_m1_config(uint32_t k, uint32_t rows, int cus, M1Config& c) {
    const uint32_t nblk = k / 32;
    const uint32_t scale = (uint32_t)(cus > 0 ? cus : 256);  // the table is for 256 CUs
    c.tpw = 1;
    switch (nblk) {
        case 64:  // K = 2048 (Qwen3-1.7B sweep: q|k|v 3.33 -> 3.14 us, gate|up 4.86 -> 4.71 us)
            c.wg = 1; c.r = 2; c.grid = (rows > 2048 && rows <= 4096 ? 4 : 12) * scale;
            // up to 2048 rows (o): eight one-row teams per workgroup sharing x,
            // fetched ahead of the weights (2.42 -> 2.22 us)
            if (rows <= 2048) { c.r = 1; c.grid = 8 * scale; c.tpw = 8; }
            if (rows > 4096 && rows <= 8192) c.r = 4;
            if (rows > 8192) c.grid = 16 * scale;
            if (rows > 65536) { c.r = 4; c.tpw = 8; c.grid = 8 * scale; }  // vocabulary-sized
            break;
        case 128:  // K = 4096
            c.wg = 1; c.r = 2; c.grid = (rows <= 8192 ? 4 : 16) * scale;
            // up to 8192 rows (q, o, k, v, q|k|v): four one-row teams per
            // workgroup sharing x, fetched ahead of the weights
            if (rows <= 8192) { c.r = 1; c.grid = 8 * scale; c.tpw = 4; }
            if (rows > 8192) c.tpw = 8;
            if (rows > 65536) { c.wg = 2; c.grid = 8 * scale; c.tpw = 4; }  // vocabulary-sized
            break;
        case 192:  // K = 6144: four one-wave teams per workgroup sharing x,
                   // fetched ahead of the weights (Qwen3-1.7B down 3.43 -> 3.09 us)
            c.wg = 1; c.r = 1; c.grid = 4 * scale; c.tpw = 4;
            break;
        case 256:  // K = 8192
            c.wg = 2; c.r = 4; c.grid = 8 * scale;
            break;
        default:  // K = 12288
            c.wg = 2; c.r = 1; c.grid = 4 * scale; c.tpw = 4;
            break;
    }
}

hipError_t launch_gemv_m1_group(const GemvGroup& g, int cus, const M1Config* forced) {
    if (g.count < 1 || g.count > kMaxSegs || !gemv_m1_supported(g.k)) return hipErrorNotSupported;
    uint32_t rows = 0;
    for (uint32_t s = 0; s < g.count; ++s) rows += g.n[s];
    M1Config c;
    default_m1_config(g.k, rows, cus, c);
    if (forced) {
        if (forced->wg) c.wg = forced->wg;
        if (forced->r) c.r = forced->r;
        if (forced->tpw) c.tpw = forced->tpw;
        if (forced->wg || forced->r || forced->grid) c.grid = forced->grid;
    }
    const uint32_t nblk = g.k / 32;
    if (c.wg < 1 || nblk % (64u * c.wg) != 0) return hipErrorNotSupported;
    if (c.tpw < 1 || 64 * c.wg * c.tpw > 512) return hipErrorNotSupported;
    // x staged in LDS with the partial sums: at most 64 KiB
    if (c.tpw > 1 && (uint64_t)g.k * (g.x_bf16 ? 2 : 4) + (uint64_t)c.tpw * 2 * c.wg * c.r * 4 > 65536)
        return hipErrorNotSupported;
    const int bpl = (int)(nblk / (64u * c.wg));
    Segs sg{};
    sg.count = g.count;
    sg.first[0] = 0;
    for (uint32_t s = 0; s < g.count; ++s) {
        sg.packed[s] = g.packed[s];
        sg.scales[s] = g.scales[s];
        sg.y[s] = g.y[s];
        sg.n[s] = g.n[s];
        sg.first[s + 1] = sg.first[s] + (g.n[s] + c.r - 1) / c.r;
    }
    for (uint32_t s = g.count; s < (uint32_t)kMaxSegs; ++s) sg.first[s + 1] = sg.first[g.count];
    const uint32_t rowsets = sg.first[g.count];
    sg.rowsets = rowsets;
    // c.grid counts teams; grid 0 (a forced configuration without a grid): one row-set per team
    uint32_t teams = c.grid == 0 || c.grid > rowsets ? rowsets : c.grid;
    // even split: every team visits the same number of row-sets (+-1)
    const uint32_t per = (rowsets + teams - 1) / teams;
    teams = (rowsets + per - 1) / per;
    const uint32_t grid = (teams + c.tpw - 1) / c.tpw;
    return g.x_bf16 ? go_cfg<true>(sg, g.x, g.k, grid, c.wg, bpl, c.r, c.tpw, g.stream)
                    : go_cfg<false>(sg, g.x, g.k, grid, c.wg, bpl, c.r, c.tpw, g.stream);
}

// M = 1 projection with the greedy-argmax epilogue (the lm_head of a greedy
// decode step): y is optional (nullptr: logits are not written), *idx gets the
// first index of the maximum. It runs the projection's own default launch
// shape when an epilogue instance of it is compiled -- one- and two-wave teams
// of 1-2 blocks per lane, 2 or 4 rows, at most 8 waves per workgroup (the
// 8B and 1.7B lm_heads) -- so the logits it writes are the projection's bit
// for bit; other shapes fall back to the one-wave vocabulary configuration,
// and where that does not fit either the caller gets hipErrorNotSupported and
// runs the projection and argmax_rows.
template <bool XBF16, int WG, int BPL, int R>
static hipError_t go_am(const Segs& sg, const void* x, uint32_t k, uint32_t grid, int tpw, uint32_t* idx, hipStream_t st) {
    const size_t lds = (tpw > 1 ? (size_t)k * (XBF16 ? 2 : 4) : 0) + (size_t)tpw * 2 * WG * R * sizeof(float);
    hipLaunchKernelGGL((gemv_m1_one_kernel<XBF16, WG, BPL, R, true>), dim3(grid), dim3(64 * WG * tpw), lds, st,
                       sg.packed[0], sg.scales[0], x, sg.n[0], k, sg.rowsets, (uint32_t)tpw, grid, sg.y[0],
                       sg.am_partial);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_argmax_reduce(sg.am_partial, 1, grid, idx, st);
}

template <bool XBF16>
static hipError_t go_am_cfg(const Segs& sg, const void* x, uint32_t k, uint32_t grid, int wg, int bpl, int r, int tpw,
                            uint32_t* idx, hipStream_t st) {
#define MX4_AM_CASE(W, B, R_) \
    if (wg == W && bpl == B && r == R_) return go_am<XBF16, W, B, R_>(sg, x, k, grid, tpw, idx, st);
    MX4_AM_CASE(1, 1, 2) MX4_AM_CASE(1, 1, 4) MX4_AM_CASE(1, 2, 2) MX4_AM_CASE(1, 2, 4)
    MX4_AM_CASE(2, 1, 2) MX4_AM_CASE(2, 1, 4)
#undef MX4_AM_CASE
    return hipErrorNotSupported;
}

static bool am_compiled(int wg, int bpl, int r) {
    return (wg == 1 && (bpl == 1 || bpl == 2) && (r == 2 || r == 4)) || (wg == 2 && bpl == 1 && (r == 2 || r == 4));
}

hipError_t launch_gemv_m1_argmax(const GemvArgs& a, uint64_t* partial, uint32_t max_partials, uint32_t* idx,
                                 int cus) {
    if (!gemv_m1_supported(a.k) || a.n == 0) return hipErrorNotSupported;
    M1Config c;
    default_m1_config(a.k, a.n, cus, c);
    const uint32_t nblk = a.k / 32;
    int bpl = (int)(nblk / (64u * c.wg));
    if (!am_compiled(c.wg, bpl, c.r) || c.tpw * c.wg > 8) {
        // the one-wave vocabulary-sized configuration (4 rows, 4 teams per CU, 4 per workgroup)
        c.wg = 1; c.r = 4; c.grid = 4 * (uint32_t)(cus > 0 ? cus : 256); c.tpw = 4;
        bpl = (int)(nblk / 64);
        if (!am_compiled(c.wg, bpl, c.r)) return hipErrorNotSupported;
    }
    Segs sg{};
    sg.count = 1;
    sg.packed[0] = a.packed;
    sg.scales[0] = a.scales;
    sg.y[0] = a.y;
    sg.n[0] = a.n;
    const uint32_t rowsets = (a.n + c.r - 1) / c.r;
    for (int q = 1; q <= kMaxSegs; ++q) sg.first[q] = rowsets;
    sg.rowsets = rowsets;
    sg.am_partial = partial;
    const int tpw = c.tpw < 1 ? 1 : c.tpw;
    if (tpw > 1 && (uint64_t)a.k * (a.x_bf16 ? 2 : 4) + (uint64_t)tpw * 2 * c.wg * c.r * 4 > 65536)
        return hipErrorNotSupported;
    uint32_t teams = c.grid == 0 || c.grid > rowsets ? rowsets : c.grid;
    const uint32_t per = (rowsets + teams - 1) / teams;
    teams = (rowsets + per - 1) / per;
    const uint32_t grid = (teams + tpw - 1) / tpw;
    if (grid > max_partials) return hipErrorNotSupported;
    return a.x_bf16 ? go_am_cfg<true>(sg, a.x, a.k, grid, c.wg, bpl, c.r, tpw, idx, a.stream)
                    : go_am_cfg<false>(sg, a.x, a.k, grid, c.wg, bpl, c.r, tpw, idx, a.stream);
}

hipError_t launch_gemv_m1(const GemvArgs& a, int cus) {
    GemvGroup g{};
    g.count = 1;
    g.packed[0] = a.packed;
    g.scales[0] = a.scales;
    g.y[0] = a.y;
    g.n[0] = a.n;
    g.k = a.k;
    g.x = a.x;
    g.x_bf16 = a.x_bf16;
    g.stream = a.stream;
    return launch_gemv_m1_group(g, cus, nullptr);
}

// Default shape of the few-token launch, from sweeps on MI355X (Qwen3
// shapes, 2..4 tokens): wide weights (4096 row-sets or more) use one
// workgroup per CU whose 8 / WG teams share one LDS copy of the token rows
// (when it fits); narrower ones four one-wave teams per workgroup sharing it,
// or, with several waves per team, independent teams (512).
static void mt_default(uint32_t rowsets, int wg, int cus, bool x_fits, uint32_t& teams, uint32_t& tpw) {
    if (rowsets >= 4096 && x_fits) {
        tpw = 8u / (uint32_t)wg;
        teams = (uint32_t)cus * tpw;
    } else if (wg == 1 && x_fits) {
        // narrower weights with one-wave teams: four teams per workgroup share
        // the token rows, fetched ahead of the weights (8B q / k at 2 tokens
        // 4.49 / 3.09 -> 3.87 / 2.71 us against independent teams)
        tpw = 4;
        teams = (uint32_t)cus * 4u;
    } else {
        tpw = 1;
        teams = (uint32_t)cus * (wg == 1 ? 4u : 2u);
    }
    if (teams > rowsets) teams = rowsets;
}

// teams: row-set walkers (0: the default); tpw: teams per workgroup sharing one
// LDS copy of the token rows (0: the default; more than one needs the copy and
// the partial sums within 64 KiB).
template <int WG, int BPL, int R, int MT>
static hipError_t go_mt(const GemvArgs& a, int cus, uint32_t teams, uint32_t tpw) {
    // a group: each weight a run of row-sets
    Segs sg{};
    uint32_t rowsets = (a.n + R - 1) / R;
    if (a.group) {
        sg.count = a.group->count;
        sg.first[0] = 0;
        for (uint32_t s = 0; s < sg.count; ++s) {
            sg.packed[s] = a.group->packed[s];
            sg.scales[s] = a.group->scales[s];
            sg.y[s] = a.group->y[s];
            sg.n[s] = a.group->n[s];
            sg.first[s + 1] = sg.first[s] + (sg.n[s] + R - 1) / R;
        }
        for (uint32_t s = sg.count; s < (uint32_t)kMaxSegs; ++s) sg.first[s + 1] = sg.first[sg.count];
        rowsets = sg.first[sg.count];
        sg.rowsets = rowsets;
    }

    constexpr uint32_t xbytes = MT * 2048u * WG * BPL * 2;
    if (teams == 0 || tpw == 0)
        mt_default(rowsets, WG, cus, xbytes + (8 / WG) * 2 * WG * R * MT * 4 <= 65536, teams, tpw);
    if (tpw < 1 || 64 * WG * tpw > 512) return hipErrorNotSupported;
    if (tpw > 1 && xbytes + tpw * 2 * WG * R * MT * 4 > 65536) return hipErrorNotSupported;
    if (teams > rowsets) teams = rowsets;
    const uint32_t grid = (teams + tpw - 1) / tpw;
    const size_t lds = (tpw > 1 ? xbytes : 0) + (size_t)tpw * 2 * WG * R * MT * sizeof(float);
    if (a.group) {
        if (tpw > 1)
            hipLaunchKernelGGL((gemv_mt_kernel<WG, BPL, R, MT, true, Segs>), dim3(grid), dim3(64 * WG * tpw), lds,
                               a.stream, nullptr, nullptr, a.x, a.m, 0u, rowsets, tpw, grid, nullptr, sg);
        else
            hipLaunchKernelGGL((gemv_mt_kernel<WG, BPL, R, MT, false, Segs>), dim3(grid), dim3(64 * WG * tpw), lds,
                               a.stream, nullptr, nullptr, a.x, a.m, 0u, rowsets, tpw, grid, nullptr, sg);
    } else {
        if (tpw > 1)
            hipLaunchKernelGGL((gemv_mt_kernel<WG, BPL, R, MT, true, NoSegs>), dim3(grid), dim3(64 * WG * tpw), lds,
                               a.stream, a.packed, a.scales, a.x, a.m, a.n, rowsets, tpw, grid, a.y, NoSegs{});
        else
            hipLaunchKernelGGL((gemv_mt_kernel<WG, BPL, R, MT, false, NoSegs>), dim3(grid), dim3(64 * WG * tpw), lds,
                               a.stream, a.packed, a.scales, a.x, a.m, a.n, rowsets, tpw, grid, a.y, NoSegs{});
    }
    return hipGetLastError();
}

bool gemv_mt_supported(uint32_t m, uint32_t k, bool x_bf16) {
    return x_bf16 && m >= 2 && m <= 4 && (k == 2048 || k == 4096 || k == 6144 || k == 8192 || k == 12288);
}

hipError_t launch_gemv_mt(const GemvArgs& a, int cus, uint32_t teams, uint32_t tpw) {
    if (!gemv_mt_supported(a.m, a.k, a.x_bf16)) return hipErrorNotSupported;
    if (a.group) {
        if (a.group->count < 1 || a.group->count > (uint32_t)kMaxSegs) return hipErrorNotSupported;
        for (uint32_t s = 0; s < a.group->count; ++s)
            if (a.group->n[s] == 0) return hipErrorNotSupported;
    } else if (a.n == 0) {
        return hipErrorNotSupported;
    }
#define MX4_MT(K, W, B)                                                                                  \
    if (a.k == K) return a.m <= 2 ? go_mt<W, B, 2, 2>(a, cus, teams, tpw) : go_mt<W, B, 2, 4>(a, cus, teams, tpw);
    MX4_MT(2048, 1, 1)
    MX4_MT(4096, 1, 2)
    MX4_MT(6144, 3, 1)
    MX4_MT(8192, 2, 2)
    // K = 12288 at 2 tokens: the M = 1 kernel's geometry (2-wave teams, one row
    // each, four teams per workgroup sharing x through LDS): 8B down 8.77 -> 8.24 us
    if (a.k == 12288 && a.m <= 2) return go_mt<2, 3, 1, 2>(a, cus, teams, tpw);
    MX4_MT(12288, 3, 2)
#undef MX4_MT
    return hipErrorNotSupported;
}

template <bool XBF16, int MT>
static hipError_t launch_generic_t(const GemvArgs& a) {
    dim3 grid((a.n + 3) / 4, (a.m + MT - 1) / MT);
    hipLaunchKernelGGL((gemv_generic_kernel<XBF16, MT>), grid, dim3(256), 0, a.stream, a.packed, a.scales,
                       a.x, a.y, a.m, a.n, a.k);
    return hipGetLastError();
}

hipError_t launch_gemv_generic(const GemvArgs& a) {
    if (a.m == 1) return a.x_bf16 ? launch_generic_t<true, 1>(a) : launch_generic_t<false, 1>(a);
    return a.x_bf16 ? launch_generic_t<true, 4>(a) : launch_generic_t<false, 4>(a);
}

}  // namespace mx4
