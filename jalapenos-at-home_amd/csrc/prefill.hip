// prefill.hip -- prefill GEMM (many token rows) on CDNA4 block-scaled MFMA:
// y[m, n] = sum_k xq[m, k] * w(n, k) with V_MFMA_SCALE_F32_32X32X64_F8F6F4.
//
// The reference runs prefill on a 16x16 FP32 tiled kernel that decodes each
// weight element into threadgroup memory (project_mxfp4,
// engine/src/matmul.metal:65-97). Here the weights stay in their MXFP4 form all
// the way into the matrix core: operand B is the packed E2M1 nibbles (element
// 2j in the low nibble of byte j, which is also the operand's element order)
// with the E8M0 byte of each 32-element block as the lane's B scale. Operand A
// is the activations after per-32 requantization (MXFP4 by the same rule as
// the weights, python/quantize_mxfp4.py:18-39, or MX-FP8 E4M3), with their
// E8M0 bytes as A scales. Products of FP4/FP8 values with power-of-two scales
// are exact; the matrix core accumulates in f32.
//
// Operand layout (32x32x64), established by in-bounds probes and pinned by the
// identity tests: for FP4, lane l holds row (l % 32) of A (column of B) and the
// 32 K values [32 (l / 32), +32) of the 64 -- one MX block; for FP8 A, lane
// group h = l / 32 holds K [16h, 16h + 16) and [32 + 16h, +16). Either way the
// scale byte of lane group h applies to K block h. C: lane l holds column
// l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4 of accumulator register v.
//
// Fragment-native layout. Read in the stored row-major layout, one operand
// fragment (32 rows x 32 bytes) touches 32 cache lines per load instruction,
// and the address path, not HBM, limits the kernel. The operands are therefore
// rewritten once into the order the matrix core consumes them: rows in groups
// of 32; for group g and k-step kk (64 elements of K) the FP4 fragment is 1 KiB
// contiguous, lane l's 16 bytes at 16 l (row 32 g + l % 32, bytes
// [32 kk + 16 (l / 32), +16) of the row); an FP8 fragment is 2 KiB, the first
// 1 KiB holding each lane's bytes [64 kk + 16 h, +16) and the second its bytes
// [64 kk + 32 + 16 h, +16). Scales: for group g and quad q (4 k-steps) 64
// lanes x 4 bytes, byte u of lane l = the E8M0 byte of block 8 q + 2 u + l / 32
// of row 32 g + l % 32, so the MFMA's byte select (op_sel) picks k-step u.
// Weights get this copy once (prepare); activations are requantized straight
// into it. Every load is then a 1 KiB coalesced burst straight into the
// registers the matrix core reads: no LDS and no barriers in the main loop.
//
// Kernel: a wave owns a (32 TM) x (32 TN) output tile over its K range and
// keeps a ring of Q slots of U k-steps of fragments in flight (the register
// file is the prefetch buffer). Four waves per workgroup: 2 x 2 tiles, two
// tiles x two K halves (KSPLIT = 2) or one tile x four K quarters (KSPLIT =
// 4); partial tiles of one output tile meet in LDS at the end and are summed
// in K order. Each fragment row-group gets its own buffer resource bounded to the
// wave's K range, so the prefetch beyond it reads zeros without touching memory.
#include "mx4_device.h"
#include "mx4_kernels.h"

namespace mx4 {

namespace {


// See skinny.hip: drain the matrix pipe before accumulators are read after a branch.
__device__ __forceinline__ void mfma_drain() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    __builtin_amdgcn_sched_barrier(0);
}

constexpr int kFmtFp8 = 0, kFmtFp4 = 4;  // MFMA operand format codes (cbsz / blgp)

template <bool A_FP8, int TM, int TN, int U>
struct Slot {
    u32x4 a[U][TM][A_FP8 ? 2 : 1];
    u32x4 b[U][TN];
};

// One k-step of the wave tile: TM x TN MFMAs; OPSEL picks the scale byte (the
// k-step within its quad).
template <int OPSEL, bool A_FP8, int TM, int TN>
__device__ __forceinline__ void kstep(const u32x4 (&a)[TM][A_FP8 ? 2 : 1], const u32x4 (&b)[TN],
                                      const uint32_t (&sa)[TM], const uint32_t (&sb)[TN], f32x16 (&acc)[TM][TN]) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        i32x8 av;
        if constexpr (A_FP8) {
            const u32x4 lo = a[i][0], hi = a[i][1];
            av = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        } else {
            const u32x4 v = a[i][0];
            av = i32x8{(int)v[0], (int)v[1], (int)v[2], (int)v[3], 0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const u32x4 w = b[j];
            const i32x8 bv = i32x8{(int)w[0], (int)w[1], (int)w[2], (int)w[3], 0, 0, 0, 0};
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc[i][j], A_FP8 ? kFmtFp8 : kFmtFp4,
                                                                        kFmtFp4, OPSEL, (int)sa[i], OPSEL, (int)sb[j]);
        }
    }
}

// Bytes from `base` to the end of an allocation of `total` bytes, at most `want`.
__device__ __forceinline__ uint32_t clamp_bytes(uint64_t want, uint64_t base, uint64_t total) {
    return (uint32_t)(base >= total ? 0 : (total - base < want ? total - base : want));
}

// Wave grid of a workgroup for a K split: 2 x 2 tiles (1), 1 x 2 tiles x two
// K halves (2), one tile x four K quarters (4).
constexpr int wave_rows(int ksplit) { return ksplit == 1 ? 2 : 1; }
constexpr int wave_cols(int ksplit) { return ksplit == 4 ? 1 : 2; }

// TM x TN tiles of 32 x 32 per wave; U k-steps per slot; Q slots in flight;
// KSPLIT K parts per workgroup; RS scale quads in flight; NKC = k-steps per
// wave when fixed at compile time (fully unrolled), 0 for a loop. One loop
// body is ROT turns of the slot ring, enough to cover whole rounds of the
// scale ring.
// The weights of one launch: segment s takes workgroup columns [tile0[s],
// tile0[s + 1]); unused segments start at 0xffffffff.
struct Segs {
    const uint8_t* wf[kMaxPrefillGroup];
    const uint8_t* wsf[kMaxPrefillGroup];
    float* y[kMaxPrefillGroup];
    uint32_t n[kMaxPrefillGroup];
    uint32_t tile0[kMaxPrefillGroup];
};

template <bool A_FP8, int TM, int TN, int U, int Q, int KSPLIT, int RS, int NKC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void prefill_kernel(
    const uint8_t* __restrict__ xf, const uint8_t* __restrict__ xsf, uint32_t m, uint32_t k, const Segs segs) {
    static_assert((Q * U) % 4 == 0, "slots must cover whole scale quads");
    constexpr int ROT = ((Q * U) / 4) % RS == 0 ? 1 : RS;
    static_assert(((ROT * Q * U) / 4) % RS == 0, "a loop body must cover whole rounds of the scale ring");
    static_assert(KSPLIT == 1 || KSPLIT == 2 || KSPLIT == 4, "K split of 1, 2 or 4 waves");
    constexpr int WM = wave_rows(KSPLIT), WN = wave_cols(KSPLIT);
    constexpr uint32_t BM = WM * 32 * TM, BN = WN * 32 * TN;
    constexpr uint32_t AF = A_FP8 ? 2048 : 1024;  // bytes of one A fragment
    const uint32_t t = threadIdx.x, lane = t % 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t / 64);
    const uint32_t wn = wave % WN;
    const uint32_t wm = KSPLIT == 1 ? wave / 2 : 0;
    const uint32_t kh = wave / (WM * WN);
    // this workgroup's weight: uniform selects over the segment table (an
    // index into the argument struct would be a memory load)
    const uint32_t bx = blockIdx.x;
    const uint8_t* __restrict__ wf = segs.wf[0];
    const uint8_t* __restrict__ wsf = segs.wsf[0];
    float* __restrict__ y = segs.y[0];
    uint32_t n = segs.n[0], t0 = 0;
#pragma unroll
    for (int s = 1; s < (int)kMaxPrefillGroup; ++s) {
        const bool in = bx >= segs.tile0[s];
        wf = in ? segs.wf[s] : wf;
        wsf = in ? segs.wsf[s] : wsf;
        y = in ? segs.y[s] : y;
        n = in ? segs.n[s] : n;
        t0 = in ? segs.tile0[s] : t0;
    }
    const uint32_t m0 = blockIdx.y * BM + wm * 32 * TM;
    const uint32_t n0 = (bx - t0) * BN + wn * 32 * TN;
    const uint32_t nk_all = k / 64, nq_all = k / 256;
    const uint32_t nk = NKC ? (uint32_t)NKC : nk_all / KSPLIT;  // k-steps of this wave
    const uint32_t k0 = kh * nk;
    const uint32_t ga = m0 / 32, gb = n0 / 32;  // first row groups
    const uint64_t a_total = (uint64_t)((m + 31) / 32) * nk_all * AF;
    const uint64_t b_total = (uint64_t)((n + 31) / 32) * nk_all * 1024;
    const uint64_t as_total = (uint64_t)((m + 31) / 32) * nq_all * 256;
    const uint64_t bs_total = (uint64_t)((n + 31) / 32) * nq_all * 256;

    // one resource per row group, bounded to this wave's K range
    __amdgpu_buffer_rsrc_t ar[TM], asr[TM], br[TN], bsr[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const uint64_t base = ((uint64_t)(ga + i) * nk_all + k0) * AF;
        const uint64_t sbase = ((uint64_t)(ga + i) * nq_all + k0 / 4) * 256;
        ar[i] = rsrc(xf + (base < a_total ? base : 0), clamp_bytes((uint64_t)nk * AF, base, a_total));
        asr[i] = rsrc(xsf + (sbase < as_total ? sbase : 0), clamp_bytes((uint64_t)nk / 4 * 256, sbase, as_total));
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const uint64_t base = ((uint64_t)(gb + j) * nk_all + k0) * 1024;
        const uint64_t sbase = ((uint64_t)(gb + j) * nq_all + k0 / 4) * 256;
        br[j] = rsrc(wf + (base < b_total ? base : 0), clamp_bytes((uint64_t)nk * 1024, base, b_total));
        bsr[j] = rsrc(wsf + (sbase < bs_total ? sbase : 0), clamp_bytes((uint64_t)nk / 4 * 256, sbase, bs_total));
    }

    using S = Slot<A_FP8, TM, TN, U>;
    constexpr uint32_t kSlots = NKC ? (uint32_t)NKC / U : 0xffffffffu;  // slots that exist (unrolled form)
    auto issue = [&](uint32_t slot, S& s) {
        if (slot >= kSlots) return;  // folded away when unrolled; never taken in the loop form
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t kk = slot * U + u;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                s.a[u][i][0] = __builtin_amdgcn_raw_buffer_load_b128(ar[i], kk * AF + 16 * lane, 0, 0);
                if constexpr (A_FP8)
                    s.a[u][i][1] = __builtin_amdgcn_raw_buffer_load_b128(ar[i], kk * AF + 1024 + 16 * lane, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j)
                s.b[u][j] = __builtin_amdgcn_raw_buffer_load_b128(br[j], kk * 1024 + 16 * lane, 0, 0);
        }
    };
    uint32_t sa[RS][TM], sb[RS][TN];
    auto issue_scales = [&](uint32_t quad, uint32_t (&a)[TM], uint32_t (&b)[TN]) {
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = __builtin_amdgcn_raw_buffer_load_b32(asr[i], quad * 256 + 4 * lane, 0, 0);
#pragma unroll
        for (int j = 0; j < TN; ++j) b[j] = __builtin_amdgcn_raw_buffer_load_b32(bsr[j], quad * 256 + 4 * lane, 0, 0);
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    S sl[Q];
#pragma unroll
    for (int r = 0; r < RS - 1; ++r) issue_scales(r, sa[r], sb[r]);
#pragma unroll
    for (int j = 0; j < Q; ++j) issue(j, sl[j]);
    // ROT turns of the ring: Q slots of U k-steps each, from k-step `base`
    auto body = [&](uint32_t base) {
#pragma unroll
        for (int rot = 0; rot < ROT; ++rot)
#pragma unroll
            for (int j = 0; j < Q; ++j) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int kl = (rot * Q + j) * U + u;
                    const int g = kl / 4, o = kl % 4;
                    if (o == 0) issue_scales(base / 4 + g + RS - 1, sa[(g + RS - 1) % RS], sb[(g + RS - 1) % RS]);
                    switch (o) {
                        case 0: kstep<0, A_FP8, TM, TN>(sl[j].a[u], sl[j].b[u], sa[g % RS], sb[g % RS], acc); break;
                        case 1: kstep<1, A_FP8, TM, TN>(sl[j].a[u], sl[j].b[u], sa[g % RS], sb[g % RS], acc); break;
                        case 2: kstep<2, A_FP8, TM, TN>(sl[j].a[u], sl[j].b[u], sa[g % RS], sb[g % RS], acc); break;
                        default: kstep<3, A_FP8, TM, TN>(sl[j].a[u], sl[j].b[u], sa[g % RS], sb[g % RS], acc); break;
                    }
                }
                // refill this slot only after its MFMAs were issued: otherwise the
                // scheduler hoists every refill to the end of the ring turn
                __builtin_amdgcn_sched_barrier(0);
                issue(base / U + rot * Q + j + Q, sl[j]);
                __builtin_amdgcn_sched_barrier(0);
            }
    };
    if constexpr (NKC != 0) {
        // straight-line code: the wait counts stay exact (in a loop the compiler
        // waits for every outstanding load at the loop head)
        static_assert(NKC % (ROT * Q * U) == 0, "the unrolled form covers whole loop bodies");
#pragma unroll
        for (uint32_t base = 0; base < (uint32_t)NKC; base += ROT * Q * U) body(base);
    } else {
        // a partial last body reads zeros past the resources' K range
        for (uint32_t base = 0; base < nk; base += ROT * Q * U) body(base);
    }
    mfma_drain();

    // K parts meet as a tree: part p + KSPLIT/2 into p, then part 1 into 0 (a
    // fixed order, so repeated calls agree bit for bit). Waves that are done
    // return; a barrier waits only for the waves still running. Partial tiles
    // cross LDS as 16-byte vectors (lane l's values 4q..4q+3 of a tile at
    // [tile][q][l]), and the last addition happens tile by tile in the store
    // loop: summing all tiles first kept every accumulator live in VGPRs, and
    // the LDS reads then went out two at a time.
    constexpr int T = TM * TN, HALF = KSPLIT / 2;
    __shared__ f32x4 red[KSPLIT > 1 ? WN * HALF * T * 4 * 64 : 1];
    auto red_at = [&](uint32_t part, int tile, int q) -> f32x4& {
        return red[(((wn * HALF + part) * T + tile) * 4 + q) * 64 + lane];
    };
    if constexpr (KSPLIT > 1) {
#pragma unroll
        for (int width = HALF; width >= 1; width /= 2) {
            if (kh >= (uint32_t)width) {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            red_at(kh - width, i * TN + j, q) =
                                f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            }
            __syncthreads();
            if (kh >= (uint32_t)width) return;
            if (width > 1) {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const f32x4 o = red_at(kh, i * TN + j, q);
#pragma unroll
                            for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += o[e];
                        }
                __syncthreads();
            }
        }
    }
    // Branch-free stores through a resource over y (prefill_supported keeps
    // row n 4 + 4 col below 2^31 over the whole grid): rows past m fall
    // outside it, and a column past n is biased by 2^31, past its end, so the
    // hardware drops both. (Guarded stores cost a branch per element.)
    // The stores carry device scope (SC1): at M = 512 the f32 output is as
    // large as the weights (25 MB for gate), and with the default scope most of
    // it waited in the L2 for the write-back at the end of the kernel. Measured
    // per call: q 10.8 -> 10.1 us, gate 21.5 -> 20.2 us, down 22.4 -> 21.9 us.
    constexpr int kStoreDeviceScope = 0x10;
    const uint32_t r32 = lane % 32, h = lane / 32;
    const __amdgpu_buffer_rsrc_t yr = rsrc(y, m * n * 4);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const uint32_t col = n0 + 32 * j + r32;
        const uint32_t cb = 4 * col + (col < n ? 0u : 0x80000000u);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            f32x4 o[4] = {};
            if constexpr (KSPLIT > 1) {
#pragma unroll
                for (int q = 0; q < 4; ++q) o[q] = red_at(0, i * TN + j, q);  // part 1's (partial) tile
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t row = m0 + 32 * i + 8 * (v / 4) + 4 * h + (v % 4);
                const float out = KSPLIT > 1 ? acc[i][j][v] + o[v / 4][v % 4] : acc[i][j][v];
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(out), yr, row * n * 4 + cb, 0,
                                                      kStoreDeviceScope);
            }
        }
    }
}

// Workgroup-shared operands: a workgroup of KH x WM x WN waves owns a BM x BN
// output tile. Each stage (U k-steps) of both operands' fragments -- and the
// scale words of its quad -- is loaded once per workgroup, straight into LDS
// by direct-to-LDS buffer loads (one 1 KiB fragment per instruction), into a
// ring of D stages with D - 1 in flight; a wave reads its TM A and TN B
// fragments of a k-step from LDS (16 bytes per lane at 16 l, the operand
// order) and issues its TM x TN MFMAs. One barrier per stage.
// KH = 1: the WM x WN waves cover the whole of K. KH = 2: two sets of WM x WN
// waves take one half of K each, every set with its own ring, so each SIMD
// runs two waves whose loads and MFMAs interleave; at the end the second
// half's tile crosses LDS and the first half adds it (a fixed order, so
// repeated calls agree bit for bit).
// PP (ping-pong, KH = 2 only): every stage is split into a memory tick (the
// stage's fragments from LDS into registers, the next loads issued) and a
// matrix tick (its MFMAs), each opened by a workgroup barrier, and the second
// K half runs one tick behind the first: on every SIMD one wave issues MFMAs
// while the other reads LDS, instead of both competing for the same phase. The
// arithmetic and its order are those of the KH = 2 kernel, so the outputs are
// the same bits.
template <bool A_FP8, int WM, int WN, int TM, int TN, int U, int D, int KH = 1>
struct LdsGeo {
    static constexpr int NW = WM * WN, NT = 64 * NW * KH;  // waves per K part; threads
    static constexpr int GA = WM * TM, GB = WN * TN;  // row groups of 32 per tile
    static constexpr int BM = 32 * GA, BN = 32 * GB;
    static constexpr int AFK = A_FP8 ? 2 : 1;         // 1 KiB pieces per A fragment
    static constexpr int A_BYTES = U * GA * AFK * 1024, B_BYTES = U * GB * 1024;
    static constexpr int SA = (GA + 3) / 4, SB = (GB + 3) / 4;  // scale loads (4 groups each)
    static constexpr int S_BYTES = NW * 1024;                     // one 1 KiB slot per wave
    static constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;
    static constexpr int RING = D * STAGE;
    static constexpr int FRAGS = U * (GA * AFK + GB), FI = FRAGS / NW;
    static constexpr int LPS = FI + 1;  // vector memory instructions per wave and stage
    static constexpr int RED = KH > 1 ? NW * TM * TN * 16 * 64 * 4 : 0;  // bytes of the K-half hand-over
    static constexpr int LDS = KH * RING > RED ? KH * RING : RED;
    // stages of 2 or 4 k-steps (a scale quad in one or two stages); every wave
    // loads the same number of fragments and one scale piece per stage; the
    // waits fit vmcnt; the rings fit the LDS; two K parts need two waves per
    // SIMD to fit in the register file
    static constexpr bool ok = (U == 2 || U == 4) && FRAGS % NW == 0 && SA + SB <= NW && D >= 2 && D <= 8 &&
                               (D - 2) * LPS <= 63 && LDS <= 160 * 1024 && (KH == 1 || (KH == 2 && NW == 4));
};

template <int LPS, int MAXA>
__device__ __forceinline__ void wait_ahead(uint32_t ahead) {
    // outstanding loads allowed: those of the `ahead` stages issued after the
    // one needed (ahead <= MAXA)
    if constexpr (MAXA >= 1) {
        if (ahead >= (uint32_t)MAXA) { wait_vm<MAXA * LPS>(); return; }
        wait_ahead<LPS, MAXA - 1>(ahead);
    } else {
        wait_vm<0>();
    }
}

template <bool A_FP8, int WM, int WN, int TM, int TN, int U, int D, int KH, bool PP>
__global__ __launch_bounds__(64 * WM * WN * KH) void prefill_lds_kernel(const uint8_t* __restrict__ xf,
                                                                       const uint8_t* __restrict__ xsf, uint32_t m,
                                                                       uint32_t k, const Segs segs) {
    using G = LdsGeo<A_FP8, WM, WN, TM, TN, U, D, KH>;
    static_assert(G::ok, "instance outside the kernel's stage, vmcnt and LDS limits");
    static_assert(!PP || KH == 2, "ping-pong alternates the two K halves");
    constexpr uint32_t AF = A_FP8 ? 2048 : 1024;
    constexpr int P = 4 / U;  // stages per scale quad
    __shared__ __attribute__((aligned(16))) uint8_t lds_all[G::LDS];
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t kh = wave_all / G::NW, wave = wave_all % G::NW;  // K part; wave within it
    uint8_t* const lds = lds_all + kh * G::RING;
    const uint32_t wm = wave / WN, wn = wave % WN;
    const uint32_t bx = blockIdx.x;
    const uint8_t* __restrict__ wf = segs.wf[0];
    const uint8_t* __restrict__ wsf = segs.wsf[0];
    float* __restrict__ y = segs.y[0];
    uint32_t n = segs.n[0], t0 = 0;
#pragma unroll
    for (int s = 1; s < (int)kMaxPrefillGroup; ++s) {
        const bool in = bx >= segs.tile0[s];
        wf = in ? segs.wf[s] : wf;
        wsf = in ? segs.wsf[s] : wsf;
        y = in ? segs.y[s] : y;
        n = in ? segs.n[s] : n;
        t0 = in ? segs.tile0[s] : t0;
    }
    const uint32_t ga0 = blockIdx.y * G::GA, gb0 = (bx - t0) * G::GB;  // first row groups of the tile
    const uint32_t nk_all = k / 64, nq_all = k / 256, stages = nk_all / U / KH;
    const uint32_t kk0 = kh * (nk_all / KH);  // first k-step of this K part (a whole scale quad)
    const uint32_t ga_n = (m + 31) / 32, gb_n = (n + 31) / 32;
    const __amdgpu_buffer_rsrc_t xr = rsrc(xf, ga_n * nk_all * AF);
    const __amdgpu_buffer_rsrc_t xsr = rsrc(xsf, ga_n * nq_all * 256);
    const __amdgpu_buffer_rsrc_t wr = rsrc(wf, gb_n * nk_all * 1024);
    const __amdgpu_buffer_rsrc_t wsr = rsrc(wsf, gb_n * nq_all * 256);

    // This wave's scale load: instruction (wave mod SA + SB) -- A groups 4i..4i+3
    // or B groups 4(i - SA).. -- into LDS slot `wave`; lane l takes 16 bytes of
    // group 4i + l / 16 (clamped to the tile's last group: the duplicate lands
    // in bytes nobody reads).
    const uint32_t si = wave % (G::SA + G::SB);
    const bool s_is_a = si < (uint32_t)G::SA;
    const uint32_t s_grp = (s_is_a ? si : si - G::SA) * 4 + lane / 16;
    const uint32_t s_last = s_is_a ? G::GA - 1 : G::GB - 1;
    const uint32_t s_row = (s_is_a ? ga0 : gb0) + (s_grp < s_last ? s_grp : s_last);
    const uint32_t s_goff = s_row * nq_all * 256 + (kk0 / 4) * 256 + (lane % 16) * 16;
    const __amdgpu_buffer_rsrc_t s_r = s_is_a ? xsr : wsr;

    auto issue = [&](uint32_t st, uint32_t slot) {
        uint8_t* base = lds + slot * G::STAGE;
#pragma unroll
        for (int q = 0; q < G::FI; ++q) {
            // fragment f of the stage: A pieces first, then B; uniform selects
            // rather than a branch (the compiler waits for every load at a join)
            const uint32_t f = q * G::NW + wave;
            const bool is_a = f < (uint32_t)(U * G::GA * G::AFK);
            const uint32_t fa = f, kka = fa / (G::GA * G::AFK), rem = fa % (G::GA * G::AFK);
            const uint32_t ia = rem / G::AFK, half = rem % G::AFK;
            const uint32_t fb = f - U * G::GA * G::AFK, kkb = fb / G::GB, jb = fb % G::GB;
            const uint32_t lds_off = is_a ? (kka * G::GA + ia) * AF + half * 1024
                                          : G::A_BYTES + (kkb * G::GB + jb) * 1024;
            const uint32_t goff = is_a ? ((ga0 + ia) * nk_all + kk0 + st * U + kka) * AF + half * 1024
                                       : ((gb0 + jb) * nk_all + kk0 + st * U + kkb) * 1024;
            load_lds16(is_a ? xr : wr, (lds_ptr)(base + lds_off), goff + 16 * lane);
        }
        load_lds16(s_r, (lds_ptr)(base + G::A_BYTES + G::B_BYTES + wave * 1024), s_goff + (st / P) * 256);
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    // k-step kk of the stage in `slot`; the scale byte of k-step (E U + kk) of the quad
    auto compute = [&](uint32_t slot, auto e_tag) {
        constexpr int E = decltype(e_tag)::value;
        const uint8_t* base = lds + slot * G::STAGE;
        const uint8_t* sbase = base + G::A_BYTES + G::B_BYTES;
        uint32_t sa[TM], sb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const uint32_t g = wm * TM + i;
            sa[i] = *reinterpret_cast<const uint32_t*>(sbase + (g / 4) * 1024 + (g % 4) * 256 + 4 * lane);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t g = wn * TN + j;
            sb[j] = *reinterpret_cast<const uint32_t*>(sbase + (G::SA + g / 4) * 1024 + (g % 4) * 256 + 4 * lane);
        }
#pragma unroll
        for (int kk = 0; kk < U; ++kk) {
            u32x4 a[TM][A_FP8 ? 2 : 1], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const uint8_t* ap = base + (kk * G::GA + wm * TM + i) * AF + 16 * lane;
                a[i][0] = *reinterpret_cast<const u32x4*>(ap);
                if constexpr (A_FP8) a[i][1] = *reinterpret_cast<const u32x4*>(ap + 1024);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j)
                b[j] = *reinterpret_cast<const u32x4*>(base + G::A_BYTES + (kk * G::GB + wn * TN + j) * 1024 + 16 * lane);
            constexpr int o0 = E * U;
            switch (o0 + kk) {
                case 0: kstep<0, A_FP8, TM, TN>(a, b, sa, sb, acc); break;
                case 1: kstep<1, A_FP8, TM, TN>(a, b, sa, sb, acc); break;
                case 2: kstep<2, A_FP8, TM, TN>(a, b, sa, sb, acc); break;
                default: kstep<3, A_FP8, TM, TN>(a, b, sa, sb, acc); break;
            }
        }
    };

#pragma unroll
    for (int p = 0; p < D - 1; ++p)
        if ((uint32_t)p < stages) issue(p, p);
    if constexpr (!PP) {
        for (uint32_t st0 = 0; st0 < stages; st0 += P) {
#pragma unroll
            for (int e = 0; e < P; ++e) {
                const uint32_t st = st0 + e;
                const uint32_t left = stages - 1 - st;
                wait_ahead<G::LPS, D - 2>(left < (uint32_t)(D - 2) ? left : (uint32_t)(D - 2));
                lds_barrier();
                if (st + D - 1 < stages) issue(st + D - 1, (st + D - 1) % D);
                if (e == 0) compute(st % D, std::integral_constant<int, 0>{});
                else if constexpr (P > 1) compute(st % D, std::integral_constant<int, (P > 1 ? 1 : 0)>{});
            }
        }
    } else {
        // the stage's operands and scale words, read in the memory tick
        u32x4 ra[U][TM][A_FP8 ? 2 : 1], rb[U][TN];
        uint32_t rsa[TM], rsb[TN];
        auto read_stage = [&](uint32_t slot) {
            const uint8_t* base = lds + slot * G::STAGE;
            const uint8_t* sbase = base + G::A_BYTES + G::B_BYTES;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const uint32_t g = wm * TM + i;
                rsa[i] = *reinterpret_cast<const uint32_t*>(sbase + (g / 4) * 1024 + (g % 4) * 256 + 4 * lane);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const uint32_t g = wn * TN + j;
                rsb[j] = *reinterpret_cast<const uint32_t*>(sbase + (G::SA + g / 4) * 1024 + (g % 4) * 256 + 4 * lane);
            }
#pragma unroll
            for (int kk = 0; kk < U; ++kk) {
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const uint8_t* ap = base + (kk * G::GA + wm * TM + i) * AF + 16 * lane;
                    ra[kk][i][0] = *reinterpret_cast<const u32x4*>(ap);
                    if constexpr (A_FP8) ra[kk][i][1] = *reinterpret_cast<const u32x4*>(ap + 1024);
                }
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    rb[kk][j] = *reinterpret_cast<const u32x4*>(base + G::A_BYTES + (kk * G::GB + wn * TN + j) * 1024 +
                                                                16 * lane);
            }
        };
        // a barrier the scheduler moves nothing across
        auto tick = []() {
            __builtin_amdgcn_sched_barrier(0);
            lds_barrier();
            __builtin_amdgcn_sched_barrier(0);
        };
        // both halves pass 2 * stages + 1 barriers here: the second half's
        // extra one comes first, the first half's last
        if (kh == 1) tick();
        for (uint32_t st0 = 0; st0 < stages; st0 += P) {
#pragma unroll
            for (int e = 0; e < P; ++e) {
                const uint32_t st = st0 + e;
                const uint32_t left = stages - 1 - st;
                // memory tick: stage st has landed (every wave of this half
                // waited for its own loads before the barrier); slot
                // (st - 1) % D was read by all of them before the previous
                // matrix tick's barrier, so the next loads may take it
                wait_ahead<G::LPS, D - 2>(left < (uint32_t)(D - 2) ? left : (uint32_t)(D - 2));
                tick();
                read_stage(st % D);
                if (st + D - 1 < stages) issue(st + D - 1, (st + D - 1) % D);
                // matrix tick (the barrier waits for the LDS reads)
                tick();
#pragma unroll
                for (int kk = 0; kk < U; ++kk) {
                    switch (e * U + kk) {
                        case 0: kstep<0, A_FP8, TM, TN>(ra[kk], rb[kk], rsa, rsb, acc); break;
                        case 1: kstep<1, A_FP8, TM, TN>(ra[kk], rb[kk], rsa, rsb, acc); break;
                        case 2: kstep<2, A_FP8, TM, TN>(ra[kk], rb[kk], rsa, rsb, acc); break;
                        default: kstep<3, A_FP8, TM, TN>(ra[kk], rb[kk], rsa, rsb, acc); break;
                    }
                }
                // the MFMAs stay in their tick (the compiler would otherwise
                // sink them past the next memory tick's barrier)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(acc[i][j]));
            }
        }
        if (kh == 0) tick();
    }
    mfma_drain();

    if constexpr (KH > 1) {
        // the second K half hands its tile to the first through LDS (the rings
        // are done: every wave has passed its last stage's barrier and read
        // its operands before this barrier), as 16-byte vectors at
        // [wave][tile][q][lane]
        f32x4* red = reinterpret_cast<f32x4*>(lds_all);
        auto red_at = [&](int tile, int q) -> f32x4& { return red[((wave * TM * TN + tile) * 4 + q) * 64 + lane]; };
        __syncthreads();
        if (kh == 1) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        red_at(i * TN + j, q) =
                            f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        }
        __syncthreads();
        if (kh == 1) return;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4 o = red_at(i * TN + j, q);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += o[e];
                }
    }

    // Branch-free device-scope stores through a resource over y, as in prefill_kernel.
    constexpr int kStoreDeviceScope = 0x10;
    const uint32_t r32 = lane % 32, h = lane / 32;
    const uint32_t m0 = ga0 * 32 + wm * 32 * TM, n0 = gb0 * 32 + wn * 32 * TN;
    const __amdgpu_buffer_rsrc_t yr = rsrc(y, m * n * 4);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const uint32_t col = n0 + 32 * j + r32;
        const uint32_t cb = 4 * col + (col < n ? 0u : 0x80000000u);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t row = m0 + 32 * i + 8 * (v / 4) + 4 * h + (v % 4);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][v]), yr, row * n * 4 + cb, 0,
                                                      kStoreDeviceScope);
            }
    }
}

// Row-major codes -> fragment-native order. One thread per 16-byte output
// chunk; rows past `rows` (the padding of the last group) are zero.
template <bool FP8>
__global__ __launch_bounds__(256) void to_fragments_kernel(const uint8_t* __restrict__ src, uint32_t rows,
                                                           uint32_t k, uint64_t chunks, uint8_t* __restrict__ dst) {
    const uint64_t c = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= chunks) return;
    const uint32_t nk = k / 64, lane = (uint32_t)(c % 64);
    uint64_t rest = c / 64;
    uint32_t half = 0;
    if constexpr (FP8) {
        half = (uint32_t)(rest % 2);
        rest /= 2;
    }
    const uint32_t kk = (uint32_t)(rest % nk);
    const uint64_t g = rest / nk;
    const uint64_t row = 32 * g + lane % 32;
    const uint32_t h = lane / 32;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (row < rows) {
        const uint64_t off = FP8 ? row * k + 64 * kk + 32 * half + 16 * h : row * (k / 2) + 32 * kk + 16 * h;
        v = *reinterpret_cast<const u32x4*>(src + off);
    }
    *reinterpret_cast<u32x4*>(dst + 16 * c) = v;
}

// Row-major E8M0 bytes [rows][k/32] -> fragment-native scale words.
__global__ __launch_bounds__(256) void scales_to_fragments_kernel(const uint8_t* __restrict__ src, uint32_t rows,
                                                                  uint32_t k, uint64_t words,
                                                                  uint32_t* __restrict__ dst) {
    const uint64_t d = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= words) return;
    const uint32_t nq = k / 256, lane = (uint32_t)(d % 64);
    const uint64_t rest = d / 64;
    const uint32_t q = (uint32_t)(rest % nq);
    const uint64_t row = 32 * (rest / nq) + lane % 32;
    const uint32_t h = lane / 32;
    uint32_t v = 0;
    if (row < rows) {
        const uint8_t* s = src + row * (k / 32) + 8 * q + h;
        v = (uint32_t)s[0] | ((uint32_t)s[2] << 8) | ((uint32_t)s[4] << 16) | ((uint32_t)s[6] << 24);
    }
    dst[d] = v;
}

template <bool A_FP8, int TM, int TN, int U, int Q, int KSPLIT, int RS, int NKC>
hipError_t go(const PrefillArgs& a) {
    constexpr uint32_t BM = wave_rows(KSPLIT) * 32 * TM, BN = wave_cols(KSPLIT) * 32 * TN;
    Segs sg{};
    uint32_t cols = 0;
    for (uint32_t s = 0; s < kMaxPrefillGroup; ++s) {
        if (s < a.count) {
            sg.wf[s] = a.wf[s];
            sg.wsf[s] = a.wsf[s];
            sg.y[s] = a.y[s];
            sg.n[s] = a.n[s];
            sg.tile0[s] = cols;
            cols += (a.n[s] + BN - 1) / BN;
        } else {
            sg.tile0[s] = 0xffffffffu;
        }
    }
    dim3 grid(cols, (a.m + BM - 1) / BM);
    hipLaunchKernelGGL((prefill_kernel<A_FP8, TM, TN, U, Q, KSPLIT, RS, NKC>), grid, dim3(256), 0, a.stream, a.xf,
                       a.xsf, a.m, a.k, sg);
    return hipGetLastError();
}

// The deepest ring of at most D stages that the kernel's limits allow (D when none is smaller than 3).
template <bool A_FP8, int WM, int WN, int TM, int TN, int U, int D, int KH = 1>
constexpr int fit_depth() {
    if constexpr (D <= 2 || LdsGeo<A_FP8, WM, WN, TM, TN, U, D, KH>::ok) return D;
    else return fit_depth<A_FP8, WM, WN, TM, TN, U, D - 1, KH>();
}

template <bool A_FP8, int WM, int WN, int TM, int TN, int U, int D, int KH = 1, bool PP = false>
hipError_t go_lds(const PrefillArgs& a) {
    using G = LdsGeo<A_FP8, WM, WN, TM, TN, U, D, KH>;
    if constexpr (!G::ok) {
        return hipErrorNotSupported;
    } else {
        // each K part starts on a whole scale quad
        if (a.k % (256 * KH) != 0) return hipErrorNotSupported;
        Segs sg{};
        uint32_t cols = 0;
        for (uint32_t s = 0; s < kMaxPrefillGroup; ++s) {
            if (s < a.count) {
                sg.wf[s] = a.wf[s];
                sg.wsf[s] = a.wsf[s];
                sg.y[s] = a.y[s];
                sg.n[s] = a.n[s];
                sg.tile0[s] = cols;
                cols += (a.n[s] + G::BN - 1) / G::BN;
            } else {
                sg.tile0[s] = 0xffffffffu;
            }
        }
        dim3 grid(cols, (a.m + G::BM - 1) / G::BM);
        hipLaunchKernelGGL((prefill_lds_kernel<A_FP8, WM, WN, TM, TN, U, D, KH, PP>), grid, dim3(G::NT), 0, a.stream,
                           a.xf, a.xsf, a.m, a.k, sg);
        return hipGetLastError();
    }
}

// Wave tiles of TM x TN fragments with K in KS parts inside the workgroup,
// four k-steps in flight per wave; unrolled for the model's K sizes. Each
// part must start on a whole scale quad (four k-steps).
template <bool A_FP8, int TM, int TN, int KS>
hipError_t go_parts(const PrefillArgs& a) {
    if (a.k % (256 * KS) != 0) return hipErrorNotSupported;
    if (a.k == 4096) return go<A_FP8, TM, TN, 1, 4, KS, 2, 4096 / 64 / KS>(a);
    if (a.k == 12288) return go<A_FP8, TM, TN, 1, 4, KS, 2, 12288 / 64 / KS>(a);
    return go<A_FP8, TM, TN, 1, 4, KS, 2, 0>(a);
}

template <bool A_FP8>
hipError_t dispatch(const PrefillArgs& a, int cus) {
    if (a.tile_m != 0 && a.split_k >= 16) {
        // workgroup-shared operands (prefill_lds_kernel): split_k = 256 P +
        // 128 (KH - 1) + 16 U + D (K in KH parts of their own waves, stages of
        // U k-steps, a ring of D; P = 1: the two K halves in ping-pong, KH = 2
        // and (U, D) = (4, 2), (4, 3), (2, 3) or (2, 4) only), tile_m x tile_n
        // workgroup tiles; a ring too deep for the LDS is cut to the deepest
        // that fits
        if (a.split_k >= 512 || (a.split_k >= 256 && a.split_k < 384)) return hipErrorNotSupported;
        const bool pp = a.split_k >= 256;
        const uint32_t kh = (a.split_k & 128) ? 2 : 1, code = a.split_k % 128;
        const uint32_t u = code / 16, d = code % 16;
#define MX4_LDS_PP                                                                                       \
            if (pp) {                                                                                    \
                if (u == 4 && d == 2) return go_lds<A_FP8, WM_c, WN_c, TM_c, TN_c, 4, 2, 2, true>(a);      \
                if (u == 4 && d == 3)                                                                    \
                    return go_lds<A_FP8, WM_c, WN_c, TM_c, TN_c, 4,                                      \
                                  fit_depth<A_FP8, WM_c, WN_c, TM_c, TN_c, 4, 3, 2>(), 2, true>(a);       \
                if (u == 2 && d == 3)                                                                    \
                    return go_lds<A_FP8, WM_c, WN_c, TM_c, TN_c, 2,                                      \
                                  fit_depth<A_FP8, WM_c, WN_c, TM_c, TN_c, 2, 3, 2>(), 2, true>(a);       \
                if (u == 2 && d == 4)                                                                    \
                    return go_lds<A_FP8, WM_c, WN_c, TM_c, TN_c, 2,                                      \
                                  fit_depth<A_FP8, WM_c, WN_c, TM_c, TN_c, 2, 4, 2>(), 2, true>(a);       \
                return hipErrorNotSupported;                                                             \
            }
#define MX4_LDS_KH(KH_)                                                                                  \
            if (kh == KH_) {                                                                             \
                if (u == 4 && d == 2) return go_lds<A_FP8, WM_c, WN_c, TM_c, TN_c, 4, 2, KH_>(a);          \
                if (u == 4 && d == 3)                                                                    \
                    return go_lds<A_FP8, WM_c, WN_c, TM_c, TN_c, 4,                                      \
                                  fit_depth<A_FP8, WM_c, WN_c, TM_c, TN_c, 4, 3, KH_>(), KH_>(a);         \
                if (u == 2 && d == 3)                                                                    \
                    return go_lds<A_FP8, WM_c, WN_c, TM_c, TN_c, 2,                                      \
                                  fit_depth<A_FP8, WM_c, WN_c, TM_c, TN_c, 2, 3, KH_>(), KH_>(a);         \
                if (u == 2 && d == 4)                                                                    \
                    return go_lds<A_FP8, WM_c, WN_c, TM_c, TN_c, 2,                                      \
                                  fit_depth<A_FP8, WM_c, WN_c, TM_c, TN_c, 2, 4, KH_>(), KH_>(a);         \
                if (u == 2 && d == 5)                                                                    \
                    return go_lds<A_FP8, WM_c, WN_c, TM_c, TN_c, 2,                                      \
                                  fit_depth<A_FP8, WM_c, WN_c, TM_c, TN_c, 2, 5, KH_>(), KH_>(a);         \
                if (u == 2 && d == 8)                                                                    \
                    return go_lds<A_FP8, WM_c, WN_c, TM_c, TN_c, 2,                                      \
                                  fit_depth<A_FP8, WM_c, WN_c, TM_c, TN_c, 2, 8, KH_>(), KH_>(a);         \
                if (u == 4 && d == 5)                                                                    \
                    return go_lds<A_FP8, WM_c, WN_c, TM_c, TN_c, 4,                                      \
                                  fit_depth<A_FP8, WM_c, WN_c, TM_c, TN_c, 4, 5, KH_>(), KH_>(a);         \
            }
#define MX4_LDS(BM_, BN_, WM_, WN_, TM_, TN_)                                                           \
        if (a.tile_m == BM_ && a.tile_n == BN_) {                                                       \
            constexpr int WM_c = WM_, WN_c = WN_, TM_c = TM_, TN_c = TN_;                               \
            MX4_LDS_PP                                                                                  \
            MX4_LDS_KH(1)                                                                               \
            MX4_LDS_KH(2)                                                                               \
            return hipErrorNotSupported;                                                                \
        }
        MX4_LDS(128, 192, 2, 2, 2, 3)
        MX4_LDS(128, 128, 2, 2, 2, 2)
        MX4_LDS(64, 128, 2, 2, 1, 2)
        MX4_LDS(128, 64, 2, 2, 2, 1)
        MX4_LDS(64, 256, 1, 4, 2, 2)
        MX4_LDS(128, 96, 4, 1, 1, 3)
        MX4_LDS(64, 192, 2, 2, 1, 3)
        MX4_LDS(64, 64, 2, 2, 1, 1)
#undef MX4_LDS
#undef MX4_LDS_KH
#undef MX4_LDS_PP
        return hipErrorNotSupported;
    }
    if (a.tile_m != 0) {
        // tuning: one explicit instance. Workgroup tiles: 128 x 192 and
        // 128 x 128 over the full K; 64 x 128 with K halves inside it; wave
        // tiles of 128 x 96 in K halves (128 x 192) or of 128 x 64, 64 x 128,
        // 128 x 96 and 128 x 128 in K quarters.
        if (a.split_k == 2 && a.tile_m == 128 && a.tile_n == 192) return go_parts<A_FP8, 4, 3, 2>(a);
        if (a.split_k == 4) {
            if (a.tile_m == 128 && a.tile_n == 64) return go_parts<A_FP8, 4, 2, 4>(a);
            if (a.tile_m == 64 && a.tile_n == 128) return go_parts<A_FP8, 2, 4, 4>(a);
            if (a.tile_m == 128 && a.tile_n == 96) return go_parts<A_FP8, 4, 3, 4>(a);
            if (a.tile_m == 128 && a.tile_n == 128) return go_parts<A_FP8, 4, 4, 4>(a);
            return hipErrorNotSupported;
        }
        if (a.tile_m == 128 && a.tile_n == 192 && a.split_k == 1 && a.k % 512 == 0)
            return go<A_FP8, 2, 3, 2, 4, 1, 2, 0>(a);
        if (a.tile_m == 128 && a.tile_n == 128 && a.split_k == 1)
            return a.k % 512 == 0 ? go<A_FP8, 2, 2, 2, 4, 1, 2, 0>(a) : go<A_FP8, 2, 2, 2, 2, 1, 1, 0>(a);
        if (a.tile_m == 64 && a.tile_n == 128 && a.split_k == 2) {
            if (a.k == 4096) return go<A_FP8, 2, 2, 2, 4, 2, 2, 32>(a);
            if (a.k == 12288) return go<A_FP8, 2, 2, 2, 4, 2, 2, 96>(a);
            if (a.k % 512 == 0) return go<A_FP8, 2, 2, 2, 4, 2, 2, 0>(a);
        }
        return hipErrorNotSupported;
    }
    uint32_t ntot = 0;
    for (uint32_t s = 0; s < a.count; ++s) ntot += a.n[s];
    // Outside 384..512 rows (where the defaults below were tuned): the
    // ping-pong tile whose workgroups come closest to one full round of the
    // CUs without passing it, the larger tile on a tie (MX-FP8: not 128 x 64,
    // whose stages of 4 do not fit; 128 x 128 in stages of 2). Measured on
    // the 8B q / gate / down weights, cold: MXFP4 q at 128 / 256 / 1024 rows
    // 10.3 / 10.2 / 18.0 -> 8.7 / 8.8 / 13.9 us, gate at 128 / 256 17.6 /
    // 17.4 -> 11.3 / 13.8, down at 128 / 256 / 1024 25.1 / 24.7 / 47.0 ->
    // 21.5 / 21.9 / 32.4; MX-FP8 q 11.6 / 11.6 / 22.0 -> 9.7 / 9.7 / 19.0,
    // gate at 128 / 256 21.8 / 21.7 -> 13.8 / 19.1, down 30.3 / 29.9 / 56.3
    // -> 24.3 / 24.9 / 46.7; at 576 / 768 rows (128 x 128) MXFP4 q 16.1 /
    // 16.5 -> 12.1 / 12.6, down 39.6 / 40.1 -> 28.4 / 30.0, MX-FP8 q 18.8 /
    // 19.6 -> 16.4 / 17.2, down 48.0 / 48.8 -> 42.1 / 44.2. Where no tile
    // fits one round (gate at 576 and above), the rules and defaults below.
    const uint32_t nc = cus > 0 ? (uint32_t)cus : 256u;
    auto rounds = [&](uint32_t bm, uint32_t bn) {
        uint32_t cols = 0;
        for (uint32_t s = 0; s < a.count; ++s) cols += (a.n[s] + bn - 1) / bn;
        return (cols * ((a.m + bm - 1) / bm) + nc - 1) / nc;
    };
    if ((a.m < 384 || a.m > 512) && a.k % 512 == 0) {
        struct T { uint32_t bm, bn; };
        const T ts[] = {{128, 128}, {64, 128}, {128, 64}, {64, 64}};
        int sel = -1;
        uint32_t sel_wgs = 0;
        for (int i = 0; i < 4; ++i) {
            if (A_FP8 && i == 2) continue;
            uint32_t cols = 0;
            for (uint32_t s = 0; s < a.count; ++s) cols += (a.n[s] + ts[i].bn - 1) / ts[i].bn;
            const uint32_t wgs = cols * ((a.m + ts[i].bm - 1) / ts[i].bm);
            if (wgs <= nc && wgs > sel_wgs) {
                sel = i;
                sel_wgs = wgs;
            }
        }
        if constexpr (A_FP8) {
            switch (sel) {
                case 0: return go_lds<true, 2, 2, 2, 2, 2, fit_depth<true, 2, 2, 2, 2, 2, 3, 2>(), 2, true>(a);
                case 1: return go_lds<true, 2, 2, 1, 2, 4, 2, 2, true>(a);
                case 3: return go_lds<true, 2, 2, 1, 1, 4, 2, 2, true>(a);
                default: break;
            }
        } else {
            switch (sel) {
                case 0: return go_lds<false, 2, 2, 2, 2, 4, 2, 2, true>(a);
                case 1: return go_lds<false, 2, 2, 1, 2, 4, 2, 2, true>(a);
                case 2: return go_lds<false, 2, 2, 2, 1, 4, 2, 2, true>(a);
                case 3: return go_lds<false, 2, 2, 1, 1, 4, 2, 2, true>(a);
                default: break;
            }
        }
    }
    // Beyond 768 rows, where no tile fits one round, the 512-row tiles of q /
    // o and down (128 x 64 or 64 x 128: 192 operand rows per k-step) against
    // 128 x 128 (256 rows per k-step for twice the outputs): whichever needs
    // fewer rounds x rows per k-step. MXFP4 runs 128 x 128 over the whole K
    // in stages of 4, 2 deep, two workgroups per CU; MX-FP8 (twice the A
    // bytes) K halves in ping-pong. 8B, cold: MXFP4 q at 1536 / 2048 / 4096
    // rows 24.8 / 32.4 / 61.2 -> 19.7 / 23.8 / 45.0 us (ping-pong 23.8 / 26.4
    // / 49.3), down 62.8 / 81.3 / 155.5 -> 48.2 / 58.9 / 113.7 (ping-pong
    // 54.3 / 61.2 / 118.0); MX-FP8 q 30.8 / 38.9 / 74.4 -> 31.2 / 35.4 / 67.2,
    // down 78.7 / 102.5 / 195.8 -> 78.7 / 89.2 / 170.5 (one ring 15-20%
    // slower). (MX-FP8 q|k|v keeps its one-ring 64 x 128 tiles: 128 x 128
    // measured the same at 1024 and 2048 rows and slower at 1536.)
    if (a.m > 768 && ntot <= 4096 && (a.k == 4096 || a.k == 12288)) {
        const uint32_t dbm = (!A_FP8 && a.k == 4096) ? 128u : 64u;
        if (rounds(128, 128) * 256 < rounds(dbm, 192 - dbm) * 192) {
            if constexpr (A_FP8) return go_lds<true, 2, 2, 2, 2, 2, fit_depth<true, 2, 2, 2, 2, 2, 3, 2>(), 2, true>(a);
            else return go_lds<false, 2, 2, 2, 2, 4, 2>(a);
        }
    }
    // Qwen3-8B shapes (K = 4096, and 12288 for down), measured on MI355X at
    // M = 512 on cold weights, the alternatives timed in one process (split_k
    // code 256 P + 128 (KH - 1) + 16 U + D of the tuning call):
    //  q / o (4096 rows): K in two halves of their own four waves (two waves
    //  per SIMD) in ping-pong; MXFP4 on 128 x 64 tiles in stages of 4 k-steps,
    //  2 deep (10.9 -> 10.8 us against stages of 2, 4 deep, and 11.2-11.5
    //  against the same halves without ping-pong; 9.9 -> 9.0 us warm), MX-FP8
    //  on 64 x 128 tiles in stages of 4, 2 deep (12.9 -> 12.3 us against
    //  stages of 2, 4 deep, 14.1-14.3 without ping-pong);
    //  q|k|v (6144 rows): MXFP4 on 128 x 128 tiles, K halves in ping-pong,
    //  stages of 4, 2 deep (15.9-16.3 -> 13.6 us against 64 x 128 tiles over
    //  the whole K in stages of 2, 4 deep); MX-FP8 keeps 64 x 128 tiles over
    //  the whole K in stages of 4, 2 deep (18.2 us; ping-pong on 128 x 128
    //  tiles the same);
    //  gate|up (24576 rows), MXFP4: 128 x 192 tiles over the whole K in stages
    //  of 2, 3 deep, two workgroups per CU (36-44 us; with K halves in
    //  ping-pong a workgroup needs the LDS of a whole CU: 42-47 us);
    //  gate alone (12288 rows) and gate|up MX-FP8: 128 x 192 tiles, K halves
    //  in ping-pong, stages of 2, 3 deep (2 for MX-FP8, by the LDS): gate
    //  MXFP4 24.1-24.7 -> 21.3-23.7 us (warm 19.5-20.0 -> 20.5-20.7), MX-FP8
    //  31.8-32.7 -> 26.6-28.0 us; gate|up MX-FP8 60.5 -> 56.5 us, against 4 x
    //  3 wave tiles in K halves without LDS;
    //  down (4096 rows, K = 12288): 64 x 128 tiles, K halves in ping-pong,
    //  stages of 2, 4 deep; MXFP4 26.7-27.1 -> 25.3-25.4 us (warm 22.6-23.7
    //  -> 20.4-20.6) against 128 x 64 tiles the same way and 27.3-28.2 us
    //  against 4 x 2 wave tiles in K quarters; MX-FP8 33.5-33.6 -> 31.0-31.3
    //  us against 2 x 4 wave tiles in K quarters (three repetitions each).
    if (a.k == 4096 && ntot <= 4096) {
        if constexpr (A_FP8) return go_lds<true, 2, 2, 1, 2, 4, 2, 2, true>(a);
        else return go_lds<false, 2, 2, 2, 1, 4, 2, 2, true>(a);
    }
    if (a.k == 4096) {
        if (ntot <= 8192) {
            // MXFP4 q|k|v once its ping-pong tiles need more than one round:
            // the same tile over the whole K, two workgroups per CU (1024 /
            // 1536 / 2048 / 4096 rows 23.6 / 34.2 / 37.7 / 70.3 -> 20.4 / 33.9
            // / 37.3 / 64.5 us)
            if constexpr (A_FP8) return go_lds<true, 2, 2, 1, 2, 4, 2>(a);
            else if (rounds(128, 128) > 1) return go_lds<false, 2, 2, 2, 2, 4, 2>(a);
            else return go_lds<false, 2, 2, 2, 2, 4, 2, 2, true>(a);
        }
        if constexpr (!A_FP8) {
            // one ring, two workgroups per CU (72 KiB each; a ping-pong one
            // needs a whole CU): gate|up, and gate or up alone once its
            // 128 x 192 tiles need more than one round of CUs (gate at 768 /
            // 1024 / 1536 / 2048 / 4096 rows 35.0 / 39.4 / 55.4 / 72.9 / 140.5
            // -> 28.6 / 33.6 / 49.5 / 63.6 / 121.5 us; the same at 512)
            if (ntot >= 16384 || rounds(128, 192) > 1) return go_lds<false, 2, 2, 2, 3, 2, 3>(a);
        }
        return go_lds<A_FP8, 2, 2, 2, 3, 2, fit_depth<A_FP8, 2, 2, 2, 3, 2, 3, 2>(), 2, true>(a);
    }
    // other K: wide N takes 4 x 3 tiles per wave with K in halves (at K =
    // 4096 before the shared kernels: gate MXFP4 23.0 -> 21.9 us, MX-FP8 36.8
    // -> 27.6 us against 2 x 3 tiles over the full K); otherwise 2 x 2 tiles
    // with K split in two inside the workgroup, fully unrolled for the
    // model's K sizes (larger tiles and K quarters measured slower there)
    if (ntot >= 8192 && a.k % 512 == 0) return go_parts<A_FP8, 4, 3, 2>(a);
    if (a.k == 12288 && ntot <= 4096) return go_lds<A_FP8, 2, 2, 1, 2, 2, 4, 2, true>(a);
    if (a.k == 12288) return go<A_FP8, 2, 2, 2, 4, 2, 2, 96>(a);
    if (a.k % 512 == 0) return go<A_FP8, 2, 2, 2, 4, 2, 2, 0>(a);
    return go<A_FP8, 2, 2, 2, 2, 1, 1, 0>(a);
}

}  // namespace

bool prefill_supported(uint32_t m, uint32_t n, uint32_t k) {
    // fragment buffers are addressed with 32-bit offsets, and so is y over
    // the whole grid (workgroup tiles of at most 128 rows and 192 columns)
    const uint64_t mp = ((uint64_t)m + 31) / 32 * 32, np = ((uint64_t)n + 31) / 32 * 32;
    const uint64_t y_span = ((uint64_t)m + 128) * n * 4 + ((uint64_t)n + 192) * 4;
    return m >= 1 && n >= 1 && k % 256 == 0 && np * (k / 2) < (1ull << 31) && mp * k < (1ull << 31) &&
           y_span < (1ull << 31);
}

uint64_t fragment_bytes(uint32_t rows, uint32_t k, bool fp8) {
    return ((uint64_t)rows + 31) / 32 * 32 * k / (fp8 ? 1 : 2);
}

uint64_t fragment_scale_bytes(uint32_t rows, uint32_t k) { return ((uint64_t)rows + 31) / 32 * 32 * (k / 32); }

hipError_t launch_to_fragments(const uint8_t* codes, const uint8_t* scales, uint32_t rows, uint32_t k, bool fp8,
                               uint8_t* codes_f, uint8_t* scales_f, hipStream_t s) {
    const uint64_t chunks = fragment_bytes(rows, k, fp8) / 16, words = fragment_scale_bytes(rows, k) / 4;
    if (chunks == 0) return hipSuccess;
    if (fp8)
        hipLaunchKernelGGL(to_fragments_kernel<true>, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, s, codes,
                           rows, k, chunks, codes_f);
    else
        hipLaunchKernelGGL(to_fragments_kernel<false>, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, s,
                           codes, rows, k, chunks, codes_f);
    hipLaunchKernelGGL(scales_to_fragments_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s, scales,
                       rows, k, words, reinterpret_cast<uint32_t*>(scales_f));
    return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs& a, int cus) {
    if (a.count < 1 || a.count > kMaxPrefillGroup) return hipErrorNotSupported;
    for (uint32_t s = 0; s < a.count; ++s)
        if (!prefill_supported(a.m, a.n[s], a.k)) return hipErrorNotSupported;
    return a.fp8 ? dispatch<true>(a, cus) : dispatch<false>(a, cus);
}

}  // namespace mx4
