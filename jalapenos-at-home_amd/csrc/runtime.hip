// runtime.hip -- context, resident weights, dispatch and the C ABI (include/mx4.h).
//
// Native counterpart of the reference's Objective-C bridges:
//  * qwen_hip_* <- engine/src/metal.m:18-117 (per-call matmul with a weight
//    cache keyed by host pointer, synchronous round trip);
//  * mx4_*      <- engine/src/gpu.m:27-128 + engine/src/gpu.rs:225-237, :469-515
//    (resident weights, one stream, GPU-timed passes, M-based dispatch).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <list>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "mx4.h"
#include "mx4_kernels.h"

namespace {

thread_local std::string g_error;

mx4_status fail(mx4_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return st;
}

#define HIP_TRY(call)                                                                        \
    do {                                                                                     \
        hipError_t e_ = (call);                                                              \
        if (e_ != hipSuccess) return fail(MX4_ERR_DEVICE, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

struct CacheKey {
    const void* w;
    const void* scales;
    uint32_t rows, cols;
    bool operator==(const CacheKey& o) const {
        return w == o.w && scales == o.scales && rows == o.rows && cols == o.cols;
    }
};
struct CacheKeyHash {
    size_t operator()(const CacheKey& k) const {
        size_t h = std::hash<const void*>()(k.w);
        h ^= std::hash<const void*>()(k.scales) + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
        h ^= ((size_t)k.rows << 32 | k.cols) + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
        return h;
    }
};

constexpr uint64_t kDefaultCacheLimit = 64ull << 30;

}  // namespace

struct mx4_weight {
    mx4_context* ctx;
    uint32_t rows, cols;
    uint8_t* packed;
    uint8_t* scales;
    void* allocation;  // owned device memory, or nullptr when wrapped
    uint32_t min_scale, max_scale;
    // fragment-native copy for the block-scaled MFMA path (built on first use
    // or by mx4_weight_prepare_prefill): codes, then scales at frag_scales
    uint8_t* frag = nullptr;
    uint8_t* frag_scales = nullptr;
    // bf16 weight [rows][cols] (a Tensor::bf16 of the reference); packed and
    // scales are null for such a weight
    uint16_t* bf16 = nullptr;
    // false once mx4_weight_drop_stored freed the row-major layout (only the
    // matrix-core copy is left: prefill entry points only)
    bool stored = true;
};

struct mx4_pass {
    hipGraph_t graph;
    hipGraphExec_t exec;
    int device;
    mx4_context* ctx;  // null once the context is destroyed
};

struct CacheEntry {
    mx4_weight* w;
    uint64_t bytes;
    std::list<CacheKey>::iterator lru;
};

struct mx4_context {
    int device = 0;
    int cus = 256;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    uint32_t* flags = nullptr;  // device scratch: [0] bad flag, [1..2] min/max scale
    // per-call drop-in state
    std::unordered_map<CacheKey, CacheEntry, CacheKeyHash> cache;
    std::list<CacheKey> lru;
    uint64_t cache_bytes = 0, cache_limit = kDefaultCacheLimit;
    void* x_stage = nullptr;
    uint64_t x_cap = 0;
    void* y_stage = nullptr;
    uint64_t y_cap = 0;
    // pinned host bounce buffers of the drop-in (hipHostMalloc): the caller's
    // pageable x and y are copied through them with host memcpy, and the
    // device transfers run from and to page-locked memory
    void* x_pin = nullptr;
    uint64_t x_pin_cap = 0;
    void* y_pin = nullptr;
    uint64_t y_pin_cap = 0;
    // prefill workspace: requantized activations + their scales
    void* work = nullptr;
    uint64_t work_cap = 0;
    // greedy-argmax keys: one per workgroup of the fused lm_head GEMV, or one
    // per piece of a row split over several blocks by mx4_argmax_rows
    uint64_t* am_partial = nullptr;
    // logits of mx4_matmul_argmax when the caller does not want them
    void* logits = nullptr;
    uint64_t logits_cap = 0;
    // split-K skinny launches: partial tiles (1 KiB each) and per-tile
    // arrival counts (zero between launches); calls are ordered on `stream`
    float* split_part = nullptr;
    uint32_t* split_count = nullptr;
    // recorded passes alive on this context: a pass holds raw pointers to
    // `work` and `logits`, so while any is alive a buffer that has to grow
    // is retired (freed when the last pass is released) instead of freed
    std::unordered_set<mx4_pass*> passes;
    std::vector<void*> retired;
    // every weight handle made on this context and not yet released: the
    // handles belong to the caller, so mx4_destroy frees their device memory
    // and detaches them (ctx = null) instead of leaving them pointing here
    std::unordered_set<mx4_weight*> weights;
};

// Workspace of mx4_matmul_prefill_noalloc: the requantized activations in
// the fragment-native layout (codes, 256-byte aligned, then scales) after a
// 256-byte head holding the requantizer's non-finite flag. A file-scope device
// array: every GPU the library runs on holds its own copy until the process
// ends, and host code reaches it only through the address hipGetSymbolAddress
// returns for that device (the array's name is a host-side stand-in).
constexpr uint64_t kNoAllocScratchBytes = 8ull << 20;
constexpr uint64_t kNoAllocHead = 256;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr uint32_t kArgmaxPartials = 8192;
// Split-K partials: 32 MiB (the exact GEMM: four K slices of a 512 x 4096
// f32 output); the skinny kernel's split takes at most 4096 tiles of 1 KiB
// of it (four K slices of up to 8192 rows at 32 tokens).
constexpr uint64_t kSplitPartBytes = 32ull << 20;
constexpr uint32_t kSplitPartTiles = 4096;
constexpr uint32_t kSplitCounts = 4096;

namespace mx4 {
hipError_t launch_fill_u32(uint32_t* p, uint32_t count, uint32_t value, hipStream_t s);
}

namespace {

// Device address of `scratch` on each device, looked up once per device (by
// the first mx4_create on it, with that device current).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
uint8_t* g_scratch_ptr[kMaxDevices] = {};

hipError_t scratch_lookup(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[device]) return hipSuccess;
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = static_cast<uint8_t*>(ptr);
    return hipSuccess;
}

uint8_t* scratch_of(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    return g_scratch_ptr[device];
}

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

bool is_gfx950(int dev) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return false;
    return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
}

// Grow a context buffer to `need` bytes. A buffer that recorded passes may
// read (`pass_visible`: the prefill workspace, the argmax logits) is kept
// alive until every pass of the context is released, so replaying an older
// pass never touches freed memory.
mx4_status ensure_buffer(mx4_context* ctx, void** buf, uint64_t* cap, uint64_t need, bool pass_visible = false) {
    if (need <= *cap) return MX4_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        return fail(MX4_ERR_NO_MEMORY,
                    "workspace of %llu bytes needed while recording a pass; reserve it first (mx4_reserve_prefill)",
                    (unsigned long long)need);
    if (*buf) {
        HIP_TRY(hipStreamSynchronize(ctx->stream));
        if (pass_visible && !ctx->passes.empty()) {
            ctx->retired.push_back(*buf);
        } else {
            HIP_TRY(hipFree(*buf));
        }
        *buf = nullptr;
        *cap = 0;
    }
    uint64_t size = need < (1u << 20) ? (1u << 20) : need;
    if (hipMalloc(buf, size) != hipSuccess) {
        *buf = nullptr;
        return fail(MX4_ERR_NO_MEMORY, "could not allocate %llu bytes of device memory",
                    (unsigned long long)size);
    }
    *cap = size;
    return MX4_OK;
}

// Grow a pinned host buffer of the drop-in (the previous transfer through it
// has completed: every drop-in call synchronizes before returning).
mx4_status ensure_pinned(mx4_context* ctx, void** buf, uint64_t* cap, uint64_t need) {
    (void)ctx;
    if (need <= *cap) return MX4_OK;
    if (*buf) HIP_TRY(hipHostFree(*buf));
    *buf = nullptr;
    *cap = 0;
    uint64_t size = need < (1u << 20) ? (1u << 20) : need;
    if (hipHostMalloc(buf, size, hipHostMallocDefault) != hipSuccess) {
        *buf = nullptr;
        return fail(MX4_ERR_NO_MEMORY, "could not allocate %llu bytes of pinned host memory",
                    (unsigned long long)size);
    }
    *cap = size;
    return MX4_OK;
}

// requantized activations in the fragment-native layout (FP4 or FP8 codes,
// 256-byte aligned) followed by their scales
uint64_t prefill_workspace_bytes(uint64_t m, uint64_t cols, bool fp8) {
    const uint64_t qbytes = mx4::fragment_bytes((uint32_t)m, (uint32_t)cols, fp8);
    return ((qbytes + 255) & ~255ull) + mx4::fragment_scale_bytes((uint32_t)m, (uint32_t)cols);
}

mx4::PrefillArgs prefill_args(mx4_context* ctx, const mx4_weight* w, const uint8_t* xf, const uint8_t* xsf,
                              float* y, uint32_t m, bool fp8) {
    mx4::PrefillArgs a{};
    a.wf[0] = w->frag;
    a.wsf[0] = w->frag_scales;
    a.y[0] = y;
    a.n[0] = w->rows;
    a.count = 1;
    a.xf = xf;
    a.xsf = xsf;
    a.m = m;
    a.k = w->cols;
    a.fp8 = fp8;
    a.stream = ctx->stream;
    return a;
}

// The weight's fragment-native copy: built once, outside any recorded pass.
mx4_status prepare_fragments(mx4_context* ctx, mx4_weight* w) {
    if (w->frag) return MX4_OK;
    if (!w->stored) return fail(MX4_ERR_UNSUPPORTED, "the weight has neither its stored layout nor its matrix-core copy");
    if (w->bf16) return fail(MX4_ERR_UNSUPPORTED, "the block-scaled MFMA path takes MXFP4 weights");
    if (w->cols % 256 != 0) return fail(MX4_ERR_UNSUPPORTED, "block-scaled MFMA path needs K %% 256 == 0");
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        return fail(MX4_ERR_NO_MEMORY,
                    "the weight's MFMA layout is built on first use; call mx4_weight_prepare_prefill before recording");
    const uint64_t cbytes = (mx4::fragment_bytes(w->rows, w->cols, false) + 255) & ~255ull;
    const uint64_t total = cbytes + mx4::fragment_scale_bytes(w->rows, w->cols);
    void* p = nullptr;
    if (hipMalloc(&p, total) != hipSuccess)
        return fail(MX4_ERR_NO_MEMORY, "could not allocate %llu bytes of device memory", (unsigned long long)total);
    uint8_t* f = static_cast<uint8_t*>(p);
    hipError_t e = mx4::launch_to_fragments(w->packed, w->scales, w->rows, w->cols, false, f, f + cbytes, ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return fail(MX4_ERR_DEVICE, "layout launch failed: %s", hipGetErrorString(e));
    }
    w->frag = f;
    w->frag_scales = f + cbytes;
    return MX4_OK;
}

mx4_status check_matmul_args(mx4_context* ctx, const void* x, mx4_dtype xt, uint32_t m,
                             const mx4_weight* w, const float* y) {
    if (!ctx) return fail(MX4_ERR_ARGUMENT, "null context");
    if (!x || !w || !y) return fail(MX4_ERR_ARGUMENT, "null x, weight or y");
    if (xt != MX4_F32 && xt != MX4_BF16) return fail(MX4_ERR_ARGUMENT, "bad activation dtype %d", (int)xt);
    if (m == 0) return fail(MX4_ERR_ARGUMENT, "m must be at least 1");
    if (((uintptr_t)x & 15) != 0) return fail(MX4_ERR_ARGUMENT, "x must be 16-byte aligned");
    if (((uintptr_t)y & 3) != 0) return fail(MX4_ERR_ARGUMENT, "y must be 4-byte aligned");
    if (!w->ctx) return fail(MX4_ERR_ARGUMENT, "the weight's context was destroyed");
    if (w->ctx != ctx) return fail(MX4_ERR_ARGUMENT, "weight belongs to another context");
    return MX4_OK;
}

// The fast kernels fold the E8M0 scale into the E2M1 converter and the
// per-block sums; that is exact for scale bytes 2..252 (every byte the
// reference quantizer emits for a nonzero block; python/quantize_mxfp4.py
// never produces more than 252). Other bytes go to the exact generic kernel.
bool scales_foldable(const mx4_weight* w) { return w->min_scale >= 2 && w->max_scale <= 252; }

// Entry points that read the weight's stored row-major layout refuse a weight
// whose layout was dropped (mx4_weight_drop_stored).
mx4_status need_stored(const mx4_weight* w) {
    if (!w->stored)
        return fail(MX4_ERR_UNSUPPORTED,
                    "the weight's stored layout was dropped; only the prefill entry points take it");
    return MX4_OK;
}

mx4_status run_matmul(mx4_context* ctx, const void* x, mx4_dtype xt, uint32_t m, const mx4_weight* w,
                      float* y, mx4_path path) {
    if (need_stored(w) != MX4_OK) return MX4_ERR_UNSUPPORTED;
    if (w->bf16) {
        // engine/src/lib.rs:255 `None` arm: one exact kernel for every M
        if (path != MX4_PATH_AUTO && path != MX4_PATH_GENERIC)
            return fail(MX4_ERR_UNSUPPORTED, "bf16 weights run on the generic path only");
        hipError_t e = mx4::launch_bf16_matmul(w->bf16, x, xt == MX4_BF16, y, m, w->rows, w->cols, ctx->stream);
        if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString(e));
        return MX4_OK;
    }
    mx4::GemvArgs a{w->packed, w->scales, x, y, m, w->rows, w->cols, xt == MX4_BF16, ctx->stream};
    if (path == MX4_PATH_AUTO) {
        // 2..4 bf16 token rows: the few-token GEMV where it measured faster
        // than the skinny kernel on the Qwen3 1.7B/8B shapes: 2 tokens below
        // vocabulary-sized weights, and 3-4 tokens on 1024-row weights at
        // K >= 4096 (8B k/v)
        const bool tokens = mx4::gemv_mt_supported(m, w->cols, xt == MX4_BF16) &&
                            ((m == 2 && w->rows < 65536) || (w->rows <= 1024 && w->cols >= 4096));
        if (((m == 1 && mx4::gemv_m1_supported(w->cols)) || tokens) && scales_foldable(w))
            path = MX4_PATH_GEMV;
        else if (m >= 2 && mx4::skinny_supported(m, w->cols) && scales_foldable(w))
            path = MX4_PATH_SKINNY;
        else if (m > 32 && mx4::gemm_exact_supported(m, w->rows, w->cols, xt == MX4_BF16) && scales_foldable(w))
            path = MX4_PATH_GEMM;
        else
            path = MX4_PATH_GENERIC;
    }
    hipError_t e;
    switch (path) {
        case MX4_PATH_GEMV:
            if (!(m == 1 && mx4::gemv_m1_supported(w->cols)) && !mx4::gemv_mt_supported(m, w->cols, xt == MX4_BF16))
                return fail(MX4_ERR_UNSUPPORTED,
                            "GEMV path needs m == 1 and K/32 in {64,128,192,256,384}, or 2 <= m <= 4 with bf16 x "
                            "and K in {2048, 4096, 6144, 8192, 12288}");
            if (!scales_foldable(w))
                return fail(MX4_ERR_UNSUPPORTED, "GEMV path folds scales into the converter; scale bytes outside 2..252 need GENERIC");
            e = m == 1 ? mx4::launch_gemv_m1(a, ctx->cus) : mx4::launch_gemv_mt(a, ctx->cus);
            break;
        case MX4_PATH_SKINNY:
            if (!mx4::skinny_supported(m, w->cols))
                return fail(MX4_ERR_UNSUPPORTED, "skinny path needs 1 <= m <= 32 and K in {2048, 4096, 6144, 8192, 12288}");
            if (!scales_foldable(w))
                return fail(MX4_ERR_UNSUPPORTED, "skinny path folds scales into bf16; scale bytes outside 2..252 need GENERIC");
            e = mx4::launch_skinny(a, ctx->cus, {ctx->split_part, ctx->split_count, kSplitPartTiles, kSplitCounts});
            break;
        case MX4_PATH_GEMM:
            if (!mx4::gemm_exact_supported(m, w->rows, w->cols, xt == MX4_BF16))
                return fail(MX4_ERR_UNSUPPORTED, "GEMM path needs K %% 128 == 0 and operands under 2 GiB");
            if (!scales_foldable(w))
                return fail(MX4_ERR_UNSUPPORTED, "GEMM path folds scales into bf16; scale bytes outside 2..252 need GENERIC");
            e = mx4::launch_gemm_exact(a, ctx->cus, nullptr, ctx->split_part, kSplitPartBytes);
            break;
        case MX4_PATH_GENERIC:
            e = mx4::launch_gemv_generic(a);
            break;
        default:
            return fail(MX4_ERR_ARGUMENT, "bad path %d", (int)path);
    }
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status new_weight(mx4_context* ctx, uint32_t rows, uint32_t cols, mx4_weight** out) {
    mx4_weight* w = new (std::nothrow) mx4_weight{};
    if (!w) return fail(MX4_ERR_NO_MEMORY, "out of host memory");
    if (!ctx->weights.insert(w).second) {
        delete w;
        return fail(MX4_ERR_NO_MEMORY, "out of host memory");
    }
    w->ctx = ctx;
    w->rows = rows;
    w->cols = cols;
    *out = w;
    return MX4_OK;
}

void cache_evict(mx4_context* ctx) {
    while (ctx->cache_bytes > ctx->cache_limit && !ctx->lru.empty()) {
        CacheKey k = ctx->lru.back();
        ctx->lru.pop_back();
        auto it = ctx->cache.find(k);
        if (it != ctx->cache.end()) {
            ctx->cache_bytes -= it->second.bytes;
            (void)hipStreamSynchronize(ctx->stream);
            mx4_weight_release(it->second.w);
            ctx->cache.erase(it);
        }
    }
}

}  // namespace

extern "C" {

const char* mx4_last_error(void) { return g_error.c_str(); }

int mx4_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    int c = 0;
    for (int i = 0; i < n; ++i) c += is_gfx950(i) ? 1 : 0;
    return c;
}

mx4_status mx4_compute_units(const mx4_context* ctx, int* cus) {
    if (!ctx || !cus) return fail(MX4_ERR_ARGUMENT, "null argument");
    *cus = ctx->cus;
    return MX4_OK;
}

mx4_status mx4_validate(uint64_t rows, uint64_t cols, uint64_t packed_len, const uint8_t* scales,
                        uint64_t scales_len) {
    // engine/src/mxfp4.rs:11-25
    if (rows == 0 || cols == 0 || cols % 32 != 0)
        return fail(MX4_ERR_SHAPE, "MXFP4 requires nonempty rows with a width divisible by 32");
    if (rows > UINT64_MAX / cols) return fail(MX4_ERR_TOO_LARGE, "tensor is too large");
    const uint64_t elements = rows * cols;
    if (packed_len != elements / 2 || scales_len != elements / 32)
        return fail(MX4_ERR_LENGTH, "MXFP4 data length does not match shape");
    if (scales_len && !scales) return fail(MX4_ERR_ARGUMENT, "null scales");
    if (std::memchr(scales, 255, scales_len)) return fail(MX4_ERR_NAN_SCALE, "MXFP4 checkpoint contains a NaN scale");
    return MX4_OK;
}

mx4_status mx4_create(int device, mx4_context** out) {
    if (!out) return fail(MX4_ERR_ARGUMENT, "null output pointer");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(MX4_ERR_DEVICE, "no HIP device available");
    if (device < 0 || device >= n) return fail(MX4_ERR_ARGUMENT, "device %d out of range (%d devices)", device, n);
    if (!is_gfx950(device)) return fail(MX4_ERR_DEVICE, "device %d is not gfx950 (MI355X)", device);
    DeviceGuard g(device);
    mx4_context* ctx = new (std::nothrow) mx4_context();
    if (!ctx) return fail(MX4_ERR_NO_MEMORY, "out of host memory");
    ctx->device = device;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) ctx->cus = prop.multiProcessorCount;
    if (hipStreamCreateWithFlags(&ctx->own, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&ctx->ev0) != hipSuccess || hipEventCreate(&ctx->ev1) != hipSuccess ||
        hipMalloc((void**)&ctx->flags, 256) != hipSuccess ||
        hipMalloc((void**)&ctx->am_partial, kArgmaxPartials * sizeof(uint64_t)) != hipSuccess ||
        hipMalloc((void**)&ctx->split_part, (size_t)kSplitPartBytes) != hipSuccess ||
        hipMalloc((void**)&ctx->split_count, kSplitCounts * sizeof(uint32_t)) != hipSuccess ||
        hipMemsetAsync(ctx->split_count, 0, kSplitCounts * sizeof(uint32_t), ctx->own) != hipSuccess ||
        hipStreamSynchronize(ctx->own) != hipSuccess) {
        mx4_destroy(ctx);
        return fail(MX4_ERR_DEVICE, "could not create stream, events or scratch on device %d", device);
    }
    // the no-alloc entry point's device workspace on this device
    const hipError_t se = scratch_lookup(device);
    if (se != hipSuccess) {
        mx4_destroy(ctx);
        return fail(MX4_ERR_DEVICE, "hipGetSymbolAddress(scratch) failed on device %d: %s", device,
                    hipGetErrorString(se));
    }
    ctx->stream = ctx->own;
    *out = ctx;
    return MX4_OK;
}

void mx4_destroy(mx4_context* ctx) {
    if (!ctx) return;
    DeviceGuard g(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (auto& kv : ctx->cache) mx4_weight_release(kv.second.w);
    ctx->cache.clear();
    // the caller's weights outlive the context as empty handles: their device
    // memory goes now, and a later mx4_weight_release only deletes the handle
    for (mx4_weight* w : ctx->weights) {
        if (w->allocation) (void)hipFree(w->allocation);
        if (w->frag) (void)hipFree(w->frag);
        w->ctx = nullptr;
        w->allocation = nullptr;
        w->frag = w->frag_scales = nullptr;
        w->packed = w->scales = nullptr;
        w->bf16 = nullptr;
        w->stored = false;
    }
    ctx->weights.clear();
    for (mx4_pass* p : ctx->passes) p->ctx = nullptr;
    for (void* b : ctx->retired) (void)hipFree(b);
    if (ctx->x_stage) (void)hipFree(ctx->x_stage);
    if (ctx->y_stage) (void)hipFree(ctx->y_stage);
    if (ctx->x_pin) (void)hipHostFree(ctx->x_pin);
    if (ctx->y_pin) (void)hipHostFree(ctx->y_pin);
    if (ctx->work) (void)hipFree(ctx->work);
    if (ctx->flags) (void)hipFree(ctx->flags);
    if (ctx->am_partial) (void)hipFree(ctx->am_partial);
    if (ctx->split_part) (void)hipFree(ctx->split_part);
    if (ctx->split_count) (void)hipFree(ctx->split_count);
    if (ctx->logits) (void)hipFree(ctx->logits);
    if (ctx->ev0) (void)hipEventDestroy(ctx->ev0);
    if (ctx->ev1) (void)hipEventDestroy(ctx->ev1);
    if (ctx->own) (void)hipStreamDestroy(ctx->own);
    delete ctx;
}

mx4_status mx4_set_stream(mx4_context* ctx, void* hip_stream) {
    if (!ctx) return fail(MX4_ERR_ARGUMENT, "null context");
    ctx->stream = hip_stream ? static_cast<hipStream_t>(hip_stream) : ctx->own;
    return MX4_OK;
}

void* mx4_get_stream(mx4_context* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

mx4_status mx4_synchronize(mx4_context* ctx) {
    if (!ctx) return fail(MX4_ERR_ARGUMENT, "null context");
    DeviceGuard g(ctx->device);
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return MX4_OK;
}

mx4_status mx4_malloc(mx4_context* ctx, uint64_t bytes, void** dev) {
    if (!ctx || !dev) return fail(MX4_ERR_ARGUMENT, "null argument");
    *dev = nullptr;
    if (bytes == 0) return fail(MX4_ERR_ARGUMENT, "zero-byte allocation");
    DeviceGuard g(ctx->device);
    if (hipMalloc(dev, bytes) != hipSuccess) {
        *dev = nullptr;
        return fail(MX4_ERR_NO_MEMORY, "could not allocate %llu bytes", (unsigned long long)bytes);
    }
    return MX4_OK;
}

mx4_status mx4_free(mx4_context* ctx, void* dev) {
    if (!ctx) return fail(MX4_ERR_ARGUMENT, "null context");
    if (!dev) return MX4_OK;
    DeviceGuard g(ctx->device);
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    HIP_TRY(hipFree(dev));
    return MX4_OK;
}

mx4_status mx4_upload(mx4_context* ctx, void* dst, const void* src, uint64_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (!bytes) return MX4_OK;
    DeviceGuard g(ctx->device);
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return MX4_OK;
}

mx4_status mx4_download(mx4_context* ctx, void* dst, const void* src, uint64_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (!bytes) return MX4_OK;
    DeviceGuard g(ctx->device);
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return MX4_OK;
}

mx4_status mx4_copy(mx4_context* ctx, void* dst, const void* src, uint64_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (!bytes) return MX4_OK;
    DeviceGuard g(ctx->device);
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return MX4_OK;
}

mx4_status mx4_weight_upload(mx4_context* ctx, const uint8_t* packed, const uint8_t* scales, uint32_t rows,
                             uint32_t cols, mx4_weight** out) {
    if (!ctx || !out || !packed || !scales) return fail(MX4_ERR_ARGUMENT, "null argument");
    *out = nullptr;
    const uint64_t elements = (uint64_t)rows * cols;
    mx4_status st = mx4_validate(rows, cols, elements / 2, scales, elements / 32);
    if (st != MX4_OK) return st;
    uint32_t lo = 255, hi = 0;
    for (uint64_t i = 0; i < elements / 32; ++i) {
        lo = scales[i] < lo ? scales[i] : lo;
        hi = scales[i] > hi ? scales[i] : hi;
    }
    DeviceGuard g(ctx->device);
    const uint64_t pbytes = elements / 2, sbytes = elements / 32;
    const uint64_t soff = (pbytes + 255) & ~255ull;
    void* mem = nullptr;
    if (hipMalloc(&mem, soff + sbytes) != hipSuccess)
        return fail(MX4_ERR_NO_MEMORY, "could not allocate %llu bytes for a weight",
                    (unsigned long long)(soff + sbytes));
    uint8_t* base = static_cast<uint8_t*>(mem);
    if (hipMemcpyAsync(base, packed, pbytes, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
        hipMemcpyAsync(base + soff, scales, sbytes, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
        (void)hipFree(mem);
        return fail(MX4_ERR_DEVICE, "weight upload failed");
    }
    mx4_weight* w = nullptr;
    st = new_weight(ctx, rows, cols, &w);
    if (st != MX4_OK) {
        (void)hipFree(mem);
        return st;
    }
    w->allocation = mem;
    w->packed = base;
    w->scales = base + soff;
    w->min_scale = lo;
    w->max_scale = hi;
    *out = w;
    return MX4_OK;
}

mx4_status mx4_weight_wrap(mx4_context* ctx, const uint8_t* packed_dev, const uint8_t* scales_dev, uint32_t rows,
                           uint32_t cols, mx4_weight** out) {
    if (!ctx || !out || !packed_dev || !scales_dev) return fail(MX4_ERR_ARGUMENT, "null argument");
    *out = nullptr;
    if (rows == 0 || cols == 0 || cols % 32 != 0)
        return fail(MX4_ERR_SHAPE, "MXFP4 requires nonempty rows with a width divisible by 32");
    if (((uintptr_t)packed_dev & 15) != 0) return fail(MX4_ERR_ARGUMENT, "packed data must be 16-byte aligned");
    DeviceGuard g(ctx->device);
    const uint64_t sbytes = (uint64_t)rows * cols / 32;
    HIP_TRY(mx4::launch_fill_u32(ctx->flags + 1, 2, 0, ctx->stream));
    HIP_TRY(mx4::launch_fill_u32(ctx->flags + 1, 1, 255, ctx->stream));
    HIP_TRY(mx4::launch_min_max_scale(scales_dev, sbytes, ctx->flags + 1, ctx->stream));
    uint32_t mm[2];
    HIP_TRY(hipMemcpyAsync(mm, ctx->flags + 1, 8, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    if (mm[1] == 255) return fail(MX4_ERR_NAN_SCALE, "MXFP4 checkpoint contains a NaN scale");
    mx4_weight* w = nullptr;
    mx4_status st = new_weight(ctx, rows, cols, &w);
    if (st != MX4_OK) return st;
    w->packed = const_cast<uint8_t*>(packed_dev);
    w->scales = const_cast<uint8_t*>(scales_dev);
    w->min_scale = mm[0];
    w->max_scale = mm[1];
    *out = w;
    return MX4_OK;
}

void mx4_weight_release(mx4_weight* w) {
    if (!w) return;
    // a weight whose context was destroyed holds no device memory any more
    if (w->ctx) {
        if (w->allocation || w->frag) {
            DeviceGuard g(w->ctx->device);
            (void)hipStreamSynchronize(w->ctx->stream);
            if (w->allocation) (void)hipFree(w->allocation);
            if (w->frag) (void)hipFree(w->frag);
        }
        w->ctx->weights.erase(w);
    }
    delete w;
}

mx4_status mx4_weight_prepare_prefill(mx4_weight* w) {
    if (!w) return fail(MX4_ERR_ARGUMENT, "null weight");
    if (!w->ctx) return fail(MX4_ERR_ARGUMENT, "the weight's context was destroyed");
    DeviceGuard g(w->ctx->device);
    return prepare_fragments(w->ctx, w);
}

mx4_status mx4_weight_upload_bf16(mx4_context* ctx, const uint16_t* data, uint32_t rows, uint32_t cols,
                                  mx4_weight** out) {
    if (!ctx || !out || !data) return fail(MX4_ERR_ARGUMENT, "null argument");
    *out = nullptr;
    if (rows == 0 || cols == 0) return fail(MX4_ERR_SHAPE, "empty weight");
    const uint64_t bytes = (uint64_t)rows * cols * 2;
    DeviceGuard g(ctx->device);
    void* mem = nullptr;
    if (hipMalloc(&mem, bytes) != hipSuccess)
        return fail(MX4_ERR_NO_MEMORY, "could not allocate %llu bytes for a weight", (unsigned long long)bytes);
    if (hipMemcpyAsync(mem, data, bytes, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
        (void)hipFree(mem);
        return fail(MX4_ERR_DEVICE, "weight upload failed");
    }
    mx4_weight* w = nullptr;
    mx4_status st = new_weight(ctx, rows, cols, &w);
    if (st != MX4_OK) {
        (void)hipFree(mem);
        return st;
    }
    w->allocation = mem;
    w->bf16 = static_cast<uint16_t*>(mem);
    *out = w;
    return MX4_OK;
}

mx4_status mx4_weight_info(const mx4_weight* w, uint32_t* rows, uint32_t* cols, const uint8_t** packed_dev,
                           const uint8_t** scales_dev) {
    if (!w) return fail(MX4_ERR_ARGUMENT, "null weight");
    if (!w->ctx) return fail(MX4_ERR_ARGUMENT, "the weight's context was destroyed");
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    if (packed_dev) *packed_dev = w->stored ? w->packed : nullptr;
    if (scales_dev) *scales_dev = w->stored ? w->scales : nullptr;
    return MX4_OK;
}

mx4_status mx4_weight_footprint(const mx4_weight* w, uint64_t* stored_bytes, uint64_t* matrix_core_bytes) {
    if (!w) return fail(MX4_ERR_ARGUMENT, "null weight");
    if (!w->ctx) return fail(MX4_ERR_ARGUMENT, "the weight's context was destroyed");
    const uint64_t e = (uint64_t)w->rows * w->cols;
    if (stored_bytes) *stored_bytes = !w->stored ? 0 : (w->bf16 ? e * 2 : e / 2 + e / 32);
    if (matrix_core_bytes)
        *matrix_core_bytes = !w->frag ? 0
                                      : ((mx4::fragment_bytes(w->rows, w->cols, false) + 255) & ~255ull) +
                                            mx4::fragment_scale_bytes(w->rows, w->cols);
    return MX4_OK;
}

mx4_status mx4_weight_release_prefill(mx4_weight* w) {
    if (!w) return fail(MX4_ERR_ARGUMENT, "null weight");
    if (!w->ctx) return fail(MX4_ERR_ARGUMENT, "the weight's context was destroyed");
    if (!w->frag) return MX4_OK;
    if (!w->stored) return fail(MX4_ERR_UNSUPPORTED, "the matrix-core copy is the weight's only layout");
    if (!w->ctx->passes.empty())
        return fail(MX4_ERR_UNSUPPORTED, "a recorded pass of the context may read this layout; release the passes first");
    DeviceGuard g(w->ctx->device);
    HIP_TRY(hipStreamSynchronize(w->ctx->stream));
    HIP_TRY(hipFree(w->frag));
    w->frag = nullptr;
    w->frag_scales = nullptr;
    return MX4_OK;
}

mx4_status mx4_weight_drop_stored(mx4_weight* w) {
    if (!w) return fail(MX4_ERR_ARGUMENT, "null weight");
    if (!w->ctx) return fail(MX4_ERR_ARGUMENT, "the weight's context was destroyed");
    if (!w->stored) return MX4_OK;
    if (w->bf16) return fail(MX4_ERR_UNSUPPORTED, "a bf16 weight has no matrix-core copy");
    if (!w->allocation) return fail(MX4_ERR_UNSUPPORTED, "a wrapped weight's memory belongs to the caller");
    if (!w->ctx->passes.empty())
        return fail(MX4_ERR_UNSUPPORTED, "a recorded pass of the context may read this layout; release the passes first");
    DeviceGuard g(w->ctx->device);
    mx4_status st = prepare_fragments(w->ctx, w);
    if (st != MX4_OK) return st;
    HIP_TRY(hipStreamSynchronize(w->ctx->stream));
    HIP_TRY(hipFree(w->allocation));
    w->allocation = nullptr;
    w->packed = nullptr;
    w->scales = nullptr;
    w->stored = false;
    return MX4_OK;
}

mx4_status mx4_matmul_path(mx4_context* ctx, const void* x, mx4_dtype xt, uint32_t m, const mx4_weight* w,
                           float* y, mx4_path path) {
    mx4_status st = check_matmul_args(ctx, x, xt, m, w, y);
    if (st != MX4_OK) return st;
    if (path == MX4_PATH_PREFILL) return fail(MX4_ERR_ARGUMENT, "use mx4_matmul_prefill for the MFMA path");
    DeviceGuard g(ctx->device);
    return run_matmul(ctx, x, xt, m, w, y, path);
}

mx4_status mx4_matmul(mx4_context* ctx, const void* x, mx4_dtype xt, uint32_t m, const mx4_weight* w, float* y) {
    return mx4_matmul_path(ctx, x, xt, m, w, y, MX4_PATH_AUTO);
}

mx4_status mx4_matmul_group(mx4_context* ctx, const void* x, mx4_dtype xt, uint32_t m, const mx4_weight* const* w,
                            float* const* y, uint32_t count) {
    if (!ctx || !w || !y) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (count < 1 || count > 4) return fail(MX4_ERR_ARGUMENT, "a group holds 1 to 4 weights");
    for (uint32_t i = 0; i < count; ++i) {
        mx4_status st = check_matmul_args(ctx, x, xt, m, w[i], y[i]);
        if (st != MX4_OK) return fail(st, "weight %u: %s", i, g_error.c_str());
        if (w[i]->cols != w[0]->cols) return fail(MX4_ERR_SHAPE, "grouped weights must share their width");
        if (need_stored(w[i]) != MX4_OK) return MX4_ERR_UNSUPPORTED;
    }
    DeviceGuard g(ctx->device);
    bool foldable = true;
    for (uint32_t i = 0; i < count; ++i) foldable &= scales_foldable(w[i]);
    if (m == 1 && mx4::gemv_m1_supported(w[0]->cols) && foldable) {
        mx4::GemvGroup gg{};
        gg.count = count;
        gg.k = w[0]->cols;
        gg.x = x;
        gg.x_bf16 = xt == MX4_BF16;
        gg.stream = ctx->stream;
        for (uint32_t i = 0; i < count; ++i) {
            gg.packed[i] = w[i]->packed;
            gg.scales[i] = w[i]->scales;
            gg.y[i] = y[i];
            gg.n[i] = w[i]->rows;
        }
        hipError_t e = mx4::launch_gemv_m1_group(gg, ctx->cus, nullptr);
        if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString(e));
        return MX4_OK;
    }
    // 2..32 token rows (a speculative verify step): one launch of the
    // few-token GEMV or the skinny kernel over all the weights' rows, chosen
    // as mx4_matmul chooses for one weight of the group's total rows
    bool stored = true;
    uint32_t total = 0;
    for (uint32_t i = 0; i < count; ++i) {
        stored &= w[i]->bf16 == nullptr;
        total += w[i]->rows;
    }
    const uint32_t k = w[0]->cols;
    const bool tokens = mx4::gemv_mt_supported(m, k, xt == MX4_BF16) &&
                        ((m == 2 && total < 65536) || (total <= 1024 && k >= 4096));
    const bool skinny = !tokens && m >= 2 && mx4::skinny_supported(m, k);
    if (count > 1 && stored && foldable && (tokens || skinny)) {
        mx4::GemvGroup gg{};
        gg.count = count;
        gg.k = k;
        gg.x = x;
        gg.x_bf16 = xt == MX4_BF16;
        gg.stream = ctx->stream;
        for (uint32_t i = 0; i < count; ++i) {
            gg.packed[i] = w[i]->packed;
            gg.scales[i] = w[i]->scales;
            gg.y[i] = y[i];
            gg.n[i] = w[i]->rows;
        }
        mx4::GemvArgs a{w[0]->packed, w[0]->scales, x, y[0], m, w[0]->rows, k, xt == MX4_BF16, ctx->stream};
        a.group = &gg;
        const hipError_t e =
            tokens ? mx4::launch_gemv_mt(a, ctx->cus)
                   : mx4::launch_skinny(a, ctx->cus, {ctx->split_part, ctx->split_count, kSplitPartTiles, kSplitCounts});
        if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString(e));
        return MX4_OK;
    }
    // more than 32 token rows (prefill in the reference's arithmetic): one
    // exact-GEMM launch over all the weights' column tiles, unsplit
    if (count > 1 && stored && foldable && m > 32) {
        mx4::GemvGroup gg{};
        gg.count = count;
        gg.k = k;
        gg.x = x;
        gg.x_bf16 = xt == MX4_BF16;
        gg.stream = ctx->stream;
        for (uint32_t i = 0; i < count; ++i) {
            gg.packed[i] = w[i]->packed;
            gg.scales[i] = w[i]->scales;
            gg.y[i] = y[i];
            gg.n[i] = w[i]->rows;
        }
        mx4::GemvArgs a{w[0]->packed, w[0]->scales, x, y[0], m, w[0]->rows, k, xt == MX4_BF16, ctx->stream};
        a.group = &gg;
        const hipError_t e = mx4::launch_gemm_exact(a, ctx->cus, nullptr, ctx->split_part, kSplitPartBytes);
        if (e == hipSuccess) return MX4_OK;
        if (e != hipErrorNotSupported) return fail(MX4_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString(e));
    }
    for (uint32_t i = 0; i < count; ++i) {
        mx4_status st = run_matmul(ctx, x, xt, m, w[i], y[i], MX4_PATH_AUTO);
        if (st != MX4_OK) return st;
    }
    return MX4_OK;
}

mx4_status mx4_gemv_config(mx4_context* ctx, const void* x, mx4_dtype xt, const mx4_weight* const* w,
                           float* const* y, uint32_t count, int team_waves, int rows_per_team, int teams_per_workgroup,
                           uint32_t teams) {
    if (!ctx || !w || !y) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (count < 1 || count > 4) return fail(MX4_ERR_ARGUMENT, "a group holds 1 to 4 weights");
    if (team_waves < 0 || rows_per_team < 0 || teams_per_workgroup < 0)
        return fail(MX4_ERR_ARGUMENT, "negative configuration");
    mx4::GemvGroup gg{};
    for (uint32_t i = 0; i < count; ++i) {
        mx4_status st = check_matmul_args(ctx, x, xt, 1, w[i], y[i]);
        if (st != MX4_OK) return st;
        if (w[i]->cols != w[0]->cols) return fail(MX4_ERR_SHAPE, "grouped weights must share their width");
        if (w[i]->bf16) return fail(MX4_ERR_UNSUPPORTED, "the GEMV configurations are for MXFP4 weights");
        if (need_stored(w[i]) != MX4_OK) return MX4_ERR_UNSUPPORTED;
        if (!scales_foldable(w[i])) return fail(MX4_ERR_UNSUPPORTED, "scale bytes outside 2..252 need the generic kernel");
        gg.packed[i] = w[i]->packed;
        gg.scales[i] = w[i]->scales;
        gg.y[i] = y[i];
        gg.n[i] = w[i]->rows;
    }
    if (!mx4::gemv_m1_supported(w[0]->cols))
        return fail(MX4_ERR_UNSUPPORTED, "GEMV path needs K/32 in {64,128,192,256,384}");
    DeviceGuard g(ctx->device);
    gg.count = count;
    gg.k = w[0]->cols;
    gg.x = x;
    gg.x_bf16 = xt == MX4_BF16;
    gg.stream = ctx->stream;
    mx4::M1Config c;
    c.wg = team_waves;
    c.r = rows_per_team;
    c.tpw = teams_per_workgroup;
    c.grid = teams;
    hipError_t e = mx4::launch_gemv_m1_group(gg, ctx->cus, &c);
    if (e == hipErrorNotSupported) return fail(MX4_ERR_UNSUPPORTED, "configuration not instantiated");
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status mx4_gemm_config(mx4_context* ctx, const void* x, mx4_dtype xt, uint32_t m, const mx4_weight* w, float* y,
                           int waves_m, int waves_n, int tiles_m, int tiles_n, int k_slices) {
    mx4_status st = check_matmul_args(ctx, x, xt, m, w, y);
    if (st != MX4_OK) return st;
    if (w->bf16) return fail(MX4_ERR_UNSUPPORTED, "the GEMM configurations are for MXFP4 weights");
    if (need_stored(w) != MX4_OK) return MX4_ERR_UNSUPPORTED;
    if (!scales_foldable(w)) return fail(MX4_ERR_UNSUPPORTED, "scale bytes outside 2..252 need the generic kernel");
    if (!mx4::gemm_exact_supported(m, w->rows, w->cols, xt == MX4_BF16))
        return fail(MX4_ERR_UNSUPPORTED, "GEMM path needs K %% 128 == 0 and operands under 2 GiB");
    if (waves_m < 0 || waves_n < 0 || tiles_m < 0 || tiles_n < 0 || k_slices < 0)
        return fail(MX4_ERR_ARGUMENT, "negative configuration");
    DeviceGuard g(ctx->device);
    mx4::GemvArgs a{w->packed, w->scales, x, y, m, w->rows, w->cols, xt == MX4_BF16, ctx->stream};
    mx4::GemmConfig c;
    c.wm = waves_m;
    c.wn = waves_n;
    c.tm = tiles_m;
    c.tn = tiles_n;
    c.ks = k_slices;
    hipError_t e = mx4::launch_gemm_exact(a, ctx->cus, &c, ctx->split_part, kSplitPartBytes);
    if (e == hipErrorNotSupported) return fail(MX4_ERR_UNSUPPORTED, "GEMM instance not compiled");
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status mx4_gemv_tokens_config(mx4_context* ctx, const void* x, uint32_t m, const mx4_weight* w, float* y,
                                  uint32_t teams, uint32_t teams_per_workgroup) {
    mx4_status st = check_matmul_args(ctx, x, MX4_BF16, m, w, y);
    if (st != MX4_OK) return st;
    if (w->bf16) return fail(MX4_ERR_UNSUPPORTED, "the GEMV configurations are for MXFP4 weights");
    if (need_stored(w) != MX4_OK) return MX4_ERR_UNSUPPORTED;
    if (!scales_foldable(w)) return fail(MX4_ERR_UNSUPPORTED, "scale bytes outside 2..252 need the generic kernel");
    if (!mx4::gemv_mt_supported(m, w->cols, true))
        return fail(MX4_ERR_UNSUPPORTED, "few-token GEMV needs 2 <= m <= 4 and K in {2048, 4096, 6144, 8192, 12288}");
    DeviceGuard g(ctx->device);
    mx4::GemvArgs a{w->packed, w->scales, x, y, m, w->rows, w->cols, true, ctx->stream};
    hipError_t e = mx4::launch_gemv_mt(a, ctx->cus, teams, teams_per_workgroup);
    if (e == hipErrorNotSupported) return fail(MX4_ERR_UNSUPPORTED, "configuration not possible");
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status mx4_matmul_prefill(mx4_context* ctx, const void* x, mx4_dtype xt, uint32_t m, const mx4_weight* w,
                              mx4_act_format act, float* y) {
    mx4_status st = check_matmul_args(ctx, x, xt, m, w, y);
    if (st != MX4_OK) return st;
    if (act != MX4_ACT_MXFP4 && act != MX4_ACT_MXFP8) return fail(MX4_ERR_ARGUMENT, "bad activation format");
    if (w->bf16) return fail(MX4_ERR_UNSUPPORTED, "the block-scaled MFMA path takes MXFP4 weights");
    if (!mx4::prefill_supported(m, w->rows, w->cols))
        return fail(MX4_ERR_UNSUPPORTED, "block-scaled MFMA path needs K %% 256 == 0 and operands under 2 GiB");
    DeviceGuard g(ctx->device);
    const bool fp8 = act == MX4_ACT_MXFP8;
    mx4_weight* wm = const_cast<mx4_weight*>(w);  // the fragment copy is a cache of the weight
    st = prepare_fragments(ctx, wm);
    if (st != MX4_OK) return st;
    const uint64_t qoff = (mx4::fragment_bytes(m, w->cols, fp8) + 255) & ~255ull;
    st = ensure_buffer(ctx, &ctx->work, &ctx->work_cap, prefill_workspace_bytes(m, w->cols, fp8), true);
    if (st != MX4_OK) return st;
    uint8_t* xf = static_cast<uint8_t*>(ctx->work);
    uint8_t* xsf = xf + qoff;
    hipError_t e = mx4::launch_quantize_fragments(x, xt == MX4_BF16, m, w->cols, fp8, xf, xsf, ctx->flags, ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "requantize launch failed: %s", hipGetErrorString(e));
    e = mx4::launch_prefill(prefill_args(ctx, wm, xf, xsf, y, m, fp8), ctx->cus);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "prefill launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status mx4_matmul_prefill_noalloc(mx4_context* ctx, const void* x, mx4_dtype xt, uint32_t m, const mx4_weight* w,
                                      mx4_act_format act, float* y) {
    mx4_status st = check_matmul_args(ctx, x, xt, m, w, y);
    if (st != MX4_OK) return st;
    if (act != MX4_ACT_MXFP4 && act != MX4_ACT_MXFP8) return fail(MX4_ERR_ARGUMENT, "bad activation format");
    if (w->bf16) return fail(MX4_ERR_UNSUPPORTED, "the block-scaled MFMA path takes MXFP4 weights");
    if (!mx4::prefill_supported(m, w->rows, w->cols))
        return fail(MX4_ERR_UNSUPPORTED, "block-scaled MFMA path needs K %% 256 == 0 and operands under 2 GiB");
    if (!w->frag)
        return fail(MX4_ERR_UNSUPPORTED,
                    "the weight has no matrix-core copy; call mx4_weight_prepare_prefill first (this entry point "
                    "allocates nothing)");
    const bool fp8 = act == MX4_ACT_MXFP8;
    const uint64_t need = kNoAllocHead + prefill_workspace_bytes(m, w->cols, fp8);
    if (need > kNoAllocScratchBytes)
        return fail(MX4_ERR_TOO_LARGE,
                    "requantized activations of %u x %u (%s) need %llu bytes; the no-alloc workspace holds %llu",
                    m, w->cols, fp8 ? "MX-FP8" : "MXFP4", (unsigned long long)need,
                    (unsigned long long)kNoAllocScratchBytes);
    uint8_t* base = scratch_of(ctx->device);
    if (!base) return fail(MX4_ERR_DEVICE, "no-alloc workspace not set up on device %d", ctx->device);
    DeviceGuard g(ctx->device);
    // head: the requantizer's non-finite flag (written, never read here: such
    // rows come out as NaN); then codes and scales as in the context workspace
    uint32_t* flag = reinterpret_cast<uint32_t*>(base);
    uint8_t* xf = base + kNoAllocHead;
    uint8_t* xsf = xf + ((mx4::fragment_bytes(m, w->cols, fp8) + 255) & ~255ull);
    hipError_t e = mx4::launch_quantize_fragments(x, xt == MX4_BF16, m, w->cols, fp8, xf, xsf, flag, ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "requantize launch failed: %s", hipGetErrorString(e));
    e = mx4::launch_prefill(prefill_args(ctx, w, xf, xsf, y, m, fp8), ctx->cus);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "prefill launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status mx4_matmul_batch(mx4_context* ctx, const mx4_op* ops, uint32_t count) {
    if (!ctx || (!ops && count)) return fail(MX4_ERR_ARGUMENT, "null argument");
    for (uint32_t i = 0; i < count; ++i) {
        mx4_status st = check_matmul_args(ctx, ops[i].x, (mx4_dtype)ops[i].x_type, ops[i].m, ops[i].w, ops[i].y);
        if (st != MX4_OK) return fail(st, "op %u: %s", i, g_error.c_str());
    }
    DeviceGuard g(ctx->device);
    for (uint32_t i = 0; i < count; ++i) {
        mx4_status st = run_matmul(ctx, ops[i].x, (mx4_dtype)ops[i].x_type, ops[i].m, ops[i].w, ops[i].y,
                                   MX4_PATH_AUTO);
        if (st != MX4_OK) return fail(st, "op %u: %s", i, g_error.c_str());
    }
    return MX4_OK;
}

mx4_status mx4_pass_begin(mx4_context* ctx) {
    if (!ctx) return fail(MX4_ERR_ARGUMENT, "null context");
    DeviceGuard g(ctx->device);
    HIP_TRY(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return MX4_OK;
}

mx4_status mx4_pass_end(mx4_context* ctx, mx4_pass** out) {
    if (!ctx || !out) return fail(MX4_ERR_ARGUMENT, "null argument");
    *out = nullptr;
    DeviceGuard g(ctx->device);
    hipGraph_t graph = nullptr;
    HIP_TRY(hipStreamEndCapture(ctx->stream, &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return fail(MX4_ERR_DEVICE, "graph instantiate failed: %s", hipGetErrorString(e));
    }
    mx4_pass* p = new (std::nothrow) mx4_pass{graph, exec, ctx->device, ctx};
    if (!p) {
        (void)hipGraphExecDestroy(exec);
        (void)hipGraphDestroy(graph);
        return fail(MX4_ERR_NO_MEMORY, "out of host memory");
    }
    ctx->passes.insert(p);
    *out = p;
    return MX4_OK;
}

mx4_status mx4_pass_launch(mx4_context* ctx, const mx4_pass* pass) {
    if (!ctx || !pass) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (pass->ctx != ctx) return fail(MX4_ERR_ARGUMENT, "pass recorded on another context");
    DeviceGuard g(ctx->device);
    HIP_TRY(hipGraphLaunch(pass->exec, ctx->stream));
    return MX4_OK;
}

void mx4_pass_release(mx4_pass* pass) {
    if (!pass) return;
    DeviceGuard g(pass->device);
    mx4_context* ctx = pass->ctx;
    if (ctx) (void)hipStreamSynchronize(ctx->stream);  // a replay may still run
    (void)hipGraphExecDestroy(pass->exec);
    (void)hipGraphDestroy(pass->graph);
    if (ctx) {
        ctx->passes.erase(pass);
        if (ctx->passes.empty()) {
            for (void* b : ctx->retired) (void)hipFree(b);
            ctx->retired.clear();
        }
    }
    delete pass;
}

mx4_status mx4_reserve_prefill(mx4_context* ctx, uint32_t max_m, uint32_t max_cols) {
    if (!ctx) return fail(MX4_ERR_ARGUMENT, "null context");
    DeviceGuard g(ctx->device);
    return ensure_buffer(ctx, &ctx->work, &ctx->work_cap, prefill_workspace_bytes(max_m, max_cols, true), true);
}

mx4_status mx4_matmul_mx(mx4_context* ctx, const uint8_t* xq, const uint8_t* xs, mx4_act_format act, uint32_t m,
                         const mx4_weight* w, float* y) {
    if (!ctx || !xq || !xs || !w || !y) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (act != MX4_ACT_MXFP4 && act != MX4_ACT_MXFP8) return fail(MX4_ERR_ARGUMENT, "bad activation format");
    if (m == 0) return fail(MX4_ERR_ARGUMENT, "m must be at least 1");
    if (w->ctx != ctx) return fail(MX4_ERR_ARGUMENT, "weight belongs to another context");
    if (w->bf16) return fail(MX4_ERR_UNSUPPORTED, "the block-scaled MFMA path takes MXFP4 weights");
    if (!mx4::prefill_supported(m, w->rows, w->cols))
        return fail(MX4_ERR_UNSUPPORTED, "block-scaled MFMA path needs K %% 256 == 0 and operands under 2 GiB");
    DeviceGuard g(ctx->device);
    const bool fp8 = act == MX4_ACT_MXFP8;
    mx4_weight* wm = const_cast<mx4_weight*>(w);
    mx4_status st = prepare_fragments(ctx, wm);
    if (st != MX4_OK) return st;
    const uint64_t qoff = (mx4::fragment_bytes(m, w->cols, fp8) + 255) & ~255ull;
    st = ensure_buffer(ctx, &ctx->work, &ctx->work_cap, prefill_workspace_bytes(m, w->cols, fp8), true);
    if (st != MX4_OK) return st;
    uint8_t* xf = static_cast<uint8_t*>(ctx->work);
    uint8_t* xsf = xf + qoff;
    hipError_t e = mx4::launch_to_fragments(xq, xs, m, w->cols, fp8, xf, xsf, ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "layout launch failed: %s", hipGetErrorString(e));
    e = mx4::launch_prefill(prefill_args(ctx, wm, xf, xsf, y, m, fp8), ctx->cus);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "prefill launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status mx4_prefill_act_bytes(uint32_t m, uint32_t cols, mx4_act_format act, uint64_t* codes_bytes,
                                 uint64_t* scales_bytes) {
    if (!codes_bytes || !scales_bytes) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (act != MX4_ACT_MXFP4 && act != MX4_ACT_MXFP8) return fail(MX4_ERR_ARGUMENT, "bad activation format");
    if (m == 0 || cols % 256 != 0) return fail(MX4_ERR_SHAPE, "need m >= 1 and cols %% 256 == 0");
    *codes_bytes = mx4::fragment_bytes(m, cols, act == MX4_ACT_MXFP8);
    *scales_bytes = mx4::fragment_scale_bytes(m, cols);
    return MX4_OK;
}

mx4_status mx4_prefill_quantize(mx4_context* ctx, const void* x, mx4_dtype xt, uint32_t m, uint32_t cols,
                                mx4_act_format act, uint8_t* codes, uint8_t* scales) {
    if (!ctx || !x || !codes || !scales) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (xt != MX4_F32 && xt != MX4_BF16) return fail(MX4_ERR_ARGUMENT, "bad activation dtype %d", (int)xt);
    if (act != MX4_ACT_MXFP4 && act != MX4_ACT_MXFP8) return fail(MX4_ERR_ARGUMENT, "bad activation format");
    if (m == 0 || cols % 256 != 0) return fail(MX4_ERR_SHAPE, "need m >= 1 and cols %% 256 == 0");
    if (((uintptr_t)x & 15) != 0 || ((uintptr_t)codes & 15) != 0 || ((uintptr_t)scales & 3) != 0)
        return fail(MX4_ERR_ARGUMENT, "x and codes must be 16-byte aligned, scales 4-byte aligned");
    DeviceGuard g(ctx->device);
    hipError_t e = mx4::launch_quantize_fragments(x, xt == MX4_BF16, m, cols, act == MX4_ACT_MXFP8, codes, scales,
                                                  ctx->flags, ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "requantize launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

namespace {

// One block-scaled MFMA launch over requantized activations for `count`
// weights of the same K (a group shares the activations), with the default
// instance (tile_m == 0) or an explicit one.
mx4_status prefill_group(mx4_context* ctx, const uint8_t* codes, const uint8_t* scales, mx4_act_format act,
                         uint32_t m, const mx4_weight* const* ws, float* const* ys, uint32_t count, uint32_t tile_m,
                         uint32_t tile_n, uint32_t split_k) {
    if (!ctx || !codes || !scales || !ws || !ys) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (count < 1 || count > mx4::kMaxPrefillGroup)
        return fail(MX4_ERR_ARGUMENT, "a prefill group holds 1 to %u weights", mx4::kMaxPrefillGroup);
    if (act != MX4_ACT_MXFP4 && act != MX4_ACT_MXFP8) return fail(MX4_ERR_ARGUMENT, "bad activation format");
    if (m == 0) return fail(MX4_ERR_ARGUMENT, "m must be at least 1");
    for (uint32_t i = 0; i < count; ++i) {
        const mx4_weight* w = ws[i];
        if (!w || !ys[i]) return fail(MX4_ERR_ARGUMENT, "null argument");
        if (w->ctx != ctx) return fail(MX4_ERR_ARGUMENT, "weight belongs to another context");
        if (w->bf16) return fail(MX4_ERR_UNSUPPORTED, "the block-scaled MFMA path takes MXFP4 weights");
        if (w->cols != ws[0]->cols) return fail(MX4_ERR_SHAPE, "the weights of a group share K");
        if (!mx4::prefill_supported(m, w->rows, w->cols))
            return fail(MX4_ERR_UNSUPPORTED, "block-scaled MFMA path needs K %% 256 == 0 and operands under 2 GiB");
    }
    DeviceGuard g(ctx->device);
    mx4::PrefillArgs a{};
    for (uint32_t i = 0; i < count; ++i) {
        mx4_weight* wm = const_cast<mx4_weight*>(ws[i]);  // the fragment copy is a cache of the weight
        mx4_status st = prepare_fragments(ctx, wm);
        if (st != MX4_OK) return st;
        a.wf[i] = wm->frag;
        a.wsf[i] = wm->frag_scales;
        a.y[i] = ys[i];
        a.n[i] = wm->rows;
    }
    a.count = count;
    a.xf = codes;
    a.xsf = scales;
    a.m = m;
    a.k = ws[0]->cols;
    a.fp8 = act == MX4_ACT_MXFP8;
    a.stream = ctx->stream;
    a.tile_m = tile_m;
    a.tile_n = tile_n;
    a.split_k = split_k;
    hipError_t e = mx4::launch_prefill(a, ctx->cus);
    if (e == hipErrorNotSupported && tile_m != 0) return fail(MX4_ERR_UNSUPPORTED, "no such prefill instance for this shape");
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "prefill launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

}  // namespace

mx4_status mx4_prefill_matmul(mx4_context* ctx, const uint8_t* codes, const uint8_t* scales, mx4_act_format act,
                              uint32_t m, const mx4_weight* w, float* y) {
    return prefill_group(ctx, codes, scales, act, m, &w, &y, 1, 0, 0, 0);
}

mx4_status mx4_prefill_matmul_group(mx4_context* ctx, const uint8_t* codes, const uint8_t* scales,
                                    mx4_act_format act, uint32_t m, const mx4_weight* const* ws, float* const* ys,
                                    uint32_t count) {
    return prefill_group(ctx, codes, scales, act, m, ws, ys, count, 0, 0, 0);
}

mx4_status mx4_prefill_config(mx4_context* ctx, const uint8_t* codes, const uint8_t* scales, mx4_act_format act,
                              uint32_t m, const mx4_weight* w, float* y, uint32_t tile_m, uint32_t tile_n,
                              uint32_t split_k) {
    return prefill_group(ctx, codes, scales, act, m, &w, &y, 1, tile_m, tile_n, split_k);
}

mx4_status mx4_prefill_group_config(mx4_context* ctx, const uint8_t* codes, const uint8_t* scales,
                                    mx4_act_format act, uint32_t m, const mx4_weight* const* ws, float* const* ys,
                                    uint32_t count, uint32_t tile_m, uint32_t tile_n, uint32_t split_k) {
    return prefill_group(ctx, codes, scales, act, m, ws, ys, count, tile_m, tile_n, split_k);
}

mx4_status mx4_matmul_prefill_group(mx4_context* ctx, const void* x, mx4_dtype xt, uint32_t m,
                                    const mx4_weight* const* ws, mx4_act_format act, float* const* ys,
                                    uint32_t count) {
    if (!ctx || !ws || !ys) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (count < 1 || count > mx4::kMaxPrefillGroup)
        return fail(MX4_ERR_ARGUMENT, "a prefill group holds 1 to %u weights", mx4::kMaxPrefillGroup);
    for (uint32_t i = 0; i < count; ++i) {
        mx4_status st = check_matmul_args(ctx, x, xt, m, ws[i], ys[i]);
        if (st != MX4_OK) return st;
        if (ws[i]->cols != ws[0]->cols) return fail(MX4_ERR_SHAPE, "the weights of a group share K");
    }
    if (act != MX4_ACT_MXFP4 && act != MX4_ACT_MXFP8) return fail(MX4_ERR_ARGUMENT, "bad activation format");
    for (uint32_t i = 0; i < count; ++i) {
        if (ws[i]->bf16) return fail(MX4_ERR_UNSUPPORTED, "the block-scaled MFMA path takes MXFP4 weights");
        if (!mx4::prefill_supported(m, ws[i]->rows, ws[i]->cols))
            return fail(MX4_ERR_UNSUPPORTED, "block-scaled MFMA path needs K %% 256 == 0 and operands under 2 GiB");
    }
    DeviceGuard g(ctx->device);
    const bool fp8 = act == MX4_ACT_MXFP8;
    const uint32_t cols = ws[0]->cols;
    // build every fragment copy before anything is enqueued
    for (uint32_t i = 0; i < count; ++i) {
        mx4_status st = prepare_fragments(ctx, const_cast<mx4_weight*>(ws[i]));
        if (st != MX4_OK) return st;
    }
    const uint64_t qoff = (mx4::fragment_bytes(m, cols, fp8) + 255) & ~255ull;
    mx4_status st = ensure_buffer(ctx, &ctx->work, &ctx->work_cap, prefill_workspace_bytes(m, cols, fp8), true);
    if (st != MX4_OK) return st;
    uint8_t* xf = static_cast<uint8_t*>(ctx->work);
    uint8_t* xsf = xf + qoff;
    hipError_t e = mx4::launch_quantize_fragments(x, xt == MX4_BF16, m, cols, fp8, xf, xsf, ctx->flags, ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "requantize launch failed: %s", hipGetErrorString(e));
    return prefill_group(ctx, xf, xsf, act, m, ws, ys, count, 0, 0, 0);
}

mx4_status mx4_matmul_argmax(mx4_context* ctx, const void* x, mx4_dtype xt, const mx4_weight* w, float* y,
                             uint32_t* idx) {
    if (!ctx || !x || !w || !idx) return fail(MX4_ERR_ARGUMENT, "null x, weight or index");
    if (xt != MX4_F32 && xt != MX4_BF16) return fail(MX4_ERR_ARGUMENT, "bad activation dtype %d", (int)xt);
    if (w->ctx != ctx) return fail(MX4_ERR_ARGUMENT, "weight belongs to another context");
    if (((uintptr_t)x & 15) != 0) return fail(MX4_ERR_ARGUMENT, "x must be 16-byte aligned");
    if (y && ((uintptr_t)y & 3) != 0) return fail(MX4_ERR_ARGUMENT, "y must be 4-byte aligned");
    if (need_stored(w) != MX4_OK) return MX4_ERR_UNSUPPORTED;
    DeviceGuard g(ctx->device);
    if (!w->bf16 && mx4::gemv_m1_supported(w->cols) && scales_foldable(w)) {
        mx4::GemvArgs a{w->packed, w->scales, x, y, 1, w->rows, w->cols, xt == MX4_BF16, ctx->stream};
        hipError_t e = mx4::launch_gemv_m1_argmax(a, ctx->am_partial, kArgmaxPartials, idx, ctx->cus);
        if (e == hipSuccess) return MX4_OK;
        if (e != hipErrorNotSupported) return fail(MX4_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString(e));
    }
    // no fused instance for this shape: the projection, then the argmax kernel
    float* logits = y;
    if (!logits) {
        mx4_status st = ensure_buffer(ctx, &ctx->logits, &ctx->logits_cap, (uint64_t)w->rows * 4, true);
        if (st != MX4_OK) return st;
        logits = static_cast<float*>(ctx->logits);
    }
    mx4_status st = run_matmul(ctx, x, xt, 1, w, logits, MX4_PATH_AUTO);
    if (st != MX4_OK) return st;
    hipError_t e = mx4::launch_argmax_rows(logits, 1, w->rows, idx, ctx->am_partial, kArgmaxPartials, ctx->cus,
                                           ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "argmax launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status mx4_embed(mx4_context* ctx, const mx4_weight* w, const uint32_t* ids, uint32_t count, uint16_t* out) {
    if (!ctx || !w || (count && (!ids || !out))) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (w->ctx != ctx) return fail(MX4_ERR_ARGUMENT, "weight belongs to another context");
    if (w->cols % 32 != 0) return fail(MX4_ERR_SHAPE, "embedding rows must be a multiple of 32 wide");
    if (((uintptr_t)out & 15) != 0) return fail(MX4_ERR_ARGUMENT, "out must be 16-byte aligned");
    if (need_stored(w) != MX4_OK) return MX4_ERR_UNSUPPORTED;
    DeviceGuard g(ctx->device);
    hipError_t e = mx4::launch_embed(w->packed, w->scales, w->bf16, ids, count, w->rows, w->cols, out, ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "embed launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status mx4_dequantize(mx4_context* ctx, const mx4_weight* w, float* out) {
    if (!ctx || !w || !out) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (w->bf16) return fail(MX4_ERR_UNSUPPORTED, "not an MXFP4 weight");
    if (need_stored(w) != MX4_OK) return MX4_ERR_UNSUPPORTED;
    DeviceGuard g(ctx->device);
    hipError_t e = mx4::launch_dequantize(w->packed, w->scales, (uint64_t)w->rows * w->cols, out, ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "dequantize launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

static mx4_status quantize_common(mx4_context* ctx, const void* in, mx4_dtype t, uint64_t rows, uint32_t cols,
                                  uint8_t* q, uint8_t* s, bool fp8) {
    if (!ctx || !in || !q || !s) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (t != MX4_F32 && t != MX4_BF16) return fail(MX4_ERR_ARGUMENT, "bad input dtype");
    if (cols % 32 != 0) return fail(MX4_ERR_SHAPE, "expected a matrix whose row width is divisible by 32");
    if (((uintptr_t)in & 15) || ((uintptr_t)q & 15)) return fail(MX4_ERR_ARGUMENT, "buffers must be 16-byte aligned");
    DeviceGuard g(ctx->device);
    HIP_TRY(mx4::launch_fill_u32(ctx->flags, 1, 0, ctx->stream));
    hipError_t e = fp8 ? mx4::launch_quantize_fp8(in, t == MX4_BF16, rows, cols, q, s, ctx->flags, ctx->stream)
                       : mx4::launch_quantize_mxfp4(in, t == MX4_BF16, rows, cols, q, s, ctx->flags, ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "quantize launch failed: %s", hipGetErrorString(e));
    uint32_t bad = 0;
    HIP_TRY(hipMemcpyAsync(&bad, ctx->flags, 4, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    if (bad) return fail(MX4_ERR_NON_FINITE, "cannot quantize non-finite weights");
    return MX4_OK;
}

mx4_status mx4_quantize(mx4_context* ctx, const void* in, mx4_dtype t, uint64_t rows, uint32_t cols,
                        uint8_t* packed, uint8_t* scales) {
    return quantize_common(ctx, in, t, rows, cols, packed, scales, false);
}

mx4_status mx4_quantize_fp8(mx4_context* ctx, const void* in, mx4_dtype t, uint64_t rows, uint32_t cols,
                            uint8_t* codes, uint8_t* scales) {
    return quantize_common(ctx, in, t, rows, cols, codes, scales, true);
}

mx4_status mx4_argmax_rows(mx4_context* ctx, const float* x, uint32_t rows, uint32_t width, uint32_t* out) {
    if (!ctx || !x || !out) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (width == 0) return fail(MX4_ERR_ARGUMENT, "argmax of an empty row");
    DeviceGuard g(ctx->device);
    hipError_t e = mx4::launch_argmax_rows(x, rows, width, out, ctx->am_partial, kArgmaxPartials, ctx->cus,
                                           ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "argmax launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status mx4_synth_bf16(mx4_context* ctx, uint64_t seed, double sigma, uint64_t start, uint64_t count,
                          uint16_t* out) {
    if (!ctx || (!out && count)) return fail(MX4_ERR_ARGUMENT, "null argument");
    DeviceGuard g(ctx->device);
    hipError_t e = mx4::launch_synth_bf16(seed, sigma, start, count, out, ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "synth launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status mx4_synth_weight(mx4_context* ctx, uint64_t seed, double sigma, uint32_t rows, uint32_t cols,
                            uint8_t* packed, uint8_t* scales) {
    if (!ctx || !packed || !scales) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (cols % 32 != 0 || rows == 0) return fail(MX4_ERR_SHAPE, "width must be a nonzero multiple of 32");
    if (((uintptr_t)packed & 15) != 0) return fail(MX4_ERR_ARGUMENT, "packed must be 16-byte aligned");
    DeviceGuard g(ctx->device);
    hipError_t e = mx4::launch_synth_weight(seed, sigma, rows, cols, packed, scales, ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "synth launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status mx4_timer_begin(mx4_context* ctx) {
    if (!ctx) return fail(MX4_ERR_ARGUMENT, "null context");
    DeviceGuard g(ctx->device);
    HIP_TRY(hipEventRecord(ctx->ev0, ctx->stream));
    return MX4_OK;
}

mx4_status mx4_timer_end(mx4_context* ctx, double* ms) {
    if (!ctx || !ms) return fail(MX4_ERR_ARGUMENT, "null argument");
    DeviceGuard g(ctx->device);
    HIP_TRY(hipEventRecord(ctx->ev1, ctx->stream));
    HIP_TRY(hipEventSynchronize(ctx->ev1));
    float f = 0.0f;
    HIP_TRY(hipEventElapsedTime(&f, ctx->ev0, ctx->ev1));
    *ms = f;
    return MX4_OK;
}

mx4_status mx4_decode_table(mx4_context* ctx, int mode, float* out) {
    if (!ctx || !out) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (mode < 0 || mode > 3) return fail(MX4_ERR_ARGUMENT, "bad mode");
    DeviceGuard g(ctx->device);
    hipError_t e = mx4::launch_decode_table(mode, out, ctx->stream);
    if (e != hipSuccess) return fail(MX4_ERR_DEVICE, "decode table launch failed: %s", hipGetErrorString(e));
    return MX4_OK;
}

mx4_status mx4_mfma_ceiling(mx4_context* ctx, int shape, int random_codes, double* pflops, double* clock_ghz) {
    if (!ctx || !pflops || !clock_ghz) return fail(MX4_ERR_ARGUMENT, "null argument");
    if (shape < 0 || shape > 3)
        return fail(MX4_ERR_ARGUMENT, "shape must be 0 (FP4 32x32x64), 1 (FP4 16x16x128), 2 (FP8 x FP4 32x32x64) "
                                      "or 3 (bf16 32x32x16)");
    DeviceGuard g(ctx->device);
    int wall_khz = 0;
    HIP_TRY(hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, ctx->device));
    if (wall_khz <= 0) return fail(MX4_ERR_DEVICE, "no constant-rate clock");
    // one workgroup of eight waves per CU; 8192 (16384 for 16x16x128; 4096 for
    // the half-rate FP8 x FP4) MFMAs per wave, about 0.3 ms at the full rate
    const uint32_t grid = (uint32_t)ctx->cus, iters = shape == 2 ? 512 : 1024;
    const uint32_t waves = mx4::mfma_ceiling_waves(grid);
    uint64_t* clocks = nullptr;
    float* sink = nullptr;
    HIP_TRY(hipMalloc(&clocks, (size_t)waves * 4 * sizeof(uint64_t)));
    if (hipMalloc(&sink, (size_t)grid * 512 * sizeof(float)) != hipSuccess) {
        (void)hipFree(clocks);
        return fail(MX4_ERR_DEVICE, "out of device memory");
    }
    mx4_status st = MX4_OK;
    std::vector<uint64_t> h((size_t)waves * 4);
    float ms = 0.0f;
    // events of its own: the context's pair may be inside a caller's mx4_timer_begin/end
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
        st = fail(MX4_ERR_DEVICE, "mfma ceiling probe: event creation failed");
    // a warm-up launch (the clock settles under the load), then the timed one
    for (int rep = 0; rep < 2 && st == MX4_OK; ++rep) {
        hipError_t e = hipEventRecord(e0, ctx->stream);
        if (e == hipSuccess) e = mx4::launch_mfma_ceiling(shape, iters, random_codes != 0, grid, clocks, sink, ctx->stream);
        if (e == hipSuccess) e = hipEventRecord(e1, ctx->stream);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        if (e != hipSuccess) st = fail(MX4_ERR_DEVICE, "mfma ceiling probe: %s", hipGetErrorString(e));
    }
    if (st == MX4_OK && hipMemcpy(h.data(), clocks, h.size() * sizeof(uint64_t), hipMemcpyDeviceToHost) != hipSuccess)
        st = fail(MX4_ERR_DEVICE, "mfma ceiling probe: copy of the clocks failed");
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(clocks);
    (void)hipFree(sink);
    if (st != MX4_OK) return st;
    std::vector<double> ghz;
    ghz.reserve(waves);
    for (uint32_t w = 0; w < waves; ++w) {
        const double dc = (double)(h[4 * w + 1] - h[4 * w]), dw = (double)(h[4 * w + 3] - h[4 * w + 2]);
        if (dw > 0) ghz.push_back(dc / dw * wall_khz * 1e-6);
    }
    if (ghz.empty() || ms <= 0.0f) return fail(MX4_ERR_DEVICE, "mfma ceiling probe: no timing");
    std::sort(ghz.begin(), ghz.end());
    *clock_ghz = ghz[ghz.size() / 2];
    *pflops = mx4::mfma_ceiling_flops(shape, iters, grid) / (ms * 1e-3) / 1e15;
    return MX4_OK;
}

// ------------------------------------------------------------ per-call drop-in

void* qwen_hip_create(void) {
    // engine/src/metal.m:18-48: a device, a queue and the pipelines, or NULL.
    mx4_context* ctx = nullptr;
    if (mx4_create(0, &ctx) != MX4_OK) {
        std::fprintf(stderr, "qwen_hip_create: %s\n", g_error.c_str());
        return nullptr;
    }
    return ctx;
}

void qwen_hip_destroy(void* context) { mx4_destroy(static_cast<mx4_context*>(context)); }

void qwen_hip_set_cache_limit(void* context, uint64_t bytes) {
    mx4_context* ctx = static_cast<mx4_context*>(context);
    if (!ctx) return;
    ctx->cache_limit = bytes;
    cache_evict(ctx);
}

bool qwen_hip_matmul(void* context, const float* x, const void* w, const uint8_t* scales, float* y,
                     uint32_t rows, uint32_t cols, uint32_t inner) {
    // engine/src/metal.m:54-117
    mx4_context* ctx = static_cast<mx4_context*>(context);
    if (!ctx || !x || !w || !y) {
        fail(MX4_ERR_ARGUMENT, "null argument");
        return false;
    }
    if (rows == 0 || cols == 0 || inner == 0) {
        fail(MX4_ERR_ARGUMENT, "empty matmul");
        return false;
    }
    DeviceGuard g(ctx->device);
    CacheKey key{w, scales, cols, inner};
    auto it = ctx->cache.find(key);
    mx4_weight* weight = nullptr;
    if (it == ctx->cache.end()) {
        // scales == NULL: w is bf16 [cols][inner] (engine/src/metal.rs:45-50)
        const mx4_status up = scales ? mx4_weight_upload(ctx, static_cast<const uint8_t*>(w), scales, cols, inner, &weight)
                                     : mx4_weight_upload_bf16(ctx, static_cast<const uint16_t*>(w), cols, inner, &weight);
        if (up != MX4_OK) return false;
        uint64_t bytes = scales ? (uint64_t)cols * inner / 2 + (uint64_t)cols * inner / 32 : (uint64_t)cols * inner * 2;
        ctx->lru.push_front(key);
        ctx->cache.emplace(key, CacheEntry{weight, bytes, ctx->lru.begin()});
        ctx->cache_bytes += bytes;
    } else {
        weight = it->second.w;
        ctx->lru.splice(ctx->lru.begin(), ctx->lru, it->second.lru);
    }
    const uint64_t xbytes = (uint64_t)rows * inner * 4, ybytes = (uint64_t)rows * cols * 4;
    if (ensure_buffer(ctx, &ctx->x_stage, &ctx->x_cap, xbytes) != MX4_OK) return false;
    if (ensure_buffer(ctx, &ctx->y_stage, &ctx->y_cap, ybytes) != MX4_OK) return false;
    if (ensure_pinned(ctx, &ctx->x_pin, &ctx->x_pin_cap, xbytes) != MX4_OK) return false;
    if (ensure_pinned(ctx, &ctx->y_pin, &ctx->y_pin_cap, ybytes) != MX4_OK) return false;
    std::memcpy(ctx->x_pin, x, xbytes);
    // From here on every exit waits for the stream: the next call writes (or
    // ensure_pinned frees) x_pin, which an upload still in flight would read.
    if (hipMemcpyAsync(ctx->x_stage, ctx->x_pin, xbytes, hipMemcpyHostToDevice, ctx->stream) != hipSuccess) {
        fail(MX4_ERR_DEVICE, "input upload failed");
        (void)hipStreamSynchronize(ctx->stream);
        return false;
    }
    if (run_matmul(ctx, ctx->x_stage, MX4_F32, rows, weight, static_cast<float*>(ctx->y_stage), MX4_PATH_AUTO) !=
        MX4_OK) {
        (void)hipStreamSynchronize(ctx->stream);
        return false;
    }
    const hipError_t ce = hipMemcpyAsync(ctx->y_pin, ctx->y_stage, ybytes, hipMemcpyDeviceToHost, ctx->stream);
    const hipError_t se = hipStreamSynchronize(ctx->stream);
    if (ce != hipSuccess || se != hipSuccess) {
        fail(MX4_ERR_DEVICE, "matmul or copy-back failed");
        return false;
    }
    std::memcpy(y, ctx->y_pin, ybytes);
    // evict only after the call completed, never the weight just used
    if (ctx->cache_bytes > ctx->cache_limit) {
        CacheKey keep = key;
        ctx->lru.remove(keep);
        cache_evict(ctx);
        ctx->lru.push_front(keep);
        auto kit = ctx->cache.find(keep);
        if (kit != ctx->cache.end()) kit->second.lru = ctx->lru.begin();
    }
    return true;
}

}  // extern "C"
