/*
 * mx4.h -- C ABI of the MI355X (gfx950) MXFP4 weight-quantized matmul.
 *
 * Plain pointers and sizes only. Two layers:
 *
 *  1. qwen_hip_*: the per-call drop-in for the reference engine's Metal bridge
 *     (fawwaz46/jalapenos-at-home engine/src/metal.rs:6-19, implemented there
 *     by engine/src/metal.m:18-117). Same signature, argument meaning, sync
 *     contract and failure value (NULL / false).
 *
 *  2. mx4_*: the resident API in the style of the reference's GPU-resident
 *     bridge (engine/src/gpu.rs:19-42, engine/src/gpu.m:27-128): weights stay
 *     in HBM, kernels are enqueued on one HIP stream, device pointers are
 *     caller-owned, and a pass can be timed with GPU events.
 *
 * Data layout (engine/src/mxfp4.rs:5-8): a weight of `rows` x `cols` (= N x K)
 * is packed u8 [rows][cols/2], element 2j in the low nibble of byte j, and
 * scales u8 [rows][cols/32], E8M0 with bias 127. Activations x are row-major
 * [m][cols] f32 (what engine/src/metal.rs:11 passes) or bf16; outputs y are
 * row-major f32 [m][rows]. Device pointers given to the resident API are
 * expected to be 16-byte aligned, as hipMalloc returns them: kernels access
 * activations, outputs and packed codes 16 bytes at a time.
 *
 * Threading: a context is not thread-safe (the reference's Metal context is
 * neither Send nor Sync). Errors: every mx4_* call returns an mx4_status;
 * mx4_last_error() gives the message of the last failure on the calling thread.
 */
#ifndef MX4_H
#define MX4_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mx4_status {
    MX4_OK = 0,
    MX4_ERR_ARGUMENT = 1,    /* null pointer, bad enum, size out of range */
    MX4_ERR_SHAPE = 2,       /* engine/src/mxfp4.rs:12-14: nonempty rows, width % 32 == 0 */
    MX4_ERR_TOO_LARGE = 3,   /* engine/src/mxfp4.rs:15-17 */
    MX4_ERR_LENGTH = 4,      /* engine/src/mxfp4.rs:18-20 */
    MX4_ERR_NAN_SCALE = 5,   /* engine/src/mxfp4.rs:21-23: scale byte 255 */
    MX4_ERR_NON_FINITE = 6,  /* python/quantize_mxfp4.py:23-24 */
    MX4_ERR_DEVICE = 7,      /* HIP runtime failure or no gfx950 device */
    MX4_ERR_NO_MEMORY = 8,
    MX4_ERR_UNSUPPORTED = 9
} mx4_status;

typedef enum mx4_dtype { MX4_F32 = 0, MX4_BF16 = 1 } mx4_dtype;

/* Which kernel family runs a matmul. AUTO follows the M-based dispatch of
 * engine/src/gpu.rs:469-515 re-tuned for gfx950. */
typedef enum mx4_path {
    MX4_PATH_AUTO = 0,
    MX4_PATH_GEMV = 1,     /* decode GEMV (no MFMA): M == 1, or 2 <= M <= 4 with bf16 x */
    MX4_PATH_SKINNY = 2,   /* exact skinny kernel on bf16 MFMA, M <= 32, K in {2,4,6,8,12}*1024 */
    MX4_PATH_GENERIC = 3,  /* exact fallback for any M and K % 32 == 0 */
    MX4_PATH_PREFILL = 4,  /* block-scaled MFMA on requantized activations */
    MX4_PATH_GEMM = 5      /* exact tiled GEMM on bf16 MFMA, any M, K % 128 == 0 */
} mx4_path;

/* Activation format on the block-scaled MFMA path (M = 512 prefill). */
typedef enum mx4_act_format {
    MX4_ACT_MXFP4 = 1,  /* requantized per 32 along K by the MXFP4 rule */
    MX4_ACT_MXFP8 = 2   /* requantized per 32 along K to MX E4M3 */
} mx4_act_format;

typedef struct mx4_context mx4_context;
typedef struct mx4_weight mx4_weight;

/* ------------------------------------------------------------------------
 * 1. Per-call drop-in (engine/src/metal.rs:6-19)
 * ------------------------------------------------------------------------ */

/* Replaces qwen_metal_create (engine/src/metal.rs:7, engine/src/metal.m:18-48).
 * Kernels are precompiled for gfx950, so no source string is taken. Returns
 * NULL (message on stderr and in mx4_last_error) when no gfx950 device exists. */
void *qwen_hip_create(void);

/* Replaces qwen_metal_destroy (engine/src/metal.rs:8, engine/src/metal.m:50-52). */
void qwen_hip_destroy(void *context);

/* Replaces qwen_metal_matmul (engine/src/metal.rs:9-18, engine/src/metal.m:54-117).
 * y[rows][cols] = x[rows][inner] . W[cols][inner]^T. scales != NULL: w is packed
 * MXFP4 [cols][inner/2] with scales [cols][inner/32]; scales == NULL: w is bf16
 * [cols][inner] (both arms supported). Device copies of w and scales are cached by host pointer (the
 * caller keeps them immutable, engine/src/metal.rs:33). Synchronous: y is valid
 * on return. Returns false on any failure. */
bool qwen_hip_matmul(void *context, const float *x, const void *w, const uint8_t *scales,
                     float *y, uint32_t rows, uint32_t cols, uint32_t inner);

/* Byte budget of the host-pointer weight cache (the Metal bridge's NSCache
 * limit, engine/src/metal.m:43-44; default 64 GiB here for 288 GB of HBM).
 * Least recently used entries are evicted beyond it. */
void qwen_hip_set_cache_limit(void *context, uint64_t bytes);

/* ------------------------------------------------------------------------
 * 2. Resident API (engine/src/gpu.rs:19-42, engine/src/gpu.m:27-128)
 * ------------------------------------------------------------------------ */

/* gpu_create (engine/src/gpu.m:27-49): binds HIP device `device` and creates
 * the context's stream (default priority) and its device scratch (argmax
 * partials, and 32 MiB of split-K partial tiles with their arrival counts).
 * The scratch is shared by every call on the context, so calls on one context
 * must stay ordered: after mx4_set_stream, work still queued on the previous
 * stream must finish before the new stream runs more. */
mx4_status mx4_create(int device, mx4_context **out);
/* Waits for the context's stream, then frees everything it holds. Weight
 * handles made on it (mx4_weight_upload*, mx4_weight_wrap) stay valid as
 * handles but are detached: their device memory is freed here, every entry
 * point given one fails with MX4_ERR_ARGUMENT ("the weight's context was
 * destroyed"), and mx4_weight_release then only deletes the handle. Passes
 * are detached the same way (mx4_pass_release). Either order of releasing
 * weights and destroying their context is therefore safe. */
void mx4_destroy(mx4_context *ctx);
const char *mx4_last_error(void);
/* Number of gfx950 devices visible (0 without a GPU; never fails). */
int mx4_device_count(void);
/* Compute units of the context's device (the launch shapes are sized by it;
 * 256 on a full MI355X, fewer on a partitioned one). No counterpart in the
 * reference (Metal sizes its grids by the matrix alone). */
mx4_status mx4_compute_units(const mx4_context *ctx, int *cus);

/* Enqueue on a caller stream (a hipStream_t) instead of the context's own;
 * NULL restores the context stream. */
mx4_status mx4_set_stream(mx4_context *ctx, void *hip_stream);
void *mx4_get_stream(mx4_context *ctx);
mx4_status mx4_synchronize(mx4_context *ctx);

/* Host-only check of MXFP4 storage, engine/src/mxfp4.rs:11-25. Needs no GPU. */
mx4_status mx4_validate(uint64_t rows, uint64_t cols, uint64_t packed_len,
                        const uint8_t *scales, uint64_t scales_len);

/* Device memory (gpu_buffer / gpu_buffer_contents / gpu_release,
 * engine/src/gpu.m:69-84). Copies are synchronous with respect to the host. */
mx4_status mx4_malloc(mx4_context *ctx, uint64_t bytes, void **dev);
mx4_status mx4_free(mx4_context *ctx, void *dev);
mx4_status mx4_upload(mx4_context *ctx, void *dev_dst, const void *host_src, uint64_t bytes);
mx4_status mx4_download(mx4_context *ctx, void *host_dst, const void *dev_src, uint64_t bytes);
/* Stream-ordered device-to-device copy. */
mx4_status mx4_copy(mx4_context *ctx, void *dev_dst, const void *dev_src, uint64_t bytes);

/* GpuTensor::new (engine/src/gpu.rs:225-237): validates (mx4_validate) and
 * copies packed + scales into HBM once; the weight stays resident. */
mx4_status mx4_weight_upload(mx4_context *ctx, const uint8_t *packed, const uint8_t *scales,
                             uint32_t rows, uint32_t cols, mx4_weight **out);
/* Tensor::bf16 (engine/src/lib.rs:43-49): a bf16 weight [rows][cols], copied
 * into HBM once. mx4_matmul / mx4_matmul_group multiply with it exactly as the
 * reference's bf16 arm (engine/src/lib.rs:255) does, f32 accumulation; the
 * MXFP4-only entry points (GEMV configurations, prefill, dequantize) reject it,
 * and mx4_weight_info reports null packed/scales for it. */
mx4_status mx4_weight_upload_bf16(mx4_context *ctx, const uint16_t *data, uint32_t rows, uint32_t cols,
                                  mx4_weight **out);
/* Wrap packed/scales already in HBM (not copied, not freed by release). The
 * scale bytes are scanned on device; a 255 byte fails with MX4_ERR_NAN_SCALE. */
mx4_status mx4_weight_wrap(mx4_context *ctx, const uint8_t *packed_dev, const uint8_t *scales_dev,
                           uint32_t rows, uint32_t cols, mx4_weight **out);
/* Frees the weight's device memory (the library's, not a wrapped caller's)
 * and its handle; after mx4_destroy of its context, only the handle. */
void mx4_weight_release(mx4_weight *w);
mx4_status mx4_weight_info(const mx4_weight *w, uint32_t *rows, uint32_t *cols,
                           const uint8_t **packed_dev, const uint8_t **scales_dev);

/* HBM a weight holds: its stored layout (packed + scales, or the bf16 matrix;
 * 0 once dropped) and its matrix-core copy for the block-scaled prefill path
 * (about 1.06x the packed size, 0 while not built). No counterpart in the
 * reference (its GPU path reads the stored layout only). */
mx4_status mx4_weight_footprint(const mx4_weight *w, uint64_t *stored_bytes, uint64_t *matrix_core_bytes);
/* Free the matrix-core copy (after a prefill phase); a later prefill call
 * builds it again, which allocates. Refused when it is the only layout left,
 * and while any recorded pass of the context is alive (a pass keeps the raw
 * pointers of the layouts it read). */
mx4_status mx4_weight_release_prefill(mx4_weight *w);
/* Keep one resident copy of a weight that serves prefill only: build the
 * matrix-core copy if needed, then free the stored layout. Afterwards only
 * the prefill entry points (mx4_matmul_prefill*, mx4_prefill_matmul*,
 * mx4_matmul_mx, mx4_matmul_prefill_noalloc) take the weight; the others fail
 * with MX4_ERR_UNSUPPORTED, and mx4_weight_info reports null packed/scales.
 * Only for weights whose memory the library owns (not mx4_weight_wrap), and
 * refused while any recorded pass of the context is alive. */
mx4_status mx4_weight_drop_stored(mx4_weight *w);

/* GpuModel::matmul (engine/src/gpu.rs:469-515): y_dev[m][rows] =
 * x_dev[m][cols] . W^T, enqueued on the context stream, exact arithmetic
 * (f32 accumulation of exact products). AUTO picks GEMV for m == 1, the
 * few-token GEMV or the exact skinny kernel for 2 <= m <= 32, and the exact
 * tiled GEMM on bf16 MFMA (MX4_PATH_GEMM) beyond -- the analogue of the
 * reference's M > 32 GEMM (engine/src/matmul.metal:65-97). Shapes the fast
 * kernels do not take (K not a multiple of 128, scale bytes outside 2..252)
 * run the exact generic kernel. */
mx4_status mx4_matmul(mx4_context *ctx, const void *x_dev, mx4_dtype x_type, uint32_t m,
                      const mx4_weight *w, float *y_dev);
/* The same with an explicit kernel family (MX4_PATH_PREFILL is not exact:
 * use mx4_matmul_prefill). */
mx4_status mx4_matmul_path(mx4_context *ctx, const void *x_dev, mx4_dtype x_type, uint32_t m,
                           const mx4_weight *w, float *y_dev, mx4_path path);
/* Up to 4 weights of the same width that read the same activations (q|k|v,
 * gate|up) in one launch: y_dev[i][m][w[i].rows] = x . W_i^T. For m == 1 this
 * is one GEMV over the concatenated rows; for 2 <= m <= 32 (a speculative
 * verify step) one launch of the few-token GEMV or the skinny kernel over all
 * the weights' rows, chosen as mx4_matmul would choose for one weight of the
 * group's total rows; for m > 32 one launch of the exact GEMM over all the
 * weights' column tiles (K unsplit); otherwise (bf16 weights, scale bytes
 * outside 2..252) the projections run one after another. Same arithmetic as
 * mx4_matmul: exact products, f32 sums, so each output equals mx4_matmul's
 * for its weight within f32 rounding (the same bits when both choose the same
 * kernel instance). */
mx4_status mx4_matmul_group(mx4_context *ctx, const void *x_dev, mx4_dtype x_type, uint32_t m,
                            const mx4_weight *const *w, float *const *y_dev, uint32_t count);

/* Tuning hook for the M == 1 GEMV over a group of 1 to 4 weights (as
 * mx4_matmul_group): waves per team (the team splits each row's K; K/32 must
 * be a multiple of 64*team), rows per team per iteration (1, 2, 4 or 8, with
 * rows * K/(2048*team) <= 8), teams per workgroup (x is staged once per
 * workgroup in LDS when more than one; at most 512 threads), and the number of
 * teams (0: one row-set each). Zero team, rows or teams_per_workgroup keep the
 * defaults. */
mx4_status mx4_gemv_config(mx4_context *ctx, const void *x_dev, mx4_dtype x_type,
                           const mx4_weight *const *w, float *const *y_dev, uint32_t count,
                           int team_waves, int rows_per_team, int teams_per_workgroup, uint32_t teams);

/* Tuning hook for the few-token GEMV (2 <= m <= 4 bf16 token rows, the
 * MX4_PATH_GEMV kernel for m > 1): the number of teams walking the row-sets
 * and of teams per workgroup sharing one LDS copy of the token rows. Zero
 * keeps the default; a shape that cannot be launched gives MX4_ERR_UNSUPPORTED. */
mx4_status mx4_gemv_tokens_config(mx4_context *ctx, const void *x_dev, uint32_t m, const mx4_weight *w,
                                  float *y_dev, uint32_t teams, uint32_t teams_per_workgroup);

/* Tuning hook for the exact tiled GEMM (MX4_PATH_GEMM): waves per workgroup
 * along M and N and 32x32 MFMA tiles per wave along M and N, one of the
 * compiled instances (2x2 waves of 2x3, 2x2, 2x1, 1x2 or 1x1 tiles; 1x4 waves of
 * 2x2, 2x1, 1x2 or 1x1; 2x4 waves of 2x2 (bf16 x only) or 1x2; 4x1 waves of
 * 1x2), and K slices across workgroups (0 or 1: none; a split needs K a
 * multiple of 128 * k_slices and k_slices * m * rows * 4 bytes within the
 * context's 32 MiB split scratch); MX4_ERR_UNSUPPORTED otherwise. Zero waves
 * keep the default, which splits K on its own when the tiles alone would
 * leave CUs idle, and for f32 activations or K >= 8192 when a larger tile
 * with K split fills one round of workgroups. */
mx4_status mx4_gemm_config(mx4_context *ctx, const void *x_dev, mx4_dtype x_type, uint32_t m, const mx4_weight *w,
                           float *y_dev, int waves_m, int waves_n, int tiles_m, int tiles_n, int k_slices);

/* Prefill on CDNA4 block-scaled MFMA (V_MFMA_SCALE_F32_*_F8F6F4): x is
 * requantized per 32 along K (MXFP4 by python/quantize_mxfp4.py:18-39, or MX
 * E4M3), then multiplied with the MXFP4 weight, f32 accumulation. The result
 * equals the exact product of dequant(requant(x)) and W within f32 rounding. */
mx4_status mx4_matmul_prefill(mx4_context *ctx, const void *x_dev, mx4_dtype x_type, uint32_t m,
                              const mx4_weight *w, mx4_act_format act, float *y_dev);

/* mx4_matmul_prefill without any allocation. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The same
 * kernels and the same result, bit for bit, as mx4_matmul_prefill; the
 * requantized activations go to a fixed workspace of the library instead of
 * the context's growable one: a file-scope device array of 8 MiB that every
 * GPU the library runs on holds until the process ends (set up by the first
 * mx4_create on the device). Limits and rules:
 *  - 256 + codes + scales of the requantized x must fit 8 MiB (m x cols
 *    MXFP4: m * cols / 2 + m * cols / 32, rows rounded up to 32; MX-FP8:
 *    m * cols + m * cols / 32): M = 512 at K = 12288 fits in both formats;
 *    larger inputs fail with MX4_ERR_TOO_LARGE;
 *  - the weight's matrix-core copy must exist (mx4_weight_prepare_prefill),
 *    else MX4_ERR_UNSUPPORTED;
 *  - calls on one GPU share the workspace, which keeps the last call's
 *    contents: calls that overlap on one GPU (other streams, other contexts on
 *    the same device) race; keep them ordered. */
mx4_status mx4_matmul_prefill_noalloc(mx4_context *ctx, const void *x_dev, mx4_dtype x_type, uint32_t m,
                                      const mx4_weight *w, mx4_act_format act, float *y_dev);

/* mx4_matmul_prefill for up to 4 weights of the same width that read the
 * same activations (q|k|v at engine/src/lib.rs:353-355, gate|up at
 * :459-467): one requantization and one block-scaled MFMA launch, the
 * weights' output columns side by side in its grid. y_dev[i][m][w[i].rows];
 * each output equals mx4_matmul_prefill's for its weight within f32 rounding
 * (the same, bit for bit, when the group's default instance is the weight's). */
mx4_status mx4_matmul_prefill_group(mx4_context *ctx, const void *x_dev, mx4_dtype x_type, uint32_t m,
                                    const mx4_weight *const *w, mx4_act_format act, float *const *y_dev,
                                    uint32_t count);

/* One projection of a batch or recorded pass: y[m][w.rows] = x[m][w.cols] . W^T. */
typedef struct mx4_op {
    const void *x;
    float *y;
    const mx4_weight *w;
    uint32_t m;
    int32_t x_type; /* mx4_dtype */
} mx4_op;

/* Enqueue projections in order on the context stream with one call: the
 * per-projection gpu_dispatch of engine/src/gpu.rs:469-515 without a host
 * round trip per launch. Every op is checked before the first launch. */
mx4_status mx4_matmul_batch(mx4_context *ctx, const mx4_op *ops, uint32_t count);

/* A recorded pass: everything enqueued on the context stream between
 * mx4_pass_begin and mx4_pass_end is captured into a HIP graph and replayed by
 * mx4_pass_launch -- the analogue of the reference's one command buffer per
 * forward pass (engine/src/gpu.rs:157, engine/src/gpu.m:87-128). No device
 * memory is allocated or freed while recording.
 *
 * A pass keeps raw device pointers: the caller's buffers and weights it
 * names must outlive it, and so does the context (launching a pass on another
 * or a destroyed context fails). The context's own workspace (prefill
 * requantization, argmax logits) may still grow after recording, through a
 * larger eager call: while any pass of the context is alive the old buffer is
 * kept and freed only when the last pass is released, so replays stay valid.
 * mx4_pass_release waits for the context stream first. */
typedef struct mx4_pass mx4_pass;
mx4_status mx4_pass_begin(mx4_context *ctx);
mx4_status mx4_pass_end(mx4_context *ctx, mx4_pass **out);
mx4_status mx4_pass_launch(mx4_context *ctx, const mx4_pass *pass);
void mx4_pass_release(mx4_pass *pass);

/* Reserve the requantization workspace of mx4_matmul_prefill / mx4_matmul_mx
 * for up to max_m rows of max_cols (either activation format), so later calls
 * -- including calls recorded into a pass, where allocation is impossible --
 * allocate nothing. */
mx4_status mx4_reserve_prefill(mx4_context *ctx, uint32_t max_m, uint32_t max_cols);

/* Build the weight's copy in the matrix-core operand order used by the
 * block-scaled MFMA path (rows in groups of 32, one 1 KiB block per group and
 * 64 columns; about 1.06x the packed size, freed with the weight). The first
 * mx4_matmul_prefill / mx4_matmul_mx on a weight builds it on its own; call
 * this first for weights used inside a recorded pass. No counterpart in the
 * reference (its Metal kernels read the stored layout). */
mx4_status mx4_weight_prepare_prefill(mx4_weight *w);

/* The block-scaled MFMA product for activations that are already requantized
 * (xq_dev: MXFP4 packed [m][cols/2] or E4M3 [m][cols]; xs_dev: E8M0 [m][cols/32],
 * as mx4_quantize / mx4_quantize_fp8 produce them). */
mx4_status mx4_matmul_mx(mx4_context *ctx, const uint8_t *xq_dev, const uint8_t *xs_dev,
                         mx4_act_format act, uint32_t m, const mx4_weight *w, float *y_dev);

/* Activations requantized once for several prefill GEMMs that read the same
 * x (q|k|v, gate|up): mx4_prefill_quantize writes them in the matrix-core
 * operand order of the block-scaled MFMA path (rows in groups of 32), and
 * mx4_prefill_matmul multiplies such activations with a weight. Sizes of the
 * two device buffers (codes, scales) for m rows of cols (cols % 256 == 0).
 * Same arithmetic as mx4_matmul_prefill, which is these two calls in one. */
mx4_status mx4_prefill_act_bytes(uint32_t m, uint32_t cols, mx4_act_format act, uint64_t *codes_bytes,
                                 uint64_t *scales_bytes);
mx4_status mx4_prefill_quantize(mx4_context *ctx, const void *x_dev, mx4_dtype x_type, uint32_t m, uint32_t cols,
                                mx4_act_format act, uint8_t *codes_dev, uint8_t *scales_dev);
mx4_status mx4_prefill_matmul(mx4_context *ctx, const uint8_t *codes_dev, const uint8_t *scales_dev,
                              mx4_act_format act, uint32_t m, const mx4_weight *w, float *y_dev);
/* mx4_prefill_matmul over 1 to 4 weights of the same width in one launch
 * (as mx4_matmul_prefill_group, on activations already requantized). */
mx4_status mx4_prefill_matmul_group(mx4_context *ctx, const uint8_t *codes_dev, const uint8_t *scales_dev,
                                    mx4_act_format act, uint32_t m, const mx4_weight *const *w,
                                    float *const *y_dev, uint32_t count);

/* Tuning hook for the prefill GEMM (arguments as mx4_prefill_matmul): the
 * workgroup tile (tile_m rows x tile_n columns) and the number of K parts
 * inside the workgroup (split_k, summed through LDS) of one compiled
 * instance: 128 x 192 x 1 (K % 512 == 0), 128 x 128 x 1, 64 x 128 x 2 and
 * 128 x 192 x 2 (K % 512 == 0), 128 x 64 x 4, 64 x 128 x 4, 128 x 96 x 4 and
 * 128 x 128 x 4 (K % 1024 == 0). split_k = 128 (H - 1) + 16 U + D (H = 1
 * or 2; (U, D) = (4, 2), (4, 3), (4, 5), (2, 3), (2, 4), (2, 5) or (2, 8))
 * selects instead the kernel whose workgroup loads each operand fragment
 * once into LDS for all its waves: stages of U k-steps (64 K each) in a ring
 * of D, workgroup tiles 128 x 192, 128 x 128, 64 x 128, 128 x 64, 64 x 256,
 * 128 x 96, 64 x 192 and 64 x 64 (K % 256 == 0); with H = 2 the workgroup
 * has two sets of four waves, each over one half of K with its own ring,
 * whose tiles are summed in LDS at the end (K % 512 == 0). Adding 256 to an
 * H = 2 code (U, D = (4, 2), (4, 3), (2, 3) or (2, 4)) runs the two halves in
 * ping-pong: each stage becomes an LDS-read phase and an MFMA phase, and the
 * second half runs one phase behind the first, with the same arithmetic (the
 * same output bits). A ring that does not fit the LDS is cut to the deepest
 * that fits (except (4, 2)), and a stage the waves cannot share evenly is not
 * compiled.
 * MX4_ERR_UNSUPPORTED when no compiled instance matches. tile_m == 0 keeps
 * the default choice. */
mx4_status mx4_prefill_config(mx4_context *ctx, const uint8_t *codes_dev, const uint8_t *scales_dev,
                              mx4_act_format act, uint32_t m, const mx4_weight *w, float *y_dev,
                              uint32_t tile_m, uint32_t tile_n, uint32_t split_k);
/* The same hook for a group of 1 to 4 weights (as mx4_prefill_matmul_group). */
mx4_status mx4_prefill_group_config(mx4_context *ctx, const uint8_t *codes_dev, const uint8_t *scales_dev,
                                    mx4_act_format act, uint32_t m, const mx4_weight *const *w,
                                    float *const *y_dev, uint32_t count, uint32_t tile_m, uint32_t tile_n,
                                    uint32_t split_k);

/* engine/src/mxfp4.rs:35-49 on device: out_dev[rows*cols] f32, bit-exact. */
mx4_status mx4_dequantize(mx4_context *ctx, const mx4_weight *w, float *out_dev);
/* python/quantize_mxfp4.py:18-39 on device, bit-exact: in_dev [rows][cols]
 * -> packed_dev [rows][cols/2], scales_dev [rows][cols/32]. Synchronous (it
 * reports non-finite input as MX4_ERR_NON_FINITE). */
mx4_status mx4_quantize(mx4_context *ctx, const void *in_dev, mx4_dtype in_type, uint64_t rows,
                        uint32_t cols, uint8_t *packed_dev, uint8_t *scales_dev);
/* MX E4M3 requantization: codes_dev [rows][cols], scales_dev [rows][cols/32]. Synchronous. */
mx4_status mx4_quantize_fp8(mx4_context *ctx, const void *in_dev, mx4_dtype in_type, uint64_t rows,
                            uint32_t cols, uint8_t *codes_dev, uint8_t *scales_dev);
/* engine/src/model.rs:288-296 per row (argmax_rows, engine/src/gpu.metal:176-212). */
mx4_status mx4_argmax_rows(mx4_context *ctx, const float *x_dev, uint32_t rows, uint32_t width,
                           uint32_t *out_dev);

/* The lm_head of a greedy decode step (engine/src/model.rs:228-238): the
 * M == 1 projection y_dev = x . W^T and the first index of its maximum
 * (engine/src/model.rs:288-296) into idx_dev[0], fused: every GEMV workgroup
 * reduces its rows to one key and a second tiny kernel picks the winner, so
 * the logits need not be written (y_dev may be NULL) or read back. Shapes
 * without a fused instance run the projection and mx4_argmax_rows. */
mx4_status mx4_matmul_argmax(mx4_context *ctx, const void *x_dev, mx4_dtype x_type, const mx4_weight *w,
                             float *y_dev, uint32_t *idx_dev);

/* Embedding lookup (engine/src/lib.rs:222-227, engine/src/gpu.metal:43-55):
 * out_dev[t][cols] = row ids_dev[t] of the table, decoded and cut to bf16 (the
 * low 16 bits dropped, as both reference paths do); MXFP4 or bf16 tables,
 * cols % 32 == 0. An id >= rows gives a zero row. A tied lm_head
 * (engine/src/gpu.rs:341-357) is the same mx4_weight used for both. */
mx4_status mx4_embed(mx4_context *ctx, const mx4_weight *w, const uint32_t *ids_dev, uint32_t count,
                     uint16_t *out_dev);

/* Synthetic inputs (the reference defines none): element i of stream `seed`
 * is bf16(RNE(f32(RNE(sigma * z_i)))) with z_i a Box-Muller normal from
 * SplitMix64 outputs 2i and 2i+1. */
mx4_status mx4_synth_bf16(mx4_context *ctx, uint64_t seed, double sigma, uint64_t start,
                          uint64_t count, uint16_t *out_dev);
/* The weight recipe: rows x cols bf16 N(0, sigma) from `seed`, quantized. */
mx4_status mx4_synth_weight(mx4_context *ctx, uint64_t seed, double sigma, uint32_t rows,
                            uint32_t cols, uint8_t *packed_dev, uint8_t *scales_dev);

/* gpu_begin / gpu_finish (engine/src/gpu.m:87-128): GPU events around the
 * work enqueued between the two calls; end waits and returns milliseconds. */
mx4_status mx4_timer_begin(mx4_context *ctx);
mx4_status mx4_timer_end(mx4_context *ctx, double *ms);

/* Measurement aid, no counterpart in the reference: the rate the matrix
 * cores sustain on the matrix-core kernels' instructions and the shader clock
 * they hold meanwhile. MFMAs of one shape -- 0: block-scaled FP4 x FP4
 * 32x32x64 (MXFP4 prefill), 1: its 16x16x128 form, 2: block-scaled FP8 x FP4
 * 32x32x64 (MX-FP8 prefill), 3: bf16 32x32x16 (exact GEMM) -- back to back on
 * every SIMD of every CU for about 0.3 ms (after one warm-up run), on random
 * codes (random_codes != 0) or on constant codes; *pflops is the achieved
 * dense rate, *clock_ghz the median over waves of the shader clock (s_memtime
 * against the constant-rate s_memrealtime). Synchronous; allocates and frees
 * its own small buffers. */
mx4_status mx4_mfma_ceiling(mx4_context *ctx, int shape, int random_codes, double *pflops, double *clock_ghz);

/* Decode table of the hardware E2M1 converter as the kernels use it,
 * out_dev[s*16 + c] for scale byte s and code c (mode 0: bit construction,
 * 1: converter at scale 1 times 2^(s-127), 2: converter with the scale
 * folded into bf16, 3: converter with the scale folded into f32). Used by the
 * exhaustive decode test. */
mx4_status mx4_decode_table(mx4_context *ctx, int mode, float *out_dev);

#ifdef __cplusplus
}
#endif

#endif
