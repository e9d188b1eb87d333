/*
 * mx4_oracle.h -- CPU oracle for the MXFP4 weight-quantized matmul.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product (jalapenos-at-home_amd/) never links, loads or calls it.
 *
 * Each function restates one piece of the reference engine's CPU path
 * (fawwaz46/jalapenos-at-home) and cites the file:line it follows. Nothing
 * here is compiled from or copied out of the reference; it is a plain-C
 * restatement built with -ffp-contract=off and no fast-math, so every float
 * operation rounds exactly like the reference's Rust (which never contracts
 * a*b+c into an FMA).
 *
 * Parity pins (see tests/test_oracle.py):
 *   decode      -- exhaustive 16 codes x 256 scale bytes against ldexp;
 *                  engine/src/mxfp4.rs:56-65 and engine/tests/mxfp4.rs:9-33
 *   validate    -- engine/tests/mxfp4.rs:35-40
 *   matmul      -- engine/tests/mxfp4.rs:9-33, :88-105 (exact answers);
 *                  fp64-accumulated bound on random inputs
 *   quantize    -- python/tests/test_mxfp4.py:18-57 (KATs); brute-force
 *                  nearest-level search; idempotence
 *   argmax      -- first-max rule on planted ties
 *   fp8 requant -- brute-force nearest E4M3 search over all 256 codes
 *   generator   -- defined here (the reference has none); pinned by closed
 *                  forms (ln/cos against libm to 1e-14) and moments
 */
#ifndef MX4_ORACLE_H
#define MX4_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* engine/src/lib.rs:74-76 */
float oracle_bf16_to_f32(uint16_t bits);
/* round-to-nearest-even f32 -> bf16 (input synthesis only) */
uint16_t oracle_f32_to_bf16(float v);

/* engine/src/mxfp4.rs:27-33 -- the compiler-rt powi the reference calls */
float oracle_powi2(int32_t exponent);
/* engine/src/mxfp4.rs:27-33 */
float oracle_mx_value(const uint8_t *packed, const uint8_t *scales, uint64_t index);
/* engine/src/mxfp4.rs:35-49 */
void oracle_mx_values(const uint8_t *packed, const uint8_t *scales, uint64_t start,
                      uint64_t end, float *out);
/* engine/src/mxfp4.rs:11-25. 0 ok, 1 bad shape, 2 too large, 3 bad lengths, 4 NaN scale */
int oracle_mx_validate(uint64_t rows, uint64_t cols, uint64_t packed_len,
                       const uint8_t *scales, uint64_t scales_len);

/* engine/src/lib.rs:240-266, MXFP4 arm: out[t*weight_rows + r] */
void oracle_matmul(const float *x, uint64_t tok_rows, uint64_t tok_len,
                   const uint8_t *packed, const uint8_t *scales, uint64_t weight_rows,
                   float *out);
/* engine/src/lib.rs:240-266, bf16 arm */
void oracle_matmul_bf16(const float *x, uint64_t tok_rows, uint64_t tok_len,
                        const uint16_t *w, uint64_t weight_rows, float *out);
/* the same loop restricted to weight rows [r0, r1): out[t*(r1-r0) + r-r0].
 * threads > 1 splits (t, r) pairs over OpenMP threads; the per-element
 * summation order is unchanged, so results are bit-identical. */
void oracle_matmul_rows(const float *x, uint64_t tok_rows, uint64_t tok_len,
                        const uint8_t *packed, const uint8_t *scales, uint64_t r0,
                        uint64_t r1, float *out, int threads);
/* fp64 accumulation of the same products (error-bound checks) */
void oracle_matmul_f64(const float *x, uint64_t tok_rows, uint64_t tok_len,
                       const uint8_t *packed, const uint8_t *scales, uint64_t weight_rows,
                       double *out);

/* python/quantize_mxfp4.py:18-39. 0 ok, 1 width not /32, 2 non-finite */
int oracle_quantize(const float *values, uint64_t rows, uint64_t cols, uint8_t *packed,
                    uint8_t *scales);
/* python/quantize_mxfp4.py:42-49 */
void oracle_dequantize(const uint8_t *packed, const uint8_t *scales, uint64_t rows,
                       uint64_t cols, float *out);

/* OCP MX v1.0 MXFP8 (E4M3) conversion with the same scale rule shape as the
 * MXFP4 quantizer: e = floor(log2 amax) - 8, RNE, saturate to +-448. Used to
 * judge the FP8-activation MFMA path. 0 ok, 1 width, 2 non-finite */
int oracle_quantize_fp8(const float *values, uint64_t rows, uint64_t cols, uint8_t *codes,
                        uint8_t *scales);
float oracle_fp8_e4m3_value(uint8_t code);
void oracle_dequantize_fp8(const uint8_t *codes, const uint8_t *scales, uint64_t rows,
                           uint64_t cols, float *out);

/* engine/src/model.rs:288-296: first index of the maximum (strict >) */
uint64_t oracle_argmax(const float *values, uint64_t n);

/* Synthetic inputs. The reference defines no generator; this one is:
 *   SplitMix64 output n of seed s -> two 53-bit uniforms per element ->
 *   Box-Muller (cos branch) in fp64 with the fixed polynomial ln/cos below
 *   -> x sigma -> f32 (RNE) -> bf16 (RNE). */
uint64_t oracle_splitmix64(uint64_t seed, uint64_t n);
double oracle_ln(double u);
double oracle_cos2pi(double turns);
double oracle_normal(uint64_t seed, uint64_t index);
void oracle_synth_bf16(uint64_t seed, double sigma, uint64_t start, uint64_t count,
                       uint16_t *out);

#ifdef __cplusplus
}
#endif

#endif
