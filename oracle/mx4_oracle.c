/*
 * mx4_oracle.c -- CPU oracle for the MXFP4 weight-quantized matmul.
 *
 * TEST INFRASTRUCTURE ONLY (the checker). Only tests/, smoke() and the
 * cpu_baseline leg of bench.py may load it; the product never does.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 *
 * Every function cites the reference file:line whose behaviour it restates;
 * paths are relative to the fawwaz46/jalapenos-at-home tree.
 */
#include "mx4_oracle.h"

#include <math.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* engine/src/mxfp4.rs:3 (and python/quantize_mxfp4.py:13) */
static const float LEVELS[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
/* python/quantize_mxfp4.py:14: (LEVELS[:-1] + LEVELS[1:]) / 2 in float32 */
static const float MIDPOINTS[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};

float oracle_bf16_to_f32(uint16_t bits) {
    /* engine/src/lib.rs:74-76: bf16 is the top half of an f32 */
    uint32_t u = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t oracle_f32_to_bf16(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
    uint32_t round = 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)((u + round) >> 16);
}

float oracle_powi2(int32_t exponent) {
    /* engine/src/mxfp4.rs:30 calls 2.0_f32.powi(e); rustc lowers powi to
     * compiler-rt's square-and-multiply followed by a reciprocal for
     * negative exponents. Every intermediate is a power of two, so the
     * result is exactly 2^e (subnormal at e=-127, inf at e=128). */
    int recip = exponent < 0;
    int32_t b = exponent;
    float a = 2.0f, r = 1.0f;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

float oracle_mx_value(const uint8_t *packed, const uint8_t *scales, uint64_t index) {
    /* engine/src/mxfp4.rs:27-33 */
    uint8_t code = (uint8_t)((packed[index / 2] >> (4 * (index % 2))) & 15);
    int32_t exponent = (int32_t)scales[index / 32] - 127;
    float magnitude = LEVELS[code & 7] * oracle_powi2(exponent);
    return (code & 8) == 0 ? magnitude : -magnitude;
}

void oracle_mx_values(const uint8_t *packed, const uint8_t *scales, uint64_t start,
                      uint64_t end, float *out) {
    /* engine/src/mxfp4.rs:35-49: one scale per 32-block, then per element */
    uint64_t n = 0;
    for (uint64_t block = start / 32; block < (end + 31) / 32; ++block) {
        float scale = oracle_powi2((int32_t)scales[block] - 127);
        uint64_t s = start > block * 32 ? start : block * 32;
        uint64_t e = end < (block + 1) * 32 ? end : (block + 1) * 32;
        for (uint64_t index = s; index < e; ++index) {
            uint8_t code = (uint8_t)((packed[index / 2] >> (4 * (index % 2))) & 15);
            float magnitude = LEVELS[code & 7] * scale;
            out[n++] = (code & 8) == 0 ? magnitude : -magnitude;
        }
    }
}

int oracle_mx_validate(uint64_t rows, uint64_t cols, uint64_t packed_len,
                       const uint8_t *scales, uint64_t scales_len) {
    /* engine/src/mxfp4.rs:11-25 */
    if (rows == 0 || cols == 0 || cols % 32 != 0) return 1;
    if (cols != 0 && rows > UINT64_MAX / cols) return 2;
    uint64_t elements = rows * cols;
    if (packed_len != elements / 2 || scales_len != elements / 32) return 3;
    for (uint64_t i = 0; i < scales_len; ++i)
        if (scales[i] == 255) return 4;
    return 0;
}

void oracle_matmul(const float *x, uint64_t tok_rows, uint64_t tok_len,
                   const uint8_t *packed, const uint8_t *scales, uint64_t weight_rows,
                   float *out) {
    /* engine/src/lib.rs:240-266 with the Some(q) arm of :251-254: f32
     * accumulator from 0.0, ascending i, separate multiply and add. */
    uint64_t n = 0;
    for (uint64_t t = 0; t < tok_rows; ++t) {
        for (uint64_t r = 0; r < weight_rows; ++r) {
            float sum = 0.0f;
            for (uint64_t i = 0; i < tok_len; ++i) {
                float product = x[t * tok_len + i] * oracle_mx_value(packed, scales, r * tok_len + i);
                sum += product;
            }
            out[n++] = sum;
        }
    }
}

void oracle_matmul_bf16(const float *x, uint64_t tok_rows, uint64_t tok_len,
                        const uint16_t *w, uint64_t weight_rows, float *out) {
    /* engine/src/lib.rs:240-266 with the None arm of :255 */
    uint64_t n = 0;
    for (uint64_t t = 0; t < tok_rows; ++t) {
        for (uint64_t r = 0; r < weight_rows; ++r) {
            float sum = 0.0f;
            for (uint64_t i = 0; i < tok_len; ++i) {
                float product = x[t * tok_len + i] * oracle_bf16_to_f32(w[r * tok_len + i]);
                sum += product;
            }
            out[n++] = sum;
        }
    }
}

static float dot_row(const float *xrow, uint64_t tok_len, const uint8_t *packed,
                     const uint8_t *scales, uint64_t r) {
    float sum = 0.0f;
    for (uint64_t i = 0; i < tok_len; ++i) {
        float product = xrow[i] * oracle_mx_value(packed, scales, r * tok_len + i);
        sum += product;
    }
    return sum;
}

void oracle_matmul_rows(const float *x, uint64_t tok_rows, uint64_t tok_len,
                        const uint8_t *packed, const uint8_t *scales, uint64_t r0,
                        uint64_t r1, float *out, int threads) {
    /* engine/src/lib.rs:240-266 restricted to weight rows [r0, r1). */
    uint64_t width = r1 - r0;
    int64_t total = (int64_t)(tok_rows * width);
#ifdef _OPENMP
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
    for (int64_t p = 0; p < total; ++p) {
        uint64_t t = (uint64_t)p / width, r = r0 + (uint64_t)p % width;
        out[p] = dot_row(x + t * tok_len, tok_len, packed, scales, r);
    }
    (void)threads;
}

void oracle_matmul_f64(const float *x, uint64_t tok_rows, uint64_t tok_len,
                       const uint8_t *packed, const uint8_t *scales, uint64_t weight_rows,
                       double *out) {
    uint64_t n = 0;
    for (uint64_t t = 0; t < tok_rows; ++t) {
        for (uint64_t r = 0; r < weight_rows; ++r) {
            double sum = 0.0;
            for (uint64_t i = 0; i < tok_len; ++i)
                sum += (double)x[t * tok_len + i] *
                       (double)oracle_mx_value(packed, scales, r * tok_len + i);
            out[n++] = sum;
        }
    }
}

int oracle_quantize(const float *values, uint64_t rows, uint64_t cols, uint8_t *packed,
                    uint8_t *scales) {
    /* python/quantize_mxfp4.py:18-39 */
    if (cols % 32 != 0) return 1;                           /* :21-22 */
    for (uint64_t i = 0; i < rows * cols; ++i)
        if (!isfinite(values[i])) return 2;                 /* :23-24 */
    uint64_t blocks = cols / 32;
    for (uint64_t r = 0; r < rows; ++r) {
        for (uint64_t b = 0; b < blocks; ++b) {
            const float *v = values + r * cols + b * 32;
            float maximum = 0.0f;                           /* :27 np.max(np.abs(...)) */
            for (int i = 0; i < 32; ++i) {
                float a = fabsf(v[i]);
                if (a > maximum) maximum = a;
            }
            int fe = 0;
            frexpf(maximum, &fe);                           /* :29 frexp(...)[1] - 3 */
            int exponent = fe - 3;
            if (exponent < -127) exponent = -127;
            if (exponent > 127) exponent = 127;
            if (maximum == 0.0f) exponent = -127;           /* :30 */
            uint8_t codes[32];
            for (int i = 0; i < 32; ++i) {
                float scaled = ldexpf(fabsf(v[i]), -exponent); /* :31 */
                int code = 0;                               /* :32 searchsorted side=left */
                while (code < 7 && MIDPOINTS[code] < scaled) ++code;
                float midpoint = MIDPOINTS[code < 6 ? code : 6]; /* :33 */
                if ((code & 1) && scaled == midpoint) ++code;    /* :34 ties to even */
                if (signbit(v[i])) code |= 8;                    /* :35 */
                codes[i] = (uint8_t)code;
            }
            for (int i = 0; i < 16; ++i)                    /* :37 low nibble = even */
                packed[r * (cols / 2) + b * 16 + i] =
                    (uint8_t)(codes[2 * i] | (codes[2 * i + 1] << 4));
            scales[r * blocks + b] = (uint8_t)(exponent + 127); /* :38 */
        }
    }
    return 0;
}

void oracle_dequantize(const uint8_t *packed, const uint8_t *scales, uint64_t rows,
                       uint64_t cols, float *out) {
    /* python/quantize_mxfp4.py:42-49: copysign(LEVELS[c&7], sign) then ldexp */
    for (uint64_t r = 0; r < rows; ++r) {
        for (uint64_t c = 0; c < cols; ++c) {
            uint8_t byte = packed[r * (cols / 2) + c / 2];
            uint8_t code = (c & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 15);
            float magnitude = LEVELS[code & 7];
            float value = copysignf(magnitude, (code & 8) ? -1.0f : 1.0f);
            out[r * cols + c] = ldexpf(value, (int)scales[r * (cols / 32) + c / 32] - 127);
        }
    }
}

float oracle_fp8_e4m3_value(uint8_t code) {
    /* OCP 8-bit float E4M3 ("fn": no inf; S.1111.111 is NaN) */
    int sign = code >> 7, e = (code >> 3) & 15, m = code & 7;
    float v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf((float)(8 + m), e - 10);
    return sign ? -v : v;
}

static uint8_t e4m3_magnitude_code(float scaled) {
    /* RNE onto the E4M3 grid, saturating at 448 (0x7e). scaled is finite, >= 0. */
    if (scaled < 0x1p-6f) {
        float q = nearbyintf(scaled * 512.0f);   /* subnormal step 2^-9; exact scaling */
        return (uint8_t)q;                       /* q == 8 is the smallest normal, 0x08 */
    }
    int fe = 0;
    frexpf(scaled, &fe);
    int E = fe - 1;                              /* scaled in [2^E, 2^(E+1)) */
    float q = nearbyintf(ldexpf(scaled, 3 - E)); /* in [8, 16] */
    if (q >= 16.0f) { q = 8.0f; E += 1; }
    if (E > 8) return 0x7e;
    int code = ((E + 7) << 3) | ((int)q - 8);
    return code > 0x7e ? 0x7e : (uint8_t)code;
}

int oracle_quantize_fp8(const float *values, uint64_t rows, uint64_t cols, uint8_t *codes,
                        uint8_t *scales) {
    if (cols % 32 != 0) return 1;
    for (uint64_t i = 0; i < rows * cols; ++i)
        if (!isfinite(values[i])) return 2;
    uint64_t blocks = cols / 32;
    for (uint64_t r = 0; r < rows; ++r) {
        for (uint64_t b = 0; b < blocks; ++b) {
            const float *v = values + r * cols + b * 32;
            float maximum = 0.0f;
            for (int i = 0; i < 32; ++i) {
                float a = fabsf(v[i]);
                if (a > maximum) maximum = a;
            }
            int fe = 0;
            frexpf(maximum, &fe);
            int exponent = fe - 1 - 8;                   /* emax(E4M3) = 8 */
            if (exponent < -127) exponent = -127;
            if (exponent > 127) exponent = 127;
            if (maximum == 0.0f) exponent = -127;
            for (int i = 0; i < 32; ++i) {
                float scaled = ldexpf(fabsf(v[i]), -exponent);
                uint8_t c = e4m3_magnitude_code(scaled);
                if (signbit(v[i])) c |= 0x80;
                codes[r * cols + b * 32 + i] = c;
            }
            scales[r * blocks + b] = (uint8_t)(exponent + 127);
        }
    }
    return 0;
}

void oracle_dequantize_fp8(const uint8_t *codes, const uint8_t *scales, uint64_t rows,
                           uint64_t cols, float *out) {
    for (uint64_t r = 0; r < rows; ++r)
        for (uint64_t c = 0; c < cols; ++c)
            out[r * cols + c] = ldexpf(oracle_fp8_e4m3_value(codes[r * cols + c]),
                                       (int)scales[r * (cols / 32) + c / 32] - 127);
}

uint64_t oracle_argmax(const float *values, uint64_t n) {
    /* engine/src/model.rs:288-296 */
    uint64_t best = 0;
    for (uint64_t i = 1; i < n; ++i)
        if (values[i] > values[best]) best = i;
    return best;
}

/* ---- synthetic inputs (defined here; the reference has no generator) ---- */

uint64_t oracle_splitmix64(uint64_t seed, uint64_t n) {
    uint64_t z = seed + (n + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

double oracle_ln(double u) {
    /* ln u = e ln2 + 2 atanh(t), t = (m-1)/(m+1), m in [sqrt(1/2), sqrt 2).
     * Fixed 13-term series; only +,-,*,/ so it rounds identically anywhere. */
    static const double inv_odd[13] = {
        0x1.0000000000000p+0, 0x1.5555555555555p-2, 0x1.999999999999ap-3,
        0x1.2492492492492p-3, 0x1.c71c71c71c71cp-4, 0x1.745d1745d1746p-4,
        0x1.3b13b13b13b14p-4, 0x1.1111111111111p-4, 0x1.e1e1e1e1e1e1ep-5,
        0x1.af286bca1af28p-5, 0x1.8618618618618p-5, 0x1.642c8590b2164p-5,
        0x1.47ae147ae147bp-5};
    uint64_t bits;
    memcpy(&bits, &u, 8);
    int e = (int)((bits >> 52) & 0x7ff) - 1023;          /* u is normal: u >= 2^-53 */
    bits = (bits & 0x000fffffffffffffull) | 0x3ff0000000000000ull;
    double m;
    memcpy(&m, &bits, 8);                                 /* m in [1, 2) */
    if (m > 0x1.6a09e667f3bcdp+0) { m = m * 0.5; e += 1; }
    double t = (m - 1.0) / (m + 1.0);
    double t2 = t * t;
    double p = inv_odd[12];
    for (int k = 11; k >= 0; --k) p = p * t2 + inv_odd[k];
    return (double)e * 0x1.62e42fefa39efp-1 + 2.0 * t * p;
}

double oracle_cos2pi(double turns) {
    /* cos(2 pi r), r = turns - round(turns) in [-1/2, 1/2]; 17-term Taylor */
    static const double inv_even_fact[17] = {
        0x1.0000000000000p+0, 0x1.0000000000000p-1, 0x1.5555555555555p-5,
        0x1.6c16c16c16c17p-10, 0x1.a01a01a01a01ap-16, 0x1.27e4fb7789f5cp-22,
        0x1.1eed8eff8d898p-29, 0x1.93974a8c07c9dp-37, 0x1.ae7f3e733b81fp-45,
        0x1.6827863b97d97p-53, 0x1.e542ba4020225p-62, 0x1.0ce396db7f853p-70,
        0x1.f2cf01972f578p-80, 0x1.88e85fc6a4e5ap-89, 0x1.0a18a2635085dp-98,
        0x1.3932c5047d60ep-108, 0x1.434d2e783f5bcp-118};
    double r = turns >= 0.5 ? turns - 1.0 : turns;       /* turns in [0, 1) */
    double th = r * 0x1.921fb54442d18p+2;
    double th2 = th * th;
    /* Horner on sum_k (-1)^k th^(2k) / (2k)! */
    double c = inv_even_fact[16];
    for (int k = 15; k >= 0; --k) {
        double a = (k & 1) ? -inv_even_fact[k] : inv_even_fact[k];
        c = a + th2 * c;
    }
    return c;
}

double oracle_normal(uint64_t seed, uint64_t index) {
    uint64_t a = oracle_splitmix64(seed, 2 * index);
    uint64_t b = oracle_splitmix64(seed, 2 * index + 1);
    double u1 = (double)((a >> 11) + 1) * 0x1p-53;        /* (0, 1] */
    double u2 = (double)(b >> 11) * 0x1p-53;              /* [0, 1) */
    return sqrt(-2.0 * oracle_ln(u1)) * oracle_cos2pi(u2);
}

void oracle_synth_bf16(uint64_t seed, double sigma, uint64_t start, uint64_t count,
                       uint16_t *out) {
    for (uint64_t i = 0; i < count; ++i) {
        double z = oracle_normal(seed, start + i) * sigma;
        out[i] = oracle_f32_to_bf16((float)z);
    }
}
