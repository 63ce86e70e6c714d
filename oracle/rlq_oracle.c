/*
 * rlq_oracle.c - CPU restatement of rust-llama's scalar quantized-matvec path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product; see rlq_oracle.h).
 * Every function follows the cited reference lines in arithmetic order.  All
 * paths are relative to the rust-llama repository root.  Compile with
 * -ffp-contract=off and without fast-math so f32 arithmetic rounds exactly as
 * the Rust source does (Rust never contracts a*b+c).
 *
 * Rust conversions restated here:
 *   `f32 as i32`, `f32 as i8`  saturate (NaN -> 0)           -> sat_i32/sat_i8
 *   `i32 as i8`, `i32 as u8`   truncate to the low byte      -> (int8_t)(uint8_t)
 *   `round()`                  half away from zero           -> roundf
 *   `round_ties_even()`        ties to even                  -> rintf (FE_TONEAREST)
 */
#include "rlq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

enum {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8,
    T_Q8_1 = 9, T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14,
    T_Q8_K = 15, T_IQ2_XXS = 16, T_IQ2_XS = 17, T_IQ3_XXS = 18, T_IQ1_S = 19,
    T_IQ4_NL = 20, T_IQ3_S = 21, T_IQ2_S = 22, T_IQ4_XS = 23, T_I8 = 24, T_I16 = 25,
    T_I32 = 26, T_I64 = 27, T_F64 = 28, T_IQ1_M = 29, T_BF16 = 30, T_TQ1_0 = 34,
    T_TQ2_0 = 35, T_MXFP4 = 39, T_NVFP4 = 40, T_Q1_0 = 41, T_Q2_0 = 42, T_F8_E4M3 = 43
};

static int set_err(oracle_error *err, int code, uint32_t dtype, uint64_t a, uint64_t b) {
    if (err) {
        err->code = code;
        err->dtype = dtype;
        err->a = a;
        err->b = b;
    }
    return code;
}
#define OK(err) set_err((err), ORC_OK, 0, 0, 0)

/* ---- scalars: lib.rs:321-373, 440-448 ---------------------------------- */

float oracle_f16_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    uint32_t exp = (bits >> 10) & 31u;
    uint32_t fraction = bits & 1023u;
    uint32_t result;
    if (exp == 0 && fraction == 0) {
        result = sign;
    } else if (exp == 0) {
        /* `fraction.leading_zeros() - 21` on a u32 holding <= 10 bits */
        uint32_t shift = (uint32_t)__builtin_clz(fraction) - 21u;
        result = sign | ((113u - shift) << 23) | (((fraction << shift) & 1023u) << 13);
    } else if (exp == 31) {
        result = sign | 0x7f800000u | (fraction << 13) | (fraction != 0 ? 0x00400000u : 0u);
    } else {
        result = sign | ((exp + 112u) << 23) | (fraction << 13);
    }
    float out;
    memcpy(&out, &result, 4);
    return out;
}

uint16_t oracle_f32_to_f16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exp = (int32_t)((bits >> 23) & 255u);
    uint32_t frac = bits & 0x7fffffu;
    if (exp == 255) return (uint16_t)(sign | (frac == 0 ? 0x7c00u : 0x7e00u));
    int32_t e = exp - 127;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e >= -14) {
        uint32_t mant = frac >> 13;
        uint32_t rest = frac & 8191u;
        if (rest > 4096u || (rest == 4096u && (mant & 1u) != 0)) mant += 1;
        uint32_t magnitude = ((uint32_t)(e + 15) << 10) + mant;
        return (uint16_t)(sign | (uint16_t)magnitude);
    }
    if (e < -25) return sign;
    uint32_t mant = frac | 0x800000u;
    uint32_t shift = (uint32_t)(-e - 1);
    uint32_t rounded = mant >> shift;
    uint32_t rest = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rest > half || (rest == half && (rounded & 1u) != 0)) rounded += 1;
    return (uint16_t)(sign | (uint16_t)rounded);
}

static uint16_t u16le(const uint8_t *b, size_t p) { return (uint16_t)(b[p] | (b[p + 1] << 8)); }
static float half_at(const uint8_t *b, size_t p) { return oracle_f16_to_f32(u16le(b, p)); }
static float f32le(const uint8_t *b, size_t p) {
    float v;
    memcpy(&v, b + p, 4);
    return v;
}
static void put_f16(uint8_t *b, size_t p, uint16_t h) {
    b[p] = (uint8_t)(h & 0xff);
    b[p + 1] = (uint8_t)(h >> 8);
}

static int32_t sat_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483647.0f) return 2147483647;
    if (v <= -2147483648.0f) return (int32_t)0x80000000u;
    return (int32_t)v;
}
static int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}
static int is_finite_f(float v) { return isfinite(v) != 0; }

/* ---- dtype tables: lib.rs:171-285 --------------------------------------- */

int oracle_dtype_known(uint32_t id) {
    switch (id) {
    case 0: case 1: case 2: case 3: case 6: case 7: case 8: case 9: case 10: case 11:
    case 12: case 13: case 14: case 15: case 16: case 17: case 18: case 19: case 20:
    case 21: case 22: case 23: case 24: case 25: case 26: case 27: case 28: case 29:
    case 30: case 34: case 35: case 39: case 40: case 41: case 42: case 43:
        return 1;
    default:
        return 0;
    }
}

uint64_t oracle_block_size(uint32_t t) {
    switch (t) {
    case T_F32: case T_F16: case T_BF16: case T_F64: case T_I8: case T_I16: case T_I32:
    case T_I64: case T_F8_E4M3:
        return 1;
    case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: case T_Q8_0: case T_Q8_1:
    case T_IQ4_NL: case T_MXFP4:
        return 32;
    case T_NVFP4: case T_Q2_0:
        return 64;
    case T_Q1_0:
        return 128;
    default:
        return 256;
    }
}

uint64_t oracle_type_size(uint32_t t) {
    switch (t) {
    case T_F32: case T_I32: return 4;
    case T_F16: case T_BF16: case T_I16: return 2;
    case T_F64: case T_I64: return 8;
    case T_I8: case T_F8_E4M3: return 1;
    case T_Q4_0: case T_IQ4_NL: case T_Q1_0: case T_Q2_0: return 18;
    case T_Q4_1: return 20;
    case T_Q5_0: return 22;
    case T_Q5_1: return 24;
    case T_Q8_0: return 34;
    case T_Q8_1: case T_NVFP4: return 36;
    case T_Q2_K: return 84;
    case T_Q3_K: return 110;
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q6_K: return 210;
    case T_Q8_K: return 292;
    case T_IQ2_XXS: case T_TQ2_0: return 66;
    case T_IQ2_XS: return 74;
    case T_IQ3_XXS: return 98;
    case T_IQ1_S: return 50;
    case T_IQ3_S: return 110;
    case T_IQ2_S: return 82;
    case T_IQ4_XS: return 136;
    case T_IQ1_M: return 56;
    case T_TQ1_0: return 54;
    case T_MXFP4: return 17;
    default: return 0;
    }
}

int oracle_row_bytes(uint32_t t, uint64_t elements, uint64_t *out, oracle_error *err) {
    if (!oracle_dtype_known(t)) return set_err(err, ORC_INVALID_TYPE, t, 0, 0);
    uint64_t bs = oracle_block_size(t);
    if (elements % bs != 0) return set_err(err, ORC_NON_MULTIPLE, t, elements, bs);
    uint64_t r;
    if (__builtin_mul_overflow(elements / bs, oracle_type_size(t), &r))
        return set_err(err, ORC_SIZE_OVERFLOW, t, 0, 0);
    if (out) *out = r;
    return OK(err);
}

/* lib.rs:310-319 */
static int validate(uint32_t t, uint64_t bytes, uint64_t elements, oracle_error *err) {
    uint64_t expected;
    int rc = oracle_row_bytes(t, elements, &expected, err);
    if (rc) return rc;
    if (bytes != expected) return set_err(err, ORC_INVALID_LENGTH, t, expected, bytes);
    return OK(err);
}

/* matvec.rs:7-18 */
int oracle_matvec_activation_dtype(uint32_t w, uint32_t *out, oracle_error *err) {
    uint32_t a;
    if (!oracle_dtype_known(w)) return set_err(err, ORC_INVALID_TYPE, w, 0, 0);
    switch (w) {
    case T_Q1_0: case T_Q2_0: case T_Q4_0: case T_Q5_0: case T_Q8_0: case T_MXFP4:
    case T_NVFP4: case T_IQ4_NL:
        a = T_Q8_0;
        break;
    case T_Q4_1: case T_Q5_1:
        a = T_Q8_1;
        break;
    case T_Q2_K: case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: case T_IQ2_XXS:
    case T_IQ2_XS: case T_IQ2_S: case T_IQ3_XXS: case T_IQ3_S: case T_IQ1_S: case T_IQ1_M:
    case T_IQ4_XS: case T_TQ1_0: case T_TQ2_0:
        a = T_Q8_K;
        break;
    case T_F32: case T_F16: case T_F8_E4M3:
        a = T_F32;
        break;
    case T_BF16:
        a = T_BF16;
        break;
    default:
        return set_err(err, ORC_UNSUPPORTED_MATVEC, w, 0, 0);
    }
    if (out) *out = a;
    return OK(err);
}

/* The weight dtypes whose dot this oracle restates. */
static int path_weight(uint32_t t) {
    return t == T_Q8_0 || t == T_Q2_K || t == T_Q3_K || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K;
}
static int k_weight(uint32_t t) { return t == T_Q2_K || t == T_Q3_K || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K; }

/* ---- Q8_K activation quantizer: activation.rs:4-51 ---------------------- */

static float q8k_inverse_scale(const float *x) {
    float absolute = 0.0f, maximum = 0.0f;
    for (int i = 0; i < 256; ++i) {
        if (fabsf(x[i]) > absolute) {
            absolute = fabsf(x[i]);
            maximum = x[i];
        }
    }
    return absolute == 0.0f ? 0.0f : -127.0f / maximum;
}

static int preflight_q8k(const float *x, uint64_t n, oracle_error *err) {
    for (uint64_t block = 0; block < n / 256; ++block) {
        float inverse = q8k_inverse_scale(x + block * 256);
        if (!is_finite_f(inverse) || (inverse != 0.0f && !is_finite_f(1.0f / inverse)))
            return set_err(err, ORC_UNREPRESENTABLE_SCALE, T_Q8_K, block, 0);
    }
    return OK(err);
}

static void encode_q8k(const float *x, uint8_t *b) {
    memset(b, 0, 292);
    float inverse = q8k_inverse_scale(x);
    if (inverse == 0.0f) return;
    for (int j = 0; j < 256; ++j) {
        int32_t q = sat_i32(rintf(inverse * x[j]));
        if (q > 127) q = 127;
        b[4 + j] = (uint8_t)q;
    }
    for (int g = 0; g < 16; ++g) {
        int16_t sum = 0;
        for (int j = 0; j < 16; ++j) sum = (int16_t)(sum + (int8_t)b[4 + g * 16 + j]);
        b[260 + g * 2] = (uint8_t)((uint16_t)sum & 0xff);
        b[261 + g * 2] = (uint8_t)((uint16_t)sum >> 8);
    }
    float d = 1.0f / inverse;
    memcpy(b, &d, 4);
}

/* ---- Q8_0 quantizer: encode.rs:115-126 (scales), 151-192 (block) -------- */

static float q8_0_scale(const float *x) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
    return amax / 127.0f;
}

static void encode_q8_0(const float *x, uint8_t *b) {
    memset(b, 0, 34);
    float d = q8_0_scale(x);
    float inv = d != 0.0f ? 1.0f / d : 0.0f;
    put_f16(b, 0, oracle_f32_to_f16(d));
    for (int j = 0; j < 32; ++j) b[2 + j] = (uint8_t)sat_i8(roundf(x[j] * inv));
}

/* ---- K encoders: encode_k.rs ---------------------------------------------- */

/* encode_k.rs:37-42; returns 0 on success */
static int nearest(float x, int32_t *out) {
    if (!is_finite_f(x) || fabsf(x) > 4194303.0f) return -1;
    *out = (int32_t)rintf(x);
    return 0;
}
static int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* encode_k.rs:43-50 */
static int put_half_checked(uint8_t *out, size_t offset, float x) {
    uint16_t bits = oracle_f32_to_f16(x);
    if ((bits & 0x7c00u) == 0x7c00u) return -1;
    put_f16(out, offset, bits);
    return 0;
}

/* encode_k.rs:70-137 with rmse = 1 and no importance weights (the Q6_K use) */
static int make_qx_rmse1(const float *x, int n, int32_t nmax, int32_t *levels, float *scale_out) {
    float maximum = 0.0f, magnitude = 0.0f;
    for (int i = 0; i < n; ++i) { /* signed_max, encode_k.rs:51-61 */
        if (fabsf(x[i]) > magnitude) {
            magnitude = fabsf(x[i]);
            maximum = x[i];
        }
    }
    if (magnitude < 1e-15f) {
        for (int i = 0; i < n; ++i) levels[i] = 0;
        *scale_out = 0.0f;
        return 0;
    }
    float inverse = (float)(-nmax) / maximum;
    float sum_lx = 0.0f, sum_l2 = 0.0f;
    for (int i = 0; i < n; ++i) {
        int32_t l;
        if (nearest(inverse * x[i], &l)) return -1;
        l = clampi(l, -nmax, nmax - 1);
        levels[i] = l + nmax;
        float w = x[i] * x[i];
        sum_lx += w * x[i] * (float)l;
        sum_l2 += w * (float)l * (float)l;
    }
    if (!is_finite_f(sum_lx) || !is_finite_f(sum_l2)) return -1;
    float scale = sum_l2 != 0.0f ? sum_lx / sum_l2 : 0.0f;
    float best = scale * sum_lx;
    for (int step = -9; step <= 9; ++step) {
        if (step == 0) continue;
        inverse = -((float)nmax + 0.1f * (float)step) / maximum;
        sum_lx = 0.0f;
        sum_l2 = 0.0f;
        for (int i = 0; i < n; ++i) {
            int32_t l;
            if (nearest(inverse * x[i], &l)) return -1;
            l = clampi(l, -nmax, nmax - 1);
            float w = x[i] * x[i];
            sum_lx += w * x[i] * (float)l;
            sum_l2 += w * (float)l * (float)l;
        }
        if (!is_finite_f(sum_lx) || !is_finite_f(sum_l2)) return -1;
        if (sum_l2 > 0.0f && sum_lx * sum_lx > best * sum_l2) {
            for (int i = 0; i < n; ++i) {
                int32_t l;
                if (nearest(inverse * x[i], &l)) return -1;
                levels[i] = nmax + clampi(l, -nmax, nmax - 1);
            }
            scale = sum_lx / sum_l2;
            best = scale * sum_lx;
        }
    }
    if (!is_finite_f(scale)) return -1;
    *scale_out = scale;
    return 0;
}

/* encode_k.rs:189-279 (make_qkx2_quants); use_mad = false for Q4_K */
static int make_affine2(const float *x, int n, int32_t nmax, const float *weights,
                        int32_t *levels, float rmin, float rdelta, int steps, int use_mad,
                        float *scale_out, float *min_out) {
    float minimum = x[0], maximum = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < minimum) minimum = x[i];
        if (x[i] > maximum) maximum = x[i];
        sum_w += weights[i];
        sum_x += weights[i] * x[i];
    }
    if (!is_finite_f(sum_w) || !is_finite_f(sum_x)) return -1;
    if (minimum > 0.0f) minimum = 0.0f;
    if (maximum == minimum) {
        for (int i = 0; i < n; ++i) levels[i] = 0;
        *scale_out = 0.0f;
        *min_out = -minimum;
        return 0;
    }
    float inverse = (float)nmax / (maximum - minimum);
    float scale = 1.0f / inverse;
    float best_error = 0.0f;
    for (int i = 0; i < n; ++i) {
        int32_t l;
        if (nearest(inverse * (x[i] - minimum), &l)) return -1;
        levels[i] = clampi(l, 0, nmax);
        float difference = scale * (float)levels[i] + minimum - x[i];
        float error = use_mad ? fabsf(difference) : difference * difference;
        best_error += weights[i] * error;
    }
    if (steps < 1) {
        if (!is_finite_f(scale)) return -1;
        *scale_out = scale;
        *min_out = -minimum;
        return 0;
    }
    int32_t candidate[32];
    for (int step = 0; step <= steps; ++step) {
        inverse = (rmin + rdelta * (float)step + (float)nmax) / (maximum - minimum);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        for (int i = 0; i < n; ++i) {
            int32_t l;
            if (nearest(inverse * (x[i] - minimum), &l)) return -1;
            l = clampi(l, 0, nmax);
            candidate[i] = l;
            float w = weights[i];
            sum_l += w * (float)l;
            sum_l2 += w * (float)l * (float)l;
            sum_xl += w * (float)l * x[i];
        }
        float determinant = sum_w * sum_l2 - sum_l * sum_l;
        if (determinant > 0.0f) {
            float candidate_scale = (sum_w * sum_xl - sum_x * sum_l) / determinant;
            float candidate_minimum = (sum_l2 * sum_x - sum_l * sum_xl) / determinant;
            if (candidate_minimum > 0.0f) {
                candidate_minimum = 0.0f;
                candidate_scale = sum_xl / sum_l2;
            }
            float error = 0.0f;
            for (int i = 0; i < n; ++i) {
                float difference = candidate_scale * (float)candidate[i] + candidate_minimum - x[i];
                difference = use_mad ? fabsf(difference) : difference * difference;
                error += weights[i] * difference;
            }
            if (error < best_error) {
                memcpy(levels, candidate, sizeof(int32_t) * (size_t)n);
                best_error = error;
                scale = candidate_scale;
                minimum = candidate_minimum;
            }
        }
    }
    if (!is_finite_f(scale) || !is_finite_f(-minimum)) return -1;
    *scale_out = scale;
    *min_out = -minimum;
    return 0;
}

/* encode_k.rs:410-419 */
static void pack_scale_min(uint8_t *out, int sub, uint8_t scale, uint8_t minimum) {
    if (sub < 4) {
        out[sub] = scale;
        out[sub + 4] = minimum;
    } else {
        out[sub + 4] = (uint8_t)((scale & 15) | ((minimum & 15) << 4));
        out[sub - 4] |= (uint8_t)((scale >> 4) << 6);
        out[sub] |= (uint8_t)((minimum >> 4) << 6);
    }
}

/* encode_k.rs:420-429 */
static void unpack_scale_min(const uint8_t *p, int sub, uint8_t *sc, uint8_t *mn) {
    if (sub < 4) {
        *sc = p[sub] & 63;
        *mn = p[sub + 4] & 63;
    } else {
        *sc = (uint8_t)((p[sub + 4] & 15) | ((p[sub - 4] >> 6) << 4));
        *mn = (uint8_t)((p[sub + 4] >> 4) | ((p[sub] >> 6) << 4));
    }
}

/* encode_k.rs:430-507: Q4_K (nmax 15, rmin -1, 20 steps; 144 bytes) and Q5_K
 * (nmax 31, rmin -0.5, 15 steps, high bits at 16..47; 176 bytes) */
static int encode_q45k_block(int five, const float *x, uint8_t *out) {
    const int32_t nmax = five ? 31 : 15;
    const int qpos = five ? 48 : 16;
    int32_t levels[256];
    float scales[8], minima[8];
    float maximum_scale = 0.0f, maximum_minimum = 0.0f;
    memset(out, 0, five ? 176 : 144);
    for (int sub = 0; sub < 8; ++sub) {
        const float *values = x + sub * 32;
        float square_sum = 0.0f;
        for (int i = 0; i < 32; ++i) square_sum = square_sum + values[i] * values[i];
        float average = sqrtf(square_sum / 32.0f);
        if (!is_finite_f(average)) return -1;
        float weights[32];
        for (int i = 0; i < 32; ++i) weights[i] = average + fabsf(values[i]);
        float scale, minimum;
        if (make_affine2(values, 32, nmax, weights, levels + sub * 32, five ? -0.5f : -1.0f, 0.1f, five ? 15 : 20,
                         0, &scale, &minimum))
            return -1;
        scales[sub] = scale;
        minima[sub] = minimum;
        if (scale > maximum_scale) maximum_scale = scale;
        if (minimum > maximum_minimum) maximum_minimum = minimum;
    }
    float inverse_scale = maximum_scale > 0.0f ? 63.0f / maximum_scale : 0.0f;
    float inverse_minimum = maximum_minimum > 0.0f ? 63.0f / maximum_minimum : 0.0f;
    for (int sub = 0; sub < 8; ++sub) {
        int32_t s, m;
        if (nearest(inverse_scale * scales[sub], &s)) return -1;
        if (nearest(inverse_minimum * minima[sub], &m)) return -1;
        if (s > 63) s = 63;
        if (m > 63) m = 63;
        pack_scale_min(out + 4, sub, (uint8_t)s, (uint8_t)m);
    }
    if (put_half_checked(out, 0, maximum_scale / 63.0f)) return -1;
    if (put_half_checked(out, 2, maximum_minimum / 63.0f)) return -1;
    for (int sub = 0; sub < 8; ++sub) {
        uint8_t sc, mn;
        unpack_scale_min(out + 4, sub, &sc, &mn);
        float scale = half_at(out, 0) * (float)sc;
        if (scale == 0.0f) continue;
        float minimum = half_at(out, 2) * (float)mn;
        for (int j = 0; j < 32; ++j) {
            int idx = sub * 32 + j;
            int32_t l;
            if (nearest((x[idx] + minimum) / scale, &l)) return -1;
            levels[idx] = clampi(l, 0, nmax);
        }
    }
    for (int group = 0; group < 4; ++group) {
        for (int j = 0; j < 32; ++j) {
            uint8_t low = (uint8_t)levels[group * 64 + j];
            uint8_t high = (uint8_t)levels[group * 64 + j + 32];
            if (five) {
                if (low > 15) out[16 + j] |= (uint8_t)(1 << (2 * group));
                if (high > 15) out[16 + j] |= (uint8_t)(2 << (2 * group));
            }
            out[qpos + group * 32 + j] = (uint8_t)((low & 15) | ((high & 15) << 4));
        }
    }
    return 0;
}
static int encode_q4k_block(const float *x, uint8_t *out) { return encode_q45k_block(0, x, out); }

/* encode_k.rs:346-355 */
static void pack_two_bits(const int32_t *levels, uint8_t *out) {
    for (int group = 0; group < 2; ++group)
        for (int j = 0; j < 32; ++j)
            out[group * 32 + j] = (uint8_t)((uint8_t)levels[group * 128 + j] | ((uint8_t)levels[group * 128 + j + 32] << 2) |
                                            ((uint8_t)levels[group * 128 + j + 64] << 4) |
                                            ((uint8_t)levels[group * 128 + j + 96] << 6));
}

/* encode_k.rs:292-345 (Q2_K: 16 groups of 16, make_affine2 with nmax 3, rmin
 * -0.5, 15 steps, absolute-error objective; 84 bytes) */
static int encode_q2k_block(const float *x, uint8_t *out) {
    int32_t levels[256];
    float scales[16], minima[16];
    float maximum_scale = 0.0f, maximum_minimum = 0.0f;
    memset(out, 0, 84);
    for (int sub = 0; sub < 16; ++sub) {
        const float *values = x + sub * 16;
        float weights[16];
        for (int i = 0; i < 16; ++i) weights[i] = fabsf(values[i]);
        float scale, minimum;
        if (make_affine2(values, 16, 3, weights, levels + sub * 16, -0.5f, 0.1f, 15, 1, &scale, &minimum))
            return -1;
        scales[sub] = scale;
        minima[sub] = minimum;
        if (scale > maximum_scale) maximum_scale = scale;
        if (minimum > maximum_minimum) maximum_minimum = minimum;
    }
    if (maximum_scale > 0.0f) {
        const float inverse = 15.0f / maximum_scale;
        for (int sub = 0; sub < 16; ++sub) {
            int32_t l;
            if (nearest(inverse * scales[sub], &l)) return -1;
            out[sub] = (uint8_t)l;
        }
        if (put_half_checked(out, 80, maximum_scale / 15.0f)) return -1;
    }
    if (maximum_minimum > 0.0f) {
        const float inverse = 15.0f / maximum_minimum;
        for (int sub = 0; sub < 16; ++sub) {
            int32_t l;
            if (nearest(inverse * minima[sub], &l)) return -1;
            out[sub] |= (uint8_t)((uint8_t)l << 4);
        }
        if (put_half_checked(out, 82, maximum_minimum / 15.0f)) return -1;
    }
    for (int sub = 0; sub < 16; ++sub) {
        const float scale = half_at(out, 80) * (float)(out[sub] & 15);
        if (scale == 0.0f) continue;
        const float minimum = half_at(out, 82) * (float)(out[sub] >> 4);
        for (int j = 0; j < 16; ++j) {
            const int idx = sub * 16 + j;
            int32_t l;
            if (nearest((x[idx] + minimum) / scale, &l)) return -1;
            levels[idx] = clampi(l, 0, 3);
        }
    }
    pack_two_bits(levels, out + 16);
    return 0;
}

/* encode_k.rs:51-61 */
static void signed_max(const float *x, int n, float *maximum, float *magnitude) {
    float mag = 0.0f, mx = 0.0f;
    for (int i = 0; i < n; ++i)
        if (fabsf(x[i]) > mag) {
            mag = fabsf(x[i]);
            mx = x[i];
        }
    *maximum = mx;
    *magnitude = mag;
}

/* encode_k.rs:138-185 (make_q3: iterative refinement, weights x^2) */
static int make_q3(const float *x, int n, int32_t nmax, int32_t *levels, float *scale_out) {
    float maximum, magnitude;
    signed_max(x, n, &maximum, &magnitude);
    if (magnitude < 1e-15f) {
        for (int i = 0; i < n; ++i) levels[i] = 0;
        *scale_out = 0.0f;
        return 0;
    }
    const float inverse = -(float)nmax / maximum;
    float sum_lx = 0.0f, sum_l2 = 0.0f;
    for (int i = 0; i < n; ++i) {
        int32_t l;
        if (nearest(inverse * x[i], &l)) return -1;
        l = clampi(l, -nmax, nmax - 1);
        levels[i] = l;
        const float w = x[i] * x[i];
        sum_lx += w * x[i] * (float)l;
        sum_l2 += w * (float)l * (float)l;
    }
    if (!is_finite_f(sum_lx) || !is_finite_f(sum_l2)) return -1;
    for (int it = 0; it < 5; ++it) {
        int changed = 0;
        for (int i = 0; i < n; ++i) {
            const float v = x[i], w = v * v;
            float lx = sum_lx - w * v * (float)levels[i];
            if (lx > 0.0f) {
                float l2 = sum_l2 - w * (float)levels[i] * (float)levels[i];
                int32_t next;
                if (nearest(v * l2 / lx, &next)) return -1;
                next = clampi(next, -nmax, nmax - 1);
                if (next != levels[i]) {
                    lx += w * v * (float)next;
                    l2 += w * (float)next * (float)next;
                    if (l2 > 0.0f && lx * lx * sum_l2 > sum_lx * sum_lx * l2) {
                        levels[i] = next;
                        sum_lx = lx;
                        sum_l2 = l2;
                        changed = 1;
                    }
                }
            }
        }
        if (!changed) break;
    }
    for (int i = 0; i < n; ++i) levels[i] += nmax;
    const float scale = sum_l2 > 0.0f ? sum_lx / sum_l2 : 0.0f;
    if (!is_finite_f(scale)) return -1;
    *scale_out = scale;
    return 0;
}

/* encode_k.rs:357-409 (Q3_K: 16 groups of 16, signed 6-bit scales, the high
 * bit of each 3-bit level in hmask; 110 bytes) */
static int encode_q3k_block(const float *x, uint8_t *out) {
    int32_t levels[256];
    float scales[16];
    float maximum_scale = 0.0f, maximum_magnitude = 0.0f;
    memset(out, 0, 110);
    for (int sub = 0; sub < 16; ++sub) {
        if (make_q3(x + sub * 16, 16, 4, levels + sub * 16, &scales[sub])) return -1;
        if (fabsf(scales[sub]) > maximum_magnitude) {
            maximum_magnitude = fabsf(scales[sub]);
            maximum_scale = scales[sub];
        }
    }
    if (maximum_scale != 0.0f) {
        const float inverse = -32.0f / maximum_scale;
        for (int sub = 0; sub < 16; ++sub) {
            int32_t l;
            if (nearest(inverse * scales[sub], &l)) return -1;
            const uint8_t u = (uint8_t)(clampi(l, -32, 31) + 32);
            if (sub < 8)
                out[96 + sub] = u & 15;
            else
                out[96 + sub - 8] |= (uint8_t)((u & 15) << 4);
            out[104 + sub % 4] |= (uint8_t)((u >> 4) << (2 * (sub / 4)));
        }
        if (put_half_checked(out, 108, 1.0f / inverse)) return -1;
    }
    for (int sub = 0; sub < 16; ++sub) {
        const uint8_t low = sub < 8 ? (out[96 + sub] & 15) : (out[96 + sub - 8] >> 4);
        const int32_t sc = (int32_t)(low | (((out[104 + sub % 4] >> (2 * (sub / 4))) & 3) << 4)) - 32;
        const float scale = half_at(out, 108) * (float)sc;
        if (scale == 0.0f) continue;
        for (int j = 0; j < 16; ++j) {
            const int idx = sub * 16 + j;
            int32_t l;
            if (nearest(x[idx] / scale, &l)) return -1;
            levels[idx] = clampi(l, -4, 3) + 4;
        }
    }
    for (int j = 0; j < 256; ++j)
        if (levels[j] > 3) {
            out[j % 32] |= (uint8_t)(1 << (j / 32));
            levels[j] -= 4;
        }
    pack_two_bits(levels, out + 32);
    return 0;
}

/* encode_k.rs:508-561 without importance weights; out is 210 bytes */
static int encode_q6k_block(const float *x, uint8_t *out) {
    int32_t levels[256];
    float scales[16];
    float maximum_scale = 0.0f, maximum_magnitude = 0.0f;
    memset(out, 0, 210);
    for (int sub = 0; sub < 16; ++sub) {
        if (make_qx_rmse1(x + sub * 16, 16, 32, levels + sub * 16, &scales[sub])) return -1;
        if (fabsf(scales[sub]) > maximum_magnitude) {
            maximum_magnitude = fabsf(scales[sub]);
            maximum_scale = scales[sub];
        }
    }
    if (maximum_magnitude < 1e-15f) return 0;
    float inverse = -128.0f / maximum_scale;
    if (put_half_checked(out, 208, 1.0f / inverse)) return -1;
    for (int sub = 0; sub < 16; ++sub) {
        int32_t l;
        if (nearest(inverse * scales[sub], &l)) return -1;
        if (l > 127) l = 127;
        out[192 + sub] = (uint8_t)l;
    }
    for (int sub = 0; sub < 16; ++sub) {
        float scale = half_at(out, 208) * (float)(int8_t)out[192 + sub];
        if (scale == 0.0f) continue;
        for (int j = 0; j < 16; ++j) {
            int idx = sub * 16 + j;
            int32_t l;
            if (nearest(x[idx] / scale, &l)) return -1;
            levels[idx] = clampi(l, -32, 31) + 32;
        }
    }
    for (int group = 0; group < 2; ++group) {
        for (int j = 0; j < 32; ++j) {
            uint8_t a = (uint8_t)levels[group * 128 + j];
            uint8_t b = (uint8_t)levels[group * 128 + j + 32];
            uint8_t c = (uint8_t)levels[group * 128 + j + 64];
            uint8_t d = (uint8_t)levels[group * 128 + j + 96];
            out[group * 64 + j] = (uint8_t)((a & 15) | ((c & 15) << 4));
            out[group * 64 + j + 32] = (uint8_t)((b & 15) | ((d & 15) << 4));
            out[128 + group * 32 + j] =
                (uint8_t)((a >> 4) | ((b >> 4) << 2) | ((c >> 4) << 4) | ((d >> 4) << 6));
        }
    }
    return 0;
}

/* ---- quantize: encode.rs:10-100, encode_k.rs:11-33 ---------------------- */

int oracle_quantize_into(uint32_t t, const float *x, uint64_t n, uint8_t *out, uint64_t out_len,
                         oracle_error *err) {
    int rc = validate(t, out_len, n, err); /* encode.rs:38 */
    if (rc) return rc;
    if (t != T_Q8_0 && t != T_Q8_K && !k_weight(t)) return set_err(err, ORC_UNIMPLEMENTED, t, 0, 0);
    if (n && (!x || !out)) return set_err(err, ORC_INVALID_ARGUMENT, t, 0, 0);
    for (uint64_t i = 0; i < n; ++i) /* encode.rs:70-74, encode_k.rs:13-17 */
        if (!is_finite_f(x[i])) return set_err(err, ORC_NON_FINITE_INPUT, t, i, 0);
    uint64_t bs = oracle_block_size(t), ts = oracle_type_size(t), nb = n / bs;
    if (k_weight(t)) {
        /* encode_k::encode stages the whole row, then quantize_into copies it */
        uint8_t *staged = (uint8_t *)malloc(out_len ? out_len : 1);
        if (!staged) return set_err(err, ORC_ALLOCATION_FAILED, t, 0, 0);
        for (uint64_t b = 0; b < nb; ++b) {
            const float *xb = x + b * bs;
            uint8_t *ob = staged + b * ts;
            int bad = t == T_Q2_K   ? encode_q2k_block(xb, ob)
                      : t == T_Q3_K ? encode_q3k_block(xb, ob)
                      : t == T_Q4_K ? encode_q4k_block(xb, ob)
                      : t == T_Q5_K ? encode_q45k_block(1, xb, ob)
                                    : encode_q6k_block(xb, ob);
            if (bad) {
                free(staged);
                return set_err(err, ORC_UNREPRESENTABLE_SCALE, t, b, 0);
            }
        }
        memcpy(out, staged, out_len);
        free(staged);
        return OK(err);
    }
    if (t == T_Q8_K) {
        rc = preflight_q8k(x, n, err);
        if (rc) return rc;
        for (uint64_t b = 0; b < nb; ++b) encode_q8k(x + b * 256, out + b * 292);
        return OK(err);
    }
    /* Q8_0: per-block scale preflight, encode.rs:80-90 (m is 0 for Q8_0) */
    for (uint64_t b = 0; b < nb; ++b) {
        float d = q8_0_scale(x + b * 32);
        if (!is_finite_f(d) || (d != 0.0f && !is_finite_f(1.0f / d)) ||
            (oracle_f32_to_f16(d) & 0x7c00u) == 0x7c00u)
            return set_err(err, ORC_UNREPRESENTABLE_SCALE, t, b, 0);
    }
    for (uint64_t b = 0; b < nb; ++b) encode_q8_0(x + b * 32, out + b * 34);
    return OK(err);
}

/* ---- decoders: decode.rs ------------------------------------------------ */

/* decode.rs:205-214 and matvec_extra.rs:212-221 (same unpacking) */
static void scale_min_k(const uint8_t *p, int j, int32_t *sc, int32_t *mn) {
    if (j < 4) {
        *sc = p[j] & 63;
        *mn = p[j + 4] & 63;
    } else {
        *sc = (p[j + 4] & 15) | ((p[j - 4] >> 6) << 4);
        *mn = (p[j + 4] >> 4) | ((p[j] >> 6) << 4);
    }
}

int oracle_dequantize_into(uint32_t t, const uint8_t *b, uint64_t len, float *y, uint64_t n,
                           oracle_error *err) {
    int rc = validate(t, len, n, err);
    if (rc) return rc;
    if (t != T_Q8_0 && t != T_Q8_K && !k_weight(t)) return set_err(err, ORC_UNIMPLEMENTED, t, 0, 0);
    if (n && (!b || !y)) return set_err(err, ORC_INVALID_ARGUMENT, t, 0, 0);
    uint64_t bs = oracle_block_size(t), ts = oracle_type_size(t);
    for (uint64_t blk = 0; blk < n / bs; ++blk) {
        const uint8_t *x = b + blk * ts;
        float *o = y + blk * bs;
        if (t == T_Q8_0) { /* decode.rs:17-23 */
            float d = half_at(x, 0);
            for (int j = 0; j < 32; ++j) o[j] = (float)(int8_t)x[2 + j] * d;
        } else if (t == T_Q8_K) { /* decode.rs:44-49 */
            float d = f32le(x, 0);
            for (int j = 0; j < 256; ++j) o[j] = d * (float)(int8_t)x[4 + j];
        } else if (t == T_Q4_K || t == T_Q5_K) { /* decode.rs:216-235 */
            const int five = t == T_Q5_K, qbase = five ? 48 : 16;
            float d = half_at(x, 0), mn = half_at(x, 2);
            for (int group = 0; group < 4; ++group) {
                for (int side = 0; side < 2; ++side) {
                    int32_t sc, m;
                    scale_min_k(x + 4, group * 2 + side, &sc, &m);
                    float dl = d * (float)sc;
                    float ml = mn * (float)m;
                    for (int j = 0; j < 32; ++j) {
                        uint8_t q = (x[qbase + group * 32 + j] >> (side * 4)) & 15;
                        if (five && (x[16 + j] & (1 << (group * 2 + side)))) q += 16;
                        o[group * 64 + side * 32 + j] = dl * (float)q - ml;
                    }
                }
            }
        } else if (t == T_Q2_K) { /* decode.rs:159-175 */
            const float d = half_at(x, 80), mn = half_at(x, 82);
            for (int group = 0; group < 2; ++group)
                for (int lane = 0; lane < 4; ++lane)
                    for (int side = 0; side < 2; ++side) {
                        const uint8_t sc = x[group * 8 + lane * 2 + side];
                        const float dl = d * (float)(sc & 15), ml = mn * (float)(sc >> 4);
                        for (int j = 0; j < 16; ++j)
                            o[group * 128 + lane * 32 + side * 16 + j] =
                                dl * (float)((x[16 + group * 32 + side * 16 + j] >> (2 * lane)) & 3) - ml;
                    }
        } else if (t == T_Q3_K) { /* decode.rs:177-202 */
            const float d = half_at(x, 108);
            const uint8_t *q = x + 32, *packed = x + 96;
            int32_t sc[16];
            for (int j = 0; j < 4; ++j) {
                sc[j] = (packed[j] & 15) | ((packed[8 + j] & 3) << 4);
                sc[4 + j] = (packed[4 + j] & 15) | (((packed[8 + j] >> 2) & 3) << 4);
                sc[8 + j] = (packed[j] >> 4) | (((packed[8 + j] >> 4) & 3) << 4);
                sc[12 + j] = (packed[4 + j] >> 4) | (((packed[8 + j] >> 6) & 3) << 4);
            }
            for (int group = 0; group < 2; ++group)
                for (int lane = 0; lane < 4; ++lane) {
                    const int mask = 1 << (group * 4 + lane);
                    for (int side = 0; side < 2; ++side) {
                        const float dl = d * (float)(sc[group * 8 + lane * 2 + side] - 32);
                        for (int j = 0; j < 16; ++j) {
                            const int pos = side * 16 + j;
                            const int32_t v = ((q[group * 32 + pos] >> (2 * lane)) & 3) - ((x[pos] & mask) ? 0 : 4);
                            o[group * 128 + lane * 32 + pos] = dl * (float)v;
                        }
                    }
                }
        } else { /* Q6_K, decode.rs:237-258 */
            float d = half_at(x, 208);
            for (int group = 0; group < 2; ++group) {
                for (int j = 0; j < 32; ++j) {
                    uint8_t lo0 = x[group * 64 + j];
                    uint8_t lo1 = x[group * 64 + 32 + j];
                    uint8_t hi = x[128 + group * 32 + j];
                    uint8_t v[4] = {(uint8_t)((lo0 & 15) | ((hi & 3) << 4)),
                                    (uint8_t)((lo1 & 15) | (((hi >> 2) & 3) << 4)),
                                    (uint8_t)((lo0 >> 4) | (((hi >> 4) & 3) << 4)),
                                    (uint8_t)((lo1 >> 4) | (((hi >> 6) & 3) << 4))};
                    for (int side = 0; side < 4; ++side)
                        o[group * 128 + side * 32 + j] =
                            d * (float)(int8_t)x[192 + group * 8 + j / 16 + side * 2] *
                            (float)((int32_t)v[side] - 32);
                }
            }
        }
    }
    return OK(err);
}

/* ---- dots: matvec.rs:105-160, matvec_extra.rs:7-30, 223-294 ------------- */

static int32_t q8k_at(const uint8_t *y, int i) { return (int8_t)y[4 + i]; }
static int32_t bsum_at(const uint8_t *y, int i) { return (int16_t)u16le(y, 260 + 2 * (size_t)i); }

/* matvec.rs:115-160, Q8_0 branch */
static float dot_q8_0(const uint8_t *x, const uint8_t *y, uint64_t nb) {
    float sum = 0.0f;
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t *xb = x + b * 34, *yb = y + b * 34;
        float dx = half_at(xb, 0), dy = half_at(yb, 0);
        int32_t integer_sum = 0;
        for (int j = 0; j < 32; ++j) integer_sum += (int8_t)xb[2 + j] * (int8_t)yb[2 + j];
        sum += (float)integer_sum * (dx * dy);
    }
    return sum;
}

/* matvec_extra.rs:200-210 */
static void q3_scales(const uint8_t *x, int32_t sc[16]) {
    const uint8_t *p = x + 96;
    for (int j = 0; j < 4; ++j) {
        sc[j] = ((p[j] & 15) | ((p[8 + j] & 3) << 4)) - 32;
        sc[4 + j] = ((p[4 + j] & 15) | (((p[8 + j] >> 2) & 3) << 4)) - 32;
        sc[8 + j] = ((p[j] >> 4) | (((p[8 + j] >> 4) & 3) << 4)) - 32;
        sc[12 + j] = ((p[4 + j] >> 4) | (((p[8 + j] >> 6) & 3) << 4)) - 32;
    }
}

/* One Q3_K / Q4_K / Q5_K / Q6_K block: the 8 lane integers and (Q4_K, Q5_K)
 * the mins sum; Q2_K: lane 0 holds the whole integer sum (matvec_extra.rs:174-197
 * keeps one accumulator) and mins its mins sum. */
static void k_block_ints(uint32_t t, const uint8_t *xb, const uint8_t *yb, int32_t ints[8],
                         int32_t *mins_out) {
    for (int l = 0; l < 8; ++l) ints[l] = 0;
    *mins_out = 0;
    if (t == T_Q2_K) { /* matvec_extra.rs:181-192 */
        int32_t mins = 0, isum = 0;
        for (int j = 0; j < 16; ++j) mins += bsum_at(yb, j) * (xb[j] >> 4);
        for (int j = 0; j < 256; ++j) {
            int group = j / 128, lane = (j % 128) / 32, pos = j % 32;
            int32_t q = (xb[16 + group * 32 + pos] >> (2 * lane)) & 3;
            isum += (xb[j / 16] & 15) * q * q8k_at(yb, j);
        }
        ints[0] = isum;
        *mins_out = mins;
    } else if (t == T_Q3_K) { /* matvec_extra.rs:234-248 */
        int32_t sc[16];
        q3_scales(xb, sc);
        for (int j = 0; j < 256; ++j) {
            int group = j / 128, lane = (j % 128) / 32, pos = j % 32;
            int32_t low = (xb[32 + group * 32 + pos] >> (2 * lane)) & 3;
            int32_t q = low - ((xb[pos] & (1 << (group * 4 + lane))) == 0 ? 4 : 0);
            ints[j % 8] += sc[j / 16] * q * q8k_at(yb, j);
        }
    } else if (t == T_Q4_K || t == T_Q5_K) { /* matvec_extra.rs:250-270 */
        const int five = t == T_Q5_K, qpos = five ? 48 : 16;
        int32_t mins = 0;
        for (int sub = 0; sub < 8; ++sub) {
            int32_t scale, mn;
            scale_min_k(xb + 4, sub, &scale, &mn);
            mins += (bsum_at(yb, 2 * sub) + bsum_at(yb, 2 * sub + 1)) * mn;
            for (int l = 0; l < 32; ++l) {
                int j = sub * 32 + l;
                int32_t q = (xb[qpos + sub / 2 * 32 + l] >> (4 * (sub % 2))) & 15;
                if (five && (xb[16 + l] & (1 << sub))) q += 16;
                ints[j % 8] += scale * q * q8k_at(yb, j);
            }
        }
        *mins_out = mins;
    } else { /* Q6_K, matvec_extra.rs:272-281 */
        for (int j = 0; j < 256; ++j) {
            int group = j / 128, side = (j % 128) / 32, pos = j % 32;
            int32_t low = (xb[group * 64 + (side % 2) * 32 + pos] >> (4 * (side / 2))) & 15;
            int32_t high = (xb[128 + group * 32 + pos] >> (2 * side)) & 3;
            int32_t q = (low | (high << 4)) - 32;
            ints[j % 8] += (int8_t)xb[192 + j / 16] * q * q8k_at(yb, j);
        }
    }
}

/* matvec_extra.rs:223-294 */
static float dot_k_lanes(uint32_t t, const uint8_t *x, const uint8_t *y, uint64_t nb) {
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sum = 0.0f;
    uint64_t ts = oracle_type_size(t);
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t *xb = x + b * ts, *yb = y + b * 292;
        int32_t ints[8], mins;
        float d;
        k_block_ints(t, xb, yb, ints, &mins);
        if (t == T_Q4_K || t == T_Q5_K) {
            d = half_at(xb, 0) * f32le(yb, 0);
            float dmin = half_at(xb, 2) * f32le(yb, 0);
            sum -= dmin * (float)mins;
        } else if (t == T_Q3_K) {
            d = half_at(xb, 108) * f32le(yb, 0);
        } else {
            d = half_at(xb, 208) * f32le(yb, 0);
        }
        for (int l = 0; l < 8; ++l) lanes[l] += d * (float)ints[l];
    }
    for (int l = 0; l < 8; ++l) sum += lanes[l];
    return sum;
}

/* matvec_extra.rs:174-198 */
static float dot_q2k(const uint8_t *x, const uint8_t *y, uint64_t nb) {
    float sum = 0.0f;
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t *xb = x + b * 84, *yb = y + b * 292;
        int32_t ints[8], mins;
        k_block_ints(T_Q2_K, xb, yb, ints, &mins);
        const float d = f32le(yb, 0) * half_at(xb, 80);
        const float mn = f32le(yb, 0) * half_at(xb, 82);
        sum += d * (float)ints[0] - mn * (float)mins;
    }
    return sum;
}

static float dot_unchecked(uint32_t t, const uint8_t *x, const uint8_t *y, uint64_t elements) {
    uint64_t nb = elements / oracle_block_size(t);
    return t == T_Q8_0 ? dot_q8_0(x, y, nb) : t == T_Q2_K ? dot_q2k(x, y, nb) : dot_k_lanes(t, x, y, nb);
}

void oracle_block_sums(uint32_t t, const uint8_t *w, const uint8_t *a, uint64_t nb,
                       int32_t *isum, int32_t *imin) {
    for (uint64_t b = 0; b < nb; ++b) {
        if (t == T_Q8_0) {
            const uint8_t *xb = w + b * 34, *yb = a + b * 34;
            int32_t s = 0;
            for (int j = 0; j < 32; ++j) s += (int8_t)xb[2 + j] * (int8_t)yb[2 + j];
            isum[b] = s;
            imin[b] = 0;
        } else {
            int32_t ints[8], mins;
            k_block_ints(t, w + b * oracle_type_size(t), a + b * 292, ints, &mins);
            int32_t s = 0;
            for (int l = 0; l < 8; ++l) s += ints[l];
            isum[b] = s;
            imin[b] = mins;
        }
    }
}

/* Tolerance helper, not a restatement: the sum of the absolute values of every
 * f32 term one row's dot adds, in f64.  Q4_K: |d_w d_a| sum_j |sc q q8| +
 * |dmin_w d_a| sum_s min_s |bsum[2s]+bsum[2s+1]|; Q6_K: |d_w d_a| sum_j
 * |sc (q6-32) q8|; Q8_0: |dx dy| sum_j |xq yq|.  Any partition of these
 * products into f32 partial sums has absolute terms bounded by this value. */
double oracle_abs_terms(uint32_t t, const uint8_t *w, const uint8_t *a, uint64_t nb) {
    double total = 0.0;
    for (uint64_t b = 0; b < nb; ++b) {
        if (t == T_Q8_0) {
            const uint8_t *xb = w + b * 34, *yb = a + b * 34;
            double s = 0.0;
            for (int j = 0; j < 32; ++j) s += fabs((double)((int8_t)xb[2 + j] * (int8_t)yb[2 + j]));
            total += fabs((double)half_at(xb, 0) * (double)half_at(yb, 0)) * s;
        } else if (t == T_Q4_K) {
            const uint8_t *xb = w + b * 144, *yb = a + b * 292;
            double s = 0.0, m = 0.0;
            for (int sub = 0; sub < 8; ++sub) {
                int32_t scale, mn;
                scale_min_k(xb + 4, sub, &scale, &mn);
                m += (double)mn * fabs((double)(bsum_at(yb, 2 * sub) + bsum_at(yb, 2 * sub + 1)));
                for (int l = 0; l < 32; ++l) {
                    int32_t q = (xb[16 + sub / 2 * 32 + l] >> (4 * (sub % 2))) & 15;
                    s += fabs((double)(scale * q * q8k_at(yb, sub * 32 + l)));
                }
            }
            const double da = fabs((double)f32le(yb, 0));
            total += fabs((double)half_at(xb, 0)) * da * s + fabs((double)half_at(xb, 2)) * da * m;
        } else if (t == T_Q2_K || t == T_Q3_K || t == T_Q5_K) {
            /* per element |scale * q * q8| (Q2_K, Q5_K) or |sc * q * q8| (Q3_K),
             * and the mins terms of Q2_K / Q5_K */
            const uint8_t *xb = w + b * oracle_type_size(t), *yb = a + b * 292;
            double s = 0.0, m = 0.0, dw, dm = 0.0;
            if (t == T_Q2_K) {
                for (int j = 0; j < 16; ++j) m += (double)(xb[j] >> 4) * fabs((double)bsum_at(yb, j));
                for (int j = 0; j < 256; ++j) {
                    int group = j / 128, lane = (j % 128) / 32, pos = j % 32;
                    int32_t q = (xb[16 + group * 32 + pos] >> (2 * lane)) & 3;
                    s += fabs((double)((xb[j / 16] & 15) * q * q8k_at(yb, j)));
                }
                dw = half_at(xb, 80), dm = half_at(xb, 82);
            } else if (t == T_Q3_K) {
                int32_t sc[16];
                q3_scales(xb, sc);
                for (int j = 0; j < 256; ++j) {
                    int group = j / 128, lane = (j % 128) / 32, pos = j % 32;
                    int32_t q = ((xb[32 + group * 32 + pos] >> (2 * lane)) & 3) -
                                ((xb[pos] & (1 << (group * 4 + lane))) == 0 ? 4 : 0);
                    s += fabs((double)(sc[j / 16] * q * q8k_at(yb, j)));
                }
                dw = half_at(xb, 108);
            } else {
                for (int sub = 0; sub < 8; ++sub) {
                    int32_t scale, mn;
                    scale_min_k(xb + 4, sub, &scale, &mn);
                    m += (double)mn * fabs((double)(bsum_at(yb, 2 * sub) + bsum_at(yb, 2 * sub + 1)));
                    for (int l = 0; l < 32; ++l) {
                        int32_t q = (xb[48 + sub / 2 * 32 + l] >> (4 * (sub % 2))) & 15;
                        if (xb[16 + l] & (1 << sub)) q += 16;
                        s += fabs((double)(scale * q * q8k_at(yb, sub * 32 + l)));
                    }
                }
                dw = half_at(xb, 0), dm = half_at(xb, 2);
            }
            const double da = fabs((double)f32le(yb, 0));
            total += fabs(dw) * da * s + fabs(dm) * da * m;
        } else {
            const uint8_t *xb = w + b * 210, *yb = a + b * 292;
            double s = 0.0;
            for (int j = 0; j < 256; ++j) {
                int group = j / 128, side = (j % 128) / 32, pos = j % 32;
                int32_t low = (xb[group * 64 + (side % 2) * 32 + pos] >> (4 * (side / 2))) & 15;
                int32_t high = (xb[128 + group * 32 + pos] >> (2 * side)) & 3;
                int32_t q = (low | (high << 4)) - 32;
                s += fabs((double)((int8_t)xb[192 + j / 16] * q * q8k_at(yb, j)));
            }
            total += fabs((double)half_at(xb, 208) * (double)f32le(yb, 0)) * s;
        }
    }
    return total;
}

int oracle_dot_packed(uint32_t t, const uint8_t *w, uint64_t w_len, const uint8_t *act,
                      uint64_t act_len, uint64_t elements, float *out, oracle_error *err) {
    uint32_t at;
    int rc = oracle_matvec_activation_dtype(t, &at, err);
    if (rc) return rc;
    if (oracle_block_size(t) == 1) return set_err(err, ORC_UNSUPPORTED_MATVEC, t, 0, 0);
    if (!path_weight(t)) return set_err(err, ORC_UNIMPLEMENTED, t, 0, 0);
    rc = validate(t, w_len, elements, err);
    if (rc) return rc;
    rc = validate(at, act_len, elements, err);
    if (rc) return rc;
    if (!out || (elements && (!w || !act))) return set_err(err, ORC_INVALID_ARGUMENT, t, 0, 0);
    *out = dot_unchecked(t, w, act, elements);
    return OK(err);
}

/* ---- matvec / matmul ---------------------------------------------------- */

typedef struct {
    uint32_t t;
    const uint8_t *w;
    uint64_t row_bytes, cols, r0, r1;
    const uint8_t *act;
    float *y;
} rows_job;

static void *rows_worker(void *p) {
    rows_job *j = (rows_job *)p;
    for (uint64_t r = j->r0; r < j->r1; ++r)
        j->y[r] = dot_unchecked(j->t, j->w + r * j->row_bytes, j->act, j->cols);
    return NULL;
}

static void run_rows(uint32_t t, const uint8_t *w, uint64_t row_bytes, uint64_t rows,
                     uint64_t cols, const uint8_t *act, float *y, int threads) {
    if (threads <= 1 || rows < (uint64_t)threads) {
        rows_job j = {t, w, row_bytes, cols, 0, rows, act, y};
        rows_worker(&j);
        return;
    }
    pthread_t tid[256];
    rows_job jobs[256];
    int started[256];
    if (threads > 256) threads = 256;
    for (int i = 0; i < threads; ++i) {
        jobs[i] = (rows_job){t, w, row_bytes, cols, rows * (uint64_t)i / (uint64_t)threads,
                             rows * (uint64_t)(i + 1) / (uint64_t)threads, act, y};
        started[i] = pthread_create(&tid[i], NULL, rows_worker, &jobs[i]) == 0;
        if (!started[i]) rows_worker(&jobs[i]);
    }
    for (int i = 0; i < threads; ++i)
        if (started[i]) pthread_join(tid[i], NULL);
}

/* matvec.rs:31-55: the checks common to matvec and (per column) matmul */
static int check_matvec(uint32_t t, uint64_t w_len, uint64_t rows, uint64_t cols,
                        uint64_t x_len, uint32_t *at, uint64_t *row_bytes, oracle_error *err) {
    int rc = oracle_matvec_activation_dtype(t, at, err);
    if (rc) return rc;
    if (!path_weight(t)) return set_err(err, ORC_UNIMPLEMENTED, t, 0, 0);
    if (rows == 0 || cols == 0) return set_err(err, ORC_INVALID_MATRIX_SHAPE, t, rows, cols);
    if (x_len != cols) return set_err(err, ORC_INVALID_VECTOR_LENGTH, t, cols, x_len);
    rc = oracle_row_bytes(t, cols, row_bytes, err);
    if (rc) return rc;
    uint64_t expected;
    if (__builtin_mul_overflow(*row_bytes, rows, &expected))
        return set_err(err, ORC_SIZE_OVERFLOW, t, 0, 0);
    if (w_len != expected) return set_err(err, ORC_INVALID_LENGTH, t, expected, w_len);
    return OK(err);
}

int oracle_matvec(uint32_t t, const uint8_t *w, uint64_t w_len, uint64_t rows, uint64_t cols,
                  const float *x, uint64_t x_len, float *y, int threads, oracle_error *err) {
    uint32_t at;
    uint64_t row_bytes, act_bytes;
    int rc = check_matvec(t, w_len, rows, cols, x_len, &at, &row_bytes, err);
    if (rc) return rc;
    if (!w || !x || !y) return set_err(err, ORC_INVALID_ARGUMENT, t, 0, 0);
    for (uint64_t i = 0; i < cols; ++i)
        if (!is_finite_f(x[i])) return set_err(err, ORC_NON_FINITE_INPUT, t, i, 0);
    rc = oracle_row_bytes(at, cols, &act_bytes, err);
    if (rc) return rc;
    uint8_t *act = (uint8_t *)malloc(act_bytes);
    if (!act) return set_err(err, ORC_ALLOCATION_FAILED, t, 0, 0);
    rc = oracle_quantize_into(at, x, cols, act, act_bytes, err);
    if (rc) {
        free(act);
        return rc;
    }
    float *tmp = (float *)malloc(sizeof(float) * rows);
    if (!tmp) {
        free(act);
        return set_err(err, ORC_ALLOCATION_FAILED, t, 0, 0);
    }
    run_rows(t, w, row_bytes, rows, cols, act, tmp, threads);
    memcpy(y, tmp, sizeof(float) * rows);
    free(tmp);
    free(act);
    return OK(err);
}

int oracle_matmul(uint32_t t, const uint8_t *w, uint64_t w_len, uint64_t rows, uint64_t cols,
                  const float *x, uint64_t batch, float *y, int threads, oracle_error *err) {
    uint32_t at;
    uint64_t row_bytes, act_bytes;
    int rc = check_matvec(t, w_len, rows, cols, cols, &at, &row_bytes, err);
    if (rc) return rc;
    if (batch == 0) return set_err(err, ORC_INVALID_MATRIX_SHAPE, t, rows, 0);
    if (!w || !x || !y) return set_err(err, ORC_INVALID_ARGUMENT, t, 0, 0);
    rc = oracle_row_bytes(at, cols, &act_bytes, err);
    if (rc) return rc;
    uint64_t total;
    if (__builtin_mul_overflow(act_bytes, batch, &total))
        return set_err(err, ORC_SIZE_OVERFLOW, t, 0, 0);
    uint8_t *act = (uint8_t *)malloc(total ? total : 1);
    float *tmp = (float *)malloc(sizeof(float) * rows * batch);
    if (!act || !tmp) {
        free(act);
        free(tmp);
        return set_err(err, ORC_ALLOCATION_FAILED, t, 0, 0);
    }
    for (uint64_t b = 0; b < batch; ++b) { /* cpu_extra.rs:820, quantize propagates errors */
        rc = oracle_quantize_into(at, x + b * cols, cols, act + b * act_bytes, act_bytes, err);
        if (rc) {
            if (err) err->b = b; /* which column; `a` keeps the per-column payload */
            free(act);
            free(tmp);
            return rc;
        }
    }
    for (uint64_t b = 0; b < batch; ++b)
        run_rows(t, w, row_bytes, rows, cols, act + b * act_bytes, tmp + b * rows, threads);
    memcpy(y, tmp, sizeof(float) * rows * batch);
    free(act);
    free(tmp);
    return OK(err);
}

uint64_t oracle_argmax(const float *x, uint64_t n) {
    uint64_t best = 0;
    for (uint64_t i = 1; i < n; ++i)
        if (x[i] > x[best]) best = i;
    return best;
}
