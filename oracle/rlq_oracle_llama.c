/*
 * rlq_oracle_llama.c - CPU restatement of rust-llama's dense Llama decode
 * step (crates/model-runtime/src/llama.rs:222-392) with quantized matrices.
 *
 * TEST INFRASTRUCTURE ONLY (see rlq_oracle.h): the checker for the GPU
 * decode step.  The product library never links or calls it.
 *
 * Every f32 operation is written in the reference's order; the file is built
 * with -ffp-contract=off, so no multiply-add is fused.  The transcendental
 * calls (powf, sinf, cosf, expf) are glibc's, as are those of the reference
 * on x86_64-linux-gnu, where Rust's f32::powf / sin_cos / exp lower to libm.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "rlq_oracle.h"

static float bits_f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t f_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static int all_finite(const float *x, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i)
        if (!isfinite(x[i])) return 0;
    return 1;
}

/* crates/quant/src/cpu_math.rs:94-123 (the SSE2 four-lane exponential).  The
 * source branches once per four-lane vector, but the two branches give the
 * same value for every lane with |n| <= 126 (scale*p + scale in both), so the
 * value of each lane depends on that lane alone. */
float oracle_sse2_exp(float x) {
    const float z = x * bits_f(0x3fb8aa3bu) + bits_f(0x4b400000u);
    const float n = z - bits_f(0x4b400000u);
    const float b = (x - n * bits_f(0x3f317200u)) - n * bits_f(0x35bfbe8eu);
    const uint32_t exponent = f_bits(z) << 23;
    const float scale = bits_f(exponent + 0x3f800000u);
    const float squared = b * b;
    const float first = bits_f(0x3c072010u) * b + bits_f(0x3d2b9f17u);
    const float second = bits_f(0x3e2aaf33u) * b + bits_f(0x3efffedbu);
    const float polynomial = (first * squared + second) * squared + bits_f(0x3f7ffff6u) * b;
    if (!(fabsf(n) > 126.0f)) return polynomial * scale + scale;
    const uint32_t shift = n <= 0.0f ? 0x82000000u : 0u;
    const float high = bits_f(shift + 0x7f000000u);
    const float low = bits_f(exponent - shift);
    if (fabsf(n) > 192.0f) return high * high;
    return (low * polynomial + low) * high;
}

/* cpu_math.rs:28-53, SSE2 policy: the four-value prefix uses the SSE2
 * exponential, the tail (len % 4 values) libm's expf. */
void oracle_silu(float *v, uint64_t n) {
    const uint64_t prefix = n / 4 * 4;
    for (uint64_t i = 0; i < prefix; ++i) v[i] = v[i] / (1.0f + oracle_sse2_exp(0.0f - v[i]));
    for (uint64_t i = prefix; i < n; ++i) v[i] = v[i] / (1.0f + expf(-v[i]));
}

/* NaN-propagating adds of cpu_math.rs:127-144 (the first NaN operand wins). */
static float ordered_add_f32(float l, float r) {
    if (isnan(l)) return bits_f(f_bits(l) | 0x00400000u);
    if (isnan(r)) return bits_f(f_bits(r) | 0x00400000u);
    return l + r;
}
static double ordered_add_f64(double l, double r) {
    uint64_t u;
    if (isnan(l)) {
        memcpy(&u, &l, 8);
        u |= 0x0008000000000000ull;
        memcpy(&l, &u, 8);
        return l;
    }
    if (isnan(r)) {
        memcpy(&u, &r, 8);
        u |= 0x0008000000000000ull;
        memcpy(&r, &u, 8);
        return r;
    }
    return l + r;
}

/* crates/model-runtime/src/math.rs:293-318 with cpu_math.rs:60-91 (SSE2):
 * exp(v - max) per four-value group, the group summed as (e0+e1)+(e2+e3) in
 * f32 and added to an f64 sum; the tail uses expf.  0 on success. */
int oracle_softmax(float *v, uint64_t n) {
    if (n == 0) return ORC_INVALID_LENGTH;
    float max = -INFINITY;
    for (uint64_t i = 0; i < n; ++i) {
        if (isnan(v[i]) || v[i] == INFINITY) return ORC_NON_FINITE_INPUT;
        max = fmaxf(max, v[i]);
    }
    if (!isfinite(max)) return ORC_NON_FINITE_INPUT;
    const uint64_t prefix = n / 4 * 4;
    double sum = 0.0;
    for (uint64_t i = 0; i < prefix; i += 4) {
        float e[4];
        for (int k = 0; k < 4; ++k) e[k] = oracle_sse2_exp(v[i + k] - max);
        for (int k = 0; k < 4; ++k) v[i + k] = e[k];
        const float pairs = ordered_add_f32(ordered_add_f32(e[0], e[1]), ordered_add_f32(e[2], e[3]));
        sum = ordered_add_f64(sum, (double)pairs);
    }
    for (uint64_t i = prefix; i < n; ++i) {
        v[i] = expf(v[i] - max);
        sum = ordered_add_f64(sum, (double)v[i]);
    }
    if (!isfinite(sum) || sum <= 0.0) return ORC_NON_FINITE_INPUT;
    const float inverse = (float)(1.0 / sum);
    for (uint64_t i = 0; i < n; ++i) v[i] *= inverse;
    return ORC_OK;
}

/* The decode step's Error::NonFinite(name) (crates/model-runtime/src/
 * lib.rs:51) as step-internal codes, one per name the reference reports:
 * NF_BASE + the check number of rlq.h's rlq_nonfinite_check (the softmax's
 * own checks, math.rs:301-311, as 8).  oracle_llama_step turns them into
 * ORC_NON_FINITE {a = check, b = layer}. */
enum {
    NF_BASE = 100,
    NF_RMS_SCALE = NF_BASE + 1,       /* math.rs:218-220 */
    NF_RMS_OUTPUT = NF_BASE + 2,      /* math.rs:227 */
    NF_MATRIX_INPUT = NF_BASE + 3,    /* math.rs:152 */
    NF_MATRIX_OUTPUT = NF_BASE + 4,   /* math.rs:167 */
    NF_ATT_SCORE = NF_BASE + 5,       /* math.rs:476-478 */
    NF_ATT_OUTPUT = NF_BASE + 6,      /* math.rs:494 */
    NF_LAYER_OUTPUT = NF_BASE + 7,    /* llama.rs:378 */
    NF_SOFTMAX = NF_BASE + 8          /* math.rs:301-311 */
};

/* math.rs:214-228: squares summed in f64, the mean rounded to f32 before
 * epsilon is added; out = x * scale * w. */
static int rms_norm_checked(const float *x, const float *w, uint64_t n, float eps, float *out) {
    double sum = 0.0;
    for (uint64_t i = 0; i < n; ++i) sum += (double)(x[i] * x[i]);
    const float scale = 1.0f / sqrtf((float)(sum / (double)n) + eps);
    if (!isfinite(scale) || scale <= 0.0f) return NF_RMS_SCALE;
    for (uint64_t i = 0; i < n; ++i) out[i] = x[i] * scale * w[i];
    return all_finite(out, n) ? ORC_OK : NF_RMS_OUTPUT;
}
int oracle_rms_norm(const float *x, const float *w, uint64_t n, float eps, float *out) {
    return rms_norm_checked(x, w, n, eps, out) == ORC_OK ? ORC_OK : ORC_NON_FINITE_INPUT;
}

/* math.rs:322-334: adjacent-pair RoPE; theta starts at the position and is
 * multiplied by base^(-2/head_dim) after each pair. */
void oracle_rope(float *v, uint64_t len, uint64_t head_dim, uint64_t position, float base) {
    const float theta_scale = powf(base, -2.0f / (float)head_dim);
    for (uint64_t h = 0; h + head_dim <= len; h += head_dim) {
        float theta = (float)position;
        for (uint64_t i = 0; i + 1 < head_dim; i += 2) {
            const float s = sinf(theta), c = cosf(theta);
            const float x = v[h + i], y = v[h + i + 1];
            v[h + i] = x * c - y * s;
            v[h + i + 1] = x * s + y * c;
            theta *= theta_scale;
        }
    }
}

/* The (sin, cos) pairs oracle_rope uses at one position: table[2i] = sin,
 * table[2i+1] = cos of pair i's angle, i < head_dim/2. */
void oracle_rope_table(uint64_t head_dim, uint64_t position, float base, float *table) {
    const float theta_scale = powf(base, -2.0f / (float)head_dim);
    float theta = (float)position;
    for (uint64_t i = 0; i < head_dim / 2; ++i) {
        table[2 * i] = sinf(theta);
        table[2 * i + 1] = cosf(theta);
        theta *= theta_scale;
    }
}

/* math.rs:427-497 with the contiguous padded layout of math.rs:365-378:
 * `count` cached rows [count][kv_heads*head_dim], the softmax row padded with
 * -inf to a multiple of 256 columns.  QK and PV products are rounded to f32
 * and summed in f64. */
static int attention_checked(const float *q, const float *keys, const float *values, uint64_t count, uint64_t heads,
                             uint64_t kv_heads, uint64_t head_dim, float scale, float *out) {
    if (count == 0 || heads == 0 || kv_heads == 0 || heads % kv_heads) return ORC_INVALID_LENGTH;
    const uint64_t width = kv_heads * head_dim, row_len = (count + 255) / 256 * 256;
    float *scores = (float *)malloc(row_len * sizeof(float));
    double *acc = (double *)calloc(heads * head_dim, sizeof(double));
    if (!scores || !acc) {
        free(scores);
        free(acc);
        return ORC_ALLOCATION_FAILED;
    }
    int rc = ORC_OK;
    for (uint64_t h = 0; h < heads && rc == ORC_OK; ++h) {
        for (uint64_t i = 0; i < row_len; ++i) scores[i] = -INFINITY;
        const uint64_t kvh = h / (heads / kv_heads);
        const float *qh = q + h * head_dim;
        for (uint64_t t = 0; t < count; ++t) {
            const float *k = keys + t * width + kvh * head_dim;
            double dot = 0.0;
            for (uint64_t d = 0; d < head_dim; ++d) dot += (double)(qh[d] * k[d]);
            const float score = (float)dot * scale;
            if (!isfinite(score)) {
                rc = NF_ATT_SCORE;
                break;
            }
            scores[t] = score;
        }
        if (rc == ORC_OK && oracle_softmax(scores, row_len) != ORC_OK) rc = NF_SOFTMAX;
        for (uint64_t t = 0; t < count && rc == ORC_OK; ++t) {
            const float p = scores[t];
            const float *v = values + t * width + kvh * head_dim;
            for (uint64_t d = 0; d < head_dim; ++d) acc[h * head_dim + d] += (double)(p * v[d]);
        }
    }
    if (rc == ORC_OK) {
        for (uint64_t i = 0; i < heads * head_dim; ++i) out[i] = (float)acc[i];
        if (!all_finite(out, heads * head_dim)) rc = NF_ATT_OUTPUT;
    }
    free(scores);
    free(acc);
    return rc;
}
int oracle_attention(const float *q, const float *keys, const float *values, uint64_t count, uint64_t heads,
                     uint64_t kv_heads, uint64_t head_dim, float scale, float *out) {
    const int rc = attention_checked(q, keys, values, count, heads, kv_heads, head_dim, scale, out);
    return rc > NF_BASE ? ORC_NON_FINITE_INPUT : rc;
}

/* Matrix::multiply (math.rs:144-169) for a quantized matrix: finite input,
 * llama_quant::matvec, finite output. */
static uint32_t layer_type(const oracle_llama_model *m, const oracle_llama_layer *L, int k) {
    return L->types[k] ? L->types[k] : m->weight_type;
}

/* A quantizer error of the matvec leaves its QuantError in *qe (the
 * reference wraps it in Error::Shape with its text). */
static int multiply(uint32_t t, const uint8_t *w, uint64_t rows, uint64_t cols, const float *x, float *y,
                    int threads, oracle_error *qe) {
    if (!all_finite(x, cols)) return NF_MATRIX_INPUT;
    uint64_t rb = 0;
    if (oracle_row_bytes(t, cols, &rb, qe) != ORC_OK) return qe->code;
    const int rc = oracle_matvec(t, w, rb * rows, rows, cols, x, cols, y, threads, qe);
    if (rc != ORC_OK) return rc;
    return all_finite(y, rows) ? ORC_OK : NF_MATRIX_OUTPUT;
}

/* LlamaModel::embedding (llama.rs:213-221): the token's row of the decoded
 * embedding matrix. */
int oracle_llama_embedding(const oracle_llama_model *m, uint32_t token, float *out) {
    if (token >= m->vocab) return ORC_INVALID_LENGTH;
    uint64_t rb = 0;
    oracle_error e;
    if (oracle_row_bytes(m->embedding_type, m->width, &rb, &e) != ORC_OK) return e.code;
    return oracle_dequantize_into(m->embedding_type, m->embedding + (uint64_t)token * rb, rb, out, m->width, &e);
}

/* Layers [first, first + count) of LlamaModel::step_inserting (llama.rs:
 * 250-305) at the end of a sequential cache (insertion = n_cached), each
 * project_layer (:307-338) then finish_layer (:340-379), over `hidden`
 * (width, in/out); the caches hold [n_layers][max_context][kv_width] f32 and
 * gain row n_cached of every layer run.  On failure *layer is the failing
 * layer and the return code is a step-internal NF_ code or a QuantError
 * (payload in *qe). */
static int run_layers(const oracle_llama_model *m, uint64_t first, uint64_t count, float *hidden, uint64_t position,
                      uint64_t n_cached, float *k_cache, float *v_cache, int threads, oracle_error *qe,
                      uint64_t *layer) {
    const uint64_t W = m->width, F = m->feed_forward, H = m->heads, KVH = m->kv_heads;
    const uint64_t hd = W / H, kvw = KVH * hd;
    const float scale = m->attention_scale != 0.0f ? m->attention_scale : 1.0f / sqrtf((float)hd);
    float *norm = (float *)malloc(W * sizeof(float)), *q = (float *)malloc(W * sizeof(float));
    float *k = (float *)malloc(kvw * sizeof(float)), *v = (float *)malloc(kvw * sizeof(float));
    float *att = (float *)malloc(W * sizeof(float)), *proj = (float *)malloc(W * sizeof(float));
    float *gate = (float *)malloc(F * sizeof(float)), *up = (float *)malloc(F * sizeof(float));
    int rc = (norm && q && k && v && att && proj && gate && up) ? ORC_OK : ORC_ALLOCATION_FAILED;
    uint64_t l = first;
    for (; l < first + count && rc == ORC_OK; ++l) {
        const oracle_llama_layer *L = &m->layers[l];
        float *kc = k_cache + l * m->max_context * kvw, *vc = v_cache + l * m->max_context * kvw;
        rc = rms_norm_checked(hidden, L->attention_norm, W, m->rms_epsilon, norm);
        if (rc == ORC_OK) rc = multiply(layer_type(m, L, 0), L->query, W, W, norm, q, threads, qe);
        if (rc == ORC_OK) rc = multiply(layer_type(m, L, 1), L->key, kvw, W, norm, k, threads, qe);
        if (rc == ORC_OK) rc = multiply(layer_type(m, L, 2), L->value, kvw, W, norm, v, threads, qe);
        if (rc != ORC_OK) break;
        oracle_rope(q, W, hd, position, m->rope_base);
        oracle_rope(k, kvw, hd, position, m->rope_base);
        memcpy(kc + n_cached * kvw, k, kvw * sizeof(float));
        memcpy(vc + n_cached * kvw, v, kvw * sizeof(float));
        rc = attention_checked(q, kc, vc, n_cached + 1, H, KVH, hd, scale, att);
        if (rc == ORC_OK) rc = multiply(layer_type(m, L, 3), L->attention_output, W, W, att, proj, threads, qe);
        if (rc != ORC_OK) break;
        for (uint64_t i = 0; i < W; ++i) hidden[i] += proj[i];
        rc = rms_norm_checked(hidden, L->feed_forward_norm, W, m->rms_epsilon, norm);
        if (rc == ORC_OK) rc = multiply(layer_type(m, L, 4), L->gate, F, W, norm, gate, threads, qe);
        if (rc == ORC_OK) rc = multiply(layer_type(m, L, 5), L->up, F, W, norm, up, threads, qe);
        if (rc != ORC_OK) break;
        oracle_silu(gate, F);
        for (uint64_t i = 0; i < F; ++i) gate[i] *= up[i];
        rc = multiply(layer_type(m, L, 6), L->down, W, F, gate, proj, threads, qe);
        if (rc != ORC_OK) break;
        for (uint64_t i = 0; i < W; ++i) hidden[i] += proj[i];
        if (!all_finite(hidden, W)) {
            rc = NF_LAYER_OUTPUT;
            break;
        }
    }
    *layer = l;
    free(norm);
    free(q);
    free(k);
    free(v);
    free(att);
    free(proj);
    free(gate);
    free(up);
    return rc;
}

/* finish_hidden (llama.rs:381-392): the final RMSNorm into `embedding`
 * (width, may be null), the output matrix into `logits` (vocab). */
static int run_finish(const oracle_llama_model *m, const float *hidden, float *embedding, float *logits, int threads,
                      oracle_error *qe) {
    const uint64_t W = m->width;
    float *norm = (float *)malloc(W * sizeof(float));
    if (!norm) return ORC_ALLOCATION_FAILED;
    int rc = rms_norm_checked(hidden, m->output_norm, W, m->rms_epsilon, norm);
    if (rc == ORC_OK) rc = multiply(m->output_type, m->output, m->vocab, W, norm, logits, threads, qe);
    if (rc == ORC_OK && embedding) memcpy(embedding, norm, W * sizeof(float));
    free(norm);
    return rc;
}

/* The first failure as the library reports it: a NonFinite check as
 * ORC_NON_FINITE {a = the check, b = the layer; n_layers for finish_hidden},
 * a quantizer's QuantError with its payload and b = the layer. */
static int report(int rc, const oracle_error *qe, uint64_t layer, oracle_error *err) {
    if (rc > NF_BASE) {
        if (err) *err = (oracle_error){ORC_NON_FINITE, 0, (uint64_t)(rc - NF_BASE), layer};
        return ORC_NON_FINITE;
    }
    if (rc != ORC_OK && err) *err = rc == qe->code ? (oracle_error){qe->code, qe->dtype, qe->a, layer}
                                                   : (oracle_error){rc, 0, 0, 0};
    return rc;
}

static int check_step(const oracle_llama_model *m, uint64_t n_cached) {
    const uint64_t W = m->width, H = m->heads, KVH = m->kv_heads;
    return (H == 0 || KVH == 0 || W % H || H % KVH || n_cached >= m->max_context) ? ORC_INVALID_LENGTH : ORC_OK;
}

/* LlamaModel::step_inserting (llama.rs:250-305) at the end of a sequential
 * cache: every layer, then finish_hidden.  `hidden` (width) is the input
 * embedding and receives the last layer's output; `logits` receives vocab
 * values.  The first failure stops the step (report()). */
int oracle_llama_step(const oracle_llama_model *m, float *hidden, uint64_t position, uint64_t n_cached,
                      float *k_cache, float *v_cache, float *logits, int threads, oracle_error *err) {
    if (err) memset(err, 0, sizeof(*err));
    int rc = check_step(m, n_cached);
    if (rc != ORC_OK) return report(rc, NULL, 0, err);
    oracle_error qe = {0, 0, 0, 0};
    uint64_t layer = 0;
    rc = run_layers(m, 0, m->n_layers, hidden, position, n_cached, k_cache, v_cache, threads, &qe, &layer);
    if (rc == ORC_OK) rc = run_finish(m, hidden, NULL, logits, threads, &qe);
    return report(rc, &qe, layer, err);
}

/* One layer of the step on its own (the checker feeds each layer the GPU's
 * own input): layer `l` over hidden (in/out) at `position`, appending KV row
 * n_cached of that layer only. */
int oracle_llama_run_layer(const oracle_llama_model *m, uint64_t l, float *hidden, uint64_t position, uint64_t n_cached,
                       float *k_cache, float *v_cache, int threads, oracle_error *err) {
    if (err) memset(err, 0, sizeof(*err));
    int rc = check_step(m, n_cached);
    if (rc == ORC_OK && l >= m->n_layers) rc = ORC_INVALID_LENGTH;
    if (rc != ORC_OK) return report(rc, NULL, 0, err);
    oracle_error qe = {0, 0, 0, 0};
    uint64_t layer = l;
    rc = run_layers(m, l, 1, hidden, position, n_cached, k_cache, v_cache, threads, &qe, &layer);
    return report(rc, &qe, layer, err);
}

/* finish_hidden alone: embedding (width, may be null) and logits (vocab)
 * from a last-layer output. */
int oracle_llama_finish(const oracle_llama_model *m, const float *hidden, float *embedding, float *logits,
                        int threads, oracle_error *err) {
    if (err) memset(err, 0, sizeof(*err));
    oracle_error qe = {0, 0, 0, 0};
    return report(run_finish(m, hidden, embedding, logits, threads, &qe), &qe, m->n_layers, err);
}
