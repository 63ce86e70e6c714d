/*
 * rlq_oracle.h - CPU restatement of rust-llama's scalar quantized-matvec path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * implementation: only the tests, the smoke check and the CPU-baseline leg of
 * the benchmark load it.  The product library never links or calls it.
 *
 * It restates, in plain C with the reference's arithmetic order, the Rust
 * crate `llama-quant` (crates/quant/src) for the dtypes on the path:
 *   Q8_0 (id 8) and Q4_K (12) / Q6_K (14) weights, Q8_0 and Q8_K (15)
 *   activations.  Each function cites the reference lines it follows.
 * Build with `make -C oracle` (gcc -O2 -ffp-contract=off -fno-fast-math), so
 * that no multiply-add is fused and every f32 operation rounds as Rust's does.
 *
 * Status codes follow the order of the reference's `QuantError` enum
 * (crates/quant/src/lib.rs:45-63); 18..20 are this build's additions.
 */
#ifndef RLQ_ORACLE_H
#define RLQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_OK = 0,
    ORC_INVALID_TYPE = 1,                 /* dtype = id */
    ORC_UNSUPPORTED_MATVEC = 2,           /* dtype */
    ORC_INVALID_VECTOR_LENGTH = 3,        /* a = expected, b = actual */
    ORC_INVALID_MATRIX_SHAPE = 4,         /* a = rows, b = cols */
    ORC_NON_MULTIPLE = 5,                 /* a = elements, b = block_size */
    ORC_SIZE_OVERFLOW = 6,
    ORC_INVALID_LENGTH = 7,               /* a = expected, b = actual */
    ORC_ALLOCATION_FAILED = 8,
    ORC_UNSUPPORTED_QUANTIZATION = 9,     /* dtype */
    ORC_UNSUPPORTED_WEIGHTED_QUANTIZATION = 10,
    ORC_IMPORTANCE_WEIGHTS_REQUIRED = 11,
    ORC_INVALID_IMPORTANCE_LENGTH = 12,
    ORC_INVALID_IMPORTANCE_WEIGHT = 13,
    ORC_UNSUPPORTED_INTEGER_CONVERSION = 14,
    ORC_INTEGER_OUT_OF_RANGE = 15,
    ORC_NON_FINITE_INPUT = 16,            /* a = index */
    ORC_UNREPRESENTABLE_SCALE = 17,       /* a = block */
    ORC_DEVICE_ERROR = 18,                /* not produced by the oracle */
    ORC_UNIMPLEMENTED = 19,               /* dtype exists upstream, not restated here */
    ORC_INVALID_ARGUMENT = 20,            /* null pointer */
    ORC_INVALID_CONFIG = 21,              /* model-runtime errors of the decode step */
    ORC_INVALID_TOKEN = 22,
    ORC_INVALID_STATE = 23,
    ORC_NON_FINITE = 31                   /* model-runtime Error::NonFinite: a = check, b = layer */
};

typedef struct oracle_error {
    int32_t code;
    uint32_t dtype;
    uint64_t a;
    uint64_t b;
} oracle_error;

/* lib.rs:323-337 and lib.rs:340-373 */
float oracle_f16_to_f32(uint16_t bits);
uint16_t oracle_f32_to_f16(float value);

/* lib.rs:210-285: 0 if id is not a known dtype */
int oracle_dtype_known(uint32_t id);
uint64_t oracle_block_size(uint32_t dtype);
uint64_t oracle_type_size(uint32_t dtype);
int oracle_row_bytes(uint32_t dtype, uint64_t elements, uint64_t *out, oracle_error *err);

/* matvec.rs:7-18 */
int oracle_matvec_activation_dtype(uint32_t wtype, uint32_t *out, oracle_error *err);

/* encode.rs:37-100 (Q8_0, Q8_K) and encode_k.rs:11-33 (Q4_K, Q6_K).
 * Validation precedes any write to `out`. */
int oracle_quantize_into(uint32_t dtype, const float *x, uint64_t n, uint8_t *out,
                         uint64_t out_len, oracle_error *err);

/* lib.rs:299-308 with decode.rs:17-23, 42-43, 44-49, 216-258 */
int oracle_dequantize_into(uint32_t dtype, const uint8_t *bytes, uint64_t len, float *out,
                           uint64_t n, oracle_error *err);

/* matvec.rs:90-103 */
int oracle_dot_packed(uint32_t wtype, const uint8_t *w, uint64_t w_len, const uint8_t *act,
                      uint64_t act_len, uint64_t elements, float *out, oracle_error *err);

/* matvec.rs:24-87.  `threads` > 1 splits rows over pthreads; each row's dot is
 * the same scalar loop, so the output is identical for every thread count.
 * `y` (rows floats) is written only on success. */
int oracle_matvec(uint32_t wtype, const uint8_t *w, uint64_t w_len, uint64_t rows,
                  uint64_t cols, const float *x, uint64_t x_len, float *y, int threads,
                  oracle_error *err);

/* crates/tensor/src/cpu_extra.rs:756-873 (MUL_MAT, 2-D case): each of the
 * `batch` input rows x[b*cols ..] is quantized separately (:820), then
 * y[b*rows + r] = dot_packed(row r, activation b) (:860). */
int oracle_matmul(uint32_t wtype, const uint8_t *w, uint64_t w_len, uint64_t rows,
                  uint64_t cols, const float *x, uint64_t batch, float *y, int threads,
                  oracle_error *err);

/* Exact per-block integer sums of one packed row against one packed
 * activation row (no validation; nblocks blocks of the weight type):
 *   Q4_K: isum = sum_j sc(j)*q(j)*q8(j) (the 8 lanes of matvec_extra.rs:256-266
 *         added together), imin = sum_s (bsum[2s]+bsum[2s+1])*min_s (:258)
 *   Q6_K: isum = sum_j sc(j/16)*(q6(j)-32)*q8(j) (:272-281), imin = 0
 *   Q8_0: isum = sum_j xq(j)*yq(j) per 32-block (matvec.rs:124-127), imin = 0 */
void oracle_block_sums(uint32_t wtype, const uint8_t *w_row, const uint8_t *act_row,
                       uint64_t nblocks, int32_t *isum, int32_t *imin);

/* Tolerance helper (not a restatement): sum over the row's blocks of the
 * absolute values of every integer product times its f32 scale, in f64.  It
 * bounds the f32 rounding of any summation order of the same terms:
 * |computed - exact| <= n * 2^-24 * abs_terms for n additions per term. */
double oracle_abs_terms(uint32_t wtype, const uint8_t *w_row, const uint8_t *act_row,
                        uint64_t nblocks);

/* Greedy sampler, crates/llama-behavior/src/sampling.rs:607-613: index of the
 * first strict maximum (n >= 1). */
uint64_t oracle_argmax(const float *x, uint64_t n);

/* ---- dense Llama decode step (rlq_oracle_llama.c) ------------------------ */

/* crates/quant/src/cpu_math.rs:94-123, one lane of the SSE2 exponential. */
float oracle_sse2_exp(float x);
/* cpu_math.rs:28-53 (SSE2 policy), in place. */
void oracle_silu(float *v, uint64_t n);
/* crates/model-runtime/src/math.rs:293-318 with cpu_math.rs:60-91, in place. */
int oracle_softmax(float *v, uint64_t n);
/* math.rs:214-228 */
int oracle_rms_norm(const float *x, const float *w, uint64_t n, float eps, float *out);
/* math.rs:322-334, in place over len values of heads of head_dim. */
void oracle_rope(float *v, uint64_t len, uint64_t head_dim, uint64_t position, float base);
/* The sin/cos pairs oracle_rope uses at `position`: table[2i] = sin,
 * table[2i+1] = cos, i < head_dim/2. */
void oracle_rope_table(uint64_t head_dim, uint64_t position, float base, float *table);
/* math.rs:427-497, contiguous padded layout (math.rs:365-378). */
int oracle_attention(const float *q, const float *keys, const float *values, uint64_t count, uint64_t heads,
                     uint64_t kv_heads, uint64_t head_dim, float scale, float *out);

/* LlamaLayer (crates/model-runtime/src/llama.rs:67-85) without biases: GGUF
 * bytes of the quantized matrices (rows x cols, rows contiguous) and f32 norm
 * weights. */
typedef struct oracle_llama_layer {
    const float *attention_norm;
    const uint8_t *query, *key, *value, *attention_output;
    const float *feed_forward_norm;
    const uint8_t *gate, *up, *down;
    /* types of query, key, value, attention_output, gate, up, down; 0 = the
     * model's weight_type (a GGUF file types every tensor on its own) */
    uint32_t types[7];
} oracle_llama_layer;

/* LlamaConfig (llama.rs:6-17) and LlamaWeights.  attention_scale 0 means
 * 1/sqrt(head_dim). */
typedef struct oracle_llama_model {
    uint64_t vocab, width, feed_forward, heads, kv_heads, max_context, n_layers;
    float rms_epsilon, rope_base, attention_scale;
    uint32_t weight_type, output_type, embedding_type;
    const uint8_t *embedding; /* vocab x width */
    const float *output_norm;
    const uint8_t *output; /* vocab x width */
    const oracle_llama_layer *layers;
} oracle_llama_model;

/* LlamaModel::embedding (llama.rs:213-221). */
int oracle_llama_embedding(const oracle_llama_model *m, uint32_t token, float *out);
/* LlamaModel::step (llama.rs:222-392) at the end of a sequential cache of
 * n_cached rows: hidden (width) in/out, caches [n_layers][max_context][kv_width]
 * gain row n_cached, logits (vocab) out.  `threads` splits matvec rows. */
int oracle_llama_step(const oracle_llama_model *m, float *hidden, uint64_t position, uint64_t n_cached,
                      float *k_cache, float *v_cache, float *logits, int threads, oracle_error *err);
/* One layer of the step (layer l over hidden, KV row n_cached of layer l),
 * and finish_hidden alone (embedding may be null). */
int oracle_llama_run_layer(const oracle_llama_model *m, uint64_t l, float *hidden, uint64_t position, uint64_t n_cached,
                           float *k_cache, float *v_cache, int threads, oracle_error *err);
int oracle_llama_finish(const oracle_llama_model *m, const float *hidden, float *embedding, float *logits,
                        int threads, oracle_error *err);

#ifdef __cplusplus
}
#endif

#endif
