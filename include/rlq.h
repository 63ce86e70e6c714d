/*
 * rlq.h - C ABI of the gfx950 (MI355X) quantized matrix-product library.
 *
 * Drop-in for rust-llama's `llama-quant` scalar matvec path (crate
 * crates/quant; public surface crates/quant/src/lib.rs:36-41) and its two
 * callers, model-runtime `Matrix::multiply` (crates/model-runtime/src/math.rs:144-169)
 * and the GGML MUL_MAT op (crates/tensor/src/cpu_extra.rs:756-873).  Weight
 * formats Q8_0 (id 8) and the K formats Q2_K (10), Q3_K (11), Q4_K (12),
 * Q5_K (13), Q6_K (14); activations are quantized to Q8_0 / Q8_K (15) on the
 * GPU, exactly as the reference's quantizers.
 *
 * Conventions
 *   - Plain pointers and sizes.  Sizes are u64 (the reference's usize).
 *   - Every function returns an rlq_status and, when `err` is non-null, fills
 *     it.  Codes 1..17 are the reference's QuantError variants in declaration
 *     order (crates/quant/src/lib.rs:45-63) with the same payloads; 18..20 are
 *     this library's own; 21..23 stand for the model-runtime errors of the
 *     decode step (crates/model-runtime/src/lib.rs Error: InvalidConfig,
 *     InvalidToken, InvalidState); 24..26 for the tensor crate's errors of
 *     MUL_MAT / MUL_MAT_ID (Shape, Bounds, Unsupported); 27..30 for the GGUF
 *     crate's (Io, Invalid, Limit, Unsupported).
 *   - Validate before mutate: on any error, no output buffer is written
 *     (crates/quant/src/matvec.rs:31-56, encode.rs:37-100).
 *   - Host functions (`rlq_matvec`, `rlq_quantize_into`, ...) take host
 *     pointers, run on the GPU of the process-wide default context and return
 *     when the result is in the caller's buffer (the reference is synchronous).
 *   - Device functions take device pointers and enqueue on `stream` (a
 *     hipStream_t passed as void*; NULL = the HIP null stream, as in HIP).  Shape
 *     and length errors are returned at once; data errors found on the GPU
 *     (non-finite input, unrepresentable scale) suppress the outputs of the
 *     failing call and are reported by the next rlq_sync().
 *   - A context or weights handle must not be used by two threads at once.
 *   - Weights and activations are little-endian GGUF bytes, rows of `cols`
 *     elements, rows contiguous (ne[0] innermost; math.rs:15-16).
 */
#ifndef RLQ_H
#define RLQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML numeric type ids on the path (crates/quant/src/lib.rs:132-169).  Any
 * id of that enum is accepted where a dtype is taken; ids outside the path
 * return RLQ_UNIMPLEMENTED after the reference's own checks. */
enum rlq_dtype {
    RLQ_Q8_0 = 8, RLQ_Q2_K = 10, RLQ_Q3_K = 11, RLQ_Q4_K = 12, RLQ_Q5_K = 13, RLQ_Q6_K = 14, RLQ_Q8_K = 15
};

typedef enum rlq_status {
    RLQ_OK = 0,
    RLQ_INVALID_TYPE = 1,               /* dtype = id */
    RLQ_UNSUPPORTED_MATVEC = 2,         /* dtype */
    RLQ_INVALID_VECTOR_LENGTH = 3,      /* a = expected, b = actual */
    RLQ_INVALID_MATRIX_SHAPE = 4,       /* a = rows, b = cols */
    RLQ_NON_MULTIPLE = 5,               /* a = elements, b = block_size */
    RLQ_SIZE_OVERFLOW = 6,
    RLQ_INVALID_LENGTH = 7,             /* a = expected, b = actual */
    RLQ_ALLOCATION_FAILED = 8,
    RLQ_UNSUPPORTED_QUANTIZATION = 9,   /* dtype */
    RLQ_UNSUPPORTED_WEIGHTED_QUANTIZATION = 10,
    RLQ_IMPORTANCE_WEIGHTS_REQUIRED = 11,
    RLQ_INVALID_IMPORTANCE_LENGTH = 12,
    RLQ_INVALID_IMPORTANCE_WEIGHT = 13,
    RLQ_UNSUPPORTED_INTEGER_CONVERSION = 14,
    RLQ_INTEGER_OUT_OF_RANGE = 15,
    RLQ_NON_FINITE_INPUT = 16,          /* a = index (within the column), b = column */
    RLQ_UNREPRESENTABLE_SCALE = 17,     /* a = block (within the column), b = column */
    RLQ_DEVICE_ERROR = 18,              /* a = hipError_t */
    RLQ_UNIMPLEMENTED = 19,             /* dtype: known to the reference, not on this path */
    RLQ_INVALID_ARGUMENT = 20,          /* null pointer or handle */
    RLQ_INVALID_CONFIG = 21,            /* a = check (see rlq_llama_create) */
    RLQ_INVALID_TOKEN = 22,             /* a = token, b = vocabulary */
    RLQ_INVALID_STATE = 23,             /* a = KV rows held, b = max_context (cache full) */
    /* TensorError variants of the GGML ops (crates/tensor/src/lib.rs:35-50) */
    RLQ_TENSOR_SHAPE = 24,              /* Shape: incompatible MUL_MAT / MUL_MAT_ID dimensions */
    RLQ_TENSOR_BOUNDS = 25,             /* Bounds: an expert id outside [-1, experts); a = its index */
    RLQ_TENSOR_UNSUPPORTED = 26,        /* Unsupported: a right-hand side neither F32 nor the
                                           activation type; dtype = that type */
    /* llama_gguf::Error variants (crates/gguf/src/lib.rs:26-32); a = the header
       byte position of the failed check (IO: a = errno, b = the position) */
    RLQ_GGUF_IO = 27,
    RLQ_GGUF_INVALID = 28,
    RLQ_GGUF_LIMIT = 29,
    RLQ_GGUF_UNSUPPORTED = 30,
    /* model-runtime Error::NonFinite (crates/model-runtime/src/lib.rs:51):
       a = the check (rlq_nonfinite_check), b = the Llama layer (n_layers for
       the final norm and the output matrix; 0 for rlq_multiply) */
    RLQ_NON_FINITE = 31,
    RLQ_SCRATCH_LIMIT = 32              /* rlq_matmul_noalloc: a = bytes needed, b = the scratch size */
} rlq_status;

/* The reference's NonFinite checks, by the name it reports. */
enum rlq_nonfinite_check {
    RLQ_CHECK_RMS_SCALE = 1,         /* "RMS normalization scale" (math.rs:218-220) */
    RLQ_CHECK_RMS_OUTPUT = 2,        /* "RMS normalization output" (math.rs:227) */
    RLQ_CHECK_MATRIX_INPUT = 3,      /* "matrix input" (math.rs:152) */
    RLQ_CHECK_MATRIX_OUTPUT = 4,     /* "matrix output" (math.rs:167) */
    RLQ_CHECK_ATTENTION_SCORE = 5,   /* "attention score" (math.rs:476-478) */
    RLQ_CHECK_ATTENTION_OUTPUT = 6,  /* "attention output" (math.rs:494) */
    RLQ_CHECK_LAYER_OUTPUT = 7       /* "Llama layer output" (llama.rs:378) */
};

typedef struct rlq_error {
    int32_t code;
    uint32_t dtype;
    uint64_t a;
    uint64_t b;
} rlq_error;

typedef struct rlq_context rlq_context;
typedef struct rlq_weights rlq_weights;

/* ---- metadata (no GPU work) -------------------------------------------- */

/* Static text for a status code. */
const char *rlq_status_string(int32_t code);

/* DType::row_bytes (crates/quant/src/lib.rs:274-285). */
int32_t rlq_row_bytes(uint32_t dtype, uint64_t elements, uint64_t *out, rlq_error *err);

/* matvec_activation_dtype (crates/quant/src/matvec.rs:7-18). */
int32_t rlq_matvec_activation_dtype(uint32_t weights_type, uint32_t *out, rlq_error *err);

/* ---- host drop-ins (synchronous, default context) ------------------------ */

/* quantize_into (crates/quant/src/encode.rs:37-100): Q8_0 / Q8_K activation
 * quantizers and the Q8_0 and Q2_K..Q6_K weight encoders
 * (crates/quant/src/encode_k.rs:11-561), run on the GPU. */
int32_t rlq_quantize_into(uint32_t dtype, const float *values, uint64_t n, uint8_t *out, uint64_t out_len,
                          rlq_error *err);

/* dequantize_into (crates/quant/src/lib.rs:299-308; decode.rs): Q8_0, Q8_K
 * and Q2_K..Q6_K. */
int32_t rlq_dequantize_into(uint32_t dtype, const uint8_t *bytes, uint64_t len, float *out, uint64_t n,
                            rlq_error *err);

/* dot_packed (crates/quant/src/matvec.rs:90-103). */
int32_t rlq_dot_packed(uint32_t weights_type, const uint8_t *weights, uint64_t weights_len,
                       const uint8_t *activation, uint64_t activation_len, uint64_t elements, float *out,
                       rlq_error *err);

/* matvec (crates/quant/src/matvec.rs:24-87): y[rows] = W[rows x cols] . x[cols].
 * Uploads the weights on every call; use rlq_weights_create + rlq_matmul to
 * keep them resident. */
int32_t rlq_matvec(uint32_t weights_type, const uint8_t *weights, uint64_t weights_len, uint64_t rows,
                   uint64_t cols, const float *input, uint64_t input_len, float *output, rlq_error *err);

/* ---- device API -------------------------------------------------------- */

/* One context per device; it owns a stream for the host drop-ins, scratch
 * memory and the device error word.  device = -1 takes the current HIP
 * device.  Device calls on one context share its scratch: queue them on one
 * stream (or order them) so that they do not overlap. */
int32_t rlq_context_create(int32_t device, rlq_context **out, rlq_error *err);
void rlq_context_destroy(rlq_context *ctx);
/* The context's own (non-blocking) hipStream_t, which the host drop-ins use. */
void *rlq_context_stream(rlq_context *ctx);

/* Matrix::from_quantized (crates/model-runtime/src/math.rs:35-70): checks the
 * dtype capability, shape and byte length, then keeps a device copy of the
 * weights in the kernels' tiled layout (16-row tiles; each (tile, block) is
 * one contiguous chunk in the order the kernels' lanes load it).  `bytes_on_device` != 0 when `bytes` is a device
 * pointer; the device is then synchronized first, so work that produced the
 * bytes on any stream is complete.  Returns after the copy is complete. */
int32_t rlq_weights_create(rlq_context *ctx, uint32_t dtype, const void *bytes, uint64_t len, uint64_t rows,
                           uint64_t cols, int32_t bytes_on_device, rlq_weights **out, rlq_error *err);
/* A stack of n2 x n3 matrices of rows x cols, a GGML weight tensor
 * [cols, rows, n2, n3] (MUL_MAT broadcast sources, MUL_MAT_ID experts with
 * n3 = 1): `bytes` holds the matrices' GGUF rows contiguously, matrix
 * (i2, i3) at offset (i3 * n2 + i2) * rows * row_bytes (the reference's
 * `contiguous()` layout, crates/tensor/src/cpu_extra.rs:788-790).  Each
 * matrix is kept in the tiled layout.  rlq_weights_create is the n2 = n3 = 1
 * case; rlq_matmul uses matrix (0, 0). */
int32_t rlq_weights_create_stacked(rlq_context *ctx, uint32_t dtype, const void *bytes, uint64_t len,
                                   uint64_t rows, uint64_t cols, uint64_t n2, uint64_t n3, int32_t bytes_on_device,
                                   rlq_weights **out, rlq_error *err);
/* Frees the device copy; it does not use the creating context, so weights may
 * be destroyed after their context. */
void rlq_weights_destroy(rlq_weights *w);
/* rows, cols, dtype of a weights handle (any output pointer may be null). */
void rlq_weights_shape(const rlq_weights *w, uint64_t *rows, uint64_t *cols, uint32_t *dtype);
/* n2, n3 of a weights handle (1, 1 for rlq_weights_create). */
void rlq_weights_stack(const rlq_weights *w, uint64_t *n2, uint64_t *n3);

/* MUL_MAT (crates/tensor/src/cpu_extra.rs:756-873) with an F32 right-hand
 * side, and Matrix::multiply for batch = 1: each of the `batch` input rows
 * x[b*cols ..] is quantized to the weights' activation type on the GPU, then
 * y[b*rows + r] = dot_packed(weights row r, activation b).  x and y are
 * device pointers (x 16-byte aligned).  Up to 8 columns share one pass over
 * the weights.  A call takes at most 8388606 columns (the error keys carry
 * the column): more return RLQ_UNIMPLEMENTED (a = batch, b = the limit), as
 * do rlq_matmul_argmax, rlq_matmul_noalloc and rlq_quantize_device. */
int32_t rlq_matmul(rlq_context *ctx, const rlq_weights *w, const float *x, uint64_t batch, float *y,
                   void *stream, rlq_error *err);

/* Matrix::multiply (crates/model-runtime/src/math.rs:144-169) of one input
 * vector x (device, cols floats, 16-byte aligned) into y (device, rows
 * floats): finite(input), llama_quant::matvec, finite(output).  Data errors at
 * rlq_sync, in the reference's order: RLQ_NON_FINITE (a =
 * RLQ_CHECK_MATRIX_INPUT) for a non-finite input; the quantizer's
 * RLQ_UNREPRESENTABLE_SCALE (a = block; the reference wraps this QuantError
 * in Error::Shape with its text); RLQ_NON_FINITE (a =
 * RLQ_CHECK_MATRIX_OUTPUT) for a non-finite output.  With an input error no
 * output is written; with an output error y holds the outputs. */
int32_t rlq_multiply(rlq_context *ctx, const rlq_weights *w, const float *x, float *y, void *stream, rlq_error *err);

/* rlq_matmul followed by the greedy sampler's choice per column
 * (crates/llama-behavior/src/sampling.rs:607-613: the first strict maximum),
 * fused into the matvec epilogue: argmax[b] = index of the largest y[b*rows+r]. */
int32_t rlq_matmul_argmax(rlq_context *ctx, const rlq_weights *w, const float *x, uint64_t batch, float *y,
                          uint32_t *argmax, void *stream, rlq_error *err);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  rlq_matmul (argmax null) or rlq_matmul_argmax (argmax
 * non-null) on the same kernels, with the same results, that allocates and
 * frees nothing: the argmax keys and the prefill GEMM's activation image
 * (batches above 8 of Q4_K weights) live in a static 32 MiB device array
 * that each GPU holds until the process ends.  A call whose workspace
 * exceeds it returns RLQ_SCRATCH_LIMIT (a = bytes needed, b = 33554432); for
 * 4096 columns that is a batch of about 3,700.  Every call on one GPU, from
 * any context, shares that GPU's array: calls that overlap on one GPU (other
 * streams, other threads) race and must be ordered by the caller. */
int32_t rlq_matmul_noalloc(rlq_context *ctx, const rlq_weights *w, const float *x, uint64_t batch, float *y,
                           uint32_t *argmax, void *stream, rlq_error *err);

/* GGML MUL_MAT with batch broadcast (crates/tensor/src/cpu_extra.rs:756-873)
 * over stacked weights W [cols, rows, w.n2, w.n3] and a right-hand side
 * X [cols, ncols, n2, n3] (n2 % w.n2 == 0, n3 % w.n3 == 0):
 *   y[((i3 * n2 + i2) * ncols + c) * rows + r] =
 *       dot_packed(row r of W(i2 / (n2 / w.n2), i3 / (n3 / w.n3)), column c of X(i2, i3)).
 * x_dtype is 0 (F32: every column is quantized to the weights' activation
 * type, once) or that activation type itself (Q8_0 / Q8_K bytes, used as
 * given).  x (16-byte aligned) and y are device pointers; rows of X are
 * contiguous, column after column.  Errors, in the reference's order:
 * RLQ_TENSOR_SHAPE (a = n2, b = n3), RLQ_TENSOR_UNSUPPORTED (x_dtype), then
 * the quantizer's data errors at rlq_sync (b = the column's index
 * (i3 * n2 + i2) * ncols + c).  A call with a data error writes no output. */
int32_t rlq_mul_mat(rlq_context *ctx, const rlq_weights *w, uint32_t x_dtype, const void *x, uint64_t ncols,
                    uint64_t n2, uint64_t n3, float *y, void *stream, rlq_error *err);

/* GGML MUL_MAT_ID (crates/tensor/src/cpu_index.rs:169-236): experts W[e],
 * e < w.n2 (w.n3 = 1), right-hand side X [cols, ncols, tokens] (x_dtype as
 * for rlq_mul_mat), expert ids [slots, tokens] (i32, device, slots %
 * ncols == 0):
 *   y[(t * slots + s) * rows + r] = dot_packed(row r of W[ids[t * slots + s]],
 *                                              column s % ncols of X(t)),
 * and 0 where the id is -1.  Every column of X is quantized once before the
 * expert products (one token with one F32 column: inside the one product
 * launch, by every workgroup).  Errors: RLQ_TENSOR_SHAPE, RLQ_TENSOR_UNSUPPORTED at
 * once; at rlq_sync RLQ_TENSOR_BOUNDS (an id < -1 or >= w.n2; a = its index
 * t * slots + s) before any quantizer data error.  A call with an error
 * writes no output. */
int32_t rlq_mul_mat_id(rlq_context *ctx, const rlq_weights *w, uint32_t x_dtype, const void *x, uint64_t ncols,
                       uint64_t tokens, const int32_t *ids, uint64_t slots, float *y, void *stream, rlq_error *err);

/* Device quantize_into (crates/quant/src/encode.rs:37-100): the activation
 * quantizers (Q8_0, Q8_K) and the weight encoders (Q8_0, Q2_K..Q6_K), GGUF
 * bytes of `batch` rows of `cols` values each.  x and out are device
 * pointers, x 16-byte aligned (RLQ_INVALID_ARGUMENT otherwise).  For the K
 * encoders a NonFiniteInput index counts over all
 * batch*cols values and UnrepresentableScale over all blocks (b = 0). */
int32_t rlq_quantize_device(rlq_context *ctx, uint32_t dtype, const float *x, uint64_t cols, uint64_t batch,
                            uint8_t *out, void *stream, rlq_error *err);

/* Wait for `stream` (NULL = the null stream), then report and clear the first
 * data error the GPU recorded since the previous rlq_sync. */
int32_t rlq_sync(rlq_context *ctx, void *stream, rlq_error *err);

/* Exact integer part of every (row, block) dot of the weights against
 * activation column 0 of x (device f32, `batch` columns of cols values, 1 <=
 * batch <= 8), computed inside the kernel rlq_matmul runs for that batch size
 * (the columns are quantized on the GPU as rlq_matmul does):
 * isum[r*nb + k] and imin[r*nb + k] for block k are the integers of
 * crates/quant/src/matvec_extra.rs:174-283 (the eight lanes added; imin is
 * the mins sum of Q2_K, Q4_K and Q5_K, 0 otherwise) and matvec.rs:124-127.
 * isum and imin are device pointers of rows*nb i32. */
int32_t rlq_block_sums(rlq_context *ctx, const rlq_weights *w, const float *x, uint64_t batch, int32_t *isum,
                       int32_t *imin, void *stream, rlq_error *err);

/* rlq_block_sums that also hands out the launch's outputs and reaches the
 * decode step's fused gate/up kernel (test surface; no reference
 * counterpart).  y (device, may be null): the outputs of the same launch,
 * batch*rows floats as rlq_matmul writes them.  flags RLQ_SUMS_SILU_PAIR:
 * the kernel rlq_llama_step runs for a Q4_K / Q5_K gate/up product
 * (batch 1; rows a multiple of 32 whose 16-row tiles alternate gate and up:
 * tile 2i holds gate rows 16i.., tile 2i+1 up rows 16i..), with the integers
 * of every row of w and y = silu(gate) * up, rows/2 floats
 * (crates/model-runtime/src/llama.rs:367-371). */
#define RLQ_SUMS_SILU_PAIR 1u
int32_t rlq_block_sums_ex(rlq_context *ctx, const rlq_weights *w, const float *x, uint64_t batch, uint32_t flags,
                          int32_t *isum, int32_t *imin, float *y, void *stream, rlq_error *err);

/* ---- dense Llama decode step ------------------------------------------------
 * LlamaModel of crates/model-runtime/src/llama.rs with quantized matrices,
 * resident on one GPU with its f32 KV cache.  Every matrix product runs the
 * decode matvec kernels with the activation quantized to Q8_K (Q8_0 for Q8_0
 * weights); the attention and the RMSNorm / RoPE / SiLU / residual steps run
 * on the GPU in the reference's arithmetic order. */
typedef struct rlq_llama rlq_llama;

/* LlamaConfig (llama.rs:6-17) and the tensor types.  weight_type is that of
 * the seven layer matrices, output_type that of the output matrix (both Q4_K,
 * Q6_K or Q8_0), embedding_type that of the token embedding (Q8_0, Q4_K or
 * Q6_K).  attention_scale 0 means 1/sqrt(head_dim). */
typedef struct rlq_llama_config {
    uint64_t vocabulary, width, feed_forward, heads, kv_heads, max_context, n_layers;
    float rms_epsilon, rope_base, attention_scale;
    uint32_t weight_type, output_type, embedding_type;
} rlq_llama_config;

/* LlamaLayer (llama.rs:67-85) without biases: GGUF bytes of the matrices
 * (rows x cols, rows contiguous: query width x width, key and value
 * kv_width x width, attention_output width x width, gate and up
 * feed_forward x width, down width x feed_forward) and f32 norm weights. */
typedef struct rlq_llama_layer {
    const float *attention_norm;
    const void *query, *key, *value, *attention_output;
    const float *feed_forward_norm;
    const void *gate, *up, *down;
    /* types of query, key, value, attention_output, gate, up, down (a GGUF
     * file types every tensor on its own: Q4_K_M keeps some attn_v and
     * ffn_down in Q6_K); 0 = rlq_llama_config.weight_type */
    uint32_t types[7];
} rlq_llama_layer;

/* LlamaWeights: embedding (vocabulary x width), output_norm, output
 * (vocabulary x width) and n_layers layers.  on_device != 0 when every tensor
 * pointer is a device pointer (`layers` itself is a host array). */
typedef struct rlq_llama_tensors {
    const void *embedding;
    const float *output_norm;
    const void *output;
    const rlq_llama_layer *layers;
    int32_t on_device;
} rlq_llama_tensors;

/* LlamaModel::new: LlamaConfig::validate (llama.rs:19-56; RLQ_INVALID_CONFIG
 * with a = 1 zero or oversized dimension, 2 epsilon, 3 heads/width/kv_heads
 * grouping, 4 odd head_dim, 5 RoPE base, 6 attention scale, 7 KV size
 * overflow) and this library's limits (RLQ_UNIMPLEMENTED: a weight type off
 * the path, width / feed_forward not multiples of 256, kv_width not a
 * multiple of 16, head_dim not a multiple of 16 or above 256, or a score workgroup's
 * G query heads' rows beyond 159 KB of LDS: only for hundreds of query heads per KV
 * head; the context length is not limited by LDS), then uploads and tiles the weights.
 * The tensors may be freed when this returns. */
int32_t rlq_llama_create(rlq_context *ctx, const rlq_llama_config *cfg, const rlq_llama_tensors *tensors,
                         rlq_llama **out, rlq_error *err);
void rlq_llama_destroy(rlq_llama *model);
/* Drop the KV rows at and above `rows` (0 starts a new sequence). */
/* The inference crate's llama loader (crates/inference/src/loader.rs:242-410)
 * over a GGUF file: hparams from the llama.* metadata (exact UINT32 / finite
 * FLOAT32 values), the vocabulary size from tokenizer.ggml.tokens, max_context
 * = min(llama.context_length, context_length), every tensor checked against
 * its GGML shape and typed on its own (per-matrix types), output.weight
 * optional (absent: the token embedding projects).  Failures: the GGUF
 * reader's codes; RLQ_GGUF_INVALID / RLQ_GGUF_UNSUPPORTED (the loader's
 * Error::Invalid / Unsupported) with a = the check: 1 context_length 0,
 * 2 architecture, 3 general.type, 4 nextn layers, 5 Hadamard transforms,
 * 6 tokenizer.ggml.tokens, 7-13 embedding_length, head_count, width % heads,
 * head_count_kv, block_count (1..512), feed_forward_length, context_length,
 * 14 rope.dimension_count, 15 key/value_length, 16 sliding window / experts,
 * 17 causal, 18-20 RoPE scaling, 21 qk_norm, 22-24 rms epsilon, freq_base,
 * attention.scale, 30-32 token_embd / output_norm / output, 40-48 the layer
 * tensors (q, k, v, output, gate, up, down, attn_norm, ffn_norm),
 * 50 rope_freqs, 51 a tensor the model does not use (b = its index);
 * RLQ_UNIMPLEMENTED for a matrix type off the path, a non-F32 norm (dtype =
 * the type, a = the check) or biases (a = 49); then rlq_llama_create's own
 * checks. */
int32_t rlq_llama_create_from_gguf(rlq_context *ctx, const char *path, uint64_t context_length, rlq_llama **out,
                                   rlq_error *err);

/* The configuration a model was created with (a GGUF-loaded one: as the
 * loader derived it; weight_type = the type of layer 0's query). */
void rlq_llama_config_of(const rlq_llama *model, rlq_llama_config *out);

int32_t rlq_llama_truncate(rlq_llama *model, uint64_t rows, rlq_error *err);
/* KV rows held: the insertion index of the next step. */
uint64_t rlq_llama_cached(const rlq_llama *model);
/* LlamaModel::embedding (llama.rs:213-221): the token's decoded embedding row
 * into hidden (device, width floats). */
int32_t rlq_llama_embedding(rlq_llama *model, uint32_t token, float *hidden, void *stream, rlq_error *err);
/* LlamaModel::step (llama.rs:222-248): appends KV row rlq_llama_cached() of
 * every layer (RoPE at `position`), runs the layers over hidden (device,
 * width floats, in/out: it receives the last layer's output) and
 * finish_hidden (:381-392): embedding (width) = RMSNorm(hidden, output_norm),
 * logits (vocabulary) = output . embedding, argmax (1 u32) = the greedy
 * choice over the logits.  embedding, logits and argmax are device pointers
 * and may each be null.  Data errors are reported by rlq_sync as the
 * reference's sequential step would report its first: RLQ_NON_FINITE with
 * the check (a) and the layer (b; n_layers for the final norm and output),
 * or RLQ_UNREPRESENTABLE_SCALE (a = block, b = layer) from an activation
 * quantizer; the step's outputs are then unspecified. */
int32_t rlq_llama_step(rlq_llama *model, float *hidden, uint64_t position, float *embedding, float *logits,
                       uint32_t *argmax, void *stream, rlq_error *err);
/* Copies (on `stream`, device to device) the last layer's intermediates of
 * the latest step: qkv = [query (width) | key (kv_width, before RoPE) | value
 * (kv_width)], attention (width, the attention output), ffn_input (width, the
 * residual stream after attention: hidden + attention_output . attention,
 * the FFN RMSNorm's input), ffn = silu(gate) * up (feed_forward, the down
 * projection's input).  Any output may be null. */
int32_t rlq_llama_intermediates(const rlq_llama *model, float *qkv, float *attention, float *ffn_input, float *ffn,
                                void *stream, rlq_error *err);

/* Test surface (no reference counterpart): while `parts` (device, n_layers
 * x (4 width + 2 kv_width + feed_forward) floats) is non-null, every
 * rlq_llama_step also copies each layer's intermediates there, layer l at
 * l * (4 width + 2 kv_width + feed_forward): [query | key (before RoPE) |
 * value] (width + 2 kv_width), the attention output (width), the residual
 * stream after attention (width), silu(gate) * up (feed_forward) and the
 * layer output (width), so a checker can feed every part of every layer its
 * own input.  NULL stops the copies. */
int32_t rlq_llama_trace(rlq_llama *model, float *parts, rlq_error *err);

/* ---- GGUF files (crates/gguf) ---------------------------------------------------
 * Host-only: no device is used.  The reader follows RawGguf (crates/gguf/src/
 * raw.rs:85-300) with Limits::default(): GGUF v2/v3 of either byte order,
 * metadata in file order, tensor descriptors whose payloads follow each other
 * padded to the alignment, tensor payloads read on demand.  Keys, strings and
 * tensor names are byte strings (lengths given); lookups compare their
 * C-string prefixes, first match in file order (the native getters). */
typedef struct rlq_gguf rlq_gguf;

/* RawGguf::open (raw.rs:66-80): header, then every tensor's payload bounds
 * checked against the file length. */
int32_t rlq_gguf_open(const char *path, rlq_gguf **out, rlq_error *err);
/* RawGguf::read_header (raw.rs:80-84) over a memory image (copied): header
 * only, payload bounds unchecked. */
int32_t rlq_gguf_read_header_memory(const uint8_t *bytes, uint64_t len, rlq_gguf **out, rlq_error *err);
void rlq_gguf_close(rlq_gguf *g);
void rlq_gguf_header(const rlq_gguf *g, uint32_t *version, uint32_t *alignment, uint64_t *data_offset,
                     uint64_t *n_kv, uint64_t *n_tensors, int32_t *big_endian);
/* Metadata entry i in file order: key bytes, GGUF value type (0..12), the
 * array element type, and count (array elements; string bytes; 1). */
int32_t rlq_gguf_kv_at(const rlq_gguf *g, uint64_t i, const uint8_t **key, uint64_t *key_len, uint32_t *type,
                       uint32_t *element_type, uint64_t *count, rlq_error *err);
/* Scalar value (j = 0) or element j of a scalar array: its bits, zero-extended
 * to 64 (bool as 0/1, as the reader normalizes it). */
int32_t rlq_gguf_kv_scalar(const rlq_gguf *g, uint64_t i, uint64_t j, uint64_t *bits, rlq_error *err);
/* String value (j = 0) or element j of a string array. */
int32_t rlq_gguf_kv_string(const rlq_gguf *g, uint64_t i, uint64_t j, const uint8_t **s, uint64_t *len,
                           rlq_error *err);
/* First entry whose key's C-string prefix equals key's (raw.rs:320-326), or -1. */
int64_t rlq_gguf_find_kv(const rlq_gguf *g, const uint8_t *key, uint64_t len);
/* Tensor descriptor i: name bytes, stored rank, dims (padded with 1 to 4),
 * type, offset within the data section and stored bytes. */
int32_t rlq_gguf_tensor_at(const rlq_gguf *g, uint64_t i, const uint8_t **name, uint64_t *name_len, uint32_t *n_dims,
                           uint64_t *dims, uint32_t *dtype, uint64_t *offset, uint64_t *bytes, rlq_error *err);
int64_t rlq_gguf_find_tensor(const rlq_gguf *g, const uint8_t *name, uint64_t len);
/* read_tensor (lib.rs:322-350): the stored bytes of tensor i; out_len must
 * equal its byte count. */
int32_t rlq_gguf_read_tensor(rlq_gguf *g, uint64_t i, void *out, uint64_t out_len, rlq_error *err);
/* write_native_header (raw.rs:346-390): the header as gguf_get_meta_data
 * writes it (the file's version and alignment, C-string tensor names,
 * trailing unit dimensions dropped, padding to the data offset).  *len gets
 * the size; out may be null to query it. */
int32_t rlq_gguf_native_header(const rlq_gguf *g, uint8_t *out, uint64_t cap, uint64_t *len, rlq_error *err);

/* One metadata entry to write.  type 0..12 (GGUF value types).  Scalars:
 * data holds the value's 1/2/4/8 little-endian bytes.  Strings (8): data
 * holds count bytes.  Arrays (9): element_type and count elements; scalar
 * elements packed in data, string elements concatenated in data with their
 * byte lengths in lengths. */
typedef struct rlq_gguf_kv {
    const uint8_t *key;
    uint64_t key_len;
    uint32_t type, element_type;
    uint64_t count;
    const void *data;
    const uint64_t *lengths;
} rlq_gguf_kv;
/* One tensor to write: dims[0] contiguous (GGML order), data = its stored
 * bytes (row_bytes(dims[0]) x dims[1] x ...). */
typedef struct rlq_gguf_tensor {
    const uint8_t *name;
    uint64_t name_len;
    uint32_t n_dims;
    uint64_t dims[4];
    uint32_t dtype;
    const void *data;
} rlq_gguf_tensor;
/* write_raw_header (writer.rs:476-486): a GGUF v3 little-endian header in the
 * given order, validated before any byte is produced (writer.rs:227-350),
 * padded to the data offset; *file_bytes = the whole file's size. */
int32_t rlq_gguf_write_header(const rlq_gguf_kv *kv, uint64_t n_kv, const rlq_gguf_tensor *tensors,
                              uint64_t n_tensors, uint8_t *out, uint64_t cap, uint64_t *len, uint64_t *file_bytes,
                              rlq_error *err);
/* write_ordered (writer.rs:550-583): header, then each payload padded with
 * zeros to the alignment. */
int32_t rlq_gguf_write(const char *path, const rlq_gguf_kv *kv, uint64_t n_kv, const rlq_gguf_tensor *tensors,
                       uint64_t n_tensors, rlq_error *err);

/* ---- measurement probes ------------------------------------------------
 * No counterpart in the reference: kernels that measure this GPU's practical
 * ceilings for the benchmark, next to the spec peaks.  Both are asynchronous
 * on `stream` and write one word per wave to `out` (4 words per workgroup
 * for rlq_probe_mfma kinds 0-3, 8 for kinds 4-8, 16 for rlq_probe_stream,
 * `waves` for rlq_probe_stream_shape) so that no work is dead. */
/* kind 0: v_mfma_i32_32x32x32_i8, kind 1: v_mfma_f32_32x32x16_f16; each of
 * the 4 waves of `workgroups` 256-thread workgroups runs 4 independent
 * accumulator chains of `iters` MFMAs from registers.  kind 2: `iters` steps
 * of four 1 KB ds_read_b128 reads per wave (the prefill GEMM's A-operand
 * pattern, 20 KB of LDS per workgroup); kind 3: the same four reads per step
 * feeding four v_mfma_f32_32x32x16_f16.  Kinds 4-8: 512-thread workgroups,
 * waves 0-3 running four v_mfma_f32_32x32x16_f16 chains of `iters` steps and
 * waves 4-7 eight f32 FMA chains of 2 * iters steps (two waves per SIMD):
 * kind 4 the MFMA waves alone, 5 the FMA waves alone, 6 both; 7 and 8 as 4
 * and 6 with the MFMA accumulators in AGPRs instead of VGPRs. */
int32_t rlq_probe_mfma(uint32_t kind, uint32_t workgroups, uint32_t iters, uint32_t *out, void *stream);
/* A read of `len` device bytes (a multiple of 1024, 16-byte aligned) by
 * `workgroups` workgroups of 16 waves, each wave instruction a 1 KB run of
 * 16-byte non-temporal loads: the one-column matvec's launch shape and load
 * pattern without its arithmetic. */
int32_t rlq_probe_stream(const void *bytes, uint64_t len, uint32_t workgroups, uint32_t *out, void *stream);
/* The same read by `workgroups` workgroups of `waves` (4, 8 or 16) waves, each
 * wave keeping `runs` (1, 2, 4 or 8) 1 KB runs in flight, with non-temporal
 * loads when `non_temporal` is nonzero, else plain ones; rlq_probe_stream is
 * (16, 2, non-temporal).  Other values: RLQ_INVALID_ARGUMENT. */
int32_t rlq_probe_stream_shape(const void *bytes, uint64_t len, uint32_t workgroups, uint32_t waves, uint32_t runs,
                               uint32_t non_temporal, uint32_t *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RLQ_H */
