// rlq_internal.hpp - host-side launchers shared between the library's
// translation units.  Not part of the C ABI (include/rlq.h is).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>
#include <mutex>
#include <vector>

namespace rlq {

enum DTypeId : uint32_t { kQ8_0 = 8, kQ2_K = 10, kQ3_K = 11, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kQ8_K = 15 };

// Activations of `batch` columns in structure-of-arrays form on the device:
//   q    int8  [batch][cols]
//   d    f32   [batch][cols / block]   (Q8_K: the f32 d; Q8_0: f32 of the
//                                       stored f16 d)
//   bsum int16 [batch][cols / 16]      (Q8_K only: the Q8_K bsums)
//   bad  u8    [batch][cols / block]   nonzero marks a block whose column
//                                      failed validation; the matvec then
//                                      writes nothing (validate-before-mutate)
struct ActPlanes {
    int8_t* q;
    float* d;
    int16_t* bsum;
    uint8_t* bad;
};

// Bytes one ActPlanes needs for `batch` columns of `cols` elements.
size_t act_planes_bytes(uint32_t act_type, uint64_t cols, uint64_t batch);
ActPlanes act_planes_carve(void* base, uint32_t act_type, uint64_t cols, uint64_t batch);

// ---- quantize.hip ----
// Activation quantizers (matvec.rs:56, cpu_extra.rs:820).  Exactly one of
// `planes` / `gguf` may be null.  Data errors go to `err_word`.
hipError_t launch_quantize_q8k(const float* x, uint64_t cols, uint64_t batch, const ActPlanes* planes,
                               uint8_t* gguf, unsigned long long* err_word, hipStream_t s);
hipError_t launch_quantize_q8_0(const float* x, uint64_t cols, uint64_t batch, const ActPlanes* planes,
                                uint8_t* gguf, unsigned long long* err_word, hipStream_t s);
// K weight encoders Q2_K..Q6_K (encode_k.rs:11-561), GGUF bytes out,
// n % 256 == 0.
hipError_t launch_encode_k(uint32_t t, const float* x, uint64_t n, uint8_t* out, unsigned long long* err_word,
                           hipStream_t s);
// GGUF activation bytes (Q8_K / Q8_0) -> planes, for pre-quantized inputs.
hipError_t launch_act_from_gguf(uint32_t act_type, const uint8_t* gguf, uint64_t cols, uint64_t batch,
                                const ActPlanes* planes, hipStream_t s);
// Finite scan over n values: NonFiniteInput{first index} into err_word.
hipError_t launch_finite_scan(const float* x, uint64_t n, unsigned long long* err_word, hipStream_t s);
// Decoders (decode.rs), GGUF bytes in.
hipError_t launch_dequantize(uint32_t dtype, const uint8_t* b, uint64_t n, float* y, hipStream_t s);
// GGUF -> tiled device layout (rlq_layout.hpp); `dev` holds layout_bytes().
hipError_t launch_repack(uint32_t dtype, const uint8_t* gguf, uint64_t rows, uint64_t cols, uint8_t* dev,
                         hipStream_t s);
hipError_t launch_fill_u64(unsigned long long* p, uint64_t n, unsigned long long v, hipStream_t s);

// ---- matvec.hip ----
// The greedy argmax of a decode launch, finished inside the launch (its last
// workgroup decodes the token ids): per-workgroup key slots, the arrival
// counter (0 between launches; set to 0 once when the state is allocated)
// and the caller's token ids.
struct MvArgmax {
    unsigned long long* slots;  // [kArgmaxMaxGrid][8]
    unsigned int* count;
    uint32_t* out;              // [batch]
};
constexpr uint32_t kArgmaxMaxGrid = 4096;  // workgroups of one argmax launch
constexpr size_t kArgmaxStateBytes = 256 + size_t(kArgmaxMaxGrid) * 8 * 8;
inline MvArgmax argmax_state(void* base, uint32_t* out) {
    return MvArgmax{(unsigned long long*)((uint8_t*)base + 256), (unsigned int*)base, out};
}

// y[b*ldy + r] = dot(row r, activation column b) for every b < batch, in
// launches of up to 8 columns.  The activations are quantized in the kernel
// prologue from f32 `x` ([batch][cols]) or taken from `pre` when x is null.
// A data error in the activations goes to `err_word` (column index in the
// key) and suppresses every output of the launch that found it.
// `am` (may be null) receives the greedy argmax of every column in am->out.
// With `dbg_isum`/`dbg_imin` (batch <= 8) the kernel that
// serves this batch size also stores the exact per-(row, block) integers of
// column 0's dot.
hipError_t launch_matvec(uint32_t wtype, const uint8_t* w, uint64_t rows, uint64_t cols, const float* x,
                         const ActPlanes* pre, uint64_t batch, float* y, uint64_t ldy, const MvArgmax* am,
                         unsigned long long* err_word, int32_t* dbg_isum, int32_t* dbg_imin, hipStream_t s);
// Decode-step options of a matvec launch (batch 1 for a transform):
//   xform   0: quantize x as given; 1: RMSNorm(x) * norm_w with `eps`
//           (crates/model-runtime/src/math.rs:214-228); 2: x holds
//           [gate (cols) | up (cols)] and silu(gate) * up is quantized
//           (crates/model-runtime/src/llama.rs:367-371)
//   resid   y = resid + dot (math.rs:203-208); may alias y
//   epilogue 0: store y; 1 (Q4_K, batch 1): the rows are gate and up 16-row
//           tiles interleaved, and y[16 i + r] = silu(gate) * up of tile pair
//           i (llama.rs:367-371), rows / 2 values
struct MvExtra {
    uint32_t xform = 0;
    float eps = 0.0f;
    const float* norm_w = nullptr;
    const float* resid = nullptr;
    uint32_t epilogue = 0;
    uint64_t column_base = 0;          // error-report index of this launch's column 0
    const uint32_t* gate = nullptr;    // device word: nonzero refuses the launch
    // MUL_MAT_ID: id_pairs (token, slot) pairs, expert ids[pair] of
    // id_experts matrices expert_bytes apart, column token * id_cols +
    // slot % id_cols of the pre-quantized planes, y + pair * ldy
    const int32_t* ids = nullptr;
    uint64_t id_pairs = 0;
    uint32_t id_slots = 0, id_cols = 0, id_experts = 0;
    uint64_t expert_bytes = 0;
    // MUL_MAT_ID of one f32 column shared by every pair (one token, one
    // column): each workgroup checks every id, quantizes the column and
    // zeroes its rows of a -1 pair itself, with no gate, planes or prepare
    // launch
    bool id_inline = false;
    // Model-runtime checks: five 5-bit ModelStage ids (RMS scale, quantizer
    // input, quantizer scale, output, output after the residual add; 0 =
    // off) and the layer of the error keys.  0: QuantError keys.
    uint32_t chk = 0, chk_layer = 0;
};
constexpr uint32_t mv_chk(uint32_t scale, uint32_t in, uint32_t quant, uint32_t out, uint32_t resid) {
    return scale | in << 5 | quant << 10 | out << 15 | resid << 20;
}
// The MUL_MAT / MUL_MAT_ID gate (one workgroup, before the products): checks
// the ids (ids may be null) and the `bad` bytes of the pre-quantized planes,
// zeroes the outputs of pairs with id -1, writes *gate.
hipError_t launch_mm_prepare(const int32_t* ids, uint64_t pairs, uint32_t experts, const uint8_t* bad, uint64_t nbad,
                             float* y, uint64_t rows, uint32_t* gate, unsigned long long* err_word, hipStream_t s);
hipError_t launch_matvec_ex(uint32_t wtype, const uint8_t* w, uint64_t rows, uint64_t cols, const float* x,
                            const ActPlanes* pre, uint64_t batch, float* y, uint64_t ldy, const MvArgmax* am,
                            unsigned long long* err_word, int32_t* dbg_isum, int32_t* dbg_imin, const MvExtra& ex,
                            hipStream_t s);
// ---- gemm.hip ----
// Prefill GEMM for Q4_K weights: y[m*ldy + r] = dot(row r, token m) for
// m < M (M > 8 in practice).  Quantizes x [M][cols] to Q8_K (as the f16
// activation image of gemm.hip) in `scratch` (gemm_planes_bytes) first; a
// data error in any token suppresses every output.  `dbg_isum`/`dbg_imin` (may be null) receive token 0's exact
// per-(row, block) integers.
size_t gemm_planes_bytes(uint64_t M, uint64_t K);
hipError_t launch_gemm_q4k(const uint8_t* w, uint64_t rows, uint64_t cols, const float* x, uint64_t M, float* y,
                           uint64_t ldy, void* scratch, unsigned long long* err_word, int32_t* dbg_isum,
                           int32_t* dbg_imin, hipStream_t s);

// ---- llama.hip ----
// The dense Llama decode step (crates/model-runtime/src/llama.rs:222-392)
// over resident weights.  Dimensions are validated by the caller.
struct LlamaDims {
    uint64_t vocab, width, feed_forward, heads, kv_heads, max_context, n_layers;
    float rms_epsilon, rope_base, attention_scale;  // attention_scale 0: 1/sqrt(head_dim)
    uint32_t weight_type, output_type, embedding_type;
};
// GGUF tensors of one layer (rows x cols, rows contiguous) and f32 norms.
struct LlamaHostLayer {
    const float* attention_norm;
    const void *query, *key, *value, *attention_output;
    const float* feed_forward_norm;
    const void *gate, *up, *down;
    uint32_t types[7];  // query, key, value, attention_output, gate, up, down (resolved, nonzero)
};
struct LlamaHostTensors {
    const void* embedding;  // vocab x width, embedding_type
    const float* output_norm;
    const void* output;  // vocab x width, output_type
    const LlamaHostLayer* layers;
    bool on_device;
};
// LDS bytes the attention workgroups need (independent of the context).
uint64_t llama_attn_lds_bytes(uint64_t heads, uint64_t kv_heads, uint64_t head_dim);
struct LlamaLayerDev {
    // tiled matrices: Q, K, V back to back in wqkv; gate and up in wgu
    // (tiles interleaved when the epilogue fuses silu(gate) * up)
    uint8_t *wqkv = nullptr, *wo = nullptr, *wgu = nullptr, *wdown = nullptr;
    float *attn_norm = nullptr, *ffn_norm = nullptr;
    uint32_t tq = 0, tk = 0, tv = 0, to = 0, tg = 0, tu = 0, td = 0;
    uint64_t off_k = 0, off_v = 0, off_up = 0;  // byte offsets of K, V in wqkv and of up in wgu
    bool fused_qkv() const { return tq == tk && tk == tv; }
    // gate/up: 0 = one launch, silu(gate) * up in its epilogue (Q4_K, Q5_K);
    // 1 = one launch over [gate; up], combined in the down projection's
    // quantizer; 2 = two launches (different types), combined the same way
    int gu_mode() const { return tg != tu ? 2 : (tg == kQ4_K || tg == kQ5_K ? 0 : 1); }
};
struct LlamaModel {
    int device = -1;
    LlamaDims d{};
    std::vector<LlamaLayerDev> layers;
    uint8_t *out_w = nullptr, *emb = nullptr;  // tiled output matrix; GGUF embedding rows
    float *out_norm = nullptr, *k_cache = nullptr, *v_cache = nullptr, *rope_tab = nullptr;
    float *qkv = nullptr, *scores = nullptr, *att = nullptr, *gu = nullptr, *logits_buf = nullptr;
    float* mid = nullptr;  // the residual stream after attention (the FFN norm's input)
    // caller's device buffer: each step copies layer l's parts to trace + l *
    // trace_stride(): [q | k | v] (k before RoPE), the attention output, the
    // residual after attention, silu(gate) * up, the layer output
    float* trace = nullptr;
    uint64_t trace_stride() const {
        const uint64_t kvw = d.kv_heads * (d.width / d.heads);
        return 4 * d.width + 2 * kvw + d.feed_forward;
    }
    float* cmax = nullptr;  // [heads][chunks of 16 tokens] chunk maxima of the scores
    void* am_state = nullptr;  // the output matvec's argmax state (kArgmaxStateBytes)
    bool repeat_all = false;  // attention sums always repeated in the reference's order
    uint64_t n_cached = 0;  // KV rows held (the insertion index of the next step)

    ~LlamaModel();
    hipError_t create(const LlamaDims& dims, const LlamaHostTensors& t, hipStream_t s);
    hipError_t embedding(uint32_t token, float* hidden, hipStream_t s) const;
    // silu(gate) * up of the last step's last layer (feed_forward floats, device)
    hipError_t ffn_activation(float* out, hipStream_t s) const;
    hipError_t ffn_activation_of(const LlamaLayerDev& L, float* out, hipStream_t s) const;
    // One step at `position` appending KV row n_cached: hidden (width, device)
    // in/out; embedding_out (width), logits (vocab) and argmax (1) may be null.
    hipError_t step(float* hidden, uint64_t position, float* embedding_out, float* logits, uint32_t* argmax,
                    unsigned long long* err_word, hipStream_t s);
};

// Argmax keys of the stored rows y[b*rows ..] (keys zeroed beforehand).
hipError_t launch_argmax_rows(const float* y, uint64_t batch, uint64_t rows, unsigned long long* keys, hipStream_t s);
// Decode argmax keys into u32 indices; reset: then set the keys back to 0.
hipError_t launch_argmax_finish(unsigned long long* keys, uint64_t batch, const float* y, uint64_t ldy, uint32_t* out,
                                hipStream_t s, bool reset = false);

// ---- per-device launch state (any number of host threads) ----
constexpr int kMaxDevices = 256;

// The compute units of the calling thread's current device, read once per
// device (256 if HIP cannot say).
int device_cus();

// One kernel's dynamic-LDS limit per device: HIP refuses a launch that asks
// for more than 64 KB unless the kernel's limit was raised first.  The limit
// only grows, under the lock, and is recorded after HIP has accepted it, so a
// thread that reads a recorded limit of at least its own size may launch.
// Objects of this class live in static storage (zero-initialized, no
// destructor that calls HIP).
class LdsLimit {
  public:
    hipError_t raise(const void* kernel, size_t bytes) {
        if (bytes <= 64 * 1024) return hipSuccess;
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
        if (bytes <= set_[dev].load(std::memory_order_acquire)) return hipSuccess;
        std::lock_guard<std::mutex> lock(mu_);
        if (bytes <= set_[dev].load(std::memory_order_relaxed)) return hipSuccess;
        e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
        if (e == hipSuccess) set_[dev].store(bytes, std::memory_order_release);
        return e;
    }

  private:
    std::mutex mu_;
    std::atomic<size_t> set_[kMaxDevices] = {};
};

}  // namespace rlq
