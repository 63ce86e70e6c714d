// llama.hip - the dense Llama decode step on the GPU
// (crates/model-runtime/src/llama.rs:222-392): per layer, the QKV matvec
// with the attention RMSNorm fused into its quantizer, RoPE + KV append +
// attention scores, softmax + P.V, the output projection with the residual
// add fused into its store, the gate/up matvec with the FFN RMSNorm fused,
// and the down projection with SiLU(gate)*up fused into its quantizer and the
// residual add into its store.  The final RMSNorm is fused into the output
// matvec, which also yields the greedy argmax.
//
// Exactness: RMSNorm, RoPE (sin/cos from a host table computed with the
// same libm calls and operation order as math.rs:322-334), the QK dot (f32
// products summed in f64 in d order, as the reference), the softmax (SSE2
// exponential of cpu_math.rs:94-123, f32 pair sums, f64 sum in column order)
// and SiLU are the reference's operations in the reference's order.  The P.V
// sums are f64 in 64-token chunks added in order; the matvecs' f32 block
// combine order is the kernels' own (integer block sums are exact).
#include <math.h>

#include <new>
#include <vector>

#include "rlq_device.hpp"
#include "rlq_internal.hpp"
#include "rlq_layout.hpp"

namespace rlq {

constexpr int kAttnChunk = 64;      // tokens per workgroup of the attention kernels
constexpr int kAttnThreads = 256;

// ---------------------------------------------------------------------------
// RoPE of one head slice in place in LDS-ready form: out[2p], out[2p+1] from
// x = in[2p], y = in[2p+1] and the (sin, cos) pair p of the position.
__device__ __forceinline__ void rope_pair(const float* in, const float* tab, uint32_t p, float* out) {
    const float x = in[2 * p], y = in[2 * p + 1], s = tab[2 * p], c = tab[2 * p + 1];
    out[2 * p] = x * c - y * s;
    out[2 * p + 1] = x * s + y * c;
}

// Scores of kv head blockIdx.y's G query heads against tokens
// [64 * blockIdx.x, +64) of the layer cache (math.rs:462-474):
// score = f32(sum_d f64(q_d * k_d)) * scale, the sum in d order.  The
// workgroup whose chunk holds the new row `fresh` applies RoPE to the new key,
// appends it and the new value to the caches, and uses its own copy of the
// key.  scores is [heads][row_stride].
__global__ __launch_bounds__(kAttnThreads) void attn_scores_kernel(const float* __restrict__ qkv,
                                                                   const float* __restrict__ rope_tab,
                                                                   float* __restrict__ kc, float* __restrict__ vc,
                                                                   uint32_t fresh, uint32_t heads, uint32_t kv_heads,
                                                                   uint32_t hd, float scale, float* __restrict__ scores,
                                                                   uint32_t row_stride,
                                                                   unsigned long long* __restrict__ err_word) {
    extern __shared__ __align__(16) float sm[];
    const uint32_t G = heads / kv_heads, kvh = blockIdx.y, t0 = blockIdx.x * kAttnChunk;
    const uint32_t width = heads * hd, kvw = kv_heads * hd, ks = hd + 1;  // odd row stride: no bank conflicts
    float* q_s = sm;              // [G][hd]
    float* k_s = sm + G * hd;     // [64][hd + 1]
    const uint32_t tid = threadIdx.x, count = fresh + 1;
    for (uint32_t i = tid; i < G * hd / 2; i += kAttnThreads) {
        const uint32_t h = i / (hd / 2), p = i % (hd / 2);
        rope_pair(qkv + (kvh * G + h) * hd, rope_tab, p, q_s + h * hd);
    }
    const bool has_fresh = fresh >= t0 && fresh < t0 + kAttnChunk;
    if (has_fresh) {
        float* krow = k_s + (fresh - t0) * ks;
        const float* kin = qkv + width + kvh * hd;
        const float* vin = qkv + width + kvw + kvh * hd;
        for (uint32_t p = tid; p < hd / 2; p += kAttnThreads) {
            float o[2];
            const float x = kin[2 * p], y = kin[2 * p + 1], s = rope_tab[2 * p], c = rope_tab[2 * p + 1];
            o[0] = x * c - y * s;
            o[1] = x * s + y * c;
            krow[2 * p] = o[0];
            krow[2 * p + 1] = o[1];
            kc[(uint64_t)fresh * kvw + kvh * hd + 2 * p] = o[0];
            kc[(uint64_t)fresh * kvw + kvh * hd + 2 * p + 1] = o[1];
        }
        for (uint32_t d = tid; d < hd; d += kAttnThreads) vc[(uint64_t)fresh * kvw + kvh * hd + d] = vin[d];
    }
    // cached keys of the chunk, one row per 16-byte-aligned slice
    const uint32_t n_here = count - t0 < (uint32_t)kAttnChunk ? count - t0 : (uint32_t)kAttnChunk;
    for (uint32_t i = tid; i < n_here * (hd / 4); i += kAttnThreads) {
        const uint32_t t = i / (hd / 4), d4 = i % (hd / 4);
        if (t0 + t == fresh) continue;
        const float4 v = *(const float4*)(kc + (uint64_t)(t0 + t) * kvw + kvh * hd + 4 * d4);
        float* dst = k_s + t * ks + 4 * d4;
        dst[0] = v.x, dst[1] = v.y, dst[2] = v.z, dst[3] = v.w;
    }
    __syncthreads();
    for (uint32_t i = tid; i < G * kAttnChunk; i += kAttnThreads) {
        const uint32_t h = i / kAttnChunk, t = i % kAttnChunk;
        if (t >= n_here) continue;
        const float* q = q_s + h * hd;
        const float* k = k_s + t * ks;
        double dot = 0.0;
        for (uint32_t d = 0; d < hd; ++d) dot += (double)(q[d] * k[d]);
        const float score = (float)dot * scale;
        if (!(fabsf(score) <= 3.402823466e38f)) report_error(err_word, error_key(0, kKindNonFinite, t0 + t));
        scores[(uint64_t)(kvh * G + h) * row_stride + t0 + t] = score;
    }
}

// Softmax of the G heads' score rows (math.rs:293-318 with the SSE2 policy of
// cpu_math.rs:60-91), recomputed by every workgroup of the kv head, then the
// chunk's part of P.V (math.rs:475-482) as f64 sums over its 64 tokens:
// part[chunk][head][d].  Columns past `count` are the -inf padding, whose
// exponentials are exactly 0.
__global__ __launch_bounds__(kAttnThreads) void attn_pv_kernel(const float* __restrict__ scores,
                                                               const float* __restrict__ vc, uint32_t count,
                                                               uint32_t heads, uint32_t kv_heads, uint32_t hd,
                                                               uint32_t row_stride, double* __restrict__ part) {
    extern __shared__ __align__(16) float sm[];
    const uint32_t G = heads / kv_heads, kvh = blockIdx.y, c = blockIdx.x, t0 = c * kAttnChunk;
    const uint32_t n4 = (count + 3) / 4 * 4, ngroups = n4 / 4, kvw = kv_heads * hd;
    float* e_s = sm;                       // [G][n4] exponentials, then probabilities
    float* g_s = sm + G * n4;              // [G][ngroups] f32 pair sums
    float* stat = g_s + G * ngroups;       // [G][2]: max, inverse
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // row maxima, one wave per head
    for (uint32_t h = wave; h < G; h += kAttnThreads / 64) {
        const float* row = scores + (uint64_t)(kvh * G + h) * row_stride;
        float m = -INFINITY;
        for (uint32_t t = lane; t < count; t += 64) m = fmaxf(m, row[t]);
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if (lane == 0) stat[2 * h] = m;
    }
    __syncthreads();
    for (uint32_t i = tid; i < G * n4; i += kAttnThreads) {
        const uint32_t h = i / n4, t = i % n4;
        const float m = stat[2 * h];
        e_s[i] = t < count ? sse2_exp(scores[(uint64_t)(kvh * G + h) * row_stride + t] - m) : 0.0f;
    }
    __syncthreads();
    for (uint32_t i = tid; i < G * ngroups; i += kAttnThreads) {
        const uint32_t h = i / ngroups, g = i % ngroups;
        const float* e = e_s + h * n4 + 4 * g;
        g_s[i] = (e[0] + e[1]) + (e[2] + e[3]);
    }
    __syncthreads();
    if (tid < G) {  // the f64 sum in column order, as the reference
        double sum = 0.0;
        for (uint32_t g = 0; g < ngroups; ++g) sum += (double)g_s[tid * ngroups + g];
        stat[2 * tid + 1] = (float)(1.0 / sum);
    }
    __syncthreads();
    const uint32_t n_here = count - t0 < (uint32_t)kAttnChunk ? count - t0 : (uint32_t)kAttnChunk;
    for (uint32_t i = tid; i < G * hd; i += kAttnThreads) {
        const uint32_t h = i / hd, d = i % hd;
        const float inv = stat[2 * h + 1];
        const float* e = e_s + h * n4 + t0;
        const float* v = vc + (uint64_t)t0 * kvw + kvh * hd + d;
        double acc = 0.0;
        for (uint32_t t = 0; t < n_here; ++t) acc += (double)((e[t] * inv) * v[(uint64_t)t * kvw]);
        part[((uint64_t)c * heads + kvh * G + h) * hd + d] = acc;
    }
}

// out[i] = f32 of the chunk parts added in chunk order.
__global__ __launch_bounds__(256) void attn_reduce_kernel(const double* __restrict__ part, uint32_t nchunks,
                                                          uint32_t n, float* __restrict__ out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    double acc = 0.0;
    for (uint32_t c = 0; c < nchunks; ++c) acc += part[(uint64_t)c * n + i];
    out[i] = (float)acc;
}

// RMSNorm of one row (math.rs:214-228) for the step's embedding output: one
// workgroup, the squares summed in f64 by one thread in index order.
__global__ __launch_bounds__(256) void rms_norm_row_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           uint32_t n, float eps, float* __restrict__ out,
                                                           unsigned long long* __restrict__ err_word) {
    __shared__ float scale_s;
    if (threadIdx.x == 0) {
        double sum = 0.0;
        for (uint32_t i = 0; i < n; ++i) sum += (double)(x[i] * x[i]);
        const float scale = 1.0f / sqrtf((float)(sum / (double)n) + eps);
        if (!(scale <= 3.402823466e38f) || !(scale > 0.0f)) report_error(err_word, error_key(0, kKindNonFinite, 0));
        scale_s = scale;
    }
    __syncthreads();
    const float scale = scale_s;
    for (uint32_t i = threadIdx.x; i < n; i += 256) out[i] = x[i] * scale * w[i];
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

namespace {

hipError_t upload_tiled(uint32_t t, const void* gguf, uint64_t rows, uint64_t cols, bool on_device, uint8_t* dst,
                        void* staging, hipStream_t s) {
    const uint8_t* src = (const uint8_t*)gguf;
    if (!on_device) {
        const uint64_t len = rows * (cols / (t == kQ8_0 ? 32 : 256)) * (t == kQ8_0 ? 34 : (t == kQ4_K ? 144 : 210));
        const hipError_t e = hipMemcpyAsync(staging, src, len, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return e;
        src = (const uint8_t*)staging;
    }
    const hipError_t e = launch_repack(t, src, rows, cols, dst, s);
    if (e != hipSuccess) return e;
    return on_device ? hipSuccess : hipStreamSynchronize(s);  // the staging buffer is reused
}

hipError_t upload_f32(const float* src, uint64_t n, bool on_device, float** dst, hipStream_t s) {
    hipError_t e = hipMalloc((void**)dst, n * sizeof(float));
    if (e != hipSuccess) return e;
    return hipMemcpyAsync(*dst, src, n * sizeof(float), on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                          s);
}

uint64_t gguf_row_bytes(uint32_t t, uint64_t cols) {
    switch (t) {
        case kQ8_0: return cols / 32 * 34;
        case kQ4_K: return cols / 256 * 144;
        case kQ6_K: return cols / 256 * 210;
        default: return 0;
    }
}

}  // namespace

LlamaModel::~LlamaModel() {
    if (device >= 0) (void)hipSetDevice(device);
    (void)hipDeviceSynchronize();
    for (LlamaLayerDev& l : layers)
        for (void* p : {(void*)l.wqkv, (void*)l.wo, (void*)l.wgu, (void*)l.wdown, (void*)l.attn_norm,
                        (void*)l.ffn_norm})
            if (p) (void)hipFree(p);
    for (void* p : {(void*)out_w, (void*)out_norm, (void*)emb, (void*)k_cache, (void*)v_cache, (void*)rope_tab,
                    (void*)qkv, (void*)scores, (void*)part, (void*)att, (void*)gu, (void*)argmax_keys,
                    (void*)logits_buf})
        if (p) (void)hipFree(p);
}

hipError_t LlamaModel::create(const LlamaDims& dims, const LlamaHostTensors& t, hipStream_t s) {
    d = dims;
    const uint64_t W = d.width, F = d.feed_forward, hd = W / d.heads, kvw = d.kv_heads * hd;
    layers.assign(d.n_layers, LlamaLayerDev{});
    // the rope table: the reference's theta sequence and libm sin/cos per position
    std::vector<float> tab(d.max_context * hd);
    const float theta_scale = powf(d.rope_base, -2.0f / (float)hd);
    for (uint64_t p = 0; p < d.max_context; ++p) {
        float theta = (float)p;
        for (uint64_t i = 0; i < hd / 2; ++i) {
            tab[p * hd + 2 * i] = sinf(theta);
            tab[p * hd + 2 * i + 1] = cosf(theta);
            theta *= theta_scale;
        }
    }
    const uint64_t row_len = (d.max_context + 255) / 256 * 256, nchunks = (d.max_context + kAttnChunk - 1) / kAttnChunk;
    // the attention workgroups' LDS grows with the context (the caller checked 160 KB)
    hipError_t e = hipFuncSetAttribute((const void*)attn_pv_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       160 * 1024);
    if (e == hipSuccess)
        e = hipFuncSetAttribute((const void*)attn_scores_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024);
    if (e == hipSuccess) e = hipMalloc((void**)&rope_tab, tab.size() * sizeof(float));
    if (e == hipSuccess) e = hipMemcpy(rope_tab, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMalloc((void**)&k_cache, d.n_layers * d.max_context * kvw * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&v_cache, d.n_layers * d.max_context * kvw * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&qkv, (W + 2 * kvw) * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&scores, d.heads * row_len * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&part, nchunks * W * sizeof(double));
    if (e == hipSuccess) e = hipMalloc((void**)&att, W * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&gu, 2 * F * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&argmax_keys, sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMalloc((void**)&logits_buf, d.vocab * sizeof(float));
    if (e != hipSuccess) return e;
    // staging for host GGUF bytes: the largest tensor
    void* staging = nullptr;
    if (!t.on_device) {
        uint64_t big = gguf_row_bytes(d.weight_type, W) * F;
        big = big > gguf_row_bytes(d.weight_type, F) * W ? big : gguf_row_bytes(d.weight_type, F) * W;
        const uint64_t o = gguf_row_bytes(d.output_type, W) * d.vocab;
        big = big > o ? big : o;
        e = hipMalloc(&staging, big);
        if (e != hipSuccess) return e;
    }
    const uint32_t wt = d.weight_type;
    auto tiled = [&](const void* src, uint64_t rows, uint64_t cols, uint8_t* dst) {
        return upload_tiled(wt, src, rows, cols, t.on_device, dst, staging, s);
    };
    for (uint64_t l = 0; l < d.n_layers && e == hipSuccess; ++l) {
        const LlamaHostLayer& hl = t.layers[l];
        LlamaLayerDev& L = layers[l];
        // Q, K, V (and gate, up) share one tiled buffer: rows are whole tiles
        const uint64_t bq = layout_bytes(wt, W, W), bk = layout_bytes(wt, kvw, W), bg = layout_bytes(wt, F, W);
        e = hipMalloc((void**)&L.wqkv, bq + 2 * bk);
        if (e == hipSuccess) e = tiled(hl.query, W, W, L.wqkv);
        if (e == hipSuccess) e = tiled(hl.key, kvw, W, L.wqkv + bq);
        if (e == hipSuccess) e = tiled(hl.value, kvw, W, L.wqkv + bq + bk);
        if (e == hipSuccess) e = hipMalloc((void**)&L.wo, layout_bytes(wt, W, W));
        if (e == hipSuccess) e = tiled(hl.attention_output, W, W, L.wo);
        if (e == hipSuccess) e = hipMalloc((void**)&L.wgu, 2 * bg);
        if (e == hipSuccess) e = tiled(hl.gate, F, W, L.wgu);
        if (e == hipSuccess) e = tiled(hl.up, F, W, L.wgu + bg);
        if (e == hipSuccess) e = hipMalloc((void**)&L.wdown, layout_bytes(wt, W, F));
        if (e == hipSuccess) e = tiled(hl.down, W, F, L.wdown);
        if (e == hipSuccess) e = upload_f32(hl.attention_norm, W, t.on_device, &L.attn_norm, s);
        if (e == hipSuccess) e = upload_f32(hl.feed_forward_norm, W, t.on_device, &L.ffn_norm, s);
    }
    if (e == hipSuccess) e = hipMalloc((void**)&out_w, layout_bytes(d.output_type, d.vocab, W));
    if (e == hipSuccess)
        e = upload_tiled(d.output_type, t.output, d.vocab, W, t.on_device, out_w, staging, s);
    if (e == hipSuccess) e = upload_f32(t.output_norm, W, t.on_device, &out_norm, s);
    const uint64_t emb_bytes = gguf_row_bytes(d.embedding_type, W) * d.vocab;
    if (e == hipSuccess) e = hipMalloc((void**)&emb, emb_bytes);
    if (e == hipSuccess)
        e = hipMemcpyAsync(emb, t.embedding, emb_bytes, t.on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                           s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (staging) (void)hipFree(staging);
    return e;
}

hipError_t LlamaModel::embedding(uint32_t token, float* hidden, hipStream_t s) const {
    const uint64_t rb = gguf_row_bytes(d.embedding_type, d.width);
    return launch_dequantize(d.embedding_type, emb + (uint64_t)token * rb, d.width, hidden, s);
}

hipError_t LlamaModel::step(float* hidden, uint64_t position, float* embedding_out, float* logits, uint32_t* argmax,
                            unsigned long long* err_word, hipStream_t s) {
    const uint64_t W = d.width, F = d.feed_forward, H = d.heads, KVH = d.kv_heads, hd = W / H, kvw = KVH * hd;
    const uint64_t fresh = n_cached, count = fresh + 1;
    const uint64_t row_stride = (d.max_context + 255) / 256 * 256;
    const uint32_t nchunks = (uint32_t)((count + kAttnChunk - 1) / kAttnChunk);
    const float scale = d.attention_scale != 0.0f ? d.attention_scale : 1.0f / sqrtf((float)hd);
    const float* tab = rope_tab + position * hd;
    const uint32_t wt = d.weight_type;
    const size_t lds_scores = (H / KVH * hd + kAttnChunk * (hd + 1)) * sizeof(float);
    const uint64_t n4 = (count + 3) / 4 * 4;
    const size_t lds_pv = (H / KVH * n4 + H / KVH * (n4 / 4) + 2 * (H / KVH)) * sizeof(float);
    hipError_t e = hipSuccess;
    for (uint64_t l = 0; l < d.n_layers && e == hipSuccess; ++l) {
        const LlamaLayerDev& L = layers[l];
        float* kc = k_cache + l * d.max_context * kvw;
        float* vc = v_cache + l * d.max_context * kvw;
        MvExtra norm1;
        norm1.xform = 1, norm1.eps = d.rms_epsilon, norm1.norm_w = L.attn_norm;
        e = launch_matvec_ex(wt, L.wqkv, W + 2 * kvw, W, hidden, nullptr, 1, qkv, W + 2 * kvw, nullptr, err_word,
                             nullptr, nullptr, norm1, s);
        if (e != hipSuccess) break;
        hipLaunchKernelGGL(attn_scores_kernel, dim3(nchunks, (uint32_t)KVH), dim3(kAttnThreads), lds_scores, s, qkv,
                           tab, kc, vc, (uint32_t)fresh, (uint32_t)H, (uint32_t)KVH, (uint32_t)hd, scale, scores,
                           (uint32_t)row_stride, err_word);
        hipLaunchKernelGGL(attn_pv_kernel, dim3(nchunks, (uint32_t)KVH), dim3(kAttnThreads), lds_pv, s, scores, vc,
                           (uint32_t)count, (uint32_t)H, (uint32_t)KVH, (uint32_t)hd, (uint32_t)row_stride, part);
        hipLaunchKernelGGL(attn_reduce_kernel, dim3((uint32_t)((W + 255) / 256)), dim3(256), 0, s, part, nchunks,
                           (uint32_t)W, att);
        e = hipGetLastError();
        if (e != hipSuccess) break;
        MvExtra res;
        res.resid = hidden;
        e = launch_matvec_ex(wt, L.wo, W, W, att, nullptr, 1, hidden, W, nullptr, err_word, nullptr, nullptr, res, s);
        if (e != hipSuccess) break;
        MvExtra norm2;
        norm2.xform = 1, norm2.eps = d.rms_epsilon, norm2.norm_w = L.ffn_norm;
        e = launch_matvec_ex(wt, L.wgu, 2 * F, W, hidden, nullptr, 1, gu, 2 * F, nullptr, err_word, nullptr, nullptr,
                             norm2, s);
        if (e != hipSuccess) break;
        MvExtra down;
        down.xform = 2, down.resid = hidden;
        e = launch_matvec_ex(wt, L.wdown, W, F, gu, nullptr, 1, hidden, W, nullptr, err_word, nullptr, nullptr, down,
                             s);
    }
    if (e != hipSuccess) return e;
    if (embedding_out) {
        hipLaunchKernelGGL(rms_norm_row_kernel, dim3(1), dim3(256), 0, s, hidden, out_norm, (uint32_t)W,
                           d.rms_epsilon, embedding_out, err_word);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (logits || argmax) {
        MvExtra norm3;
        norm3.xform = 1, norm3.eps = d.rms_epsilon, norm3.norm_w = out_norm;
        if (argmax) {
            e = launch_fill_u64(argmax_keys, 1, 0ull, s);
            if (e != hipSuccess) return e;
        }
        // logits land in the caller's buffer, or in the model's own when only
        // the argmax is wanted
        float* y = logits ? logits : logits_buf;
        e = launch_matvec_ex(d.output_type, out_w, d.vocab, W, hidden, nullptr, 1, y, d.vocab,
                             argmax ? argmax_keys : nullptr, err_word, nullptr, nullptr, norm3, s);
        if (e == hipSuccess && argmax) e = launch_argmax_finish(argmax_keys, 1, y, d.vocab, argmax, s);
        if (e != hipSuccess) return e;
    }
    ++n_cached;
    return hipSuccess;
}

}  // namespace rlq
