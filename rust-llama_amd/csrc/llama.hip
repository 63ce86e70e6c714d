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
// same libm calls and operation order as math.rs:322-334), the softmax
// exponentials (SSE2 exponential of cpu_math.rs:94-123) and pair sums, and
// SiLU are the reference's operations in the reference's order.  The f64 sums
// of the QK dots, the softmax totals and the P.V outputs run in parallel
// orders whose f32 results are certified equal to the reference's (or
// repeated in its order: certified_f32, pv_interval, f64_sum_exact), so scores,
// probabilities and attention outputs are bit-exact.  The one-column
// matvecs of every weight type combine their exact integer block sums in the
// reference's f32 order.
#include <math.h>
#include <stdlib.h>

#include <new>
#include <stdexcept>
#include <vector>

#include "rlq_device.hpp"
#include "rlq_internal.hpp"
#include "rlq_layout.hpp"

namespace rlq {

constexpr int kAttnChunk = 16;      // tokens per workgroup of the scores kernel
constexpr int kAttnThreads = 256;
constexpr uint32_t kAttnMaxHd = 256;  // head dimension limit
constexpr uint32_t kScKeyRegs = kAttnMaxHd * kAttnChunk / 4 / kAttnThreads;  // float4 of a chunk's keys per thread
constexpr uint32_t kScKeyPad = 16;  // floats after each key row in LDS
static_assert(kAttnMaxHd <= kAttnThreads, "the new key row: one element per thread");

constexpr uint32_t kPvDims = 4;       // head dimensions per P.V workgroup: one float4 of each value row
constexpr uint32_t kPvMaxWaves = 8;   // waves per P.V workgroup: one per query head of the kv head
constexpr uint32_t kPvRegGroups = 4;  // column groups of four per lane whose values and exponentials stay in registers
constexpr uint32_t kPvRepTerms = 256;  // f64 terms per round of a sequential P.V repeat

// The value cache of a layer is slice-major: [kv_heads * hd / 4][max_context]
// float4, slice kvh * hd / 4 + d / 4 holding dimensions d .. d + 3 of kv head
// kvh for every token, so a P.V workgroup reads one contiguous run.
__host__ __device__ inline uint64_t v_cache_index(uint32_t kvh, uint32_t hd, uint32_t d, uint64_t token,
                                                  uint64_t max_context) {
    return ((uint64_t)(kvh * (hd / 4) + d / 4) * max_context + token) * 4 + d % 4;
}

// P.V waves per workgroup, and its LDS: one kPvRepTerms f64 buffer per wave
// for the sequential repeats (it does not grow with the context: the scores
// and values stream from HBM).
__host__ __device__ inline uint32_t pv_waves(uint32_t G) { return G < kPvMaxWaves ? G : kPvMaxWaves; }
__host__ __device__ inline uint32_t attn_pv_lds_bytes(uint32_t G) { return pv_waves(G) * kPvRepTerms * 8; }
__host__ __device__ inline uint32_t attn_scores_lds(uint32_t G, uint32_t hd) {
    return (G * hd + kAttnChunk * (hd + kScKeyPad)) * 4;
}

uint64_t llama_attn_lds_bytes(uint64_t heads, uint64_t kv_heads, uint64_t head_dim) {
    const uint64_t G = heads / kv_heads;
    const uint64_t pv = attn_pv_lds_bytes((uint32_t)G);
    const uint64_t sc = attn_scores_lds((uint32_t)G, (uint32_t)head_dim);
    return pv > sc ? pv : sc;
}

// ---------------------------------------------------------------------------
// RoPE of one head slice in place in LDS-ready form: out[2p], out[2p+1] from
// x = in[2p], y = in[2p+1] and the (sin, cos) pair p of the position.
__device__ __forceinline__ void rope_pair(const float* in, const float* tab, uint32_t p, float* out) {
    const float x = in[2 * p], y = in[2 * p + 1], s = tab[2 * p], c = tab[2 * p + 1];
    out[2 * p] = x * c - y * s;
    out[2 * p + 1] = x * s + y * c;
}

// The reference adds the f64 terms of its attention sums in one fixed order
// and rounds the total to f32 (math.rs:467-471, 309-313, 475-488).  These
// kernels add the same terms in a parallel order.  Two orders of the same n
// additions differ by at most 2 (n - 1) 2^-53 sum|term|, so when every value
// that close to `sum` rounds to the same f32 (f32 rounding is monotone, so
// the two ends decide it), the reference's total rounds to that f32 as well.
// `f` maps the f64 total to the f32 result (a cast, or the cast of 1/total).
// Returns false when that cannot be certified; the caller then repeats the
// sum in the reference's order.
template <typename F>
__device__ __forceinline__ bool certified_f32(double sum, double abs_sum, uint32_t n, F f, float* out) {
    const double eps = (double)n * 2.3e-16 * abs_sum;  // 2^-52 with a margin for the rounding of eps itself
    *out = f(sum);
    return f(sum - eps) == f(sum + eps);
}
__device__ __forceinline__ float f64_to_f32(double x) { return (float)x; }

// Whether every order of an f64 sum of f32 terms gives the exact sum: with M
// the smallest |term| (0 when a term is zero) and A >= sum |term|, every term
// of magnitude >= M is a multiple of q = ulp(M) (2^-149 for a subnormal M),
// so when A < 2^53 q every partial sum in any order is a multiple of q below
// 2^53 q, exactly representable, and every f64 addition is exact.
__device__ __forceinline__ bool f64_sum_exact(double A, float M) {
    const uint32_t b = (__float_as_uint(M) >> 23) & 0xffu;  // q = 2^(b - 150), 2^-149 for b = 0
    const double lim = __longlong_as_double((long long)((uint64_t)((b == 0u ? 1u : b) + 53u + 1023u - 150u) << 52));
    return M > 0.0f && M < INFINITY && A * (1.0 + 1e-3) < lim;
}

// Scores of kv head blockIdx.y's G query heads against tokens
// [16 * blockIdx.x, +16) of the layer cache (math.rs:462-474):
// score = f32(sum_d f64(q_d * k_d)) * scale, the sum in d order.  The
// workgroup whose chunk holds the new row `fresh` applies RoPE to the new key,
// appends it and the new value to the caches, and uses its own copy of the
// key.  scores is [heads][row_stride]; cmax[head][chunk] (stride cstride)
// receives each chunk's maximum score.  Four lanes share a (head, token) dot:
// quarter j takes the float4s j, j + 4, ... of the row, and a wave holds one
// head's 16 tokens.
__global__ __launch_bounds__(kAttnThreads) void attn_scores_kernel(
    const float* __restrict__ qkv, const float* __restrict__ rope_tab, float* __restrict__ kc, float* __restrict__ vc,
    uint32_t max_context, uint32_t fresh, uint32_t heads, uint32_t kv_heads, uint32_t hd, float scale,
    float* __restrict__ scores, uint32_t row_stride, float* __restrict__ cmax, uint32_t cstride,
    unsigned long long* __restrict__ err_word, uint32_t layer, uint32_t repeat_all) {
    extern __shared__ __align__(16) float sm[];
    const uint32_t G = heads / kv_heads, kvh = blockIdx.y, c = blockIdx.x, t0 = c * kAttnChunk;
    // key rows at a stride of hd + 16 floats: the two rows one eight-lane LDS
    // pass reads (four quarters each) start 16 banks apart
    const uint32_t width = heads * hd, kvw = kv_heads * hd, ks = hd + kScKeyPad;
    float* q_s = sm;              // [G][hd]
    float* k_s = sm + G * hd;     // [16][hd + 16]
    const uint32_t tid = threadIdx.x, count = fresh + 1, q4 = hd / 4;
    const uint32_t n_here = count - t0 < (uint32_t)kAttnChunk ? count - t0 : (uint32_t)kAttnChunk;
    // the chunk's cached keys: every load issued before any is used
    float4 kr[kScKeyRegs];
#pragma unroll
    for (uint32_t k = 0; k < kScKeyRegs; ++k) {
        const uint32_t i = tid + k * kAttnThreads, t = i / q4;
        kr[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (t < n_here && t0 + t != fresh)
            kr[k] = load_stream_f4(kc + (uint64_t)(t0 + t) * kvw + kvh * hd + 4 * (i % q4));
    }
    // the new key's pair and value element of this thread (hd <= the
    // workgroup's threads), loaded with the cached keys
    const bool has_fresh = fresh >= t0 && fresh < t0 + kAttnChunk;
    float fx = 0.0f, fy = 0.0f, fsn = 0.0f, fcs = 0.0f, fv = 0.0f;
    if (has_fresh) {
        const float* kin = qkv + width + kvh * hd;
        if (tid < hd / 2) fx = kin[2 * tid], fy = kin[2 * tid + 1], fsn = rope_tab[2 * tid], fcs = rope_tab[2 * tid + 1];
        if (tid < hd) fv = qkv[width + kvw + kvh * hd + tid];
    }
    for (uint32_t i = tid; i < G * hd / 2; i += kAttnThreads) {
        const uint32_t h = i / (hd / 2), p = i % (hd / 2);
        rope_pair(qkv + (kvh * G + h) * hd, rope_tab, p, q_s + h * hd);
    }
    if (has_fresh) {
        if (tid < hd / 2) {
            const float o0 = fx * fcs - fy * fsn, o1 = fx * fsn + fy * fcs;
            float* krow = k_s + (fresh - t0) * ks;
            krow[2 * tid] = o0;
            krow[2 * tid + 1] = o1;
            kc[(uint64_t)fresh * kvw + kvh * hd + 2 * tid] = o0;
            kc[(uint64_t)fresh * kvw + kvh * hd + 2 * tid + 1] = o1;
        }
        if (tid < hd) vc[v_cache_index(kvh, hd, tid, fresh, max_context)] = fv;
    }
#pragma unroll
    for (uint32_t k = 0; k < kScKeyRegs; ++k) {
        const uint32_t i = tid + k * kAttnThreads, t = i / q4;
        if (t < n_here && t0 + t != fresh) *(float4*)(k_s + t * ks + 4 * (i % q4)) = kr[k];
    }
    __syncthreads();
    // pair (h, t) = i takes lanes 4i .. 4i + 3; the trip count is uniform per
    // wave (G * 16 pairs, 16 per wave), so every lane reaches the shuffles
    const uint32_t quarter = tid & 3;
    for (uint32_t i = tid >> 2; i < G * kAttnChunk; i += kAttnThreads / 4) {
        const uint32_t h = i / kAttnChunk, t = i % kAttnChunk;
        const bool live = t < n_here;
        const float* q = q_s + h * hd;
        const float* k = k_s + t * ks;
        // four interleaved partial sums per lane, then the four lanes'; the
        // f32 total is certified against the reference's d-order sum (exact
        // in every order, f64_sum_exact, or by the bound of certified_f32), or
        // recomputed in that order.  The magnitudes are summed in f32
        // (relative error < 2^-16 for hd <= 256, covered by the factor 1.01).
        double a[4] = {0.0, 0.0, 0.0, 0.0};
        float b = 0.0f, mn = INFINITY;
        if (live) {
            for (uint32_t d = 4 * quarter; d < hd; d += 16) {
                const float4 q4v = *(const float4*)(q + d), k4 = *(const float4*)(k + d);
                const float x0 = q4v.x * k4.x, x1 = q4v.y * k4.y, x2 = q4v.z * k4.z, x3 = q4v.w * k4.w;
                a[0] += (double)x0, a[1] += (double)x1, a[2] += (double)x2, a[3] += (double)x3;
                b += (fabsf(x0) + fabsf(x1)) + (fabsf(x2) + fabsf(x3));
                mn = fminf(mn, fminf(fminf(fabsf(x0), fabsf(x1)), fminf(fabsf(x2), fabsf(x3))));
            }
        }
        double part = (a[0] + a[1]) + (a[2] + a[3]);
        part += dpp_d<kQuadXor1>(part);  // the four lanes of the pair, by DPP
        part += dpp_d<kQuadXor2>(part);
        b += dpp_f<kQuadXor1>(b);
        b += dpp_f<kQuadXor2>(b);
        mn = fminf(mn, dpp_f<kQuadXor1>(mn));
        mn = fminf(mn, dpp_f<kQuadXor2>(mn));
        float score = -INFINITY;
        if (live) {
            float dotf;
            const bool exact = f64_sum_exact(1.01 * (double)b, mn);
            if (exact) dotf = (float)part;
            if ((!exact && !certified_f32(part, 1.01 * (double)b, hd, f64_to_f32, &dotf)) || repeat_all) {
                // sixteen products loaded and formed ahead of their adds
                double dot = 0.0;
                for (uint32_t d = 0; d < hd; d += 16) {
                    float x[16];
#pragma unroll
                    for (uint32_t u = 0; u < 4; ++u) {
                        const float4 qa = *(const float4*)(q + d + 4 * u), ka = *(const float4*)(k + d + 4 * u);
                        x[4 * u] = qa.x * ka.x, x[4 * u + 1] = qa.y * ka.y;
                        x[4 * u + 2] = qa.z * ka.z, x[4 * u + 3] = qa.w * ka.w;
                    }
#pragma unroll
                    for (uint32_t u = 0; u < 16; ++u) dot += (double)x[u];
                }
                dotf = (float)dot;
            }
            score = dotf * scale;
            if (quarter == 0) {
                if (!(fabsf(score) <= 3.402823466e38f)) report_error(err_word, model_key(layer, kStScore, t0 + t));
                scores[(uint64_t)(kvh * G + h) * row_stride + t0 + t] = score;
            }
        }
        // the maximum of the wave's 16 pairs (one head's 16 tokens)
        const float m = wave_max_dpp(score);
        if ((tid & 63) == 0) cmax[(kvh * G + h) * cstride + c] = m;
    }
}

// Softmax of the G heads' score rows (math.rs:293-318 with the SSE2 policy of
// cpu_math.rs:60-91) and P.V (math.rs:475-488) for 4 of the head dimensions:
// workgroup (blockIdx.x, blockIdx.y) = (dimensions 4 * blockIdx.x .., kv head),
// one wave per query head of the kv head (heads past kPvMaxWaves loop over the
// waves).  The waves never wait for each other: each one takes its head's
// maximum from the chunk maxima, the exponentials of every column and their
// total, and the four P.V sums.  The columns go in groups of four (the
// reference's SSE2 vectors); lane r takes groups r, r + 64, ...  Its first
// kPvRegGroups groups' values (shared by the wave's heads) are loaded when the
// kernel starts and their exponentials kept from the row total; later groups
// are reloaded and their exponentials recomputed (the same f32 function of the
// same inputs), so the LDS does not grow with the context.  The softmax total
// is certified against the reference's order (certified_f32).  Each P.V sum
// adds the reference's f64 terms f64(p * v) in another order (per lane, then
// the wave in a fixed tree); its f32 result is certified (pv_interval) or the
// sum is repeated in the reference's column order.  Columns past `count` have
// exponential 0 and are not added.
// (The four exponentials are computed whatever the count and masked after,
// so no lane branches and their evaluations interleave.)
__device__ __forceinline__ void exp_group(float4 x, uint32_t t, uint32_t count, float m, float (&e)[4]) {
    const float v[4] = {sse2_exp(x.x - m), sse2_exp(x.y - m), sse2_exp(x.z - m), sse2_exp(x.w - m)};
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) e[j] = __uint_as_float(__float_as_uint(v[j]) & (t + j < count ? ~0u : 0u));
}

// Whether the f32 rounding of a P.V sum added in the kernel's order (sum; at
// most tl columns per lane) is the f32 rounding of the reference's
// sequential sum (math.rs:482-488).  A = sum |term|, M = min |term| (0 when
// a term is zero), wsum = sum over the column groups g (four columns, in
// column order, R of them) of (R - 1 - g) |group sum|, each group sum the
// growth of a lane's f64 sum rounded to f32 (within 2^-23 of itself plus
// 4 2^-53 A of the exact one).
//  - by an interval (pv_interval): the reference's k-th partial sum rounds by at most
//    2^-53 of itself, and its prefix P_k lies within |E_g| + A_g of zero (E_g
//    the sum of the groups before column k's group g, |E_g| <= the sum of
//    their |group sums|, A_g the group's sum |term|), so its sum is within
//    2^-53 (4 wsum 1.001 + 4 (4 2^-53 R^2 + 1) A) of the exact one; the kernel's within
//    2^-53 (tl A + 40 A) (each lane's columns, then the wave's tree of six
//    levels).  When both ends of that interval round to one f32, so does the
//    reference's sum;
//  - else exactly (f64_sum_exact of A and M).
// The interval's coefficient of A: 4 (4 2^-53 R^2 + 1) + tl + 40.
__device__ __forceinline__ double pv_coef_a(double tl, double R) {
    return 4.0 * (4.0 * 1.1102230246251565e-16 * R * R + 1.0) + tl + 40.0;
}
// The interval test with C = 4 wsum + pv_coef_a A (C computed in f32 per
// lane and per 16-lane row: relative error below 1e-6, covered by one more
// factor 1.001).
__device__ __forceinline__ bool pv_interval(double sum, double C) {
    const double B = 1.1102230246251565e-16 * 1.02 * 1.001 * 1.001 * C;
    return (float)(sum - B) == (float)(sum + B);
}

__device__ __forceinline__ float f4_at(const float4& v, uint32_t j) {
    return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}

// Sum / minimum over each 16-lane row (DPP only).
__device__ __forceinline__ float row16_sum_f(float v) {
    v += dpp_f<kQuadXor1>(v);
    v += dpp_f<kQuadXor2>(v);
    v += dpp_f<kRowHalfMirror>(v);
    return v + dpp_f<kRowRor8>(v);
}
__device__ __forceinline__ float row16_min_f(float v) {
    v = fminf(v, dpp_f<kQuadXor1>(v));
    v = fminf(v, dpp_f<kQuadXor2>(v));
    v = fminf(v, dpp_f<kRowHalfMirror>(v));
    return fminf(v, dpp_f<kRowRor8>(v));
}

__global__ __launch_bounds__(kPvMaxWaves * 64) void attn_pv_kernel(
    const float* __restrict__ scores, const float* __restrict__ cmax, uint32_t cstride, uint32_t nch,
    const float* __restrict__ vc, uint32_t max_context, uint32_t count, uint32_t heads, uint32_t kv_heads, uint32_t hd,
    uint32_t row_stride, float* __restrict__ att, unsigned long long* __restrict__ err_word, uint32_t layer,
    uint32_t repeat_all) {
    extern __shared__ __align__(16) double rep_s[];  // [waves][kPvRepTerms]: the sequential repeats
    const uint32_t G = heads / kv_heads, kvh = blockIdx.y, d0 = blockIdx.x * kPvDims;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const uint32_t ngroups = (count + 3) / 4;
    const float4* vsrc = (const float4*)(vc + v_cache_index(kvh, hd, d0, 0, max_context));
    double* buf = rep_s + wave * kPvRepTerms;
    float4 vr[kPvRegGroups][4];
#pragma unroll
    for (uint32_t k = 0; k < kPvRegGroups; ++k)
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const uint32_t t = 4 * (lane + 64 * k) + j;
            vr[k][j] = t < count ? vsrc[t] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    const double tl = 4.0 * ((ngroups + 63) / 64);  // columns per lane
    for (uint32_t h = wave; h < G; h += nw) {        // (wave-uniform)
        const uint32_t row = kvh * G + h;
        const float* srow = scores + (uint64_t)row * row_stride;
        float4 sr[kPvRegGroups];
#pragma unroll
        for (uint32_t k = 0; k < kPvRegGroups; ++k) {
            const uint32_t g = lane + 64 * k;
            sr[k] = g < ngroups ? *(const float4*)(srow + 4 * g) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        float m = -INFINITY;
        for (uint32_t c = lane; c < nch; c += 64) m = fmaxf(m, cmax[row * cstride + c]);
        m = wave_max_dpp(m);
        // exponentials and f32 pair sums of each group (math.rs:303-313), the
        // lane's pair sums added in f64
        float er[kPvRegGroups][4];
        double sum = 0.0;
#pragma unroll
        for (uint32_t k = 0; k < kPvRegGroups; ++k) {
            const uint32_t g = lane + 64 * k;
            exp_group(sr[k], 4 * g, count, m, er[k]);  // zero past the row (4 g >= count there)
            sum += (double)((er[k][0] + er[k][1]) + (er[k][2] + er[k][3]));
        }
        for (uint32_t g = lane + 64 * kPvRegGroups; g < ngroups; g += 64) {
            float e[4];
            exp_group(*(const float4*)(srow + 4 * g), 4 * g, count, m, e);
            sum += (double)((e[0] + e[1]) + (e[2] + e[3]));
        }
        sum = wave_sum_f64(sum);
        // the row total, certified against the reference's column-order f64
        // sum (the pair sums are >= 0: sum = sum |.|), else repeated in that
        // order: 64 pair sums per load, added lane by lane
        float inv;
        if (!certified_f32(sum, sum, ngroups, [](double x) { return (float)(1.0 / x); }, &inv) || repeat_all) {
            double seq = 0.0;
            for (uint32_t base = 0; base < ngroups; base += 64) {
                float ps = 0.0f;
                if (base + lane < ngroups) {
                    float e[4];
                    exp_group(*(const float4*)(srow + 4 * (base + lane)), 4 * (base + lane), count, m, e);
                    ps = (e[0] + e[1]) + (e[2] + e[3]);
                }
                const uint32_t n = ngroups - base < 64 ? ngroups - base : 64;
                for (uint32_t l = 0; l < n; ++l) seq += (double)readlane_f(ps, (int)l);
            }
            inv = (float)(1.0 / seq);
        }
        // P.V with p = e * inverse (math.rs:313-315, 478-480), one f64 chain
        // per dimension over the lane's groups, and the certificate's
        // statistics of the terms (pv_interval, f64_sum_exact)
        double a[4] = {0.0, 0.0, 0.0, 0.0};
        float as[4] = {0.0f, 0.0f, 0.0f, 0.0f}, ws[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        // the reference adds `count` columns: a column past it (in the last
        // group) has e = 0 and v = 0, a +0 term, which leaves the f64 sum (never
        // -0) and the magnitude sums unchanged
        auto add = [&](const float (&e)[4], const float4 (&v)[4], uint32_t g) {
            double a0[4];
#pragma unroll
            for (uint32_t d = 0; d < 4; ++d) a0[d] = a[d];
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                const float p = e[j] * inv;
                const float t[4] = {p * v[j].x, p * v[j].y, p * v[j].z, p * v[j].w};
#pragma unroll
                for (uint32_t d = 0; d < 4; ++d) {
                    a[d] += (double)t[d];
                    as[d] += fabsf(t[d]);
                }
            }
            // the group's sum as the lane sum's growth (within 4 2^-53 A of it)
            const float wg = (float)(ngroups - 1 - g);
#pragma unroll
            for (uint32_t d = 0; d < 4; ++d) ws[d] = __builtin_fmaf(wg, fabsf((float)(a[d] - a0[d])), ws[d]);
        };
#pragma unroll
        for (uint32_t k = 0; k < kPvRegGroups; ++k) {
            const uint32_t g = lane + 64 * k;
            if (g >= ngroups) break;
            add(er[k], vr[k], g);
        }
        for (uint32_t g = lane + 64 * kPvRegGroups; g < ngroups; g += 64) {
            float e[4];
            exp_group(*(const float4*)(srow + 4 * g), 4 * g, count, m, e);
            float4 v[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j)
                v[j] = 4 * g + j < count ? vsrc[4 * g + j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            add(e, v, g);
        }
        // each output: the wave's sums (the four outputs' reductions side by
        // side; every lane gets the same values, so the branches below are
        // wave-uniform), certified or repeated in the reference's column
        // order: the lanes compute kPvRepTerms terms per round into the wave's
        // LDS buffer, and lane 0 adds them in order, sixteen loads ahead of its
        // adds
        double s16[4], C16[4];
        const float ka = (float)pv_coef_a(tl, (double)ngroups);
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            s16[j] = row16_sum_f64(a[j]);
            C16[j] = (double)row16_sum_f(4.0f * ws[j] + ka * as[j]);
        }
        float out[4];
        bool cert[4];
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const double s = rows_sum_f64(s16[j]);
            out[j] = (float)s;
            cert[j] = pv_interval(s, rows_sum_f64(C16[j]));
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            if (!cert[j]) {  // (rare) every order exact?  The smallest |term| of the lane's columns, again
                float mn = INFINITY;
                auto low = [&](const float (&e)[4], const float4 (&v)[4], uint32_t g) {
#pragma unroll
                    for (uint32_t jj = 0; jj < 4; ++jj) {
                        const float t = (e[jj] * inv) * f4_at(v[jj], j);
                        mn = fminf(mn, 4 * g + jj < count ? fabsf(t) : INFINITY);
                    }
                };
#pragma unroll
                for (uint32_t k = 0; k < kPvRegGroups; ++k) {
                    const uint32_t g = lane + 64 * k;
                    if (g < ngroups) low(er[k], vr[k], g);
                }
                for (uint32_t g = lane + 64 * kPvRegGroups; g < ngroups; g += 64) {
                    float e[4];
                    exp_group(*(const float4*)(srow + 4 * g), 4 * g, count, m, e);
                    float4 v[4];
#pragma unroll
                    for (uint32_t jj = 0; jj < 4; ++jj)
                        v[jj] = 4 * g + jj < count ? vsrc[4 * g + jj] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    low(e, v, g);
                }
                const double A = rows_sum_f64((double)row16_sum_f(as[j]));
                const float m16 = row16_min_f(mn);
                cert[j] = f64_sum_exact(A, fminf(fminf(readlane_f(m16, 0), readlane_f(m16, 16)),
                                                 fminf(readlane_f(m16, 32), readlane_f(m16, 48))));
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            if (repeat_all || !cert[j]) {
                const float* vcol = vc + v_cache_index(kvh, hd, d0 + j, 0, max_context);
                double seq = 0.0;
                for (uint32_t base = 0; base < ngroups; base += kPvRepTerms / 4) {
                    const uint32_t g = base + lane;
                    if (g < ngroups) {
                        float e[4];
                        exp_group(*(const float4*)(srow + 4 * g), 4 * g, count, m, e);
#pragma unroll
                        for (uint32_t jj = 0; jj < 4; ++jj) {
                            const uint32_t t = 4 * g + jj;
                            buf[4 * lane + jj] = t < count ? (double)((e[jj] * inv) * vcol[(uint64_t)t * 4]) : 0.0;
                        }
                    }
                    // one wave's LDS operations are performed in order
                    if (lane == 0) {
                        const uint32_t nt = count - 4 * base < kPvRepTerms ? count - 4 * base : kPvRepTerms;
                        uint32_t i = 0;
                        for (; i + 16 <= nt; i += 16) {
                            double x[16];
#pragma unroll
                            for (uint32_t k = 0; k < 16; ++k) x[k] = buf[i + k];
#pragma unroll
                            for (uint32_t k = 0; k < 16; ++k) seq += x[k];
                        }
                        for (; i < nt; ++i) seq += buf[i];
                    }
                    __builtin_amdgcn_wave_barrier();
                }
                out[j] = (float)readlane_d(seq, 0);
            }
        }
        if (lane == 0) {
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j)
                if (!finite(out[j])) report_error(err_word, model_key(layer, kStAttnOut, 0));  // math.rs:494
            *(float4*)(att + (uint64_t)row * hd + d0) = make_float4(out[0], out[1], out[2], out[3]);
        }
    }
}

// RMSNorm of one row (math.rs:214-228) for the step's embedding output: one
// workgroup, the squares summed in f64 by one thread in index order.
// silu(g) * u of [g | u] (llama.rs:367-371), for the inspection of a step
// whose down projection combined them in its quantizer.
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ gu, uint32_t n,
                                                       float* __restrict__ out) {
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        const float g = gu[i];
        out[i] = (g / (1.0f + sse2_exp(0.0f - g))) * gu[n + i];
    }
}

hipError_t LlamaModel::ffn_activation_of(const LlamaLayerDev& L, float* out, hipStream_t s) const {
    const uint32_t F = (uint32_t)d.feed_forward;
    if (L.gu_mode() == 0) return hipMemcpyAsync(out, gu, F * sizeof(float), hipMemcpyDeviceToDevice, s);
    hipLaunchKernelGGL(silu_mul_kernel, dim3((F + 255) / 256), dim3(256), 0, s, gu, F, out);
    return hipGetLastError();
}

hipError_t LlamaModel::ffn_activation(float* out, hipStream_t s) const {
    if (layers.empty()) return hipSuccess;  // no layer: nothing to copy
    return ffn_activation_of(layers.back(), out, s);  // the last layer's
}

__global__ __launch_bounds__(256) void rms_norm_row_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           uint32_t n, float eps, float* __restrict__ out,
                                                           unsigned long long* __restrict__ err_word, uint32_t layer) {
    __shared__ float scale_s;
    if (threadIdx.x == 0) {
        double sum = 0.0;
        for (uint32_t i = 0; i < n; ++i) sum += (double)(x[i] * x[i]);
        const float scale = 1.0f / sqrtf((float)(sum / (double)n) + eps);
        if (!(scale <= 3.402823466e38f) || !(scale > 0.0f))  // math.rs:218-220
            report_error(err_word, model_key(layer, kStAttnNormScale, 0));
        scale_s = scale;
    }
    __syncthreads();
    const float scale = scale_s;
    for (uint32_t i = threadIdx.x; i < n; i += 256) {
        const float v = x[i] * scale * w[i];
        if (!finite(v)) report_error(err_word, model_key(layer, kStAttnNormOut, 0));  // math.rs:227
        out[i] = v;
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

namespace {

uint64_t gguf_row_bytes(uint32_t t, uint64_t cols) {
    switch (t) {
        case kQ8_0: return cols / 32 * 34;
        case kQ2_K: return cols / 256 * 84;
        case kQ3_K: return cols / 256 * 110;
        case kQ4_K: return cols / 256 * 144;
        case kQ5_K: return cols / 256 * 176;
        case kQ6_K: return cols / 256 * 210;
        default: return 0;
    }
}

hipError_t upload_tiled(uint32_t t, const void* gguf, uint64_t rows, uint64_t cols, bool on_device, uint8_t* dst,
                        void* staging, hipStream_t s) {
    const uint8_t* src = (const uint8_t*)gguf;
    if (!on_device) {
        const uint64_t len = rows * gguf_row_bytes(t, cols);
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

}  // namespace

LlamaModel::~LlamaModel() {
    if (device >= 0) (void)hipSetDevice(device);
    (void)hipDeviceSynchronize();
    for (LlamaLayerDev& l : layers)
        for (void* p : {(void*)l.wqkv, (void*)l.wo, (void*)l.wgu, (void*)l.wdown, (void*)l.attn_norm,
                        (void*)l.ffn_norm})
            if (p) (void)hipFree(p);
    for (void* p : {(void*)out_w, (void*)out_norm, (void*)emb, (void*)k_cache, (void*)v_cache, (void*)rope_tab,
                    (void*)qkv, (void*)scores, (void*)att, (void*)mid, (void*)gu, am_state,
                    (void*)logits_buf, (void*)cmax})
        if (p) (void)hipFree(p);
}

hipError_t LlamaModel::create(const LlamaDims& dims, const LlamaHostTensors& t, hipStream_t s) {
    // RLQ_ATTN_REPEAT_ALL=1: every QK dot and softmax total repeated in the
    // reference's order, as when its certificate fails (tests compare the two)
    const char* rep = getenv("RLQ_ATTN_REPEAT_ALL");
    repeat_all = rep && rep[0] == '1';
    d = dims;
    const uint64_t W = d.width, F = d.feed_forward, hd = W / d.heads, kvw = d.kv_heads * hd;
    // host memory: the layer records and the RoPE table (max_context x hd
    // floats); a failed reservation is an allocation error, not an abort
    std::vector<float> tab;
    try {
        layers.assign(d.n_layers, LlamaLayerDev{});
        tab.resize(d.max_context * hd);
    } catch (const std::bad_alloc&) {
        return hipErrorOutOfMemory;
    } catch (const std::length_error&) {
        return hipErrorOutOfMemory;
    }
    // the rope table: the reference's theta sequence and libm sin/cos per position
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
    // the attention workgroups' LDS grows with the group size and head width
    // (the caller checked that it fits next to the kernels' few static bytes);
    // the limits only grow, so models of other shapes in the process keep working
    static LdsLimit pv_limit, scores_limit;
    const uint32_t G = (uint32_t)(d.heads / d.kv_heads);
    hipError_t e = pv_limit.raise((const void*)attn_pv_kernel, attn_pv_lds_bytes(G));
    if (e == hipSuccess) e = scores_limit.raise((const void*)attn_scores_kernel, attn_scores_lds(G, (uint32_t)hd));
    if (e == hipSuccess) e = hipMalloc((void**)&rope_tab, tab.size() * sizeof(float));
    if (e == hipSuccess) e = hipMemcpy(rope_tab, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice);
    uint64_t cache_bytes = 0;  // per cache: n_layers x max_context x kv_width floats
    if (__builtin_mul_overflow(d.max_context * kvw, (uint64_t)sizeof(float), &cache_bytes) ||
        __builtin_mul_overflow(cache_bytes, d.n_layers, &cache_bytes))
        return hipErrorOutOfMemory;
    if (e == hipSuccess) e = hipMalloc((void**)&k_cache, cache_bytes);
    if (e == hipSuccess) e = hipMalloc((void**)&v_cache, cache_bytes);
    if (e == hipSuccess) e = hipMalloc((void**)&qkv, (W + 2 * kvw) * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&scores, d.heads * row_len * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&cmax, d.heads * nchunks * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&att, W * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&mid, W * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&gu, 2 * F * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&am_state, kArgmaxStateBytes);
    if (e == hipSuccess) e = launch_fill_u64((unsigned long long*)am_state, 1, 0ull, s);  // the arrival counter
    if (e == hipSuccess) e = hipMalloc((void**)&logits_buf, d.vocab * sizeof(float));
    if (e != hipSuccess) return e;
    // staging for host GGUF bytes: the largest tensor; the gate/up stage of
    // the interleaving copy
    uint64_t big = gguf_row_bytes(d.output_type, W) * d.vocab, stage_gu = 0;
    for (uint64_t l = 0; l < d.n_layers; ++l) {
        const uint32_t* ty = t.layers[l].types;
        for (int k = 0; k < 7; ++k) {
            const uint64_t rows = k < 4 ? (k == 1 || k == 2 ? kvw : W) : (k == 6 ? W : F), cols = k == 6 ? F : W;
            const uint64_t b = gguf_row_bytes(ty[k], cols) * rows;
            big = big > b ? big : b;
        }
        if (ty[4] == ty[5] && (ty[4] == kQ4_K || ty[4] == kQ5_K)) {
            const uint64_t b = 2 * layout_bytes(ty[4], F, W);
            stage_gu = stage_gu > b ? stage_gu : b;
        }
    }
    void* staging = nullptr;
    if (!t.on_device) {
        e = hipMalloc(&staging, big);
        if (e != hipSuccess) return e;
    }
    uint8_t* gu_stage = nullptr;
    if (e == hipSuccess && stage_gu) e = hipMalloc((void**)&gu_stage, stage_gu);
    auto tiled = [&](uint32_t ty, const void* src, uint64_t rows, uint64_t cols, uint8_t* dst) {
        return upload_tiled(ty, src, rows, cols, t.on_device, dst, staging, s);
    };
    for (uint64_t l = 0; l < d.n_layers && e == hipSuccess; ++l) {
        const LlamaHostLayer& hl = t.layers[l];
        LlamaLayerDev& L = layers[l];
        L.tq = hl.types[0], L.tk = hl.types[1], L.tv = hl.types[2], L.to = hl.types[3];
        L.tg = hl.types[4], L.tu = hl.types[5], L.td = hl.types[6];
        // Q, K, V back to back in one buffer: rows are whole tiles, so with one
        // type the three are one tiled matrix of W + 2 kvw rows
        const uint64_t bq = layout_bytes(L.tq, W, W), bk = layout_bytes(L.tk, kvw, W), bv = layout_bytes(L.tv, kvw, W);
        L.off_k = bq, L.off_v = bq + bk;
        e = hipMalloc((void**)&L.wqkv, bq + bk + bv);
        if (e == hipSuccess) e = tiled(L.tq, hl.query, W, W, L.wqkv);
        if (e == hipSuccess) e = tiled(L.tk, hl.key, kvw, W, L.wqkv + L.off_k);
        if (e == hipSuccess) e = tiled(L.tv, hl.value, kvw, W, L.wqkv + L.off_v);
        if (e == hipSuccess) e = hipMalloc((void**)&L.wo, layout_bytes(L.to, W, W));
        if (e == hipSuccess) e = tiled(L.to, hl.attention_output, W, W, L.wo);
        // gu_mode 0 (Q4_K / Q5_K): gate and up tiles interleaved (tile 2i =
        // gate tile i, 2i + 1 = up tile i), so one workgroup holds both halves
        // of silu(gate) * up; otherwise [gate; up], whose product [g | u] the
        // down projection's quantizer combines
        const uint64_t bg = layout_bytes(L.tg, F, W), bu = layout_bytes(L.tu, F, W);
        L.off_up = bg;
        if (e == hipSuccess) e = hipMalloc((void**)&L.wgu, bg + bu);
        if (e == hipSuccess && L.gu_mode() != 0) {
            e = tiled(L.tg, hl.gate, F, W, L.wgu);
            if (e == hipSuccess) e = tiled(L.tu, hl.up, F, W, L.wgu + L.off_up);
        } else if (e == hipSuccess) {
            e = tiled(L.tg, hl.gate, F, W, gu_stage);
            if (e == hipSuccess) e = tiled(L.tu, hl.up, F, W, gu_stage + bg);
        }
        if (e == hipSuccess && L.gu_mode() == 0) {
            const uint64_t tb = bg / (F / kTileRows);  // bytes of one tile
            e = hipMemcpy2DAsync(L.wgu, 2 * tb, gu_stage, tb, tb, F / kTileRows, hipMemcpyDeviceToDevice, s);
            if (e == hipSuccess)
                e = hipMemcpy2DAsync(L.wgu + tb, 2 * tb, gu_stage + bg, tb, tb, F / kTileRows, hipMemcpyDeviceToDevice,
                                     s);
            if (e == hipSuccess) e = hipStreamSynchronize(s);  // the stage is reused by the next layer
        }
        if (e == hipSuccess) e = hipMalloc((void**)&L.wdown, layout_bytes(L.td, W, F));
        if (e == hipSuccess) e = tiled(L.td, hl.down, W, F, L.wdown);
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
    if (gu_stage) (void)hipFree(gu_stage);
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
    const size_t lds_scores = attn_scores_lds((uint32_t)(H / KVH), (uint32_t)hd);
    const size_t lds_pv = attn_pv_lds_bytes((uint32_t)(H / KVH));
    const uint32_t cstride = (uint32_t)((d.max_context + kAttnChunk - 1) / kAttnChunk);
    hipError_t e = hipSuccess;
    for (uint64_t l = 0; l < d.n_layers && e == hipSuccess; ++l) {
        const LlamaLayerDev& L = layers[l];
        float* kc = k_cache + l * d.max_context * kvw;
        float* vc = v_cache + l * d.max_context * kvw;
        const uint32_t lay = (uint32_t)l;
        MvExtra norm1;
        norm1.xform = 1, norm1.eps = d.rms_epsilon, norm1.norm_w = L.attn_norm;
        norm1.chk = mv_chk(kStAttnNormScale, kStAttnNormOut, kStQkvQuant, kStQkvOut, 0), norm1.chk_layer = lay;
        if (L.fused_qkv()) {
            e = launch_matvec_ex(L.tq, L.wqkv, W + 2 * kvw, W, hidden, nullptr, 1, qkv, W + 2 * kvw, nullptr, err_word,
                                 nullptr, nullptr, norm1, s);
        } else {  // one launch per type (each quantizes the same normalized input); two
                  // neighbours of one type are one matrix (a Q4_K_M layer's Q and K:
                  // 1.951 ms per token against 2.030 with three launches)
            const bool qk = L.tq == L.tk, kv = !qk && L.tk == L.tv;
            e = launch_matvec_ex(L.tq, L.wqkv, qk ? W + kvw : W, W, hidden, nullptr, 1, qkv, qk ? W + kvw : W, nullptr,
                                 err_word, nullptr, nullptr, norm1, s);
            if (e == hipSuccess && !qk)
                e = launch_matvec_ex(L.tk, L.wqkv + L.off_k, kv ? 2 * kvw : kvw, W, hidden, nullptr, 1, qkv + W,
                                     kv ? 2 * kvw : kvw, nullptr, err_word, nullptr, nullptr, norm1, s);
            if (e == hipSuccess && !kv)
                e = launch_matvec_ex(L.tv, L.wqkv + L.off_v, kvw, W, hidden, nullptr, 1, qkv + W + kvw, kvw, nullptr,
                                     err_word, nullptr, nullptr, norm1, s);
        }
        if (e != hipSuccess) break;
        hipLaunchKernelGGL(attn_scores_kernel, dim3(nchunks, (uint32_t)KVH), dim3(kAttnThreads), lds_scores, s, qkv,
                           tab, kc, vc, (uint32_t)d.max_context, (uint32_t)fresh, (uint32_t)H, (uint32_t)KVH,
                           (uint32_t)hd, scale, scores, (uint32_t)row_stride, cmax, cstride, err_word, lay,
                           repeat_all ? 1u : 0u);
        hipLaunchKernelGGL(attn_pv_kernel, dim3((uint32_t)(hd / kPvDims), (uint32_t)KVH),
                           dim3(64 * pv_waves((uint32_t)(H / KVH))), lds_pv, s,
                           scores, cmax, cstride, nchunks, vc, (uint32_t)d.max_context, (uint32_t)count, (uint32_t)H,
                           (uint32_t)KVH, (uint32_t)hd, (uint32_t)row_stride, att, err_word, lay,
                           repeat_all ? 1u : 0u);
        e = hipGetLastError();
        if (e != hipSuccess) break;
        // the residual stream after attention goes to `mid` (the FFN norm's
        // input); the down projection adds its output to it into hidden
        MvExtra res;
        res.resid = hidden;
        res.chk = mv_chk(0, kStOIn, kStOQuant, kStOOut, 0), res.chk_layer = lay;
        e = launch_matvec_ex(L.to, L.wo, W, W, att, nullptr, 1, mid, W, nullptr, err_word, nullptr, nullptr, res, s);
        if (e != hipSuccess) break;
        // gate/up with the FFN norm: the fused epilogue leaves silu(gate) * up
        // in gu, the plain one [gate | up] for the down projection to combine
        MvExtra norm2;
        norm2.xform = 1, norm2.eps = d.rms_epsilon, norm2.norm_w = L.ffn_norm, norm2.epilogue = L.gu_mode() == 0 ? 1 : 0;
        norm2.chk = mv_chk(kStFfnNormScale, kStFfnNormOut, kStGuQuant, kStGuOut, 0), norm2.chk_layer = lay;
        if (L.gu_mode() != 2) {
            e = launch_matvec_ex(L.tg, L.wgu, 2 * F, W, mid, nullptr, 1, gu, 2 * F, nullptr, err_word, nullptr,
                                 nullptr, norm2, s);
        } else {
            e = launch_matvec_ex(L.tg, L.wgu, F, W, mid, nullptr, 1, gu, F, nullptr, err_word, nullptr, nullptr,
                                 norm2, s);
            if (e == hipSuccess)
                e = launch_matvec_ex(L.tu, L.wgu + L.off_up, F, W, mid, nullptr, 1, gu + F, F, nullptr, err_word,
                                     nullptr, nullptr, norm2, s);
        }
        if (e != hipSuccess) break;
        MvExtra down;
        down.resid = mid;
        down.chk = mv_chk(0, kStDownIn, kStDownQuant, kStDownOut, kStLayerOut), down.chk_layer = lay;
        if (L.gu_mode() != 0) down.xform = 2;
        e = launch_matvec_ex(L.td, L.wdown, W, F, gu, nullptr, 1, hidden, W, nullptr, err_word, nullptr, nullptr, down,
                             s);
        if (e == hipSuccess && trace) {  // the checker's copy of every layer's parts
            float* tr = trace + l * trace_stride();
            e = hipMemcpyAsync(tr, qkv, (W + 2 * kvw) * sizeof(float), hipMemcpyDeviceToDevice, s);
            tr += W + 2 * kvw;
            if (e == hipSuccess) e = hipMemcpyAsync(tr, att, W * sizeof(float), hipMemcpyDeviceToDevice, s);
            if (e == hipSuccess) e = hipMemcpyAsync(tr + W, mid, W * sizeof(float), hipMemcpyDeviceToDevice, s);
            if (e == hipSuccess) e = ffn_activation_of(L, tr + 2 * W, s);
            if (e == hipSuccess)
                e = hipMemcpyAsync(tr + 2 * W + F, hidden, W * sizeof(float), hipMemcpyDeviceToDevice, s);
        }
    }
    if (e != hipSuccess) return e;
    if (embedding_out) {
        hipLaunchKernelGGL(rms_norm_row_kernel, dim3(1), dim3(256), 0, s, hidden, out_norm, (uint32_t)W,
                           d.rms_epsilon, embedding_out, err_word, (uint32_t)d.n_layers);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (logits || argmax) {
        MvExtra norm3;
        norm3.xform = 1, norm3.eps = d.rms_epsilon, norm3.norm_w = out_norm;
        // finish_hidden (llama.rs:381-392): checks numbered as a layer's first
        // four, with layer = n_layers
        norm3.chk = mv_chk(kStAttnNormScale, kStAttnNormOut, kStQkvQuant, kStQkvOut, 0);
        norm3.chk_layer = (uint32_t)d.n_layers;
        // logits land in the caller's buffer, or in the model's own when only
        // the argmax is wanted; the greedy token is finished inside the launch
        float* y = logits ? logits : logits_buf;
        const MvArgmax am = argmax_state(am_state, argmax);
        e = launch_matvec_ex(d.output_type, out_w, d.vocab, W, hidden, nullptr, 1, y, d.vocab, argmax ? &am : nullptr,
                             err_word, nullptr, nullptr, norm3, s);
        if (e != hipSuccess) return e;
    }
    ++n_cached;
    return hipSuccess;
}

}  // namespace rlq
