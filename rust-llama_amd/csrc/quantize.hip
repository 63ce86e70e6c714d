// quantize.hip - gfx950 quantizers, encoders, decoders and layout repack.
//
// Reference arithmetic (paths relative to the rust-llama repository):
//   Q8_K activation  crates/quant/src/activation.rs:4-51
//   Q8_0             crates/quant/src/encode.rs:115-126 (scale), 151-192 (block),
//                    preflight encode.rs:79-90
//   K encoders       crates/quant/src/encode_k.rs:37-561 (Q2_K 292-355,
//                    Q3_K 138-185 and 357-409, Q4_K / Q5_K 410-507, Q6_K
//                    70-137 and 508-561, make_qkx2_quants 189-279)
//   decoders         crates/quant/src/decode.rs:17-49, 205-258
// Compiled with -ffp-contract=off, so every f32 expression below rounds step
// by step as the Rust source does; division and sqrt are correctly rounded
// (HIP's default for f32).
#include "rlq_device.hpp"
#include "rlq_internal.hpp"
#include "rlq_layout.hpp"

namespace rlq {

static inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

size_t act_planes_bytes(uint32_t t, uint64_t cols, uint64_t batch) {
    const uint64_t bs = t == kQ8_K ? 256 : 32;
    size_t n = align256(cols * batch) + align256(cols / bs * batch * 4) + align256(cols / bs * batch);
    if (t == kQ8_K) n += align256(cols / 16 * batch * 2);
    return n;
}

ActPlanes act_planes_carve(void* base, uint32_t t, uint64_t cols, uint64_t batch) {
    const uint64_t bs = t == kQ8_K ? 256 : 32;
    uint8_t* p = (uint8_t*)base;
    ActPlanes a;
    a.q = (int8_t*)p;
    p += align256(cols * batch);
    a.d = (float*)p;
    p += align256(cols / bs * batch * 4);
    a.bad = p;
    p += align256(cols / bs * batch);
    a.bsum = t == kQ8_K ? (int16_t*)p : nullptr;
    return a;
}

// ---------------------------------------------------------------------------
// Q8_K activation quantizer: one wave per 256-element block, 4 values a lane.
// grid = (cols / 256, batch)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void quantize_q8k_kernel(const float* __restrict__ x, uint64_t cols,
                                                          ActPlanes planes, uint8_t* __restrict__ gguf,
                                                          unsigned long long* err_word) {
    const uint32_t lane = threadIdx.x;
    const uint64_t blk = blockIdx.x, col = blockIdx.y, nb = cols / 256;
    const float4 v4 = *(const float4*)(x + col * cols + blk * 256 + lane * 4);
    const float e[4] = {v4.x, v4.y, v4.z, v4.w};

    // NonFiniteInput: first index in this block (encode.rs:70-74).
    uint32_t bad = 0xffffffffu;
#pragma unroll
    for (int k = 3; k >= 0; --k)
        if (!finite(e[k])) bad = lane * 4 + k;
    const uint32_t first_bad = wave_min_u32(bad);
    bool invalid = first_bad != 0xffffffffu;
    if (invalid && lane == 0) report_error(err_word, error_key(col, kKindNonFinite, blk * 256 + first_bad));

    // inverse_scale (activation.rs:4-17): the FIRST value of largest |x|.
    float a = 0.0f, av = 0.0f;
    uint32_t ai = 0xffffffffu;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (fabsf(e[k]) > a) {
            a = fabsf(e[k]);
            av = e[k];
            ai = lane * 4 + k;
        }
    const float amax = wave_max(invalid ? 0.0f : a);
    const uint32_t idx = wave_min_u32(a == amax ? ai : 0xffffffffu);
    float inverse = 0.0f;
    if (amax != 0.0f && !invalid) {
        const float maximum = __shfl(av, (int)(idx >> 2), 64);
        inverse = -127.0f / maximum;
    }
    // preflight_q8k (activation.rs:20-28)
    if (!invalid && (!finite(inverse) || (inverse != 0.0f && !finite(1.0f / inverse)))) {
        invalid = true;
        if (lane == 0) report_error(err_word, error_key(col, kKindScale, blk));
    }

    // encode_q8k (activation.rs:30-51)
    uint32_t packed = 0;
    int32_t s = 0;
    if (inverse != 0.0f && !invalid) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            int32_t q = (int32_t)__builtin_rintf(inverse * e[k]);
            q = q < 127 ? q : 127;
            packed |= ((uint32_t)q & 0xffu) << (8 * k);
            s += (int8_t)q;
        }
    }
    s += dpp_i<kQuadXor1>(s);
    s += dpp_i<kQuadXor2>(s);
    const float d = (inverse != 0.0f && !invalid) ? 1.0f / inverse : 0.0f;

    if (planes.q) {
        *(uint32_t*)(planes.q + col * cols + blk * 256 + lane * 4) = packed;
        if (lane == 0) {
            planes.d[col * nb + blk] = d;
            planes.bad[col * nb + blk] = invalid ? 1 : 0;
        }
        if ((lane & 3) == 0) planes.bsum[col * (cols / 16) + blk * 16 + lane / 4] = (int16_t)s;
    }
    if (gguf) {
        uint8_t* o = gguf + (col * nb + blk) * 292;
        if (lane == 0) *(float*)o = d;
        *(uint32_t*)(o + 4 + lane * 4) = packed;
        if ((lane & 3) == 0) *(int16_t*)(o + 260 + 2 * (lane / 4)) = (int16_t)s;
    }
}

hipError_t launch_quantize_q8k(const float* x, uint64_t cols, uint64_t batch, const ActPlanes* planes,
                               uint8_t* gguf, unsigned long long* err_word, hipStream_t s) {
    ActPlanes p = planes ? *planes : ActPlanes{nullptr, nullptr, nullptr, nullptr};
    dim3 grid((unsigned)(cols / 256), (unsigned)batch);
    hipLaunchKernelGGL(quantize_q8k_kernel, grid, dim3(64), 0, s, x, cols, p, gguf, err_word);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Q8_0 quantizer (activations and weights): 8 lanes per 32-block, 4 values a
// lane, 8 blocks per wave.  grid = (ceil(cols/32 / 8), batch)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void quantize_q8_0_kernel(const float* __restrict__ x, uint64_t cols,
                                                           ActPlanes planes, uint8_t* __restrict__ gguf,
                                                           unsigned long long* err_word) {
    const uint32_t lane = threadIdx.x, sub = lane & 7;
    const uint64_t nb = cols / 32, col = blockIdx.y;
    const uint64_t blk = (uint64_t)blockIdx.x * 8 + (lane >> 3);
    const bool active = blk < nb;
    float e[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (active) {
        const float4 v4 = *(const float4*)(x + col * cols + blk * 32 + sub * 4);
        e[0] = v4.x, e[1] = v4.y, e[2] = v4.z, e[3] = v4.w;
    }
    uint32_t bad = 0xffffffffu;
#pragma unroll
    for (int k = 3; k >= 0; --k)
        if (!finite(e[k])) bad = (uint32_t)(blk * 32 + sub * 4 + k);
    // first non-finite of the 8-lane group
    for (int m = 1; m < 8; m <<= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)bad, m, 8);
        bad = o < bad ? o : bad;
    }
    bool invalid = bad != 0xffffffffu;
    if (invalid && sub == 0 && active) report_error(err_word, error_key(col, kKindNonFinite, bad));

    // scales(): amax = fold(0, max(a, |v|)); d = amax / 127 (encode.rs:123-126)
    float amax = fmaxf(fmaxf(fabsf(e[0]), fabsf(e[1])), fmaxf(fabsf(e[2]), fabsf(e[3])));
    for (int m = 1; m < 8; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 8));
    if (invalid) amax = 0.0f;
    const float d = amax / 127.0f;
    const uint32_t dh = float_to_half_bits(d);
    // preflight (encode.rs:80-90); m is 0 for Q8_0
    if (!invalid && (!finite(d) || (d != 0.0f && !finite(1.0f / d)) || (dh & 0x7c00u) == 0x7c00u)) {
        invalid = true;
        if (sub == 0 && active) report_error(err_word, error_key(col, kKindScale, blk));
    }
    const float inv = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t packed = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        // `(x * inv).round() as i8`: half away from zero, saturating
        float r = __builtin_roundf(e[k] * inv);
        r = r > 127.0f ? 127.0f : (r < -128.0f ? -128.0f : r);
        packed |= ((uint32_t)(int32_t)r & 0xffu) << (8 * k);
    }
    if (!active) return;
    if (planes.q) {
        *(uint32_t*)(planes.q + col * cols + blk * 32 + sub * 4) = packed;
        if (sub == 0) {
            planes.d[col * nb + blk] = half_bits_to_float_exact(dh);
            planes.bad[col * nb + blk] = invalid ? 1 : 0;
        }
    }
    if (gguf) {
        uint8_t* o = gguf + (col * nb + blk) * 34;
        if (sub == 0) {
            o[0] = (uint8_t)(dh & 0xff);
            o[1] = (uint8_t)(dh >> 8);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) o[2 + sub * 4 + k] = (uint8_t)(packed >> (8 * k));
    }
}

hipError_t launch_quantize_q8_0(const float* x, uint64_t cols, uint64_t batch, const ActPlanes* planes,
                                uint8_t* gguf, unsigned long long* err_word, hipStream_t s) {
    ActPlanes p = planes ? *planes : ActPlanes{nullptr, nullptr, nullptr, nullptr};
    const uint64_t nb = cols / 32;
    dim3 grid((unsigned)((nb + 7) / 8), (unsigned)batch);
    hipLaunchKernelGGL(quantize_q8_0_kernel, grid, dim3(64), 0, s, x, cols, p, gguf, err_word);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GGUF activation bytes -> planes (no validation: dot_packed takes the packed
// activation as given, matvec.rs:90-103).  One thread per 4 quantized values.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void act_from_gguf_kernel(uint32_t t, const uint8_t* __restrict__ src, uint64_t cols,
                                                            uint64_t batch, ActPlanes planes) {
    const uint64_t bs = t == kQ8_K ? 256 : 32, ts = t == kQ8_K ? 292 : 34, qoff = t == kQ8_K ? 4 : 2;
    const uint64_t units = batch * cols / 4;
    for (uint64_t u = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units;
         u += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t e = u * 4, blk = e / bs, within = e % bs;  // blk counts over all columns
        const uint8_t* b = src + blk * ts;
        uint32_t w = 0;
        for (int k = 0; k < 4; ++k) w |= (uint32_t)b[qoff + within + k] << (8 * k);
        *(uint32_t*)(planes.q + e) = w;
        if (within == 0) {
            float d;
            if (t == kQ8_K) __builtin_memcpy(&d, b, 4);
            else d = half_bits_to_float_exact((uint32_t)b[0] | ((uint32_t)b[1] << 8));
            planes.d[blk] = d;
            planes.bad[blk] = 0;
        }
        if (t == kQ8_K && (within % 16) == 0)
            planes.bsum[e / 16] = (int16_t)((uint32_t)b[260 + 2 * (within / 16)] |
                                            ((uint32_t)b[261 + 2 * (within / 16)] << 8));
    }
}

hipError_t launch_act_from_gguf(uint32_t t, const uint8_t* gguf, uint64_t cols, uint64_t batch,
                                const ActPlanes* planes, hipStream_t s) {
    const uint64_t units = batch * cols / 4, grid = (units + 255) / 256;
    hipLaunchKernelGGL(act_from_gguf_kernel, dim3((unsigned)(grid ? (grid < 65536 ? grid : 65536) : 1)), dim3(256),
                       0, s, t, gguf, cols, batch, *planes);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Finite scan (the encoders' first check, encode_k.rs:13-17)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void finite_scan_kernel(const float* __restrict__ x, uint64_t n,
                                                          unsigned long long* err_word) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        if (!finite(x[i])) report_error(err_word, error_key(0, kKindNonFinite, i));
}

hipError_t launch_finite_scan(const float* x, uint64_t n, unsigned long long* err_word, hipStream_t s) {
    const uint64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(finite_scan_kernel, dim3((unsigned)(blocks < 4096 ? (blocks ? blocks : 1) : 4096)),
                       dim3(256), 0, s, x, n, err_word);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// K-quant weight encoders
// ---------------------------------------------------------------------------

// encode_k.rs:37-42: false on failure
__device__ __forceinline__ bool nearest(float x, int32_t& out) {
    if (!finite(x) || fabsf(x) > 4194303.0f) return false;
    out = (int32_t)__builtin_rintf(x);
    return true;
}
__device__ __forceinline__ int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

// make_qkx2_quants restatement, encode_k.rs:189-279; MAD selects the
// weighted absolute error (Q2_K) over the weighted squared error.
// Returns false on the reference's Err(()).
template <bool MAD>
__device__ __forceinline__ float fit_error(float difference) {
    return MAD ? fabsf(difference) : difference * difference;
}
template <int N, bool MAD>
__device__ bool make_affine2(const float (&x)[N], int32_t nmax, const float (&weights)[N], int32_t (&levels)[N],
                             float rmin, float rdelta, int steps, float& scale_out, float& min_out) {
    float minimum = x[0], maximum = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
#pragma unroll
    for (int i = 1; i < N; ++i) {
        if (x[i] < minimum) minimum = x[i];
        if (x[i] > maximum) maximum = x[i];
        sum_w += weights[i];
        sum_x += weights[i] * x[i];
    }
    if (!finite(sum_w) || !finite(sum_x)) return false;
    if (minimum > 0.0f) minimum = 0.0f;
    if (maximum == minimum) {
#pragma unroll
        for (int i = 0; i < N; ++i) levels[i] = 0;
        scale_out = 0.0f;
        min_out = -minimum;
        return true;
    }
    float inverse = (float)nmax / (maximum - minimum);
    float scale = 1.0f / inverse;
    float best_error = 0.0f;
    bool ok = true;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        int32_t l = 0;
        ok &= nearest(inverse * (x[i] - minimum), l);
        levels[i] = clampi(l, 0, nmax);
        const float difference = scale * (float)levels[i] + minimum - x[i];
        best_error += weights[i] * fit_error<MAD>(difference);
    }
    if (!ok) return false;
    for (int step = 0; step <= steps; ++step) {
        inverse = (rmin + rdelta * (float)step + (float)nmax) / (maximum - minimum);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        int32_t candidate[N];
#pragma unroll
        for (int i = 0; i < N; ++i) {
            int32_t l = 0;
            ok &= nearest(inverse * (x[i] - minimum), l);
            l = clampi(l, 0, nmax);
            candidate[i] = l;
            const float w = weights[i];
            sum_l += w * (float)l;
            sum_l2 += w * (float)l * (float)l;
            sum_xl += w * (float)l * x[i];
        }
        if (!ok) return false;
        const float determinant = sum_w * sum_l2 - sum_l * sum_l;
        if (determinant > 0.0f) {
            float candidate_scale = (sum_w * sum_xl - sum_x * sum_l) / determinant;
            float candidate_minimum = (sum_l2 * sum_x - sum_l * sum_xl) / determinant;
            if (candidate_minimum > 0.0f) {
                candidate_minimum = 0.0f;
                candidate_scale = sum_xl / sum_l2;
            }
            float error = 0.0f;
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const float difference = candidate_scale * (float)candidate[i] + candidate_minimum - x[i];
                error += weights[i] * fit_error<MAD>(difference);
            }
            if (error < best_error) {
#pragma unroll
                for (int i = 0; i < N; ++i) levels[i] = candidate[i];
                best_error = error;
                scale = candidate_scale;
                minimum = candidate_minimum;
            }
        }
    }
    if (!finite(scale) || !finite(-minimum)) return false;
    scale_out = scale;
    min_out = -minimum;
    return true;
}

// Q4_K / Q5_K (encode_k.rs:430-507): 8 lanes per super-block (one 32-value
// sub-block each), 8 blocks a WG.  Q5_K: levels 0..31 (rmin -0.5, 15 steps),
// the fifth bits in bytes 16..47 and the nibbles from byte 48 (176 bytes).
template <bool FIVE>
__global__ __launch_bounds__(64) void encode_q45k_kernel(const float* __restrict__ x, uint64_t nblocks,
                                                         uint8_t* __restrict__ out, unsigned long long* err_word) {
    constexpr int32_t kNmax = FIVE ? 31 : 15;
    constexpr uint32_t kBytes = FIVE ? 176 : 144, kQs = FIVE ? 48 : 16;
    __shared__ uint8_t lv[8][256];
    const uint32_t lane = threadIdx.x, gb = lane >> 3, sub = lane & 7;
    const uint64_t blk = (uint64_t)blockIdx.x * 8 + gb;
    const bool active = blk < nblocks;
    float xs[32];
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        float4 v = active ? *(const float4*)(x + blk * 256 + sub * 32 + i) : make_float4(0, 0, 0, 0);
        xs[i] = v.x, xs[i + 1] = v.y, xs[i + 2] = v.z, xs[i + 3] = v.w;
    }
    bool ok = true;
    // encode_k.rs:437-451
    float square_sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) square_sum = square_sum + xs[i] * xs[i];
    const float average = sqrtf(square_sum / 32.0f);
    ok &= finite(average);
    float weights[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) weights[i] = average + fabsf(xs[i]);
    int32_t levels[32];
    float scale = 0.0f, minimum = 0.0f;
    if (ok) ok &= make_affine2<32, false>(xs, kNmax, weights, levels, FIVE ? -0.5f : -1.0f, 0.1f, FIVE ? 15 : 20, scale, minimum);

    // maximum_scale / maximum_minimum: strict `>` from +0.0 (encode_k.rs:454-459)
    float ms = scale > 0.0f ? scale : 0.0f, mm = minimum > 0.0f ? minimum : 0.0f;
    for (int m = 1; m < 8; m <<= 1) {
        const float os = __shfl_xor(ms, m, 8), om = __shfl_xor(mm, m, 8);
        ms = os > ms ? os : ms;
        mm = om > mm ? om : mm;
    }
    const float inverse_scale = ms > 0.0f ? 63.0f / ms : 0.0f;
    const float inverse_minimum = mm > 0.0f ? 63.0f / mm : 0.0f;
    int32_t qs = 0, qm = 0;
    ok &= nearest(inverse_scale * scale, qs);
    ok &= nearest(inverse_minimum * minimum, qm);
    qs = qs < 63 ? qs : 63;
    qm = qm < 63 ? qm : 63;
    // pack_scale_min for sub 0..7 in order (encode_k.rs:410-419), same in every lane
    uint8_t packed[12];
#pragma unroll
    for (int i = 0; i < 12; ++i) packed[i] = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint8_t s8 = (uint8_t)__shfl(qs, (int)((lane & ~7u) + k), 64);
        const uint8_t m8 = (uint8_t)__shfl(qm, (int)((lane & ~7u) + k), 64);
        if (k < 4) {
            packed[k] = s8;
            packed[k + 4] = m8;
        } else {
            packed[k + 4] = (uint8_t)((s8 & 15) | ((m8 & 15) << 4));
            packed[k - 4] |= (uint8_t)((s8 >> 4) << 6);
            packed[k] |= (uint8_t)((m8 >> 4) << 6);
        }
    }
    const uint32_t dh = float_to_half_bits(ms / 63.0f);
    const uint32_t mh = float_to_half_bits(mm / 63.0f);
    ok &= (dh & 0x7c00u) != 0x7c00u;
    ok &= (mh & 0x7c00u) != 0x7c00u;
    // unpack_scale_min for this sub-block (encode_k.rs:420-429), re-quantize
    uint8_t sc, mn;
    if (sub < 4) {
        sc = packed[sub] & 63;
        mn = packed[sub + 4] & 63;
    } else {
        sc = (uint8_t)((packed[sub + 4] & 15) | ((packed[sub - 4] >> 6) << 4));
        mn = (uint8_t)((packed[sub + 4] >> 4) | ((packed[sub] >> 6) << 4));
    }
    const float scale2 = half_bits_to_float_exact(dh) * (float)sc;
    if (scale2 != 0.0f) {
        const float minimum2 = half_bits_to_float_exact(mh) * (float)mn;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            int32_t l = 0;
            ok &= nearest((xs[i] + minimum2) / scale2, l);
            levels[i] = clampi(l, 0, kNmax);
        }
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) lv[gb][sub * 32 + i] = (uint8_t)levels[i];
    // block-wide failure
    int okw = ok ? 1 : 0;
    for (int m = 1; m < 8; m <<= 1) okw &= __shfl_xor(okw, m, 8);
    __syncthreads();
    if (!active) return;
    if (!okw && sub == 0) report_error(err_word, error_key(0, kKindScale, blk));
    uint8_t* o = out + blk * kBytes;
    if (sub == 0) {
        o[0] = (uint8_t)(dh & 0xff);
        o[1] = (uint8_t)(dh >> 8);
        o[2] = (uint8_t)(mh & 0xff);
        o[3] = (uint8_t)(mh >> 8);
#pragma unroll
        for (int i = 0; i < 12; ++i) o[4 + i] = packed[i];
    }
    // qs bytes sub*16 .. +15 (encode_k.rs:491-505)
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const int byte = sub * 16 + k, group = byte / 32, j = byte % 32;
        const uint8_t low = lv[gb][group * 64 + j], high = lv[gb][group * 64 + j + 32];
        o[kQs + byte] = (uint8_t)((low & 15) | ((high & 15) << 4));
    }
    if constexpr (FIVE) {
        // fifth-bit bytes sub*4 .. +3: bit 2g of byte j from level 64g + j,
        // bit 2g + 1 from level 64g + j + 32
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int j = sub * 4 + k;
            uint32_t h = 0;
#pragma unroll
            for (int g = 0; g < 4; ++g)
                h |= (lv[gb][g * 64 + j] > 15 ? 1u : 0u) << (2 * g) | (lv[gb][g * 64 + j + 32] > 15 ? 2u : 0u) << (2 * g);
            o[16 + j] = (uint8_t)h;
        }
    }
}

// make_qx with rmse = 1 and no importance weights, encode_k.rs:70-137.
__device__ bool make_qx_rmse1(const float (&x)[16], int32_t nmax, int32_t (&levels)[16], float& scale_out) {
    float maximum = 0.0f, magnitude = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if (fabsf(x[i]) > magnitude) {
            magnitude = fabsf(x[i]);
            maximum = x[i];
        }
    if (magnitude < 1e-15f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) levels[i] = 0;
        scale_out = 0.0f;
        return true;
    }
    bool ok = true;
    float inverse = (float)(-nmax) / maximum;
    float sum_lx = 0.0f, sum_l2 = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int32_t l = 0;
        ok &= nearest(inverse * x[i], l);
        l = clampi(l, -nmax, nmax - 1);
        levels[i] = l + nmax;
        const float w = x[i] * x[i];
        sum_lx += w * x[i] * (float)l;
        sum_l2 += w * (float)l * (float)l;
    }
    if (!ok || !finite(sum_lx) || !finite(sum_l2)) return false;
    float scale = sum_l2 != 0.0f ? sum_lx / sum_l2 : 0.0f;
    float best = scale * sum_lx;
    for (int step = -9; step <= 9; ++step) {
        if (step == 0) continue;
        inverse = -((float)nmax + 0.1f * (float)step) / maximum;
        sum_lx = 0.0f;
        sum_l2 = 0.0f;
        int32_t cand[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int32_t l = 0;
            ok &= nearest(inverse * x[i], l);
            l = clampi(l, -nmax, nmax - 1);
            cand[i] = nmax + l;
            const float w = x[i] * x[i];
            sum_lx += w * x[i] * (float)l;
            sum_l2 += w * (float)l * (float)l;
        }
        if (!ok || !finite(sum_lx) || !finite(sum_l2)) return false;
        if (sum_l2 > 0.0f && sum_lx * sum_lx > best * sum_l2) {
#pragma unroll
            for (int i = 0; i < 16; ++i) levels[i] = cand[i];
            scale = sum_lx / sum_l2;
            best = scale * sum_lx;
        }
    }
    if (!finite(scale)) return false;
    scale_out = scale;
    return true;
}

// Q6_K: 16 lanes per super-block (one 16-value sub-block each), 4 blocks a WG.
__global__ __launch_bounds__(64) void encode_q6k_kernel(const float* __restrict__ x, uint64_t nblocks,
                                                        uint8_t* __restrict__ out, unsigned long long* err_word) {
    __shared__ uint8_t lv[4][256];
    const uint32_t lane = threadIdx.x, gb = lane >> 4, sub = lane & 15;
    const uint64_t blk = (uint64_t)blockIdx.x * 4 + gb;
    const bool active = blk < nblocks;
    float xs[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
        float4 v = active ? *(const float4*)(x + blk * 256 + sub * 16 + i) : make_float4(0, 0, 0, 0);
        xs[i] = v.x, xs[i + 1] = v.y, xs[i + 2] = v.z, xs[i + 3] = v.w;
    }
    int32_t levels[16];
    float scale = 0.0f;
    bool ok = make_qx_rmse1(xs, 32, levels, scale);

    // first sub-block of largest |scale| (strict `>` from 0, encode_k.rs:525-528)
    uint64_t key = fabsf(scale) > 0.0f ? (((uint64_t)__float_as_uint(fabsf(scale)) << 32) | (15u - sub)) : 0;
    for (int m = 1; m < 16; m <<= 1) {
        const uint64_t o = __shfl_xor(key, m, 16);
        key = o > key ? o : key;
    }
    const int winner = key ? (int)(15u - (uint32_t)(key & 0xffffffffu)) : 0;
    const float maximum_scale = key ? __shfl(scale, (int)(lane & ~15u) + winner, 64) : 0.0f;
    const float maximum_magnitude = fabsf(maximum_scale);
    const bool zero_block = maximum_magnitude < 1e-15f;

    uint32_t dh = 0;
    int32_t sc_i = 0;
    if (!zero_block) {
        const float inverse = -128.0f / maximum_scale;
        dh = float_to_half_bits(1.0f / inverse);
        ok &= (dh & 0x7c00u) != 0x7c00u;
        ok &= nearest(inverse * scale, sc_i);
        sc_i = sc_i < 127 ? sc_i : 127;
        const float scale2 = half_bits_to_float_exact(dh) * (float)(int8_t)(uint8_t)sc_i;
        if (scale2 != 0.0f) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                int32_t l = 0;
                ok &= nearest(xs[i] / scale2, l);
                levels[i] = clampi(l, -32, 31) + 32;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) lv[gb][sub * 16 + i] = (uint8_t)levels[i];
    int okw = ok ? 1 : 0;
    for (int m = 1; m < 16; m <<= 1) okw &= __shfl_xor(okw, m, 16);
    __syncthreads();
    if (!active) return;
    if (!okw && sub == 0) report_error(err_word, error_key(0, kKindScale, blk));
    uint8_t* o = out + blk * 210;
    if (zero_block) {  // the block stays all zero (encode_k.rs:530-532)
        for (int k = sub; k < 210; k += 16) o[k] = 0;
        return;
    }
    // ql bytes sub*8 .. +7, qh bytes sub*4 .. +3 (encode_k.rs:548-559)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int byte = sub * 8 + k, g = byte / 64, r = byte % 64;
        const uint8_t* L = lv[gb] + g * 128;
        o[byte] = r < 32 ? (uint8_t)((L[r] & 15) | ((L[r + 64] & 15) << 4))
                         : (uint8_t)((L[r] & 15) | ((L[r + 64] & 15) << 4));
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int byte = sub * 4 + k, g = byte / 32, j = byte % 32;
        const uint8_t* L = lv[gb] + g * 128;
        o[128 + byte] = (uint8_t)((L[j] >> 4) | ((L[j + 32] >> 4) << 2) | ((L[j + 64] >> 4) << 4) |
                                  ((L[j + 96] >> 4) << 6));
    }
    o[192 + sub] = (uint8_t)sc_i;
    if (sub == 0) {
        o[208] = (uint8_t)(dh & 0xff);
        o[209] = (uint8_t)(dh >> 8);
    }
}

// Q2_K (encode_k.rs:292-355): 16 lanes per super-block (one 16-value
// sub-block each), 4 blocks a WG.  Scales and minima are 4-bit against the
// f16 d (byte 80) and dmin (byte 82); levels 0..3, two bits each from byte 16.
__global__ __launch_bounds__(64) void encode_q2k_kernel(const float* __restrict__ x, uint64_t nblocks,
                                                        uint8_t* __restrict__ out, unsigned long long* err_word) {
    __shared__ uint8_t lv[4][256];
    const uint32_t lane = threadIdx.x, gb = lane >> 4, sub = lane & 15;
    const uint64_t blk = (uint64_t)blockIdx.x * 4 + gb;
    const bool active = blk < nblocks;
    float xs[16], weights[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
        float4 v = active ? *(const float4*)(x + blk * 256 + sub * 16 + i) : make_float4(0, 0, 0, 0);
        xs[i] = v.x, xs[i + 1] = v.y, xs[i + 2] = v.z, xs[i + 3] = v.w;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) weights[i] = fabsf(xs[i]);
    int32_t levels[16];
    float scale = 0.0f, minimum = 0.0f;
    bool ok = make_affine2<16, true>(xs, 3, weights, levels, -0.5f, 0.1f, 15, scale, minimum);

    // maximum_scale / maximum_minimum: strict `>` from +0.0 (encode_k.rs:313-318)
    float ms = scale > 0.0f ? scale : 0.0f, mm = minimum > 0.0f ? minimum : 0.0f;
    for (int k = 1; k < 16; k <<= 1) {
        const float os = __shfl_xor(ms, k, 16), om = __shfl_xor(mm, k, 16);
        ms = os > ms ? os : ms;
        mm = om > mm ? om : mm;
    }
    // the scale byte: `nearest(..) as u8`, then `|= (nearest(..) as u8) << 4`
    uint32_t sbyte = 0, dh = 0, mh = 0;
    if (ms > 0.0f) {
        int32_t l = 0;
        ok &= nearest(15.0f / ms * scale, l);
        sbyte = (uint8_t)l;
        dh = float_to_half_bits(ms / 15.0f);
        ok &= (dh & 0x7c00u) != 0x7c00u;
    }
    if (mm > 0.0f) {
        int32_t l = 0;
        ok &= nearest(15.0f / mm * minimum, l);
        sbyte |= (uint8_t)((uint8_t)l << 4);
        mh = float_to_half_bits(mm / 15.0f);
        ok &= (mh & 0x7c00u) != 0x7c00u;
    }
    const float scale2 = half_bits_to_float_exact(dh) * (float)(sbyte & 15);
    if (scale2 != 0.0f) {
        const float minimum2 = half_bits_to_float_exact(mh) * (float)(sbyte >> 4);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int32_t l = 0;
            ok &= nearest((xs[i] + minimum2) / scale2, l);
            levels[i] = clampi(l, 0, 3);
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) lv[gb][sub * 16 + i] = (uint8_t)levels[i];
    int okw = ok ? 1 : 0;
    for (int k = 1; k < 16; k <<= 1) okw &= __shfl_xor(okw, k, 16);
    __syncthreads();
    if (!active) return;
    if (!okw && sub == 0) report_error(err_word, error_key(0, kKindScale, blk));
    uint8_t* o = out + blk * 84;
    o[sub] = (uint8_t)sbyte;
    // two-bit bytes sub*4 .. +3 (pack_two_bits, encode_k.rs:347-355)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int byte = sub * 4 + k, g = byte / 32, j = byte % 32;
        const uint8_t* L = lv[gb] + g * 128 + j;
        o[16 + byte] = (uint8_t)(L[0] | (L[32] << 2) | (L[64] << 4) | (L[96] << 6));
    }
    if (sub == 0) {
        o[80] = (uint8_t)(dh & 0xff);
        o[81] = (uint8_t)(dh >> 8);
        o[82] = (uint8_t)(mh & 0xff);
        o[83] = (uint8_t)(mh >> 8);
    }
}

// make_q3 (encode_k.rs:138-185): signed levels -nmax .. nmax - 1 fitted to
// x with weights x^2, then up to five passes of single-level moves that
// raise (sum w l x)^2 / sum w l^2, then shifted to 0 .. 2 nmax - 1.
__device__ bool make_q3_levels(const float (&x)[16], int32_t nmax, int32_t (&levels)[16], float& scale_out) {
    float maximum = 0.0f, magnitude = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if (fabsf(x[i]) > magnitude) {
            magnitude = fabsf(x[i]);
            maximum = x[i];
        }
    if (magnitude < 1e-15f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) levels[i] = 0;
        scale_out = 0.0f;
        return true;
    }
    const float inverse = (float)(-nmax) / maximum;
    float sum_lx = 0.0f, sum_l2 = 0.0f;
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int32_t l = 0;
        ok &= nearest(inverse * x[i], l);
        l = clampi(l, -nmax, nmax - 1);
        levels[i] = l;
        const float w = x[i] * x[i];
        sum_lx += w * x[i] * (float)l;
        sum_l2 += w * (float)l * (float)l;
    }
    if (!ok || !finite(sum_lx) || !finite(sum_l2)) return false;
    for (int pass = 0; pass < 5; ++pass) {
        bool changed = false;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float v = x[i], w = v * v;
            float lx = sum_lx - w * v * (float)levels[i];
            if (lx > 0.0f) {
                float l2 = sum_l2 - w * (float)levels[i] * (float)levels[i];
                int32_t next = 0;
                if (!nearest(v * l2 / lx, next)) return false;
                next = clampi(next, -nmax, nmax - 1);
                if (next != levels[i]) {
                    lx += w * v * (float)next;
                    l2 += w * (float)next * (float)next;
                    if (l2 > 0.0f && lx * lx * sum_l2 > sum_lx * sum_lx * l2) {
                        levels[i] = next;
                        sum_lx = lx;
                        sum_l2 = l2;
                        changed = true;
                    }
                }
            }
        }
        if (!changed) break;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) levels[i] += nmax;
    const float scale = sum_l2 > 0.0f ? sum_lx / sum_l2 : 0.0f;
    if (!finite(scale)) return false;
    scale_out = scale;
    return true;
}

// Q3_K (encode_k.rs:357-409): 16 lanes per super-block (one 16-value
// sub-block each), 4 blocks a WG.  Bytes 0..31 hold the third bit of each
// level (bit j / 32 of byte j % 32), 32..95 the low two bits, 96..107 the
// signed 6-bit scales (+32), 108 the f16 d.
__global__ __launch_bounds__(64) void encode_q3k_kernel(const float* __restrict__ x, uint64_t nblocks,
                                                        uint8_t* __restrict__ out, unsigned long long* err_word) {
    __shared__ uint8_t lv[4][256];
    const uint32_t lane = threadIdx.x, gb = lane >> 4, sub = lane & 15, base = lane & ~15u;
    const uint64_t blk = (uint64_t)blockIdx.x * 4 + gb;
    const bool active = blk < nblocks;
    float xs[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
        float4 v = active ? *(const float4*)(x + blk * 256 + sub * 16 + i) : make_float4(0, 0, 0, 0);
        xs[i] = v.x, xs[i + 1] = v.y, xs[i + 2] = v.z, xs[i + 3] = v.w;
    }
    int32_t levels[16];
    float scale = 0.0f;
    bool ok = make_q3_levels(xs, 4, levels, scale);

    // first sub-block of largest |scale| (strict `>` from 0, encode_k.rs:367-370)
    uint64_t key = fabsf(scale) > 0.0f ? (((uint64_t)__float_as_uint(fabsf(scale)) << 32) | (15u - sub)) : 0;
    for (int k = 1; k < 16; k <<= 1) {
        const uint64_t o = __shfl_xor(key, k, 16);
        key = o > key ? o : key;
    }
    const int winner = key ? (int)(15u - (uint32_t)(key & 0xffffffffu)) : 0;
    const float maximum_scale = key ? __shfl(scale, (int)base + winner, 64) : 0.0f;

    // the scale's byte value l + 32 (0 when every scale is 0, d = 0)
    int32_t u = 0;
    uint32_t dh = 0;
    if (maximum_scale != 0.0f) {
        const float inverse = -32.0f / maximum_scale;
        int32_t l = 0;
        ok &= nearest(inverse * scale, l);
        u = clampi(l, -32, 31) + 32;
        dh = float_to_half_bits(1.0f / inverse);
        ok &= (dh & 0x7c00u) != 0x7c00u;
    }
    const float scale2 = half_bits_to_float_exact(dh) * (float)(u - 32);
    if (scale2 != 0.0f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int32_t l = 0;
            ok &= nearest(xs[i] / scale2, l);
            levels[i] = clampi(l, -4, 3) + 4;
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) lv[gb][sub * 16 + i] = (uint8_t)levels[i];
    // the scale bytes' inputs from the other lanes of the block
    const int32_t u_hi = __shfl(u, (int)(base + ((sub + 8) & 15)), 64);
    int32_t u_top[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) u_top[q] = __shfl(u, (int)(base + (sub & 3) + 4 * q), 64);
    int okw = ok ? 1 : 0;
    for (int k = 1; k < 16; k <<= 1) okw &= __shfl_xor(okw, k, 16);
    __syncthreads();
    if (!active) return;
    if (!okw && sub == 0) report_error(err_word, error_key(0, kKindScale, blk));
    uint8_t* o = out + blk * 110;
    // third bits: bytes 2 sub, 2 sub + 1
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int j = sub * 2 + k;
        uint32_t h = 0;
#pragma unroll
        for (int b = 0; b < 8; ++b) h |= (lv[gb][j + 32 * b] > 3 ? 1u : 0u) << b;
        o[j] = (uint8_t)h;
    }
    // low two bits: bytes 32 + sub*4 .. +3 (pack_two_bits of the levels less 4)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int byte = sub * 4 + k, g = byte / 32, j = byte % 32;
        const uint8_t* L = lv[gb] + g * 128 + j;
        o[32 + byte] = (uint8_t)((L[0] & 3) | ((L[32] & 3) << 2) | ((L[64] & 3) << 4) | ((L[96] & 3) << 6));
    }
    if (sub < 8) {
        o[96 + sub] = (uint8_t)((u & 15) | ((u_hi & 15) << 4));
    } else if (sub < 12) {
        uint32_t t = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) t |= (uint32_t)(u_top[q] >> 4) << (2 * q);
        o[104 + (sub - 8)] = (uint8_t)t;
    } else if (sub == 12) {
        o[108] = (uint8_t)(dh & 0xff);
        o[109] = (uint8_t)(dh >> 8);
    }
}

// All K encoders (encode_k.rs:11-33): n values as one run of n / 256 blocks.
hipError_t launch_encode_k(uint32_t t, const float* x, uint64_t n, uint8_t* out, unsigned long long* err_word,
                           hipStream_t s) {
    const uint64_t nb = n / 256;
    if (nb == 0) return hipSuccess;
    const dim3 by8((unsigned)((nb + 7) / 8)), by4((unsigned)((nb + 3) / 4));
    switch (t) {
        case kQ2_K: hipLaunchKernelGGL(encode_q2k_kernel, by4, dim3(64), 0, s, x, nb, out, err_word); break;
        case kQ3_K: hipLaunchKernelGGL(encode_q3k_kernel, by4, dim3(64), 0, s, x, nb, out, err_word); break;
        case kQ4_K: hipLaunchKernelGGL(encode_q45k_kernel<false>, by8, dim3(64), 0, s, x, nb, out, err_word); break;
        case kQ5_K: hipLaunchKernelGGL(encode_q45k_kernel<true>, by8, dim3(64), 0, s, x, nb, out, err_word); break;
        case kQ6_K: hipLaunchKernelGGL(encode_q6k_kernel, by4, dim3(64), 0, s, x, nb, out, err_word); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Decoders (decode.rs), one thread per output value.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float half_at(const uint8_t* b, int p) {
    return half_bits_to_float_exact((uint32_t)b[p] | ((uint32_t)b[p + 1] << 8));
}

__global__ __launch_bounds__(256) void dequantize_kernel(uint32_t t, const uint8_t* __restrict__ src, uint64_t n,
                                                         float* __restrict__ y) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        float v;
        if (t == kQ8_0) {  // decode.rs:17-23
            const uint8_t* b = src + (i / 32) * 34;
            v = (float)(int8_t)b[2 + i % 32] * half_at(b, 0);
        } else if (t == kQ8_K) {  // decode.rs:44-49
            const uint8_t* b = src + (i / 256) * 292;
            float d;
            __builtin_memcpy(&d, b, 4);
            v = d * (float)(int8_t)b[4 + i % 256];
        } else if (t == kQ4_K || t == kQ5_K) {  // decode.rs:216-235 (Q5_K: + 16 from qh)
            const bool five = t == kQ5_K;
            const uint8_t* b = src + (i / 256) * (five ? 176 : 144);
            const int e = (int)(i % 256), group = e / 64, side = (e % 64) / 32, j = e % 32;
            const int sub = group * 2 + side;
            const uint8_t* p = b + 4;
            uint8_t sc, m;
            if (sub < 4) {
                sc = p[sub] & 63;
                m = p[sub + 4] & 63;
            } else {
                sc = (uint8_t)((p[sub + 4] & 15) | ((p[sub - 4] >> 6) << 4));
                m = (uint8_t)((p[sub + 4] >> 4) | ((p[sub] >> 6) << 4));
            }
            const float dl = half_at(b, 0) * (float)sc;
            const float ml = half_at(b, 2) * (float)m;
            uint8_t q = (b[(five ? 48 : 16) + group * 32 + j] >> (side * 4)) & 15;
            if (five && ((b[16 + j] >> sub) & 1)) q += 16;
            v = dl * (float)q - ml;
        } else if (t == kQ2_K) {  // decode.rs:159-175
            const uint8_t* b = src + (i / 256) * 84;
            const int e = (int)(i % 256), group = e / 128, lane = (e % 128) / 32, pos = e % 32;
            const uint8_t sc = b[group * 8 + lane * 2 + pos / 16];
            const float dl = half_at(b, 80) * (float)(sc & 15), ml = half_at(b, 82) * (float)(sc >> 4);
            v = dl * (float)((b[16 + group * 32 + pos] >> (2 * lane)) & 3) - ml;
        } else if (t == kQ3_K) {  // decode.rs:177-202
            const uint8_t* b = src + (i / 256) * 110;
            const int e = (int)(i % 256), group = e / 128, lane = (e % 128) / 32, pos = e % 32;
            const int k = group * 8 + lane * 2 + pos / 16, j = k % 4;  // scale index k = 4 * (k / 4) + j
            const uint8_t* p = b + 96;
            const int lo = k < 8 ? p[(k / 4) * 4 + j] & 15 : p[(k / 4 - 2) * 4 + j] >> 4;
            const int sc = lo | (((p[8 + j] >> (2 * (k / 4))) & 3) << 4);
            const int q = ((b[32 + group * 32 + pos] >> (2 * lane)) & 3) - (((b[pos] >> (group * 4 + lane)) & 1) ? 0 : 4);
            v = half_at(b, 108) * (float)(sc - 32) * (float)q;
        } else {  // Q6_K, decode.rs:237-258
            const uint8_t* b = src + (i / 256) * 210;
            const int e = (int)(i % 256), group = e / 128, side = (e % 128) / 32, j = e % 32;
            const uint8_t lo = b[group * 64 + (side & 1) * 32 + j];
            const uint8_t hi = b[128 + group * 32 + j];
            const int q = ((lo >> (4 * (side >> 1))) & 15) | (((hi >> (2 * side)) & 3) << 4);
            v = half_at(b, 208) * (float)(int8_t)b[192 + group * 8 + j / 16 + side * 2] * (float)(q - 32);
        }
        y[i] = v;
    }
}

hipError_t launch_dequantize(uint32_t t, const uint8_t* b, uint64_t n, float* y, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const uint64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, s, t,
                       b, n, y);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GGUF -> tiled device layout (rlq_layout.hpp).  One thread per source byte;
// the destination is zeroed first, which fills the padding rows of the last
// tile and the missing odd Q8_0 block.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fill_zero16_kernel(uint4* __restrict__ p, uint64_t n16) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0, 0, 0, 0);
}

__global__ __launch_bounds__(256) void repack_tiled_kernel(uint32_t t, const uint8_t* __restrict__ src, uint64_t rows,
                                                           uint64_t nb, uint32_t ts, uint8_t* __restrict__ dst) {
    const uint64_t per_row = nb * ts, total = rows * per_row;
    for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t row = e / per_row, rem = e % per_row, blk = rem / ts;
        const uint32_t byte = (uint32_t)(rem % ts);
        dst[layout_offset(t, row, blk, byte, nb)] = src[e];
    }
}

hipError_t launch_repack(uint32_t t, const uint8_t* gguf, uint64_t rows, uint64_t cols, uint8_t* dev,
                         hipStream_t s) {
    const uint64_t n16 = layout_bytes(t, rows, cols) / 16;
    hipLaunchKernelGGL(fill_zero16_kernel, dim3(2048), dim3(256), 0, s, (uint4*)dev, n16);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t bs = t == kQ8_0 ? 32 : 256;
    const uint32_t ts = t == kQ8_0 ? 34 : t == kQ2_K ? 84 : t == kQ3_K ? 110 : t == kQ4_K ? 144 : t == kQ5_K ? 176 : 210;
    hipLaunchKernelGGL(repack_tiled_kernel, dim3(8192), dim3(256), 0, s, t, gguf, rows, cols / bs, ts, dev);
    return hipGetLastError();
}

__global__ void fill_u64_kernel(unsigned long long* p, uint64_t n, unsigned long long v) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

hipError_t launch_fill_u64(unsigned long long* p, uint64_t n, unsigned long long v, hipStream_t s) {
    const uint64_t grid = (n + 255) / 256;
    hipLaunchKernelGGL(fill_u64_kernel, dim3((unsigned)(grid ? (grid < 1024 ? grid : 1024) : 1)), dim3(256), 0, s,
                       p, n, v);
    return hipGetLastError();
}

}  // namespace rlq
