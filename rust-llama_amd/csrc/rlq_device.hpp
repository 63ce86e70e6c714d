// rlq_device.hpp - device helpers shared by the gfx950 kernels.
//
// Everything here is compiled with -ffp-contract=off: f32 expressions round
// operation by operation, as the reference's Rust source does, and fused
// multiply-adds appear only where a kernel asks for one explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rlq {

constexpr int kWave = 64;

// ---- f16 <-> f32 --------------------------------------------------------

// Hardware conversion: exact for every non-NaN half (f16 denormals are kept
// by the default gfx9 FP mode).
__device__ __forceinline__ float half_to_float(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu));
}

// Binary32 -> binary16 with ties-to-even and signed canonical NaNs, bit for bit
// as crates/quant/src/lib.rs:340-373 (f32_to_f16).  Used by the encoders,
// where the stored bits must equal the reference's.
__device__ __forceinline__ uint32_t float_to_half_bits(float value) {
    const uint32_t bits = __float_as_uint(value);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const int32_t exp = (int32_t)((bits >> 23) & 255u);
    const uint32_t frac = bits & 0x7fffffu;
    if (exp == 255) return sign | (frac == 0 ? 0x7c00u : 0x7e00u);
    const int32_t e = exp - 127;
    if (e > 15) return sign | 0x7c00u;
    if (e >= -14) {
        uint32_t mant = frac >> 13;
        const uint32_t rest = frac & 8191u;
        if (rest > 4096u || (rest == 4096u && (mant & 1u) != 0)) mant += 1;
        return (sign | ((((uint32_t)(e + 15)) << 10) + mant)) & 0xffffu;
    }
    if (e < -25) return sign;
    const uint32_t mant = frac | 0x800000u;
    const uint32_t shift = (uint32_t)(-e - 1);
    uint32_t rounded = mant >> shift;
    const uint32_t rest = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rest > half || (rest == half && (rounded & 1u) != 0)) rounded += 1;
    return (sign | rounded) & 0xffffu;
}

// Binary16 -> binary32 bit for bit as lib.rs:323-337 (NaNs quieted).  The
// encoders read back the half they stored through this.
__device__ __forceinline__ float half_bits_to_float_exact(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 31u;
    const uint32_t fraction = h & 1023u;
    uint32_t result;
    if (exp == 0 && fraction == 0) {
        result = sign;
    } else if (exp == 0) {
        const uint32_t shift = (uint32_t)__builtin_clz(fraction) - 21u;
        result = sign | ((113u - shift) << 23) | (((fraction << shift) & 1023u) << 13);
    } else if (exp == 31) {
        result = sign | 0x7f800000u | (fraction << 13) | (fraction != 0 ? 0x00400000u : 0u);
    } else {
        result = sign | ((exp + 112u) << 23) | (fraction << 13);
    }
    return __uint_as_float(result);
}

__device__ __forceinline__ bool finite(float v) { return __builtin_isfinite(v); }

// ---- integer dot ---------------------------------------------------------

// v_dot4_i32_i8: acc + sum of four signed byte products.
__device__ __forceinline__ int32_t dot4(uint32_t a, uint32_t b, int32_t acc) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, acc, false);
}

// ---- cross-lane reductions (wave64) -------------------------------------

// DPP control codes (GFX9 encoding).
constexpr int kQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;  // lane i <-> 7-i within each 8 lanes
constexpr int kRowRor8 = 0x128;        // rotate right by 8 within each 16 lanes

template <int Ctrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xf, 0xf, false));
}
template <int Ctrl>
__device__ __forceinline__ int32_t dpp_i(int32_t v) {
    return __builtin_amdgcn_update_dpp(0, v, Ctrl, 0xf, 0xf, false);
}

// Sum over each aligned group of 8 lanes; every lane of the group gets it.
__device__ __forceinline__ int32_t group8_sum(int32_t v) {
    v += dpp_i<kQuadXor1>(v);
    v += dpp_i<kQuadXor2>(v);
    v += dpp_i<kRowHalfMirror>(v);
    return v;
}

// f64 moved by DPP: the two halves separately.
template <int Ctrl>
__device__ __forceinline__ double dpp_d(double v) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)dpp_i<Ctrl>((int32_t)(uint32_t)u);
    const uint32_t hi = (uint32_t)dpp_i<Ctrl>((int32_t)(uint32_t)(u >> 32));
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
// Sum over each aligned row of 16 lanes in a fixed order; every lane of the
// row gets it (DPP only: no LDS traffic).
__device__ __forceinline__ double row16_sum_f64(double v) {
    v += dpp_d<kQuadXor1>(v);
    v += dpp_d<kQuadXor2>(v);
    v += dpp_d<kRowHalfMirror>(v);
    v += dpp_d<kRowRor8>(v);
    return v;
}

// The value of lane l (uniform: the wave's scalar read of one lane).
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Sum over all 64 lanes ((row 0 + row 1) + (row 2 + row 3) of the 16-lane
// row sums); every lane gets it.  These wave reductions read the rows with
// scalar lane reads: call them with every lane of the wave active.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<kQuadXor1>(v);
    v += dpp_f<kQuadXor2>(v);
    v += dpp_f<kRowHalfMirror>(v);
    v += dpp_f<kRowRor8>(v);
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

__device__ __forceinline__ int32_t wave_sum_i(int32_t v) {
    v += dpp_i<kQuadXor1>(v);
    v += dpp_i<kQuadXor2>(v);
    v += dpp_i<kRowHalfMirror>(v);
    v += dpp_i<kRowRor8>(v);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}
// The four 16-lane rows' (row-uniform) values combined as (row 0 + row 1) +
// (row 2 + row 3).
__device__ __forceinline__ double rows_sum_f64(double v) {
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}
// Sum over all 64 lanes in a fixed order (the 16-lane rows by DPP, then the
// rows); every lane gets it.
__device__ __forceinline__ double wave_sum_f64(double v) { return rows_sum_f64(row16_sum_f64(v)); }
// Maximum over all 64 lanes (DPP inside the rows, then the rows).
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_f<kQuadXor1>(v));
    v = fmaxf(v, dpp_f<kQuadXor2>(v));
    v = fmaxf(v, dpp_f<kRowHalfMirror>(v));
    v = fmaxf(v, dpp_f<kRowRor8>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    for (int m = 1; m < 64; m <<= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)v, m, 64);
        v = o < v ? o : v;
    }
    return v;
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
    for (int m = 1; m < 64; m <<= 1) {
        const uint64_t o = __shfl_xor(v, m, 64);
        v = o < v ? o : v;
    }
    return v;
}

// ---- loads ---------------------------------------------------------------

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte global load that streams past the caches (weights are read once).
__device__ __forceinline__ uint4 load_stream16(const void* p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// The same for four floats read once per launch: the cached keys of the
// attention scores.  Llama-3-8B decode step at a context of 1024, ms per token
// on one box: plain loads 1.7437-1.7441, non-temporal keys 1.7071-1.7085,
// non-temporal values 1.7333-1.7334, both 1.7355-1.7356 (the values stay
// plain).
__device__ __forceinline__ float4 load_stream_f4(const void* p) {
    const f32x4 v = __builtin_nontemporal_load((const f32x4*)p);
    return make_float4(v.x, v.y, v.z, v.w);
}

// ---- the reference's SSE2 exponential -------------------------------------
// One lane of crates/quant/src/cpu_math.rs:94-123 with its exact f32
// constants and operation order (the file is built without contraction).
// The source picks one branch per four-lane vector, but both branches give
// scale*p + scale for every lane with |n| <= 126, so each lane's value
// depends on that lane alone.
__device__ __forceinline__ float sse2_exp(float x) {
    const float z = x * __uint_as_float(0x3fb8aa3bu) + __uint_as_float(0x4b400000u);
    const float n = z - __uint_as_float(0x4b400000u);
    const float b = (x - n * __uint_as_float(0x3f317200u)) - n * __uint_as_float(0x35bfbe8eu);
    const uint32_t exponent = __float_as_uint(z) << 23;
    const float scale = __uint_as_float(exponent + 0x3f800000u);
    const float squared = b * b;
    const float first = __uint_as_float(0x3c072010u) * b + __uint_as_float(0x3d2b9f17u);
    const float second = __uint_as_float(0x3e2aaf33u) * b + __uint_as_float(0x3efffedbu);
    const float polynomial = (first * squared + second) * squared + __uint_as_float(0x3f7ffff6u) * b;
    // both branches computed and one selected (no divergent branch, so the
    // exponentials of a lane interleave)
    const float plain = polynomial * scale + scale;
    const uint32_t shift = n <= 0.0f ? 0x82000000u : 0u;
    const float high = __uint_as_float(shift + 0x7f000000u);
    const float low = __uint_as_float(exponent - shift);
    const float wide = fabsf(n) > 192.0f ? high * high : (low * polynomial + low) * high;
    return fabsf(n) > 126.0f ? wide : plain;
}

// ---- device error word ---------------------------------------------------
//
// One u64 per context, UINT64_MAX when clear.  The first data error in the
// reference's reporting order wins an atomicMin:
//   key = (column + 1) << 41 | kind << 40 | index
// kind 0 = NonFiniteInput{index}, kind 1 = UnrepresentableScale{block}.  In
// the reference every check of one activation row runs before the next row
// is quantized (crates/tensor/src/cpu_extra.rs:815-822), and within one row
// the finite scan precedes the scale preflight (encode.rs:70-77).  Keys with
// a column field of 0 are call-level errors found before any row is
// quantized: MUL_MAT_ID's expert-id check (TensorError::Bounds,
// crates/tensor/src/cpu_index.rs:197-202), key = index of the first bad id.
constexpr int kKindNonFinite = 0;
constexpr int kKindScale = 1;

__device__ __forceinline__ uint64_t error_key(uint64_t column, int kind, uint64_t index) {
    return ((column + 1) << 41) | ((uint64_t)kind << 40) | (index & ((1ull << 40) - 1));
}
__device__ __forceinline__ uint64_t bounds_key(uint64_t index) { return index & ((1ull << 40) - 1); }

__device__ __forceinline__ void report_error(unsigned long long* word, uint64_t key) {
    atomicMin(word, (unsigned long long)key);
}

// Model-runtime errors (crates/model-runtime: Matrix::multiply and the Llama
// decode step) use the column field's largest value, so they sort after every
// quantizer key of a plain call:
//   key = 0x7fffff << 41 | layer << 25 | stage << 20 | index
// The stage numbers the step's checks in the reference's order within a
// layer (ModelStage), so the smallest key is the first check the reference's
// sequential step would fail: an earlier layer first, then an earlier stage.
constexpr uint64_t kModelField = 0x7fffffull;
enum ModelStage : uint32_t {
    kStAttnNormScale = 1,   // math.rs:218-220 "RMS normalization scale"
    kStAttnNormOut = 2,     // math.rs:227 "RMS normalization output" (the Q/K/V quantizer's input)
    kStQkvQuant = 3,        // the Q/K/V activation's QuantError (UnrepresentableScale)
    kStQkvOut = 4,          // math.rs:167 "matrix output"
    kStScore = 5,           // math.rs:476-478 "attention score"
    kStAttnOut = 6,         // math.rs:494 "attention output"
    kStOIn = 7,             // math.rs:152 "matrix input"
    kStOQuant = 8,
    kStOOut = 9,
    kStFfnNormScale = 10,
    kStFfnNormOut = 11,
    kStGuQuant = 12,
    kStGuOut = 13,
    kStDownIn = 14,         // silu(gate) * up, the down projection's input
    kStDownQuant = 15,
    kStDownOut = 16,
    kStLayerOut = 17,       // llama.rs:378 "Llama layer output"
};
__device__ __forceinline__ uint64_t model_key(uint32_t layer, uint32_t stage, uint64_t index) {
    return (kModelField << 41) | ((uint64_t)(layer & 0xffffu) << 25) | ((uint64_t)(stage & 31u) << 20) |
           (index < 0xfffffull ? index : 0xfffffull);
}

}  // namespace rlq
