// rlq_q8k.hpp - the Q8_K activation quantizer shared by the fused matvec
// prologue and the prefill activation kernel (crates/quant/src/activation.rs:4-51).
#pragma once

#include "rlq_device.hpp"

namespace rlq {

// ---- 16-lane row reductions (DPP; every lane of the row gets the result) ----
constexpr int kRowMirror = 0x140;  // lane i <-> 15 - i within each 16 lanes

__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f<kQuadXor1>(v));
    v = fmaxf(v, dpp_f<kQuadXor2>(v));
    v = fmaxf(v, dpp_f<kRowHalfMirror>(v));
    return fmaxf(v, dpp_f<kRowMirror>(v));
}
__device__ __forceinline__ uint32_t umin_(uint32_t a, uint32_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint32_t row16_umin(uint32_t v) {
    v = umin_(v, (uint32_t)dpp_i<kQuadXor1>((int32_t)v));
    v = umin_(v, (uint32_t)dpp_i<kQuadXor2>((int32_t)v));
    v = umin_(v, (uint32_t)dpp_i<kRowHalfMirror>((int32_t)v));
    return umin_(v, (uint32_t)dpp_i<kRowMirror>((int32_t)v));
}

__device__ __forceinline__ float row16_min(float v) {
    v = fminf(v, dpp_f<kQuadXor1>(v));
    v = fminf(v, dpp_f<kQuadXor2>(v));
    v = fminf(v, dpp_f<kRowHalfMirror>(v));
    return fminf(v, dpp_f<kRowMirror>(v));
}

// One Q8_K block (activation.rs:4-51) quantized by the 16 lanes of a DPP row;
// lane r16 holds values 16 r16 .. 16 r16 + 15 of the block.  Every branch
// below is uniform over the row.
//  - Non-finite input: an FMA chain with 0 turns any inf/NaN into NaN; only
//    then is the first non-finite index searched (NonFiniteInput{index}).
//  - inverse_scale keeps the FIRST value of largest |x|.  With the row's max
//    and min, the sign of that value is known unless both +amax and -amax
//    occur; only then is the first such index searched.
//  - q = round_ties_even(inverse * x): the product is rounded to f32 first,
//    then adding 1.5 * 2^23 rounds it to an integer (ties to even) that sits
//    in the low mantissa bits, whose low byte is q as int8.  |inverse * x| <=
//    127 (1 + 2^-23)^2 < 127.5, so q <= 127 and the reference's min(127) never
//    applies.
struct Q8KRow {
    uint32_t q[4];
    float d;
    int32_t bsum;     // sum of this lane's 16 q
    int kind;         // -1 valid, kKindNonFinite, kKindScale
    uint32_t index;   // NonFiniteInput index within the block
};

__device__ __forceinline__ Q8KRow q8k_row16(const float (&v)[16], uint32_t r16) {
    Q8KRow o;
    o.q[0] = o.q[1] = o.q[2] = o.q[3] = 0;
    o.d = 0.0f;
    o.bsum = 0;
    o.kind = -1;
    o.index = 0;
    float t = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) t = __builtin_fmaf(v[k], 0.0f, t);
    if (row16_umin(t == t ? 1u : 0u) == 0) {
        uint32_t nf = 0xffffffffu;
#pragma unroll
        for (int k = 15; k >= 0; --k)
            if (!finite(v[k])) nf = 16 * r16 + k;
        o.kind = kKindNonFinite;
        o.index = row16_umin(nf);
        return o;
    }
    float mx = __builtin_fmaxf(v[0], v[1]), mn = __builtin_fminf(v[0], v[1]);
#pragma unroll
    for (int k = 2; k < 16; k += 2) {
        mx = fmaxf(mx, fmaxf(v[k], v[k + 1]));
        mn = fminf(mn, fminf(v[k], v[k + 1]));
    }
    mx = row16_max(mx);
    mn = row16_min(mn);
    float maximum;
    if (mx > -mn) {
        maximum = mx;
    } else if (-mn > mx) {
        maximum = mn;
    } else if (mx == 0.0f) {
        return o;  // all zero: canonical zero block
    } else {      // +amax and -amax both occur: the first one wins
        uint32_t key = 0xffffffffu;
#pragma unroll
        for (int k = 15; k >= 0; --k)
            if (fabsf(v[k]) == mx) key = (16 * r16 + k) << 1 | (__float_as_uint(v[k]) >> 31);
        maximum = (row16_umin(key) & 1u) ? mn : mx;
    }
    const float inverse = -127.0f / maximum;
    if (!finite(inverse) || !finite(1.0f / inverse)) {
        o.kind = kKindScale;
        return o;
    }
    uint32_t b[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float r = inverse * v[k];
        b[k] = __float_as_uint(r + 12582912.0f);
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t lo = __builtin_amdgcn_perm(b[4 * w + 1], b[4 * w], 0x0c0c0400u);
        const uint32_t hi = __builtin_amdgcn_perm(b[4 * w + 3], b[4 * w + 2], 0x04000c0cu);
        o.q[w] = lo | hi;
    }
    int32_t sum = dot4(o.q[0], 0x01010101u, 0);
    sum = dot4(o.q[1], 0x01010101u, sum);
    sum = dot4(o.q[2], 0x01010101u, sum);
    o.bsum = dot4(o.q[3], 0x01010101u, sum);
    o.d = 1.0f / inverse;
    return o;
}

// The Q4_K / Q5_K slot order of an activation image (rlq_layout.hpp,
// q45_pos_of_slot): the two lanes of a quad pair hold the 16 values of one
// sub-block half each (lane bit 0 = half h'), q their natural bytes.  Slot
// word k' (k' = 0..7) of the sub-block is (u0[k'], u0[k'+8], u1[k'], u1[k'+8])
// with u0, u1 the two halves; the lane of half h' returns words 4h'..4h'+3,
// i.e. slots 16h'..16h'+15, which it stores where its natural bytes would
// go.  Both lanes of the pair must be active.
__device__ __forceinline__ uint4 q45_slots(const uint32_t (&q)[4], uint32_t odd) {
    // (u[k'], u[k'+8]) pairs of this half, two per word
    const uint32_t Q0 = __builtin_amdgcn_perm(q[2], q[0], 0x05010400u);
    const uint32_t Q1 = __builtin_amdgcn_perm(q[2], q[0], 0x07030602u);
    const uint32_t Q2 = __builtin_amdgcn_perm(q[3], q[1], 0x05010400u);
    const uint32_t Q3 = __builtin_amdgcn_perm(q[3], q[1], 0x07030602u);
    // the even lane sends its pairs 4..7, the odd lane its pairs 0..3
    const uint32_t R0 = (uint32_t)dpp_i<kQuadXor1>((int32_t)(odd ? Q0 : Q2));
    const uint32_t R1 = (uint32_t)dpp_i<kQuadXor1>((int32_t)(odd ? Q1 : Q3));
    const uint32_t lo0 = odd ? R0 : Q0, hi0 = odd ? Q2 : R0;
    const uint32_t lo1 = odd ? R1 : Q1, hi1 = odd ? Q3 : R1;
    return make_uint4(__builtin_amdgcn_perm(hi0, lo0, 0x05040100u), __builtin_amdgcn_perm(hi0, lo0, 0x07060302u),
                      __builtin_amdgcn_perm(hi1, lo1, 0x05040100u), __builtin_amdgcn_perm(hi1, lo1, 0x07060302u));
}

}  // namespace rlq
