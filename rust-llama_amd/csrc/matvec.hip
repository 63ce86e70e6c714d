// matvec.hip - decode matvec (batch 1..8) for Q2_K..Q6_K / Q8_0 weights on gfx950.
//
// Contract (paths relative to the rust-llama repository):
//   y[b][r] = dot_packed(row r, activation column b), the activation being
//   column b of x quantized to Q8_K (K formats) or Q8_0 (Q8_0 weights)
//     Q8_0  crates/quant/src/matvec.rs:115-160  (Q8_0 branch :124-128)
//     Q2_K  crates/quant/src/matvec_extra.rs:174-198
//     Q3_K  crates/quant/src/matvec_extra.rs:200-210, 234-248, 286-293
//     Q4_K  crates/quant/src/matvec_extra.rs:212-271, 286-293
//     Q5_K  crates/quant/src/matvec_extra.rs:250-271 (the Q4_K branch plus qh)
//     Q6_K  crates/quant/src/matvec_extra.rs:272-283, 286-293
//   quantizers crates/quant/src/activation.rs:4-51 (Q8_K),
//              crates/quant/src/encode.rs:115-126, 151-192 (Q8_0)
//
// Design.  One kernel per weight format, for any batch of up to 8 columns.
//  - Weights are read in the tiled device layout (rlq_layout.hpp): a wave owns
//    16-row tiles and streams each tile's chunks with 16-byte loads issued D
//    chunks ahead of use, so HBM reads overlap the arithmetic.
//  - The prologue of every workgroup quantizes all batch columns of x into LDS
//    (the fused activation quantizer), after the first weight loads are in
//    flight.  A data error (non-finite input, unrepresentable scale) is
//    reported to the error word and the workgroup writes nothing.
//  - Integer products run on v_mfma_i32_16x16x64_i8 with the weights as the
//    B operand (16 rows = 16 columns of the product) and the activations as
//    the A operand.  The A rows are (batch column, sub-block) pairs and every
//    A row is zero outside the K range of its sub-block, so each output is
//    the exact integer dot of one sub-block for one column; the K-quant
//    sub-block scales are applied to those integers on the VALU.  The MFMA
//    work is the same for every batch size.
//  - Lane l of a wave owns weight row n = l % 16 and output columns that
//    depend on l / 16; every (row, column) sum lives in one lane, so no cross
//    lane reduction is needed.
//
// F32 order.  Per (row, column) the lane adds one f32 term per block (Q8_0:
// exactly the reference's `sum += isum as f32 * (dx * dy)` in block order, so
// Q8_0 results equal the reference bit for bit).  Q4_K / Q6_K add
// d * isum - dmin * imin per block from the exact block integers, where the
// reference keeps eight lane accumulators; the difference is f32 rounding of
// the same exact integers.  Q2_K adds d * isum - dmin * imin per block in
// block order in one lane, which is the reference's own sequence: Q2_K
// results equal the reference bit for bit.
#include "rlq_device.hpp"
#include "rlq_internal.hpp"
#include "rlq_layout.hpp"
#include "rlq_q8k.hpp"

namespace rlq {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef short i16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ i32x4 mfma_i8(i32x4 a, i32x4 b) {
    const i32x4 z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, z, 0, 0, 0);
}

__device__ __forceinline__ i32x4 lo_nibbles(uint4 v) {
    return i32x4{(int)(v.x & 0x0f0f0f0fu), (int)(v.y & 0x0f0f0f0fu), (int)(v.z & 0x0f0f0f0fu),
                 (int)(v.w & 0x0f0f0f0fu)};
}
__device__ __forceinline__ i32x4 hi_nibbles(uint4 v) {
    return i32x4{(int)((v.x >> 4) & 0x0f0f0f0fu), (int)((v.y >> 4) & 0x0f0f0f0fu), (int)((v.z >> 4) & 0x0f0f0f0fu),
                 (int)((v.w >> 4) & 0x0f0f0f0fu)};
}

// High nibbles of 16 bytes with two 64-bit shifts: bits shifted across the
// word boundary land in the masked-off high nibble of byte 3.
__device__ __forceinline__ void hi_nibbles64(uint4 v, uint32_t (&o)[4]) {
    const uint64_t a = ((((uint64_t)v.y << 32) | v.x) >> 4) & 0x0f0f0f0f0f0f0f0full;
    const uint64_t b = ((((uint64_t)v.w << 32) | v.z) >> 4) & 0x0f0f0f0f0f0f0f0full;
    o[0] = (uint32_t)a, o[1] = (uint32_t)(a >> 32), o[2] = (uint32_t)b, o[3] = (uint32_t)(b >> 32);
}

__device__ __forceinline__ int32_t dot2(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(i16x2, a), __builtin_bit_cast(i16x2, b), c, false);
}

__device__ __forceinline__ uint32_t ubyte(uint32_t w, int k) { return __builtin_amdgcn_ubfe(w, 8 * k, 8); }
__device__ __forceinline__ int32_t sbyte(uint32_t w, int k) { return __builtin_amdgcn_sbfe((int)w, 8 * k, 8); }

// ---- greedy argmax key -------------------------------------------------------
// Largest value wins, then the lowest row (sampling.rs:607-613 keeps the first
// strict maximum).  -0.0 is folded onto +0.0 because they compare equal.  A
// NaN never wins a strict `>` and maps to 0, except at row 0: the reference's
// scan starts from row 0 and nothing compares greater than a NaN, so a NaN
// there is the answer; its key is the largest (it decodes to row 0).
__device__ __forceinline__ unsigned long long argmax_key(float v, uint64_t row) {
    if (v != v) return row == 0 ? ~0ull : 0ull;
    uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)b << 32) | (0xffffffffull - (row & 0xffffffffull));
}

// Max over the 16 lanes of each row (lane & 15), result in every lane.
__device__ __forceinline__ unsigned long long row16_max_u64(unsigned long long v) {
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
        const unsigned long long o = __shfl_xor(v, m, 64);
        v = o > v ? o : v;
    }
    return v;
}

// ---------------------------------------------------------------------------
// Kernel arguments and the LDS image of the quantized activations
// ---------------------------------------------------------------------------
struct MvArgs {
    const uint8_t* w;                 // weights, device layout
    uint32_t rows, nb;                // rows; GGUF blocks per row
    uint32_t ntiles, nchunks;         // 16-row tiles; chunks per tile
    uint32_t batch;                   // columns in this launch, 1..8
    uint32_t cols;
    const float* x;                   // f32 activations [batch][cols], or null
    ActPlanes pre;                    // pre-quantized activations when x is null
    float* y;                         // y[b * ldy + row]
    uint64_t ldy;
    // Greedy argmax of every column (crates/llama-behavior/src/sampling.rs:
    // 607-618), finished inside the launch (finish_argmax): am_slots
    // [gridDim.x][batch] per-workgroup keys, am_count the launch's arrival
    // counter (0 before and after every launch), am_out [batch] token ids; null
    // am_out: no argmax
    unsigned long long* am_slots;
    unsigned int* am_count;
    uint32_t* am_out;
    unsigned long long* err_word;
    uint32_t err_column0;             // column index of this launch's column 0
    int32_t* dbg_isum;                // [rows][nb] exact integers vs column 0, or null
    int32_t* dbg_imin;
    // Input transform applied before quantization (batch 1; MvXform) and the
    // residual added to every output (y = resid + dot; may alias y), or null.
    uint32_t xform;
    float eps;
    const float* norm_w;
    const float* resid;
    // kEpSiluPair: the rows are gate and up tiles interleaved ([gate tile i,
    // up tile i] as tiles 2i, 2i + 1) and y[16 i + r] = silu(gate) * up
    uint32_t epilogue;
    // When non-null and nonzero, every workgroup exits before touching
    // anything: the call was refused on the device (MUL_MAT / MUL_MAT_ID).
    const uint32_t* gate;
    // MUL_MAT_ID: workgroup row blockIdx.y is (token, slot) pair id_base +
    // blockIdx.y: expert ids[pair] (of id_experts, expert_bytes apart), the
    // pre-quantized column token * id_cols + slot % id_cols, output rows at
    // y + pair * ldy.  Null ids: one matrix, one grid row.
    const int32_t* ids;
    uint32_t id_base, id_slots, id_cols, id_experts;
    uint64_t expert_bytes;
    // ids checked in the kernel (id_total pairs), x the one shared f32
    // column; zero_pair: this workgroup's pair has id -1 (set by mv_enter)
    uint32_t id_inline, id_total, zero_pair;
    // Model-runtime checks (Matrix::multiply, the decode step): a nonzero chk
    // packs five 5-bit ModelStage ids (MvChk order; 0 = that check is off)
    // and every data error becomes a model_key of layer chk_layer; chk 0
    // keeps the quantizers' own QuantError keys
    uint32_t chk, chk_layer;
    // The batch-1 kernel's balanced deal over this many CUs (0: the tiles
    // are grid-strided)
    uint32_t deal_cus;
};

// the fields of chk, in the order of mv_chk's arguments
enum MvChk : int { kChkScale = 0, kChkIn = 1, kChkQuant = 2, kChkOut = 3, kChkResid = 4 };
__device__ __forceinline__ uint32_t chk_stage(const MvArgs& a, int f) { return (a.chk >> (5 * f)) & 31u; }

// Keys of the quantizer's data errors: QuantError keys of column
// err_column0 + b, or the model stages of the input check and the scale.
__device__ __forceinline__ uint64_t quant_nonfinite_key(const MvArgs& a, uint32_t b, uint64_t index) {
    return a.chk ? model_key(a.chk_layer, chk_stage(a, kChkIn), 0) : error_key(a.err_column0 + b, kKindNonFinite, index);
}
__device__ __forceinline__ uint64_t quant_scale_key(const MvArgs& a, uint32_t b, uint64_t block) {
    return a.chk ? model_key(a.chk_layer, chk_stage(a, kChkQuant), block) : error_key(a.err_column0 + b, kKindScale, block);
}
__device__ __forceinline__ uint64_t rms_scale_key(const MvArgs& a) {
    return a.chk ? model_key(a.chk_layer, chk_stage(a, kChkScale), 0) : error_key(a.err_column0, kKindNonFinite, 0);
}
// finite(&output, ...) of a model check stage (math.rs:181-187)
__device__ __forceinline__ void check_finite(const MvArgs& a, int f, float v) {
    const uint32_t st = chk_stage(a, f);
    if (st && !finite(v)) report_error(a.err_word, model_key(a.chk_layer, st, 0));
}

// Kernel entry: false when the workgroup has nothing to do (a refused call,
// an expert slot with id -1, whose outputs the prepare kernel zeroed).  With
// id_inline every workgroup checks every id first (the reference checks them
// all before it quantizes anything, crates/tensor/src/cpu_index.rs:197-202):
// one out of [-1, experts) refuses the call, the first is reported as
// TensorError::Bounds; a -1 pair goes on (to quantize the shared column and
// refuse with the others if it is bad) and then writes zeros.
__device__ __forceinline__ bool mv_enter(MvArgs& a) {
    if (a.gate && *a.gate) return false;
    if (!a.ids) return true;
    if (a.id_inline) {
        int bad = 0;
        for (uint32_t i = threadIdx.x; i < a.id_total; i += blockDim.x) {
            const int32_t id = a.ids[i];
            bad |= id < -1 || id >= (int32_t)a.id_experts;
        }
        if (__syncthreads_or(bad)) {
            if (a.id_base == 0 && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
                uint32_t first = 0;
                while (first < a.id_total && a.ids[first] >= -1 && a.ids[first] < (int32_t)a.id_experts) ++first;
                report_error(a.err_word, bounds_key(first));
            }
            return false;
        }
        const uint32_t pair = a.id_base + blockIdx.y;
        const int32_t id = a.ids[pair];
        a.zero_pair = id < 0;
        if (id >= 0) a.w += (uint64_t)id * a.expert_bytes;
        a.y += (uint64_t)pair * a.ldy;
        return true;
    }
    const uint32_t pair = a.id_base + blockIdx.y;
    const int32_t id = a.ids[pair];
    if (id < 0 || (uint32_t)id >= a.id_experts) return false;
    const uint32_t token = pair / a.id_slots, slot = pair % a.id_slots;
    const uint64_t col = (uint64_t)token * a.id_cols + slot % a.id_cols;
    const uint32_t nb = a.nb;
    a.w += (uint64_t)id * a.expert_bytes;
    a.pre.q += col * a.cols;
    a.pre.d += col * nb;
    a.pre.bad += col * nb;
    if (a.pre.bsum) a.pre.bsum += col * (a.cols / 16);
    a.y += (uint64_t)pair * a.ldy;
    a.err_column0 = (uint32_t)col;
    return true;
}

// LDS: q8 [batch][S] | d f32 [nb][8] | (Q2_K, Q4_K, Q5_K) bsums i16 [nb][8][16] | 256
// zero bytes | 16 f64 (the RMSNorm reduction of the input transform).  S = cols + 16 is an odd multiple of 16, so the A-operand reads
// of the eight columns fall in distinct banks.  Lanes whose MFMA A operand is
// all zero read the zero bytes instead of taking a branch.
struct LdsMap {
    uint32_t S, d_off, bs_off, zero_off, red_off, am_off, total;
};

__host__ __device__ inline LdsMap lds_map(uint32_t t, uint32_t cols, uint32_t batch) {
    LdsMap m;
    const uint32_t nb = cols / (t == kQ8_0 ? 32 : 256);
    m.S = cols + 16;
    m.d_off = (m.S * batch + 15u) & ~15u;
    m.bs_off = m.d_off + nb * 32;
    m.zero_off = m.bs_off + (t == kQ4_K || t == kQ5_K || t == kQ2_K ? nb * 256 : 0);
    m.red_off = m.zero_off + 256;  // f64 row sums of the RMSNorm: [wave][4], up to 16 waves
    m.am_off = m.red_off + 512;    // argmax: 8 u64 keys, then the last-workgroup flag
    m.total = m.am_off + 80;
    return m;
}

// Q4_K / Q5_K bsums of one (block, column) are stored in the order [kq][4]:
// K quarter kq = 2g + h finds the 16-value groups it multiplies (half h of
// sub-blocks 2g, 2g+1, 2g+4, 2g+5) in one 8-byte word.  Slot of group
// grp = 2 * sub + half.  Q2_K keeps the natural order (slot = group).
__device__ __forceinline__ uint32_t bs_slot(uint32_t grp) {
    const uint32_t sub = grp >> 1, half = grp & 1;
    return (2 * ((sub >> 1) & 1) + half) * 4 + (sub & 1) + 2 * (sub >> 2);
}
// kBsOne / kBsOneCompact: the one-column Q4_K / Q5_K kernels' image
// (store_one_unit, expanded or compact)
enum BsumOrder { kBsNone = 0, kBsQuarters = 1, kBsNatural = 2, kBsOne = 3, kBsOneCompact = 4 };
__host__ __device__ constexpr int bsum_order(uint32_t t) {
    return t == kQ4_K || t == kQ5_K ? kBsQuarters : (t == kQ2_K ? kBsNatural : kBsNone);
}

// The activation image of the one-column Q4_K / Q5_K kernels.  Expanded
// (lds_map of four columns' room): every 4-byte word k of the slot-order
// Q8_K image (q45_slots) in a 16-byte record of its own at 16 k, at word
// position k % 4, the other 12 bytes zero, so one 16-byte read yields an MFMA
// A operand that is zero outside one lane class (q45_one_ints); compact: the
// slot-order image itself, masked in registers.  Per block, the eight
// sub-block sums of q8 (i16) at bs_off + 16 blk.  A lane pair (r16, r16 ^ 1)
// stores the 16 slot bytes v and the bsum of unit r16 of block blk.
__device__ __forceinline__ void store_one_unit(uint8_t* lds, const LdsMap& L, uint32_t blk, uint32_t r16, uint4 v,
                                               int32_t bsum, bool exp) {
    if (exp) {
        uint8_t* p = lds + blk * 1024 + r16 * 64;
        *(uint4*)(p) = make_uint4(v.x, 0u, 0u, 0u);
        *(uint4*)(p + 16) = make_uint4(0u, v.y, 0u, 0u);
        *(uint4*)(p + 32) = make_uint4(0u, 0u, v.z, 0u);
        *(uint4*)(p + 48) = make_uint4(0u, 0u, 0u, v.w);
    } else {
        *(uint4*)(lds + blk * 256 + r16 * 16) = v;
    }
    const int32_t sub = bsum + dpp_i<kQuadXor1>(bsum);  // both halves of the sub-block
    if ((r16 & 1) == 0) *(int16_t*)(lds + L.bs_off + blk * 16 + r16) = (int16_t)sub;
}

// ---------------------------------------------------------------------------
// Prologue: activations into LDS
// ---------------------------------------------------------------------------

// The activations are quantized in 16-value units (one Q8_K bsum group, half
// a Q8_0 block): unit u of the launch is column u / (cols/16), values
// 16 * (u % (cols/16)) ..; wave w takes units 64 (w + k W) + lane.
__device__ __forceinline__ void load_unit(const MvArgs& a, uint32_t u, float (&v)[16]) {
    const uint32_t upc = a.cols / 16;
    const float4* src = (const float4*)(a.x + (uint64_t)(u / upc) * a.cols + (u % upc) * 16);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 f = src[k];
        v[4 * k] = f.x, v[4 * k + 1] = f.y, v[4 * k + 2] = f.z, v[4 * k + 3] = f.w;
    }
}

// This lane's first unit, loaded before the weight prefetch: loads retire in
// order, so the quantizer's wait for x does not also wait for the weights.
__device__ __forceinline__ void prefetch_unit(const MvArgs& a, uint32_t wave, float (&v)[16]) {
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = 0.0f;
    const uint32_t u = wave * 64 + (threadIdx.x & 63);
    if (a.x && u < (a.cols / 16) * a.batch) load_unit(a, u, v);
}

// Input transforms of the decode step, applied to the f32 input before it is
// quantized (batch 1):
//   kXfRmsNorm   x * scale * norm_w with scale = 1 / sqrt(f32(sum x^2 / K) + eps),
//                the squares summed in f64 (crates/model-runtime/src/math.rs:214-228)
//   kXfSiluMul   silu(g) * u over x = [g (K values) | u (K values)]
//                (crates/model-runtime/src/llama.rs:367-371, SiLU of
//                crates/quant/src/cpu_math.rs:28-53)
enum MvXform : uint32_t { kXfNone = 0, kXfRmsNorm = 1, kXfSiluMul = 2 };
enum MvEpilogue : uint32_t { kEpStore = 0, kEpSiluPair = 1 };

__device__ __forceinline__ void load16(const float* p, float (&v)[16]) {
    const float4* src = (const float4*)p;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 f = src[k];
        v[4 * k] = f.x, v[4 * k + 1] = f.y, v[4 * k + 2] = f.z, v[4 * k + 3] = f.w;
    }
}

// RMSNorm scale of the launch's single input column: every lane adds the
// squares of its own units in f64, the wave sums are parked in LDS and every
// thread adds them in wave order, so all threads hold the same value.  The
// reference adds the squares one after another (math.rs:216); two orders of
// the same n nonnegative f64 terms differ by at most 2 (n - 1) 2^-53 of their
// sum, so when both ends of that interval give the same f32 mean, the
// reference's mean is that f32 too.  Otherwise (rare: an interval that
// straddles an f32 rounding boundary) thread 0 repeats the sum in the
// reference's order.
template <int W>
__device__ __forceinline__ float rms_scale(const MvArgs& a, uint8_t* lds, const LdsMap& L, uint32_t wave,
                                           const float (&v0)[16]) {
    const uint32_t units = a.cols / 16, lane = threadIdx.x & 63;
    double ss = 0.0;
    for (uint32_t base = wave * 64; base < units; base += W * 64) {
        const uint32_t u = base + lane;
        if (u >= units) continue;
        float v[16];
        if (base == wave * 64) {
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = v0[k];
        } else {
            load_unit(a, u, v);
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) ss += (double)(v[k] * v[k]);
    }
    ss = row16_sum_f64(ss);
    double* red = (double*)(lds + L.red_off);
    if ((lane & 15) == 0) red[wave * 4 + (lane >> 4)] = ss;
    __syncthreads();
    double total = 0.0;
#pragma unroll
    for (int w = 0; w < 4 * W; ++w) total += red[w];
    const double n = (double)a.cols, err = n * 2.3e-16 * total;  // 2^-52 n sum, with a margin
    if ((float)((total - err) / n) != (float)((total + err) / n)) {  // every thread takes the same branch
        __syncthreads();  // every thread has read red[]
        if (threadIdx.x == 0) {
            double seq = 0.0;
            for (uint32_t i = 0; i < a.cols; ++i) seq += (double)(a.x[i] * a.x[i]);
            red[0] = seq;
        }
        __syncthreads();
        total = red[0];
    }
    return 1.0f / sqrtf((float)(total / n) + a.eps);
}

// The input transform of the decode step, applied to the 16 values of unit u
// (element e0 of the launch's single column) before they are quantized.
__device__ __forceinline__ void apply_xform(const MvArgs& a, uint32_t e0, float scale, float (&v)[16]) {
    if (a.xform == kXfRmsNorm) {
        float w[16];
        load16(a.norm_w + e0, w);
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = v[k] * scale * w[k];
    } else if (a.xform == kXfSiluMul) {
        float up[16];
        load16(a.x + a.cols + e0, up);
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = (v[k] / (1.0f + sse2_exp(0.0f - v[k]))) * up[k];
    }
}

// Q8_K of all batch columns into LDS.  A 16-lane row quantizes one 256-value
// block, 16 values per lane (one bsum group per lane).  Returns false in
// every thread when any block of any column is invalid.
template <int W, int BSUMS>
__device__ __forceinline__ bool stage_q8k(const MvArgs& a, uint8_t* lds, const LdsMap& L, uint32_t wave, const float (&v0)[16]) {
    const uint32_t K = a.cols, upc = K / 16, units = upc * a.batch;
    const uint32_t lane = threadIdx.x & 63, r16 = lane & 15;
    int bad = 0;
    float scale = 1.0f;
    if (a.xform == kXfRmsNorm) {
        scale = rms_scale<W>(a, lds, L, wave, v0);
        if (!(scale <= 3.402823466e38f) || !(scale > 0.0f)) {  // math.rs:218-220
            bad = 1;
            if (threadIdx.x == 0) report_error(a.err_word, rms_scale_key(a));
        }
    }
    for (uint32_t base = wave * 64; base < units; base += W * 64) {
        const uint32_t u = base + lane;
        if (u >= units) continue;  // whole 16-lane rows drop out together (units % 16 == 0)
        const uint32_t b = u / upc, e0 = (u % upc) * 16, blk = e0 / 256;
        float v[16];
        if (base == wave * 64) {
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = v0[k];
        } else {
            load_unit(a, u, v);
        }
        apply_xform(a, e0, scale, v);
        const Q8KRow o = q8k_row16(v, r16);
        if (o.kind >= 0) {
            bad = 1;
            if (r16 == 0)
                report_error(a.err_word, o.kind == kKindNonFinite ? quant_nonfinite_key(a, b, blk * 256ull + o.index)
                                                                  : quant_scale_key(a, b, blk));
        }
        if (BSUMS == kBsOne || BSUMS == kBsOneCompact)  // (one column)
            store_one_unit(lds, L, blk, r16, q45_slots(o.q, r16 & 1), o.bsum, BSUMS == kBsOne);
        else
            *(uint4*)(lds + b * L.S + e0) =
                BSUMS == kBsQuarters ? q45_slots(o.q, r16 & 1) : make_uint4(o.q[0], o.q[1], o.q[2], o.q[3]);
        if (r16 == 0) *(float*)(lds + L.d_off + (blk * 8 + b) * 4) = o.d;
        if (BSUMS != kBsNone && BSUMS != kBsOne && BSUMS != kBsOneCompact)
            *(int16_t*)(lds + L.bs_off + (blk * 8 + b) * 32 + (BSUMS == kBsQuarters ? bs_slot(r16) : r16) * 2) =
                (int16_t)o.bsum;
    }
    return __syncthreads_or(bad) == 0;
}

template <int W>
__device__ __forceinline__ bool stage_q8_0(const MvArgs& a, uint8_t* lds, const LdsMap& L, uint32_t wave, const float (&v0)[16]) {
    const uint32_t K = a.cols, upc = K / 16, units = upc * a.batch;
    const uint32_t lane = threadIdx.x & 63;
    int bad = 0;
    float scale = 1.0f;
    if (a.xform == kXfRmsNorm) {
        scale = rms_scale<W>(a, lds, L, wave, v0);
        if (!(scale <= 3.402823466e38f) || !(scale > 0.0f)) {  // math.rs:218-220
            bad = 1;
            if (threadIdx.x == 0) report_error(a.err_word, rms_scale_key(a));
        }
    }
    for (uint32_t base = wave * 64; base < units; base += W * 64) {
        const uint32_t u = base + lane;
        if (u >= units) continue;  // lane pairs drop out together (units is even)
        const uint32_t b = u / upc, e0 = (u % upc) * 16, blk = e0 / 32, half = (e0 / 16) & 1u;
        float v[16];
        if (base == wave * 64) {
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = v0[k];
        } else {
            load_unit(a, u, v);
        }
        apply_xform(a, e0, scale, v);
        uint32_t nf = 0xffffffffu;
#pragma unroll
        for (int k = 15; k >= 0; --k)
            if (!finite(v[k])) nf = half * 16 + k;
        nf = umin_(nf, (uint32_t)dpp_i<kQuadXor1>((int32_t)nf));
        const bool nonfinite = nf != 0xffffffffu;
        // scales(): amax = fold(0, max(a, |v|)); d = amax / 127
        float am = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) am = fmaxf(am, fabsf(v[k]));
        am = fmaxf(am, dpp_f<kQuadXor1>(am));
        const float d = nonfinite ? 0.0f : am / 127.0f;
        const uint32_t dh = float_to_half_bits(d);
        // preflight (encode.rs:80-90): d, 1/d and the stored half must be finite
        const bool scale_bad =
            !nonfinite && (!finite(d) || (d != 0.0f && !finite(1.0f / d)) || (dh & 0x7c00u) == 0x7c00u);
        const bool invalid = nonfinite || scale_bad;
        if (invalid) {
            bad = 1;
            if (half == 0)
                report_error(a.err_word, nonfinite ? quant_nonfinite_key(a, b, blk * 32ull + nf)
                                                   : quant_scale_key(a, b, blk));
        }
        const float inv = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t qw[4] = {0, 0, 0, 0};
        if (!invalid) {
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                // `(x * inv).round() as i8`: half away from zero, saturating
                float r = __builtin_roundf(v[k] * inv);
                r = r > 127.0f ? 127.0f : (r < -128.0f ? -128.0f : r);
                qw[k / 4] |= ((uint32_t)(int32_t)r & 0xffu) << (8 * (k % 4));
            }
        }
        *(uint4*)(lds + b * L.S + e0) = make_uint4(qw[0], qw[1], qw[2], qw[3]);
        if (half == 0) *(float*)(lds + L.d_off + (blk * 8 + b) * 4) = half_bits_to_float_exact(dh);
    }
    return __syncthreads_or(bad) == 0;
}

// Pre-quantized activations (planes in global memory) into LDS; one: the
// one-column Q4_K / Q5_K image (store_one_unit, expanded when exp).
template <int W>
__device__ __forceinline__ bool stage_planes(const MvArgs& a, uint8_t* lds, const LdsMap& L, uint32_t wtype,
                                             bool one = false, bool exp = false) {
    const uint32_t K = a.cols, bs = wtype == kQ8_0 ? 32 : 256, nb = K / bs;
    const uint32_t tid = threadIdx.x, nt = W * 64;
    const bool slots = wtype == kQ4_K || wtype == kQ5_K;
    for (uint32_t i = tid; i < a.batch * (K / 16); i += nt) {  // lane pairs hold unit pairs (i, i ^ 1)
        const uint32_t b = i / (K / 16), e = (i % (K / 16)) * 16;
        const uint4 v = *(const uint4*)(a.pre.q + (uint64_t)b * K + e);
        const uint32_t q[4] = {v.x, v.y, v.z, v.w};
        if (one) store_one_unit(lds, L, e / 256, (e % 256) / 16, q45_slots(q, i & 1), a.pre.bsum[i], exp);
        else *(uint4*)(lds + b * L.S + e) = slots ? q45_slots(q, i & 1) : v;
    }
    int bad = 0;
    for (uint32_t i = tid; i < a.batch * nb; i += nt) {
        const uint32_t b = i / nb, blk = i % nb;
        *(float*)(lds + L.d_off + (blk * 8 + b) * 4) = a.pre.d[i];
        bad |= a.pre.bad[i];
    }
    const int order = bsum_order(wtype);
    if (order != kBsNone && !one) {
        for (uint32_t i = tid; i < a.batch * (K / 16); i += nt) {
            const uint32_t b = i / (K / 16), g = i % (K / 16);
            const uint32_t slot = order == kBsQuarters ? bs_slot(g % 16) : g % 16;
            *(int16_t*)(lds + L.bs_off + ((g / 16) * 8 + b) * 32 + slot * 2) = a.pre.bsum[i];
        }
    }
    return __syncthreads_or(bad) == 0;
}

// The planes of a K-format launch loaded before its weights, when they fit
// kPlaneRegs uint4 of q8 per thread (batch * cols <= 64 W * 16 kPlaneRegs):
// every staging load then precedes the weight loads, so its wait does not
// wait for them (loads retire in order).  One float of d, one flag byte and
// four bsums per thread.
constexpr uint32_t kPlaneRegs = 4;
struct PlanePrefetch {
    uint4 q[kPlaneRegs];
    float d;
    uint32_t bad;
    uint2 bs;
};
__host__ __device__ inline bool planes_fit(uint32_t threads, uint32_t batch, uint32_t cols, uint32_t nb) {
    return batch * (cols / 16) <= kPlaneRegs * threads && batch * nb <= threads;
}
template <int W>
__device__ __forceinline__ void prefetch_planes(const MvArgs& a, PlanePrefetch& p) {
    const uint32_t tid = threadIdx.x, K = a.cols, upc = K / 16, units = a.batch * upc;
#pragma unroll
    for (uint32_t r = 0; r < kPlaneRegs; ++r) {
        const uint32_t i = tid + r * W * 64;
        p.q[r] = i < units ? *(const uint4*)(a.pre.q + (uint64_t)(i / upc) * K + (i % upc) * 16) : make_uint4(0, 0, 0, 0);
    }
    p.d = 0.0f;
    p.bad = 0;
    if (tid < a.batch * a.nb) {
        p.d = a.pre.d[tid];
        p.bad = a.pre.bad[tid];
    }
    p.bs = tid < units / 4 ? *(const uint2*)(a.pre.bsum + 4 * tid) : make_uint2(0, 0);
}
// stage_planes from the prefetched registers (Q8_K planes of Q4_K / Q5_K:
// the slot order and quarter-ordered bsums)
template <int W>
__device__ __forceinline__ bool stage_planes_prefetched(const MvArgs& a, uint8_t* lds, const LdsMap& L,
                                                        const PlanePrefetch& p) {
    const uint32_t tid = threadIdx.x, K = a.cols, upc = K / 16, units = a.batch * upc, nb = a.nb;
#pragma unroll
    for (uint32_t r = 0; r < kPlaneRegs; ++r) {
        const uint32_t i = tid + r * W * 64;
        const uint32_t q[4] = {p.q[r].x, p.q[r].y, p.q[r].z, p.q[r].w};
        const uint4 v = q45_slots(q, tid & 1);  // (both lanes of a pair, before the bound)
        if (i < units) *(uint4*)(lds + (i / upc) * L.S + (i % upc) * 16) = v;
    }
    if (tid < a.batch * nb) *(float*)(lds + L.d_off + ((tid % nb) * 8 + tid / nb) * 4) = p.d;
    if (tid < units / 4) {
        const int16_t v[4] = {(int16_t)p.bs.x, (int16_t)(p.bs.x >> 16), (int16_t)p.bs.y, (int16_t)(p.bs.y >> 16)};
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) {
            const uint32_t i = 4 * tid + k, b = i / upc, g = i % upc;
            *(int16_t*)(lds + L.bs_off + ((g / 16) * 8 + b) * 32 + bs_slot(g % 16) * 2) = v[k];
        }
    }
    return __syncthreads_or(p.bad != 0) == 0;
}

// ---------------------------------------------------------------------------
// Per-tile epilogue shared by the three kernels: store y and fold the argmax.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void store_out(const MvArgs& a, uint32_t row, uint32_t b, float v,
                                          unsigned long long& best) {
    if (row < a.rows && b < a.batch) {
        const uint64_t i = (uint64_t)b * a.ldy + row;
        if (a.chk) check_finite(a, kChkOut, v);
        if (a.resid) v = a.resid[i] + v;  // math.rs:203-208: hidden += projected
        if (a.chk) check_finite(a, kChkResid, v);
        a.y[i] = v;
        const unsigned long long k = argmax_key(v, row);
        best = k > best ? k : best;
    }
}

// The argmax keys of a workgroup: every lane's best key of column b folded
// (max over its 16-lane row, then an LDS max) into the workgroup's key.
__device__ __forceinline__ void fold_argmax(const MvArgs& a, uint8_t* lds, const LdsMap& L, uint32_t b,
                                            unsigned long long best) {
    if (!a.am_out) return;
    best = row16_max_u64(best);
    if ((threadIdx.x & 15) == 0 && b < a.batch && best) atomicMax((unsigned long long*)(lds + L.am_off) + b, best);
}

// The end of every decode kernel that takes an argmax (every thread of the
// workgroup calls it, after its last fold).  Each workgroup writes its keys to
// its own slot with agent-scope atomic exchanges, waits for them, and then
// counts itself in; the last workgroup to arrive reads every slot, writes the
// token ids and sets the counter back to 0.  All cross-workgroup data moves
// through agent-scope atomics (coherent across the device's L2s), so no cache
// write-back is needed.  The two round trips lengthen every workgroup's tail
// (Q8_0 151936x896: about 4 us of a 31 us launch); sixteen group counters in
// place of the one measured the same, so the time is the round trips, not
// contention on the counter.
//
// The ordering of the slot exchanges before the count rests on the hardware,
// not on a release/acquire pair of the memory model: each exchanging thread
// waits for its exchange's returned value (an atomic returns once it has been
// performed at the device-coherent level), then the workgroup barrier, then
// the count.  A release on the count is what the model asks for, but on
// gfx950 it writes the workgroup's whole L2 back (buffer_wbl2): measured, the
// Q8_0 151936x896 argmax launch went from 30.8 to 50.0 us and Q6_K 128256x4096
// batch 8 from 82.2 to 83.6 us.  The argmax tests over every kernel and
// batch size guard the assumption.
__device__ __forceinline__ void finish_argmax(const MvArgs& a, uint8_t* lds, const LdsMap& L) {
    if (!a.am_out) return;
    unsigned long long* keys = (unsigned long long*)(lds + L.am_off);
    int* last = (int*)(keys + 8);
    const uint32_t tid = threadIdx.x, nt = blockDim.x, G = gridDim.x;
    __syncthreads();
    if (tid < a.batch) {
        const unsigned long long old = __hip_atomic_exchange(a.am_slots + (uint64_t)blockIdx.x * a.batch + tid,
                                                             keys[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __asm__ volatile("" : : "v"(old));  // the exchange has been performed before the count below
    }
    __syncthreads();
    if (tid == 0)
        *last = __hip_atomic_fetch_add(a.am_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1;
    __syncthreads();
    if (!*last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const uint32_t nbat = a.batch;
    if ((nbat & (nbat - 1)) == 0) {
        // batch 1, 2, 4 or 8: the G * batch slot keys (slot w * batch + b)
        // eight per thread at a time, every one of them column tid % batch
        // (blockDim is a multiple of 64); the eight loads are issued before
        // any key is compared, so the pass costs one global round trip per
        // 8 * blockDim keys, not one per key a thread reads (the maximum does
        // not depend on the order)
        const uint32_t total = G * nbat;
        unsigned long long v = 0;
        if (total <= nt) {  // at most one key per thread
            if (tid < total) v = __hip_atomic_load(a.am_slots + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            for (uint32_t i0 = tid; i0 < total; i0 += 8 * nt) {
                unsigned long long k[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint32_t i = i0 + u * nt;
                    k[u] = i < total ? __hip_atomic_load(a.am_slots + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                     : 0ull;
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) v = k[u] > v ? k[u] : v;
            }
        }
        // lanes of one column are those with the same lane % batch
        for (uint32_t m = nbat; m < 64; m <<= 1) {
            const unsigned long long o = __shfl_xor(v, m, 64);
            v = o > v ? o : v;
        }
        if ((tid & 63) < nbat && v) atomicMax(keys + (tid & 63), v);
    } else {
        for (uint32_t b = 0; b < nbat; ++b) {
            unsigned long long best = 0;
            for (uint32_t w = tid; w < G; w += nt) {
                const unsigned long long k = __hip_atomic_load(a.am_slots + (uint64_t)w * nbat + b, __ATOMIC_RELAXED,
                                                               __HIP_MEMORY_SCOPE_AGENT);
                best = k > best ? k : best;
            }
#pragma unroll
            for (int m = 1; m < 64; m <<= 1) {
                const unsigned long long o = __shfl_xor(best, m, 64);
                best = o > best ? o : best;
            }
            if ((tid & 63) == 0 && best) atomicMax(keys + b, best);
        }
    }
    __syncthreads();
    if (tid < a.batch) {
        const unsigned long long k = keys[tid];
        a.am_out[tid] = k == 0 ? 0u : (uint32_t)(0xffffffffull - (k & 0xffffffffull));
    }
    if (tid == 0) __hip_atomic_store(a.am_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// MUL_MAT_ID slot with id -1 (cpu_index.rs:204), once the call is known to
// stand: the rows this workgroup would have computed are 0.  One wave per
// tile (tiles gw, gw + tw, ...), or tile slots of the K-split kernels.
__device__ __forceinline__ void zero_wave_tiles(const MvArgs& a, uint32_t gw, uint32_t tw, uint32_t n, uint32_t kq) {
    for (uint32_t t = gw; t < a.ntiles; t += tw) {
        const uint32_t row = t * kTileRows + n;
        if (kq == 0 && row < a.rows) a.y[row] = 0.0f;
    }
}
template <int W, int TS>
__device__ __forceinline__ void zero_slot_tiles(const MvArgs& a, uint32_t tmax, uint32_t tstride) {
    for (uint32_t it = threadIdx.x; it < tmax * TS * 16; it += W * 64) {
        const uint32_t r = it % 16, slot = it / 16;
        const uint32_t t = blockIdx.x * TS + slot % TS + (slot / TS) * tstride, row = t * kTileRows + r;
        if (t < a.ntiles && row < a.rows) a.y[row] = 0.0f;
    }
}

// ---------------------------------------------------------------------------
// The balanced deal of the decode kernels: the tiles dealt out in equal
// shares of bytes per CU (otherwise they are grid-strided over the tile
// slots).  With C CUs, ntiles = u C / 2 (u half tiles a CU, 3 <= u <= 8) and
// k = grid / C workgroups of TS tile slots per CU, workgroup g = m C + c
// (m < k) fills slot j = TS m + ts of "CU" c: tile j C + c while j < u / 2,
// then for odd u rows 8 (c & 1) .. + 7 of tile (u / 2) C + c / 2, and nothing
// after.  In that half tile lane row n loads and computes row (n & 7) |
// 8 (c & 1), so lane pairs read the same bytes (one fetch), and only the
// lanes of the own half store.  With the dispatcher's k workgroups per CU (one
// of each m) every CU streams the same bytes; every row's sums are those of
// the grid-strided deal, bit for bit.
// ---------------------------------------------------------------------------
struct TileDeal {
    uint32_t tile;     // the slot's tile (one per slot)
    uint32_t count;    // 1, or 0 for an idle slot
    uint32_t half;     // 1: the tile is a half tile
    uint32_t hsel;     // its half: rows 8 hsel .. 8 hsel + 7
};
template <int TS>
__device__ __forceinline__ TileDeal balanced_deal(uint32_t C, uint32_t ntiles, uint32_t ts) {
    const uint32_t q = ntiles / C, cls = blockIdx.x / C, c = blockIdx.x - cls * C, j = TS * cls + ts;
    TileDeal d{0, 1, 0, 0};
    if (j < q) d.tile = j * C + c;
    else if (j == q && ntiles > q * C) d.tile = q * C + c / 2, d.half = 1, d.hsel = c & 1;
    else d.count = 0;
    return d;
}

// ---------------------------------------------------------------------------
// Software pipeline over a wave's steps: buf[i] holds the loads of step
// s0 + i, issued D steps before use.  The steady-state loop issues exactly one
// step's loads per step, so every path through it has the same loads in
// flight and the compiler's wait counts let D - 1 steps stay outstanding; the
// drain loop (at most two passes) issues only what remains.
// ---------------------------------------------------------------------------
template <int D, typename Step, typename Issue, typename Compute>
__device__ __forceinline__ void pipeline(uint32_t steps, Step (&buf)[D], Issue& issue, Compute& compute) {
    uint32_t s0 = 0;
    for (; s0 + 2 * D <= steps; s0 += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            const Step cur = buf[i];
            issue(buf[i]);
            compute(cur);
        }
    }
    for (; s0 < steps; s0 += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            if (s0 + i >= steps) break;
            const Step cur = buf[i];
            if (s0 + i + D < steps) issue(buf[i]);
            compute(cur);
        }
    }
}

// ---------------------------------------------------------------------------
// Q4_K and Q5_K (the same kernels; Q5_K adds the fifth bit from qh)
// ---------------------------------------------------------------------------
template <uint32_t T>
struct Q4Step {
    uint4 w0, w1, h;
};
template <>
struct Q4Step<kQ5_K> {
    uint4 w0, w1, h, qh;
};

// Chunk geometry of the two formats (rlq_layout.hpp).
template <uint32_t T>
struct Q45 {
    static constexpr uint32_t chunk = T == kQ5_K ? kQ5KChunk : kQ4KChunk;
    static constexpr uint32_t head = T == kQ5_K ? 2560 : 2048;
};

template <uint32_t T>
__device__ __forceinline__ void q45_issue(Q4Step<T>& st, const uint8_t* base, uint32_t lane, uint32_t n,
                                          uint32_t kq) {
    st.w0 = load_stream16(base + lane * 16);
    st.w1 = load_stream16(base + 1024 + lane * 16);
    st.h = load_stream16(base + Q45<T>::head + n * 16);
    if constexpr (T == kQ5_K) st.qh = load_stream16(base + 2048 + n * 32 + 16 * (kq & 1));
}

// Q5_K fifth bits of this lane's four nibble sets, as 0x10 per byte: qh byte
// 16h + i holds bit `sub` of element 32 sub + 16h + i; the lane's sets are
// sub-blocks 2g (w0 low), 2g+1 (w0 high), 2g+4 (w1 low), 2g+5 (w1 high),
// g = kq / 2 (matvec_extra.rs:257-262 with the Q5_K qh term).
struct Q5High {
    uint32_t l0[4], h0[4], l1[4], h1[4];
};
__device__ __forceinline__ Q5High q5_high(uint4 qh, uint32_t kq) {
    const uint32_t sh = 2 * (kq >> 1);
    const uint32_t q[4] = {qh.x >> sh, qh.y >> sh, qh.z >> sh, qh.w >> sh};
    Q5High o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o.l0[i] = (q[i] << 4) & 0x10101010u;
        o.h0[i] = (q[i] << 3) & 0x10101010u;
        o.l1[i] = q[i] & 0x10101010u;
        o.h1[i] = (q[i] >> 1) & 0x10101010u;
    }
    return o;
}

// Common kernel prologue: wave indices, the first x unit, the weight prefetch
// of steps 0..D-1 (clamped to the last tile, so it never leaves the buffer),
// and the activation staging.  `ld_tile`/`ld_chunk` track the next step to
// load: tile gw + k*tw, chunk c.
#define RLQ_MV_PROLOGUE(WT, CHUNKS)                                                                   \
    if (!mv_enter(a)) return;                                                                         \
    extern __shared__ __align__(16) uint8_t lds[];                                                    \
    const LdsMap L = lds_map(WT, a.cols, a.batch);                                                   \
    const uint32_t lane = threadIdx.x & 63, n = lane & 15, kq = lane >> 4;                            \
    /* wave-uniform indices in scalar registers: loop control stays on the SALU */                    \
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);                           \
    const uint32_t gw = blockIdx.x * W + wave, tw = gridDim.x * W;                                    \
    const uint32_t nch = (CHUNKS);                                                                    \
    const uint32_t steps = gw < a.ntiles ? ((a.ntiles - 1 - gw) / tw + 1) * nch : 0;                  \
    if (threadIdx.x < 16) *(uint4*)(lds + L.zero_off + threadIdx.x * 16) = make_uint4(0, 0, 0, 0);   \
    if (threadIdx.x < 8) ((unsigned long long*)(lds + L.am_off))[threadIdx.x] = 0ull;                 \
    float xv[16];                                                                                     \
    prefetch_unit(a, wave, xv);                                                                       \
    uint32_t ld_tile = gw < a.ntiles ? gw : a.ntiles - 1, ld_chunk = 0;                               \
    auto next_load = [&]() {                                                                          \
        if (++ld_chunk == nch) {                                                                      \
            ld_chunk = 0;                                                                             \
            if (ld_tile + tw < a.ntiles) ld_tile += tw;                                               \
        }                                                                                             \
    };

__device__ __forceinline__ int32_t mad24(int32_t a, int32_t b, int32_t c) { return __mul24(a, b) + c; }

// Scales and mins of sub-blocks j and j + 1 (j even) of a Q4_K block from its
// 12 packed bytes w1..w3 (matvec_extra.rs:212-221): for j < 4 the low six
// bits of bytes j, j+4; for j >= 4 four bits of byte j+4 and the top two bits
// of bytes j-4 / j.  As words: sc[0..3] = w1 & 0x3f.., mn[0..3] = w2 & 0x3f..,
// sc[4..7] = (w3 & 0x0f..) | ((w1 >> 2) & 0x30..), mn[4..7] =
// ((w3 >> 4) & 0x0f..) | ((w2 >> 2) & 0x30..), one value per byte.
struct Q4Scales {
    uint32_t scA, scB, mnA, mnB;
};
__device__ __forceinline__ Q4Scales q4k_scales(uint4 h) {
    Q4Scales q;
    q.scA = h.y & 0x3f3f3f3fu;
    q.scB = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
    q.mnA = h.z & 0x3f3f3f3fu;
    q.mnB = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
    return q;
}

// Decode kernels with DBG also store the exact per-(row, block) integers of
// column 0 (isum: the scaled sub-block dots; imin: the mins term).

// Exact integers of one chunk for this lane's row n and columns b0, b0 + 1:
// the scaled sub-block dots I and the mins sums M (matvec_extra.rs:252-262).
// The A operand: lane row r holds column r / 2, sub-block parity r % 2, and is
// nonzero only in the K quarters (kq / 2 == r % 2) of that sub-block; p is
// this lane's A row at the chunk's block, bs the columns' bsums of the block.
struct Q45Ints {
    int32_t I0, I1, M0, M1;
};
template <uint32_t T>
__device__ __forceinline__ Q45Ints q45_mfma_ints(const Q4Step<T>& cur, const uint8_t* p, const uint8_t* bs_blk_b0,
                                                 uint32_t kq) {
    const Q4Scales q = q4k_scales(cur.h);
    const i32x4 al0 = *(const i32x4*)(p), ah0 = *(const i32x4*)(p + 32);
    const i32x4 al1 = *(const i32x4*)(p + 128), ah1 = *(const i32x4*)(p + 160);
    i32x4 wl0 = lo_nibbles(cur.w0), wh0 = hi_nibbles(cur.w0);
    i32x4 wl1 = lo_nibbles(cur.w1), wh1 = hi_nibbles(cur.w1);
    if constexpr (T == kQ5_K) {
        const Q5High hb = q5_high(cur.qh, kq);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            wl0[i] |= (int)hb.l0[i];
            wh0[i] |= (int)hb.h0[i];
            wl1[i] |= (int)hb.l1[i];
            wh1[i] |= (int)hb.h1[i];
        }
    }
    // sub-blocks: dl0 {0, 2}, dh0 {1, 3}, dl1 {4, 6}, dh1 {5, 7}; element
    // 2j + w of each is column b0 + j, sub-block parity w
    const i32x4 dl0 = mfma_i8(al0, wl0);
    const i32x4 dh0 = mfma_i8(ah0, wh0);
    const i32x4 dl1 = mfma_i8(al1, wl1);
    const i32x4 dh1 = mfma_i8(ah1, wh1);
    const int32_t c0 = ubyte(q.scA, 0), c1 = ubyte(q.scA, 1), c2 = ubyte(q.scA, 2), c3 = ubyte(q.scA, 3);
    const int32_t c4 = ubyte(q.scB, 0), c5 = ubyte(q.scB, 1), c6 = ubyte(q.scB, 2), c7 = ubyte(q.scB, 3);
    Q45Ints o;
    // |dot| <= 32*31*128 and scales <= 63: 24-bit operands, exact products
    o.I0 = mad24(c0, dl0[0], mad24(c2, dl0[1], mad24(c1, dh0[0], __mul24(c3, dh0[1]))));
    o.I0 = mad24(c4, dl1[0], mad24(c6, dl1[1], mad24(c5, dh1[0], mad24(c7, dh1[1], o.I0))));
    o.I1 = mad24(c0, dl0[2], mad24(c2, dl0[3], mad24(c1, dh0[2], __mul24(c3, dh0[3]))));
    o.I1 = mad24(c4, dl1[2], mad24(c6, dl1[3], mad24(c5, dh1[2], mad24(c7, dh1[3], o.I1))));
    // mins: sum_s min_s * (bsum[2s] + bsum[2s+1])  (matvec_extra.rs:258)
    const uint32_t m01 = __builtin_amdgcn_perm(0u, q.mnA, 0x0c010c00u);
    const uint32_t m23 = __builtin_amdgcn_perm(0u, q.mnA, 0x0c030c02u);
    const uint32_t m45 = __builtin_amdgcn_perm(0u, q.mnB, 0x0c010c00u);
    const uint32_t m67 = __builtin_amdgcn_perm(0u, q.mnB, 0x0c030c02u);
    const uint4* bs = (const uint4*)bs_blk_b0;
    const uint4 bA0 = bs[0], bA1 = bs[1], bB0 = bs[2], bB1 = bs[3];
    o.M0 = dot2(m67, bA1.w, dot2(m23, bA1.z, dot2(m67, bA1.y, dot2(m23, bA1.x,
           dot2(m45, bA0.w, dot2(m01, bA0.z, dot2(m45, bA0.y, dot2(m01, bA0.x, 0))))))));
    o.M1 = dot2(m67, bB1.w, dot2(m23, bB1.z, dot2(m67, bB1.y, dot2(m23, bB1.x,
           dot2(m45, bB0.w, dot2(m01, bB0.z, dot2(m45, bB0.y, dot2(m01, bB0.x, 0))))))));
    return o;
}

// Q4_K / Q5_K, three to eight columns, K split over KS waves per tile: the
// MFMA step q45_mfma_ints, with a workgroup of W waves holding TS = W / KS
// tile slots and the waves of a slot taking blocks kp, kp + KS, ... of its
// tile (every SIMD holds several waves, the grid is a few hundred
// workgroups).  The columns are quantized by the whole workgroup (stage_q8k)
// while the first weight chunks load.  Lane (n, kq) holds the partial sums of
// row n, columns 2 kq and 2 kq + 1 of its K part; a tile's parts are parked
// in LDS [tmax][TS][KS][16][8] and counted with a workgroup-scope atomic, and
// the wave that completes the count adds them in K order after its last step
// (so no global store sits between its weight loads).
__host__ __device__ inline uint32_t ks_part_off(uint32_t T, uint32_t cols, uint32_t batch) {
    return (lds_map(T, cols, batch).total + 15u) & ~15u;
}
__host__ __device__ inline uint32_t ks_lds_bytes(uint32_t T, uint32_t cols, uint32_t batch, uint32_t tmax, uint32_t ts,
                                                 uint32_t ks) {
    return ks_part_off(T, cols, batch) + tmax * ts * ks * 16u * 8u * 4u + tmax * ts * 4u;
}

// PL: planes input that fits the prefetch registers (prefetch_planes).
// BAL: the balanced deal over a.deal_cus CUs (balanced_deal; one matrix).
template <uint32_t T, int W, int KS, int D, bool DBG, bool PL, bool BAL = false>
__global__ __launch_bounds__(W * 64) void q45_mv_ks_kernel(MvArgs a) {
    constexpr int TS = W / KS;
    static_assert(!BAL || TS == 2 || TS == 4, "the balanced deal takes two or four tile slots");
    if (!mv_enter(a)) return;
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsMap L = lds_map(T, a.cols, a.batch);
    float* part = (float*)(lds + ks_part_off(T, a.cols, a.batch));
    const uint32_t lane = threadIdx.x & 63, n = lane & 15, kq = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t ts = wave / KS, kp = wave % KS;
    const uint32_t nb = a.nb, ntiles = a.ntiles;
    const uint32_t tstride = gridDim.x * TS, t0 = blockIdx.x * TS + ts;
    // this wave's tiles: tile_of(i) for i < my_tiles; half_ti the ordinal of
    // its half tile (none: ~0) and hsel its half (BAL: balanced_deal)
    uint32_t tmax, my_tiles, half_ti = ~0u, hsel = 0, bt = 0;
    if constexpr (BAL) {
        const TileDeal d = balanced_deal<TS>(a.deal_cus, ntiles, ts);
        tmax = 1, my_tiles = d.count, bt = d.tile, hsel = d.hsel;
        if (d.half) half_ti = 0;
    } else {
        tmax = (ntiles + tstride - 1) / tstride;
        my_tiles = t0 < ntiles ? (ntiles - 1 - t0) / tstride + 1 : 0;
    }
    auto tile_of = [&](uint32_t i) -> uint32_t {
        if constexpr (BAL) return bt;
        else return t0 + i * tstride;
    };
    auto own_row = [&](uint32_t i) { return i != half_ti || (n >> 3) == hsel; };
    const uint32_t nh = (n & 7) | (hsel << 3);
    const uint32_t bpt = kp < nb ? (nb - 1 - kp) / KS + 1 : 0;  // blocks of each tile this wave takes
    const uint32_t steps = my_tiles * bpt;
    const uint32_t nk = (uint32_t)KS < nb ? (uint32_t)KS : nb;  // waves of a tile that take blocks
    uint32_t* cnt = (uint32_t*)(part + tmax * TS * KS * 16 * 8);
    for (uint32_t i = threadIdx.x; i < tmax * TS; i += W * 64) cnt[i] = 0;
    if (threadIdx.x < 16) *(uint4*)(lds + L.zero_off + threadIdx.x * 16) = make_uint4(0, 0, 0, 0);
    if (threadIdx.x < 8) ((unsigned long long*)(lds + L.am_off))[threadIdx.x] = 0ull;
    float xv[16];
    PlanePrefetch pp;
    if constexpr (PL) prefetch_planes<W>(a, pp);
    else prefetch_unit(a, wave, xv);

    const uint32_t kp0 = kp < nb ? kp : nb - 1;
    uint32_t ld_tile = t0 < ntiles ? t0 : ntiles - 1, ld_blk = kp0;
    if constexpr (BAL) ld_tile = my_tiles ? bt : 0;
    Q4Step<T> buf[D];
    auto issue = [&](Q4Step<T>& st) {
        const uint8_t* base = a.w + ((uint64_t)ld_tile * nb + ld_blk) * Q45<T>::chunk;
        if (BAL && half_ti == 0) q45_issue<T>(st, base, kq * 16 + nh, nh, kq);  // the half tile
        else q45_issue<T>(st, base, lane, n, kq);
        ld_blk += KS;
        if (ld_blk >= nb) {
            ld_blk = kp0;
            if (!BAL && ld_tile + tstride < ntiles) ld_tile += tstride;
        }
    };
#pragma unroll
    for (int i = 0; i < D; ++i) issue(buf[i]);

    // the counters' zeros are in place with the activations (one barrier)
    bool ok;
    if constexpr (PL) ok = stage_planes_prefetched<W>(a, lds, L, pp);
    else ok = a.x ? stage_q8k<W, kBsQuarters>(a, lds, L, wave, xv) : stage_planes<W>(a, lds, L, T);
    if (!ok) return finish_argmax(a, lds, L);
    if (a.zero_pair) return zero_slot_tiles<W, TS>(a, tmax, tstride);

    // A operand: lane row r = n holds column r / 2, sub-block parity r % 2; it
    // is nonzero only in the K quarters (kq / 2 == r % 2) of that sub-block.
    const uint32_t ab = n >> 1, which = n & 1;
    const bool a_live = which == (kq >> 1) && ab < a.batch;
    const uint8_t* a_ptr = a_live ? lds + ab * L.S + 64 * which + 16 * (kq & 1) : lds + L.zero_off;
    const uint32_t a_step = a_live ? 256 : 0;
    const uint32_t b0 = 2 * kq;  // this lane's output columns b0, b0 + 1

    float acc0 = 0.0f, acc1 = 0.0f;
    uint32_t ti = 0, blk = kp, j = 0, tile = tile_of(0);
    auto compute = [&](const Q4Step<T>& cur) {
        const Q45Ints o = q45_mfma_ints<T>(cur, a_ptr + blk * a_step, lds + L.bs_off + (blk * 8 + b0) * 32, kq);
        const float2 da = *(const float2*)(lds + L.d_off + (blk * 8 + b0) * 4);
        const float dw = half_to_float(cur.h.x), dmw = half_to_float(cur.h.x >> 16);
        acc0 += (dw * da.x) * (float)o.I0 - (dmw * da.x) * (float)o.M0;
        acc1 += (dw * da.y) * (float)o.I1 - (dmw * da.y) * (float)o.M1;
        if (DBG && kq == 0) {
            const uint32_t row = tile * kTileRows + n;
            if (row < a.rows && own_row(ti)) {
                a.dbg_isum[(uint64_t)row * nb + blk] = o.I0;
                a.dbg_imin[(uint64_t)row * nb + blk] = o.M0;
            }
        }
        blk += KS;
        if (++j == bpt) {  // this wave's share of the tile is done: park its sums
            const uint32_t slot = ti * TS + ts;
            *(float2*)(part + ((slot * KS + kp) * 16 + n) * 8 + b0) = make_float2(acc0, acc1);
            // one wave's LDS operations are performed in order: the partials
            // are in place before the count
            if (lane == 0) {
                const uint32_t prev =
                    __hip_atomic_fetch_add(cnt + slot, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
                if (prev == nk - 1) cnt[slot] = nk + 1 + wave;  // this wave finishes the tile
            }
            acc0 = acc1 = 0.0f;
            j = 0;
            blk = kp;
            tile = tile_of(++ti);
        }
    };
    pipeline<D>(steps, buf, issue, compute);

    // the tiles this wave completed: add their K parts in order and store
    unsigned long long best0 = 0, best1 = 0;
    for (uint32_t i = 0; i < my_tiles; ++i) {
        const uint32_t slot = i * TS + ts, row = tile_of(i) * kTileRows + n;
        if (cnt[slot] != nk + 1 + wave || !own_row(i)) continue;  // (the mark is wave-uniform)
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int k = 0; k < KS; ++k)
            if ((uint32_t)k < nk) {
                const float2 v = *(const float2*)(part + ((slot * KS + k) * 16 + n) * 8 + b0);
                s0 += v.x;
                s1 += v.y;
            }
        store_out(a, row, b0, s0, best0);
        store_out(a, row, b0 + 1, s1, best1);
    }
    fold_argmax(a, lds, L, b0, best0);
    fold_argmax(a, lds, L, b0 + 1, best1);
    finish_argmax(a, lds, L);
}

// ---------------------------------------------------------------------------
// The reference's f32 order for one column (matvec_extra.rs:223-294)
// ---------------------------------------------------------------------------
// The reference keeps eight f32 accumulators lanes[j % 8] over all blocks of
// a row: per block, integers[l] = the exact dot over the elements j with
// j % 8 == l, then (Q4_K / Q5_K) sum -= dmin * mins, then lanes[l] +=
// d * integers[l]; at the end sum += lanes[0], ..., lanes[7].  The one-column
// Q4_K / Q5_K kernels reproduce that sequence bit for bit: each block's eight
// terms d * integers[l] and its mins term dmin * mins are parked in LDS, and
// the row's sum is then formed in the reference's order (exact_row_sum).

// Sums over lane pairs l, l ^ 32 and l, l ^ 16 (v_permlane32_swap /
// v_permlane16_swap exchange the two halves, resp. adjacent 16-lane rows, of
// a value with itself), in every lane.
__device__ __forceinline__ int32_t sum_xor32(int32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    return (int32_t)(r[0] + r[1]);
}
__device__ __forceinline__ int32_t sum_xor16(int32_t v) {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    return (int32_t)(r[0] + r[1]);
}

// Parked terms per (tile slot, block): [4][16] float2, lane kq of row n
// holding classes 2 kq and 2 kq + 1, then [16] f32, the block's mins term of
// row n (the four lanes of a row store the same value).
constexpr uint32_t kParkBlockBytes = 4 * 16 * 8 + 16 * 4;
__host__ __device__ inline uint32_t park_bytes(uint32_t nb) { return nb * kParkBlockBytes; }

// The A operand of lane (r = n, kq) in the one-column MFMA step: A row r
// stands for lane class c = 2 (r / 4) + (r / 2) % 2 of sub-block parity
// g = r % 2 (sub-blocks 2g, 2g+1, 2g+4, 2g+5 of the four MFMAs).  The
// weights' K quarter kq holds sub-blocks 2 (kq / 2), ... at slots
// 16 (kq % 2) .., whose 4-byte word k holds class 4 (kq % 2) + k
// (rlq_layout.hpp), so the row is live in quarter kq = 2g + c / 4 only, with
// word c % 4 of that quarter's activation: one record of the expanded image
// (store_one_unit).  Output element i of lane (n, kq) is then the exact dot of
// weight row n over class 2 kq + i / 2 of the MFMA's sub-block of parity i % 2.
struct OneA {
    const uint8_t* p;           // this lane's A bytes at block 0 (the zero bytes when not live)
    uint32_t step, o1, o2, o3;  // per block; sub-blocks 2g+1, 2g+4, 2g+5
    uint32_t m[4];              // compact image: the word mask
};
__device__ __forceinline__ OneA one_a_operand(uint8_t* lds, const LdsMap& L, uint32_t n, uint32_t kq, bool exp) {
    const uint32_t c = 2 * (n >> 2) + ((n >> 1) & 1), g = n & 1;
    const bool live = kq == 2 * g + (c >> 2);
    const uint32_t O = 64 * (kq >> 1) + 16 * (kq & 1), x = exp ? 4u : 1u;
    OneA o;
    o.p = live ? lds + x * O + (exp ? 16 * (c & 3) : 0u) : lds + L.zero_off;
    o.step = live ? 256u * x : 0u;
    o.o1 = live ? x * 32u : 0u;
    o.o2 = live ? x * 128u : 0u;
    o.o3 = live ? x * 160u : 0u;
#pragma unroll
    for (uint32_t w = 0; w < 4; ++w) o.m[w] = live && w == (c & 3) ? ~0u : 0u;
    return o;
}

// The LDS operands of one chunk: the four A operands (masked in registers for
// the compact image), the block's sub-block sums and Q8_K scale.  a: the
// lane's A record at the block (one_a_operand).
struct OneLoads {
    i32x4 a0, a1, a2, a3;
    uint4 S;
    float da;
};
template <bool EXP>
__device__ __forceinline__ OneLoads one_loads(const OneA& A, const uint8_t* a, const uint8_t* ss, const uint8_t* dp) {
    auto aop = [&](const uint8_t* q) {
        const i32x4 v = *(const i32x4*)q;
        if constexpr (EXP) return v;
        else return i32x4{v[0] & (int)A.m[0], v[1] & (int)A.m[1], v[2] & (int)A.m[2], v[3] & (int)A.m[3]};
    };
    return OneLoads{aop(a), aop(a + A.o1), aop(a + A.o2), aop(a + A.o3), *(const uint4*)ss, *(const float*)dp};
}

// Exact integers of one Q4_K / Q5_K chunk for lane (n, kq): the reference's
// integers[2 kq] and integers[2 kq + 1] of row n over all eight sub-blocks,
// and the whole mins sum (matvec_extra.rs:252-270), from the chunk's LDS
// operands r.
struct Q45One {
    int32_t I0, I1, M;
};
template <uint32_t T>
__device__ __forceinline__ Q45One q45_one_ints(const Q4Step<T>& cur, const OneLoads& r, uint32_t kq) {
    typedef short s2 __attribute__((ext_vector_type(2)));
    const Q4Scales q = q4k_scales(cur.h);
    uint32_t l0[4] = {cur.w0.x & 0x0f0f0f0fu, cur.w0.y & 0x0f0f0f0fu, cur.w0.z & 0x0f0f0f0fu, cur.w0.w & 0x0f0f0f0fu};
    uint32_t h0[4], h1[4];
    hi_nibbles64(cur.w0, h0);
    uint32_t l1[4] = {cur.w1.x & 0x0f0f0f0fu, cur.w1.y & 0x0f0f0f0fu, cur.w1.z & 0x0f0f0f0fu, cur.w1.w & 0x0f0f0f0fu};
    hi_nibbles64(cur.w1, h1);
    if constexpr (T == kQ5_K) {
        const Q5High hb = q5_high(cur.qh, kq);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            l0[i] |= hb.l0[i];
            h0[i] |= hb.h0[i];
            l1[i] |= hb.l1[i];
            h1[i] |= hb.h1[i];
        }
    }
    auto vec = [](const uint32_t (&w)[4]) { return i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]}; };
    const i32x4 dl0 = mfma_i8(r.a0, vec(l0));
    const i32x4 dh0 = mfma_i8(r.a1, vec(h0));
    const i32x4 dl1 = mfma_i8(r.a2, vec(l1));
    const i32x4 dh1 = mfma_i8(r.a3, vec(h1));
    // scale pairs of the MFMAs' sub-blocks (0, 2), (1, 3), (4, 6), (5, 7) as
    // i16 pairs; a class's dots |.| <= 31 * 128 * 4 fit i16 as well
    const uint32_t s02 = __builtin_amdgcn_perm(0u, q.scA, 0x0c020c00u), s13 = __builtin_amdgcn_perm(0u, q.scA, 0x0c030c01u);
    const uint32_t s46 = __builtin_amdgcn_perm(0u, q.scB, 0x0c020c00u), s57 = __builtin_amdgcn_perm(0u, q.scB, 0x0c030c01u);
    auto pk = [](int32_t lo, int32_t hi) { return __builtin_bit_cast(s2, __builtin_amdgcn_perm((uint32_t)hi, (uint32_t)lo, 0x05040100u)); };
    auto cls = [&](int e) {
        int32_t I = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, s02), pk(dl0[2 * e], dl0[2 * e + 1]), 0, false);
        I = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, s13), pk(dh0[2 * e], dh0[2 * e + 1]), I, false);
        I = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, s46), pk(dl1[2 * e], dl1[2 * e + 1]), I, false);
        return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, s57), pk(dh1[2 * e], dh1[2 * e + 1]), I, false);
    };
    Q45One o;
    o.I0 = cls(0);
    o.I1 = cls(1);
    // mins: sum_s min_s * (bsum[2s] + bsum[2s+1]) over the block's sub-block sums
    const uint4 S = r.S;
    const uint32_t m01 = __builtin_amdgcn_perm(0u, q.mnA, 0x0c010c00u), m23 = __builtin_amdgcn_perm(0u, q.mnA, 0x0c030c02u);
    const uint32_t m45 = __builtin_amdgcn_perm(0u, q.mnB, 0x0c010c00u), m67 = __builtin_amdgcn_perm(0u, q.mnB, 0x0c030c02u);
    int32_t M = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, m01), __builtin_bit_cast(s2, S.x), 0, false);
    M = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, m23), __builtin_bit_cast(s2, S.y), M, false);
    M = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, m45), __builtin_bit_cast(s2, S.z), M, false);
    o.M = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, m67), __builtin_bit_cast(s2, S.w), M, false);
    return o;
}

// Park one block's terms of lane (n, kq): d * integers[2 kq], d *
// integers[2 kq + 1] (matvec_extra.rs:287-289, each product rounded to f32)
// and the mins term dmin * mins (:268).  pk: the slot's records (park_bytes).
__device__ __forceinline__ void park_terms(uint8_t* pk, uint32_t nb, uint32_t blk, uint32_t lane, float d,
                                           int32_t I0, int32_t I1, float mn) {
    ((float2*)pk)[blk * 64 + lane] = make_float2(d * (float)I0, d * (float)I1);
    ((float*)(pk + nb * 512))[blk * 16 + (lane & 15)] = mn;
}

// Lane n of 16-lane row 0 gets v of lane n + 16 r (r = 1, 2, 3); every lane
// of the wave must be active.
__device__ __forceinline__ float row_from(float v, int r) {
    const unsigned u = __float_as_uint(v);
    if (r == 1) return __uint_as_float(__builtin_amdgcn_permlane16_swap(u, u, false, false)[1]);
    if (r == 2) return __uint_as_float(__builtin_amdgcn_permlane32_swap(u, u, false, false)[1]);
    const unsigned r1 = __builtin_amdgcn_permlane16_swap(u, u, false, false)[1];  // rows 1, 1, 3, 3
    return __uint_as_float(__builtin_amdgcn_permlane32_swap(r1, r1, false, false)[1]);
}

// The row's f32 in the reference's order from its parked terms (nb blocks;
// pk the slot's records): lanes[l] over the blocks in order, sum minus the
// mins terms in order, then sum + lanes[0..7].  Lane kq = 0 of row n returns
// it (the other lanes return other sums); every lane of the wave must take
// part.
__device__ __forceinline__ float exact_row_sum(const uint8_t* pk, uint32_t nb, uint32_t lane) {
    const float2* p = (const float2*)pk + lane;                    // classes 2 kq, 2 kq + 1 of row n
    const float* q = (const float*)(pk + nb * 512) + (lane & 15);  // the mins terms
    float l0 = 0.0f, l1 = 0.0f, s = 0.0f;
    uint32_t b = 0;
    for (; b + 8 <= nb; b += 8) {  // eight blocks' loads before their adds
        float2 v[8];
        float m[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            v[k] = p[(b + k) * 64];
            m[k] = q[(b + k) * 16];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            l0 += v[k].x;
            l1 += v[k].y;
            s -= m[k];
        }
    }
    for (; b < nb; ++b) {
        const float2 v = p[b * 64];
        l0 += v.x;
        l1 += v.y;
        s -= q[b * 16];
    }
    // lane n of row 0 takes the rows' lanes n + 16 j in order j = 0..3 by lane
    // swaps (v_permlane16_swap brings row 1 to row 0, v_permlane32_swap rows 2
    // and 3): the order of the reference's lanes[0..7]
    const float a1 = row_from(l0, 1), a2 = row_from(l0, 2), a3 = row_from(l0, 3);
    const float b1 = row_from(l1, 1), b2 = row_from(l1, 2), b3 = row_from(l1, 3);
    s += l0;
    s += l1;
    s += a1;
    s += b1;
    s += a2;
    s += b2;
    s += a3;
    s += b3;
    return s;
}

// Q4_K / Q5_K, one column with a shared Q8_K image (the SiLU-pair epilogue,
// pre-quantized planes, MUL_MAT_ID pairs).
//
// A workgroup of W waves works on TS = W / KS tiles at a time; the KS waves of
// a tile take its blocks kp, kp + KS, ... (kp = the wave's K part), so a tile's
// bytes stream through KS waves and every SIMD holds several waves.  Lane
// (n, kq) gets the integers of lane classes 2 kq, 2 kq + 1 of row n from four
// MFMAs (q45_one_ints); every block's terms are parked in LDS, and after the
// last tile the workgroup forms each row's sum in the reference's order
// (exact_row_sum).
template <int W, int KS>
struct SmallGeom {
    static constexpr int TS = W / KS;
};

// LDS bytes of the small kernel: the activations (store_one_unit) plus the
// parked terms [tmax][TS][nb] (park_terms), tmax = tiles per (workgroup,
// tile slot).
// LDS of the one-column kernels: the image (expanded: 4 cols bytes), d f32
// [nb][8] (column 0 used), the sub-block sums [nb][8] i16, the zero bytes,
// the RMSNorm reduction and the argmax keys.
__host__ __device__ inline LdsMap lds_map_one(uint32_t t, uint32_t cols, bool exp) {
    LdsMap m;
    const uint32_t nb = cols / 256;
    m.S = 0;
    m.d_off = (exp ? 4u : 1u) * cols;
    m.bs_off = m.d_off + nb * 32;
    m.zero_off = m.bs_off + nb * 16;
    m.red_off = m.zero_off + 256;
    m.am_off = m.red_off + 512;
    m.total = m.am_off + 80;
    return m;
}
__host__ __device__ inline uint32_t one_part_off(uint32_t cols, bool exp) {
    return (lds_map_one(kQ4_K, cols, exp).total + 15u) & ~15u;
}
__host__ __device__ inline uint32_t small_lds_bytes(uint32_t cols, uint32_t tmax, uint32_t ts, bool exp) {
    return one_part_off(cols, exp) + tmax * ts * park_bytes(cols / 256);
}

// (two workgroups of 8 waves per CU: at most 128 VGPRs).  EXP: the expanded
// activation image (store_one_unit), else the compact one.
template <uint32_t T, int W, int KS, int D, bool DBG, bool EXP>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(4))) void q4k_mv_small_kernel(MvArgs a) {
    constexpr int TS = SmallGeom<W, KS>::TS;
    if (!mv_enter(a)) return;
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsMap L = lds_map_one(T, a.cols, EXP);
    const uint32_t lane = threadIdx.x & 63, n = lane & 15, kq = lane >> 4;
    // wave-uniform indices in scalar registers: loop control stays on the SALU
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t ts = wave / KS, kp = wave % KS;
    const uint32_t nb = a.nb, ntiles = a.ntiles;
    const uint32_t tstride = gridDim.x * TS, t0 = blockIdx.x * TS + ts;
    const uint32_t tmax = (ntiles + tstride - 1) / tstride;
    const uint32_t my_tiles = t0 < ntiles ? (ntiles - 1 - t0) / tstride + 1 : 0;
    const uint32_t bpt = kp < nb ? (nb - 1 - kp) / KS + 1 : 0;  // blocks of each tile this wave takes
    const uint32_t steps = my_tiles * bpt;
    uint8_t* park = lds + one_part_off(a.cols, EXP);

    if (threadIdx.x < 16) *(uint4*)(lds + L.zero_off + threadIdx.x * 16) = make_uint4(0, 0, 0, 0);
    if (threadIdx.x < 8) ((unsigned long long*)(lds + L.am_off))[threadIdx.x] = 0ull;
    float xv[16];
    prefetch_unit(a, wave, xv);

    // loads run D steps ahead; past the wave's last step they repeat a valid chunk
    const uint32_t kp0 = kp < nb ? kp : nb - 1;
    uint32_t ld_tile = t0 < ntiles ? t0 : ntiles - 1, ld_blk = kp0;
    Q4Step<T> buf[D];
    auto issue = [&](Q4Step<T>& st) {
        q45_issue<T>(st, a.w + ((uint64_t)ld_tile * nb + ld_blk) * Q45<T>::chunk, lane, n, kq);
        ld_blk += KS;
        if (ld_blk >= nb) {
            ld_blk = kp0;
            if (ld_tile + tstride < ntiles) ld_tile += tstride;
        }
    };
#pragma unroll
    for (int i = 0; i < D; ++i) issue(buf[i]);

    const bool ok = a.x ? stage_q8k<W, EXP ? kBsOne : kBsOneCompact>(a, lds, L, wave, xv)
                        : stage_planes<W>(a, lds, L, T, true, EXP);
    if (!ok) return finish_argmax(a, lds, L);
    if (a.zero_pair) return zero_slot_tiles<W, TS>(a, tmax, tstride);

    const OneA A = one_a_operand(lds, L, n, kq, EXP);
    const uint32_t pbytes = park_bytes(nb);
    uint32_t ti = 0, tile = t0, blk = kp, j = 0;
    auto compute = [&](const Q4Step<T>& cur) {
        const OneLoads r = one_loads<EXP>(A, A.p + blk * A.step, lds + L.bs_off + blk * 16, lds + L.d_off + blk * 32);
        const Q45One o = q45_one_ints<T>(cur, r, kq);
        const float dw = half_to_float(cur.h.x), dmw = half_to_float(cur.h.x >> 16);
        park_terms(park + (ti * TS + ts) * pbytes, nb, blk, lane, dw * r.da, o.I0, o.I1, (dmw * r.da) * (float)o.M);
        if (DBG) {  // exact block integers: the eight classes
            const int32_t I = sum_xor32(sum_xor16(o.I0 + o.I1));
            const uint32_t row = tile * kTileRows + n;
            if (kq == 0 && row < a.rows) {
                a.dbg_isum[(uint64_t)row * nb + blk] = I;
                a.dbg_imin[(uint64_t)row * nb + blk] = o.M;
            }
        }
        blk += KS;
        if (++j == bpt) {
            j = 0;
            blk = kp;
            ++ti;
            tile += tstride;
        }
    };
    pipeline<D>(steps, buf, issue, compute);
    __syncthreads();

    // each row's sum in the reference's order, one wave per tile slot (pair)
    if (TS % 2 == 0 && a.epilogue == kEpSiluPair) {
        // tile slots (2 q, 2 q + 1) hold gate and up rows of the same 16
        // outputs (llama.rs:367-371: gate = silu(gate); gate *= up)
        for (uint32_t it = wave; it < tmax * (TS / 2); it += W) {
            const uint32_t q = it % (TS / 2), til = it / (TS / 2);
            const uint32_t t = blockIdx.x * TS + 2 * q + til * tstride;  // the gate tile, even
            if (t + 1 >= ntiles) continue;                                // (wave-uniform)
            const uint8_t* pg = park + (til * TS + 2 * q) * pbytes;
            const float gs = exact_row_sum(pg, nb, lane);
            const float us = exact_row_sum(pg + pbytes, nb, lane);
            if (kq != 0) continue;
            if (a.chk) {  // the gate and up outputs themselves (math.rs:167)
                check_finite(a, kChkOut, gs);
                check_finite(a, kChkOut, us);
            }
            a.y[(t / 2) * kTileRows + n] = (gs / (1.0f + sse2_exp(0.0f - gs))) * us;
        }
        return;
    }
    unsigned long long best = 0;
    for (uint32_t slot = wave; slot < tmax * TS; slot += W) {
        const uint32_t t = blockIdx.x * TS + slot % TS + (slot / TS) * tstride;
        if (t >= ntiles) continue;  // (wave-uniform)
        const float v = exact_row_sum(park + slot * pbytes, nb, lane);
        const uint32_t row = t * kTileRows + n;
        if (kq == 0 && row < a.rows) store_out(a, row, 0, v, best);
    }
    if (a.am_out) {
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) {
            const unsigned long long o = __shfl_xor(best, m, 64);
            best = o > best ? o : best;
        }
        if (lane == 0 && best) atomicMax((unsigned long long*)(lds + L.am_off), best);
    }
    finish_argmax(a, lds, L);
}

// Batch-1 Q4_K/Q5_K kernel for one f32 column (no ids, no gate).  Each wave
// quantizes only the blocks it multiplies (blocks kp, kp + KS, ... of every
// tile it takes, at most four) while its first weight chunks are in flight, so
// a workgroup's Q8_K image costs one barrier (two with the RMSNorm transform)
// and no shared quantization pass.  Every block's terms are parked in LDS
// (park_terms) and a tile's K parts are counted with a workgroup-scope
// atomic; the wave that brings the count to the tile's part count forms each
// row's sum in the reference's order (exact_row_sum) and stores it (no
// barrier between tiles).  LDS after the Q8_K image: parked terms
// [tmax][TS][nb], counters [tmax][TS], residuals [tmax][TS][16].
__host__ __device__ inline uint32_t b1_lds_bytes(uint32_t cols, uint32_t tmax, uint32_t ts) {
    return one_part_off(cols, true) + tmax * ts * (park_bytes(cols / 256) + 4u + 16u * 4u);
}

// The RMSNorm scale (math.rs:210-221) from the values of the workgroup's own
// blocks: every element of the column is held by exactly one lane (the waves
// of tile slot 0 cover every block), its square is added in f64 by that lane,
// the lane sums meet in LDS and every thread adds the wave sums in wave
// order.  The certificate of rms_scale decides whether that sum fixes the
// reference's f32 mean; otherwise thread 0 repeats the sum in the reference's
// order.  Every workgroup computes the same value.
template <int W>
__device__ __forceinline__ float b1_rms_scale(const MvArgs& a, uint8_t* lds, const LdsMap& L, uint32_t wave,
                                              bool mine, const float (&v)[16]) {
    double ss = 0.0;
    if (mine) {
#pragma unroll
        for (int k = 0; k < 16; ++k) ss += (double)(v[k] * v[k]);
    }
    ss = row16_sum_f64(ss);
    double* red = (double*)(lds + L.red_off);
    if ((threadIdx.x & 15) == 0) red[wave * 4 + ((threadIdx.x & 63) >> 4)] = ss;
    __syncthreads();
    double total = 0.0;
#pragma unroll
    for (int w = 0; w < 4 * W; ++w) total += red[w];
    const double n = (double)a.cols, err = n * 2.3e-16 * total;
    if ((float)((total - err) / n) != (float)((total + err) / n)) {  // every thread takes the same branch
        __syncthreads();
        if (threadIdx.x == 0) {
            double seq = 0.0;
            for (uint32_t i = 0; i < a.cols; ++i) seq += (double)(a.x[i] * a.x[i]);
            red[0] = seq;
        }
        __syncthreads();
        total = red[0];
    }
    return 1.0f / sqrtf((float)(total / n) + a.eps);
}

// FULL: the decode step's extras (the RMSNorm input transform, the residual
// add), the output checks of a model stage (chk) and the in-launch argmax;
// without them none is compiled in.
// BAL: the balanced deal over a.deal_cus CUs (balanced_deal).
template <uint32_t T, int W, int KS, int D, bool DBG, bool FULL, bool BAL = false>
__global__ __launch_bounds__(W * 64) void q45_mv_b1_kernel(MvArgs a) {
    constexpr int TS = W / KS;
    static_assert(!BAL || TS == 2 || TS == 4, "the balanced deal takes two or four tile slots");
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsMap L = lds_map_one(T, a.cols, true);
    const uint32_t lane = threadIdx.x & 63, n = lane & 15, kq = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t ts = wave / KS, kp = wave % KS;
    const uint32_t nb = a.nb, ntiles = a.ntiles;
    const uint32_t tstride = gridDim.x * TS, t0 = blockIdx.x * TS + ts;
    // this wave's tiles: tile_of(i) for i < my_tiles; half_ti the ordinal of
    // its half tile (none: ~0) and hsel its half
    uint32_t tmax, my_tiles, half_ti = ~0u, hsel = 0, bt = 0;
    if constexpr (BAL) {
        const TileDeal d = balanced_deal<TS>(a.deal_cus, ntiles, ts);
        tmax = 1, my_tiles = d.count, bt = d.tile, hsel = d.hsel;
        if (d.half) half_ti = 0;
    } else {
        tmax = (ntiles + tstride - 1) / tstride;
        my_tiles = t0 < ntiles ? (ntiles - 1 - t0) / tstride + 1 : 0;
    }
    auto tile_of = [&](uint32_t i) -> uint32_t {
        if constexpr (BAL) return bt;
        else return t0 + i * tstride;
    };
    // whether lane row n is this workgroup's row of tile i; the row a lane
    // loads in the half tile
    auto own_row = [&](uint32_t i) { return i != half_ti || (n >> 3) == hsel; };
    const uint32_t nh = (n & 7) | (hsel << 3);
    const uint32_t bpt = kp < nb ? (nb - 1 - kp) / KS + 1 : 0;  // blocks of each tile this wave takes
    const uint32_t steps = my_tiles * bpt;
    const uint32_t nk = (uint32_t)KS < nb ? (uint32_t)KS : nb;  // waves of a tile that take blocks
    // LDS after the Q8_K image: parked terms [tmax * TS][nb] (park_terms),
    // counters [tmax * TS], residuals [tmax * TS][16]
    uint8_t* park = lds + one_part_off(a.cols, true);
    const uint32_t pbytes = park_bytes(nb);
    uint32_t* cnt = (uint32_t*)(park + tmax * TS * pbytes);
    float* rs = (float*)(cnt + tmax * TS);
    for (uint32_t i = threadIdx.x; i < tmax * TS; i += W * 64) cnt[i] = 0;
    if (threadIdx.x < 16) *(uint4*)(lds + L.zero_off + threadIdx.x * 16) = make_uint4(0, 0, 0, 0);  // dead A lanes
    const bool rms = FULL && a.xform == kXfRmsNorm;
    if (FULL && threadIdx.x < 8) ((unsigned long long*)(lds + L.am_off))[threadIdx.x] = 0ull;

    // loaded before the weights: the first own block of each 16-lane row
    // (the waves of tile slot 0 cover every block), its RMSNorm weights and
    // the residuals of this slot's tiles (at most four, the host checks)
    const uint32_t r16 = lane & 15;
    const bool mine = ts == 0 && kq < bpt;
    const uint32_t xblk = kp + KS * kq;
    float xv[16], nw[16], res = 0.0f;
    if (mine) load16(a.x + xblk * 256 + r16 * 16, xv);
    if (rms && mine) load16(a.norm_w + xblk * 256 + r16 * 16, nw);
    const bool res_lane = FULL && a.resid && kp == 0 && kq < my_tiles;
    if (res_lane) {
        const uint32_t row = tile_of(kq) * kTileRows + n;
        if (row < a.rows) res = a.resid[row];
    }
    const uint32_t kp0 = kp < nb ? kp : nb - 1;
    uint32_t ld_tile = t0 < ntiles ? t0 : ntiles - 1, ld_blk = kp0;
    if constexpr (BAL) ld_tile = my_tiles ? bt : 0;
    Q4Step<T> buf[D];
    auto issue = [&](Q4Step<T>& st) {
        const uint8_t* base = a.w + ((uint64_t)ld_tile * nb + ld_blk) * Q45<T>::chunk;
        if (BAL && half_ti == 0) q45_issue<T>(st, base, kq * 16 + nh, nh, kq);  // the half tile
        else q45_issue<T>(st, base, lane, n, kq);
        ld_blk += KS;
        if (ld_blk >= nb) {
            ld_blk = kp0;
            if (!BAL && ld_tile + tstride < ntiles) ld_tile += tstride;
        }
    };
#pragma unroll
    for (int i = 0; i < D; ++i) issue(buf[i]);

    // Q8_K of the own blocks (quantize_row_q8_K, 16 lanes per block)
    int bad = 0;
    if (rms) {
        const float scale = b1_rms_scale<W>(a, lds, L, wave, mine, xv);
        if (!(scale <= 3.402823466e38f) || !(scale > 0.0f)) {  // math.rs:218-220
            bad = 1;
            if (threadIdx.x == 0) report_error(a.err_word, rms_scale_key(a));
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) xv[k] = xv[k] * scale * nw[k];
    }
    if (res_lane) rs[(kq * TS + ts) * 16 + n] = res;
    if (mine) {
        const Q8KRow o = q8k_row16(xv, r16);
        if (o.kind >= 0) {
            bad = 1;
            if (r16 == 0)
                report_error(a.err_word, o.kind == kKindNonFinite ? quant_nonfinite_key(a, 0, xblk * 256ull + o.index)
                                                                  : quant_scale_key(a, 0, xblk));
        }
        store_one_unit(lds, L, xblk, r16, q45_slots(o.q, r16 & 1), o.bsum, true);
        if (r16 == 0) *(float*)(lds + L.d_off + xblk * 32) = o.d;
    }
    // the counters' zeros, every own block, the residuals and every wave's
    // error flag
    if (__syncthreads_or(bad)) {
        if (FULL) finish_argmax(a, lds, L);
        return;
    }

    const OneA A = one_a_operand(lds, L, n, kq, true);
    unsigned long long best = 0;
    uint32_t ti = 0, blk = kp, j = 0, tile = tile_of(0);
    auto compute = [&](const Q4Step<T>& cur) {
        const OneLoads r = one_loads<true>(A, A.p + blk * A.step, lds + L.bs_off + blk * 16, lds + L.d_off + blk * 32);
        const Q45One o = q45_one_ints<T>(cur, r, kq);
        const float dw = half_to_float(cur.h.x), dmw = half_to_float(cur.h.x >> 16);
        park_terms(park + (ti * TS + ts) * pbytes, nb, blk, lane, dw * r.da, o.I0, o.I1, (dmw * r.da) * (float)o.M);
        if (DBG) {  // exact block integers: the eight classes
            const int32_t I = sum_xor32(sum_xor16(o.I0 + o.I1));
            const uint32_t row = tile * kTileRows + n;
            if (kq == 0 && row < a.rows && own_row(ti)) {
                a.dbg_isum[(uint64_t)row * nb + blk] = I;
                a.dbg_imin[(uint64_t)row * nb + blk] = o.M;
            }
        }
        blk += KS;
        if (++j == bpt) {  // this wave's share of the tile is parked: count it
            const uint32_t slot = ti * TS + ts;
            // one wave's LDS operations are performed in order: the terms are
            // in place before the count
            if (lane == 0) {
                const uint32_t prev =
                    __hip_atomic_fetch_add(cnt + slot, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
                // the last part: this wave finishes the tile after its last
                // step (no global store or atomic between the weight loads)
                if (prev == nk - 1) cnt[slot] = nk + 1 + wave;
            }
            j = 0;
            blk = kp;
            tile = tile_of(++ti);
        }
    };
    pipeline<D>(steps, buf, issue, compute);

    // the tiles this wave completed: each row's sum in the reference's order
    // (every lane of the wave takes part; rows past the matrix and the other
    // half of a half tile are not stored)
    for (uint32_t i = 0; i < my_tiles; ++i) {
        const uint32_t slot = i * TS + ts, row = tile_of(i) * kTileRows + n;
        if (cnt[slot] != nk + 1 + wave) continue;  // (wave-uniform)
        float s = exact_row_sum(park + slot * pbytes, nb, lane);
        if (kq != 0 || row >= a.rows || !own_row(i)) continue;
        if (FULL && a.chk) check_finite(a, kChkOut, s);
        if (FULL && a.resid) {
            s = rs[slot * 16 + n] + s;  // math.rs:203-208: hidden += projected
            if (a.chk) check_finite(a, kChkResid, s);
        }
        a.y[row] = s;
        if (FULL) {
            const unsigned long long key = argmax_key(s, row);
            best = key > best ? key : best;
        }
    }
    if (FULL) {
        fold_argmax(a, lds, L, kq, best);
        finish_argmax(a, lds, L);
    }
}

// ---------------------------------------------------------------------------
// Q6_K
// ---------------------------------------------------------------------------
struct Q6Step {
    uint4 l0, l1, h0, h1, sc;
    uint32_t d;
};

// Signed 6-bit values q - 32 of 16 elements as int8: low nibbles from ql and
// two bits from qh moved to bits 4..5, then +0x60 ^ 0x80 per byte maps
// q in 0..63 to q - 32 without carries between bytes.
__device__ __forceinline__ uint32_t q6_lo(uint32_t ql, uint32_t qh, uint32_t lsh) {
    return ((ql & 0x0f0f0f0fu) + ((qh << lsh) & 0x30303030u) + 0x60606060u) ^ 0x80808080u;
}
__device__ __forceinline__ uint32_t q6_hi(uint32_t ql, uint32_t qh, uint32_t rsh) {
    return (((ql >> 4) & 0x0f0f0f0fu) + ((qh >> rsh) & 0x30303030u) + 0x60606060u) ^ 0x80808080u;
}

template <int W, int D, bool DBG>
__global__ __launch_bounds__(W * 64) void q6k_mv_kernel(MvArgs a) {
    RLQ_MV_PROLOGUE(kQ6_K, a.nb)
    const uint32_t nb = a.nb;
    Q6Step buf[D];
    auto issue = [&](Q6Step& st) {
        const uint8_t* base = a.w + ((uint64_t)ld_tile * nb + ld_chunk) * kQ6KChunk;
        st.l0 = load_stream16(base + lane * 16);
        st.l1 = load_stream16(base + 1024 + lane * 16);
        st.h0 = load_stream16(base + 2048 + n * 64 + 32 * (kq >> 1));
        st.h1 = load_stream16(base + 2048 + n * 64 + 32 * (kq >> 1) + 16);
        st.sc = load_stream16(base + 3072 + n * 16);
        st.d = __builtin_nontemporal_load((const uint16_t*)(base + 3328 + n * 2));
        next_load();
    };
#pragma unroll
    for (int i = 0; i < D; ++i) issue(buf[i]);

    const bool ok = a.x ? stage_q8k<W, kBsNone>(a, lds, L, wave, xv) : stage_planes<W>(a, lds, L, kQ6_K);
    if (!ok) return finish_argmax(a, lds, L);
    if (a.zero_pair) return zero_wave_tiles(a, gw, tw, n, kq);

    // This lane's weights: ql bytes 32kq.. (g = kq/2, s1 = kq%2) give the
    // elements of 16-element scale groups 8g + 2s1 + h (low nibbles) and
    // 8g + 2s1 + 4 + h (high nibbles), h = 0, 1.
    const uint32_t s1 = kq & 1, lsh = 4 - 2 * s1, rsh = 2 * s1;
    // A operand: lane row r = n holds column r / 4 (+4 for the second column
    // group) and is nonzero in K quarter kq == r % 4 only.
    const uint32_t abl = n >> 2, which = n & 3;
    const uint32_t a_grp = 8 * (which >> 1) + 2 * (which & 1);
    const uint8_t* a_row = lds + abl * L.S + 16 * a_grp;
    const bool two_groups = a.batch > 4;
    const bool a_live0 = which == kq && abl < a.batch;
    const bool a_live1 = which == kq && abl + 4 < a.batch;
    const uint8_t* a_ptr0 = a_live0 ? a_row : lds + L.zero_off;
    const uint8_t* a_ptr1 = a_live1 ? a_row + 4 * L.S : lds + L.zero_off;
    const uint32_t a_step0 = a_live0 ? 256 : 0, a_step1 = a_live1 ? 256 : 0;

    float acc0 = 0.0f, acc1 = 0.0f;
    unsigned long long best0 = 0, best1 = 0;
    uint32_t tile = gw, blk = 0;
    auto compute = [&](const Q6Step& cur) {
        // operands (high, h): scale groups {0,2,8,10} + 4*high + h
        const i32x4 w00 = {(int)q6_lo(cur.l0.x, cur.h0.x, lsh), (int)q6_lo(cur.l0.y, cur.h0.y, lsh),
                           (int)q6_lo(cur.l0.z, cur.h0.z, lsh), (int)q6_lo(cur.l0.w, cur.h0.w, lsh)};
        const i32x4 w01 = {(int)q6_lo(cur.l1.x, cur.h1.x, lsh), (int)q6_lo(cur.l1.y, cur.h1.y, lsh),
                           (int)q6_lo(cur.l1.z, cur.h1.z, lsh), (int)q6_lo(cur.l1.w, cur.h1.w, lsh)};
        const i32x4 w10 = {(int)q6_hi(cur.l0.x, cur.h0.x, rsh), (int)q6_hi(cur.l0.y, cur.h0.y, rsh),
                           (int)q6_hi(cur.l0.z, cur.h0.z, rsh), (int)q6_hi(cur.l0.w, cur.h0.w, rsh)};
        const i32x4 w11 = {(int)q6_hi(cur.l1.x, cur.h1.x, rsh), (int)q6_hi(cur.l1.y, cur.h1.y, rsh),
                           (int)q6_hi(cur.l1.z, cur.h1.z, rsh), (int)q6_hi(cur.l1.w, cur.h1.w, rsh)};
        const float dw = half_to_float(cur.d);
        // integer dot of one column group: output element i of operand (high, h)
        // is scale group {0,2,8,10}[i] + 4 high + h
        auto group = [&](const uint8_t* p) {
            const i32x4 a00 = *(const i32x4*)(p), a01 = *(const i32x4*)(p + 16);
            const i32x4 a10 = *(const i32x4*)(p + 64), a11 = *(const i32x4*)(p + 80);
            const i32x4 d00 = mfma_i8(a00, w00), d01 = mfma_i8(a01, w01);
            const i32x4 d10 = mfma_i8(a10, w10), d11 = mfma_i8(a11, w11);
            int32_t I = sbyte(cur.sc.x, 0) * d00[0] + sbyte(cur.sc.x, 2) * d00[1] + sbyte(cur.sc.z, 0) * d00[2] +
                        sbyte(cur.sc.z, 2) * d00[3];
            I += sbyte(cur.sc.x, 1) * d01[0] + sbyte(cur.sc.x, 3) * d01[1] + sbyte(cur.sc.z, 1) * d01[2] +
                 sbyte(cur.sc.z, 3) * d01[3];
            I += sbyte(cur.sc.y, 0) * d10[0] + sbyte(cur.sc.y, 2) * d10[1] + sbyte(cur.sc.w, 0) * d10[2] +
                 sbyte(cur.sc.w, 2) * d10[3];
            I += sbyte(cur.sc.y, 1) * d11[0] + sbyte(cur.sc.y, 3) * d11[1] + sbyte(cur.sc.w, 1) * d11[2] +
                 sbyte(cur.sc.w, 3) * d11[3];
            return I;
        };
        const int32_t I0 = group(a_ptr0 + blk * a_step0);
        acc0 += (dw * *(const float*)(lds + L.d_off + (blk * 8 + kq) * 4)) * (float)I0;
        if (DBG && kq == 0) {
            const uint32_t row = tile * kTileRows + n;
            if (row < a.rows) {
                a.dbg_isum[(uint64_t)row * nb + blk] = I0;
                a.dbg_imin[(uint64_t)row * nb + blk] = 0;
            }
        }
        if (two_groups) {
            const int32_t I1 = group(a_ptr1 + blk * a_step1);
            acc1 += (dw * *(const float*)(lds + L.d_off + (blk * 8 + kq + 4) * 4)) * (float)I1;
        }
        if (++blk == nb) {
            const uint32_t row = tile * kTileRows + n;
            store_out(a, row, kq, acc0, best0);
            store_out(a, row, kq + 4, acc1, best1);
            acc0 = acc1 = 0.0f;
            blk = 0;
            tile += tw;
        }
    };
    pipeline<D>(steps, buf, issue, compute);
    fold_argmax(a, lds, L, kq, best0);
    fold_argmax(a, lds, L, kq + 4, best1);
    finish_argmax(a, lds, L);
}

// Q6_K, one column, in the reference's f32 order (matvec_extra.rs:272-293):
// eight lane accumulators lanes[j % 8] per row over all blocks, then
// sum = 0 + lanes[0] + ... + lanes[7].  The weight chunks and lane roles are
// those of q6k_mv_kernel; the A rows split each scale group's dot by lane
// class.  A row r holds class c = r % 8 of K quarter r / 8 (first MFMA of a
// pair) or 2 + r / 8 (second): the activation of that quarter's scale group
// masked to the elements j with j % 8 == c (bytes c and c + 8 of the
// group's 16).  Output i of the pair in lane (n, kq) is then the exact dot of
// weight row n over class 4 (kq % 2) + i of scale group
// {0, 2, 8, 10}[kq / 2] + off (first) or {8, 10}[kq / 2] + off (second), with
// off = 0, 1, 4, 5 for the four weight operands; the lanes kq and kq ^ 2
// hold the other eight groups of the same classes.  A wave takes whole tiles
// and walks their blocks in order, so the accumulators stay in registers.
// Loads of one Q6_K chunk (rlq_layout.hpp): the ql pieces of lane `ln` and
// the high bits, scales and super-scale of row `r` (a lane's own: ln = lane,
// r = n; a half tile's lane pairs load row r of the pair, ln = 16 kq + r).
__device__ __forceinline__ void q6_issue(Q6Step& st, const uint8_t* base, uint32_t ln, uint32_t r, uint32_t kq) {
    st.l0 = load_stream16(base + ln * 16);
    st.l1 = load_stream16(base + 1024 + ln * 16);
    st.h0 = load_stream16(base + 2048 + r * 64 + 32 * (kq >> 1));
    st.h1 = load_stream16(base + 2048 + r * 64 + 32 * (kq >> 1) + 16);
    st.sc = load_stream16(base + 3072 + r * 16);
    st.d = __builtin_nontemporal_load((const uint16_t*)(base + 3328 + r * 2));
}

// The one-column class operands of lane (n, kq): A row n stands for class
// n % 8 of K quarter n / 8 (first MFMA of a pair) or 2 + n / 8 (second); the
// lane's activations (K quarter kq of the block's image, a_step bytes per
// block, or the zero bytes where neither MFMA is live) masked by m0 / m1 to
// the class's bytes.
struct Q6OneOps {
    const uint8_t* a_ptr;
    uint32_t a_step, lsh, rsh, g2;
    uint32_t m0[4], m1[4];
};
__device__ __forceinline__ Q6OneOps q6_one_ops(const uint8_t* lds, const LdsMap& L, uint32_t n, uint32_t kq) {
    Q6OneOps o;
    const uint32_t s1 = kq & 1;
    o.lsh = 4 - 2 * s1, o.rsh = 2 * s1;
    const uint32_t cls = n & 7, qsel = n >> 3;
    const bool live0 = kq == qsel, live1 = kq == 2 + qsel;
    o.a_ptr = live0 || live1 ? lds + 16 * (8 * (kq >> 1) + 2 * (kq & 1)) : lds + L.zero_off;
    o.a_step = live0 || live1 ? 256 : 0;
    const uint32_t byte = 0xffu << (8 * (cls & 3));
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t mk = (uint32_t)(w & 1) == (cls >> 2) ? byte : 0u;
        o.m0[w] = live0 ? mk : 0u;
        o.m1[w] = live1 ? mk : 0u;
    }
    o.g2 = 16 * (kq >> 1);  // bit offset of scale bytes 2 (kq / 2), + 1 in each scale word
    return o;
}
// Block integers of one chunk in lane (n, kq): I[i] = the exact dot of row n
// over class 4 (kq % 2) + i (elements j with j % 8 == class), scale groups
// included, summed over the lane's K half (lanes kq and kq ^ 2 hold the
// other half until the caller's sum_xor32).  p = the block's activations.
__device__ __forceinline__ void q6_one_ints(const Q6Step& cur, const Q6OneOps& o, const uint8_t* p, int32_t (&I)[4]) {
    const i32x4 w00 = {(int)q6_lo(cur.l0.x, cur.h0.x, o.lsh), (int)q6_lo(cur.l0.y, cur.h0.y, o.lsh),
                       (int)q6_lo(cur.l0.z, cur.h0.z, o.lsh), (int)q6_lo(cur.l0.w, cur.h0.w, o.lsh)};
    const i32x4 w01 = {(int)q6_lo(cur.l1.x, cur.h1.x, o.lsh), (int)q6_lo(cur.l1.y, cur.h1.y, o.lsh),
                       (int)q6_lo(cur.l1.z, cur.h1.z, o.lsh), (int)q6_lo(cur.l1.w, cur.h1.w, o.lsh)};
    const i32x4 w10 = {(int)q6_hi(cur.l0.x, cur.h0.x, o.rsh), (int)q6_hi(cur.l0.y, cur.h0.y, o.rsh),
                       (int)q6_hi(cur.l0.z, cur.h0.z, o.rsh), (int)q6_hi(cur.l0.w, cur.h0.w, o.rsh)};
    const i32x4 w11 = {(int)q6_hi(cur.l1.x, cur.h1.x, o.rsh), (int)q6_hi(cur.l1.y, cur.h1.y, o.rsh),
                       (int)q6_hi(cur.l1.z, cur.h1.z, o.rsh), (int)q6_hi(cur.l1.w, cur.h1.w, o.rsh)};
    // one weight operand: its scale groups' signed scales sa (first MFMA)
    // and sb (second); |dot| <= 2 * 32 * 128 and |scale| <= 128 fit the
    // 24-bit multiplies
    auto pair = [&](const i32x4& wop, uint32_t aoff, int32_t sa, int32_t sb) {
        const uint4 x = *(const uint4*)(p + aoff);
        const i32x4 A0 = {(int)(x.x & o.m0[0]), (int)(x.y & o.m0[1]), (int)(x.z & o.m0[2]), (int)(x.w & o.m0[3])};
        const i32x4 A1 = {(int)(x.x & o.m1[0]), (int)(x.y & o.m1[1]), (int)(x.z & o.m1[2]), (int)(x.w & o.m1[3])};
        const i32x4 d0 = mfma_i8(A0, wop), d1 = mfma_i8(A1, wop);
#pragma unroll
        for (int i = 0; i < 4; ++i) I[i] = mad24(sa, d0[i], mad24(sb, d1[i], I[i]));
    };
    const uint32_t g2 = o.g2;
    pair(w00, 0, __builtin_amdgcn_sbfe((int)cur.sc.x, g2, 8), __builtin_amdgcn_sbfe((int)cur.sc.z, g2, 8));
    pair(w01, 16, __builtin_amdgcn_sbfe((int)cur.sc.x, g2 + 8, 8), __builtin_amdgcn_sbfe((int)cur.sc.z, g2 + 8, 8));
    pair(w10, 64, __builtin_amdgcn_sbfe((int)cur.sc.y, g2, 8), __builtin_amdgcn_sbfe((int)cur.sc.w, g2, 8));
    pair(w11, 80, __builtin_amdgcn_sbfe((int)cur.sc.y, g2 + 8, 8), __builtin_amdgcn_sbfe((int)cur.sc.w, g2 + 8, 8));
}

template <int W, int D, bool DBG>
__global__ __launch_bounds__(W * 64) void q6k_mv_one_kernel(MvArgs a) {
    RLQ_MV_PROLOGUE(kQ6_K, a.nb)
    const uint32_t nb = a.nb;
    Q6Step buf[D];
    auto issue = [&](Q6Step& st) {
        q6_issue(st, a.w + ((uint64_t)ld_tile * nb + ld_chunk) * kQ6KChunk, lane, n, kq);
        next_load();
    };
#pragma unroll
    for (int i = 0; i < D; ++i) issue(buf[i]);

    const bool ok = a.x ? stage_q8k<W, kBsNone>(a, lds, L, wave, xv) : stage_planes<W>(a, lds, L, kQ6_K);
    if (!ok) return finish_argmax(a, lds, L);
    if (a.zero_pair) return zero_wave_tiles(a, gw, tw, n, kq);

    const Q6OneOps ops = q6_one_ops(lds, L, n, kq);

    float lanes[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // classes 4 (kq % 2) + i
    unsigned long long best = 0;
    uint32_t tile = gw, blk = 0;
    auto compute = [&](const Q6Step& cur) {
        int32_t I[4] = {0, 0, 0, 0};
        q6_one_ints(cur, ops, ops.a_ptr + blk * ops.a_step, I);
        const float d = half_to_float(cur.d) * *(const float*)(lds + L.d_off + blk * 32);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            I[i] = sum_xor32(I[i]);
            lanes[i] += d * (float)I[i];  // matvec_extra.rs:287-289
        }
        if (DBG) {
            const int32_t It = sum_xor16(I[0] + I[1] + I[2] + I[3]);
            const uint32_t row = tile * kTileRows + n;
            if (kq == 0 && row < a.rows) {
                a.dbg_isum[(uint64_t)row * nb + blk] = It;
                a.dbg_imin[(uint64_t)row * nb + blk] = 0;
            }
        }
        if (++blk == nb) {  // sum = 0 + lanes[0] + ... + lanes[7] (:290-292)
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) sum += __shfl(lanes[i], (int)n, 64);
#pragma unroll
            for (int i = 0; i < 4; ++i) sum += __shfl(lanes[i], (int)(n + 16), 64);
            if (kq == 0) store_out(a, tile * kTileRows + n, 0, sum, best);
#pragma unroll
            for (int i = 0; i < 4; ++i) lanes[i] = 0.0f;
            blk = 0;
            tile += tw;
        }
    };
    pipeline<D>(steps, buf, issue, compute);
    fold_argmax(a, lds, L, kq, best);
    finish_argmax(a, lds, L);
}

// ---------------------------------------------------------------------------
// Q2_K and Q3_K: 16-element scale groups, two bits (+ a high-mask bit) per value
// ---------------------------------------------------------------------------
// Lane (n, kq) loads qs bytes 16kq .. +15 of row n: qs byte 32G + p (G = kq/2,
// p = 16(kq%2) + i) holds element 128G + 32s + p in bits 2s..2s+1, s = 0..3.
// MFMA s therefore gives this lane's B operand the 16 values of scale group
// sg(kq, s) = 8G + 2s + kq%2 (elements 16 sg ..).  A row r = n holds column
// r / 4 (+4 for the second column group) and is nonzero in K quarter r % 4
// only, with the activations of sg(r % 4, s): output element t of MFMA s in
// lane (n, kq) is the integer dot of weight row n with column kq over scale
// group sg(t, s), so every lane holds whole block integers for its column.
template <uint32_t T>
struct K16Step;
template <>
struct K16Step<kQ3_K> {
    uint4 q, hm;
    uint3 sc;
    uint32_t d;
};
template <>
struct K16Step<kQ2_K> {
    uint4 q, sc;
    uint32_t dd;
};

// The sixteen Q3_K scales as signed bytes, sc[4k..4k+3] in word k
// (matvec_extra.rs:200-210): low nibbles from bytes 0..7, two high bits from
// bytes 8..11; q - 32 per byte without carries (+0x60, ^0x80).
__device__ __forceinline__ void q3_scale_words(uint3 p, uint32_t (&c)[4]) {
    c[0] = (p.x & 0x0f0f0f0fu) | ((p.z << 4) & 0x30303030u);
    c[1] = (p.y & 0x0f0f0f0fu) | ((p.z << 2) & 0x30303030u);
    c[2] = ((p.x >> 4) & 0x0f0f0f0fu) | (p.z & 0x30303030u);
    c[3] = ((p.y >> 4) & 0x0f0f0f0fu) | ((p.z >> 2) & 0x30303030u);
#pragma unroll
    for (int k = 0; k < 4; ++k) c[k] = (c[k] + 0x60606060u) ^ 0x80808080u;
}

// Q2_K mins of one column: the sum over the 16 groups of min * bsum
// (matvec_extra.rs:183-185); bs = the column's 16 bsums of the block in LDS.
__device__ __forceinline__ int32_t q2_mins(uint4 sc, const uint8_t* bs) {
    const uint4 b0 = ((const uint4*)bs)[0], b1 = ((const uint4*)bs)[1];
    const uint32_t m[4] = {(sc.x >> 4) & 0x0f0f0f0fu, (sc.y >> 4) & 0x0f0f0f0fu, (sc.z >> 4) & 0x0f0f0f0fu,
                           (sc.w >> 4) & 0x0f0f0f0fu};
    const uint32_t bw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    int32_t M = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        M = dot2(__builtin_amdgcn_perm(0u, m[k], 0x0c010c00u), bw[2 * k], M);
        M = dot2(__builtin_amdgcn_perm(0u, m[k], 0x0c030c02u), bw[2 * k + 1], M);
    }
    return M;
}

// Loads of one chunk (rlq_layout.hpp): this lane's qs piece, the row's high
// mask half (Q3_K), scales and super-scales.
template <uint32_t T>
__device__ __forceinline__ void k16_issue(K16Step<T>& st, const uint8_t* base, uint32_t lane, uint32_t n,
                                          uint32_t kq) {
    st.q = load_stream16(base + lane * 16);
    if constexpr (T == kQ3_K) {
        st.hm = load_stream16(base + 1024 + n * 32 + 16 * (kq & 1));
        const uint32_t* sp = (const uint32_t*)(base + 1536 + n * 12);
        st.sc = make_uint3(__builtin_nontemporal_load(sp), __builtin_nontemporal_load(sp + 1),
                           __builtin_nontemporal_load(sp + 2));
        st.d = __builtin_nontemporal_load((const uint16_t*)(base + 1728 + n * 2));
    } else {
        st.sc = load_stream16(base + 1024 + n * 16);
        st.dd = __builtin_nontemporal_load((const uint32_t*)(base + 1280 + n * 4));
    }
}

// The B operands of the four MFMAs of one chunk and the sixteen scales as
// bytes (hsh = 4 * (kq / 2), the lane's high-mask bit offset).
template <uint32_t T>
struct K16Ops {
    i32x4 wv[4];
    uint32_t c[4];
};
template <uint32_t T>
__device__ __forceinline__ K16Ops<T> k16_ops(const K16Step<T>& cur, uint32_t hsh) {
    K16Ops<T> o;
    const uint32_t q[4] = {cur.q.x, cur.q.y, cur.q.z, cur.q.w};
    if constexpr (T == kQ3_K) {
        const uint32_t hm[4] = {cur.hm.x >> hsh, cur.hm.y >> hsh, cur.hm.z >> hsh, cur.hm.w >> hsh};
#pragma unroll
        for (int sft = 0; sft < 4; ++sft)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // low | hbit << 2 in 0..7, minus 4 per byte (+0x7c, ^0x80):
                // q = low - (hbit ? 0 : 4)  (matvec_extra.rs:240-244)
                const uint32_t hb = sft < 3 ? hm[i] << (2 - sft) : hm[i] >> 1;
                const uint32_t v = ((q[i] >> (2 * sft)) & 0x03030303u) | (hb & 0x04040404u);
                o.wv[sft][i] = (int)((v + 0x7c7c7c7cu) ^ 0x80808080u);
            }
        q3_scale_words(cur.sc, o.c);
    } else {
#pragma unroll
        for (int sft = 0; sft < 4; ++sft)
#pragma unroll
            for (int i = 0; i < 4; ++i) o.wv[sft][i] = (int)((q[i] >> (2 * sft)) & 0x03030303u);
        o.c[0] = cur.sc.x & 0x0f0f0f0fu, o.c[1] = cur.sc.y & 0x0f0f0f0fu;
        o.c[2] = cur.sc.z & 0x0f0f0f0fu, o.c[3] = cur.sc.w & 0x0f0f0f0fu;
    }
    return o;
}

// Integer dot of one column group (A rows from p): sg(t, s) = 8(t/2) + 2s +
// t%2 is byte 2(s%2) + t%2 of scale word 2(t/2) + s/2.
template <uint32_t T>
__device__ __forceinline__ int32_t k16_isum(const K16Ops<T>& o, const uint8_t* p) {
    auto scale = [&](uint32_t word, int byte) -> int32_t {
        return T == kQ3_K ? sbyte(word, byte) : (int32_t)ubyte(word, byte);
    };
    int32_t I = 0;
#pragma unroll
    for (int sft = 0; sft < 4; ++sft) {
        const i32x4 av = *(const i32x4*)(p + 32 * sft);
        const i32x4 dv = mfma_i8(av, o.wv[sft]);
        const int bl = 2 * (sft & 1), wl = sft >> 1;
        I = mad24(scale(o.c[wl], bl), dv[0], I);
        I = mad24(scale(o.c[wl], bl + 1), dv[1], I);
        I = mad24(scale(o.c[2 + wl], bl), dv[2], I);
        I = mad24(scale(o.c[2 + wl], bl + 1), dv[3], I);
    }
    return I;
}

// The f32 term one block adds for column `col` (da = its activation scale):
// Q3_K d * isum with d = f16(d) * y.d; Q2_K d * isum - mn * mins with
// d = y.d * f16(d), mn = y.d * f16(dmin) (matvec_extra.rs:193-195, 246).
template <uint32_t T>
__device__ __forceinline__ float k16_term(const K16Step<T>& cur, float da, int32_t I, int32_t M) {
    if constexpr (T == kQ3_K) {
        return (half_to_float(cur.d) * da) * (float)I;
    } else {
        return (da * half_to_float(cur.dd)) * (float)I - (da * half_to_float(cur.dd >> 16)) * (float)M;
    }
}

// A-operand setup shared by the two kernels: A row r = n holds column r / 4
// (+4 for the second group), nonzero in K quarter r % 4 only.
struct K16A {
    const uint8_t *p0, *p1;
    uint32_t step0, step1;
};
__device__ __forceinline__ K16A k16_a(const uint8_t* lds, const LdsMap& L, uint32_t batch, uint32_t n, uint32_t kq) {
    const uint32_t abl = n >> 2, which = n & 3;
    const uint8_t* a_row = lds + abl * L.S + 128 * (which >> 1) + 16 * (which & 1);
    const bool live0 = which == kq && abl < batch, live1 = which == kq && abl + 4 < batch;
    return K16A{live0 ? a_row : lds + L.zero_off, live1 ? a_row + 4 * L.S : lds + L.zero_off, live0 ? 256u : 0u,
                live1 ? 256u : 0u};
}

// One wave per tile: every lane adds its column's block terms in block order.
template <uint32_t T, int W, int D, bool DBG>
__global__ __launch_bounds__(W * 64) void k16_mv_kernel(MvArgs a) {
    constexpr uint32_t kChunk = T == kQ3_K ? kQ3KChunk : kQ2KChunk;
    RLQ_MV_PROLOGUE(T, a.nb)
    const uint32_t nb = a.nb;
    K16Step<T> buf[D];
    auto issue = [&](K16Step<T>& st) {
        k16_issue<T>(st, a.w + ((uint64_t)ld_tile * nb + ld_chunk) * kChunk, lane, n, kq);
        next_load();
    };
#pragma unroll
    for (int i = 0; i < D; ++i) issue(buf[i]);

    const bool ok = a.x ? stage_q8k<W, bsum_order(T)>(a, lds, L, wave, xv) : stage_planes<W>(a, lds, L, T);
    if (!ok) return finish_argmax(a, lds, L);
    if (a.zero_pair) return zero_wave_tiles(a, gw, tw, n, kq);

    const K16A A = k16_a(lds, L, a.batch, n, kq);
    const bool two_groups = a.batch > 4;
    const uint32_t hsh = 4 * (kq >> 1);

    float acc0 = 0.0f, acc1 = 0.0f;
    unsigned long long best0 = 0, best1 = 0;
    uint32_t tile = gw, blk = 0;
    auto compute = [&](const K16Step<T>& cur) {
        const K16Ops<T> o = k16_ops<T>(cur, hsh);
        const float da0 = *(const float*)(lds + L.d_off + (blk * 8 + kq) * 4);
        const int32_t I0 = k16_isum<T>(o, A.p0 + blk * A.step0);
        int32_t M0 = 0;
        if constexpr (T == kQ2_K) M0 = kq < a.batch ? q2_mins(cur.sc, lds + L.bs_off + (blk * 8 + kq) * 32) : 0;
        acc0 += k16_term<T>(cur, da0, I0, M0);
        if (DBG && kq == 0) {
            const uint32_t row = tile * kTileRows + n;
            if (row < a.rows) {
                a.dbg_isum[(uint64_t)row * nb + blk] = I0;
                a.dbg_imin[(uint64_t)row * nb + blk] = M0;
            }
        }
        if (two_groups) {
            const float da1 = *(const float*)(lds + L.d_off + (blk * 8 + kq + 4) * 4);
            const int32_t I1 = k16_isum<T>(o, A.p1 + blk * A.step1);
            int32_t M1 = 0;
            if constexpr (T == kQ2_K)
                M1 = kq + 4 < a.batch ? q2_mins(cur.sc, lds + L.bs_off + (blk * 8 + kq + 4) * 32) : 0;
            acc1 += k16_term<T>(cur, da1, I1, M1);
        }
        if (++blk == nb) {
            const uint32_t row = tile * kTileRows + n;
            store_out(a, row, kq, acc0, best0);
            store_out(a, row, kq + 4, acc1, best1);
            acc0 = acc1 = 0.0f;
            blk = 0;
            tile += tw;
        }
    };
    pipeline<D>(steps, buf, issue, compute);
    fold_argmax(a, lds, L, kq, best0);
    fold_argmax(a, lds, L, kq + 4, best1);
    finish_argmax(a, lds, L);
}

// K split over KS waves per tile (TS = W / KS tile slots per workgroup), for
// matrices with too few tiles to fill the chip one wave per tile.  Each wave
// takes blocks kp, kp + KS, ... of its slot's tiles and parks every block's
// f32 term per (row, column) in LDS; after the last tile the workgroup adds
// each row's terms in block order from 0, which is the reference's own
// sequence for Q2_K.  LDS: the activation image, then the terms
// [tmax * TS][nb][16][batch] f32.
__host__ __device__ inline uint32_t k16_part_off(uint32_t t, uint32_t cols, uint32_t batch) {
    return (lds_map(t, cols, batch).total + 15u) & ~15u;
}

// BAL: the balanced deal over a.deal_cus CUs (balanced_deal; one matrix).
template <uint32_t T, int W, int KS, int D, bool DBG, bool BAL = false>
__global__ __launch_bounds__(W * 64) void k16_mv_split_kernel(MvArgs a) {
    constexpr int TS = W / KS;
    static_assert(!BAL || TS == 2 || TS == 4, "the balanced deal takes two or four tile slots");
    constexpr uint32_t kChunk = T == kQ3_K ? kQ3KChunk : kQ2KChunk;
    if (!mv_enter(a)) return;
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsMap L = lds_map(T, a.cols, a.batch);
    float* part = (float*)(lds + k16_part_off(T, a.cols, a.batch));
    const uint32_t lane = threadIdx.x & 63, n = lane & 15, kq = lane >> 4;
    // wave-uniform indices in scalar registers: loop control stays on the SALU
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t ts = wave / KS, kp = wave % KS;
    const uint32_t nb = a.nb, ntiles = a.ntiles, batch = a.batch;
    const uint32_t tstride = gridDim.x * TS, t0 = blockIdx.x * TS + ts;
    // this wave's tiles: tile_of(i) for i < my_tiles; half_ti the ordinal of
    // its half tile (none: ~0) and hsel its half
    uint32_t tmax, my_tiles, half_ti = ~0u, hsel = 0, bt = 0;
    if constexpr (BAL) {
        const TileDeal d = balanced_deal<TS>(a.deal_cus, ntiles, ts);
        tmax = 1, my_tiles = d.count, bt = d.tile, hsel = d.hsel;
        if (d.half) half_ti = 0;
    } else {
        tmax = (ntiles + tstride - 1) / tstride;
        my_tiles = t0 < ntiles ? (ntiles - 1 - t0) / tstride + 1 : 0;
    }
    auto tile_of = [&](uint32_t i) -> uint32_t {
        if constexpr (BAL) return bt;
        else return t0 + i * tstride;
    };
    auto own_row = [&](uint32_t i) { return i != half_ti || (n >> 3) == hsel; };
    const uint32_t nh = (n & 7) | (hsel << 3);
    const uint32_t bpt = kp < nb ? (nb - 1 - kp) / KS + 1 : 0;  // blocks of each tile this wave takes
    const uint32_t steps = my_tiles * bpt;

    if (threadIdx.x < 16) *(uint4*)(lds + L.zero_off + threadIdx.x * 16) = make_uint4(0, 0, 0, 0);
    if (threadIdx.x < 8) ((unsigned long long*)(lds + L.am_off))[threadIdx.x] = 0ull;
    float xv[16];
    prefetch_unit(a, wave, xv);

    // loads run D steps ahead; past the wave's last step they repeat a valid chunk
    const uint32_t kp0 = kp < nb ? kp : nb - 1;
    uint32_t ld_tile = t0 < ntiles ? t0 : ntiles - 1, ld_blk = kp0;
    if constexpr (BAL) ld_tile = my_tiles ? bt : 0;
    K16Step<T> buf[D];
    auto issue = [&](K16Step<T>& st) {
        const uint8_t* base = a.w + ((uint64_t)ld_tile * nb + ld_blk) * kChunk;
        if (BAL && half_ti == 0) k16_issue<T>(st, base, kq * 16 + nh, nh, kq);  // the half tile
        else k16_issue<T>(st, base, lane, n, kq);
        ld_blk += KS;
        if (ld_blk >= nb) {
            ld_blk = kp0;
            if (!BAL && ld_tile + tstride < ntiles) ld_tile += tstride;
        }
    };
#pragma unroll
    for (int i = 0; i < D; ++i) issue(buf[i]);

    const bool ok = a.x ? stage_q8k<W, bsum_order(T)>(a, lds, L, wave, xv) : stage_planes<W>(a, lds, L, T);
    if (!ok) return finish_argmax(a, lds, L);
    if (a.zero_pair) return zero_slot_tiles<W, TS>(a, tmax, tstride);

    const K16A A = k16_a(lds, L, batch, n, kq);
    const bool two_groups = batch > 4;
    const uint32_t hsh = 4 * (kq >> 1);
    uint32_t ti = 0, tile = tile_of(0), blk = kp, j = 0;
    auto compute = [&](const K16Step<T>& cur) {
        const K16Ops<T> o = k16_ops<T>(cur, hsh);
        float* pt = part + ((uint64_t)((ti * TS + ts) * nb + blk) * 16 + n) * batch;
        const int32_t I0 = k16_isum<T>(o, A.p0 + blk * A.step0);
        int32_t M0 = 0;
        if (kq < batch) {
            if constexpr (T == kQ2_K) M0 = q2_mins(cur.sc, lds + L.bs_off + (blk * 8 + kq) * 32);
            pt[kq] = k16_term<T>(cur, *(const float*)(lds + L.d_off + (blk * 8 + kq) * 4), I0, M0);
        }
        if (DBG && kq == 0) {
            const uint32_t row = tile * kTileRows + n;
            if (row < a.rows && own_row(ti)) {
                a.dbg_isum[(uint64_t)row * nb + blk] = I0;
                a.dbg_imin[(uint64_t)row * nb + blk] = M0;
            }
        }
        if (two_groups) {
            const int32_t I1 = k16_isum<T>(o, A.p1 + blk * A.step1);
            if (kq + 4 < batch) {
                int32_t M1 = 0;
                if constexpr (T == kQ2_K) M1 = q2_mins(cur.sc, lds + L.bs_off + (blk * 8 + kq + 4) * 32);
                pt[kq + 4] = k16_term<T>(cur, *(const float*)(lds + L.d_off + (blk * 8 + kq + 4) * 4), I1, M1);
            }
        }
        blk += KS;
        if (++j == bpt) {
            j = 0;
            blk = kp;
            tile = tile_of(++ti);
        }
    };
    pipeline<D>(steps, buf, issue, compute);
    __syncthreads();

    // every parked (tile, row, column): its block terms added in block order
    for (uint32_t b = 0; b < batch; ++b) {
        unsigned long long best = 0;
        for (uint32_t it = threadIdx.x; it < tmax * TS * 16; it += W * 64) {
            const uint32_t r = it % 16, slot = it / 16, tsl = slot % TS, til = slot / TS;
            uint32_t t = blockIdx.x * TS + tsl + til * tstride;
            bool own = true;
            if constexpr (BAL) {  // the slot's tile in the deal, and its own rows
                const TileDeal d = balanced_deal<TS>(a.deal_cus, ntiles, tsl);
                t = d.count ? d.tile : ntiles;
                own = !d.half || (r >> 3) == d.hsel;
            }
            const uint32_t row = t * kTileRows + r;
            if (t < ntiles && row < a.rows && own) {
                const float* pr = part + ((uint64_t)slot * nb * 16 + r) * batch + b;
                float v = 0.0f;
                for (uint32_t k = 0; k < nb; ++k) v += pr[(uint64_t)k * 16 * batch];
                store_out(a, row, b, v, best);
            }
        }
        if (a.am_out) {
#pragma unroll
            for (int m = 1; m < 64; m <<= 1) {
                const unsigned long long o = __shfl_xor(best, m, 64);
                best = o > best ? o : best;
            }
            if (lane == 0 && best) atomicMax((unsigned long long*)(lds + L.am_off) + b, best);
        }
    }
    finish_argmax(a, lds, L);
}

// ---------------------------------------------------------------------------
// Q8_0: one step is a pair of 32-element blocks
// ---------------------------------------------------------------------------
struct Q8Step {
    uint4 q;
    uint32_t d;
};

template <int W, int D, bool DBG>
__global__ __launch_bounds__(W * 64) void q8_0_mv_kernel(MvArgs a) {
    RLQ_MV_PROLOGUE(kQ8_0, a.nchunks)
    const uint32_t nb = a.nb, np = a.nchunks;
    Q8Step buf[D];
    auto issue = [&](Q8Step& st) {
        const uint8_t* base = a.w + ((uint64_t)ld_tile * np + ld_chunk) * kQ80Chunk;
        st.q = load_stream16(base + lane * 16);
        st.d = __builtin_nontemporal_load((const uint32_t*)(base + 1024 + n * 4));
        next_load();
    };
#pragma unroll
    for (int i = 0; i < D; ++i) issue(buf[i]);

    const bool ok = a.x ? stage_q8_0<W>(a, lds, L, wave, xv) : stage_planes<W>(a, lds, L, kQ8_0);
    if (!ok) return finish_argmax(a, lds, L);
    if (a.zero_pair) return zero_wave_tiles(a, gw, tw, n, kq);

    // A operand: lane row r = n holds column r / 2 and block 2p + r % 2; it is
    // nonzero in the K quarters (kq / 2 == r % 2) of that block.
    const uint32_t ab = n >> 1, which = n & 1;
    const bool a_live = which == (kq >> 1) && ab < a.batch;
    const uint8_t* a_ptr = a_live ? lds + ab * L.S + 32 * which + 16 * (kq & 1) : lds + L.zero_off;
    const uint32_t a_step = a_live ? 64 : 0;
    const uint32_t b0 = 2 * kq;

    float acc0 = 0.0f, acc1 = 0.0f;
    unsigned long long best0 = 0, best1 = 0;
    uint32_t tile = gw, p = 0;
    auto compute = [&](const Q8Step& cur) {
        const bool second = 2 * p + 1 < nb;  // false only for the odd last block of a row
        i32x4 av = *(const i32x4*)(a_ptr + p * a_step);
        if (!second && which) av = i32x4{0, 0, 0, 0};
        const i32x4 dot = mfma_i8(av, i32x4{(int)cur.q.x, (int)cur.q.y, (int)cur.q.z, (int)cur.q.w});
        // sum += isum as f32 * (dx * dy), block 2p then 2p + 1 (matvec.rs:124-128)
        const float dx0 = half_to_float(cur.d), dx1 = half_to_float(cur.d >> 16);
        const float2 dy0 = *(const float2*)(lds + L.d_off + (2 * p * 8 + b0) * 4);
        acc0 += (float)dot[0] * (dx0 * dy0.x);
        acc1 += (float)dot[2] * (dx0 * dy0.y);
        if (second) {
            const float2 dy1 = *(const float2*)(lds + L.d_off + ((2 * p + 1) * 8 + b0) * 4);
            acc0 += (float)dot[1] * (dx1 * dy1.x);
            acc1 += (float)dot[3] * (dx1 * dy1.y);
        }
        if (DBG && kq == 0) {
            const uint32_t row = tile * kTileRows + n;
            if (row < a.rows) {
                a.dbg_isum[(uint64_t)row * nb + 2 * p] = dot[0];
                a.dbg_imin[(uint64_t)row * nb + 2 * p] = 0;
                if (second) {
                    a.dbg_isum[(uint64_t)row * nb + 2 * p + 1] = dot[1];
                    a.dbg_imin[(uint64_t)row * nb + 2 * p + 1] = 0;
                }
            }
        }
        if (++p == np) {
            const uint32_t row = tile * kTileRows + n;
            store_out(a, row, b0, acc0, best0);
            store_out(a, row, b0 + 1, acc1, best1);
            acc0 = acc1 = 0.0f;
            p = 0;
            tile += tw;
        }
    };
    pipeline<D>(steps, buf, issue, compute);
    fold_argmax(a, lds, L, b0, best0);
    fold_argmax(a, lds, L, b0 + 1, best1);
    finish_argmax(a, lds, L);
}

// Q8_0 with K split over KS waves per tile (the MFMA step of q8_0_mv_kernel):
// W waves hold TS = W / KS tile slots and the waves of a slot take chunks
// (block pairs) kp, kp + KS, ... of its tile, so a matrix of a few hundred
// tiles still spreads over every CU.  Every block's f32 term
// isum * (dx * dy) is parked in LDS [tmax][TS][nb][16][8] and the wave that
// completes a tile's count adds them in block order, the reference's order
// (matvec.rs:124-128): the outputs stay bit-exact.  COMPACT parks only the
// batch's columns ([..][16][batch]: long rows whose eight-column records
// would not fit LDS; slower where both fit, 4096x4096 10.0 against 8.8 us).
template <int W, int KS, int D, bool DBG, bool COMPACT = false>
__global__ __launch_bounds__(W * 64) void q8_0_mv_ks_kernel(MvArgs a) {
    constexpr int TS = W / KS;
    if (!mv_enter(a)) return;
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsMap L = lds_map(kQ8_0, a.cols, a.batch);
    float* part = (float*)(lds + ks_part_off(kQ8_0, a.cols, a.batch));
    const uint32_t lane = threadIdx.x & 63, n = lane & 15, kq = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t ts = wave / KS, kp = wave % KS;
    const uint32_t nb = a.nb, np = a.nchunks, ntiles = a.ntiles;
    const uint32_t tstride = gridDim.x * TS, t0 = blockIdx.x * TS + ts;
    const uint32_t tmax = (ntiles + tstride - 1) / tstride;
    const uint32_t my_tiles = t0 < ntiles ? (ntiles - 1 - t0) / tstride + 1 : 0;
    const uint32_t cpt = kp < np ? (np - 1 - kp) / KS + 1 : 0;  // chunks of each tile this wave takes
    const uint32_t steps = my_tiles * cpt;
    const uint32_t nk = (uint32_t)KS < np ? (uint32_t)KS : np;  // waves of a tile that take chunks
    const uint32_t pc = COMPACT ? a.batch : 8u;  // columns parked per row
    uint32_t* cnt = (uint32_t*)(part + tmax * TS * nb * 16 * pc);
    for (uint32_t i = threadIdx.x; i < tmax * TS; i += W * 64) cnt[i] = 0;
    if (threadIdx.x < 16) *(uint4*)(lds + L.zero_off + threadIdx.x * 16) = make_uint4(0, 0, 0, 0);
    if (threadIdx.x < 8) ((unsigned long long*)(lds + L.am_off))[threadIdx.x] = 0ull;
    float xv[16];
    prefetch_unit(a, wave, xv);

    const uint32_t kp0 = kp < np ? kp : np - 1;
    uint32_t ld_tile = t0 < ntiles ? t0 : ntiles - 1, ld_chunk = kp0;
    Q8Step buf[D];
    auto issue = [&](Q8Step& st) {
        const uint8_t* base = a.w + ((uint64_t)ld_tile * np + ld_chunk) * kQ80Chunk;
        st.q = load_stream16(base + lane * 16);
        st.d = __builtin_nontemporal_load((const uint32_t*)(base + 1024 + n * 4));
        ld_chunk += KS;
        if (ld_chunk >= np) {
            ld_chunk = kp0;
            if (ld_tile + tstride < ntiles) ld_tile += tstride;
        }
    };
#pragma unroll
    for (int i = 0; i < D; ++i) issue(buf[i]);

    const bool ok = a.x ? stage_q8_0<W>(a, lds, L, wave, xv) : stage_planes<W>(a, lds, L, kQ8_0);
    if (!ok) return finish_argmax(a, lds, L);
    if (a.zero_pair) return zero_slot_tiles<W, TS>(a, tmax, tstride);

    // A operand: lane row r = n holds column r / 2 and block 2p + r % 2; it is
    // nonzero in the K quarters (kq / 2 == r % 2) of that block.
    const uint32_t ab = n >> 1, which = n & 1;
    const bool a_live = which == (kq >> 1) && ab < a.batch;
    const uint8_t* a_ptr = a_live ? lds + ab * L.S + 32 * which + 16 * (kq & 1) : lds + L.zero_off;
    const uint32_t a_step = a_live ? 64 : 0;
    const uint32_t b0 = 2 * kq;

    uint32_t ti = 0, p = kp, j = 0, tile = t0;
    auto compute = [&](const Q8Step& cur) {
        const bool second = 2 * p + 1 < nb;  // false only for the odd last block of a row
        i32x4 av = *(const i32x4*)(a_ptr + p * a_step);
        if (!second && which) av = i32x4{0, 0, 0, 0};
        const i32x4 dot = mfma_i8(av, i32x4{(int)cur.q.x, (int)cur.q.y, (int)cur.q.z, (int)cur.q.w});
        // the terms isum as f32 * (dx * dy) of blocks 2p and 2p + 1
        // (matvec.rs:124-128), parked for the in-order sum
        const float dx0 = half_to_float(cur.d), dx1 = half_to_float(cur.d >> 16);
        const float2 dy0 = *(const float2*)(lds + L.d_off + (2 * p * 8 + b0) * 4);
        float* pt = part + (((ti * TS + ts) * nb + 2 * p) * 16 + n) * pc + b0;
        if constexpr (COMPACT) {
            if (b0 < pc) pt[0] = (float)dot[0] * (dx0 * dy0.x);
            if (b0 + 1 < pc) pt[1] = (float)dot[2] * (dx0 * dy0.y);
        } else {
            *(float2*)pt = make_float2((float)dot[0] * (dx0 * dy0.x), (float)dot[2] * (dx0 * dy0.y));
        }
        if (second) {
            const float2 dy1 = *(const float2*)(lds + L.d_off + ((2 * p + 1) * 8 + b0) * 4);
            if constexpr (COMPACT) {
                if (b0 < pc) pt[16 * pc] = (float)dot[1] * (dx1 * dy1.x);
                if (b0 + 1 < pc) pt[16 * pc + 1] = (float)dot[3] * (dx1 * dy1.y);
            } else {
                *(float2*)(pt + 16 * 8) = make_float2((float)dot[1] * (dx1 * dy1.x), (float)dot[3] * (dx1 * dy1.y));
            }
        }
        if (DBG && kq == 0) {
            const uint32_t row = tile * kTileRows + n;
            if (row < a.rows) {
                a.dbg_isum[(uint64_t)row * nb + 2 * p] = dot[0];
                a.dbg_imin[(uint64_t)row * nb + 2 * p] = 0;
                if (second) {
                    a.dbg_isum[(uint64_t)row * nb + 2 * p + 1] = dot[1];
                    a.dbg_imin[(uint64_t)row * nb + 2 * p + 1] = 0;
                }
            }
        }
        p += KS;
        if (++j == cpt) {  // this wave's share of the tile is parked: count it
            const uint32_t slot = ti * TS + ts;
            // one wave's LDS operations are performed in order: the terms are
            // in place before the count
            if (lane == 0) {
                const uint32_t prev =
                    __hip_atomic_fetch_add(cnt + slot, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
                if (prev == nk - 1) cnt[slot] = nk + 1 + wave;  // this wave finishes the tile
            }
            j = 0;
            p = kp;
            ++ti;
            tile += tstride;
        }
    };
    pipeline<D>(steps, buf, issue, compute);

    unsigned long long best0 = 0, best1 = 0;
    for (uint32_t i = 0; i < my_tiles; ++i) {
        const uint32_t slot = i * TS + ts, row = (t0 + i * tstride) * kTileRows + n;
        if (cnt[slot] != nk + 1 + wave) continue;  // (the mark is wave-uniform)
        float s0 = 0.0f, s1 = 0.0f;
        if constexpr (COMPACT) {
            // (a lane's columns past the batch read column pc - 1 and are not stored)
            const uint32_t c0 = b0 < pc ? b0 : pc - 1, c1 = b0 + 1 < pc ? b0 + 1 : pc - 1;
            for (uint32_t blk = 0; blk < nb; ++blk) {
                const float* v = part + ((slot * nb + blk) * 16 + n) * pc;
                s0 += v[c0];
                s1 += v[c1];
            }
        } else {
            for (uint32_t blk = 0; blk < nb; ++blk) {
                const float2 v = *(const float2*)(part + ((slot * nb + blk) * 16 + n) * 8 + b0);
                s0 += v.x;
                s1 += v.y;
            }
        }
        store_out(a, row, b0, s0, best0);
        store_out(a, row, b0 + 1, s1, best1);
    }
    fold_argmax(a, lds, L, b0, best0);
    fold_argmax(a, lds, L, b0 + 1, best1);
    finish_argmax(a, lds, L);
}
// Q3_K, one column, in the reference's f32 order (matvec_extra.rs:235-248,
// 287-292): eight lane accumulators lanes[j % 8] per row over all blocks,
// integers[l] the sum over the scale groups g of scale_g times the group's
// dot over the elements j with j % 8 == l, then sum = 0 + lanes[0] + ... +
// lanes[7].  The chunk loads and B operands are those of the K16 kernels
// (lane (n, kq), operand s: elements 128 (kq / 2) + 32 s + 16 (kq % 2) + i of
// row n, scale group 8 (kq / 2) + 2 s + kq % 2); the A rows split each
// group's dot by lane class as in q6k_mv_one_kernel: A row r holds class
// c = r % 8 of K quarter r / 8 (first MFMA of a pair) or 2 + r / 8 (second),
// the activations of that quarter's elements masked to the bytes c and c + 8.
// Output i of the pair in lane (n, kq) is the dot over class 4 (kq % 2) + i
// of scale group 2 s + kq / 2 (first) or 8 + 2 s + kq / 2 (second); the lanes
// kq and kq ^ 2 hold the other eight groups.  A wave takes whole tiles and
// walks their blocks in order, so the accumulators stay in registers.
template <int W, int D, bool DBG>
__global__ __launch_bounds__(W * 64) void q3k_mv_one_kernel(MvArgs a) {
    RLQ_MV_PROLOGUE(kQ3_K, a.nb)
    const uint32_t nb = a.nb;
    K16Step<kQ3_K> buf[D];
    auto issue = [&](K16Step<kQ3_K>& st) {
        k16_issue<kQ3_K>(st, a.w + ((uint64_t)ld_tile * nb + ld_chunk) * kQ3KChunk, lane, n, kq);
        next_load();
    };
#pragma unroll
    for (int i = 0; i < D; ++i) issue(buf[i]);

    const bool ok = a.x ? stage_q8k<W, kBsNone>(a, lds, L, wave, xv) : stage_planes<W>(a, lds, L, kQ3_K);
    if (!ok) return finish_argmax(a, lds, L);
    if (a.zero_pair) return zero_wave_tiles(a, gw, tw, n, kq);

    const uint32_t hsh = 4 * (kq >> 1), sb0 = kq >> 1;  // high-mask bits; scale byte of the output groups
    const uint32_t cls = n & 7, qsel = n >> 3;
    const bool live0 = kq == qsel, live1 = kq == 2 + qsel;
    const uint8_t* a_ptr = live0 || live1 ? lds + 128 * (kq >> 1) + 16 * (kq & 1) : lds + L.zero_off;
    const uint32_t a_step = live0 || live1 ? 256 : 0;
    const uint32_t byte = 0xffu << (8 * (cls & 3));
    uint32_t m0[4], m1[4];  // the masks of the two MFMAs (zero where not live)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t mk = (uint32_t)(w & 1) == (cls >> 2) ? byte : 0u;
        m0[w] = live0 ? mk : 0u;
        m1[w] = live1 ? mk : 0u;
    }

    float lanes[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // classes 4 (kq % 2) + i
    unsigned long long best = 0;
    uint32_t tile = gw, blk = 0;
    auto compute = [&](const K16Step<kQ3_K>& cur) {
        const K16Ops<kQ3_K> o = k16_ops<kQ3_K>(cur, hsh);
        const uint8_t* p = a_ptr + blk * a_step;
        int32_t I[4] = {0, 0, 0, 0};
#pragma unroll
        for (int sft = 0; sft < 4; ++sft) {
            const uint4 x = *(const uint4*)(p + 32 * sft);
            const i32x4 A0 = {(int)(x.x & m0[0]), (int)(x.y & m0[1]), (int)(x.z & m0[2]), (int)(x.w & m0[3])};
            const i32x4 A1 = {(int)(x.x & m1[0]), (int)(x.y & m1[1]), (int)(x.z & m1[2]), (int)(x.w & m1[3])};
            const i32x4 d0 = mfma_i8(A0, o.wv[sft]), d1 = mfma_i8(A1, o.wv[sft]);
            // the signed 6-bit scales of groups 2 s + kq / 2 and 8 + 2 s + kq / 2
            const int32_t sa = sbyte(o.c[sft >> 1], 2 * (sft & 1) + sb0);
            const int32_t sb = sbyte(o.c[2 + (sft >> 1)], 2 * (sft & 1) + sb0);
#pragma unroll
            for (int i = 0; i < 4; ++i) I[i] = mad24(sa, d0[i], mad24(sb, d1[i], I[i]));
        }
        const float d = half_to_float(cur.d) * *(const float*)(lds + L.d_off + blk * 32);  // :246
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            I[i] = sum_xor32(I[i]);
            lanes[i] += d * (float)I[i];  // matvec_extra.rs:287-289
        }
        if (DBG) {
            const int32_t It = sum_xor16(I[0] + I[1] + I[2] + I[3]);
            const uint32_t row = tile * kTileRows + n;
            if (kq == 0 && row < a.rows) {
                a.dbg_isum[(uint64_t)row * nb + blk] = It;
                a.dbg_imin[(uint64_t)row * nb + blk] = 0;
            }
        }
        if (++blk == nb) {  // sum = 0 + lanes[0] + ... + lanes[7] (:290-292)
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) sum += __shfl(lanes[i], (int)n, 64);
#pragma unroll
            for (int i = 0; i < 4; ++i) sum += __shfl(lanes[i], (int)(n + 16), 64);
            if (kq == 0) store_out(a, tile * kTileRows + n, 0, sum, best);
#pragma unroll
            for (int i = 0; i < 4; ++i) lanes[i] = 0.0f;
            blk = 0;
            tile += tw;
        }
    };
    pipeline<D>(steps, buf, issue, compute);
    fold_argmax(a, lds, L, kq, best);
    finish_argmax(a, lds, L);
}

// Q3_K and Q6_K, one column, the blocks of each tile split over KS waves:
// the class dots of q3k_mv_one_kernel / q6k_mv_one_kernel, each block's four
// class terms d * integers[l] (rounded to f32, matvec_extra.rs:287-289)
// parked in LDS per lane (classes 0..3 in lane kq = 0 of row n, 4..7 in lane
// kq = 1), and after the last step one wave per tile slot forms each row's
// sum in the reference's order: lanes[l] over the blocks in order, then
// sum = 0 + lanes[0] + ... + lanes[7].  LDS after the Q8_K image:
// [tmax][TS][nb][32] float4.  BAL: the balanced deal over a.deal_cus CUs
// (balanced_deal; one tile per slot, a half tile read by lane pairs and
// stored by its own half).
__host__ __device__ inline uint32_t split_part_off(uint32_t t, uint32_t cols) {
    return (lds_map(t, cols, 1).total + 15u) & ~15u;
}
__host__ __device__ inline uint32_t split_lds(uint32_t t, uint32_t cols, uint32_t tmax, uint32_t ts) {
    return split_part_off(t, cols) + tmax * ts * (cols / 256) * 512u;
}

// The Q3_K class operands of lane (n, kq), as q3k_mv_one_kernel's: the
// lane's activations (a_step bytes per block; the zero bytes where neither
// MFMA of a pair is live) masked by m0 / m1 to class n % 8.
struct Q3OneOps {
    const uint8_t* a_ptr;
    uint32_t a_step, hsh, sb0;
    uint32_t m0[4], m1[4];
};
__device__ __forceinline__ Q3OneOps q3_one_ops(const uint8_t* lds, const LdsMap& L, uint32_t n, uint32_t kq) {
    Q3OneOps o;
    o.hsh = 4 * (kq >> 1), o.sb0 = kq >> 1;
    const uint32_t cls = n & 7, qsel = n >> 3;
    const bool live0 = kq == qsel, live1 = kq == 2 + qsel;
    o.a_ptr = live0 || live1 ? lds + 128 * (kq >> 1) + 16 * (kq & 1) : lds + L.zero_off;
    o.a_step = live0 || live1 ? 256 : 0;
    const uint32_t byte = 0xffu << (8 * (cls & 3));
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t mk = (uint32_t)(w & 1) == (cls >> 2) ? byte : 0u;
        o.m0[w] = live0 ? mk : 0u;
        o.m1[w] = live1 ? mk : 0u;
    }
    return o;
}
__device__ __forceinline__ void q3_one_ints(const K16Step<kQ3_K>& cur, const Q3OneOps& ops, const uint8_t* p,
                                            int32_t (&I)[4]) {
    const K16Ops<kQ3_K> o = k16_ops<kQ3_K>(cur, ops.hsh);
#pragma unroll
    for (int sft = 0; sft < 4; ++sft) {
        const uint4 x = *(const uint4*)(p + 32 * sft);
        const i32x4 A0 = {(int)(x.x & ops.m0[0]), (int)(x.y & ops.m0[1]), (int)(x.z & ops.m0[2]), (int)(x.w & ops.m0[3])};
        const i32x4 A1 = {(int)(x.x & ops.m1[0]), (int)(x.y & ops.m1[1]), (int)(x.z & ops.m1[2]), (int)(x.w & ops.m1[3])};
        const i32x4 d0 = mfma_i8(A0, o.wv[sft]), d1 = mfma_i8(A1, o.wv[sft]);
        const int32_t sa = sbyte(o.c[sft >> 1], 2 * (sft & 1) + ops.sb0);
        const int32_t sb = sbyte(o.c[2 + (sft >> 1)], 2 * (sft & 1) + ops.sb0);
#pragma unroll
        for (int i = 0; i < 4; ++i) I[i] = mad24(sa, d0[i], mad24(sb, d1[i], I[i]));
    }
}

template <uint32_t T>
using SplitStep = std::conditional_t<T == kQ6_K, Q6Step, K16Step<kQ3_K>>;
template <uint32_t T>
using SplitOps = std::conditional_t<T == kQ6_K, Q6OneOps, Q3OneOps>;

template <uint32_t T, int W, int KS, int D, bool DBG, bool BAL = false>
__global__ __launch_bounds__(W * 64) void split_one_kernel(MvArgs a) {
    static_assert(T == kQ3_K || T == kQ6_K, "the one-column split kernel takes Q3_K and Q6_K");
    constexpr int TS = W / KS;
    static_assert(!BAL || TS == 2 || TS == 4, "the balanced deal takes two or four tile slots");
    if (!mv_enter(a)) return;
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsMap L = lds_map(T, a.cols, a.batch);
    const uint32_t lane = threadIdx.x & 63, n = lane & 15, kq = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t ts = wave / KS, kp = wave % KS;
    const uint32_t nb = a.nb, ntiles = a.ntiles;
    const uint32_t tstride = gridDim.x * TS, t0 = blockIdx.x * TS + ts;
    uint32_t tmax, my_tiles, half = 0, hsel = 0, bt = 0;
    if constexpr (BAL) {
        const TileDeal dl = balanced_deal<TS>(a.deal_cus, ntiles, ts);
        tmax = 1, my_tiles = dl.count, bt = dl.tile, half = dl.half, hsel = dl.hsel;
    } else {
        tmax = (ntiles + tstride - 1) / tstride;
        my_tiles = t0 < ntiles ? (ntiles - 1 - t0) / tstride + 1 : 0;
    }
    const uint32_t nh = (n & 7) | (hsel << 3);  // the row a lane loads in a half tile
    const uint32_t bpt = kp < nb ? (nb - 1 - kp) / KS + 1 : 0;  // blocks of each tile this wave takes
    const uint32_t steps = my_tiles * bpt;
    float4* park = (float4*)(lds + split_part_off(T, a.cols));

    if (threadIdx.x < 16) *(uint4*)(lds + L.zero_off + threadIdx.x * 16) = make_uint4(0, 0, 0, 0);
    if (threadIdx.x < 8) ((unsigned long long*)(lds + L.am_off))[threadIdx.x] = 0ull;
    float xv[16];
    prefetch_unit(a, wave, xv);

    // loads run D steps ahead; past the wave's last step they repeat a valid chunk
    const uint32_t kp0 = kp < nb ? kp : nb - 1;
    uint32_t ld_tile = t0 < ntiles ? t0 : ntiles - 1, ld_blk = kp0;
    if constexpr (BAL) ld_tile = my_tiles ? bt : 0;
    SplitStep<T> buf[D];
    auto issue = [&](SplitStep<T>& st) {
        const uint8_t* base = a.w + ((uint64_t)ld_tile * nb + ld_blk) * (T == kQ6_K ? kQ6KChunk : kQ3KChunk);
        const uint32_t ln = BAL && half ? kq * 16 + nh : lane, r = BAL && half ? nh : n;  // (a half tile)
        if constexpr (T == kQ6_K) q6_issue(st, base, ln, r, kq);
        else k16_issue<kQ3_K>(st, base, ln, r, kq);
        ld_blk += KS;
        if (ld_blk >= nb) {
            ld_blk = kp0;
            if (!BAL && ld_tile + tstride < ntiles) ld_tile += tstride;
        }
    };
#pragma unroll
    for (int i = 0; i < D; ++i) issue(buf[i]);

    const bool ok = a.x ? stage_q8k<W, kBsNone>(a, lds, L, wave, xv) : stage_planes<W>(a, lds, L, T);
    if (!ok) return finish_argmax(a, lds, L);
    if (a.zero_pair) return zero_slot_tiles<W, TS>(a, tmax, tstride);

    SplitOps<T> ops;
    if constexpr (T == kQ6_K) ops = q6_one_ops(lds, L, n, kq);
    else ops = q3_one_ops(lds, L, n, kq);

    uint32_t ti = 0, tile = BAL ? bt : t0, blk = kp, j = 0;
    auto compute = [&](const SplitStep<T>& cur) {
        int32_t I[4] = {0, 0, 0, 0};
        if constexpr (T == kQ6_K) q6_one_ints(cur, ops, ops.a_ptr + blk * ops.a_step, I);
        else q3_one_ints(cur, ops, ops.a_ptr + blk * ops.a_step, I);
        const float d = half_to_float(cur.d) * *(const float*)(lds + L.d_off + blk * 32);  // :246
#pragma unroll
        for (int i = 0; i < 4; ++i) I[i] = sum_xor32(I[i]);
        if (kq < 2)
            park[((ti * TS + ts) * nb + blk) * 32 + lane] =
                make_float4(d * (float)I[0], d * (float)I[1], d * (float)I[2], d * (float)I[3]);
        if (DBG) {
            const int32_t It = sum_xor16(I[0] + I[1] + I[2] + I[3]);
            const uint32_t row = tile * kTileRows + n;
            if (kq == 0 && row < a.rows && (!half || (n >> 3) == hsel)) {
                a.dbg_isum[(uint64_t)row * nb + blk] = It;
                a.dbg_imin[(uint64_t)row * nb + blk] = 0;
            }
        }
        blk += KS;
        if (++j == bpt) {
            j = 0;
            blk = kp;
            ++ti;
            tile += tstride;
        }
    };
    pipeline<D>(steps, buf, issue, compute);
    __syncthreads();

    // each row's sum in the reference's order, one wave per tile slot (in a
    // half tile lane pairs hold the same row; the own half stores it)
    unsigned long long best = 0;
    for (uint32_t slot = wave; slot < tmax * TS; slot += W) {  // (wave-uniform)
        uint32_t t = blockIdx.x * TS + slot % TS + (slot / TS) * tstride;
        bool own = true;
        if constexpr (BAL) {
            const TileDeal dl = balanced_deal<TS>(a.deal_cus, ntiles, slot);
            if (!dl.count) continue;
            t = dl.tile;
            own = !dl.half || (n >> 3) == dl.hsel;
        }
        if (t >= ntiles) continue;
        const float4* pk = park + (uint64_t)slot * nb * 32 + (lane & 31);
        float c0 = 0.0f, c1 = 0.0f, c2 = 0.0f, c3 = 0.0f;
        uint32_t b = 0;
        for (; b + 8 <= nb; b += 8) {  // eight blocks' loads before their adds
            float4 v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = pk[(b + k) * 32];
#pragma unroll
            for (int k = 0; k < 8; ++k) c0 += v[k].x, c1 += v[k].y, c2 += v[k].z, c3 += v[k].w;
        }
        for (; b < nb; ++b) {
            const float4 v = pk[b * 32];
            c0 += v.x, c1 += v.y, c2 += v.z, c3 += v.w;
        }
        // classes 4..7 of row n sit in lane n + 16 (row 1 of the wave)
        const float h0 = row_from(c0, 1), h1 = row_from(c1, 1), h2 = row_from(c2, 1), h3 = row_from(c3, 1);
        float sum = 0.0f;
        sum += c0;
        sum += c1;
        sum += c2;
        sum += c3;
        sum += h0;
        sum += h1;
        sum += h2;
        sum += h3;
        const uint32_t row = t * kTileRows + n;
        if (kq == 0 && row < a.rows && own) store_out(a, row, 0, sum, best);
    }
    fold_argmax(a, lds, L, 0, best);
    finish_argmax(a, lds, L);
}

#undef RLQ_MV_PROLOGUE

// ---------------------------------------------------------------------------
// host dispatch
// ---------------------------------------------------------------------------
constexpr int kMvWaves = 4;
constexpr size_t kMaxLds = 160 * 1024;

int device_cus() {
    static std::atomic<int> cus[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int v = cus[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cus[dev].store(v, std::memory_order_relaxed);  // every thread stores the same count
    return v;
}

// Grid rows (MUL_MAT_ID pairs of this launch, else 1) and the workgroups per
// row: the device's budget of `cap` workgroups is shared by the rows.
static uint32_t grid_rows(const MvArgs& a, uint32_t pairs) { return a.ids ? pairs : 1u; }
static uint32_t grid_cols(uint32_t want, uint32_t cap, uint32_t rows) {
    const uint32_t per = cap / rows > 0 ? cap / rows : 1u;
    return want < per ? want : per;
}

// per_cu workgroups of W waves per CU at most (Q8_0 151936x896 with W = 4:
// 25.8 us at three, 27.5 at two; Q6_K 128256x4096 with the argmax: one of 8
// waves 71.8 us, two of 4 72.7-75.4, and at 8 columns 83.3 against 88.4).
// The kernel is a template argument so that each kernel keeps its own limit.
template <int W, void (*kernel)(MvArgs)>
static hipError_t launch_one(const MvArgs& a, size_t lds, hipStream_t s, uint32_t pairs, uint32_t per_cu = 2) {
    static LdsLimit lds_limit;
    if (const hipError_t e = lds_limit.raise((const void*)kernel, lds); e != hipSuccess) return e;
    const uint32_t want = (a.ntiles + W - 1) / W;
    const uint32_t gy = grid_rows(a, pairs);
    const uint32_t grid = grid_cols(want, per_cu * (uint32_t)device_cus(), gy);
    if (a.am_out && grid > kArgmaxMaxGrid) return hipErrorInvalidValue;
    hipLaunchKernelGGL(kernel, dim3(grid, gy), dim3(W * 64), lds, s, a);
    return hipGetLastError();
}

// Small-batch Q4_K kernel: W waves per workgroup, K of each tile split over
// KS waves, about kSmallWgPerCu workgroups per CU.
constexpr int kSmallW = 8, kSmallKS = 8, kSmallD = 2, kSmallWgPerCu = 2;

// The one-column small kernel: the grid and the LDS of its parked terms
// [tmax][TS][nb].  lds_limit is the kernel's own dynamic-LDS limit.
template <int W, int KS>
static hipError_t launch_parked(void (*kernel)(MvArgs), LdsLimit& lds_limit, const MvArgs& a, hipStream_t s,
                                uint32_t pairs, bool exp) {
    constexpr int TS = W / KS;
    if (a.batch != 1) return hipErrorInvalidValue;
    const uint32_t want = (a.ntiles + TS - 1) / TS;
    const uint32_t gy = grid_rows(a, pairs);
    uint32_t grid = grid_cols(want, (uint32_t)kSmallWgPerCu * (uint32_t)device_cus(), gy);
    // enough workgroups that every one parks at most `room` tiles' terms
    const size_t off = one_part_off(a.cols, exp), per_tile = (size_t)TS * park_bytes(a.nb);
    if (off >= kMaxLds || (kMaxLds - off) / per_tile == 0) return hipErrorInvalidValue;
    const uint64_t room = (kMaxLds - off) / per_tile, need = (a.ntiles + room * TS - 1) / (room * TS);
    if (grid < need) grid = (uint32_t)need;
    const uint32_t tstride = grid * TS, tmax = (a.ntiles + tstride - 1) / tstride;
    const size_t lds = small_lds_bytes(a.cols, tmax, TS, exp);
    if (lds > kMaxLds || (a.am_out && grid > kArgmaxMaxGrid)) return hipErrorInvalidValue;
    if (const hipError_t e = lds_limit.raise((const void*)kernel, lds); e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, dim3(grid, gy), dim3(W * 64), lds, s, a);
    return hipGetLastError();
}

// The expanded image where one tile's terms per slot fit beside it (K up
// to about 16K), else the compact one.
template <uint32_t T, int W, int KS, int D, bool DBG>
static hipError_t launch_small(const MvArgs& a, hipStream_t s, uint32_t pairs) {
    static LdsLimit lds_exp, lds_cmp;
    constexpr int TS = W / KS;
    if (one_part_off(a.cols, true) + (size_t)TS * park_bytes(a.nb) <= kMaxLds)
        return launch_parked<W, KS>(q4k_mv_small_kernel<T, W, KS, D, DBG, true>, lds_exp, a, s, pairs, true);
    return launch_parked<W, KS>(q4k_mv_small_kernel<T, W, KS, D, DBG, false>, lds_cmp, a, s, pairs, false);
}

// The batch-1 kernel: grid as launch_parked (enough workgroups that the
// parked partials fit in LDS), the LDS of b1_lds_bytes.
template <int W, int KS>
static void b1_grid(const MvArgs& a, uint32_t& grid, uint32_t& tmax) {
    constexpr int TS = W / KS;
    grid = grid_cols((a.ntiles + TS - 1) / TS, (uint32_t)kSmallWgPerCu * (uint32_t)device_cus(), 1);
    const size_t off = one_part_off(a.cols, true), per_tile = (size_t)TS * (park_bytes(a.nb) + 4u + 64u);
    const uint64_t room = off < kMaxLds ? (kMaxLds - off) / per_tile : 0;
    if (room == 0) {
        grid = tmax = 0;
        return;
    }
    const uint64_t need = (a.ntiles + room * TS - 1) / (room * TS);
    if (grid < need) grid = (uint32_t)need;
    tmax = (a.ntiles + grid * TS - 1) / (grid * TS);
}

// Whether the batch-1 kernel with W waves and a K split of KS takes a call:
// at most 4 blocks per wave, no SiLU pair, the residual only with at most 4
// tiles per slot (they are loaded up front).
template <int W, int KS>
static bool b1_takes(const MvArgs& a) {
    if (a.nb > 4u * KS || a.epilogue != kEpStore) return false;
    uint32_t grid, tmax;
    b1_grid<W, KS>(a, grid, tmax);
    return grid > 0 && (!a.resid || tmax <= 4);
}

// The balanced deal: u = 2 ntiles / CUs half tiles a CU, 3 <= u <= 8 (0:
// the tiles do not divide so), in workgroups of TS tile slots (the CU's
// (u + 1) / 2 slots, rounded up to whole workgroups).
static uint32_t b1_bal_units(const MvArgs& a) {
    const uint32_t cus = (uint32_t)device_cus();
    if (cus == 0 || (2ull * a.ntiles) % cus != 0) return 0;
    const uint64_t u = 2ull * a.ntiles / cus;
    return u < 3 || u > 8 || (u % 2 == 1 && cus % 2 != 0) ? 0 : (uint32_t)u;
}
template <int TS>
static void b1_bal_grid(const MvArgs& a, uint32_t& grid, uint32_t& tmax) {
    const uint32_t u = b1_bal_units(a);
    grid = u ? ((u + 1) / 2 + TS - 1) / TS * (uint32_t)device_cus() : 0;
    tmax = u ? 1 : 0;
}

template <int W, int KS>
static bool b1_bal_takes(const MvArgs& a) {
    constexpr int TS = W / KS;
    if ((TS != 2 && TS != 4) || a.nb > 4u * KS || a.epilogue != kEpStore) return false;
    uint32_t grid, tmax;
    b1_bal_grid<TS>(a, grid, tmax);
    return grid > 0 && b1_lds_bytes(a.cols, tmax, TS) <= kMaxLds;
}

template <uint32_t T, int W, int KS, int D, bool DBG, bool FULL, bool BAL = false>
static hipError_t launch_b1(const MvArgs& a, hipStream_t s) {
    constexpr int TS = W / KS;
    static LdsLimit lds_limit;
    auto kernel = q45_mv_b1_kernel<T, W, KS, D, DBG, FULL, BAL>;
    uint32_t grid, tmax;
    if constexpr (BAL) b1_bal_grid<TS>(a, grid, tmax);
    else b1_grid<W, KS>(a, grid, tmax);
    const size_t lds = b1_lds_bytes(a.cols, tmax, TS);
    if (grid == 0 || lds > kMaxLds || (a.am_out && grid > kArgmaxMaxGrid) || (a.resid && tmax > 4))
        return hipErrorInvalidValue;
    if (const hipError_t e = lds_limit.raise((const void*)kernel, lds); e != hipSuccess) return e;
    MvArgs b = a;
    b.deal_cus = BAL ? (uint32_t)device_cus() : 0;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(W * 64), lds, s, b);
    return hipGetLastError();
}

// Chunks in flight per wave: one with 16 waves per CU, two with 8, three
// with 4 (the weight chunks a CU has in flight before its activations arrive
// delay them, and too few starve the stream: 14336x4096 in the balanced deal
// 7.6 us at one against 7.9 at two, the down projection 4096x14336 10.0
// against 10.4; Q/K/V 6144x4096 with 8 waves 6.8 at two, 7.3 at one, 6.9 at
// three; O 4096x4096 with 4 waves 5.65 at three, 5.8 at two, 6.4 at one).
constexpr int b1_depth(int W) { return W >= 16 ? 1 : W >= 8 ? 2 : 3; }

template <uint32_t T, int W, int KS, bool BAL = false>
static hipError_t launch_b1_any(const MvArgs& a, bool dbg, bool full, hipStream_t s) {
    constexpr int D = b1_depth(W);
    return dbg ? (full ? launch_b1<T, W, KS, D, true, true, BAL>(a, s)
                       : launch_b1<T, W, KS, D, true, false, BAL>(a, s))
               : (full ? launch_b1<T, W, KS, D, false, true, BAL>(a, s)
                       : launch_b1<T, W, KS, D, false, false, BAL>(a, s));
}

// The K-split MFMA kernel for 3 to 8 columns: grid as launch_parked.
template <uint32_t T, int W, int KS, int D, bool DBG, bool PL, bool BAL = false>
static hipError_t launch_ks_pl(const MvArgs& a, hipStream_t s, uint32_t pairs) {
    constexpr int TS = W / KS;
    static LdsLimit lds_limit;
    auto kernel = q45_mv_ks_kernel<T, W, KS, D, DBG, PL, BAL>;
    const uint32_t gy = grid_rows(a, pairs);
    uint32_t grid, tmax;
    if constexpr (BAL) {  // one matrix, one grid row
        b1_bal_grid<TS>(a, grid, tmax);
        if (grid == 0 || gy != 1 || a.ids) return hipErrorInvalidValue;
    } else {
        grid = grid_cols((a.ntiles + TS - 1) / TS, (uint32_t)kSmallWgPerCu * (uint32_t)device_cus(), gy);
        const size_t off = ks_part_off(T, a.cols, a.batch), per_tile = (size_t)TS * KS * 16u * 8u * 4u + TS * 4u;
        if (off >= kMaxLds || (kMaxLds - off) / per_tile == 0) return hipErrorInvalidValue;
        const uint64_t room = (kMaxLds - off) / per_tile, need = (a.ntiles + room * TS - 1) / (room * TS);
        if (grid < need) grid = (uint32_t)need;
        const uint32_t tstride = grid * TS;
        tmax = (a.ntiles + tstride - 1) / tstride;
    }
    const size_t lds = ks_lds_bytes(T, a.cols, a.batch, tmax, TS, KS);
    if (lds > kMaxLds || (a.am_out && grid > kArgmaxMaxGrid)) return hipErrorInvalidValue;
    if (const hipError_t e = lds_limit.raise((const void*)kernel, lds); e != hipSuccess) return e;
    MvArgs b = a;
    b.deal_cus = BAL ? (uint32_t)device_cus() : 0;
    hipLaunchKernelGGL(kernel, dim3(grid, gy), dim3(W * 64), lds, s, b);
    return hipGetLastError();
}

// The K-split Q8_0 kernel: taken when one workgroup's tile slots hold one
// tile each (a few hundred tiles) and their parked block terms fit LDS.
template <int W, int KS, bool COMPACT = false>
static bool q8_0_ks_takes(const MvArgs& a, uint32_t pairs) {
    constexpr int TS = W / KS;
    const uint32_t gy = grid_rows(a, pairs);
    const uint32_t grid = grid_cols((a.ntiles + TS - 1) / TS, (uint32_t)kSmallWgPerCu * (uint32_t)device_cus(), gy);
    const uint64_t tmax = (a.ntiles + (uint64_t)grid * TS - 1) / ((uint64_t)grid * TS);
    const uint64_t pc = COMPACT ? a.batch : 8;
    return tmax == 1 && ks_part_off(kQ8_0, a.cols, a.batch) + (uint64_t)TS * a.nb * 16 * pc * 4 + TS * 4 <= kMaxLds;
}

template <int W, int KS, bool DBG, bool COMPACT = false>
static hipError_t launch_q8_0_ks(const MvArgs& a, hipStream_t s, uint32_t pairs) {
    constexpr int TS = W / KS;
    static LdsLimit lds_limit;
    auto kernel = q8_0_mv_ks_kernel<W, KS, 2, DBG, COMPACT>;
    const uint32_t gy = grid_rows(a, pairs);
    const uint32_t grid = grid_cols((a.ntiles + TS - 1) / TS, (uint32_t)kSmallWgPerCu * (uint32_t)device_cus(), gy);
    const size_t pc = COMPACT ? a.batch : 8;
    const size_t lds = ks_part_off(kQ8_0, a.cols, a.batch) + (size_t)TS * a.nb * 16 * pc * 4 + TS * 4;
    if ((a.ntiles + (uint64_t)grid * TS - 1) / ((uint64_t)grid * TS) != 1 || lds > kMaxLds ||
        (a.am_out && grid > kArgmaxMaxGrid))
        return hipErrorInvalidValue;
    if (const hipError_t e = lds_limit.raise((const void*)kernel, lds); e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, dim3(grid, gy), dim3(W * 64), lds, s, a);
    return hipGetLastError();
}

// Whether the balanced deal's LDS (one tile per slot) fits.
template <uint32_t T, int W, int KS>
static bool ks_bal_takes(const MvArgs& a) {
    constexpr int TS = W / KS;
    uint32_t grid, tmax;
    b1_bal_grid<TS>(a, grid, tmax);
    return grid > 0 && ks_lds_bytes(T, a.cols, a.batch, tmax, TS, KS) <= kMaxLds;
}

template <uint32_t T, int W, int KS, int D, bool DBG, bool BAL = false>
static hipError_t launch_ks(const MvArgs& a, hipStream_t s, uint32_t pairs) {
    return !a.x && planes_fit(W * 64, a.batch, a.cols, a.nb) ? launch_ks_pl<T, W, KS, D, DBG, true, BAL>(a, s, pairs)
                                                             : launch_ks_pl<T, W, KS, D, DBG, false, BAL>(a, s, pairs);
}

// Q4_K / Q5_K: the VALU kernel for one or two columns, MFMA above.
template <uint32_t T>
static hipError_t launch_q45(const MvArgs& a, uint32_t nbat, bool dbg, uint32_t epilogue, size_t lds, hipStream_t s,
                             uint32_t pairs) {
    // one f32 column: the batch-1 kernel (measured, Q4_K, us against the
    // shared-quantization kernel: 14336x4096 7.9 / 9.2 in the balanced deal
    // below; 6144x4096 5.5 / 6.6; 4096x4096 5.2 / 6.2
    // with one slot of a split of 4; 4096x14336 9.6 / 10.6 with a split of
    // 16).  Its FULL variant takes the decode step's RMSNorm input and
    // residual, model checks and the argmax (Q/K/V 6144x4096 with RMSNorm
    // 6.9 / 7.1, O 4096x4096 with the residual 6.0 / 6.3, down 4096x14336
    // 10.2 / 10.9).  The SiLU pair stays with the kernel below (28672x4096:
    // 15.2 us in the batch-1 kernel with two slots, 14.6 with four).
    if (nbat == 1 && a.x && (a.xform == kXfNone || a.xform == kXfRmsNorm) && !a.ids && !a.gate &&
        epilogue == kEpStore) {
        const bool full = a.chk || a.am_out || a.resid || a.xform != kXfNone;
        if (a.nb > 16) {
            if (b1_takes<16, 16>(a)) return launch_b1_any<T, 16, 16>(a, dbg, full, s);
        } else if (a.ntiles >= 384) {
            // the balanced deal: one workgroup per CU, its tile slots the
            // CU's (14336x4096: 7.9 us with four slots of 16 waves, 8.15 with
            // two workgroups of two slots, 8.45 grid-strided; 6144x4096 5.5
            // with two slots, 6.4 with four)
            const uint32_t u = b1_bal_units(a);
            if (u >= 5 && b1_bal_takes<16, 4>(a)) return launch_b1_any<T, 16, 4, true>(a, dbg, full, s);
            if (u >= 3 && u <= 4 && b1_bal_takes<8, 4>(a)) return launch_b1_any<T, 8, 4, true>(a, dbg, full, s);
            if (b1_takes<8, 4>(a)) return launch_b1_any<T, 8, 4>(a, dbg, full, s);
        } else if (b1_takes<4, 4>(a)) {
            return launch_b1_any<T, 4, 4>(a, dbg, full, s);
        }
    }
    // the SiLU pair epilogue: four tile slots per workgroup (two gate/up
    // pairs, a K split of two; 28672x4096 measured 14.6 us against 15.3 us
    // with one pair and a split of four)
    // (each variant has a DBG twin that also stores the block integers, so
    // rlq_block_sums checks the very kernel rlq_matmul runs)
    if (epilogue == kEpSiluPair)
        return dbg ? launch_small<T, kSmallW, kSmallW / 4, kSmallD, true>(a, s, pairs)
                   : launch_small<T, kSmallW, kSmallW / 4, kSmallD, false>(a, s, pairs);
    // one column beyond the one-column kernels' LDS (the compact image and
    // one tile's parked terms: about 46K columns) runs the batched kernel
    // below, within the f32 tolerance instead of bit for bit
    const bool one = nbat == 1 && one_part_off(a.cols, false) + (size_t)park_bytes(a.nb) <= kMaxLds;
    // two tile slots per workgroup (a K split of four): small matrices of at
    // most 4096 columns and 512 tiles (measured: 6144x4096 runs 1 us faster)
    if (one && a.nb <= 16 && a.ntiles <= 512)
        return dbg ? launch_small<T, kSmallW, kSmallW / 2, kSmallD, true>(a, s, pairs)
                   : launch_small<T, kSmallW, kSmallW / 2, kSmallD, false>(a, s, pairs);
    // more than 16 blocks per row (4096x14336, the down projection): 16 waves
    // per workgroup, K split 16 ways (measured 10.4 us vs 10.7 us with 8)
    if (one && a.nb > 16)
        return dbg ? launch_small<T, 2 * kSmallW, 2 * kSmallKS, kSmallD, true>(a, s, pairs)
                   : launch_small<T, 2 * kSmallW, 2 * kSmallKS, kSmallD, false>(a, s, pairs);
    if (one)
        return dbg ? launch_small<T, kSmallW, kSmallKS, kSmallD, true>(a, s, pairs)
                   : launch_small<T, kSmallW, kSmallKS, kSmallD, false>(a, s, pairs);
    // two to eight columns: the K-split MFMA kernel (14336x4096 batch 2:
    // 11.1 us against 11.5 us for the VALU kernel with two columns).  One
    // matrix takes the balanced deal, one workgroup per CU: four tile slots
    // of 16 waves from u = 5, two of 8 below (14336x4096 batches 2 / 4 / 8
    // 10.3 / 11.2 / 12.9 us against 11.3 / 12.9 / 16.1 grid-strided; 6144x4096
    // 7.6 / 8.6 / 10.9 against 7.8 / 8.9 / 11.0)
    if (!a.ids && grid_rows(a, pairs) == 1) {
        const uint32_t u = b1_bal_units(a);
        if (u >= 5 && ks_bal_takes<T, 16, 4>(a))  // one chunk in flight per wave (batch 4: 10.6 us against 11.2 at two)
            return dbg ? launch_ks<T, 16, 4, 1, true, true>(a, s, pairs) : launch_ks<T, 16, 4, 1, false, true>(a, s, pairs);
        if (u >= 3 && ks_bal_takes<T, 8, 4>(a))
            return dbg ? launch_ks<T, 8, 4, 2, true, true>(a, s, pairs) : launch_ks<T, 8, 4, 2, false, true>(a, s, pairs);
    }
    // no more tiles than CUs and long rows: one 16-wave slot of a K split of
    // 16 per workgroup (4096x14336 Q4_K batch 2 / 4 / 8: 12.3 / 15.3 / 16.6 us
    // against 15.7 / 19.6 / 21.3 with two 8-wave slots on half the CUs)
    if (a.ntiles * grid_rows(a, pairs) <= (uint32_t)device_cus() && a.nb >= 32)
        return dbg ? launch_ks<T, 16, 16, 1, true>(a, s, pairs) : launch_ks<T, 16, 16, 1, false>(a, s, pairs);
    return dbg ? launch_ks<T, 8, 4, 2, true>(a, s, pairs) : launch_ks<T, 8, 4, 2, false>(a, s, pairs);
}

// The one-column split kernels (Q3_K, Q6_K): 8 waves, two tile slots of a
// K split of 4, or, at no more tiles than CUs, 16 waves, one slot of a K
// split of 16 (Q3_K 4096x14336: 13.2 us against 19.8 with two slots, 13.6
// with 8 waves of a split of 8); about kSmallWgPerCu workgroups per CU and
// enough that the parked terms fit LDS (one workgroup's slots at least:
// split_fits).
static bool split_fits(uint32_t t, const MvArgs& a, uint32_t ts = 2) {
    const size_t off = split_part_off(t, a.cols), per_tile = (size_t)ts * a.nb * 512u;
    return off < kMaxLds && (kMaxLds - off) / per_tile > 0;
}
// The balanced deal (one matrix of 10240-16384 rows on 256 CUs): one
// workgroup of 16 waves per CU, four slots of a K split of 4 (two 8-wave
// slots at 6144 and 8192 rows measured no faster: Q3_K 8.9 against 8.7 us,
// Q6_K 9.4 against 9.2 at 6144 rows).
template <uint32_t T, int W, int KS, bool DBG>
static hipError_t launch_split_bal(const MvArgs& a, hipStream_t s) {
    constexpr int TS = W / KS;
    static LdsLimit lds_limit;
    auto kernel = split_one_kernel<T, W, KS, W >= 16 ? 1 : 2, DBG, true>;
    uint32_t grid, tmax;
    b1_bal_grid<TS>(a, grid, tmax);
    const size_t lds = split_lds(T, a.cols, tmax, TS);
    if (grid == 0 || a.ids || lds > kMaxLds || (a.am_out && grid > kArgmaxMaxGrid)) return hipErrorInvalidValue;
    if (const hipError_t e = lds_limit.raise((const void*)kernel, lds); e != hipSuccess) return e;
    MvArgs b = a;
    b.deal_cus = (uint32_t)device_cus();
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(W * 64), lds, s, b);
    return hipGetLastError();
}
// The grid of a split launch: about kSmallWgPerCu workgroups per CU, more
// when the tiles of a slot would not fit LDS; false when no grid fits (LDS,
// or the argmax's workgroup limit).
template <uint32_t T, int W, int KS>
static bool split_grid(const MvArgs& a, uint32_t pairs, uint32_t& grid, uint32_t& tmax) {
    constexpr int TS = W / KS;
    if (!split_fits(T, a, TS)) return false;
    const uint32_t gy = grid_rows(a, pairs);
    grid = grid_cols((a.ntiles + TS - 1) / TS, (uint32_t)kSmallWgPerCu * (uint32_t)device_cus(), gy);
    const size_t off = split_part_off(T, a.cols), per_tile = (size_t)TS * a.nb * 512u;
    const uint64_t room = (kMaxLds - off) / per_tile, need = (a.ntiles + room * TS - 1) / (room * TS);
    if (need > 65535) return false;
    if (grid < need) grid = (uint32_t)need;
    const uint32_t tstride = grid * TS;
    tmax = (a.ntiles + tstride - 1) / tstride;
    return split_lds(T, a.cols, tmax, TS) <= kMaxLds && !(a.am_out && grid > kArgmaxMaxGrid);
}
template <uint32_t T, int W, int KS, bool DBG>
static hipError_t launch_split(const MvArgs& a, hipStream_t s, uint32_t pairs) {
    constexpr int TS = W / KS;
    static LdsLimit lds_limit;
    // two steps in flight, one for Q6_K with 16 waves (its 21-register steps
    // would spill beside the operands within 128 registers)
    auto kernel = split_one_kernel<T, W, KS, T == kQ6_K && W >= 16 ? 1 : 2, DBG>;
    uint32_t grid, tmax;
    if (!split_grid<T, W, KS>(a, pairs, grid, tmax)) return hipErrorInvalidValue;
    const size_t lds = split_lds(T, a.cols, tmax, TS);
    if (const hipError_t e = lds_limit.raise((const void*)kernel, lds); e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, dim3(grid, grid_rows(a, pairs)), dim3(W * 64), lds, s, a);
    return hipGetLastError();
}
// Q6_K with one column takes the split kernels up to 1024 tiles (16384
// rows; us against the whole-tile kernel: 1024x4096 6.3 / 19.1, 4096x4096
// 6.9 / 19.4, 4096x14336 15.2 / 56.2, 14336x4096 13.4 / 19.9) and the
// whole-tile kernel above (28672x4096 25.5 / 22.7, 128256x4096 about 94
// both; the output head).
constexpr uint64_t kQ6SplitMaxTiles = 1024;

template <uint32_t T>
static hipError_t launch_split_one(const MvArgs& a, bool dbg, hipStream_t s, uint32_t pairs, bool& taken) {
    taken = true;
    uint32_t grid, tmax;
    const uint32_t u = !a.ids && grid_rows(a, pairs) == 1 ? b1_bal_units(a) : 0;
    if (u >= 5 && split_lds(T, a.cols, 1, 4) <= kMaxLds)
        return dbg ? launch_split_bal<T, 16, 4, true>(a, s) : launch_split_bal<T, 16, 4, false>(a, s);
    if (a.ntiles * grid_rows(a, pairs) > (uint32_t)device_cus() && split_grid<T, 8, 4>(a, pairs, grid, tmax))
        return dbg ? launch_split<T, 8, 4, true>(a, s, pairs) : launch_split<T, 8, 4, false>(a, s, pairs);
    if (split_grid<T, 16, 16>(a, pairs, grid, tmax))
        return dbg ? launch_split<T, 16, 16, true>(a, s, pairs) : launch_split<T, 16, 16, false>(a, s, pairs);
    taken = false;
    return hipSuccess;
}

// Q2_K / Q3_K: up to four columns the K-split kernel, while its parked terms
// fit LDS next to the activations (matrices of up to about 2^17 rows at 4096
// columns); one wave per tile otherwise (measured at 14336x4096: batch 1
// 9.4 us split vs 11.3 us, batch 8 22.8 us vs 20.7 us).
constexpr int kK16W = 8, kK16KS = 8, kK16D = 2;

template <uint32_t T, bool DBG, int W = kK16W, int KS = kK16KS>
static hipError_t launch_k16_split(const MvArgs& a, size_t lds, uint32_t grid, uint32_t gy, hipStream_t s) {
    static LdsLimit lds_limit;
    auto kernel = k16_mv_split_kernel<T, W, KS, W >= 16 ? 1 : kK16D, DBG>;
    if (a.am_out && grid > kArgmaxMaxGrid) return hipErrorInvalidValue;
    if (const hipError_t e = lds_limit.raise((const void*)kernel, lds); e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, dim3(grid, gy), dim3(W * 64), lds, s, a);
    return hipGetLastError();
}

// The K-split kernel in the balanced deal (one matrix): W waves, K split KS,
// one tile per slot.
template <uint32_t T, int W, int KS, bool DBG>
static hipError_t launch_k16_bal(const MvArgs& a, hipStream_t s) {
    constexpr int TS = W / KS;
    static LdsLimit lds_limit;
    // one chunk in flight per wave with 16 waves (14336x4096 Q3_K 9.73 us
    // against 9.98 at two, Q2_K 8.45 against 8.53)
    auto kernel = k16_mv_split_kernel<T, W, KS, W >= 16 ? 1 : kK16D, DBG, true>;
    uint32_t grid, tmax;
    b1_bal_grid<TS>(a, grid, tmax);
    const uint64_t lds = k16_part_off(T, a.cols, a.batch) + (uint64_t)tmax * TS * a.nb * 16ull * a.batch * 4ull;
    if (grid == 0 || a.ids || a.batch > 8 || lds > kMaxLds || (a.am_out && grid > kArgmaxMaxGrid))
        return hipErrorInvalidValue;
    if (const hipError_t e = lds_limit.raise((const void*)kernel, lds); e != hipSuccess) return e;
    MvArgs b = a;
    b.deal_cus = (uint32_t)device_cus();
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(W * 64), lds, s, b);
    return hipGetLastError();
}

template <uint32_t T>
static hipError_t launch_k16(const MvArgs& a, bool dbg, size_t lds_plain, hipStream_t s, uint32_t pairs) {
    // Q3_K, one column: the reference's f32 order; the blocks of each tile
    // split over several waves while the parked terms fit LDS, else one wave
    // per tile (14336x4096: balanced 12.0 us, split 13.0, one wave per tile
    // 15.3; the kernels in their own order took 10.2)
    if (T == kQ3_K && a.batch == 1) {
        bool taken;
        const hipError_t e = launch_split_one<kQ3_K>(a, dbg, s, pairs, taken);
        if (taken) return e;
        return dbg ? launch_one<kMvWaves, q3k_mv_one_kernel<kMvWaves, 3, true>>(a, lds_plain, s, pairs)
                   : launch_one<kMvWaves, q3k_mv_one_kernel<kMvWaves, 3, false>>(a, lds_plain, s, pairs);
    }
    // one matrix of 10240..16384 rows (on 256 CUs): the balanced deal, one
    // workgroup of 16 waves per CU, four slots of a K split of 4 (14336x4096
    // Q2_K batches 1 / 2 / 4 / 5 / 8: 8.6 / 9.5 / 11.0 / 14.1 / 16.6 us against
    // 9.6 / 11.1 / 14.6 / 18.1 / 20.6; Q3_K 9.9 / 10.9 / 12.5 / 14.6 / 17.0
    // against 11.2 / 12.7 / 16.2 / 18.5 / 20.7)
    if (!a.ids && grid_rows(a, pairs) == 1 && b1_bal_units(a) >= 5 &&
        k16_part_off(T, a.cols, a.batch) + 4ull * a.nb * 16ull * a.batch * 4ull <= kMaxLds)
        return dbg ? launch_k16_bal<T, 16, 4, true>(a, s) : launch_k16_bal<T, 16, 4, false>(a, s);
    // 6144..8192 rows: the balanced deal in 8-wave workgroups of two slots
    // (Q2_K 6144x4096 batch 1 / 4: 6.9 / 9.4 us against 7.8 / 12.9)
    if (!a.ids && grid_rows(a, pairs) == 1 && b1_bal_units(a) >= 3 && b1_bal_units(a) <= 4 &&
        k16_part_off(T, a.cols, a.batch) + 2ull * a.nb * 16ull * a.batch * 4ull <= kMaxLds)
        return dbg ? launch_k16_bal<T, 8, 4, true>(a, s) : launch_k16_bal<T, 8, 4, false>(a, s);
    constexpr int TS = kK16W / kK16KS;
    const uint32_t want = (a.ntiles + TS - 1) / TS;
    const uint32_t gy = grid_rows(a, pairs);
    const uint32_t grid = grid_cols(want, (uint32_t)kSmallWgPerCu * (uint32_t)device_cus(), gy);
    const uint64_t tstride = (uint64_t)grid * TS, tmax = (a.ntiles + tstride - 1) / tstride;
    const uint64_t lds = k16_part_off(T, a.cols, a.batch) + tmax * TS * a.nb * 16ull * a.batch * 4ull;
    // no more tiles than CUs and long rows: 16 waves of a K split of 16 in the
    // one tile slot (4096x14336 Q2_K batch 1 / 2 / 4: 10.8 / 13.5 / 20.4 us
    // against 12.3 / 15.8 / 24.5 with 8 waves; Q3_K batch 4 21.4 against 24.0)
    if (a.batch <= 4 && lds <= kMaxLds && TS == 1 && a.ntiles * gy <= (uint32_t)device_cus() && a.nb >= 32)
        return dbg ? launch_k16_split<T, true, 16, 16>(a, lds, grid, gy, s)
                   : launch_k16_split<T, false, 16, 16>(a, lds, grid, gy, s);
    if (a.batch <= 4 && lds <= kMaxLds)
        return dbg ? launch_k16_split<T, true>(a, lds, grid, gy, s) : launch_k16_split<T, false>(a, lds, grid, gy, s);
    return dbg ? launch_one<kMvWaves, k16_mv_kernel<T, kMvWaves, 4, true>>(a, lds_plain, s, pairs)
               : launch_one<kMvWaves, k16_mv_kernel<T, kMvWaves, 4, false>>(a, lds_plain, s, pairs);
}

hipError_t launch_matvec(uint32_t wtype, const uint8_t* w, uint64_t rows, uint64_t cols, const float* x,
                         const ActPlanes* pre, uint64_t batch, float* y, uint64_t ldy, const MvArgmax* am,
                         unsigned long long* err_word, int32_t* dbg_isum, int32_t* dbg_imin, hipStream_t s) {
    return launch_matvec_ex(wtype, w, rows, cols, x, pre, batch, y, ldy, am, err_word, dbg_isum, dbg_imin, MvExtra{},
                            s);
}

hipError_t launch_matvec_ex(uint32_t wtype, const uint8_t* w, uint64_t rows, uint64_t cols, const float* x,
                            const ActPlanes* pre, uint64_t batch, float* y, uint64_t ldy, const MvArgmax* am,
                            unsigned long long* err_word, int32_t* dbg_isum, int32_t* dbg_imin, const MvExtra& ex,
                            hipStream_t s) {
    const uint32_t bs = wtype == kQ8_0 ? 32 : 256;
    if (rows == 0 || cols == 0 || cols % bs != 0 || rows > 0xffffffffull - kTileRows || cols > (1u << 30))
        return hipErrorInvalidValue;
    if (dbg_isum && batch > 8) return hipErrorInvalidValue;
    // the transforms read one f32 column (RMSNorm weights, or [gate | up])
    if (ex.xform != kXfNone &&
        (batch != 1 || !x || ex.xform > kXfSiluMul || (ex.xform == kXfRmsNorm && !ex.norm_w)))
        return hipErrorInvalidValue;
    // the SiLU pair epilogue: one Q4_K / Q5_K column, whole tile pairs, no argmax or residual
    if (ex.epilogue != kEpStore &&
        (ex.epilogue != kEpSiluPair || batch != 1 || (wtype != kQ4_K && wtype != kQ5_K) ||
         rows % (2 * kTileRows) != 0 || am || ex.resid))
        return hipErrorInvalidValue;
    // expert pairs: one pre-quantized column each, plain stores; or, checked
    // in the kernel, one shared f32 column
    if (ex.ids && (batch != 1 || am || dbg_isum || ex.resid || ex.xform != kXfNone ||
                   ex.epilogue != kEpStore || ex.id_pairs == 0 || ex.id_pairs > 0xffffffffull || ex.id_slots == 0 ||
                   ex.id_cols == 0 || (ex.id_inline ? (!x || pre || ex.id_cols != 1 || ex.gate)
                                                     : (x || !pre))))
        return hipErrorInvalidValue;
    // two Q6_K columns of a matrix of no more tiles than CUs: one column per
    // pass, each on the split kernels (4096x14336: 30.0 us against 49.1 for
    // both columns walking whole tiles; 4096x4096 13.6 against 17.9; three
    // columns measure no faster)
    const bool q6_columns = wtype == kQ6_K && batch == 2 && !ex.ids &&
                            (rows + kTileRows - 1) / kTileRows <= (uint64_t)device_cus();
    uint64_t b0 = 0;
    while (b0 < batch) {
        uint32_t nbat = (uint32_t)(batch - b0 < 8 ? batch - b0 : 8);
        if (q6_columns) nbat = 1;
        while (nbat > 1 && lds_map(wtype, (uint32_t)cols, nbat).total > kMaxLds) --nbat;
        const size_t lds = lds_map(wtype, (uint32_t)cols, nbat).total;
        if (lds > kMaxLds) return hipErrorInvalidValue;
        MvArgs a{};
        a.w = w;
        a.rows = (uint32_t)rows;
        a.nb = (uint32_t)(cols / bs);
        a.ntiles = (uint32_t)layout_tiles(rows);
        a.nchunks = (uint32_t)layout_chunks_per_tile(wtype, cols);
        a.batch = nbat;
        a.cols = (uint32_t)cols;
        a.x = x ? x + b0 * cols : nullptr;
        if (pre) {
            a.pre.q = pre->q + b0 * cols;
            a.pre.d = pre->d + b0 * (cols / bs);
            a.pre.bsum = pre->bsum ? pre->bsum + b0 * (cols / 16) : nullptr;
            a.pre.bad = pre->bad + b0 * (cols / bs);
        }
        a.y = y + b0 * ldy;
        a.ldy = ldy;
        a.am_out = am ? am->out + b0 : nullptr;
        a.am_slots = am ? am->slots : nullptr;
        a.am_count = am ? am->count : nullptr;
        a.err_word = err_word;
        a.err_column0 = (uint32_t)(ex.column_base + b0);
        a.dbg_isum = b0 == 0 ? dbg_isum : nullptr;  // column 0 only
        a.dbg_imin = b0 == 0 ? dbg_imin : nullptr;
        a.xform = ex.xform;
        a.eps = ex.eps;
        a.norm_w = ex.norm_w;
        a.resid = ex.resid ? ex.resid + b0 * ldy : nullptr;
        a.epilogue = ex.epilogue;
        a.gate = ex.gate;
        a.ids = ex.ids;
        a.id_slots = ex.id_slots;
        a.id_cols = ex.id_cols;
        a.id_experts = ex.id_experts;
        a.expert_bytes = ex.expert_bytes;
        a.id_inline = ex.ids && ex.id_inline ? 1u : 0u;
        a.id_total = (uint32_t)ex.id_pairs;
        a.chk = ex.chk;
        a.chk_layer = ex.chk_layer;
        constexpr int W = kMvWaves;
        const bool dbg = a.dbg_isum != nullptr;
        auto dispatch = [&](uint32_t pairs) -> hipError_t {
            switch (wtype) {
                case kQ4_K: return launch_q45<kQ4_K>(a, nbat, dbg, ex.epilogue, lds, s, pairs);
                case kQ5_K: return launch_q45<kQ5_K>(a, nbat, dbg, ex.epilogue, lds, s, pairs);
                case kQ3_K: return launch_k16<kQ3_K>(a, dbg, lds, s, pairs);
                case kQ2_K: return launch_k16<kQ2_K>(a, dbg, lds, s, pairs);
                case kQ6_K:
                    // one workgroup of 8 waves per CU, three chunks in flight per
                    // wave (128256x4096 + argmax, batch 8: 78.5 us against 79.6
                    // with four and 80.3 with five; batch 1 71.1 with three or four);
                    // one column in the reference's f32 order
                    if (nbat == 1) {
                        if ((uint64_t)a.ntiles * grid_rows(a, pairs) <= kQ6SplitMaxTiles) {
                            bool taken;
                            const hipError_t e = launch_split_one<kQ6_K>(a, dbg, s, pairs, taken);
                            if (taken) return e;
                        }
                        return dbg ? launch_one<2 * W, q6k_mv_one_kernel<2 * W, 3, true>>(a, lds, s, pairs, 1)
                                   : launch_one<2 * W, q6k_mv_one_kernel<2 * W, 3, false>>(a, lds, s, pairs, 1);
                    }
                    return dbg ? launch_one<2 * W, q6k_mv_kernel<2 * W, 3, true>>(a, lds, s, pairs, 1)
                               : launch_one<2 * W, q6k_mv_kernel<2 * W, 3, false>>(a, lds, s, pairs, 1);
                default:
                    // the K split by block pairs per row (batch 1 / 4 / 8, us, against
                    // 8 waves of a 4-way split): a 16-way split of 16 waves from 32
                    // pairs (896x4864 9.0 / 11.2 / 14.3 against 23.5 / 27.9 / 34.6,
                    // 4096x4096 8.8 / 10.5 / 13.1 against 12.7 / 15.1 / 29.6), an
                    // 8-way split of 16 waves from 12 (14336x4096 20.5 / 24.2 against
                    // 24.5 / 29.2 where the 16-way split would need two tiles per slot;
                    // 4864x896 6.53 against 6.62, 10.5 with the 16-way split)
                    // (the 16-way split while its tiles fit one workgroup per CU:
                    // 6144x4096 10.8 us against 15.3 with 384 workgroups on 256 CUs)
                    if (a.nchunks >= 32 && a.ntiles * grid_rows(a, pairs) <= (uint32_t)device_cus() &&
                        q8_0_ks_takes<16, 16>(a, pairs))
                        return dbg ? launch_q8_0_ks<16, 16, true>(a, s, pairs) : launch_q8_0_ks<16, 16, false>(a, s, pairs);
                    if (a.nchunks >= 12 && q8_0_ks_takes<16, 8>(a, pairs))
                        return dbg ? launch_q8_0_ks<16, 8, true>(a, s, pairs) : launch_q8_0_ks<16, 8, false>(a, s, pairs);
                    if (q8_0_ks_takes<8, 4>(a, pairs))
                        return dbg ? launch_q8_0_ks<8, 4, true>(a, s, pairs) : launch_q8_0_ks<8, 4, false>(a, s, pairs);
                    // rows too long for eight parked columns: the batch's only
                    // (4096x14336 batch 1: 23.9 us against 61.3 walking whole tiles)
                    if (a.nchunks >= 32 && q8_0_ks_takes<16, 16, true>(a, pairs))
                        return dbg ? launch_q8_0_ks<16, 16, true, true>(a, s, pairs)
                                   : launch_q8_0_ks<16, 16, false, true>(a, s, pairs);
                    // ten chunks in flight per wave (151936x896 + argmax: 30.3 us
                    // against 30.9 with eight, 31.8 with six)
                    return dbg ? launch_one<W, q8_0_mv_kernel<W, 10, true>>(a, lds, s, pairs, 3)
                               : launch_one<W, q8_0_mv_kernel<W, 10, false>>(a, lds, s, pairs, 3);
            }
        };
        if (!a.ids) {
            const hipError_t e = dispatch(1);
            if (e != hipSuccess) return e;
        } else {  // grid rows are pairs, at most 65535 per launch
            for (uint64_t p0 = 0; p0 < ex.id_pairs; p0 += 65535) {
                a.id_base = (uint32_t)p0;
                const hipError_t e = dispatch((uint32_t)(ex.id_pairs - p0 < 65535 ? ex.id_pairs - p0 : 65535));
                if (e != hipSuccess) return e;
            }
        }
        b0 += nbat;
    }
    return hipSuccess;
}

// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// MUL_MAT / MUL_MAT_ID prepare (one workgroup): the reference checks every
// expert id before it quantizes anything (crates/tensor/src/cpu_index.rs:
// 197-202) and writes no output when any check or any column's quantization
// fails.  The gate is 1 when an id is outside [-1, experts) (the first one is
// reported as TensorError::Bounds) or any pre-quantized block is bad;
// otherwise the outputs of the pairs with id -1 are zeroed (the reference's
// `zeros` output, cpu_index.rs:204) and the gate is 0.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mm_prepare_kernel(const int32_t* __restrict__ ids, uint64_t pairs,
                                                         int32_t experts, const uint8_t* __restrict__ bad,
                                                         uint64_t nbad, float* __restrict__ y, uint64_t rows,
                                                         uint32_t* gate, unsigned long long* err_word) {
    __shared__ unsigned long long first_s;
    __shared__ int flag_s;
    if (threadIdx.x == 0) first_s = ~0ull, flag_s = 0;
    __syncthreads();
    unsigned long long first = ~0ull;
    for (uint64_t i = threadIdx.x; i < pairs; i += 256) {
        const int32_t id = ids[i];
        if ((id < -1 || id >= experts) && i < first) first = i;
    }
    int any_bad = 0;
    for (uint64_t i = threadIdx.x; i < nbad; i += 256) any_bad |= bad[i];
    if (first != ~0ull) atomicMin(&first_s, first);
    if (any_bad) atomicOr(&flag_s, 1);
    __syncthreads();
    const bool refused = first_s != ~0ull || flag_s != 0;
    if (threadIdx.x == 0) {
        *gate = refused ? 1u : 0u;
        if (first_s != ~0ull) report_error(err_word, bounds_key(first_s));
    }
    if (refused || !ids) return;
    for (uint64_t p = 0; p < pairs; ++p)
        if (ids[p] == -1)
            for (uint64_t r = threadIdx.x; r < rows; r += 256) y[p * rows + r] = 0.0f;
}

hipError_t launch_mm_prepare(const int32_t* ids, uint64_t pairs, uint32_t experts, const uint8_t* bad, uint64_t nbad,
                             float* y, uint64_t rows, uint32_t* gate, unsigned long long* err_word, hipStream_t s) {
    hipLaunchKernelGGL(mm_prepare_kernel, dim3(1), dim3(256), 0, s, ids, ids ? pairs : 0, (int32_t)experts, bad, nbad,
                       y, rows, gate, err_word);
    return hipGetLastError();
}

__global__ void argmax_finish_kernel(unsigned long long* keys, uint64_t batch, const float* y, uint64_t ldy,
                                     uint32_t* out, bool reset) {
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= batch) return;
    const float y0 = y[b * ldy];
    const unsigned long long k = keys[b];
    if (reset) keys[b] = 0ull;
    // A NaN first logit is never replaced by the reference's strict `>` scan.
    out[b] = (y0 != y0 || k == 0) ? 0u : (uint32_t)(0xffffffffull - (k & 0xffffffffull));
}

// Greedy argmax keys of stored rows (the GEMM path): keys[b] = max over r of
// argmax_key(y[b*rows + r], r); keys must start at 0.
__global__ __launch_bounds__(256) void argmax_rows_kernel(const float* __restrict__ y, uint64_t rows,
                                                          unsigned long long* keys) {
    const uint64_t b = blockIdx.y;
    unsigned long long best = 0;
    for (uint64_t r = (uint64_t)blockIdx.x * 256 + threadIdx.x; r < rows; r += (uint64_t)gridDim.x * 256) {
        const unsigned long long k = argmax_key(y[b * rows + r], r);
        best = k > best ? k : best;
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const unsigned long long o = __shfl_xor(best, m, 64);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0 && best) atomicMax(keys + b, best);
}

hipError_t launch_argmax_rows(const float* y, uint64_t batch, uint64_t rows, unsigned long long* keys, hipStream_t s) {
    const uint64_t per = (rows + 255) / 256;
    hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)(per < 64 ? per : 64), (unsigned)batch), dim3(256), 0, s, y,
                       rows, keys);
    return hipGetLastError();
}

hipError_t launch_argmax_finish(unsigned long long* keys, uint64_t batch, const float* y, uint64_t ldy, uint32_t* out,
                                hipStream_t s, bool reset) {
    hipLaunchKernelGGL(argmax_finish_kernel, dim3((unsigned)((batch + 63) / 64)), dim3(64), 0, s, keys, batch, y, ldy,
                       out, reset);
    return hipGetLastError();
}

}  // namespace rlq
