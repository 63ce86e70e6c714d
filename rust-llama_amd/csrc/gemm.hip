// gemm.hip - prefill GEMM for Q4_K weights on gfx950: y[m][n] = dot(row n, token m)
// for many tokens at once, on fp16 MFMA with exact integer operands.
//
// Contract: the GGML MUL_MAT semantics of crates/tensor/src/cpu_extra.rs:756-873
// -- every token (column) is quantized to Q8_K on its own (:820) and every
// output is dot_packed(weight row, token) (:860), i.e. the Q4_K dot of
// crates/quant/src/matvec_extra.rs:212-271, 286-293.  Prefill in the
// reference is M such matvecs (crates/inference/src/lib.rs:407,
// crates/model-runtime/src/context.rs:452); this kernel computes the same
// exact per-block integers for all M tokens in one pass over the weights.
//
// Integer decomposition.  Per (token m, row n, block of 256):
//   I  = sum_j (sc_s(j) * q_j) * x_j        sc: 6-bit sub-block scale, q: 4 bits
//   Mn = sum_s mn_s * bsum32_s(m)           mn: 6-bit sub-block min
//   y += da_m * (d_n * I - dmin_n * Mn)     f32, block by block
// Both sums run on v_mfma_f32_32x32x16_f16 with integer-valued operands: the
// weight operand is sc*q <= 945 and the activation operand q8 in [-127, 127],
// both exact in f16; products are exact in f32, and every partial sum of a
// chain is an integer bounded by sum_j |sc q x|.  While that bound stays below
// 2^24 the f32 accumulation is exact in any order.  The activation quantizer
// flags a (token, block) with sum |x| > 17753 (945 * 17753 < 2^24); a token
// tile folds such a block in two halves (128 values: 128*945*127 < 2^24)
// instead of once.  The mins use bsum16 (|.| <= 2032) against
// mn (<= 63): always exact.  So I and Mn equal the reference's i32 sums, and
// float(I) (the f32 of an exact integer, or the f32 sum of two exact halves)
// is the reference's `sumi as f32`; only the f32 order of the per-block terms
// differs from the reference's.
#include "rlq_device.hpp"
#include "rlq_internal.hpp"
#include "rlq_layout.hpp"
#include "rlq_q8k.hpp"

namespace rlq {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// Tiling
//
// Workgroup: 8 waves over 128 tokens x 256 weight rows (16 layout tiles of 16
// rows), one workgroup per CU (two waves per SIMD).  Wave w owns rows
// 32w .. 32w+31 (one MFMA column tile) and the 128 tokens as four 32-token
// tiles T: each dequantized weight operand feeds four MFMAs.  Accumulators
// and f32 outputs y live in VGPRs.  (Four waves over 128 rows, two workgroups
// per CU, two stages ahead: 86-89 us at 512x4096x14336 against 83.6-83.9.)
//
// K is walked in groups of 64 values (4 k-steps of 16).  A group's operands
// are one LDS stage, filled by global_load_lds_dwordx4 (global -> LDS without
// VGPRs) kAhead stages ahead in a ring of kSlots; per-block data (weight block
// headers, the activation record) sit in a ring of two regions.
// ---------------------------------------------------------------------------
constexpr uint32_t kGemmWaves = 8;                 // one 32-row MFMA column tile each
constexpr uint32_t kGemmTM = 128;                  // tokens per workgroup
constexpr uint32_t kGemmTN = 32 * kGemmWaves;      // weight rows per workgroup
constexpr uint32_t kGemmThreads = 64 * kGemmWaves;
constexpr uint32_t kUnsafeAbsSum = 17753;  // floor((2^24 - 1) / 945)

// Activation image, written by gemm_act_kernel.  Per token tile of 128: nb*4
// groups, then nb block records.
//   group (b, g): [k-step 4][k half 2][token 128][8 halves]  16 KB
//   record b:     bsum16 [k half 2][token 128][8 halves]      4 KB
//                 da [token 128] f32                         512 B
//                 flags [token 128] u8                       128 B
// Group g, k-step s, k half h, slot t holds the value at block position
// 64g + 32(s/2) + q45_pos_of_slot(16h + 8(s%2) + kPerm[t]), kPerm =
// {0,2,1,3,4,6,5,7}: the order in which the weight dequantizer below produces
// sc*q from the weights' slots (rlq_layout.hpp).  flags: bit 0 a
// data error in the token's block, bit 1 sum |q8| > kUnsafeAbsSum.
constexpr uint32_t kActGroupBytes = 16384;
constexpr uint32_t kRecDa = 4096, kRecFlags = 4608, kActRecordBytes = 4736;
constexpr uint64_t kActTileBlockBytes = 4 * kActGroupBytes + kActRecordBytes;

__device__ __forceinline__ uint64_t act_group_offset(uint32_t b, uint32_t g) {
    return ((uint64_t)b * 4 + g) * kActGroupBytes;
}
__device__ __forceinline__ uint64_t act_record_offset(uint32_t nb, uint32_t b) {
    return (uint64_t)nb * 4 * kActGroupBytes + (uint64_t)b * kActRecordBytes;
}

// LDS per workgroup: a ring of kSlots stages [A 16 KB][W kGemmTN/16 tiles x
// 512 B], filled kAhead stages ahead; two regions [headers kGemmTN x 16 B][record]
// (the stage kAhead ahead of a block's last one belongs at most to the next
// block, so two regions never collide while kAhead <= 4).
constexpr uint32_t kAhead = 3, kSlots = kAhead + 1;
constexpr uint32_t kSlotW = kActGroupBytes, kSlotBytes = kSlotW + kGemmTN / 16 * 512;
constexpr uint32_t kRegions = 2, kRegRec = kGemmTN * 16, kRegionBytes = kRegRec + kActRecordBytes;
constexpr uint32_t kGemmLds = kSlots * kSlotBytes + kRegions * kRegionBytes;
static_assert(kAhead >= 1 && kAhead <= 4 && 16 % kGemmWaves == 0 && kActRecordBytes % (16 * kGemmWaves) == 0, "");
// LDS-DMA loads per wave and stage (A pieces, W pieces), and the extra ones of
// a block's first stage (headers, record)
constexpr int kLoadsStage = 16 / kGemmWaves + 1;
constexpr int kLoadsFirst = 1 + (kActRecordBytes / kGemmWaves + 1023) / 1024;
// loads a wave may still have pending at the barrier of a stage of group G:
// those of the kAhead - 1 stages after it
constexpr int pending_loads(int G) {
    int n = 0;
    for (int k = 1; k < (int)kAhead; ++k) n += kLoadsStage + ((G + k) % 4 == 0 ? kLoadsFirst : 0);
    return n;
}

// ---------------------------------------------------------------------------
// Activations: f32 x [M][K] -> the image above.  Tokens >= M are zeros.  One
// workgroup per (token tile, block); each 16-lane DPP row quantizes one
// token's block (q8k_row16), lane r16 holding positions 16 r16 .. +15.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int32_t row16_sum_i(int32_t v) {
    v += dpp_i<kQuadXor1>(v);
    v += dpp_i<kQuadXor2>(v);
    v += dpp_i<kRowHalfMirror>(v);
    v += dpp_i<kRowRor8>(v);
    return v;
}

__global__ __launch_bounds__(256) void gemm_act_kernel(const float* __restrict__ x, uint32_t M, uint32_t K,
                                                       uint8_t* __restrict__ img, unsigned long long* err_word,
                                                       uint32_t err_column0) {
    // workgroup: 16 tokens of one (token tile, block); 16-lane row `row` = one token
    const uint32_t nb = K / 256, chunks = kGemmTM / 16;
    const uint32_t chunk = blockIdx.x % chunks, b = (blockIdx.x / chunks) % nb, mt = blockIdx.x / chunks / nb;
    const uint32_t r16 = threadIdx.x & 15, tok = chunk * 16 + (threadIdx.x >> 4);
    const uint32_t m = mt * kGemmTM + tok;
    uint8_t* tile = img + (uint64_t)mt * nb * kActTileBlockBytes;
    float v[16];
    if (m < M) {
        const float4* src = (const float4*)(x + (uint64_t)m * K + b * 256 + r16 * 16);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 f = src[k];
            v[4 * k] = f.x, v[4 * k + 1] = f.y, v[4 * k + 2] = f.z, v[4 * k + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = 0.0f;
    }
    const Q8KRow o = q8k_row16(v, r16);
    if (o.kind >= 0 && r16 == 0)
        report_error(err_word, o.kind == kKindNonFinite
                                   ? error_key(err_column0 + m, kKindNonFinite, b * 256ull + o.index)
                                   : error_key(err_column0 + m, kKindScale, b));
    // the weights' slot order (q45_slots): slot 16 hh + t holds position
    // q45_pos_of_slot(16 hh + t) of the sub-block
    const uint4 sl = q45_slots(o.q, r16 & 1);
    const uint32_t sw[4] = {sl.x, sl.y, sl.z, sl.w};
    int32_t q[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) q[t] = (int32_t)(int8_t)(sw[t / 4] >> (8 * (t % 4)));
    // slots 16 (r16%2) + t of sub-block r16/2: group r16/4, k-steps 2((r16/2)%2) + t/8, k half r16%2
    uint8_t* ag = tile + act_group_offset(b, r16 / 4);
    const uint32_t s0 = 2 * ((r16 >> 1) & 1), hh = r16 & 1;
    constexpr int kPerm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
#pragma unroll
    for (int so = 0; so < 2; ++so) {
        f16x8 h;
#pragma unroll
        for (int t = 0; t < 8; ++t) h[t] = (_Float16)q[8 * so + kPerm[t]];
        *(f16x8*)(ag + ((s0 + so) * 2 + hh) * 2048 + tok * 16) = h;
    }
    uint8_t* rec = tile + act_record_offset(nb, b);
    *(_Float16*)(rec + (r16 / 8) * 2048 + tok * 16 + (r16 % 8) * 2) = (_Float16)o.bsum;
    int32_t sa = 0;
#pragma unroll
    for (int t = 0; t < 16; ++t) sa += q[t] < 0 ? -q[t] : q[t];
    sa = row16_sum_i(sa);
    const int32_t bad = row16_sum_i(o.kind >= 0 ? 1 : 0);
    if (r16 == 0) {
        *(float*)(rec + kRecDa + tok * 4) = o.d;
        rec[kRecFlags + tok] = (uint8_t)((bad ? 1u : 0u) | ((uint32_t)sa > kUnsafeAbsSum ? 2u : 0u));
    }
}

// ---------------------------------------------------------------------------
// GEMM
// ---------------------------------------------------------------------------
struct GemmArgs {
    const uint8_t* w;  // Q4_K, tiled device layout (rlq_layout.hpp)
    uint32_t rows, nb, ntiles16;
    const uint8_t* img;  // activation image
    uint32_t M, NT, MT;  // tokens; workgroup tiles along rows and tokens
    float* y;            // y[m * ldy + n]
    uint64_t ldy;
    int32_t* dbg_isum;  // exact integers of token 0, or null
    int32_t* dbg_imin;
};

__device__ __forceinline__ f32x16 mfma16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// global -> LDS, 16 bytes per lane: lane l's 16 bytes at sbase + voff go to
// LDS address lds + 16 l (lds and sbase wave-uniform).  Issued as inline asm:
// the compiler would otherwise treat the LDS write as aliasing every later LDS
// read and wait for all outstanding loads before each; the stage barriers
// below order these loads instead.
__device__ __forceinline__ void g2l(const void* sbase, uint32_t voff, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds));
}

// Wait until at most N of this wave's vector-memory operations are pending and
// its LDS operations are done, then barrier: the LDS-DMA loads of the stage
// about to be read (all but the newest N) have landed for every wave.
template <int N>
__device__ __forceinline__ void stage_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }

// Byte K (< 64) of w as the f16 pair (w_K, w_K): bits 0x64kk are 1024 + w_K.
template <int K>
__device__ __forceinline__ f16x2 byte_pair(uint32_t w) {
    const uint32_t sel = (uint32_t)K | 4u << 8 | (uint32_t)K << 16 | 4u << 24;
    return as_h2(__builtin_amdgcn_perm(0x64646464u, w, sel)) - (f16x2){(_Float16)1024.0f, (_Float16)1024.0f};
}

// Q4_K block header (16 bytes: d, dmin, 12 scale bytes) -> 6-bit scales and
// mins, four per word (get_scale_min_k4, crates/quant/src/decode.rs:216-235).
struct Q4Words {
    uint32_t scA, scB, mnA, mnB;  // sub-blocks 0-3 and 4-7
};
__device__ __forceinline__ Q4Words q4_words(uint4 h) {
    Q4Words q;
    q.scA = h.y & 0x3f3f3f3fu;
    q.scB = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
    q.mnA = h.z & 0x3f3f3f3fu;
    q.mnB = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
    return q;
}

// Scale pairs of one group's two sub-blocks: low nibbles (sub-block 2g) are
// dequantized from 1024 + q as (1024 + q) sc - 1024 sc, high nibbles (2g + 1)
// from 1024 + 16 q as (1024 + 16 q) (sc / 16) - 64 sc; each v_pk_fma_f16 is
// exact (the exact result q*sc <= 945 is an f16).
struct GroupScales {
    f16x2 lo, lo_neg, hi, hi_neg;
};
template <int G>
__device__ __forceinline__ GroupScales group_scales(const Q4Words& q) {
    const uint32_t w = G < 2 ? q.scA : q.scB;
    const f16x2 a = byte_pair<2 * (G % 2)>(w), b = byte_pair<2 * (G % 2) + 1>(w);
    GroupScales s;
    s.lo = a;
    s.lo_neg = a * (f16x2){(_Float16)-1024.0f, (_Float16)-1024.0f};
    s.hi = b * (f16x2){(_Float16)0.0625f, (_Float16)0.0625f};
    s.hi_neg = b * (f16x2){(_Float16)-64.0f, (_Float16)-64.0f};
    return s;
}

// Per-row data of the block being folded: f32 d and dmin and the mins operand
// (lane half h: mn_{4h} .. mn_{4h+3}, each twice, against bsum16 8h .. 8h+7).
struct FoldRow {
    float d, dmin;
    f16x8 mins;
};
__device__ __forceinline__ FoldRow fold_row(uint4 hdr, uint32_t kh) {
    const Q4Words q = q4_words(hdr);
    const uint32_t w = kh ? q.mnB : q.mnA;
    FoldRow f;
    f.d = half_to_float(hdr.x);
    f.dmin = half_to_float(hdr.x >> 16);
    const f16x2 p0 = byte_pair<0>(w), p1 = byte_pair<1>(w), p2 = byte_pair<2>(w), p3 = byte_pair<3>(w);
    f.mins[0] = p0[0], f.mins[1] = p0[1], f.mins[2] = p1[0], f.mins[3] = p1[1];
    f.mins[4] = p2[0], f.mins[5] = p2[1], f.mins[6] = p3[0], f.mins[7] = p3[1];
    return f;
}

// Everything one workgroup needs, fixed for the launch.
struct GemmCtx {
    uint8_t* smem;
    uint32_t lds;  // LDS address of smem
    uint32_t nb, rows, nt, mt, wave, lane, ln, kh;
    const uint8_t* act_tile;  // activation image of token tile mt
    const uint8_t* w_first;   // first weight layout tile of the workgroup
    uint32_t w_lane;          // this lane's offset (from w_first) of its weight-piece load
    uint32_t h_lane;          // ... and of its header load
    int32_t* dbg_isum;
    int32_t* dbg_imin;
};

__device__ __forceinline__ const uint8_t* region_ptr(const GemmCtx& c, uint32_t block) {
    return c.smem + kSlots * kSlotBytes + (block % kRegions) * kRegionBytes;
}

// Issue part P (0..3) of the LDS-DMA loads of stage s = 4 b + G (clamped
// past the last block); a group issues the stage kAhead ahead's four parts
// between its k-steps, so a full memory queue stalls the wave while its MFMAs
// run.  Every wave issues kLoadsStage loads per stage, plus kLoadsFirst when
// G == 0: the stage barriers' vmcnt counts (pending_loads) depend on it.
template <int G, int P>
__device__ __forceinline__ void issue_part(const GemmCtx& c, uint32_t s) {
    const uint32_t bu = s / 4, b = bu < c.nb ? bu : c.nb - 1;
    const uint32_t slot = c.lds + (s % kSlots) * kSlotBytes;
    if (P < 2) {
        // wave w loads the 1 KB pieces per * w .. per * w + per - 1 of the 16
        constexpr uint32_t per = 16 / kGemmWaves;
        const uint8_t* ag = c.act_tile + act_group_offset(b, G) + c.wave * per * 1024;
#pragma unroll
        for (uint32_t j = P * per / 2; j < (P + 1) * per / 2; ++j)
            g2l(ag + j * 1024, c.lane * 16, slot + (c.wave * per + j) * 1024);
    } else if (P == 2) {
        // layout tile t: the qs bytes of group G of its 16 rows are the 512 bytes at
        // (G/2) * 1024 + (G%2) * 512 of the block's chunk; wave w loads tiles 2w, 2w+1
        const uint8_t* wb = c.w_first + (uint64_t)b * kQ4KChunk + (G / 2) * 1024 + (G % 2) * 512;
        g2l(wb, c.w_lane, slot + kSlotW + c.wave * 1024);
        if (G == 0) {
            const uint32_t reg = c.lds + kSlots * kSlotBytes + (bu % kRegions) * kRegionBytes;
            if (c.lane < 32) g2l(c.w_first + (uint64_t)b * kQ4KChunk, c.h_lane, reg + c.wave * 512);
        }
    } else if (G == 0) {
        // the record: rb bytes (rl lanes) per wave
        constexpr uint32_t rb = kActRecordBytes / kGemmWaves, rl = rb / 16;
        const uint32_t reg = c.lds + kSlots * kSlotBytes + (bu % kRegions) * kRegionBytes;
        const uint8_t* rec = c.act_tile + act_record_offset(c.nb, b) + c.wave * rb;
        if (rl >= 64 || c.lane < rl) g2l(rec, c.lane * 16, reg + kRegRec + c.wave * rb);
        if (rl > 64 && c.lane < rl - 64) g2l(rec + 1024, c.lane * 16, reg + kRegRec + c.wave * rb + 1024);
    }
}

template <int G>
__device__ __forceinline__ void issue_part_at(const GemmCtx& c, uint32_t s, int P) {
    switch (P) {  // P is a constant after unrolling
        case 0: issue_part<G, 0>(c, s); break;
        case 1: issue_part<G, 1>(c, s); break;
        case 2: issue_part<G, 2>(c, s); break;
        default: issue_part<G, 3>(c, s); break;
    }
}

template <int G>
__device__ __forceinline__ void issue_stage(const GemmCtx& c, uint32_t s) {
    issue_part<G, 0>(c, s);
    issue_part<G, 1>(c, s);
    issue_part<G, 2>(c, s);
    issue_part<G, 3>(c, s);
}

// v_and_or_b32 (VOP3 takes no literal: the mask comes in an SGPR, the bias in a VGPR)
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t bias) {
    uint32_t d;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(v), "s"(mask), "v"(bias));
    return d;
}

// B operand of k-step S of a group for one lane: its 16-byte piece holds
// block positions 64g + 16h + i (low nibble) and 64g + 32 + 16h + i (high
// nibble), i = 0..15.  S = 0, 1: low nibbles of bytes 8S .. 8S+7; S = 2, 3:
// high nibbles of bytes 8(S-2) .. ; slot order kPerm.  sh: the piece's words
// shifted right by 8.
template <int S>
__device__ __forceinline__ f16x8 dequant_q4(const uint4& pc, const uint4& sh, const GroupScales& sc, uint32_t bias) {
    const uint32_t w0 = (S & 1) ? pc.z : pc.x, w1 = (S & 1) ? pc.w : pc.y;
    const uint32_t v0 = (S & 1) ? sh.z : sh.x, v1 = (S & 1) ? sh.w : sh.y;
    const uint32_t mask = S < 2 ? 0x000f000fu : 0x00f000f0u;
    const f16x2 scale = S < 2 ? sc.lo : sc.hi, neg = S < 2 ? sc.lo_neg : sc.hi_neg;
    const f16x2 r0 = __builtin_elementwise_fma(as_h2(and_or(w0, mask, bias)), scale, neg);
    const f16x2 r1 = __builtin_elementwise_fma(as_h2(and_or(v0, mask, bias)), scale, neg);
    const f16x2 r2 = __builtin_elementwise_fma(as_h2(and_or(w1, mask, bias)), scale, neg);
    const f16x2 r3 = __builtin_elementwise_fma(as_h2(and_or(v1, mask, bias)), scale, neg);
    f16x8 v;
    v[0] = r0[0], v[1] = r0[1], v[2] = r1[0], v[3] = r1[1];
    v[4] = r2[0], v[5] = r2[1], v[6] = r3[0], v[7] = r3[1];
    return v;
}

// Accumulator tile T of a finished fold unit into y.  MINS: the unit ends a
// block (its mins term is due).  DBG stores token 0's integers (add: the unit
// is a second half; its integer adds to the first half's).
template <int T, bool MINS, bool DBG>
__device__ __forceinline__ void fold_tile(const GemmCtx& c, const f32x16 (&h)[4], float (&y)[4][16],
                                          const FoldRow& fr, const uint8_t* reg, uint32_t b, bool add) {
    f32x16 mn = {};
    if (MINS) {
        const f16x8 bs = *(const f16x8*)(reg + kRegRec + c.kh * 2048 + (32 * T + c.ln) * 16);
        mn = mfma16(bs, fr.mins, (f32x16){});
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 da = *(const float4*)(reg + kRegRec + kRecDa + (32 * T + 8 * q + 4 * c.kh) * 4);
        const float dav[4] = {da.x, da.y, da.z, da.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = 4 * q + k;
            float t = fr.d * h[T][i];
            if (MINS) t = __builtin_fmaf(-fr.dmin, mn[i], t);
            y[T][i] = __builtin_fmaf(dav[k], t, y[T][i]);
        }
    }
    if (DBG && T == 0) {
        const uint32_t row = c.nt * kGemmTN + 32 * c.wave + c.ln;
        if (c.mt == 0 && c.kh == 0 && row < c.rows) {
            int32_t* p = c.dbg_isum + (uint64_t)row * c.nb + b;
            *p = (add ? *p : 0) + (int32_t)h[T][0];
            if (MINS) c.dbg_imin[(uint64_t)row * c.nb + b] = (int32_t)mn[0];
        }
    }
}

template <bool MINS, bool DBG>
__device__ __forceinline__ void fold_all(const GemmCtx& c, const f32x16 (&h)[4], float (&y)[4][16],
                                         const uint8_t* reg, uint32_t b, bool add) {
    const uint32_t tl = 2 * c.wave + (c.ln >> 4);
    const FoldRow fr = fold_row(*(const uint4*)(reg + tl * 256 + (c.ln & 15) * 16), c.kh);
    fold_tile<0, MINS, DBG>(c, h, y, fr, reg, b, add);
    fold_tile<1, MINS, DBG>(c, h, y, fr, reg, b, add);
    fold_tile<2, MINS, DBG>(c, h, y, fr, reg, b, add);
    fold_tile<3, MINS, DBG>(c, h, y, fr, reg, b, add);
}

#define RLQ_SWITCH4(v, F)     \
    switch (v) {              \
        case 0: F(0); break;  \
        case 1: F(1); break;  \
        case 2: F(2); break;  \
        default: F(3); break; \
    }

// One block: 4 groups of 4 k-steps into h, folded into y after the block, or
// after each half when a token of the tile has the block flagged.
template <bool DBG>
__device__ __forceinline__ void gemm_block(const GemmCtx& c, uint32_t b, f32x16 (&h)[4], float (&y)[4][16]) {
    const uint8_t* reg = region_ptr(c, b);
    const uint32_t tl = 2 * c.wave + (c.ln >> 4);
    const uint32_t bias = 0x64006400u;
    Q4Words qw;
    bool split = false;
#pragma unroll
    for (int G = 0; G < 4; ++G) {
        const uint32_t s = b * 4 + G;
        // stage s has landed for every wave; slot (s - 1) % 3 is free again
        if (DBG) {
            stage_barrier<0>();
        } else {
#define RLQ_BAR(k) stage_barrier<pending_loads(k)>()
            RLQ_SWITCH4(G, RLQ_BAR)
#undef RLQ_BAR
        }
        if (G == 0) {  // the block's region arrived with its first stage
            qw = q4_words(*(const uint4*)(reg + tl * 256 + (c.ln & 15) * 16));
            const uint32_t f0 = reg[kRegRec + kRecFlags + c.lane], f1 = reg[kRegRec + kRecFlags + 64 + c.lane];
            split = __ballot(((f0 | f1) & 2u) != 0) != 0;  // the same for every wave of the workgroup
        }
        const uint8_t* slot = c.smem + (s % kSlots) * kSlotBytes;
        GroupScales sc;
#define RLQ_SC(k) sc = group_scales<k>(qw)
        RLQ_SWITCH4(G, RLQ_SC)
#undef RLQ_SC
        const uint4 pc = *(const uint4*)(slot + kSlotW + tl * 512 + c.kh * 256 + (c.ln & 15) * 16);
        const uint4 sh = make_uint4(pc.x >> 8, pc.y >> 8, pc.z >> 8, pc.w >> 8);
        // software pipeline over the group's 4 k-steps: the A reads of k-step
        // S+1 are in flight and its B operand is dequantized while the MFMAs
        // of k-step S run
        const uint8_t* abase = slot + c.kh * 2048 + c.ln * 16;
        f16x8 a[2][4], bq[2];
#pragma unroll
        for (int T = 0; T < 4; ++T) a[0][T] = *(const f16x8*)(abase + T * 512);
        bq[0] = dequant_q4<0>(pc, sh, sc, bias);
#pragma unroll
        for (int S = 0; S < 4; ++S) {
            if (S < 3) {
#pragma unroll
                for (int T = 0; T < 4; ++T) a[(S + 1) & 1][T] = *(const f16x8*)(abase + (S + 1) * 4096 + T * 512);
            }
            __builtin_amdgcn_sched_barrier(0);
            const bool fresh = S == 0 && G == 0;
#pragma unroll
            for (int T = 0; T < 4; ++T) h[T] = mfma16(a[S & 1][T], bq[S & 1], fresh ? (f32x16){} : h[T]);
            // part S of the stage kAhead ahead
#define RLQ_ISSUE(k) issue_part_at<((k) + kAhead) % 4>(c, s + kAhead, S)
            RLQ_SWITCH4(G, RLQ_ISSUE)
#undef RLQ_ISSUE
            if (S < 3) {
#define RLQ_DQ(k) bq[(S + 1) & 1] = dequant_q4<(k) < 3 ? (k) + 1 : 3>(pc, sh, sc, bias)
                RLQ_SWITCH4(S, RLQ_DQ)
#undef RLQ_DQ
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (G == 1 && split) {  // first half folded on its own; the second starts from zero
            fold_all<false, DBG>(c, h, y, reg, b, false);
#pragma unroll
            for (int T = 0; T < 4; ++T) h[T] = (f32x16){};
        }
        if (G == 3) fold_all<true, DBG>(c, h, y, reg, b, split);
    }
}

template <bool DBG>
__global__ __launch_bounds__(kGemmThreads, 8 / kGemmWaves) void q4k_gemm_kernel(GemmArgs g) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // XCD-aware order: workgroups i, i + 8, ... share an XCD (and its L2); give
    // each XCD a contiguous run of row tiles with all their token tiles, so
    // the XCD reads its weights from HBM once
    const uint32_t G = g.NT * g.MT;
    uint32_t id = blockIdx.x;
    if (G % 8 == 0) id = (id % 8) * (G / 8) + id / 8;
    GemmCtx c;
    c.smem = smem;
    c.nb = g.nb;
    c.rows = g.rows;
    c.nt = id / g.MT;
    c.mt = id % g.MT;
    c.wave = wave;
    c.lane = lane;
    c.ln = lane & 31;
    c.kh = lane >> 5;
    c.act_tile = g.img + (uint64_t)c.mt * g.nb * kActTileBlockBytes;
    c.dbg_isum = g.dbg_isum;
    c.dbg_imin = g.dbg_imin;
    c.lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
    // weight loads: tiles past the last one read the last one (rows >= g.rows are never stored)
    const uint32_t t0 = c.nt * (kGemmTN / 16), tmax = g.ntiles16 - 1, tstride = g.nb * kQ4KChunk;
    c.w_first = g.w + (uint64_t)t0 * tstride;
    const uint32_t tw = t0 + 2 * wave + (lane >> 5);
    c.w_lane = ((tw < tmax ? tw : tmax) - t0) * tstride + (lane & 31) * 16;
    const uint32_t th = t0 + 2 * wave + ((lane >> 4) & 1);
    c.h_lane = ((th < tmax ? th : tmax) - t0) * tstride + 2048 + (lane & 15) * 16;

    // the first stages' loads go out before the flag scan, so the two wait together
    issue_stage<0>(c, 0);
    if (kAhead > 1) issue_stage<1>(c, 1);
    if (kAhead > 2) issue_stage<2>(c, 2);
    if (kAhead > 3) issue_stage<3>(c, 3);
    // a data error in any token: this call writes nothing (flag bit 0 of every
    // record); eight words per thread in flight at once
    int bad = 0;
    const uint32_t words = g.MT * g.nb * (kGemmTM / 4);
    for (uint32_t i0 = threadIdx.x; i0 < words; i0 += 8 * kGemmThreads) {
        uint32_t f[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {  // past the end: the last word again (no branch between the loads)
            const uint32_t i = i0 + k * kGemmThreads < words ? i0 + k * kGemmThreads : words - 1;
            const uint32_t rec = i / (kGemmTM / 4), part = i % (kGemmTM / 4);
            const uint8_t* base = g.img + (uint64_t)(rec / g.nb) * g.nb * kActTileBlockBytes +
                                  act_record_offset(g.nb, rec % g.nb) + kRecFlags;
            f[k] = ((const uint32_t*)base)[part];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) bad |= (int)(f[k] & 0x01010101u);
    }
    if (__syncthreads_or(bad)) {
        // the LDS-DMA loads must land before the workgroup's LDS is released
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }

    float y[4][16];
#pragma unroll
    for (int T = 0; T < 4; ++T)
#pragma unroll
        for (int i = 0; i < 16; ++i) y[T][i] = 0.0f;
    f32x16 h[4];
    for (uint32_t b = 0; b < c.nb; ++b) gemm_block<DBG>(c, b, h, y);
    // LDS-DMA loads past the end may still be in flight: they must land before
    // the workgroup's LDS can go to another workgroup
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    const uint32_t row = c.nt * kGemmTN + 32 * wave + c.ln;
#pragma unroll
    for (int T = 0; T < 4; ++T)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t m = c.mt * kGemmTM + 32 * T + 8 * (i / 4) + 4 * c.kh + (i % 4);
            if (m < g.M && row < g.rows) g.y[(uint64_t)m * g.ldy + row] = y[T][i];
        }
}

// ---------------------------------------------------------------------------
static uint64_t gemm_padded_tokens(uint64_t M) { return (M + kGemmTM - 1) / kGemmTM * kGemmTM; }

size_t gemm_planes_bytes(uint64_t M, uint64_t K) {
    return gemm_padded_tokens(M) / kGemmTM * (K / 256) * kActTileBlockBytes;
}

hipError_t launch_gemm_q4k(const uint8_t* w, uint64_t rows, uint64_t cols, const float* x, uint64_t M, float* y,
                           uint64_t ldy, void* scratch, unsigned long long* err_word, int32_t* dbg_isum,
                           int32_t* dbg_imin, hipStream_t s) {
    if (rows == 0 || cols == 0 || cols % 256 || M == 0 || rows > 0xffffffffull || cols > (1u << 30) ||
        M > (1u << 24))
        return hipErrorInvalidValue;
    const uint64_t nb = cols / 256, MT = gemm_padded_tokens(M) / kGemmTM;
    const uint64_t NT = (rows + kGemmTN - 1) / kGemmTN;
    if (MT * NT > 0x7fffffffull || MT * nb * (kGemmTM / 16) > 0x7fffffffull) return hipErrorInvalidValue;
    uint8_t* img = (uint8_t*)scratch;
    hipLaunchKernelGGL(gemm_act_kernel, dim3((unsigned)(MT * nb * (kGemmTM / 16))), dim3(256), 0, s, x, (uint32_t)M,
                       (uint32_t)cols, img, err_word, 0u);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    GemmArgs g{};
    g.w = w;
    g.rows = (uint32_t)rows;
    g.nb = (uint32_t)nb;
    g.ntiles16 = (uint32_t)layout_tiles(rows);
    g.img = img;
    g.M = (uint32_t)M;
    g.NT = (uint32_t)NT;
    g.MT = (uint32_t)MT;
    g.y = y;
    g.ldy = ldy;
    g.dbg_isum = dbg_isum;
    g.dbg_imin = dbg_imin;
    static LdsLimit lds_plain, lds_dbg;
    e = dbg_isum ? lds_dbg.raise((const void*)q4k_gemm_kernel<true>, kGemmLds)
                 : lds_plain.raise((const void*)q4k_gemm_kernel<false>, kGemmLds);
    if (e != hipSuccess) return e;
    const dim3 grid((unsigned)(MT * NT));
    if (dbg_isum) hipLaunchKernelGGL(q4k_gemm_kernel<true>, grid, dim3(kGemmThreads), kGemmLds, s, g);
    else hipLaunchKernelGGL(q4k_gemm_kernel<false>, grid, dim3(kGemmThreads), kGemmLds, s, g);
    return hipGetLastError();
}

}  // namespace rlq
