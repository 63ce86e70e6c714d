// gemm.hip - prefill GEMM for Q4_K weights on gfx950: y[m][n] = dot(row n, token m)
// for many tokens at once, on int8 MFMA.
//
// Contract: the GGML MUL_MAT semantics of crates/tensor/src/cpu_extra.rs:756-873
// -- every token (column) is quantized to Q8_K on its own (:820) and every
// output is dot_packed(weight row, token) (:860), i.e. the Q4_K dot of
// crates/quant/src/matvec_extra.rs:212-271, 286-293.  Prefill in the
// reference is M such matvecs (crates/inference/src/lib.rs:407,
// crates/model-runtime/src/context.rs:452); this kernel computes the same
// exact per-block integers for all M tokens in one pass over the weights.
//
// Integer decomposition.  Per (token m, row n, block):
//   I  = sum_s sc_s * sum_{j in s} q_j x_j        (sc: 6-bit sub-block scale)
//   Mn = sum_s mn_s * bsum32_s(m)                 (mn: 6-bit sub-block min)
//   y += d_n * da_m * I - dmin_n * da_m * Mn      (f32, block by block)
// sc * q does not fit int8, so sc = 8a + b (a, b <= 7) and the weights are
// dequantized to two int8 planes a*q and b*q (each <= 105): I = 8 C_a + C_b
// with C_a, C_b accumulated over the whole block by v_mfma_i32_32x32x32_i8.
// The mins term runs on v_mfma_i32_32x32x16_i8 with bsum32 split into base-128
// digits (lo in 0..127, hi in -32..31): Mn = C_lo + 128 C_hi.  Every integer is
// exact; only the f32 accumulation order differs from the reference's.
#include "rlq_device.hpp"
#include "rlq_internal.hpp"
#include "rlq_layout.hpp"
#include "rlq_q8k.hpp"

namespace rlq {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Activations: f32 x [M][K] -> Q8_K planes for the GEMM
//   q8  int8 [Mp][K]          (Mp = M rounded up to the token tile)
//   da  f32  [Mp][nb]
//   bsd int8 [Mp][nb][16]     lo digits of bsum32_s in 0..7, hi digits in 8..15
//   bad u32  [Mp]             1 when a block of the token is invalid
// Tokens >= M are written as zeros.  One workgroup of 256 lanes per token:
// a 16-lane DPP row quantizes one 256-value block (q8k_row16).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gemm_act_kernel(const float* __restrict__ x, uint32_t M, uint32_t K,
                                                       int8_t* __restrict__ q8, float* __restrict__ da,
                                                       int8_t* __restrict__ bsd, uint32_t* __restrict__ bad,
                                                       unsigned long long* err_word, uint32_t err_column0) {
    const uint32_t m = blockIdx.x, lane = threadIdx.x & 63, r16 = lane & 15;
    const uint32_t nb = K / 256, upr = K / 16;  // 16-value units per token
    int any_bad = 0;
    for (uint32_t u = threadIdx.x; u < upr; u += 256) {  // upr % 16 == 0: rows of 16 stay whole
        const uint32_t blk = u / 16;
        float v[16];
        if (m < M) {
            const float4* src = (const float4*)(x + (uint64_t)m * K + u * 16);
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
        if (o.kind >= 0) {
            any_bad = 1;
            if (r16 == 0)
                report_error(err_word, o.kind == kKindNonFinite
                                           ? error_key(err_column0 + m, kKindNonFinite, blk * 256ull + o.index)
                                           : error_key(err_column0 + m, kKindScale, blk));
        }
        *(uint4*)(q8 + (uint64_t)m * K + u * 16) = make_uint4(o.q[0], o.q[1], o.q[2], o.q[3]);
        if (r16 == 0) da[(uint64_t)m * nb + blk] = o.d;
        // bsum32 of sub-block s = bsum[2s] + bsum[2s+1], as base-128 digits
        const int32_t s32 = o.bsum + dpp_i<kQuadXor1>(o.bsum);
        if ((r16 & 1) == 0) {
            int8_t* dst = bsd + ((uint64_t)m * nb + blk) * 16 + (r16 >> 1);
            dst[0] = (int8_t)(s32 & 127);
            dst[8] = (int8_t)(s32 >> 7);
        }
    }
    const int token_bad = __syncthreads_or(any_bad);
    if (threadIdx.x == 0) bad[m] = token_bad ? 1u : 0u;
}

// ---------------------------------------------------------------------------
// GEMM
// ---------------------------------------------------------------------------
struct GemmArgs {
    const uint8_t* w;  // Q4_K, tiled device layout (rlq_layout.hpp)
    uint32_t rows, nb, ntiles16;
    const int8_t* q8;
    const float* da;
    const int8_t* bsd;
    const uint32_t* bad;
    uint32_t M, Mp, K;
    float* y;  // y[m * ldy + n]
    uint64_t ldy;
    int32_t* dbg_isum;  // exact integers of token 0, or null
    int32_t* dbg_imin;
};

// Workgroup: 8 waves over 128 tokens x 128 weight rows; wave (tg, rg) = (w % 4,
// w / 4) computes tokens 32 tg .. +31 against rows 64 rg .. +63 (two 32-row
// MFMA column tiles).  The two int8 planes of the workgroup's 128 rows are
// double-buffered in LDS: while the MFMAs of block b read one buffer, the
// waves dequantize block b+1 (loaded into registers one block ahead) into the
// other, and one barrier per block separates the two.
constexpr int kGemmWaves = 8;
constexpr int kGemmTM = 128;  // tokens per workgroup
constexpr int kGemmTN = 128;  // weight rows per workgroup (eight 16-row tiles)

__device__ __forceinline__ i32x16 mfma32(i32x4 a, i32x4 b, i32x16 c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ i32x16 mfma32k16(long a, long b) {
    i32x16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0;
    return __builtin_amdgcn_mfma_i32_32x32x16_i8(a, b, z, 0, 0, 0);
}

// bytes * s for four unsigned bytes <= 15 and s <= 7: no product leaves its byte
__device__ __forceinline__ uint32_t bytes_times(uint32_t w, uint32_t s) {
    const u16x2 p = __builtin_bit_cast(u16x2, w) * (u16x2){(unsigned short)s, (unsigned short)s};
    return __builtin_bit_cast(uint32_t, p);
}

// One LDS buffer: planes [plane][row tile of 32][sub-block][k half][row][16 B],
// in the B-operand lane order of v_mfma_i32_32x32x32_i8, plus the rows' mins
// and d, dmin and the tokens' activation scales of the block.
struct GemmStage {
    uint8_t planes[2][4][8][2][32][16];
    uint32_t mins[4][32][2];
    float dw[kGemmTN], dmw[kGemmTN], da[kGemmTM];
};

// Raw Q4_K chunk of one 16-row tile (lane roles of the decode layout).
struct RawTile {
    uint4 w0, w1, h;
};

__device__ __forceinline__ void dequant_tile(GemmStage& st, const RawTile& r, bool live, uint32_t tile_in_wg,
                                             uint32_t lane) {
    const uint32_t sn = lane & 15, skq = lane >> 4, sg = skq >> 1, sh = skq & 1;
    const uint32_t row = 16 * tile_in_wg + sn, rt = row >> 5, rn = row & 31;
    const uint32_t scA = live ? r.h.y & 0x3f3f3f3fu : 0;
    const uint32_t scB = live ? (r.h.w & 0x0f0f0f0fu) | ((r.h.y >> 2) & 0x30303030u) : 0;
#pragma unroll
    for (int P = 0; P < 2; ++P) {
        const uint4 wv = P ? r.w1 : r.w0;
        const uint32_t scw = P ? scB : scA;
        const uint32_t s_lo = 4 * P + 2 * sg, s_hi = s_lo + 1;
        const uint32_t c_lo = __builtin_amdgcn_ubfe(scw, 16 * sg, 8), c_hi = __builtin_amdgcn_ubfe(scw, 16 * sg + 8, 8);
        const uint32_t lo[4] = {wv.x & 0x0f0f0f0fu, wv.y & 0x0f0f0f0fu, wv.z & 0x0f0f0f0fu, wv.w & 0x0f0f0f0fu};
        const uint32_t hi[4] = {(wv.x >> 4) & 0x0f0f0f0fu, (wv.y >> 4) & 0x0f0f0f0fu, (wv.z >> 4) & 0x0f0f0f0fu,
                                (wv.w >> 4) & 0x0f0f0f0fu};
        *(uint4*)st.planes[0][rt][s_lo][sh][rn] = make_uint4(
            bytes_times(lo[0], c_lo >> 3), bytes_times(lo[1], c_lo >> 3), bytes_times(lo[2], c_lo >> 3),
            bytes_times(lo[3], c_lo >> 3));
        *(uint4*)st.planes[1][rt][s_lo][sh][rn] = make_uint4(
            bytes_times(lo[0], c_lo & 7), bytes_times(lo[1], c_lo & 7), bytes_times(lo[2], c_lo & 7),
            bytes_times(lo[3], c_lo & 7));
        *(uint4*)st.planes[0][rt][s_hi][sh][rn] = make_uint4(
            bytes_times(hi[0], c_hi >> 3), bytes_times(hi[1], c_hi >> 3), bytes_times(hi[2], c_hi >> 3),
            bytes_times(hi[3], c_hi >> 3));
        *(uint4*)st.planes[1][rt][s_hi][sh][rn] = make_uint4(
            bytes_times(hi[0], c_hi & 7), bytes_times(hi[1], c_hi & 7), bytes_times(hi[2], c_hi & 7),
            bytes_times(hi[3], c_hi & 7));
    }
    if (skq == 0) {
        st.mins[rt][rn][0] = live ? r.h.z & 0x3f3f3f3fu : 0;
        st.mins[rt][rn][1] = live ? ((r.h.w >> 4) & 0x0f0f0f0fu) | ((r.h.z >> 2) & 0x30303030u) : 0;
        st.dw[row] = live ? half_to_float(r.h.x) : 0.0f;
        st.dmw[row] = live ? half_to_float(r.h.x >> 16) : 0.0f;
    }
}

template <bool DBG>
__global__ __launch_bounds__(kGemmWaves * 64) void q4k_gemm_kernel(GemmArgs g) {
    extern __shared__ __align__(16) uint8_t smem[];
    GemmStage* stage = (GemmStage*)smem;  // [2]

    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tg = wave & 3, rg = wave >> 2;
    const uint32_t n0 = blockIdx.x * kGemmTN, m0 = blockIdx.y * kGemmTM;
    const uint32_t nb = g.nb;

    // a data error in any token: this call writes nothing
    int any_bad = 0;
    for (uint32_t i = threadIdx.x; i < g.M; i += kGemmWaves * 64) any_bad |= g.bad[i] != 0;
    if (__syncthreads_or(any_bad)) return;

    // MFMA lane roles: A (tokens) row l % 32, k half l / 32; B (weights) column
    // l % 32, k half l / 32; output element i = token 8(i/4) + 4(l/32) + i%4 of
    // the wave's 32, weight row l % 32 of the column tile.
    const uint32_t ln = lane & 31, kh = lane >> 5;
    const uint32_t tok = m0 + 32 * tg + ln;  // this lane's A row (< Mp)
    // staging: wave w loads and dequantizes 16-row tile w of the workgroup
    const uint32_t tile16 = n0 / 16 + wave;
    const bool tile_live = tile16 < g.ntiles16;
    const uint8_t* wbase = g.w + (uint64_t)(tile_live ? tile16 : 0) * nb * kQ4KChunk;
    auto load_raw = [&](uint32_t b) {
        RawTile r;
        const uint8_t* base = wbase + (uint64_t)b * kQ4KChunk;
        r.w0 = load_stream16(base + lane * 16);
        r.w1 = load_stream16(base + 1024 + lane * 16);
        r.h = load_stream16(base + 2048 + (lane & 15) * 16);
        return r;
    };
    const int8_t* arow = g.q8 + (uint64_t)tok * g.K + 16 * kh;
    const int8_t* mrow = g.bsd + (uint64_t)tok * nb * 16 + 8 * kh;
    auto load_a = [&](uint32_t b, i32x4 (&A)[8], long& Am) {
#pragma unroll
        for (int s = 0; s < 8; ++s) A[s] = *(const i32x4*)(arow + b * 256 + 32 * s);
        Am = *(const long*)(mrow + b * 16);
    };

    // prologue: block 0 staged, block 1 in flight
    RawTile raw = load_raw(0);
    i32x4 A[8];
    long Am;
    load_a(0, A, Am);
    dequant_tile(stage[0], raw, tile_live, wave, lane);
    for (uint32_t t = threadIdx.x; t < kGemmTM; t += kGemmWaves * 64) stage[0].da[t] = g.da[(uint64_t)(m0 + t) * nb];
    if (nb > 1) raw = load_raw(1);
    __syncthreads();

    float acc[2][16];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[c][i] = 0.0f;

    for (uint32_t b = 0; b < nb; ++b) {
        const GemmStage& cur = stage[b & 1];
#pragma unroll
        for (int c = 0; c < 2; ++c) {  // one 32-row column tile at a time
            const uint32_t rt = 2 * rg + c;
            i32x16 ca, cb;
#pragma unroll
            for (int i = 0; i < 16; ++i) ca[i] = cb[i] = 0;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                ca = mfma32(A[s], *(const i32x4*)cur.planes[0][rt][s][kh][ln], ca);
                cb = mfma32(A[s], *(const i32x4*)cur.planes[1][rt][s][kh][ln], cb);
            }
            const long mn = *(const long*)cur.mins[rt][ln];
            const i32x16 clo = mfma32k16(Am, kh == 0 ? mn : 0);
            const i32x16 chi = mfma32k16(Am, kh == 1 ? mn : 0);
            const uint32_t wrow = 32 * rt + ln;
            const float dw = cur.dw[wrow], dmw = cur.dmw[wrow];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t ti = 32 * tg + 8 * (i / 4) + 4 * kh + (i % 4);
                const float dai = cur.da[ti];
                const int32_t I = 8 * ca[i] + cb[i];
                const int32_t Mn = clo[i] + 128 * chi[i];
                acc[c][i] += (dw * dai) * (float)I - (dmw * dai) * (float)Mn;
                if (DBG && m0 + ti == 0) {
                    const uint32_t row = n0 + wrow;
                    if (row < g.rows) {
                        g.dbg_isum[(uint64_t)row * nb + b] = I;
                        g.dbg_imin[(uint64_t)row * nb + b] = Mn;
                    }
                }
            }
        }
        // next block's activations: in flight during the staging and barrier
        if (b + 1 < nb) load_a(b + 1, A, Am);

        if (b + 1 < nb) {  // stage block b+1 into the other buffer
            GemmStage& nxt = stage[(b + 1) & 1];
            dequant_tile(nxt, raw, tile_live, wave, lane);
            for (uint32_t t = threadIdx.x; t < kGemmTM; t += kGemmWaves * 64)
                nxt.da[t] = g.da[(uint64_t)(m0 + t) * nb + b + 1];
            if (b + 2 < nb) raw = load_raw(b + 2);
        }
        __syncthreads();
    }

#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const uint32_t row = n0 + 32 * (2 * rg + c) + ln;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t m = m0 + 32 * tg + 8 * (i / 4) + 4 * kh + (i % 4);
            if (m < g.M && row < g.rows) g.y[(uint64_t)m * g.ldy + row] = acc[c][i];
        }
    }
}

// ---------------------------------------------------------------------------
size_t gemm_planes_bytes(uint64_t M, uint64_t K) {
    const uint64_t Mp = (M + kGemmTM - 1) / kGemmTM * kGemmTM, nb = K / 256;
    auto al = [](uint64_t v) { return (v + 255) & ~(uint64_t)255; };
    return al(Mp * K) + al(Mp * nb * 4) + al(Mp * nb * 16) + al(Mp * 4);
}

hipError_t launch_gemm_q4k(const uint8_t* w, uint64_t rows, uint64_t cols, const float* x, uint64_t M, float* y,
                           uint64_t ldy, void* scratch, unsigned long long* err_word, int32_t* dbg_isum,
                           int32_t* dbg_imin, hipStream_t s) {
    if (rows == 0 || cols == 0 || cols % 256 || M == 0 || rows > 0xffffffffull || cols > (1u << 30) ||
        M > (1u << 24))
        return hipErrorInvalidValue;
    const uint64_t Mp = (M + kGemmTM - 1) / kGemmTM * kGemmTM, nb = cols / 256;
    auto al = [](uint64_t v) { return (v + 255) & ~(uint64_t)255; };
    uint8_t* p = (uint8_t*)scratch;
    int8_t* q8 = (int8_t*)p;
    p += al(Mp * cols);
    float* da = (float*)p;
    p += al(Mp * nb * 4);
    int8_t* bsd = (int8_t*)p;
    p += al(Mp * nb * 16);
    uint32_t* bad = (uint32_t*)p;
    hipLaunchKernelGGL(gemm_act_kernel, dim3((unsigned)Mp), dim3(256), 0, s, x, (uint32_t)M, (uint32_t)cols, q8, da,
                       bsd, bad, err_word, 0u);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    GemmArgs g{};
    g.w = w;
    g.rows = (uint32_t)rows;
    g.nb = (uint32_t)nb;
    g.ntiles16 = (uint32_t)layout_tiles(rows);
    g.q8 = q8;
    g.da = da;
    g.bsd = bsd;
    g.bad = bad;
    g.M = (uint32_t)M;
    g.Mp = (uint32_t)Mp;
    g.K = (uint32_t)cols;
    g.y = y;
    g.ldy = ldy;
    g.dbg_isum = dbg_isum;
    g.dbg_imin = dbg_imin;
    static bool lds_set = false;
    const size_t lds = 2 * sizeof(GemmStage);
    if (!lds_set) {
        e = hipFuncSetAttribute((const void*)q4k_gemm_kernel<false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)q4k_gemm_kernel<true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)lds);
        if (e != hipSuccess) return e;
        lds_set = true;
    }
    const dim3 grid((unsigned)((rows + kGemmTN - 1) / kGemmTN), (unsigned)(Mp / kGemmTM));
    if (dbg_isum) hipLaunchKernelGGL(q4k_gemm_kernel<true>, grid, dim3(kGemmWaves * 64), lds, s, g);
    else hipLaunchKernelGGL(q4k_gemm_kernel<false>, grid, dim3(kGemmWaves * 64), lds, s, g);
    return hipGetLastError();
}

}  // namespace rlq
