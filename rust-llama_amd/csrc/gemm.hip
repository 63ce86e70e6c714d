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

constexpr int kGemmWaves = 4;
constexpr int kGemmTM = 32 * kGemmWaves;  // tokens per workgroup: 32 per wave
constexpr int kGemmTN = 64;               // weight rows per workgroup: two 32-row MFMA column tiles

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

__global__ __launch_bounds__(kGemmWaves * 64) void q4k_gemm_kernel(GemmArgs g) {
    // B operands of the two planes in the lane order of v_mfma_i32_32x32x32_i8:
    // [plane][col tile][sub-block][k half][row n][16 bytes]
    __shared__ __align__(16) uint8_t planes[2][2][8][2][32][16];
    __shared__ __align__(16) uint32_t mins[2][32][2];  // [col tile][row][mn 0..3 | mn 4..7]
    __shared__ float dws[kGemmTN], dmws[kGemmTN], das[kGemmTM];

    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
    const uint32_t tok = m0 + 32 * wave + ln;  // this lane's A row (< Mp)
    // staging role: wave t dequantizes 16-row tile t of the workgroup's 64 rows
    const uint32_t sn = lane & 15, skq = lane >> 4, sg = skq >> 1, sh = skq & 1;
    const uint32_t srow = 16 * wave + sn, sc_tile = srow >> 5, sc_n = srow & 31;
    const uint32_t tile16 = n0 / 16 + wave;

    float acc[2][16];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[c][i] = 0.0f;

    for (uint32_t b = 0; b < nb; ++b) {
        // ---- stage: two int8 planes, the mins and d, dmin of the 64 rows
        if (tile16 < g.ntiles16) {
            const uint8_t* base = g.w + ((uint64_t)tile16 * nb + b) * kQ4KChunk;
            const uint4 w0 = load_stream16(base + lane * 16);
            const uint4 w1 = load_stream16(base + 1024 + lane * 16);
            const uint4 h = load_stream16(base + 2048 + sn * 16);
            const uint32_t scA = h.y & 0x3f3f3f3fu;
            const uint32_t scB = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
            const uint32_t mnA = h.z & 0x3f3f3f3fu;
            const uint32_t mnB = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
            // this lane: sub-blocks 2g, 2g+1 (w0, g = sg) and 2g'... (w1, g' = 2 + sg), half sh
#pragma unroll
            for (int P = 0; P < 2; ++P) {
                const uint4 wv = P ? w1 : w0;
                const uint32_t scw = P ? scB : scA;
                const uint32_t s_lo = 4 * P + 2 * sg, s_hi = s_lo + 1;
                const uint32_t c_lo = __builtin_amdgcn_ubfe(scw, 16 * sg, 8);
                const uint32_t c_hi = __builtin_amdgcn_ubfe(scw, 16 * sg + 8, 8);
                const uint32_t lo[4] = {wv.x & 0x0f0f0f0fu, wv.y & 0x0f0f0f0fu, wv.z & 0x0f0f0f0fu,
                                        wv.w & 0x0f0f0f0fu};
                const uint32_t hi[4] = {(wv.x >> 4) & 0x0f0f0f0fu, (wv.y >> 4) & 0x0f0f0f0fu,
                                        (wv.z >> 4) & 0x0f0f0f0fu, (wv.w >> 4) & 0x0f0f0f0fu};
                *(uint4*)planes[0][sc_tile][s_lo][sh][sc_n] =
                    make_uint4(bytes_times(lo[0], c_lo >> 3), bytes_times(lo[1], c_lo >> 3),
                               bytes_times(lo[2], c_lo >> 3), bytes_times(lo[3], c_lo >> 3));
                *(uint4*)planes[1][sc_tile][s_lo][sh][sc_n] =
                    make_uint4(bytes_times(lo[0], c_lo & 7), bytes_times(lo[1], c_lo & 7),
                               bytes_times(lo[2], c_lo & 7), bytes_times(lo[3], c_lo & 7));
                *(uint4*)planes[0][sc_tile][s_hi][sh][sc_n] =
                    make_uint4(bytes_times(hi[0], c_hi >> 3), bytes_times(hi[1], c_hi >> 3),
                               bytes_times(hi[2], c_hi >> 3), bytes_times(hi[3], c_hi >> 3));
                *(uint4*)planes[1][sc_tile][s_hi][sh][sc_n] =
                    make_uint4(bytes_times(hi[0], c_hi & 7), bytes_times(hi[1], c_hi & 7),
                               bytes_times(hi[2], c_hi & 7), bytes_times(hi[3], c_hi & 7));
            }
            if (skq == 0) {
                mins[sc_tile][sc_n][0] = mnA;
                mins[sc_tile][sc_n][1] = mnB;
                dws[srow] = half_to_float(h.x);
                dmws[srow] = half_to_float(h.x >> 16);
            }
        } else {  // rows past the matrix: zero planes
#pragma unroll
            for (int P = 0; P < 2; ++P)
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const uint32_t s_ = 4 * P + 2 * sg + q;
                    *(uint4*)planes[0][sc_tile][s_][sh][sc_n] = make_uint4(0, 0, 0, 0);
                    *(uint4*)planes[1][sc_tile][s_][sh][sc_n] = make_uint4(0, 0, 0, 0);
                }
            if (skq == 0) {
                mins[sc_tile][sc_n][0] = mins[sc_tile][sc_n][1] = 0;
                dws[srow] = dmws[srow] = 0.0f;
            }
        }
        for (uint32_t t = threadIdx.x; t < kGemmTM; t += kGemmWaves * 64) das[t] = g.da[(uint64_t)(m0 + t) * nb + b];
        __syncthreads();

        // ---- this wave's 32 tokens x 64 rows
        i32x4 A[8];
        const int8_t* ap = g.q8 + (uint64_t)tok * g.K + b * 256 + 16 * kh;
#pragma unroll
        for (int s = 0; s < 8; ++s) A[s] = *(const i32x4*)(ap + 32 * s);
        const long Am = *(const long*)(g.bsd + ((uint64_t)tok * nb + b) * 16 + 8 * kh);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            i32x16 ca, cb;
#pragma unroll
            for (int i = 0; i < 16; ++i) ca[i] = cb[i] = 0;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                ca = mfma32(A[s], *(const i32x4*)planes[0][c][s][kh][ln], ca);
                cb = mfma32(A[s], *(const i32x4*)planes[1][c][s][kh][ln], cb);
            }
            const long mn = *(const long*)mins[c][ln];
            const i32x16 clo = mfma32k16(Am, kh == 0 ? mn : 0);
            const i32x16 chi = mfma32k16(Am, kh == 1 ? mn : 0);
            const float dw = dws[32 * c + ln], dmw = dmws[32 * c + ln];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t ti = 32 * wave + 8 * (i / 4) + 4 * kh + (i % 4);
                const float dai = das[ti];
                const int32_t I = 8 * ca[i] + cb[i];
                const int32_t Mn = clo[i] + 128 * chi[i];
                acc[c][i] += (dw * dai) * (float)I - (dmw * dai) * (float)Mn;
                if (g.dbg_isum && m0 + ti == 0) {
                    const uint32_t row = n0 + 32 * c + ln;
                    if (row < g.rows) {
                        g.dbg_isum[(uint64_t)row * nb + b] = I;
                        g.dbg_imin[(uint64_t)row * nb + b] = Mn;
                    }
                }
            }
        }
        __syncthreads();
    }

#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const uint32_t row = n0 + 32 * c + ln;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t m = m0 + 32 * wave + 8 * (i / 4) + 4 * kh + (i % 4);
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
    const dim3 grid((unsigned)((rows + kGemmTN - 1) / kGemmTN), (unsigned)(Mp / kGemmTM));
    hipLaunchKernelGGL(q4k_gemm_kernel, grid, dim3(kGemmWaves * 64), 0, s, g);
    return hipGetLastError();
}

}  // namespace rlq
