// matvec.hip - HBM-bound decode matvec for Q4_K / Q6_K / Q8_0 weights on gfx950.
//
// Contract (paths relative to the rust-llama repository):
//   y[b][r] = dot_packed(row r, activation column b)
//     Q8_0  crates/quant/src/matvec.rs:115-160  (Q8_0 branch :124-128)
//     Q4_K  crates/quant/src/matvec_extra.rs:252-271, 286-293
//     Q6_K  crates/quant/src/matvec_extra.rs:272-283, 286-293
// Integer products are exact (v_dot4_i32_i8); each lane scales its exact
// integer partial by the block's f32 d, as the reference scales each of its
// eight integer lanes (matvec_extra.rs:286-288).  The f32 summation order
// differs from the reference's eight serial lanes; results agree to ~1e-7
// relative.
//
// Work mapping: a wave owns R consecutive rows.  Eight lanes own one weight
// block (lane c = 0..7 holds one 16-byte slice of it), so one wave instruction
// reads eight consecutive blocks (1152 B for Q4_K).  All weight loads of a
// pass are issued before the activation is staged into LDS, so HBM latency
// overlaps the staging.  Activations (all batch columns) live in LDS.
#include "rlq_device.hpp"
#include "rlq_internal.hpp"

namespace rlq {

constexpr int kWaves = 4;  // waves per workgroup
constexpr int kThreads = kWaves * kWave;

// ---- Q4_K lane decode ----------------------------------------------------

// 6-bit scale and min of sub-block j from the packed 12 bytes held as three
// little-endian words (matvec_extra.rs:212-221).
__device__ __forceinline__ void q4k_scale_min(uint32_t w1, uint32_t w2, uint32_t w3, int j, int32_t& sc,
                                              int32_t& mn) {
    if (j < 4) {
        sc = (int32_t)__builtin_amdgcn_ubfe(w1, 8 * j, 6);
        mn = (int32_t)__builtin_amdgcn_ubfe(w2, 8 * j, 6);
    } else {
        const int k = 8 * (j - 4);
        sc = (int32_t)(__builtin_amdgcn_ubfe(w3, k, 4) | (__builtin_amdgcn_ubfe(w1, k + 6, 2) << 4));
        mn = (int32_t)(__builtin_amdgcn_ubfe(w3, k + 4, 4) | (__builtin_amdgcn_ubfe(w2, k + 6, 2) << 4));
    }
}

// Lane c of a Q4_K block holds qs bytes 16c..16c+15: group g = c/2, half h =
// c%2.  Low nibbles are elements 64g + 16h + i (sub-block 2g), high nibbles
// elements 64g + 32 + 16h + i (sub-block 2g+1), i = 0..15.
struct Q4KLane {
    uint32_t lo[4], hi[4];
    int32_t sc_lo, sc_hi, mn;  // mn: min of the sub-block whose bsum this lane adds
    float dw, dmw;
};

__device__ __forceinline__ Q4KLane q4k_lane(uint4 hdr, uint4 qs, int c) {
    Q4KLane L;
    const int g = c >> 1, h = c & 1;
    int32_t mn_lo, mn_hi;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g, L.sc_lo, mn_lo);
    q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g + 1, L.sc_hi, mn_hi);
    L.mn = h ? mn_hi : mn_lo;
    const uint32_t v[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        L.lo[i] = v[i] & 0x0f0f0f0fu;
        L.hi[i] = (v[i] >> 4) & 0x0f0f0f0fu;
    }
    L.dw = half_to_float(hdr.x);
    L.dmw = half_to_float(hdr.x >> 16);
    return L;
}

// Exact integer partials of one lane against one activation block:
//   I = sc_lo * sum(lo . q8) + sc_hi * sum(hi . q8)
//   M = min_s * (bsum[2s] + bsum[2s+1]) for s = 2g + h  (matvec_extra.rs:258)
__device__ __forceinline__ void q4k_ints(const Q4KLane& L, const int8_t* a_blk, const int32_t* bs32_blk, int c,
                                         int32_t& I, int32_t& M) {
    const int g = c >> 1, h = c & 1;
    const uint4 alo = *(const uint4*)(a_blk + 64 * g + 16 * h);
    const uint4 ahi = *(const uint4*)(a_blk + 64 * g + 32 + 16 * h);
    int32_t ilo = dot4(L.lo[0], alo.x, 0);
    ilo = dot4(L.lo[1], alo.y, ilo);
    ilo = dot4(L.lo[2], alo.z, ilo);
    ilo = dot4(L.lo[3], alo.w, ilo);
    int32_t ihi = dot4(L.hi[0], ahi.x, 0);
    ihi = dot4(L.hi[1], ahi.y, ihi);
    ihi = dot4(L.hi[2], ahi.z, ihi);
    ihi = dot4(L.hi[3], ahi.w, ihi);
    I = L.sc_lo * ilo + L.sc_hi * ihi;
    M = L.mn * bs32_blk[2 * g + h];
}

// ---- Q6_K lane decode ----------------------------------------------------

// Lane c of a Q6_K block: g = c/4, s0 = (c/2)%2, p0 = 16(c%2).  It holds
// ql bytes 16c..16c+15 and qh bytes 32g + p0 .. +15, i.e. the 6-bit values of
// elements ja = 128g + 32 s0 + p0 + i (low nibble) and jb = ja + 64 (high
// nibble), i = 0..15 (matvec_extra.rs:273-279).  Both 16-element runs sit
// inside one scale group: sa = ja/16, sb = sa + 4.
struct Q6KLane {
    uint32_t qa[4], qb[4];  // unsigned 6-bit values, four per word
    int32_t sca, scb;
    float dw;
};

__device__ __forceinline__ Q6KLane q6k_lane(uint4 ql, uint4 qh, uint4 sc, uint32_t d16, int c) {
    Q6KLane L;
    const int g = c >> 2, s0 = (c >> 1) & 1;
    const uint32_t l[4] = {ql.x, ql.y, ql.z, ql.w}, hh[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        L.qa[i] = (l[i] & 0x0f0f0f0fu) | (((hh[i] >> (2 * s0)) & 0x03030303u) << 4);
        L.qb[i] = ((l[i] >> 4) & 0x0f0f0f0fu) | (((hh[i] >> (2 * s0 + 4)) & 0x03030303u) << 4);
    }
    // sa = 8g + 2 s0 + (c&1) is byte (2 s0 + (c&1)) of scale word 2g; sb = sa + 4
    // is the same byte of word 2g + 1.
    const int sh = 8 * (2 * s0 + (c & 1));
    L.sca = (int32_t)(int8_t)((g ? sc.z : sc.x) >> sh);
    L.scb = (int32_t)(int8_t)((g ? sc.w : sc.y) >> sh);
    L.dw = half_to_float(d16);
    return L;
}

// I = sc_a * sum((qa - 32) q8) + sc_b * sum((qb - 32) q8).  The -32 offset is
// applied through the 16-element activation sums: sum(q q8) - 32 bsum.
__device__ __forceinline__ int32_t q6k_ints(const Q6KLane& L, const int8_t* a_blk, const int32_t* bs16_blk, int c) {
    const int g = c >> 2, s0 = (c >> 1) & 1, p0 = 16 * (c & 1);
    const int ja = 128 * g + 32 * s0 + p0;
    const uint4 aa = *(const uint4*)(a_blk + ja);
    const uint4 ab = *(const uint4*)(a_blk + ja + 64);
    int32_t ia = dot4(L.qa[0], aa.x, 0);
    ia = dot4(L.qa[1], aa.y, ia);
    ia = dot4(L.qa[2], aa.z, ia);
    ia = dot4(L.qa[3], aa.w, ia);
    int32_t ib = dot4(L.qb[0], ab.x, 0);
    ib = dot4(L.qb[1], ab.y, ib);
    ib = dot4(L.qb[2], ab.z, ib);
    ib = dot4(L.qb[3], ab.w, ib);
    const int sa = ja >> 4;
    return L.sca * (ia - 32 * bs16_blk[sa]) + L.scb * (ib - 32 * bs16_blk[sa + 4]);
}

// ---- Q8_0 lane ---------------------------------------------------------
// Two lanes per 32-element block, lane half k holds elements 16k..16k+15.
__device__ __forceinline__ int32_t q8_0_ints(uint4 w, const int8_t* a16) {
    const uint4 a = *(const uint4*)a16;
    int32_t s = dot4(w.x, a.x, 0);
    s = dot4(w.y, a.y, s);
    s = dot4(w.z, a.z, s);
    return dot4(w.w, a.w, s);
}

// ---- greedy argmax key -----------------------------------------------------
// Largest value wins, then the lowest row (sampling.rs:607-613 keeps the first
// strict maximum).  -0.0 is folded onto +0.0 because they compare equal; NaN
// maps to 0 and never wins (the finish step handles a NaN at row 0).
__device__ __forceinline__ unsigned long long argmax_key(float v, uint64_t row) {
    if (v != v) return 0ull;
    uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)b << 32) | (0xffffffffull - (row & 0xffffffffull));
}

// ---- activation staging into LDS -------------------------------------------
// LDS layout: q8 [B][K] | d [B][nb] f32 | sums [B][S] i32, where S is nb*8
// (Q4_K: 32-element sums bsum[2s]+bsum[2s+1]) or K/16 (Q6_K: the bsums).
// Returns true when no staged block carries the error mark.
template <int B>
__device__ __forceinline__ bool stage_q8k(const ActPlanes& act, uint64_t K, uint32_t nb, bool pair_sums, int8_t* s_q,
                                          float* s_d, int32_t* s_sum) {
    const uint32_t tid = threadIdx.x;
    const uint64_t qwords = (uint64_t)B * K / 16;
    for (uint64_t i = tid; i < qwords; i += kThreads) ((uint4*)s_q)[i] = ((const uint4*)act.q)[i];
    int bad = 0;
    for (uint32_t i = tid; i < B * nb; i += kThreads) {
        s_d[i] = act.d[i];
        bad |= act.bad[i];
    }
    if (pair_sums) {
        for (uint32_t i = tid; i < B * nb * 8; i += kThreads)
            s_sum[i] = (int32_t)act.bsum[2 * i] + (int32_t)act.bsum[2 * i + 1];
    } else {
        for (uint32_t i = tid; i < B * nb * 16; i += kThreads) s_sum[i] = act.bsum[i];
    }
    return __syncthreads_or(bad) == 0;
}

template <int B>
__device__ __forceinline__ bool stage_q8_0(const ActPlanes& act, uint64_t K, uint32_t nb, int8_t* s_q, float* s_d) {
    const uint32_t tid = threadIdx.x;
    const uint64_t qwords = (uint64_t)B * K / 16;
    for (uint64_t i = tid; i < qwords; i += kThreads) ((uint4*)s_q)[i] = ((const uint4*)act.q)[i];
    int bad = 0;
    for (uint32_t i = tid; i < B * nb; i += kThreads) {
        s_d[i] = act.d[i];
        bad |= act.bad[i];
    }
    return __syncthreads_or(bad) == 0;
}

// Per-row epilogue: reduce each column's lane partials, store, update argmax.
template <int B>
__device__ __forceinline__ void finish_row(float (&acc)[B], uint64_t row, uint64_t rows, float* y, uint64_t ldy,
                                           unsigned long long (&best)[B]) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
        const float v = wave_sum(acc[b]);
        if (row < rows) {
            if ((threadIdx.x & 63) == b) y[(uint64_t)b * ldy + row] = v;
            const unsigned long long k = argmax_key(v, row);
            best[b] = k > best[b] ? k : best[b];
        }
    }
}

template <int B>
__device__ __forceinline__ void publish_argmax(const unsigned long long (&best)[B], unsigned long long* key) {
    if (!key) return;
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int b = 0; b < B; ++b)
            if (best[b]) atomicMax(key + b, best[b]);
    }
}

// ---------------------------------------------------------------------------
// Q4_K: R rows per wave, IT block-octets per pass.
// ---------------------------------------------------------------------------
template <int B, int R, int IT>
__global__ __launch_bounds__(kThreads) void q4k_matvec_kernel(const uint8_t* __restrict__ W, uint64_t rows,
                                                              uint32_t nb, ActPlanes act, float* __restrict__ y,
                                                              uint64_t ldy, unsigned long long* argmax_key_out) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint64_t K = (uint64_t)nb * 256;
    int8_t* s_q = (int8_t*)smem;
    float* s_d = (float*)(smem + B * K);
    int32_t* s_sum = (int32_t*)(s_d + B * nb);

    const int lane = threadIdx.x & 63, c = lane & 7, bi = lane >> 3;
    const uint64_t row0 = ((uint64_t)blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
    const uint32_t per_pass = 8 * IT;
    const uint32_t passes = (nb + per_pass - 1) / per_pass;

    uint4 wh[R][IT], wq[R][IT];
    auto issue = [&](uint32_t pass) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const uint32_t blk = pass * per_pass + it * 8 + bi;
                const uint64_t row = row0 + r;
                if (row < rows && blk < nb) {
                    const uint8_t* base = W + (row * nb + blk) * 144;
                    wh[r][it] = load_stream16(base);
                    wq[r][it] = load_stream16(base + 16 + 16 * c);
                } else {
                    wh[r][it] = make_uint4(0, 0, 0, 0);
                    wq[r][it] = make_uint4(0, 0, 0, 0);
                }
            }
    };
    issue(0);
    if (!stage_q8k<B>(act, K, nb, true, s_q, s_d, s_sum)) return;

    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[r][b] = 0.0f;

    for (uint32_t pass = 0; pass < passes; ++pass) {
        if (pass) issue(pass);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const uint32_t blk = pass * per_pass + it * 8 + bi;
                if (blk >= nb) continue;
                const Q4KLane L = q4k_lane(wh[r][it], wq[r][it], c);
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    int32_t I, M;
                    q4k_ints(L, s_q + b * K + blk * 256, s_sum + (b * nb + blk) * 8, c, I, M);
                    const float da = s_d[b * nb + blk];
                    const float d = L.dw * da, dmin = L.dmw * da;
                    acc[r][b] += d * (float)I - dmin * (float)M;
                }
            }
    }
    unsigned long long best[B];
#pragma unroll
    for (int b = 0; b < B; ++b) best[b] = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) finish_row<B>(acc[r], row0 + r, rows, y, ldy, best);
    publish_argmax<B>(best, argmax_key_out);
}

// ---------------------------------------------------------------------------
// Q6_K (planar device layout): R rows per wave, IT block-octets per pass.
// ---------------------------------------------------------------------------
template <int B, int R, int IT>
__global__ __launch_bounds__(kThreads) void q6k_matvec_kernel(const uint8_t* __restrict__ W, uint64_t rows,
                                                              uint32_t nb, ActPlanes act, float* __restrict__ y,
                                                              uint64_t ldy, unsigned long long* argmax_key_out) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint64_t K = (uint64_t)nb * 256;
    int8_t* s_q = (int8_t*)smem;
    float* s_d = (float*)(smem + B * K);
    int32_t* s_sum = (int32_t*)(s_d + B * nb);

    const uint64_t nq = rows * nb;
    const uint8_t* P_ql = W;
    const uint8_t* P_qh = W + nq * 128;
    const uint8_t* P_sc = W + nq * 192;
    const uint16_t* P_d = (const uint16_t*)(W + nq * 208);

    const int lane = threadIdx.x & 63, c = lane & 7, bi = lane >> 3;
    const int qh_chunk = 2 * (c >> 2) + (c & 1);
    const uint64_t row0 = ((uint64_t)blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
    const uint32_t per_pass = 8 * IT;
    const uint32_t passes = (nb + per_pass - 1) / per_pass;

    uint4 wl[R][IT], wqh[R][IT], wsc[R][IT];
    uint32_t wd[R][IT];
    auto issue = [&](uint32_t pass) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const uint32_t blk = pass * per_pass + it * 8 + bi;
                const uint64_t row = row0 + r;
                if (row < rows && blk < nb) {
                    const uint64_t q = row * nb + blk;
                    wl[r][it] = load_stream16(P_ql + q * 128 + 16 * c);
                    wqh[r][it] = load_stream16(P_qh + q * 64 + 16 * qh_chunk);
                    wsc[r][it] = load_stream16(P_sc + q * 16);
                    wd[r][it] = __builtin_nontemporal_load(P_d + q);
                } else {
                    wl[r][it] = wqh[r][it] = wsc[r][it] = make_uint4(0, 0, 0, 0);
                    wd[r][it] = 0;
                }
            }
    };
    issue(0);
    if (!stage_q8k<B>(act, K, nb, false, s_q, s_d, s_sum)) return;

    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[r][b] = 0.0f;

    for (uint32_t pass = 0; pass < passes; ++pass) {
        if (pass) issue(pass);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const uint32_t blk = pass * per_pass + it * 8 + bi;
                if (blk >= nb) continue;
                const Q6KLane L = q6k_lane(wl[r][it], wqh[r][it], wsc[r][it], wd[r][it], c);
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    const int32_t I = q6k_ints(L, s_q + b * K + blk * 256, s_sum + (b * nb + blk) * 16, c);
                    const float d = L.dw * s_d[b * nb + blk];
                    acc[r][b] += d * (float)I;
                }
            }
    }
    unsigned long long best[B];
#pragma unroll
    for (int b = 0; b < B; ++b) best[b] = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) finish_row<B>(acc[r], row0 + r, rows, y, ldy, best);
    publish_argmax<B>(best, argmax_key_out);
}

// ---------------------------------------------------------------------------
// Q8_0 (planar device layout: qs [q][32] | d [q] f16): two lanes per block,
// 32 blocks per wave instruction, IT instructions per pass.
// ---------------------------------------------------------------------------
template <int B, int R, int IT>
__global__ __launch_bounds__(kThreads) void q8_0_matvec_kernel(const uint8_t* __restrict__ W, uint64_t rows,
                                                               uint32_t nb, ActPlanes act, float* __restrict__ y,
                                                               uint64_t ldy, unsigned long long* argmax_key_out) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint64_t K = (uint64_t)nb * 32;
    int8_t* s_q = (int8_t*)smem;
    float* s_d = (float*)(smem + ((B * K + 15) & ~(uint64_t)15));

    const uint64_t nq = rows * nb;
    const uint16_t* P_d = (const uint16_t*)(W + nq * 32);
    const int lane = threadIdx.x & 63, half = lane & 1, bi = lane >> 1;
    const uint64_t row0 = ((uint64_t)blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
    const uint32_t per_pass = 32 * IT;
    const uint32_t passes = (nb + per_pass - 1) / per_pass;

    uint4 wq[R][IT];
    uint32_t wd[R][IT];
    auto issue = [&](uint32_t pass) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const uint32_t blk = pass * per_pass + it * 32 + bi;
                const uint64_t row = row0 + r;
                if (row < rows && blk < nb) {
                    const uint64_t q = row * nb + blk;
                    wq[r][it] = load_stream16(W + q * 32 + 16 * half);
                    wd[r][it] = __builtin_nontemporal_load(P_d + q);
                } else {
                    wq[r][it] = make_uint4(0, 0, 0, 0);
                    wd[r][it] = 0;
                }
            }
    };
    issue(0);
    if (!stage_q8_0<B>(act, K, nb, s_q, s_d)) return;

    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[r][b] = 0.0f;

    for (uint32_t pass = 0; pass < passes; ++pass) {
        if (pass) issue(pass);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const uint32_t blk = pass * per_pass + it * 32 + bi;
                if (blk >= nb) continue;
                const float dx = half_to_float(wd[r][it]);
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    const int32_t I = q8_0_ints(wq[r][it], s_q + b * K + blk * 32 + 16 * half);
                    acc[r][b] += (float)I * (dx * s_d[b * nb + blk]);
                }
            }
    }
    unsigned long long best[B];
#pragma unroll
    for (int b = 0; b < B; ++b) best[b] = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) finish_row<B>(acc[r], row0 + r, rows, y, ldy, best);
    publish_argmax<B>(best, argmax_key_out);
}

// ---------------------------------------------------------------------------
// host dispatch
// ---------------------------------------------------------------------------
static size_t matvec_lds(uint32_t wtype, uint64_t B, uint64_t K) {
    if (wtype == kQ8_0) return ((B * K + 15) & ~(uint64_t)15) + B * (K / 32) * 4;
    const uint64_t nb = K / 256;
    return B * K + B * nb * 4 + B * (wtype == kQ4_K ? nb * 8 : nb * 16) * 4;
}

constexpr size_t kMaxLds = 64 * 1024;

template <int B>
static hipError_t launch_b(uint32_t wtype, const uint8_t* w, uint64_t rows, uint64_t cols, const ActPlanes& act,
                           float* y, uint64_t ldy, unsigned long long* key, hipStream_t s) {
    const size_t lds = matvec_lds(wtype, B, cols);
    if (wtype == kQ4_K) {
        constexpr int R = B == 1 ? 4 : (B <= 4 ? 2 : 1);
        const uint64_t grid = (rows + kWaves * R - 1) / (kWaves * R);
        hipLaunchKernelGGL((q4k_matvec_kernel<B, R, 2>), dim3((unsigned)grid), dim3(kThreads), lds, s, w, rows,
                           (uint32_t)(cols / 256), act, y, ldy, key);
    } else if (wtype == kQ6_K) {
        constexpr int R = B == 1 ? 2 : 1;
        const uint64_t grid = (rows + kWaves * R - 1) / (kWaves * R);
        hipLaunchKernelGGL((q6k_matvec_kernel<B, R, 2>), dim3((unsigned)grid), dim3(kThreads), lds, s, w, rows,
                           (uint32_t)(cols / 256), act, y, ldy, key);
    } else {
        constexpr int R = B == 1 ? 4 : (B <= 4 ? 2 : 1);
        const uint64_t grid = (rows + kWaves * R - 1) / (kWaves * R);
        hipLaunchKernelGGL((q8_0_matvec_kernel<B, R, 1>), dim3((unsigned)grid), dim3(kThreads), lds, s, w, rows,
                           (uint32_t)(cols / 32), act, y, ldy, key);
    }
    return hipGetLastError();
}

static ActPlanes offset_planes(const ActPlanes& a, uint32_t wtype, uint64_t cols, uint64_t b0) {
    ActPlanes o;
    const uint64_t bs = wtype == kQ8_0 ? 32 : 256;
    o.q = a.q + b0 * cols;
    o.d = a.d + b0 * (cols / bs);
    o.bsum = a.bsum ? a.bsum + b0 * (cols / 16) : nullptr;
    o.bad = a.bad + b0 * (cols / bs);
    return o;
}

hipError_t launch_matvec(uint32_t wtype, const uint8_t* w, uint64_t rows, uint64_t cols, const ActPlanes* act,
                         uint64_t batch, float* y, uint64_t ldy, unsigned long long* argmax_key, hipStream_t s) {
    // Columns are processed in groups small enough for the LDS staging.
    uint64_t b0 = 0;
    while (b0 < batch) {
        uint64_t nbat = batch - b0 < 8 ? batch - b0 : 8;
        while (nbat > 1 && matvec_lds(wtype, nbat, cols) > kMaxLds) --nbat;
        if (matvec_lds(wtype, nbat, cols) > kMaxLds) return hipErrorInvalidValue;
        const ActPlanes a = offset_planes(*act, wtype, cols, b0);
        float* yb = y + b0 * ldy;
        unsigned long long* kb = argmax_key ? argmax_key + b0 : nullptr;
        hipError_t e;
        switch (nbat) {
            case 1: e = launch_b<1>(wtype, w, rows, cols, a, yb, ldy, kb, s); break;
            case 2: e = launch_b<2>(wtype, w, rows, cols, a, yb, ldy, kb, s); break;
            case 3: e = launch_b<3>(wtype, w, rows, cols, a, yb, ldy, kb, s); break;
            case 4: e = launch_b<4>(wtype, w, rows, cols, a, yb, ldy, kb, s); break;
            case 5: e = launch_b<5>(wtype, w, rows, cols, a, yb, ldy, kb, s); break;
            case 6: e = launch_b<6>(wtype, w, rows, cols, a, yb, ldy, kb, s); break;
            case 7: e = launch_b<7>(wtype, w, rows, cols, a, yb, ldy, kb, s); break;
            default: e = launch_b<8>(wtype, w, rows, cols, a, yb, ldy, kb, s); break;
        }
        if (e != hipSuccess) return e;
        b0 += nbat;
    }
    return hipSuccess;
}

// ---------------------------------------------------------------------------
// Exact per-(row, block) integer sums against activation column 0, through
// the same lane decoders as the matvec kernels.  One wave per row, eight
// blocks (Q8_0: 32) per step.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void block_sums_kernel(uint32_t wtype, const uint8_t* __restrict__ W, uint64_t rows,
                                                        uint32_t nb, ActPlanes act, int32_t* isum, int32_t* imin) {
    const uint64_t row = blockIdx.x;
    const int lane = threadIdx.x;
    if (wtype == kQ8_0) {
        const int half = lane & 1;
        for (uint32_t base = 0; base < nb; base += 32) {
            const uint32_t blk = base + (lane >> 1);
            int32_t I = 0;
            if (blk < nb) {
                const uint4 w = *(const uint4*)(W + (row * nb + blk) * 32 + 16 * half);
                I = q8_0_ints(w, act.q + blk * 32 + 16 * half);
            }
            I += __shfl_xor(I, 1, 64);
            if (blk < nb && half == 0) {
                isum[row * nb + blk] = I;
                imin[row * nb + blk] = 0;
            }
        }
        return;
    }
    const int c = lane & 7, bi = lane >> 3;
    const uint64_t nq = rows * nb;
    for (uint32_t base = 0; base < nb; base += 8) {
        const uint32_t blk = base + bi;
        int32_t I = 0, M = 0;
        if (blk < nb) {
            const uint64_t q = row * nb + blk;
            if (wtype == kQ4_K) {
                const uint8_t* b = W + q * 144;
                const Q4KLane L = q4k_lane(*(const uint4*)b, *(const uint4*)(b + 16 + 16 * c), c);
                int32_t bs32[8];
#pragma unroll
                for (int s = 0; s < 8; ++s) bs32[s] = (int32_t)act.bsum[blk * 16 + 2 * s] + act.bsum[blk * 16 + 2 * s + 1];
                q4k_ints(L, act.q + blk * 256, bs32, c, I, M);
            } else {
                const int qh_chunk = 2 * (c >> 2) + (c & 1);
                const Q6KLane L = q6k_lane(*(const uint4*)(W + q * 128 + 16 * c),
                                           *(const uint4*)(W + nq * 128 + q * 64 + 16 * qh_chunk),
                                           *(const uint4*)(W + nq * 192 + q * 16),
                                           ((const uint16_t*)(W + nq * 208))[q], c);
                int32_t bs16[16];
#pragma unroll
                for (int s = 0; s < 16; ++s) bs16[s] = act.bsum[blk * 16 + s];
                I = q6k_ints(L, act.q + blk * 256, bs16, c);
            }
        }
        I = group8_sum(I);
        M = group8_sum(M);
        if (blk < nb && c == 0) {
            isum[row * nb + blk] = I;
            imin[row * nb + blk] = M;
        }
    }
}

hipError_t launch_block_sums(uint32_t wtype, const uint8_t* w, uint64_t rows, uint64_t cols, const ActPlanes* act,
                             int32_t* isum, int32_t* imin, hipStream_t s) {
    const uint32_t nb = (uint32_t)(cols / (wtype == kQ8_0 ? 32 : 256));
    hipLaunchKernelGGL(block_sums_kernel, dim3((unsigned)rows), dim3(64), 0, s, wtype, w, rows, nb, *act, isum, imin);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
__global__ void argmax_finish_kernel(const unsigned long long* keys, uint64_t batch, const float* y, uint64_t ldy,
                                     uint32_t* out) {
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= batch) return;
    const float y0 = y[b * ldy];
    const unsigned long long k = keys[b];
    // A NaN first logit is never replaced by the reference's strict `>` scan.
    out[b] = (y0 != y0 || k == 0) ? 0u : (uint32_t)(0xffffffffull - (k & 0xffffffffull));
}

hipError_t launch_argmax_finish(const unsigned long long* keys, uint64_t batch, const float* y, uint64_t ldy,
                                uint32_t* out, hipStream_t s) {
    hipLaunchKernelGGL(argmax_finish_kernel, dim3((unsigned)((batch + 63) / 64)), dim3(64), 0, s, keys, batch, y, ldy,
                       out);
    return hipGetLastError();
}

}  // namespace rlq
