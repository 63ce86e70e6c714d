// probe.hip - measurement probes, the practical ceilings reported next to the
// MI355X spec peaks (bench.py practical_peaks):
//  - rlq_probe_mfma: chained MFMAs from registers, no memory traffic:
//    v_mfma_i32_32x32x32_i8 (the int8 peak the prefill target is quoted on)
//    and v_mfma_f32_32x32x16_f16 (the instruction the prefill GEMM issues);
//    LDS reads alone in the prefill GEMM's A-operand pattern (four 1 KB
//    ds_read_b128 per step); and the GEMM's inner ratio, four such reads
//    feeding four f16 MFMAs; and whether MFMAs of one wave and FMAs of
//    another overlap on one SIMD, with the MFMA accumulators in VGPRs or in
//    AGPRs;
//  - rlq_probe_stream: a plain read of a buffer with the one-column matvec's
//    launch shape (one workgroup of 16 waves per CU) and load pattern (each
//    wave instruction a 1 KB run of 16-byte non-temporal loads), XORed and
//    never written back: the time a pass over the matvec's bytes takes with
//    no arithmetic; rlq_probe_stream_shape the same read with other
//    workgroup sizes, runs in flight per wave and load kinds.
#include "rlq_device.hpp"
#include "rlq.h"
#include "rlq_internal.hpp"

namespace rlq {

typedef int32_t p_i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t p_i32x16 __attribute__((ext_vector_type(16)));
typedef float p_f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 p_f16x8 __attribute__((ext_vector_type(8)));

// Four independent accumulator chains per wave, `iters` MFMAs each; every
// wave stores one word of its accumulators so nothing is left dead.
template <int KIND>
__global__ __launch_bounds__(256) void mfma_probe_kernel(uint32_t iters, uint32_t* out) {
    const uint32_t lane = threadIdx.x & 63, gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    if constexpr (KIND == 0) {
        const p_i32x4 a = {(int)(lane * 0x01010101u), 3, 5, 7}, b = {11, (int)lane, 13, 17};
        p_i32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (uint32_t i = 0; i < iters; ++i) {
            c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, b, c3, 0, 0, 0);
        }
        if (lane == 0) out[gw] = (uint32_t)(c0[0] ^ c1[1] ^ c2[2] ^ c3[3]);
    } else if constexpr (KIND == 1) {
        p_f16x8 a, b;
#pragma unroll
        for (int k = 0; k < 8; ++k) a[k] = (_Float16)(lane + k), b[k] = (_Float16)(k - 3);
        p_f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (uint32_t i = 0; i < iters; ++i) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, b, c3, 0, 0, 0);
        }
        if (lane == 0) out[gw] = __float_as_uint(c0[0] + c1[1] + c2[2] + c3[3]);
    } else {
        // the prefill GEMM's A reads: per step four 16-byte reads per lane at
        // 512-byte strides, a different 4 KB quarter of a 20 KB region per step
        __shared__ __align__(16) uint8_t sm[20480];
        for (uint32_t i = threadIdx.x; i < 20480 / 16; i += 256) ((uint4*)sm)[i] = make_uint4(i, 3 * i, 5 * i, 7 * i);
        __syncthreads();
        uint4 x = make_uint4(0, 0, 0, 0);
        p_f16x8 b;
#pragma unroll
        for (int k = 0; k < 8; ++k) b[k] = (_Float16)(k - 3);
        p_f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (uint32_t i = 0; i < iters; ++i) {
            asm volatile("" ::: "memory");  // every step reads LDS again
            const uint8_t* base = sm + (i & 3) * 4096 + lane * 16;
            if constexpr (KIND == 2) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint4 v = *(const uint4*)(base + t * 512);
                    x.x ^= v.x, x.y ^= v.y, x.z ^= v.z, x.w ^= v.w;
                }
            } else {
                const p_f16x8 a0 = *(const p_f16x8*)base, a1 = *(const p_f16x8*)(base + 512);
                const p_f16x8 a2 = *(const p_f16x8*)(base + 1024), a3 = *(const p_f16x8*)(base + 1536);
                c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b, c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b, c1, 0, 0, 0);
                c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2, b, c2, 0, 0, 0);
                c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a3, b, c3, 0, 0, 0);
            }
        }
        if (lane == 0) out[gw] = (x.x ^ x.y ^ x.z ^ x.w) + __float_as_uint(c0[0] + c1[1] + c2[2] + c3[3]);
    }
}

// MFMA and VALU work of different waves on one SIMD: 8 waves per workgroup
// (two per SIMD), waves 0-3 running four f16 MFMA chains of `iters` steps,
// waves 4-7 eight f32 FMA chains of 2 * iters steps.  MFMA_HALF / VALU_HALF
// select the halves that run (the other exits); AG keeps the MFMA
// accumulators in AGPRs (an inline-asm operand that needs one makes the
// compiler pick the AGPR form of the MFMAs), else they are VGPRs.
template <bool MFMA_HALF, bool VALU_HALF, bool AG>
__global__ __launch_bounds__(512) void coexec_probe_kernel(uint32_t iters, uint32_t* out) {
    if constexpr (AG) {
        float z = 0.0f;
        asm volatile("; %0" : "+a"(z));
    }
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, gw = blockIdx.x * 8 + wave;
    float r = 0.0f;
    if (wave < 4) {
        if (!MFMA_HALF) return;
        p_f16x8 a, b;
#pragma unroll
        for (int k = 0; k < 8; ++k) a[k] = (_Float16)(lane + k), b[k] = (_Float16)(k - 3);
        p_f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (uint32_t i = 0; i < iters; ++i) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, b, c3, 0, 0, 0);
        }
        r = c0[0] + c1[1] + c2[2] + c3[3];
    } else {
        if (!VALU_HALF) return;
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = (float)(lane + k);
        const float m = 1.0000001f, o = 0.5f * (float)lane;
        for (uint32_t i = 0; i < 2 * iters; ++i) {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = __builtin_fmaf(v[k], m, o);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) r += v[k];
    }
    if (lane == 0) out[gw] = __float_as_uint(r);
}

// Workgroup g of `grid` (W waves) reads its equal share of the n16 16-byte
// units in 1 KB runs: wave w takes runs w, w + W, ... of the share, R of them
// in flight (NT: non-temporal loads), XORed and never written back.
template <int W, int R, bool NT>
__global__ __launch_bounds__(W * 64) void stream_probe_kernel(const uint8_t* p, uint64_t n16, uint32_t* out) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t runs = n16 / 64, per = (runs + gridDim.x - 1) / gridDim.x;
    const uint64_t r0 = (uint64_t)blockIdx.x * per, r1 = r0 + per < runs ? r0 + per : runs;
    uint32_t x = 0;
    uint64_t r = r0 + wave;
    for (; r + (uint64_t)(R - 1) * W < r1; r += (uint64_t)R * W) {  // the R runs all below r1
        uint4 v[R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const uint8_t* q = p + ((r + (uint64_t)k * W) * 64 + lane) * 16;
            v[k] = NT ? load_stream16(q) : *(const uint4*)q;
        }
        __builtin_amdgcn_sched_barrier(0);  // all R loads issued before the first use
#pragma unroll
        for (int k = 0; k < R; ++k) x ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    for (; r < r1; r += W) {
        const uint8_t* q = p + (r * 64 + lane) * 16;
        const uint4 v = NT ? load_stream16(q) : *(const uint4*)q;
        x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    x ^= (uint32_t)__shfl_xor((int)x, 32, 64);
    if (lane == 0) out[blockIdx.x * W + wave] = x;
}

template <int W, int R, bool NT>
static void launch_stream(const void* bytes, uint64_t len, uint32_t workgroups, uint32_t* out, hipStream_t s) {
    hipLaunchKernelGGL((stream_probe_kernel<W, R, NT>), dim3(workgroups), dim3(W * 64), 0, s, (const uint8_t*)bytes,
                       len / 16, out);
}
template <int W, bool NT>
static bool launch_stream_runs(uint32_t runs, const void* bytes, uint64_t len, uint32_t workgroups, uint32_t* out,
                               hipStream_t s) {
    switch (runs) {
        case 1: launch_stream<W, 1, NT>(bytes, len, workgroups, out, s); return true;
        case 2: launch_stream<W, 2, NT>(bytes, len, workgroups, out, s); return true;
        case 4: launch_stream<W, 4, NT>(bytes, len, workgroups, out, s); return true;
        case 8: launch_stream<W, 8, NT>(bytes, len, workgroups, out, s); return true;
        default: return false;
    }
}

}  // namespace rlq

using namespace rlq;

extern "C" int32_t rlq_probe_mfma(uint32_t kind, uint32_t workgroups, uint32_t iters, uint32_t* out, void* stream) {
    if (kind > 8 || workgroups == 0 || !out) return RLQ_INVALID_ARGUMENT;
    const hipStream_t s = (hipStream_t)stream;
    const dim3 g(workgroups), b4(256), b8(512);
    switch (kind) {
        case 0: hipLaunchKernelGGL(mfma_probe_kernel<0>, g, b4, 0, s, iters, out); break;
        case 1: hipLaunchKernelGGL(mfma_probe_kernel<1>, g, b4, 0, s, iters, out); break;
        case 2: hipLaunchKernelGGL(mfma_probe_kernel<2>, g, b4, 0, s, iters, out); break;
        case 3: hipLaunchKernelGGL(mfma_probe_kernel<3>, g, b4, 0, s, iters, out); break;
        case 4: hipLaunchKernelGGL((coexec_probe_kernel<true, false, false>), g, b8, 0, s, iters, out); break;
        case 5: hipLaunchKernelGGL((coexec_probe_kernel<false, true, false>), g, b8, 0, s, iters, out); break;
        case 6: hipLaunchKernelGGL((coexec_probe_kernel<true, true, false>), g, b8, 0, s, iters, out); break;
        case 7: hipLaunchKernelGGL((coexec_probe_kernel<true, false, true>), g, b8, 0, s, iters, out); break;
        default: hipLaunchKernelGGL((coexec_probe_kernel<true, true, true>), g, b8, 0, s, iters, out); break;
    }
    return hipGetLastError() == hipSuccess ? RLQ_OK : RLQ_DEVICE_ERROR;
}

extern "C" int32_t rlq_probe_stream_shape(const void* bytes, uint64_t len, uint32_t workgroups, uint32_t waves,
                                          uint32_t runs, uint32_t non_temporal, uint32_t* out, void* stream) {
    if (!bytes || !out || workgroups == 0 || len % 1024 != 0 || ((uintptr_t)bytes & 15)) return RLQ_INVALID_ARGUMENT;
    if (waves != 4 && waves != 8 && waves != 16) return RLQ_INVALID_ARGUMENT;
    const hipStream_t s = (hipStream_t)stream;
    bool ok;
    switch (waves * 2 + (non_temporal ? 1 : 0)) {
        case 8: ok = launch_stream_runs<4, false>(runs, bytes, len, workgroups, out, s); break;
        case 9: ok = launch_stream_runs<4, true>(runs, bytes, len, workgroups, out, s); break;
        case 16: ok = launch_stream_runs<8, false>(runs, bytes, len, workgroups, out, s); break;
        case 17: ok = launch_stream_runs<8, true>(runs, bytes, len, workgroups, out, s); break;
        case 32: ok = launch_stream_runs<16, false>(runs, bytes, len, workgroups, out, s); break;
        case 33: ok = launch_stream_runs<16, true>(runs, bytes, len, workgroups, out, s); break;
        default: ok = false;
    }
    if (!ok) return RLQ_INVALID_ARGUMENT;
    return hipGetLastError() == hipSuccess ? RLQ_OK : RLQ_DEVICE_ERROR;
}

extern "C" int32_t rlq_probe_stream(const void* bytes, uint64_t len, uint32_t workgroups, uint32_t* out,
                                    void* stream) {
    return rlq_probe_stream_shape(bytes, len, workgroups, 16, 2, 1, out, stream);
}
