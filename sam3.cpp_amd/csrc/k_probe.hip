// k_probe.hip — measurement kernels: the HBM streaming rate and the MFMA
// issue rate this part actually reaches, the denominators the benchmark's
// roofline fractions are read against next to the published peaks.
//
// Streaming: every thread moves 64 contiguous bytes per step (four 16-byte
// loads issued before any use), 2048 threads per CU, grid-stride over the
// buffer, so each wave keeps 4 KB in flight.  "read" folds the data into one
// word per thread (written out so the loads stay), "copy" writes it back
// to another buffer, "write" stores a constant.
//
// MFMA: each wave runs eight independent accumulator chains of one MFMA form
// with operands in registers (no memory traffic inside the loop), so the
// matrix pipe, not a dependency, sets the pace; the accumulators are folded
// into one word per wave at the end.
#include "s3e_internal.h"

namespace s3e {
namespace {

constexpr int PROBE_THREADS = 256;

__global__ __launch_bounds__(PROBE_THREADS) void k_stream(int mode, uint4 *__restrict__ dst,
                                                          const uint4 *__restrict__ src, int64_t n4,
                                                          uint32_t *__restrict__ sink) {
    const int64_t stride = (int64_t)gridDim.x * PROBE_THREADS * 4;
    uint32_t acc = 0;
    for (int64_t i = ((int64_t)blockIdx.x * PROBE_THREADS + threadIdx.x) * 4; i < n4; i += stride) {
        if (mode == 2) {
            const uint4 c = make_uint4((uint32_t)i, 1u, 2u, 3u);
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (i + j < n4) dst[i + j] = c;
            continue;
        }
        uint4 v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = i + j < n4 ? src[i + j] : make_uint4(0u, 0u, 0u, 0u);
        if (mode == 1) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (i + j < n4) dst[i + j] = v[j];
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
        }
    }
    if (mode == 0) sink[(int64_t)blockIdx.x * PROBE_THREADS + threadIdx.x] = acc;
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// kind 0: v_mfma_i32_32x32x32_i8; 1: v_mfma_f32_32x32x16_f16;
// 2: v_mfma_scale_f32_32x32x64_f8f6f4 on fp6 (E3M2) operands;
// 3: v_mfma_f32_32x32x8_f16
template <int KIND>
__global__ __launch_bounds__(PROBE_THREADS) void k_mfma(int64_t iters, uint32_t seed, uint32_t *__restrict__ sink) {
    constexpr int CH = 8;  // independent accumulator chains
    const int lane = threadIdx.x & 63;
    const uint32_t s = seed ^ (uint32_t)(lane * 0x9E3779B9u);
    uint32_t out = 0;
    if constexpr (KIND == 0) {
        v4i a, b;  // 16 int8 per lane
        for (int j = 0; j < 4; j++) { a[j] = (int)(s * (j + 1)); b[j] = (int)(s ^ (j * 0x01010101u)); }
        v16i c[CH];
        for (int k = 0; k < CH; k++)
            for (int r = 0; r < 16; r++) c[k][r] = (int)(s + k * 16 + r);  // distinct chains
        for (int64_t it = 0; it < iters; it++)
#pragma unroll
            for (int k = 0; k < CH; k++) c[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[k], 0, 0, 0);
        for (int k = 0; k < CH; k++)
            for (int r = 0; r < 16; r++) out += (uint32_t)c[k][r] * (uint32_t)(2 * k + 1);
    } else if constexpr (KIND == 1 || KIND == 3) {
        v8h a, b;
        for (int j = 0; j < 8; j++) {
            a[j] = (_Float16)((float)((s >> j) & 7) * 0.125f);
            b[j] = (_Float16)((float)((s >> (j + 3)) & 7) * 0.125f);
        }
        v16f c[CH];
        for (int k = 0; k < CH; k++)
            for (int r = 0; r < 16; r++) c[k][r] = (float)(k * 16 + r) + (float)(s & 255);  // distinct chains
        for (int64_t it = 0; it < iters; it++)
#pragma unroll
            for (int k = 0; k < CH; k++) {
                if constexpr (KIND == 1) c[k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[k], 0, 0, 0);
                else
                    c[k] = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_shufflevector(a, a, 0, 1, 2, 3),
                                                                __builtin_shufflevector(b, b, 0, 1, 2, 3), c[k], 0, 0,
                                                                0);
            }
        for (int k = 0; k < CH; k++)
            for (int r = 0; r < 16; r++) out += __builtin_bit_cast(uint32_t, c[k][r]) * (uint32_t)(2 * k + 1);
    } else {
        v8i a, b;
        for (int j = 0; j < 8; j++) { a[j] = j < 6 ? (int)(s * (j + 3)) : 0; b[j] = j < 6 ? (int)(s ^ (j << 9)) : 0; }
        v16f c[CH];
        for (int k = 0; k < CH; k++)
            for (int r = 0; r < 16; r++) c[k][r] = (float)(k * 16 + r) + (float)(s & 255);  // distinct chains
        for (int64_t it = 0; it < iters; it++)
#pragma unroll
            for (int k = 0; k < CH; k++)
                c[k] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c[k], 3, 3, 0, 127, 0, 127);
        for (int k = 0; k < CH; k++)
            for (int r = 0; r < 16; r++) out += __builtin_bit_cast(uint32_t, c[k][r]) * (uint32_t)(2 * k + 1);
    }
    // one word per wave
    for (int o = 32; o > 0; o >>= 1) out += (uint32_t)__shfl_xor((int)out, o, 64);
    if (lane == 0) sink[((int64_t)blockIdx.x * PROBE_THREADS + threadIdx.x) >> 6] = out;
}

}  // namespace

hipError_t launch_probe_stream(int mode, void *dst, const void *src, size_t bytes, uint32_t *sink, int blocks,
                               hipStream_t st) {
    if (mode < 0 || mode > 2 || bytes % 16 != 0 || blocks <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_stream, dim3((unsigned)blocks), dim3(PROBE_THREADS), 0, st, mode, (uint4 *)dst,
                       (const uint4 *)src, (int64_t)(bytes / 16), sink);
    return hipGetLastError();
}

hipError_t launch_probe_mfma(int kind, int64_t iters, int blocks, uint32_t *sink, hipStream_t st) {
    if (iters <= 0 || blocks <= 0) return hipErrorInvalidValue;
    switch (kind) {
        case 0: hipLaunchKernelGGL(k_mfma<0>, dim3((unsigned)blocks), dim3(PROBE_THREADS), 0, st, iters, 7u, sink); break;
        case 1: hipLaunchKernelGGL(k_mfma<1>, dim3((unsigned)blocks), dim3(PROBE_THREADS), 0, st, iters, 7u, sink); break;
        case 2: hipLaunchKernelGGL(k_mfma<2>, dim3((unsigned)blocks), dim3(PROBE_THREADS), 0, st, iters, 7u, sink); break;
        case 3: hipLaunchKernelGGL(k_mfma<3>, dim3((unsigned)blocks), dim3(PROBE_THREADS), 0, st, iters, 7u, sink); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace s3e
