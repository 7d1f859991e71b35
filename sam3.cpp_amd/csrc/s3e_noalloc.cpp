// s3e_noalloc.cpp — s3e_mul_mat_noalloc: s3e_mul_mat for callers that cannot
// allocate device memory (code under HIP graph capture, serving loops that
// forbid hipMalloc).  The activation conversion that s3e_mul_mat allocates per
// call goes to `scratch`, one file-scope device array per GPU of a fixed
// size, held until the process ends.  Every call on a GPU shares that GPU's
// array and leaves its contents behind: calls that overlap on one GPU
// (different streams, threads or contexts) race.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "s3e_internal.h"
#include "s3e_rt.h"

using namespace s3e;

namespace {

static __device__ __align__(256) unsigned char scratch[S3E_NOALLOC_SCRATCH_BYTES];

std::mutex g_mu;
constexpr int kMaxDevices = 64;
void *g_scratch[kMaxDevices] = {};

// Zero n 16-byte words (a fill kernel rather than hipMemsetAsync, so that
// the call can be captured into a graph).
__global__ __launch_bounds__(256) void k_zero16(uint4 *__restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = make_uint4(0u, 0u, 0u, 0u);
}

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

}  // namespace

namespace s3e {

int noalloc_init(int device, void **out) {
    if (device < 0 || device >= kMaxDevices) {
        set_error("s3e_ctx_create: device %d beyond the %d this library tracks", device, kMaxDevices);
        return S3E_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error("s3e_ctx_create: scratch address on device %d: %s", device, hipGetErrorString(e));
            return S3E_ERR_HIP;
        }
        g_scratch[device] = p;
    }
    *out = g_scratch[device];
    return S3E_OK;
}

}  // namespace s3e

extern "C" int s3e_mul_mat_noalloc(s3e_ctx *ctx, const s3e_weight *w, const float *X, int64_t M, const float *bias,
                                   float *Y) try {
    if (!ctx || !w || !X || !Y) { set_error("s3e_mul_mat_noalloc: NULL argument"); return S3E_ERR_INVALID; }
    if (M < 0) { set_error("s3e_mul_mat_noalloc: negative M"); return S3E_ERR_INVALID; }
    const Weight &W = w->w;
    if (W.K % 32 != 0) {
        set_error("s3e_mul_mat_noalloc: K=%lld is not a multiple of 32", (long long)W.K);
        return S3E_ERR_UNSUPPORTED;
    }
    if (!ctx->scratch) { set_error("s3e_mul_mat_noalloc: context has no scratch"); return S3E_ERR_INVALID; }
    if (M == 0) return S3E_OK;
    const AKind ak = act_kind_for(W.kind);
    EpiArgs ea;
    ea.bias = bias;
    ea.y = Y;
    ea.ldy = W.N;
    Act a;
    a.kind = ak;
    a.ld = W.K;
    a.mp = round_up(M, ROW_PAD);
    hipError_t e = hipSetDevice(ctx->device);
    if (ak == A_F32) {  // f32 weights take the rows as they are
        a.x = (void *)X;
        if (e == hipSuccess) e = launch_gemm(W, a, M, EPI_F32, ea, ctx->stream);
    } else {
        // [values M × K][d: (Kp/128) groups × mp rows × 4 fp16][s: same, Q8_1]
        const bool q8 = ak == A_Q8_0 || ak == A_Q8_1;
        const int64_t vbytes = align256(M * W.K * (q8 ? 1 : 2));
        const int64_t pbytes = q8 ? align256(W.Kp / 128 * a.mp * 8) : 0;
        const int64_t need = vbytes + pbytes * (ak == A_Q8_1 ? 2 : 1);
        if (need > (int64_t)S3E_NOALLOC_SCRATCH_BYTES) {
            set_error("s3e_mul_mat_noalloc: %lld rows of K=%lld need %lld scratch bytes, more than the %lld available",
                      (long long)M, (long long)W.K, (long long)need, (long long)S3E_NOALLOC_SCRATCH_BYTES);
            return S3E_ERR_INVALID;
        }
        uint8_t *base = (uint8_t *)ctx->scratch;
        a.x = base;
        if (q8) {
            a.d = (uint16_t *)(base + vbytes);
            if (ak == A_Q8_1) a.s = (uint16_t *)(base + vbytes + pbytes);
            // scale planes start at zero: rows past M and blocks past K are
            // read by the last tiles and stages
            const int64_t n16 = pbytes * (ak == A_Q8_1 ? 2 : 1) / 16;
            if (e == hipSuccess) {
                hipLaunchKernelGGL(k_zero16, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, ctx->stream,
                                   (uint4 *)(base + vbytes), n16);
                e = hipGetLastError();
            }
        }
        if (e == hipSuccess) e = launch_rows_quant(ak, X, M, W.K, a, ctx->stream);
        if (e == hipSuccess) e = launch_gemm(W, a, M, EPI_F32, ea, ctx->stream);
    }
    if (e != hipSuccess) { set_error("s3e_mul_mat_noalloc: %s", hipGetErrorString(e)); return S3E_ERR_HIP; }
    return S3E_OK;
} S3E_CATCH("s3e_mul_mat_noalloc")
