// k_image.hip — image preprocessing on the device: the uint8 bilinear resize
// of sam3_resize_bilinear (sam3.cpp:3441-3484) fused with the normalisation
// into the encoder's CHW f32 input, sam3_preprocess_image (sam3.cpp:3487-3514,
// (v − 0.5)/0.5) or sam2_preprocess_image (sam3.cpp:3518-3544, ImageNet mean
// and std).
//
// One thread per output pixel computes its three channels.  The resize runs
// in double precision with the reference's operation order (half-pixel
// centres clamped at 0, edge replication on the high side, weights
// (1 − w, w), round half up by truncating v + 0.5), so the resized bytes are
// the reference's bit for bit: every step is a correctly rounded IEEE
// operation on both sides and no contraction happens (-ffp-contract=off).
// The normalisation is two correctly rounded f32 operations, as on the host.
#include "s3e_internal.h"

namespace s3e {
namespace {

struct PrepImg {
    const uint8_t *hwc;
    float *chw;
    int w, h, S, norm;
};

__global__ __launch_bounds__(256) void k_preprocess(PrepImg p) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t plane = (int64_t)p.S * p.S;
    if (i >= plane) return;
    const int y = (int)(i / p.S), x = (int)(i - (int64_t)y * p.S);
    float v[3];
    if (p.w == p.S && p.h == p.S) {
        const uint8_t *q = p.hwc + i * 3;
#pragma unroll
        for (int c = 0; c < 3; c++) v[c] = (float)q[c];
    } else {
        const double sx = (double)p.w / p.S, sy = (double)p.h / p.S;
        double fy = (y + 0.5) * sy - 0.5;
        if (fy < 0.0) fy = 0.0;
        const int y0 = (int)fy, y1 = (y0 < p.h - 1) ? y0 + 1 : y0;
        const double wy = fy - y0, wy0 = 1.0 - wy;
        double fx = (x + 0.5) * sx - 0.5;
        if (fx < 0.0) fx = 0.0;
        const int x0 = (int)fx, x1 = (x0 < p.w - 1) ? x0 + 1 : x0;
        const double wx = fx - x0, wx0 = 1.0 - wx;
        const uint8_t *r0 = p.hwc + (int64_t)y0 * p.w * 3, *r1 = p.hwc + (int64_t)y1 * p.w * 3;
#pragma unroll
        for (int c = 0; c < 3; c++) {
            const double p00 = r0[x0 * 3 + c], p01 = r0[x1 * 3 + c];
            const double p10 = r1[x0 * 3 + c], p11 = r1[x1 * 3 + c];
            const double vv = wy0 * (wx0 * p00 + wx * p01) + wy * (wx0 * p10 + wx * p11);
            int iv = (int)(vv + 0.5);
            iv = iv < 0 ? 0 : (iv > 255 ? 255 : iv);
            v[c] = (float)iv;
        }
    }
    const float mean[3] = {0.485f, 0.456f, 0.406f}, stdv[3] = {0.229f, 0.224f, 0.225f};
#pragma unroll
    for (int c = 0; c < 3; c++) {
        const float u = v[c] / 255.0f;
        p.chw[c * plane + i] = p.norm == 1 ? (u - mean[c]) / stdv[c] : (u - 0.5f) / 0.5f;
    }
}

}  // namespace

hipError_t launch_preprocess(const uint8_t *hwc, int w, int h, int S, int norm, float *chw, hipStream_t st) {
    if (!hwc || !chw || w <= 0 || h <= 0 || S <= 0 || (norm != 0 && norm != 1)) return hipErrorInvalidValue;
    // byte offsets of the source stay within int for the per-row index math
    if ((int64_t)w * 3 > INT32_MAX / 2) return hipErrorInvalidValue;
    const PrepImg p{hwc, chw, w, h, S, norm};
    const int64_t n = (int64_t)S * S;
    hipLaunchKernelGGL(k_preprocess, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace s3e
