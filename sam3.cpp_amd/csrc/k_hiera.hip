// k_hiera.hip — data movement of the SAM 2.x Hiera encoder around the shared
// GEMM and attention kernels (sam2_build_hiera_graph, sam3.cpp:4462-4527;
// sam2_hiera_block_forward, sam3.cpp:4295-4457; the FPN top-down path,
// sam3.cpp:4567-4590).  All activations are NHWC: token (y, x) is a row of
// channels.
#include "s3e_internal.h"

namespace s3e {
namespace {

// im2col of the patch embedding (Conv2d 3→E, k×k, stride, pad): CHW f32
// [3][S][S] → rows [OH·OW][ldk] in F32 or F16 (ggml's im2col in the kernel
// type), K ordered [c][ky][kx] as the kernel rows are; taps outside the image
// and columns K..ldk are zero.
__global__ void k_im2col_conv(const float *__restrict__ chw, int S, int k, int stride, int pad, int OW, int64_t T,
                              int64_t ldk, int kind, void *out, _Float16 *lo) {
    // 32-bit index arithmetic (the launcher keeps T·ldk below 2^31)
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint32_t)(T * ldk)) return;
    const uint32_t t = idx / (uint32_t)ldk;
    const int kk = (int)(idx - t * (uint32_t)ldk);
    float val = 0.f;
    if (kk < 3 * k * k) {
        const int c = kk / (k * k), r = kk % (k * k), ky = r / k, kx = r % k;
        const int oy = (int)(t / (uint32_t)OW), ox = (int)(t - (uint32_t)oy * OW);
        const int iy = oy * stride + ky - pad, ix = ox * stride + kx - pad;
        if (iy >= 0 && iy < S && ix >= 0 && ix < S) val = chw[(int64_t)c * S * S + (int64_t)iy * S + ix];
    }
    if (kind == A_F16 || kind == A_F16X2) {
        const _Float16 h = to_half(val);
        ((_Float16 *)out)[idx] = h;
        if (kind == A_F16X2) lo[idx] = (_Float16)(val - (float)h);  // fp16 of the exact difference
    } else {
        ((float *)out)[idx] = val;
    }
}

// Attention operands of one Hiera block from the QKV GEMM output (f32
// [H·W][3C], bias already added).  Windows of wh × ww tokens, row-major over
// nwx per row, cover the zero-padded grid; a padded position takes the QKV
// bias, as ggml_pad's zero rows do after the projection.  Q is max-pooled
// 2×2 inside each window under Q stride (sam2_maxpool_2d on the window's
// grid).  Heads are zero-padded from HD to HDp channels.  Q, K: [b·NH + h]
// [pos][HDp]; Vᵀ: [b·NH + h][HDp][ldv] with keys in vt_slot order and zeros
// for keys Nkv .. ldv − 1.  With lo planes the values are split hi + lo.
struct Prep {
    const float *qkv, *bias;
    int64_t ld;  // row stride of qkv in floats
    int H, W, C, NH, HD, HDp;
    int wh, ww, nwx, qs;
    int Nq, Nkv, ldv, NW;
    _Float16 *q, *k, *vt, *q_lo, *k_lo, *vt_lo;
};

__device__ __forceinline__ float qkv_at(const Prep &p, int b, int py, int px, int col) {
    const int wy = b / p.nwx, wx = b % p.nwx;
    const int y = wy * p.wh + py, x = wx * p.ww + px;
    if (y < p.H && x < p.W) return p.qkv[((int64_t)y * p.W + x) * p.ld + col];
    return p.bias[col];
}

__device__ __forceinline__ void put(_Float16 *hi, _Float16 *lo, int64_t i, float v) {
    const _Float16 h = to_half(v);
    hi[i] = h;
    if (lo) lo[i] = (_Float16)(v - (float)h);
}

// mode 0: Q (one thread per (b, h, query, d)); 1: K; 2: Vᵀ (keys up to ldv)
__global__ void k_hiera_prep(Prep p, int mode, int64_t total) {
    // 32-bit index arithmetic (the launcher keeps totals below 2^31)
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint32_t)total) return;
    const uint32_t r = i / (uint32_t)p.HDp;
    const int d = (int)(i - r * (uint32_t)p.HDp);
    const uint32_t npos = mode == 0 ? p.Nq : (mode == 1 ? p.Nkv : p.ldv);
    const uint32_t bh32 = r / npos;
    const int pos = (int)(r - bh32 * npos);
    const int64_t bh = bh32;
    const int b = (int)(bh32 / (uint32_t)p.NH), h = (int)(bh32 - (uint32_t)b * p.NH);
    float v = 0.f;
    if (d < p.HD && pos < (mode == 0 ? p.Nq : p.Nkv)) {
        const int col = (p.ld == 3LL * p.C ? mode * p.C : 0) + h * p.HD + d;
        if (mode == 0 && p.qs) {
            const int qw = p.ww / 2;
            const int qy = pos / qw, qx = pos % qw;
            v = fmaxf(fmaxf(qkv_at(p, b, 2 * qy, 2 * qx, col), qkv_at(p, b, 2 * qy, 2 * qx + 1, col)),
                      fmaxf(qkv_at(p, b, 2 * qy + 1, 2 * qx, col), qkv_at(p, b, 2 * qy + 1, 2 * qx + 1, col)));
        } else {
            v = qkv_at(p, b, pos / p.ww, pos % p.ww, col);
        }
    }
    if (mode == 0) put(p.q, p.q_lo, (bh * p.Nq + pos) * p.HDp + d, v);
    else if (mode == 1) put(p.k, p.k_lo, (bh * p.Nkv + pos) * p.HDp + d, v);
    else put(p.vt, p.vt_lo, (bh * p.HDp + d) * p.ldv + vt_slot(pos), v);
}

// Window positions outside the grid (ggml pads the normed input with zeros, so
// after the projection they hold the QKV bias; zeros past HD) for Q (without
// Q stride), K and Vᵀ, and the Vᵀ slots from Nkv to ldv (zeros).  Threads
// cover only those places: first (padded grid position, head, 8 channels) —
// the padded positions are the rows H..Hp−1 of the padded Hp × Wp grid, then
// columns W..Wp−1 of rows 0..H−1 — then (window·head, tail slot, 8 channels).
// 32-bit index arithmetic (the launcher keeps the counts below 2^31).
__global__ void k_hiera_pad(Prep p, int with_q, uint32_t n_pad, uint32_t n_tail) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t nch = p.HDp / 8;
    if (i < n_pad) {
        const uint32_t r = i / nch, q = r / (uint32_t)p.NH;
        const int d0 = (int)(i - r * nch) * 8, h = (int)(r - q * p.NH);
        const uint32_t Wp = (uint32_t)p.nwx * p.ww, Hp = (uint32_t)(p.NW / p.nwx) * p.wh;
        const uint32_t below = (Hp - p.H) * Wp;  // positions in the rows past the grid
        uint32_t y, x;
        if (q < below) {
            y = p.H + q / Wp;
            x = q - (y - p.H) * Wp;
        } else {
            const uint32_t q2 = q - below, wr = Wp - p.W;
            y = q2 / wr;
            x = p.W + (q2 - y * wr);
        }
        const uint32_t wy = y / p.wh, wx = x / p.ww;
        const int b = (int)(wy * p.nwx + wx);
        const int pos = (int)((y - wy * p.wh) * p.ww + (x - wx * p.ww));
        const int64_t bh = (int64_t)b * p.NH + h;
        const int64_t vrow = bh * p.HDp;
        const int64_t slot = vt_slot(pos);
        for (int d = d0; d < d0 + 8; d++) {
            const bool real = d < p.HD;
            const float bk = real ? p.bias[p.C + h * p.HD + d] : 0.f;
            put(p.k, p.k_lo, (bh * p.Nkv + pos) * p.HDp + d, bk);
            if (real) put(p.vt, p.vt_lo, (vrow + d) * p.ldv + slot, p.bias[2 * p.C + h * p.HD + d]);
            if (with_q) put(p.q, p.q_lo, (bh * p.Nkv + pos) * p.HDp + d, real ? p.bias[h * p.HD + d] : 0.f);
        }
        return;
    }
    const uint32_t j = i - n_pad;
    if (j >= n_tail) return;
    const uint32_t tails = (uint32_t)(p.ldv - p.Nkv);
    const uint32_t r = j / nch, bh = r / tails;
    const int d0 = (int)(j - r * nch) * 8;
    const int64_t slot = vt_slot(p.Nkv + (int)(r - bh * tails));
    const int64_t vrow = (int64_t)bh * p.HDp;
    for (int d = d0; d < d0 + 8; d++) {
        p.vt[(vrow + d) * p.ldv + slot] = (_Float16)0.f;
        if (p.vt_lo) p.vt_lo[(vrow + d) * p.ldv + slot] = (_Float16)0.f;
    }
}

// dst [side²][D] += nearest ×2 upsampling of src [(side/2)²][D]
// (ggml_upscale NEAREST, then ggml_add; sam3.cpp:4575-4580)
__global__ void k_upsample_add(float *__restrict__ dst, const float *__restrict__ src, int side, int D,
                               int64_t n4) {
    // 32-bit index arithmetic (the launcher keeps n4 below 2^31)
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint32_t)n4) return;
    const uint32_t d4 = D / 4;
    const uint32_t pix32 = i / d4;
    const int64_t pix = pix32;
    const int c = (int)(i - pix32 * d4) * 4;
    const int y = (int)(pix32 / (uint32_t)side), x = (int)(pix32 - (uint32_t)y * side);
    const float4 u = *(const float4 *)(src + ((int64_t)(y / 2) * (side / 2) + x / 2) * D + c);
    float4 *o = (float4 *)(dst + pix * D + c);
    const float4 a = *o;
    *o = make_float4(__fadd_rn(a.x, u.x), __fadd_rn(a.y, u.y), __fadd_rn(a.z, u.z), __fadd_rn(a.w, u.w));
}

}  // namespace

hipError_t launch_im2col_conv(const float *chw, int S, int k, int stride, int pad, int64_t ldk, AKind kind,
                              void *out, hipStream_t st, void *lo) {
    const int O = (S + 2 * pad - k) / stride + 1;
    if ((kind != A_F16 && kind != A_F32 && kind != A_F16X2) || (kind == A_F16X2 && !lo) || ldk < 3LL * k * k)
        return hipErrorInvalidValue;
    const int64_t T = (int64_t)O * O, total = T * ldk;
    if (total >= INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_im2col_conv, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, chw, S, k, stride,
                       pad, O, T, ldk, (int)kind, out, (_Float16 *)lo);
    return hipGetLastError();
}

namespace {

Prep make_prep(const HieraPrepArgs &a) {
    Prep p;
    p.qkv = a.qkv;
    p.bias = a.bias;
    p.ld = a.qkv_ld > 0 ? a.qkv_ld : 3LL * a.C;
    p.H = a.H; p.W = a.W; p.C = a.C; p.NH = a.NH; p.HD = a.HD; p.HDp = a.HDp;
    p.qs = a.q_stride;
    if (a.window > 0) {
        p.wh = p.ww = a.window;
        p.nwx = (a.W + a.window - 1) / a.window;
        p.NW = p.nwx * ((a.H + a.window - 1) / a.window);
    } else {
        p.wh = a.H;
        p.ww = a.W;
        p.nwx = 1;
        p.NW = 1;
    }
    p.Nkv = p.wh * p.ww;
    p.Nq = a.q_stride ? (p.wh / 2) * (p.ww / 2) : p.Nkv;
    p.ldv = (int)vt_ld_for(p.Nkv);
    p.q = a.q; p.k = a.k; p.vt = a.vt; p.q_lo = a.q_lo; p.k_lo = a.k_lo; p.vt_lo = a.vt_lo;
    return p;
}

}  // namespace

// With qkv_ld = C (Q rows only), the Q pass alone; with the full QKV rows,
// all three operands.
hipError_t launch_hiera_prep(const HieraPrepArgs &a, hipStream_t st) {
    const Prep p = make_prep(a);
    if (p.HD > p.HDp || p.HDp % 8 != 0 || (p.ld != 3LL * p.C && p.ld != p.C)) return hipErrorInvalidValue;
    const int64_t bh = (int64_t)p.NW * p.NH;
    const int64_t tq = bh * p.Nq * p.HDp, tk = bh * p.Nkv * p.HDp, tv = bh * p.ldv * p.HDp;
    if (tv >= INT32_MAX || tk >= INT32_MAX || tq >= INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_hiera_prep, dim3((unsigned)((tq + 255) / 256)), dim3(256), 0, st, p, 0, tq);
    if (p.ld == 3LL * p.C) {
        hipLaunchKernelGGL(k_hiera_prep, dim3((unsigned)((tk + 255) / 256)), dim3(256), 0, st, p, 1, tk);
        hipLaunchKernelGGL(k_hiera_prep, dim3((unsigned)((tv + 255) / 256)), dim3(256), 0, st, p, 2, tv);
    }
    return hipGetLastError();
}

hipError_t launch_hiera_pad(const HieraPrepArgs &a, hipStream_t st) {
    const Prep p = make_prep(a);
    if (p.HD > p.HDp || !p.k || !p.vt || !p.bias || (!a.q_stride && !p.q)) return hipErrorInvalidValue;
    const int64_t Wp = (int64_t)p.nwx * p.ww, Hp = (int64_t)(p.NW / p.nwx) * p.wh;
    if (Wp < p.W || Hp < p.H || (int64_t)(p.NW / p.nwx) * p.nwx != p.NW || p.ldv < p.Nkv) return hipErrorInvalidValue;
    const int64_t n_pad = (Hp * Wp - (int64_t)p.H * p.W) * p.NH * (p.HDp / 8);
    const int64_t n_tail = (int64_t)p.NW * p.NH * (p.ldv - p.Nkv) * (p.HDp / 8);
    // nothing to fill when the windows tile the grid and hold whole 16-key groups
    if (n_pad + n_tail == 0) return hipSuccess;
    if (n_pad + n_tail >= INT32_MAX) return hipErrorInvalidValue;
    const int64_t total = n_pad + n_tail;
    hipLaunchKernelGGL(k_hiera_pad, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, p, a.q_stride ? 0 : 1,
                       (uint32_t)n_pad, (uint32_t)n_tail);
    return hipGetLastError();
}

hipError_t launch_upsample_add(float *dst, const float *src, int side, int D, hipStream_t st) {
    if (D % 4 != 0 || side % 2 != 0) return hipErrorInvalidValue;
    const int64_t n4 = (int64_t)side * side * (D / 4);
    if (n4 >= INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_upsample_add, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, dst, src, side, D, n4);
    return hipGetLastError();
}

}  // namespace s3e
