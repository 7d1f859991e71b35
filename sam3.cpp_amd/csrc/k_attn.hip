// k_attn.hip — fused flash attention on gfx950 fp16 MFMA, the engine's
// replacement for ggml_flash_attn_ext (sam3.cpp:3774; isolated core at
// sam3.cpp:6778-6823): O = softmax(scale·QKᵀ)·V, no mask, head dim 64.
//
// Layout: Q, K are fp16 [BH][N][64]; V arrives transposed, fp16 [BH][64][ldv],
// which the QKV GEMM epilogue writes directly.  One work-group = 4 waves =
// 128 queries of one (batch, head); each wave owns 32 queries.  The scores
// are computed transposed, Sᵀ = K·Qᵀ (v_mfma_f32_32x32x16_f16, A = 32 keys ×
// 16 d from LDS, B = Qᵀ held in registers for the whole kernel), so that in
// the accumulator every lane holds 16 keys of ONE query (column = lane % 32)
// and the softmax statistics are per-lane scalars.  The output is formed
// transposed too, Oᵀ = Vᵀ·Pᵀ: the probabilities go from the Sᵀ accumulator
// registers straight into the B operand (fp16) with no data movement, and the
// keys of each K=16 MFMA step are the ones that lane already holds; the Vᵀ
// A-operand is read from LDS with the same key order.
//
// Precision.  SPLIT = false rounds Q, K, V and P to fp16 (fp32 accumulate).
// SPLIT = true carries every operand as an fp16 pair x = hi + lo (hi =
// fp16(x), lo = fp16(x − hi): 22 significant bits) and forms each product
// as hi·hi + hi·lo + lo·hi on MFMA, which reproduces fp32 attention to
// ~1e-7.  Quantized models need SPLIT: the attention output is re-quantized
// to Q8 for the projection GEMM, and an fp16-level error there flips
// rounding decisions, turning a 1e-4 difference into whole quantization
// steps.
//
// Online softmax in the exp2 domain: x = s·scale·log2(e), running max m and
// per-lane partial sum l, rescale of Oᵀ by exp2(m_old − m_new) per 64-key
// tile; the two lanes sharing a query (l, l^32) agree on m through one
// cross-half shuffle per tile and add their partial l at the end.
//
// The result leaves the kernel already in the next GEMM's activation format
// (Q8_0 / Q8_1 per 32-d block exactly as ggml quantizes a row, fp16, or
// f32), at row token(b, i) — the window un-partition of sam3.cpp:3784 folded
// into the store address.
#include "s3e_internal.h"

namespace s3e {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int AW = 4;           // waves per work-group
constexpr int QT = 32 * AW;     // queries per work-group
constexpr int KT = 64;          // keys per tile
constexpr int KROW = 72;        // LDS row stride in halves (144 B)
constexpr int TILE = KT * KROW; // halves per LDS tile

__device__ __forceinline__ uint16_t f2h_bits(float v) { return half_bits(v); }

__device__ __forceinline__ v16f mfma(const v8h &a, const v8h &b, const v16f &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <bool SPLIT>
__global__ __launch_bounds__(256, 2) void k_attn(AttnArgs a, int ldv) {
    constexpr int NP = SPLIT ? 2 : 1;  // planes: hi (and lo)
    __shared__ __attribute__((aligned(16))) _Float16 Ks[NP * TILE];
    __shared__ __attribute__((aligned(16))) _Float16 Vs[NP * TILE];

    const int bh = blockIdx.y;
    const int q0 = blockIdx.x * QT;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, lr = lane & 31, lh = lane >> 5;
    const int qi = q0 + wave * 32 + lr;
    const bool qvalid = qi < a.Nq;

    v8h qf[NP][4];
    {
        const int64_t off = ((int64_t)bh * a.Nq + (qvalid ? qi : 0)) * 64;
#pragma unroll
        for (int pl = 0; pl < NP; pl++) {
            const _Float16 *qrow = (pl == 0 ? a.q : a.q_lo) + off;
#pragma unroll
            for (int ds = 0; ds < 4; ds++) {
                v8h z = {};
                qf[pl][ds] = qvalid ? *(const v8h *)(qrow + ds * 16 + lh * 8) : z;
            }
        }
    }
    const float c = a.scale * 1.44269504088896340736f;
    float mrun = -INFINITY, lsum = 0.f;
    v16f o[2];
#pragma unroll
    for (int r = 0; r < 16; r++) { o[0][r] = 0.f; o[1][r] = 0.f; }

    const int64_t koff = (int64_t)bh * a.Nkv * 64, voff = (int64_t)bh * 64 * ldv;
    const int ntiles = (a.Nkv + KT - 1) / KT;

    uint4 rk[NP][2], rv[NP][2];
    auto gload = [&](int j) {
#pragma unroll
        for (int pl = 0; pl < NP; pl++) {
            const _Float16 *kb = (pl == 0 ? a.k : a.k_lo) + koff;
            const _Float16 *vb = (pl == 0 ? a.vt : a.vt_lo) + voff;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int cidx = t + 256 * i;
                const int row = cidx >> 3, c16 = cidx & 7;
                const int key = j * KT + row;
                rk[pl][i] = key < a.Nkv ? *(const uint4 *)(kb + (int64_t)key * 64 + c16 * 8) : make_uint4(0, 0, 0, 0);
                const int k0 = j * KT + c16 * 8;
                rv[pl][i] = k0 < ldv ? *(const uint4 *)(vb + (int64_t)row * ldv + k0) : make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int pl = 0; pl < NP; pl++)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int cidx = t + 256 * i;
                const int row = cidx >> 3, c16 = cidx & 7;
                *(uint4 *)(Ks + pl * TILE + row * KROW + c16 * 8) = rk[pl][i];
                *(uint4 *)(Vs + pl * TILE + row * KROW + c16 * 8) = rv[pl][i];
            }
    };

    gload(0);
    for (int j = 0; j < ntiles; j++) {
        __syncthreads();  // previous tile fully consumed
        lstore();
        __syncthreads();
        if (j + 1 < ntiles) gload(j + 1);

        // Sᵀ = K·Qᵀ for 64 keys × 32 queries
        v16f s[2];
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
            v16f acc = {};
#pragma unroll
            for (int ds = 0; ds < 4; ds++) {
                const int o_ = (kt * 32 + lr) * KROW + ds * 16 + lh * 8;
                const v8h kh = *(const v8h *)(Ks + o_);
                if constexpr (SPLIT) {
                    const v8h kl = *(const v8h *)(Ks + TILE + o_);
                    acc = mfma(kl, qf[0][ds], acc);
                    acc = mfma(kh, qf[1][ds], acc);
                }
                acc = mfma(kh, qf[0][ds], acc);
            }
            s[kt] = acc;
        }
        const bool tail = (j + 1) * KT > a.Nkv;
        float mloc = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float x = s[kt][r] * c;
                if (tail) {
                    const int key = j * KT + kt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                    if (key >= a.Nkv) x = -INFINITY;
                }
                s[kt][r] = x;
                mloc = fmaxf(mloc, x);
            }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        const float mnew = fmaxf(mrun, mloc);
        const float alpha = exp2f(mrun - mnew);
        mrun = mnew;
        float ps = 0.f;
        v8h pb[NP][2][2];
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int jj = 0; jj < 2; jj++)
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float pv = exp2f(s[kt][8 * jj + i] - mnew);
                    ps += pv;
                    const _Float16 ph = (_Float16)pv;
                    pb[0][kt][jj][i] = ph;
                    if constexpr (SPLIT) pb[NP - 1][kt][jj][i] = (_Float16)(pv - (float)ph);
                }
        lsum = lsum * alpha + ps;
#pragma unroll
        for (int r = 0; r < 16; r++) { o[0][r] *= alpha; o[1][r] *= alpha; }

        // Oᵀ += Vᵀ·Pᵀ
#pragma unroll
        for (int dt = 0; dt < 2; dt++)
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int jj = 0; jj < 2; jj++) {
                    const int o_ = (dt * 32 + lr) * KROW + kt * 32 + 16 * jj + 4 * lh;
                    const v4h lo = *(const v4h *)(Vs + o_);
                    const v4h hi = *(const v4h *)(Vs + o_ + 8);
                    const v8h vh = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    if constexpr (SPLIT) {
                        const v4h lo2 = *(const v4h *)(Vs + TILE + o_);
                        const v4h hi2 = *(const v4h *)(Vs + TILE + o_ + 8);
                        const v8h vl = {lo2[0], lo2[1], lo2[2], lo2[3], hi2[0], hi2[1], hi2[2], hi2[3]};
                        o[dt] = mfma(vl, pb[0][kt][jj], o[dt]);
                        o[dt] = mfma(vh, pb[NP - 1][kt][jj], o[dt]);
                    }
                    o[dt] = mfma(vh, pb[0][kt][jj], o[dt]);
                }
    }

    lsum += __shfl_xor(lsum, 32, 64);
    const float inv = (lsum == 0.f) ? 0.f : 1.0f / lsum;
#pragma unroll
    for (int r = 0; r < 16; r++) { o[0][r] *= inv; o[1][r] *= inv; }

    // output row for (batch b, query qi)
    const int b = bh / a.NH, h = bh % a.NH;
    int64_t orow;
    if (a.grid > 0) {
        const int nwx = a.grid / a.window;
        const int wy = b / nwx, wx = b % nwx;
        const int iy = (qvalid ? qi : 0) / a.window, ix = (qvalid ? qi : 0) % a.window;
        orow = (int64_t)(wy * a.window + iy) * a.grid + wx * a.window + ix;
    } else {
        orow = (int64_t)b * a.Nq + qi;
    }
    const Act &out = a.out;
    const int64_t colbase = (int64_t)h * 64;
#pragma unroll
    for (int dt = 0; dt < 2; dt++) {
        if (out.kind == A_Q8_0 || out.kind == A_Q8_1) {
            // ggml quantize_row_q8_0/q8_1 of the 32 values d = dt*32 .. dt*32+31,
            // split 16/16 between lanes l and l^32
            float amax = 0.f;
#pragma unroll
            for (int r = 0; r < 16; r++) amax = fmaxf(amax, fabsf(o[dt][r]));
            amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
            const float d = amax / 127.f;
            const float id = (amax != 0.f) ? 127.f / amax : 0.f;
            int sum = 0;
            uint32_t w[4];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                uint32_t packed = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int q = (int)__builtin_rintf(o[dt][4 * g + i] * id);
                    sum += q;
                    packed |= ((uint32_t)(q & 0xff)) << (8 * i);
                }
                w[g] = packed;
            }
            sum += __shfl_xor(sum, 32, 64);
            if (qvalid) {
                int8_t *dst = (int8_t *)out.x + orow * out.ld + colbase + dt * 32 + 4 * lh;
#pragma unroll
                for (int g = 0; g < 4; g++) *(uint32_t *)(dst + 8 * g) = w[g];
                if (lh == 0) {
                    const int64_t blk = scale_index(out.mp, orow, (colbase + dt * 32) / QK);
                    out.d[blk] = f2h_bits(d);
                    if (out.kind == A_Q8_1) out.s[blk] = f2h_bits(d * (float)sum);
                }
            }
        } else if (qvalid) {
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int64_t col = colbase + dt * 32 + 8 * g + 4 * lh;
                if (out.kind == A_F32) {
                    *(float4 *)((float *)out.x + orow * out.ld + col) =
                        make_float4(o[dt][4 * g], o[dt][4 * g + 1], o[dt][4 * g + 2], o[dt][4 * g + 3]);
                } else {
                    const uint32_t w0 = (uint32_t)f2h_bits(o[dt][4 * g]) | ((uint32_t)f2h_bits(o[dt][4 * g + 1]) << 16);
                    const uint32_t w1 = (uint32_t)f2h_bits(o[dt][4 * g + 2]) | ((uint32_t)f2h_bits(o[dt][4 * g + 3]) << 16);
                    *(uint2 *)((_Float16 *)out.x + orow * out.ld + col) = make_uint2(w0, w1);
                }
            }
        }
    }
}

}  // namespace

hipError_t launch_attn(const AttnArgs &a, hipStream_t st) {
    // V rows are read 8 keys at a time: their stride is Nkv rounded up to 8
    // (the producers pad with zeros).
    const int ldv = (a.Nkv + 7) / 8 * 8;
    const dim3 grid((unsigned)((a.Nq + QT - 1) / QT), (unsigned)a.BH);
    if (a.q_lo) hipLaunchKernelGGL(k_attn<true>, grid, dim3(256), 0, st, a, ldv);
    else hipLaunchKernelGGL(k_attn<false>, grid, dim3(256), 0, st, a, ldv);
    return hipGetLastError();
}

}  // namespace s3e
