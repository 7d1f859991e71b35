// k_gemm.hip — Y[M][N] = X[M][K] · W[N][K]ᵀ on gfx950 MFMA, the engine's
// replacement for ggml_mul_mat (sam3.cpp:3738, 3779, 3792, 3795, 3815).
//
// Quantized weights (Q4_0, Q4_1, Q8_0) meet activations that were quantized
// per 32-element block exactly as ggml's CPU path does (Q8_0 / Q8_1).  For
// each 32-element block b the kernel forms the exact integer sum
//     S_b[m][n] = Σ_{k∈b} qx[m][k]·qw[n][k]
// with one v_mfma_i32_32x32x32_i8 (K = 32 = one ggml block), the exact fp32
// block scale c_b[m][n] = dx[m][b]·dw[n][b] (both fp16, so the product is
// exact) with one v_mfma_f32_32x32x16_f16 whose only non-zero K slot holds
// the two scales, and accumulates acc += float(S_b)·c_b in fp32.  Q4_1 adds
// Σ_b m_w[n][b]·s_x[m][b] with one more fp16 MFMA per 4 blocks that
// accumulates straight into acc.  F16 weights run on fp16 MFMA against
// activations rounded to fp16; F32 weights run on fp32 MFMA.
//
// Tiling: 256 threads (4 waves as 2×2), 128×128 output tile, each wave 64×64
// = 2×2 MFMA tiles of 32×32.  K advances in stages of 128 bytes per row
// (4 quant blocks, 64 fp16 or 32 f32), double-buffered in LDS with a
// register prefetch of the next stage.  Q4 nibbles are expanded to int8 on
// the way into LDS.  Work-group ids are remapped so that consecutive tiles
// land on the same XCD (ids are dealt round-robin over 8 XCDs).
//
// Epilogues run from an fp32 copy of the tile in LDS, one 32-column chunk
// per thread, so that 32-wide quant blocks, RoPE pairs and fp16 rows are
// whole inside one thread.
#include "s3e_internal.h"

namespace s3e {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = GEMM_BN, NTHR = 256;
constexpr int ROWB = 128;                        // data bytes per tile row per stage
constexpr int LROW = 144;                        // LDS row stride in bytes
constexpr int OFF_A = 0;
constexpr int OFF_B = BM * LROW;
constexpr int OFF_AD = OFF_B + BN * LROW;        // fp16 [4][BM] activation scales
constexpr int OFF_AS = OFF_AD + 4 * BM * 2;      // fp16 [4][BM] activation sums (Q8_1)
constexpr int OFF_BD = OFF_AS + 4 * BM * 2;      // fp16 [4][BN] weight scales
constexpr int OFF_BMIN = OFF_BD + 4 * BN * 2;    // fp16 [4][BN] weight minima (Q4_1)
constexpr int STAGE = OFF_BMIN + 4 * BN * 2;
constexpr int LDS_BYTES = 2 * STAGE;
constexpr int CLD = BN + 4;                      // fp32 C-tile row stride
static_assert(BM * CLD * 4 <= LDS_BYTES, "C tile must fit in the stage buffers");

struct GemmParams {
    const uint8_t *a;
    const uint16_t *a_d, *a_s;
    int64_t a_ld_bytes, a_nblk;
    const uint8_t *b;
    const uint16_t *b_d, *b_m;
    int64_t b_ld_bytes, b_nblk;
    int M, N, K, nstages, tiles_m, tiles_n, ntiles;
    EpiArgs e;
};

__device__ __forceinline__ uint32_t q4_center(uint32_t x) {
    // bytes in [0,15] → bytes (x-8) as int8, without cross-byte borrows
    return ((x | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

__device__ __forceinline__ float gelu_erf(float x) {
    const float SQRT_2_INV = 0.70710678118654752440084436210484f;
    return 0.5f * x * (1.0f + erff(x * SQRT_2_INV));
}

__device__ __forceinline__ uint16_t f2h_bits(float v) { return half_bits(v); }

// Quantize 32 values to one Q8 block the way ggml's x86 quantize_row_q8_0 /
// q8_1 do: d = amax/127, id = 127/amax, q = round-half-even(v·id).
__device__ __forceinline__ void quant_block32(const float *v, int8_t *qdst, uint16_t *ddst,
                                              uint16_t *sdst) {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.f;
    const float id = (amax != 0.f) ? 127.f / amax : 0.f;
    int sum = 0;
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint32_t packed = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = (int)__builtin_rintf(v[4 * j + i] * id);
            sum += q;
            packed |= ((uint32_t)(q & 0xff)) << (8 * i);
        }
        w[j] = packed;
    }
    uint4 *dst = (uint4 *)qdst;
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    *ddst = f2h_bits(d);
    // s = fp16(fp32(d·Σq)): f2h_bits keeps the fp32 rounding of the product
    if (sdst) *sdst = f2h_bits(d * (float)sum);
}

template <int WK>
struct Traits {
    static constexpr bool quant = (WK == WK_Q4_0 || WK == WK_Q4_1 || WK == WK_Q8_0);
    static constexpr bool q4 = (WK == WK_Q4_0 || WK == WK_Q4_1);
    static constexpr int esize = quant ? 1 : (WK == WK_F16 ? 2 : 4);   // activation bytes/elem
    static constexpr int stage_elems = ROWB / esize;
};

template <int WK, int EPI>
__global__ __launch_bounds__(NTHR, 2) void k_gemm(GemmParams p) {
    using T = Traits<WK>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];

    // XCD-aware remap: hardware deals work-group ids round-robin over 8 XCDs;
    // give each XCD a contiguous run of tiles so they share its L2.
    const int nb = gridDim.x;
    const int per = nb >> 3;
    const int logical = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (logical >= p.ntiles) return;
    const int tm = logical / p.tiles_n, tn = logical % p.tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;

    const int t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lh = lane >> 5;

    const int kbytes = p.K * T::esize;      // valid bytes per activation row
    const int nblk_valid = p.K / QK;

    // ---- register staging for one pipeline stage ----
    uint4 ra[4];
    uint4 rb[4];
    uint16_t rad[4], ras[4];
    uint2 rbd, rbm;

    auto gload = [&](int s) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = t + NTHR * i;
            const int row = c >> 3, c16 = c & 7;
            const int kb = s * ROWB + c16 * 16;
            const bool ok = (m0 + row < p.M) && (kb < kbytes);
            ra[i] = ok ? *(const uint4 *)(p.a + (int64_t)(m0 + row) * p.a_ld_bytes + kb)
                       : make_uint4(0, 0, 0, 0);
        }
        if constexpr (T::q4) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int c = t + NTHR * i;
                const int col = c >> 2, blk = c & 3;
                rb[i] = *(const uint4 *)(p.b + (int64_t)(n0 + col) * p.b_ld_bytes +
                                         (int64_t)(s * 4 + blk) * 16);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = t + NTHR * i;
                const int col = c >> 3, c16 = c & 7;
                rb[i] = *(const uint4 *)(p.b + (int64_t)(n0 + col) * p.b_ld_bytes +
                                         (int64_t)s * ROWB + c16 * 16);
            }
        }
        if constexpr (T::quant) {
            if (t < BM) {
                const bool rok = (m0 + t < p.M);
#pragma unroll
                for (int blk = 0; blk < 4; blk++) {
                    const int kb = s * 4 + blk;
                    const bool ok = rok && kb < nblk_valid;
                    rad[blk] = ok ? p.a_d[(int64_t)(m0 + t) * p.a_nblk + kb] : (uint16_t)0;
                    if constexpr (WK == WK_Q4_1) {
                        ras[blk] = ok ? p.a_s[(int64_t)(m0 + t) * p.a_nblk + kb] : (uint16_t)0;
                    }
                }
            } else {
                const int col = t - BM;
                rbd = *(const uint2 *)(p.b_d + (int64_t)(n0 + col) * p.b_nblk + s * 4);
                if constexpr (WK == WK_Q4_1) {
                    rbm = *(const uint2 *)(p.b_m + (int64_t)(n0 + col) * p.b_nblk + s * 4);
                }
            }
        }
    };

    auto lstore = [&](int buf) {
        uint8_t *L = lds + buf * STAGE;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = t + NTHR * i;
            const int row = c >> 3, c16 = c & 7;
            *(uint4 *)(L + OFF_A + row * LROW + c16 * 16) = ra[i];
        }
        if constexpr (T::q4) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int c = t + NTHR * i;
                const int col = c >> 2, blk = c & 3;
                const uint4 w = rb[i];
                uint4 lo = make_uint4(w.x & 0x0F0F0F0Fu, w.y & 0x0F0F0F0Fu, w.z & 0x0F0F0F0Fu,
                                      w.w & 0x0F0F0F0Fu);
                uint4 hi = make_uint4((w.x >> 4) & 0x0F0F0F0Fu, (w.y >> 4) & 0x0F0F0F0Fu,
                                      (w.z >> 4) & 0x0F0F0F0Fu, (w.w >> 4) & 0x0F0F0F0Fu);
                if constexpr (WK == WK_Q4_0) {
                    lo = make_uint4(q4_center(lo.x), q4_center(lo.y), q4_center(lo.z), q4_center(lo.w));
                    hi = make_uint4(q4_center(hi.x), q4_center(hi.y), q4_center(hi.z), q4_center(hi.w));
                }
                uint8_t *dst = L + OFF_B + col * LROW + blk * 32;
                *(uint4 *)dst = lo;
                *(uint4 *)(dst + 16) = hi;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = t + NTHR * i;
                const int col = c >> 3, c16 = c & 7;
                *(uint4 *)(L + OFF_B + col * LROW + c16 * 16) = rb[i];
            }
        }
        if constexpr (T::quant) {
            if (t < BM) {
#pragma unroll
                for (int blk = 0; blk < 4; blk++) {
                    *(uint16_t *)(L + OFF_AD + (blk * BM + t) * 2) = rad[blk];
                    if constexpr (WK == WK_Q4_1) *(uint16_t *)(L + OFF_AS + (blk * BM + t) * 2) = ras[blk];
                }
            } else {
                const int col = t - BM;
                const uint16_t bd[4] = {(uint16_t)(rbd.x & 0xffff), (uint16_t)(rbd.x >> 16),
                                        (uint16_t)(rbd.y & 0xffff), (uint16_t)(rbd.y >> 16)};
#pragma unroll
                for (int blk = 0; blk < 4; blk++) *(uint16_t *)(L + OFF_BD + (blk * BN + col) * 2) = bd[blk];
                if constexpr (WK == WK_Q4_1) {
                    const uint16_t bm[4] = {(uint16_t)(rbm.x & 0xffff), (uint16_t)(rbm.x >> 16),
                                            (uint16_t)(rbm.y & 0xffff), (uint16_t)(rbm.y >> 16)};
#pragma unroll
                    for (int blk = 0; blk < 4; blk++) *(uint16_t *)(L + OFF_BMIN + (blk * BN + col) * 2) = bm[blk];
                }
            }
        }
    };

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    const int arow0 = wm * 64 + lr, brow0 = wn * 64 + lr;

    auto compute = [&](int buf) {
        const uint8_t *L = lds + buf * STAGE;
        if constexpr (T::quant) {
            const v16i zi = {};
            const v16f zf = {};
            // One block at a time keeps S and C of only the current block live
            // (4 tiles × 32 registers); unrolling over blocks spills.
#pragma unroll 1
            for (int blk = 0; blk < 4; blk++) {
                v4i av[2], bv[2];
                v8h ha[2], hb[2];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    av[i] = *(const v4i *)(L + OFF_A + (arow0 + 32 * i) * LROW + blk * 32 + lh * 16);
                    bv[i] = *(const v4i *)(L + OFF_B + (brow0 + 32 * i) * LROW + blk * 32 + lh * 16);
                    const _Float16 da = *(const _Float16 *)(L + OFF_AD + (blk * BM + arow0 + 32 * i) * 2);
                    const _Float16 db = *(const _Float16 *)(L + OFF_BD + (blk * BN + brow0 + 32 * i) * 2);
                    v8h x = {};
                    v8h y = {};
                    x[0] = lh ? (_Float16)0 : da;
                    y[0] = lh ? (_Float16)0 : db;
                    ha[i] = x;
                    hb[i] = y;
                }
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const v16i S = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[j], zi, 0, 0, 0);
                        const v16f C = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha[i], hb[j], zf, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[i][j][r] = __builtin_fmaf((float)S[r], C[r], acc[i][j][r]);
                    }
            }
            if constexpr (WK == WK_Q4_1) {
                v8h sa[2], mb[2];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    v8h x = {};
                    v8h y = {};
#pragma unroll
                    for (int blk = 0; blk < 4; blk++) {
                        const _Float16 sv = *(const _Float16 *)(L + OFF_AS + (blk * BM + arow0 + 32 * i) * 2);
                        const _Float16 mv = *(const _Float16 *)(L + OFF_BMIN + (blk * BN + brow0 + 32 * i) * 2);
                        x[blk] = lh ? (_Float16)0 : sv;
                        y[blk] = lh ? (_Float16)0 : mv;
                    }
                    sa[i] = x;
                    mb[i] = y;
                }
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sa[i], mb[j], acc[i][j], 0, 0, 0);
            }
        } else if constexpr (WK == WK_F16) {
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                v8h av[2], bv[2];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    av[i] = *(const v8h *)(L + OFF_A + (arow0 + 32 * i) * LROW + ks * 32 + lh * 16);
                    bv[i] = *(const v8h *)(L + OFF_B + (brow0 + 32 * i) * LROW + ks * 32 + lh * 16);
                }
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < 16; ks++) {
                float av[2], bv[2];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    av[i] = *(const float *)(L + OFF_A + (arow0 + 32 * i) * LROW + (ks * 2 + lh) * 4);
                    bv[i] = *(const float *)(L + OFF_B + (brow0 + 32 * i) * LROW + (ks * 2 + lh) * 4);
                }
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
            }
        }
    };

    // ---- main loop: one barrier per stage ----
    gload(0);
    lstore(0);
    __syncthreads();
    for (int s = 0; s < p.nstages; s++) {
        const int cur = s & 1;
        if (s + 1 < p.nstages) gload(s + 1);
        compute(cur);
        if (s + 1 < p.nstages) lstore(cur ^ 1);
        __syncthreads();
    }

    // ---- stage the fp32 tile in LDS ----
    float *Ct = (float *)lds;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = wm * 64 + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
                const int col = wn * 64 + 32 * j + lr;
                Ct[row * CLD + col] = acc[i][j][r];
            }
    __syncthreads();

    const EpiArgs &e = p.e;
    if constexpr (EPI == EPI_QKV) {
        const int sel = n0 / e.E;  // 0 = Q, 1 = K, 2 = V (a tile never straddles)
        const int Nw = e.window * e.window;
        const int nwx = e.grid / e.window;
        if (sel == 2) {
            // V is written transposed, [b][h][d][p]: one token row per thread so
            // that a wave's stores for one d cover consecutive positions.
            const int row = t & 127, cg = t >> 7;
            const int gm = m0 + row;
            if (gm < p.M) {
                const int py = gm / e.grid, px = gm % e.grid;
                const int b = (py / e.window) * nwx + px / e.window;
                const int pp = (py % e.window) * e.window + px % e.window;
#pragma unroll 4
                for (int c4 = 0; c4 < 16; c4++) {
                    const float4 v = *(const float4 *)(Ct + row * CLD + cg * 64 + c4 * 4);
                    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int gn = n0 + cg * 64 + c4 * 4 + i;
                        const int rem = gn - 2 * e.E;
                        const int h = rem / e.HD, d = rem % e.HD;
                        const float val = vv[i] + e.bias[gn];
                        const int64_t o = ((int64_t)(b * e.NH + h) * e.HD + d) * e.vt_ld + pp;
                        const _Float16 hv = to_half(val);
                        e.vt[o] = hv;
                        if (e.vt_lo) e.vt_lo[o] = (_Float16)(val - (float)hv);
                    }
                }
            }
        } else {
#pragma unroll
            for (int it = 0; it < 2; it++) {
                const int ch = t + NTHR * it;
                const int row = ch >> 2, cc = ch & 3;
                const int gm = m0 + row;
                if (gm >= p.M) continue;
                const int gn0 = n0 + cc * 32;
                float v[32];
#pragma unroll
                for (int j = 0; j < 32; j += 4) {
                    const float4 x = *(const float4 *)(Ct + row * CLD + cc * 32 + j);
                    v[j] = x.x + e.bias[gn0 + j];
                    v[j + 1] = x.y + e.bias[gn0 + j + 1];
                    v[j + 2] = x.z + e.bias[gn0 + j + 2];
                    v[j + 3] = x.w + e.bias[gn0 + j + 3];
                }
                const int py = gm / e.grid, px = gm % e.grid;
                const int b = (py / e.window) * nwx + px / e.window;
                const int pp = (py % e.window) * e.window + px % e.window;
                const int rem = gn0 - sel * e.E;
                const int h = rem / e.HD, d0 = rem % e.HD;
                if (e.freqs) {
                    // sam3_apply_rope: out_re = re·cos − im·sin, out_im = re·sin + im·cos,
                    // each product rounded on its own (separate ggml ops).
                    const float *f = e.freqs + ((int64_t)pp * (e.HD / 2) + d0 / 2) * 2;
#pragma unroll
                    for (int j = 0; j < 32; j += 2) {
                        const float c = f[j], s = f[j + 1];
                        const float re = v[j], im = v[j + 1];
                        const float a0 = __fmul_rn(re, c), a1 = __fmul_rn(im, s);
                        const float a2 = __fmul_rn(re, s), a3 = __fmul_rn(im, c);
                        v[j] = __fsub_rn(a0, a1);
                        v[j + 1] = __fadd_rn(a2, a3);
                    }
                }
                const int64_t o = ((int64_t)(b * e.NH + h) * Nw + pp) * e.HD + d0;
                _Float16 *lo = sel == 0 ? e.q_lo : e.k_lo;
                uint32_t w[16], wl[16];
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const _Float16 h0 = to_half(v[2 * j]), h1 = to_half(v[2 * j + 1]);
                    w[j] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                    const _Float16 l0 = (_Float16)(v[2 * j] - (float)h0);
                    const _Float16 l1 = (_Float16)(v[2 * j + 1] - (float)h1);
                    wl[j] = (uint32_t)__builtin_bit_cast(uint16_t, l0) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
                }
                uint4 *d4 = (uint4 *)((sel == 0 ? e.q : e.k) + o);
                d4[0] = make_uint4(w[0], w[1], w[2], w[3]);
                d4[1] = make_uint4(w[4], w[5], w[6], w[7]);
                d4[2] = make_uint4(w[8], w[9], w[10], w[11]);
                d4[3] = make_uint4(w[12], w[13], w[14], w[15]);
                if (lo) {
                    uint4 *l4 = (uint4 *)(lo + o);
                    l4[0] = make_uint4(wl[0], wl[1], wl[2], wl[3]);
                    l4[1] = make_uint4(wl[4], wl[5], wl[6], wl[7]);
                    l4[2] = make_uint4(wl[8], wl[9], wl[10], wl[11]);
                    l4[3] = make_uint4(wl[12], wl[13], wl[14], wl[15]);
                }
            }
        }
    } else {
#pragma unroll
        for (int it = 0; it < 2; it++) {
            const int ch = t + NTHR * it;
            const int row = ch >> 2, cc = ch & 3;
            const int gm = m0 + row;
            if (gm >= p.M) continue;
            const int gn0 = n0 + cc * 32;
            if (gn0 >= p.N) continue;
            float v[32];
#pragma unroll
            for (int j = 0; j < 32; j += 4) {
                const float4 x = *(const float4 *)(Ct + row * CLD + cc * 32 + j);
                v[j] = x.x; v[j + 1] = x.y; v[j + 2] = x.z; v[j + 3] = x.w;
            }
            const bool full = (gn0 + 32 <= p.N);
            if constexpr (EPI == EPI_F32 || EPI == EPI_RESID) {
                float *y = e.y + (int64_t)gm * e.ldy + gn0;
#pragma unroll
                for (int j = 0; j < 32; j++) {
                    if (!full && gn0 + j >= p.N) break;
                    const float bv = e.bias ? __fadd_rn(v[j], e.bias[gn0 + j]) : v[j];
                    if constexpr (EPI == EPI_RESID) y[j] = __fadd_rn(y[j], bv);
                    else y[j] = bv;
                }
            } else if constexpr (EPI == EPI_POS) {
                const int py = gm / e.grid, px = gm % e.grid;
                const float *pr = e.pos + ((int64_t)(py % e.pos_grid) * e.pos_grid + (px % e.pos_grid)) * p.N + gn0;
                float *y = e.y + (int64_t)gm * e.ldy + gn0;
#pragma unroll
                for (int j = 0; j < 32; j++) {
                    if (!full && gn0 + j >= p.N) break;
                    y[j] = __fadd_rn(v[j], pr[j]);
                }
            } else if constexpr (EPI == EPI_GELU) {
                // full 32-column block guaranteed by the launcher (N % 32 == 0)
#pragma unroll
                for (int j = 0; j < 32; j++) v[j] = gelu_erf(__fadd_rn(v[j], e.bias[gn0 + j]));
                const Act &o = e.out;
                if (o.kind == A_F16) {
                    _Float16 *dst = (_Float16 *)o.x + (int64_t)gm * o.ld + gn0;
                    uint32_t w[16];
#pragma unroll
                    for (int j = 0; j < 16; j++)
                        w[j] = (uint32_t)f2h_bits(v[2 * j]) | ((uint32_t)f2h_bits(v[2 * j + 1]) << 16);
                    uint4 *d4 = (uint4 *)dst;
                    d4[0] = make_uint4(w[0], w[1], w[2], w[3]);
                    d4[1] = make_uint4(w[4], w[5], w[6], w[7]);
                    d4[2] = make_uint4(w[8], w[9], w[10], w[11]);
                    d4[3] = make_uint4(w[12], w[13], w[14], w[15]);
                } else if (o.kind == A_F32) {
                    float *dst = (float *)o.x + (int64_t)gm * o.ld + gn0;
#pragma unroll
                    for (int j = 0; j < 32; j++) dst[j] = v[j];
                } else {
                    const int64_t blk = (int64_t)gm * (o.ld / QK) + gn0 / QK;
                    quant_block32(v, (int8_t *)o.x + (int64_t)gm * o.ld + gn0, o.d + blk,
                                  o.kind == A_Q8_1 ? o.s + blk : nullptr);
                }
            }
        }
    }
}

template <int WK, int EPI>
hipError_t launch_one(const GemmParams &p, hipStream_t st) {
    const int grid = ((p.ntiles + 7) / 8) * 8;
    hipLaunchKernelGGL((k_gemm<WK, EPI>), dim3(grid), dim3(NTHR), 0, st, p);
    return hipGetLastError();
}

template <int WK>
hipError_t dispatch_epi(Epi epi, const GemmParams &p, hipStream_t st) {
    switch (epi) {
        case EPI_F32: return launch_one<WK, EPI_F32>(p, st);
        case EPI_RESID: return launch_one<WK, EPI_RESID>(p, st);
        case EPI_POS: return launch_one<WK, EPI_POS>(p, st);
        case EPI_GELU: return launch_one<WK, EPI_GELU>(p, st);
        case EPI_QKV: return launch_one<WK, EPI_QKV>(p, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_gemm(const Weight &w, const Act &a, int64_t M, Epi epi, const EpiArgs &ea,
                       hipStream_t st) {
    if (M <= 0) return hipSuccess;
    GemmParams p{};
    const int esize = (w.kind == WK_F16) ? 2 : (w.kind == WK_F32 ? 4 : 1);
    p.a = (const uint8_t *)a.x;
    p.a_d = a.d;
    p.a_s = a.s;
    p.a_ld_bytes = a.ld * esize;
    p.a_nblk = a.ld / QK;
    p.b = (const uint8_t *)w.q;
    p.b_d = w.d;
    p.b_m = w.m;
    switch (w.kind) {
        case WK_Q4_0: case WK_Q4_1: p.b_ld_bytes = w.Kbp * 16; break;
        case WK_Q8_0: p.b_ld_bytes = w.Kp; break;
        case WK_F16: p.b_ld_bytes = w.Kp * 2; break;
        default: p.b_ld_bytes = w.Kp * 4; break;
    }
    p.b_nblk = w.Kbp;
    p.M = (int)M;
    p.N = (int)w.N;
    p.K = (int)w.K;
    p.nstages = (int)((w.K + stage_k(w.kind) - 1) / stage_k(w.kind));
    p.tiles_m = (int)((M + BM - 1) / BM);
    p.tiles_n = (int)(w.Np / BN);
    p.ntiles = p.tiles_m * p.tiles_n;
    p.e = ea;
    switch (w.kind) {
        case WK_Q4_0: return dispatch_epi<WK_Q4_0>(epi, p, st);
        case WK_Q4_1: return dispatch_epi<WK_Q4_1>(epi, p, st);
        case WK_Q8_0: return dispatch_epi<WK_Q8_0>(epi, p, st);
        case WK_F16: return dispatch_epi<WK_F16>(epi, p, st);
        case WK_F32: return dispatch_epi<WK_F32>(epi, p, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace s3e
