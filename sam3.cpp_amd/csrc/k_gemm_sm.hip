// k_gemm_sm.hip — small-M products Y[M][N] = X[M][K] · W[N][K]ᵀ for M ≤ 64
// (ggml_mul_mat at a few rows: the weight-streaming regime), one or many
// independent products per launch.
//
// At 64 rows each weight byte feeds at most 64 multiply-adds, so the product
// is bound by streaming the weights from HBM, not by MFMA.  The kernel
// therefore reads the weights once, at their ggml size (Q4 as nibbles, 18 or
// 20 bytes per 32 weights with the scales), from a block-interleaved copy
// made on the device at first use:
//     block b of column n at  (b·Np + n)·BB   (BB = 16 / 32 / 64 bytes for
//                                              Q4_* nibbles / Q8_0 / F16)
// so that the 32 columns of a wave read 32 consecutive chunks of a block.
// Nibble j of a Q4 chunk is ggml's: byte j holds element j (low) and
// element j + 16 (high).  Scales stay in the engine's stage-major planes.
//
// Work: a wave owns a strip of 32 columns and a range of the K stages (4
// blocks each).  A work-group's 4 waves cover 4/KS adjacent strips × KS
// K ranges (KS = 4 is built: four waves share one strip's K range, which
// keeps each wave's dependent chain short; a whole strip per wave measured
// no faster and needs more registers); split partial sums are added in LDS
// in a fixed order (deterministic).  A lone product with few strips (N =
// 1024: 32 work-groups for 256 CUs) also splits K across kg work-groups per
// strip: each writes its sum to a workspace and a second pass adds the kg
// sums in index order.  The next stage is loaded while one is
// consumed.  Per 32-element block and 32-row tile
// the arithmetic is the large-M kernel's: the exact integer block sum on
// v_mfma_i32_32x32x32_i8 (Q4_0 nibbles n become the signed codes n − 8 four
// bytes at a time: (n + 0x78) ^ 0x80 per byte, no carry between bytes), the
// exact scale product 2·dx·dw on a one-hot v_mfma_f32_32x32x16_f16, and
// acc += float(S)·c on the VALU; Q4_1 adds Σ m_w·s_x per stage on fp16 MFMA.
// F16 weights run on v_mfma_f32_32x32x16_f16 directly.
#include "s3e_internal.h"

namespace s3e {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int SM_WAVES = 4;

template <int WK>
struct SmCfg {
    static constexpr bool quant = WK != WK_F16;
    static constexpr bool q4 = WK == WK_Q4_0 || WK == WK_Q4_1;
    static constexpr bool q41 = WK == WK_Q4_1;
    static constexpr int BB = q4 ? 16 : (WK == WK_Q8_0 ? 32 : 64);  // bytes per column per block
    static constexpr int WL = WK == WK_F16 ? 8 : 4;                  // 16-byte weight loads per stage per lane
};

// Operands of one stage (4 blocks) for MT row tiles.
template <int WK, int MT>
struct SmStage {
    uint4 w[SmCfg<WK>::WL];
    uint2 wd, wm;
    uint4 a[MT][SmCfg<WK>::WL];
    uint2 ad[MT], as[MT];
};

template <int WK, int MT, int KS>
__global__ __launch_bounds__(64 * SM_WAVES, 2) void k_gemm_sm(SmArgs p) {
    using C = SmCfg<WK>;
    constexpr int SPW = SM_WAVES / KS;  // strips per work-group
    __shared__ float red[KS > 1 ? SM_WAVES : 1][MT * 32][33];

    const int wg = blockIdx.x;
    const SmGemm G = p.many ? p.many[p.wg_gemm[wg]] : p.one;
    const int t = threadIdx.x, lane = t & 63, lr = lane & 31, lh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int ls = wave / KS, kr = wave % KS;
    // kg work-groups share a column group, each over its own K range, and
    // with p.rt = 2 each 32-row tile has work-groups of its own (MT = 1)
    const int kgi = (wg - G.wg0) % p.kg, wr = (wg - G.wg0) / p.kg;
    const int r0 = (wr % p.rt) * 32, cg = wr / p.rt;
    const int n0 = (cg * SPW + ls) * 32;
    const int n = n0 + lr;  // < Np: weights are padded to whole 128-column groups
    const bool live = n0 < G.N;
    const int ka = G.nst * kgi / p.kg, kn = G.nst * (kgi + 1) / p.kg - ka;
    const int s0 = ka + kn * kr / KS, s1 = live ? ka + kn * (kr + 1) / KS : s0;
    const int M = p.M;

    int rows[MT];
#pragma unroll
    for (int i = 0; i < MT; i++) rows[i] = min(r0 + 32 * i + lr, M - 1);

    auto load = [&](int s, SmStage<WK, MT> &f) {
        const int b0 = 4 * s;
#pragma unroll
        for (int j = 0; j < C::WL; j++) {
            // Q4: block j (both lane halves read the same 16 bytes); Q8_0: block j,
            // half lh; F16: block j / 2, slab j % 2, half lh
            const int blk = C::q4 ? b0 + j : (WK == WK_Q8_0 ? b0 + j : b0 + j / 2);
            const int sub = C::q4 ? 0 : (WK == WK_Q8_0 ? lh : 2 * (j & 1) + lh);
            f.w[j] = *(const uint4 *)(G.w + ((int64_t)blk * G.np + n) * C::BB + sub * 16);
        }
        if constexpr (C::quant) {
            f.wd = *(const uint2 *)(G.wd + ((int64_t)s * G.np + n) * 4);
            if constexpr (C::q41) f.wm = *(const uint2 *)(G.wm + ((int64_t)s * G.np + n) * 4);
        }
#pragma unroll
        for (int i = 0; i < MT; i++) {
            if constexpr (C::quant) {
                const int8_t *xr = (const int8_t *)G.x + (int64_t)rows[i] * G.ldx;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int k = min((b0 + j) * 32 + lh * 16, G.K - 16);
                    f.a[i][j] = *(const uint4 *)(xr + k);
                }
                f.ad[i] = *(const uint2 *)(G.xd + ((int64_t)s * G.xmp + rows[i]) * 4);
                if constexpr (C::q41) f.as[i] = *(const uint2 *)(G.xs + ((int64_t)s * G.xmp + rows[i]) * 4);
            } else {
                const _Float16 *xr = (const _Float16 *)G.x + (int64_t)rows[i] * G.ldx;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int k = min((b0 + j / 2) * 32 + (j & 1) * 16 + lh * 8, G.K - 8);
                    f.a[i][j] = *(const uint4 *)(xr + k);
                }
            }
        }
    };

    v16f acc[MT];  // Q4_1: the minimum term accumulates here too
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][r] = 0.f;

    auto compute = [&](const SmStage<WK, MT> &f) {
        if constexpr (C::quant) {
            const v16i zi = {};
            const v16f zf = {};
            const uint32_t wdw[2] = {f.wd.x, f.wd.y};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v4i b;
                if constexpr (C::q4) {
                    const int sh = 4 * lh;  // low nibbles: elements 0..15, high: 16..31
                    b[0] = (int)((f.w[j].x >> sh) & 0x0F0F0F0Fu);
                    b[1] = (int)((f.w[j].y >> sh) & 0x0F0F0F0Fu);
                    b[2] = (int)((f.w[j].z >> sh) & 0x0F0F0F0Fu);
                    b[3] = (int)((f.w[j].w >> sh) & 0x0F0F0F0Fu);
                    if constexpr (WK == WK_Q4_0)
#pragma unroll
                        for (int e = 0; e < 4; e++) b[e] = (int)(((uint32_t)b[e] + 0x78787878u) ^ 0x80808080u);
                } else {
                    b = __builtin_bit_cast(v4i, f.w[j]);
                }
                const uint32_t hw = (wdw[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
                const v4u hb = {hw, 0u, 0u, 0u};
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    const v4i a = __builtin_bit_cast(v4i, f.a[i][j]);
                    v16i S = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, zi, 0, 0, 0);
                    const uint32_t adw[2] = {f.ad[i].x, f.ad[i].y};
                    const uint32_t ha_ = (adw[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
                    const v4u ha = {ha_, 0u, 0u, 0u};
                    const v16f Cs = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, ha),
                                                                          __builtin_bit_cast(v8h, hb), zf, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[i][r] = __builtin_fmaf((float)S[r], Cs[r], acc[i][r]);
                }
            }
            if constexpr (C::q41) {
                const v4u hb = {f.wm.x, f.wm.y, 0u, 0u};
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    const v4u ha = {f.as[i].x, f.as[i].y, 0u, 0u};
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, ha),
                                                                    __builtin_bit_cast(v8h, hb), acc[i], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const v8h b = __builtin_bit_cast(v8h, f.w[j]);
#pragma unroll
                for (int i = 0; i < MT; i++)
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, f.a[i][j]), b, acc[i], 0,
                                                                    0, 0);
            }
        }
    };

    // stage s + 1 is in flight while stage s is consumed
    if (s0 < s1) {
        SmStage<WK, MT> cur, nxt;
        load(s0, cur);
        for (int s = s0; s < s1; s++) {
            const bool more = s + 1 < s1;
            if (more) load(s + 1, nxt);
            compute(cur);
            if (more) cur = nxt;
        }
    }

    constexpr float kScale = C::quant ? 0.5f : 1.0f;  // the scale products are doubled
    if constexpr (KS == 1) {
        if (!live) return;
        const int gn = n0 + lr;
        const float bv = (G.bias && gn < G.N) ? G.bias[gn] : 0.f;
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = r0 + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (row < M && gn < G.N) G.y[(int64_t)row * G.ldy + gn] = acc[i][r] * kScale + bv;
            }
    } else {
        // partial sums of the KS K ranges of each strip → LDS → fixed-order sum
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                red[wave][32 * i + 8 * (r >> 2) + 4 * lh + (r & 3)][lr] = acc[i][r];
        __syncthreads();
        if (p.kg == 1) {
            for (int o = t; o < SPW * MT * 32 * 32; o += 64 * SM_WAVES) {
                const int st = o / (MT * 32 * 32), row = (o >> 5) % (MT * 32), col = o & 31;
                const int gn = (cg * SPW + st) * 32 + col;
                if (r0 + row >= M || gn >= G.N) continue;
                float v = red[st * KS][row][col];
#pragma unroll
                for (int w = 1; w < KS; w++) v += red[st * KS + w][row][col];
                v *= kScale;
                if (G.bias) v += G.bias[gn];
                G.y[(int64_t)(r0 + row) * G.ldy + gn] = v;
            }
            return;
        }
        // split over work-groups: each writes its K range's sum to part
        // [kg][M][N] and k_sm_reduce adds the kg sums in index order
        for (int o = t; o < SPW * MT * 32 * 32; o += 64 * SM_WAVES) {
            const int st = o / (MT * 32 * 32), row = (o >> 5) % (MT * 32), col = o & 31;
            const int gn = (cg * SPW + st) * 32 + col;
            if (r0 + row >= M || gn >= G.N) continue;
            float v = red[st * KS][row][col];
#pragma unroll
            for (int w = 1; w < KS; w++) v += red[st * KS + w][row][col];
            p.part[((int64_t)kgi * M + r0 + row) * G.N + gn] = v;
        }
    }
}

// Y = scale · Σ_k part[k] + bias over the kg ≤ SM_KG_MAX partial sums of a
// split small-M product, added in index order (one thread per output; the kg
// loads are all issued before the first add).
__global__ __launch_bounds__(256) void k_sm_reduce(const float *__restrict__ part, int kg, int64_t mn, int N,
                                                  float scale, const float *__restrict__ bias, float *__restrict__ y,
                                                  int64_t ldy) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= mn) return;
    float pv[SM_KG_MAX];
#pragma unroll
    for (int k = 0; k < SM_KG_MAX; k++) pv[k] = k < kg ? part[k * mn + i] : 0.f;
    float v = 0.f;
#pragma unroll
    for (int k = 0; k < SM_KG_MAX; k++) v += pv[k];  // + 0 past kg leaves v unchanged
    const int64_t row = i / N;
    const int col = (int)(i - row * N);
    v *= scale;
    if (bias) v += bias[col];
    y[row * ldy + col] = v;
}

#define LDS_PTR(p) ((__attribute__((address_space(3))) void *)(p))

// Batched variant: a work-group owns 4 adjacent strips (128 columns), one
// per wave, over the whole K range, so the activation stage (the same for
// the four waves) is staged once in LDS by direct-to-LDS loads (rows of 128
// bytes, 256 for F16, 16-byte chunks XOR-swizzled by row).  Quantized weights
// and their scales go to LDS the same way, each wave its own strip's, so that
// AHEAD stages are in flight while one is consumed with no registers held
// for them; F16 weights (8 KB per wave and stage) stream into registers one
// stage ahead instead.  One barrier per stage releases the buffers the stage
// before read.
template <int WK, int MT>
struct SmbCfg {
    static constexpr bool quant = WK != WK_F16;
    static constexpr bool q41 = WK == WK_Q4_1;
    static constexpr int ROWB = quant ? 128 : 256;
    static constexpr int A_BYTES = MT * 32 * ROWB;
    static constexpr int SC_BYTES = quant ? MT * 32 * 8 : 0;               // 4 block scales per row
    static constexpr int SS_BYTES = q41 ? MT * 32 * 8 : 0;                  // 4 block sums per row
    static constexpr int NA = A_BYTES / 4096;                               // 1 KB DMA runs per wave
    // quantized weights in LDS: per wave [4 blocks][32 columns][BB bytes],
    // then the columns' 4 scales (and Q4_1 minima), 8 bytes each
    static constexpr int BB = SmCfg<WK>::BB;
    static constexpr int WW = quant ? 128 * BB : 0;
    static constexpr int NWI = WW / 1024;                                   // 1 KB DMA runs per wave
    static constexpr int W_OFF = A_BYTES + SC_BYTES + SS_BYTES;
    static constexpr int WD_OFF = W_OFF + SM_WAVES * WW;
    static constexpr int WM_OFF = WD_OFF + (quant ? SM_WAVES * 256 : 0);
    static constexpr int STAGE = WM_OFF + (q41 ? SM_WAVES * 256 : 0);
    // two buffers: stage s + 1 lands while stage s is consumed.  The
    // products are bound by overlapping one wave's MFMA with another's VALU,
    // so small buffers that let three work-groups share a CU (Q4_0 at 64
    // rows: 36 KB, 145 VGPRs) beat deeper rings (4 buffers: 2.37 TB/s
    // against 2.77 over a 256-product sweep)
    static constexpr int NBUF = 2;
    static constexpr int AHEAD = NBUF - 1;                                  // stages issued ahead
    // vector memory instructions a lane issues per stage (quantized path)
    static constexpr int LOADS = NA + NWI + (quant ? 2 : 0) + (q41 ? 2 : 0);
};

template <int R>
__device__ __forceinline__ int smb_swz(int r) { return R == 128 ? ((r >> 1) & 7) : (r & 15); }

template <int LOADS, int AHEAD>
__device__ __forceinline__ void smb_wait(int ahead) {
    // stage s has landed when at most `ahead` later stages' loads are outstanding
    static_assert(AHEAD >= 1 && AHEAD <= 3, "deeper rings need more cases");
    if (AHEAD >= 3 && ahead >= 2) wait_and_barrier<(AHEAD >= 3 ? 2 * LOADS : 0)>();
    else if (AHEAD >= 2 && ahead >= 1) wait_and_barrier<(AHEAD >= 2 ? LOADS : 0)>();
    else wait_and_barrier<0>();
}

template <int WK, int MT>
__global__ __launch_bounds__(64 * SM_WAVES, 2) void k_gemm_smb(SmArgs p) {
    using C = SmCfg<WK>;
    using B = SmbCfg<WK, MT>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[B::NBUF * B::STAGE];

    const int wg = blockIdx.x;
    const SmGemm G = p.many ? p.many[p.wg_gemm[wg]] : p.one;
    const int t = threadIdx.x, lane = t & 63, lr = lane & 31, lh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int n0 = __builtin_amdgcn_readfirstlane(((wg - G.wg0) * SM_WAVES + wave) * 32);
    const int n = n0 + lr;  // < Np (weights padded to 128-column groups)
    const bool live = n0 < __builtin_amdgcn_readfirstlane(G.N);
    const int nst = __builtin_amdgcn_readfirstlane(G.nst), M = __builtin_amdgcn_readfirstlane(p.M);
    const int esize = B::quant ? 1 : 2;
    const int64_t kbytes = (int64_t)G.K * esize;

    // DMA sources of this wave's activation runs: lane fills LDS bytes
    // [16·lane, 16·lane + 16) of run r, i.e. row (1024·r + 16·lane) / ROWB at
    // slot c; it fetches the chunk c ^ swz(row) of that row
    int64_t a_row[B::NA];
    int a_ch[B::NA], a_dst[B::NA];
#pragma unroll
    for (int j = 0; j < B::NA; j++) {
        const int run = wave + SM_WAVES * j;
        const int byte = run * 1024 + lane * 16;
        const int row = byte / B::ROWB, slot = (byte % B::ROWB) / 16;
        a_row[j] = (int64_t)min(row, M - 1) * G.ldx * esize;
        a_ch[j] = (slot ^ smb_swz<B::ROWB>(row)) * 16;
        a_dst[j] = run * 1024;
    }
    // DMA sources of this wave's weight runs (quantized): lane fills bytes
    // [16·lane, 16·lane + 16) of run i of the wave's [block][column][BB] area
    int64_t w_src[B::NWI > 0 ? B::NWI : 1];
#pragma unroll
    for (int i = 0; i < B::NWI; i++) {
        const int o = i * 1024 + lane * 16;
        const int j = o / (32 * B::BB), c = (o % (32 * B::BB)) / B::BB, sub = o % B::BB;
        w_src[i] = ((int64_t)j * G.np + n0 + c) * B::BB + sub;
    }
    auto issue = [&](int s) {
        uint8_t *L = lds + (s % B::NBUF) * B::STAGE;
#pragma unroll
        for (int j = 0; j < B::NA; j++) {
            const int64_t off = min((int64_t)s * B::ROWB + a_ch[j], kbytes - 16);
            __builtin_amdgcn_global_load_lds((const void *)((const uint8_t *)G.x + a_row[j] + off),
                                             LDS_PTR(L + a_dst[j]), 16, 0, 0);
        }
        if constexpr (B::quant) {
            // the rows' 4 block scales of stage s are one run of MT·32·8 bytes in
            // the stage-major plane; every wave moves it (identical bytes)
            const int run = (wave * 256) % B::SC_BYTES;  // this wave's 256-byte run
            const int64_t src = ((int64_t)s * G.xmp) * 8 + run + lane * 4;
            __builtin_amdgcn_global_load_lds((const void *)((const uint8_t *)G.xd + src),
                                             LDS_PTR(L + B::A_BYTES + run), 4, 0, 0);
            if constexpr (B::q41)
                __builtin_amdgcn_global_load_lds((const void *)((const uint8_t *)G.xs + src),
                                                 LDS_PTR(L + B::A_BYTES + B::SC_BYTES + run), 4, 0, 0);
            // this wave's weights (4 blocks = 4·np·BB bytes per stage) and the
            // 8 scale bytes of each of its 32 columns
            const int64_t wst = (int64_t)4 * s * G.np * B::BB;
#pragma unroll
            for (int i = 0; i < B::NWI; i++)
                __builtin_amdgcn_global_load_lds((const void *)(G.w + wst + w_src[i]),
                                                 LDS_PTR(L + B::W_OFF + wave * B::WW + i * 1024), 16, 0, 0);
            const int64_t dsrc = ((int64_t)s * G.np + n0) * 8 + lane * 4;
            __builtin_amdgcn_global_load_lds((const void *)((const uint8_t *)G.wd + dsrc),
                                             LDS_PTR(L + B::WD_OFF + wave * 256), 4, 0, 0);
            if constexpr (B::q41)
                __builtin_amdgcn_global_load_lds((const void *)((const uint8_t *)G.wm + dsrc),
                                                 LDS_PTR(L + B::WM_OFF + wave * 256), 4, 0, 0);
        }
    };

    v16f acc[MT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][r] = 0.f;

    if constexpr (B::quant) {
        auto compute = [&](int s) {
            const uint8_t *L = lds + (s % B::NBUF) * B::STAGE;
            const uint8_t *Wl = L + B::W_OFF + wave * B::WW;
            const v16i zi = {};
            const v16f zf = {};
            // the rows' 4 block scales are the raw K = 8 operand of the scale
            // product; the weight side is one-hot at block j (both K halves)
            v4h ha[MT];
            uint2 as[MT];
#pragma unroll
            for (int i = 0; i < MT; i++) {
                const uint2 ad = lds_u2(L + B::A_BYTES + (32 * i + lr) * 8);
                ha[i] = __builtin_bit_cast(v4h, v2u{ad.x, ad.y});
                if constexpr (C::q41) as[i] = lds_u2(L + B::A_BYTES + B::SC_BYTES + (32 * i + lr) * 8);
            }
            const uint2 wd = lds_u2(L + B::WD_OFF + wave * 256 + lr * 8);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v4i b;
                if constexpr (C::q4) {
                    const v4i wq = *(const v4i *)(Wl + (j * 32 + lr) * 16);
                    const int sh = 4 * lh;  // low nibbles: elements 0..15, high: 16..31
#pragma unroll
                    for (int e = 0; e < 4; e++) b[e] = (int)(((uint32_t)wq[e] >> sh) & 0x0F0F0F0Fu);
                    if constexpr (WK == WK_Q4_0)
#pragma unroll
                        for (int e = 0; e < 4; e++) b[e] = (int)(((uint32_t)b[e] + 0x78787878u) ^ 0x80808080u);
                } else {
                    b = *(const v4i *)(Wl + (j * 32 + lr) * 32 + lh * 16);
                }
                const uint32_t w = j < 2 ? wd.x : wd.y;
                const uint32_t m = (j & 1) ? (w & 0xFFFF0000u) : (w & 0xFFFFu);
                const v4h hb = __builtin_bit_cast(v4h, j < 2 ? v2u{m, 0u} : v2u{0u, m});
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    const int r = 32 * i + lr;
                    const v4i a = *(const v4i *)(L + r * B::ROWB + (((2 * j + lh) ^ smb_swz<B::ROWB>(r)) << 4));
                    v16i S = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, zi, 0, 0, 0);
                    const v16f Cs = __builtin_amdgcn_mfma_f32_32x32x8f16(ha[i], hb, zf, 0, 0, 0);
#pragma unroll
                    for (int r2 = 0; r2 < 16; r2++) acc[i][r2] = __builtin_fmaf((float)S[r2], Cs[r2], acc[i][r2]);
                }
            }
            if constexpr (C::q41) {
                const uint2 wm = lds_u2(L + B::WM_OFF + wave * 256 + lr * 8);
                const v4u hb = {wm.x, wm.y, 0u, 0u};
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    const v4u ha = {as[i].x, as[i].y, 0u, 0u};
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, ha),
                                                                    __builtin_bit_cast(v8h, hb), acc[i], 0, 0, 0);
                }
            }
        };
        // stages s + 1 .. s + AHEAD − 1 are in flight while stage s is
        // consumed; every wave issues B::LOADS instructions per stage (idle
        // strips load the zero padding columns), so stage s has landed when
        // at most the later issued stages' loads are outstanding.  The barrier
        // at the top of step s also frees the buffer stage s + AHEAD
        // overwrites (read by stage s − 1).
        for (int i = 0; i < B::AHEAD && i < nst; i++) issue(i);
        for (int s = 0; s < nst; s++) {
            smb_wait<B::LOADS, B::AHEAD>(min(B::AHEAD - 1, nst - 1 - s));
            if (s + B::AHEAD < nst) issue(s + B::AHEAD);
            if (live) compute(s);
        }
    } else {
        struct WStage {
            uint4 w[C::WL];
        };
        auto load_w = [&](int s, WStage &f) {
            const int b0 = 4 * s;
#pragma unroll
            for (int j = 0; j < C::WL; j++) {
                // block j / 2, slab j % 2, half lh
                f.w[j] = gload16(G.w + ((int64_t)(b0 + j / 2) * G.np + n) * C::BB + (2 * (j & 1) + lh) * 16);
            }
        };
        auto compute = [&](int s, const WStage &f) {
            const uint8_t *L = lds + (s % B::NBUF) * B::STAGE;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const v8h b = __builtin_bit_cast(v8h, f.w[j]);
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    const int r = 32 * i + lr;
                    const v8h a = *(const v8h *)(L + r * B::ROWB + (((2 * j + lh) ^ smb_swz<B::ROWB>(r)) << 4));
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[i], 0, 0, 0);
                }
            }
        };
        // stage s + 1 (activations in LDS, weights in registers) is in flight
        // while stage s is consumed; the barrier at the top of an iteration
        // also frees the buffer stage s + 1 overwrites
        WStage cur, nxt;
        issue(0);
        if (live) load_w(0, cur);
        for (int s = 0; s < nst; s++) {
            wait_and_barrier<0>();
            const bool more = s + 1 < nst;
            if (more) issue(s + 1);
            if (more && live) load_w(s + 1, nxt);
            if (live) compute(s, cur);
            if (more && live) cur = nxt;
        }
    }

    if (!live) return;
    constexpr float kScale = C::quant ? 0.5f : 1.0f;  // the scale products are doubled
    const int gn = n0 + lr;
    if (gn >= G.N) return;
    const float bv = G.bias ? G.bias[gn] : 0.f;
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
            if (row < M) G.y[(int64_t)row * G.ldy + gn] = acc[i][r] * kScale + bv;
        }
}

// Block-interleaved copy for the small-M kernel from the large-M layout
// ([Np][Kp] codes, Q4_0 stored as nibble − 8).  One thread per (block, column).
__global__ void k_pack_sm(const uint8_t *__restrict__ q, int64_t kp, int64_t np, int64_t kb, int wk,
                          uint8_t *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= kb * np) return;
    const int64_t b = i / np, nn = i % np;
    if (wk == WK_Q4_0 || wk == WK_Q4_1) {
        const int8_t *src = (const int8_t *)q + nn * kp + b * 32;
        const int off = wk == WK_Q4_0 ? 8 : 0;
        uint32_t w[4];
#pragma unroll
        for (int d = 0; d < 4; d++) {
            uint32_t v = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int j = 4 * d + e;
                const uint32_t lo = (uint32_t)(src[j] + off) & 15u, hi = (uint32_t)(src[j + 16] + off) & 15u;
                v |= (lo | (hi << 4)) << (8 * e);
            }
            w[d] = v;
        }
        *(uint4 *)(out + i * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        const int bb = wk == WK_Q8_0 ? 32 : 64;
        const uint4 *src = (const uint4 *)(q + (nn * kp + b * 32) * (bb / 32));
        uint4 *dst = (uint4 *)(out + i * bb);
        for (int c = 0; c < bb / 16; c++) dst[c] = src[c];
    }
}

}  // namespace

int64_t sm_weight_bytes(const Weight &w) {
    const int64_t kb4 = (w.Kp + 127) / 128 * 4;
    const int bb = (w.kind == WK_Q4_0 || w.kind == WK_Q4_1) ? 16 : (w.kind == WK_Q8_0 ? 32 : 64);
    return kb4 * w.Np * bb;
}

hipError_t launch_pack_sm(const Weight &w, void *out, hipStream_t st) {
    if (w.kind != WK_Q4_0 && w.kind != WK_Q4_1 && w.kind != WK_Q8_0 && w.kind != WK_F16) return hipErrorInvalidValue;
    hipError_t e = hipMemsetAsync(out, 0, (size_t)sm_weight_bytes(w), st);
    if (e != hipSuccess) return e;
    const int64_t kb = w.Kp / 32, total = kb * w.Np;
    hipLaunchKernelGGL(k_pack_sm, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, (const uint8_t *)w.q, w.Kp,
                       w.Np, kb, (int)w.kind, (uint8_t *)out);
    return hipGetLastError();
}

int sm_wgs(int64_t N, int ks) { return (int)(((N + 31) / 32 + SM_WAVES / ks - 1) / (SM_WAVES / ks)); }

hipError_t launch_gemm_smb(WKind kind, const SmArgs &a, int wgs, hipStream_t st) {
    if (a.M <= 0 || a.M > 64 || wgs <= 0 || (a.many && !a.wg_gemm)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)wgs), block(64 * SM_WAVES);
    const bool two = a.M > 32;
#define S3E_SMB(WK)                                                                              \
    do {                                                                                         \
        if (two) hipLaunchKernelGGL((k_gemm_smb<WK, 2>), grid, block, 0, st, a);                 \
        else hipLaunchKernelGGL((k_gemm_smb<WK, 1>), grid, block, 0, st, a);                     \
    } while (0)
    switch (kind) {
        case WK_Q4_0: S3E_SMB(WK_Q4_0); break;
        case WK_Q4_1: S3E_SMB(WK_Q4_1); break;
        case WK_Q8_0: S3E_SMB(WK_Q8_0); break;
        case WK_F16: S3E_SMB(WK_F16); break;
        default: return hipErrorInvalidValue;
    }
#undef S3E_SMB
    return hipGetLastError();
}

hipError_t launch_gemm_sm(WKind kind, const SmArgs &a, int wgs, int ks, hipStream_t st) {
    if (a.M <= 0 || a.M > 64 || wgs <= 0 || ks != 4 || (a.many && !a.wg_gemm)) return hipErrorInvalidValue;
    if (a.kg < 1 || a.kg > SM_KG_MAX || (a.kg > 1 && (a.many || !a.part || wgs % a.kg != 0)))
        return hipErrorInvalidValue;
    if (a.rt != 1 && (a.rt != 2 || a.M <= 32 || a.many || wgs % (2 * a.kg) != 0)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)wgs), block(64 * SM_WAVES);
    const bool two = a.M > 32 && a.rt == 1;
#define S3E_SM(WK)                                                                                       \
    do {                                                                                                 \
        if (two) hipLaunchKernelGGL((k_gemm_sm<WK, 2, 4>), grid, block, 0, st, a);                       \
        else hipLaunchKernelGGL((k_gemm_sm<WK, 1, 4>), grid, block, 0, st, a);                           \
    } while (0)
    switch (kind) {
        case WK_Q4_0: S3E_SM(WK_Q4_0); break;
        case WK_Q4_1: S3E_SM(WK_Q4_1); break;
        case WK_Q8_0: S3E_SM(WK_Q8_0); break;
        case WK_F16: S3E_SM(WK_F16); break;
        default: return hipErrorInvalidValue;
    }
#undef S3E_SM
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.kg == 1) return e;
    const SmGemm &g = a.one;
    const int64_t mn = (int64_t)a.M * g.N;
    const float scale = kind == WK_F16 ? 1.0f : 0.5f;  // the quantized scale products are doubled
    hipLaunchKernelGGL(k_sm_reduce, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, st, (const float *)a.part, a.kg,
                       mn, g.N, scale, g.bias, g.y, g.ldy);
    return hipGetLastError();
}

}  // namespace s3e
