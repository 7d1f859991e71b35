// k_conv.hip — the SimpleFPN neck's GEMMs on gfx950 fp16 MFMA
// (sam3_build_neck_graph, sam3.cpp:3863-3921): 1×1 convolutions and 3×3
// implicit-GEMM convolutions over NHWC activations (a pixel is a row of
// channels).  The 2×2 stride-2 transposed convolutions, whose fp16 kernels
// are plain fp16 GEMMs with a scattering epilogue, run in k_gemm
// (EPI_DECONV).
//
// Operands.  F16 weights (F16 files) meet fp16 activations: one
// v_mfma_f32_32x32x16_f16 per 32×32×16 step, exactly ggml's fp16 products
// with fp32 accumulation.  F32 weights (quantized files) are held as two
// fp16 planes w·2^k = wh + wl and meet activations held the same way
// (x = xh + xl): xh·wh + xh·wl + xl·wh, three MFMAs whose products are exact
// in fp32, so the result carries fp32 accuracy (the dropped xl·wl is
// ~2^-22 relative).
//
// Tiling.  A work-group computes 128 pixels × 256 channels with 8 waves
// (2 along M × 4 along N, 64×64 each: 2×2 MFMA tiles, so every A and B
// fragment read from LDS feeds two MFMAs, four with the split planes), or
// 256 pixels with 16 waves for the large split 3×3.  K advances in stages
// of 32 elements (64-byte rows per plane), streamed by
// global_load_lds_dwordx4 through a 3-deep LDS ring (2-deep for 256
// pixels): two stages (one) in flight while one is consumed.  64-byte rows put four rows in one 256-byte
// bank cycle; 16-byte chunk c of row r sits at slot c ^ ((r >> 2) & 3), which
// keeps the lane-ordered DMA writes and the 16-row MFMA operand reads free of
// bank conflicts.
//
// 3×3 convolutions (pad 1) are implicit GEMMs: K is ordered [ky][kx][Cin]
// (the weights are reordered at upload), a stage lies inside one tap, and
// each lane's DMA source is its pixel's neighbour for that tap or a zero row
// outside the image, so no im2col buffer exists.
//
// Epilogues write straight from the accumulators (lane = column, 16 rows
// per 32×32 tile): + bias into f32, fp16 or split-fp16 rows.
#include "s3e_internal.h"

namespace s3e {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

#define LDS_PTR(p) ((__attribute__((address_space(3))) void *)(p))

constexpr int BN = 256;
constexpr int ROWB = 64;   // bytes per row per stage and plane (32 fp16)
constexpr int WN = 4, MT = 2, NT = 2;  // waves along N, 32×32 tiles per wave

// Tile height BM = 128 (8 waves, 3-deep ring) or 256 (16 waves, 2-deep ring:
// every pixel tile streams the whole weight matrix, so taller tiles read it
// half as often; used where there are enough pixels to fill the chip).
template <bool SPLIT, int BM_>
struct Lay {
    static constexpr int BM = BM_, WAVES = BM / 16, NTH = 64 * WAVES, WM = BM / 64;
    static constexpr int NBUF = BM == 256 ? 2 : 3;
    static constexpr int planes = SPLIT ? 2 : 1;
    static constexpr int A = BM * ROWB, B = BN * ROWB;  // bytes of one plane
    static constexpr int OFF_A = 0, OFF_ALO = A;
    static constexpr int OFF_B = planes * A, OFF_BLO = OFF_B + B;
    static constexpr int STAGE = planes * (A + B);
    static constexpr int LDS = NBUF * STAGE;
    static constexpr int NA = A / 1024 / WAVES;  // 1 KB DMA runs per wave per stage and plane
    static constexpr int NB = B / 1024 / WAVES;
    static constexpr int NLOAD = planes * (NA + NB);
};

struct ConvParams {
    const uint8_t *a, *a_lo;  // activation rows (bytes), a_ld bytes apart
    int64_t a_ld, a_kbytes;
    const uint8_t *b, *b_lo;  // weight rows [Np][Kp] fp16
    int64_t b_ld;
    int M, N, nstages, tiles_m, tiles_n, ntiles;
    float alpha;              // split: 2^-k of the weight planes
    int cw, ch, spt;          // 3×3 geometry (spt = stages per tap)
    const uint8_t *zero;
    EpiArgs e;
};

__device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }

__device__ __forceinline__ void store_act(const Act &o, int64_t row, int64_t col, float v) {
    const int64_t i = row * o.ld + col;
    if (o.kind == A_F32) {
        ((float *)o.x)[i] = v;
        return;
    }
    const _Float16 h = to_half(v);
    ((_Float16 *)o.x)[i] = h;
    if (o.kind == A_F16X2) ((_Float16 *)o.lo)[i] = (_Float16)(v - (float)h);
}

template <int BM_>
constexpr int conv_nth = 64 * (BM_ / 16);  // threads of a work-group (Lay::NTH)

template <bool SPLIT, int CONV, int EPI, int BM_>
__global__ __launch_bounds__(conv_nth<BM_>, (SPLIT || BM_ == 256) ? 1 : 2) void k_conv(ConvParams p) {
    using L = Lay<SPLIT, BM_>;
    constexpr int BM = L::BM, WAVES = L::WAVES, NBUF = L::NBUF;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[L::LDS];

    // ---- tile: each XCD (ids dealt round-robin over 8) takes a contiguous
    // range of tiles, rastered in groups of 8 tile-rows
    const int per = gridDim.x >> 3;
    const int logical = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (logical >= p.ntiles) return;
    constexpr int GROUP = 8;
    const int group = logical / (GROUP * p.tiles_n);
    const int first_m = group * GROUP;
    const int gsz = min(p.tiles_m - first_m, GROUP);
    const int rem = logical - group * GROUP * p.tiles_n;
    const int m0 = (first_m + rem % gsz) * BM, n0 = (rem / gsz) * BN;

    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int lane = t & 63;
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, lh = lane >> 5;

    // ---- DMA: a 1 KB run is 16 rows of 64 B; lane writes slot lane & 3 of
    // row lane >> 2 and fetches the chunk that belongs there
    int64_t a_row[L::NA];
    int a_cofs[L::NA], a_y[L::NA], a_x[L::NA];
#pragma unroll
    for (int j = 0; j < L::NA; j++) {
        const int row = 16 * (wave * L::NA + j) + (lane >> 2);
        const int gm = min(m0 + row, p.M - 1);
        a_row[j] = (int64_t)gm * p.a_ld;
        a_cofs[j] = ((lane & 3) ^ swz(row)) << 4;
        if constexpr (CONV) {
            a_y[j] = gm / p.cw;
            a_x[j] = gm - a_y[j] * p.cw;
        }
    }
    const int64_t a_last = p.a_kbytes - 16;
    int64_t b_row[L::NB];
#pragma unroll
    for (int j = 0; j < L::NB; j++) {
        const int col = 16 * (wave * L::NB + j) + (lane >> 2);
        b_row[j] = (int64_t)(n0 + col) * p.b_ld + (((lane & 3) ^ swz(col)) << 4);
    }

    auto issue = [&](int s) {
        uint8_t *S = lds + (s % NBUF) * L::STAGE;
        if constexpr (CONV) {
            const int tap = s / p.spt, kc = s - tap * p.spt;
            const int dy = tap / 3 - 1, dx = tap - (tap / 3) * 3 - 1;
            const int64_t shift = (int64_t)(dy * p.cw + dx) * p.a_ld + kc * ROWB;
#pragma unroll
            for (int j = 0; j < L::NA; j++) {
                const bool in = (unsigned)(a_y[j] + dy) < (unsigned)p.ch && (unsigned)(a_x[j] + dx) < (unsigned)p.cw;
                const int64_t o = a_row[j] + shift + a_cofs[j];
                const uint8_t *z = p.zero + a_cofs[j];
                __builtin_amdgcn_global_load_lds((const void *)(in ? p.a + o : z),
                                                 LDS_PTR(S + L::OFF_A + (wave * L::NA + j) * 1024), 16, 0, 0);
                if constexpr (SPLIT)
                    __builtin_amdgcn_global_load_lds((const void *)(in ? p.a_lo + o : z),
                                                     LDS_PTR(S + L::OFF_ALO + (wave * L::NA + j) * 1024), 16, 0, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < L::NA; j++) {
                const int64_t o = a_row[j] + min((int64_t)s * ROWB + a_cofs[j], a_last);
                __builtin_amdgcn_global_load_lds((const void *)(p.a + o),
                                                 LDS_PTR(S + L::OFF_A + (wave * L::NA + j) * 1024), 16, 0, 0);
                if constexpr (SPLIT)
                    __builtin_amdgcn_global_load_lds((const void *)(p.a_lo + o),
                                                     LDS_PTR(S + L::OFF_ALO + (wave * L::NA + j) * 1024), 16, 0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < L::NB; j++) {
            const int64_t o = b_row[j] + (int64_t)s * ROWB;
            __builtin_amdgcn_global_load_lds((const void *)(p.b + o),
                                             LDS_PTR(S + L::OFF_B + (wave * L::NB + j) * 1024), 16, 0, 0);
            if constexpr (SPLIT)
                __builtin_amdgcn_global_load_lds((const void *)(p.b_lo + o),
                                                 LDS_PTR(S + L::OFF_BLO + (wave * L::NB + j) * 1024), 16, 0, 0);
        }
    };

    // ---- operand offsets: tile rows start at multiples of 32, so the swizzle
    // of row wm·64 + 32i + lr is swz(lr)
    const int xr = swz(lr);
    int a_off[MT], b_off[NT];
#pragma unroll
    for (int i = 0; i < MT; i++) a_off[i] = (wm * 64 + 32 * i + lr) * ROWB;
#pragma unroll
    for (int n = 0; n < NT; n++) b_off[n] = (wn * 64 + 32 * n + lr) * ROWB;
    int cofs[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) cofs[ks] = ((2 * ks + lh) ^ xr) << 4;

    v16f acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][n][r] = 0.f;

    auto compute = [&](int s) {
        const uint8_t *S = lds + (s % NBUF) * L::STAGE;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            v8h ah[MT], bh[NT], al[MT], bl[NT];
#pragma unroll
            for (int i = 0; i < MT; i++) {
                ah[i] = *(const v8h *)(S + L::OFF_A + a_off[i] + cofs[ks]);
                if constexpr (SPLIT) al[i] = *(const v8h *)(S + L::OFF_ALO + a_off[i] + cofs[ks]);
            }
#pragma unroll
            for (int n = 0; n < NT; n++) {
                bh[n] = *(const v8h *)(S + L::OFF_B + b_off[n] + cofs[ks]);
                if constexpr (SPLIT) bl[n] = *(const v8h *)(S + L::OFF_BLO + b_off[n] + cofs[ks]);
            }
#pragma unroll
            for (int i = 0; i < MT; i++)
#pragma unroll
                for (int n = 0; n < NT; n++)
                    acc[i][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bh[n], acc[i][n], 0, 0, 0);
            if constexpr (SPLIT) {
                // x·w = (xh + xl)(wh + wl) ≈ xh·wh + xh·wl + xl·wh
#pragma unroll
                for (int i = 0; i < MT; i++)
#pragma unroll
                    for (int n = 0; n < NT; n++)
                        acc[i][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bl[n], acc[i][n], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < MT; i++)
#pragma unroll
                    for (int n = 0; n < NT; n++)
                        acc[i][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bh[n], acc[i][n], 0, 0, 0);
            }
        }
    };

    // ---- main loop: stages s+1 and s+2 in flight while stage s is consumed
    const int ns = p.nstages;
    issue(0);
    if constexpr (NBUF == 3) {
        if (ns > 1) issue(1);
        for (int s = 0; s < ns; s++) {
            if (s + 1 < ns) wait_and_barrier<L::NLOAD>();
            else wait_and_barrier<0>();
            if (s + 2 < ns) issue(s + 2);
            compute(s);
        }
    } else {
        // 2-deep: stage s landed and stage s−1's buffer released, then s+1 in
        // flight while s is consumed
        for (int s = 0; s < ns; s++) {
            wait_and_barrier<0>();
            if (s + 1 < ns) issue(s + 1);
            compute(s);
        }
    }

    // ---- epilogue from the accumulators: lane holds column lr of each 32×32
    // tile, rows 8·(r / 4) + 4·lh + r % 4
    const EpiArgs &e = p.e;
    const float alpha = SPLIT ? p.alpha : 1.0f;
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int gn = n0 + wn * 64 + 32 * n + lr;
        if (gn >= p.N) continue;
        const int co = gn;
        const float bv = e.bias[co];
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int gm = m0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (gm >= p.M) continue;
                float b = bv;
                if constexpr (CONV == 1) {
                    if (e.bias_cls) {
                        const int py = gm / p.cw, px = gm - py * p.cw;
                        const int cy = py == 0 ? 0 : (py == p.ch - 1 ? 2 : 1);
                        const int cx = px == 0 ? 0 : (px == p.cw - 1 ? 2 : 1);
                        b = e.bias[(3 * cy + cx) * p.N + co];
                    }
                }
                float v = __fadd_rn(acc[i][n][r] * alpha, b);
                if constexpr (EPI == EPI_F32) e.y[(int64_t)gm * e.ldy + gn] = v;
                else store_act(e.out, gm, gn, v);
            }
    }
}

template <bool SPLIT, int CONV, int EPI, int BM = 128>
hipError_t launch_one(ConvParams &p, hipStream_t st) {
    p.tiles_m = (p.M + BM - 1) / BM;
    p.ntiles = p.tiles_m * p.tiles_n;
    const int grid = ((p.ntiles + 7) / 8) * 8;
    hipLaunchKernelGGL((k_conv<SPLIT, CONV, EPI, BM>), dim3(grid), dim3(Lay<SPLIT, BM>::NTH), 0, st, p);
    return hipGetLastError();
}

template <bool SPLIT>
hipError_t dispatch(Epi epi, bool conv3, ConvParams &p, hipStream_t st) {
    if (conv3) {
        if (epi != EPI_F32) return hipErrorInvalidValue;
        // split 3×3 with more than two 128-pixel tiles per CU: 256-pixel tiles
        if constexpr (SPLIT)
            if (p.M > 128 * 512) return launch_one<SPLIT, 1, EPI_F32, 256>(p, st);
        return launch_one<SPLIT, 1, EPI_F32>(p, st);
    }
    switch (epi) {
        case EPI_F32: return launch_one<SPLIT, 0, EPI_F32>(p, st);
        case EPI_ACT: return launch_one<SPLIT, 0, EPI_ACT>(p, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_conv(const Weight &w, const Act &a, int64_t M, Epi epi, const EpiArgs &ea,
                       const ConvGeom *g, hipStream_t st) {
    if (M <= 0) return hipSuccess;
    if (w.kind != WK_F16 && w.kind != WK_F16X3) return hipErrorInvalidValue;
    const bool split = w.kind == WK_F16X3;
    if (split != (a.kind == A_F16X2) || (a.kind != A_F16 && a.kind != A_F16X2)) return hipErrorInvalidValue;
    // weight rows padded to whole stages and whole 256-column tiles
    if (w.Kp % 32 != 0 || w.Np % BN != 0) return hipErrorInvalidValue;
    ConvParams p{};
    p.a = (const uint8_t *)a.x;
    p.a_lo = (const uint8_t *)a.lo;
    p.a_ld = a.ld * 2;
    p.a_kbytes = w.K * 2;
    p.b = (const uint8_t *)w.q;
    p.b_lo = (const uint8_t *)w.lo;
    p.b_ld = w.Kp * 2;
    p.M = (int)M;
    p.N = (int)w.N;
    p.nstages = (int)(w.Kp / 32);
    p.tiles_n = (int)(w.Np / BN);
    p.alpha = w.alpha;
    p.e = ea;
    if (g) {
        // a stage of 32 channels stays inside one tap: Cin = 32·spt
        if (g->spt <= 0 || w.K != 9LL * 32 * g->spt || a.ld != 32LL * g->spt || (int64_t)g->w * g->h != M ||
            !g->zero)
            return hipErrorInvalidValue;
        p.cw = g->w;
        p.ch = g->h;
        p.spt = g->spt;
        p.zero = (const uint8_t *)g->zero;
    }
    return split ? dispatch<true>(epi, g != nullptr, p, st) : dispatch<false>(epi, g != nullptr, p, st);
}

}  // namespace s3e
