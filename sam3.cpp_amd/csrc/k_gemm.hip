// k_gemm.hip — Y[M][N] = X[M][K] · W[N][K]ᵀ on gfx950 MFMA, the engine's
// replacement for ggml_mul_mat (sam3.cpp:3738, 3779, 3792, 3795, 3815).
//
// Quantized weights (Q4_0, Q4_1, Q8_0) meet activations that were quantized
// per 32-element block exactly as ggml's CPU path does (Q8_0 / Q8_1).  For
// each 32-element block b the kernel forms the exact integer sum
//     S_b[m][n] = Σ_{k∈b} qx[m][k]·qw[n][k]
// with one v_mfma_i32_32x32x32_i8 (K = 32 = one ggml block), the exact fp32
// block scale 2·dx[m][b]·dw[n][b] with one v_mfma_f32_32x32x8_f16 whose
// operands hold each lane's own scale in its first K slot and zeros elsewhere
// (both lane halves carry the scale, hence the exact factor 2, removed at the
// end; the K = 8 form issues faster than K = 16 and the product needs one
// slot), and accumulates acc += float(S_b)·c_b in fp32 on the VALU.  Q4_1
// adds Σ_b m_w[n][b]·s_x[m][b] with one more fp16 MFMA per 4 blocks into its
// own accumulator.  Q4_0 weights with an fp6 copy run in k_gemm_f6 (below),
// where the block sum comes out of the fp6 MFMA already in fp32.  F16
// weights run on fp16 MFMA against activations rounded to fp16; F32 weights
// run on fp32 MFMA, or, uploaded as fp16 pairs (WK_F16X3: w·2^k = wh + wl)
// against activations held the same way (x = xh + xl), as xh·wh + xh·wl +
// xl·wh on fp16 MFMA — each product exact in fp32, the dropped xl·wl ~2^-22
// relative — in stages of 32 K whose hi and lo planes are 64-byte LDS rows
// (chunk c of row r at slot c ^ ((r >> 2) & 3)).
//
// Per work-group: a 64×128 output tile and 4 waves (2 along M × 2 along N,
// each 32×64; three work-groups per CU) or, for Q4_1, 8 waves (2 × 4, each
// 32×32; two per CU).  K advances in stages of 128 bytes per row (4 quant
// blocks, 64 fp16 or 32 f32).  Stages stream through a 2- or 3-deep LDS ring
// filled by global_load_lds_dwordx4 (no register staging): the next stages
// are in flight while stage s is consumed, and one barrier per stage orders
// reuse.
// LDS rows are 128 bytes with 16-byte chunks XOR-swizzled by row (chunk c of
// row r at slot c ^ ((r >> 1) & 7)), which keeps both the lane-ordered DMA
// writes and the MFMA operand reads free of bank conflicts without padding.  Scales
// arrive from stage-major planes, so a stage's scales for the tile are one
// contiguous run.  Work-group ids are remapped so that each XCD (ids are dealt
// round-robin over 8) gets a contiguous range of tiles, rastered in groups of
// 8 tile-rows so that concurrently running tiles share operands in its L2.
//
// Epilogues run from an fp32 copy of the tile in LDS: 32-column chunks per
// thread where 32-wide quant blocks, RoPE pairs and fp16 rows must be whole
// inside one thread, float4 columns per lane for plain f32 stores.
#include "s3e_internal.h"

#include <algorithm>

namespace s3e {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef uint64_t v4u64 __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));

#define LDS_PTR(p) ((__attribute__((address_space(3))) void *)(p))

constexpr int BN = GEMM_BN;   // 128
constexpr int ROWB = 128;     // bytes per tile row per stage
constexpr int CLD = BN + 4;   // fp32 C-tile row stride

// Tile configurations.  WAVES = 8: waves 2 (M) × 4 (N), each BM/2 × 32,
// 3-deep ring, 4 waves per SIMD at BM = 64 (two work-groups per CU).
// WAVES = 4: waves 2 × 2, each BM/2 × 64 (two MFMA column tiles share one A
// fragment and one scale operand), 2-deep ring, three work-groups per CU.
template <int WK, int BM_, int WAVES_>
struct Cfg {
    static constexpr int BM = BM_;
    static constexpr int WAVES = WAVES_;
    static constexpr int NTH = 64 * WAVES;
    static constexpr bool quant = (WK == WK_Q4_0 || WK == WK_Q4_1 || WK == WK_Q8_0);
    static constexpr bool q41 = (WK == WK_Q4_1);
    // WK_F16X3: fp32 operands as fp16 pairs x = hi + lo, each plane of a stage
    // 32 K wide (64-byte rows: the hi plane of the tile, then the lo plane)
    static constexpr bool split = (WK == WK_F16X3);
    static constexpr int esize = quant ? 1 : ((WK == WK_F16 || split) ? 2 : 4);
    static constexpr int WM = 2, WN = WAVES / 2;
    static constexpr int MT = BM / (32 * WM);            // 32-row MFMA tiles per wave
    static constexpr int NT = BN / (32 * WN);            // 32-column MFMA tiles per wave
    static constexpr int NBUF = WAVES == 4 ? 2 : 3;      // LDS ring depth
    static constexpr int OFF_A = 0;
    static constexpr int OFF_B = BM * ROWB;
    static constexpr int OFF_ALO = BM * 64, OFF_BLO = OFF_B + BN * 64;  // split: lo planes
    static constexpr int OFF_SC = OFF_B + BN * ROWB;     // scales: AD | BD | AS | BMIN
    static constexpr int OFF_AD = OFF_SC;
    static constexpr int OFF_BD = OFF_AD + (quant ? BM * 8 : 0);
    static constexpr int OFF_AS = OFF_BD + (quant ? BN * 8 : 0);
    static constexpr int OFF_BMIN = OFF_AS + (q41 ? BM * 8 : 0);
    static constexpr int STAGE = OFF_BMIN + (q41 ? BN * 8 : 0);
    static constexpr int NA = BM / (8 * WAVES);          // 1 KB A loads per wave per stage
    static constexpr int NB = BN / (8 * WAVES);          // 1 KB B loads per wave per stage
    static constexpr int SC = (STAGE - OFF_SC) / 256;    // 256 B scale loads per stage
    static constexpr int NS = (SC + WAVES - 1) / WAVES;  // ... per wave
    static constexpr int NLOAD = NA + NB + NS;
    static constexpr int RING = NBUF * STAGE;
    static constexpr int LDS = RING > BM * CLD * 4 ? RING : BM * CLD * 4;
    // quant blocks: with one MFMA column tile per wave, blocks are software
    // pipelined (MFMAs of block b+1 in flight during the VALU of block b);
    // with two, the second tile's MFMAs cover the first tile's VALU and the
    // registers of a second block set are not needed
    static constexpr bool PIPE = NT * MT <= 1;
};

struct GemmParams {
    const uint8_t *a;             // activation values, rows of a_ld bytes
    const uint8_t *a_d, *a_s;     // stage-major fp16 planes, a_mp rows per group
    int64_t a_ld, a_kbytes, a_mp;
    int a_rec, b_rec;             // bytes the operand buffer loads may address
    int ksplit;                   // > 1: K split into ranges, raw partial tiles to part [ksplit][M][N]
    float *part;
    const uint8_t *b;             // weight values, rows of b_ld bytes
    const uint8_t *b_d, *b_m;     // stage-major fp16 planes, b_np rows per group
    int64_t b_ld, b_np;
    int M, N, nstages, tiles_m, tiles_n, ntiles;
    const uint8_t *a_lo, *b_lo;   // WK_F16X3: the lo planes (same layouts as a / b)
    float alpha;                  // WK_F16X3: the weight planes hold w·2^k; alpha = 2^−k
    EpiArgs e;
};

__device__ __forceinline__ uint16_t f2h_bits(float v) { return half_bits(v); }

// Quantize 32 values to one Q8 block the way ggml's x86 quantize_row_q8_0 /
// q8_1 do: d = amax/127, id = 127/amax, q = round-half-even(v·id).  The
// product v·id is rounded to float first, then to an integer by adding
// 1.5·2^23 (exact round-half-even for |v·id| ≤ 127), whose low byte is q.
__device__ __forceinline__ void quant_block32(const float *v, int8_t *qdst, uint16_t *ddst,
                                              uint16_t *sdst) {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.f;
    const float id = (amax != 0.f) ? 127.f / amax : 0.f;
    constexpr uint32_t MAGIC = 0x4B400000u;  // bits of 1.5·2^23
    uint32_t usum = 0;
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint32_t u[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            u[i] = __builtin_bit_cast(uint32_t, __fadd_rn(__fmul_rn(v[4 * j + i], id), 12582912.0f));
            usum += u[i];
        }
        const uint32_t lo = __builtin_amdgcn_perm(u[1], u[0], 0x0c0c0400u);
        const uint32_t hi = __builtin_amdgcn_perm(u[3], u[2], 0x0c0c0400u);
        w[j] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
    const int sum = (int)(usum - 32u * MAGIC);
    uint4 *dst = (uint4 *)qdst;
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    *ddst = f2h_bits(d);
    // s = fp16(fp32(d·Σq)): f2h_bits keeps the fp32 rounding of the product
    if (sdst) *sdst = f2h_bits(d * (float)sum);
}

// The same quantization into the A_F6 layout (row `row`, block `blk` of an
// activation with nst stages of 128): the codes split q = 16·h + l, each part
// as three 8-byte words of fp6 E3M2 codes.
__device__ __forceinline__ void quant_block32_f6(const float *v, uint64_t *base, int64_t nst, int64_t row,
                                                 int64_t blk, uint16_t *ddst) {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.f;
    const float id = (amax != 0.f) ? 127.f / amax : 0.f;
    f32x16 he, ho, le, lo;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        float a, b, c, e;
        f6_split(v[2 * i], id, a, b);
        f6_split(v[2 * i + 1], id, c, e);
        he[i] = a;
        le[i] = b;
        ho[i] = c;
        lo[i] = e;
    }
    const u32x6 ph = pack_bf6(he, ho), pl = pack_bf6(le, lo);
#pragma unroll
    for (int t = 0; t < 3; t++) {
        base[f6_act_word(nst, row, blk, 0, t)] = (uint64_t)ph[2 * t] | ((uint64_t)ph[2 * t + 1] << 32);
        base[f6_act_word(nst, row, blk, 1, t)] = (uint64_t)pl[2 * t] | ((uint64_t)pl[2 * t + 1] << 32);
    }
    *ddst = f2h_bits(d);
}

// XOR swizzle of the 16-byte chunks of LDS row r: chunk c lives at slot
// c ^ swz(r).  gfx950's LDS has 64 banks of 4 bytes, so one 128-byte row
// covers half of them and rows r, r+2, ... share banks: swz(r) = (r >> 1) & 7
// gives the 16 rows that one ds_read_b128 phase touches distinct bank groups.
#ifndef S3E_SWZ_SHIFT
#define S3E_SWZ_SHIFT 1
#endif
__device__ __forceinline__ int swz(int r) { return (r >> S3E_SWZ_SHIFT) & 7; }
// Rows of 64 bytes (split planes): four rows share a 256-byte bank cycle;
// 16-byte chunk c of row r sits at slot c ^ ((r >> 2) & 3).
__device__ __forceinline__ int swz64(int r) { return (r >> 2) & 3; }

// 4 bytes per lane, likewise (scale planes).  A buffer load, unlike
// global_load_lds, is not a flat-segment access, so the compiler keeps the
// LDS read counter in order and can wait for operand reads one by one.
__device__ __forceinline__ void dma4_buf(const void *base, int nrec, void *lds, int voff, int soff) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, nrec, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, LDS_PTR(lds), 4, voff, soff, 0, 0);
}

// 16 bytes per lane from base + voff + soff (a raw buffer of nrec bytes) into
// LDS at lds + 16·lane.  base, nrec and soff are wave-uniform, so the buffer
// descriptor lives in scalar registers and the uniform part of the address
// costs no vector instruction.
__device__ __forceinline__ void dma16_buf(const void *base, int nrec, void *lds, int voff, int soff) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, nrec, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, LDS_PTR(lds), 16, voff, soff, 0, 0);
}

// Epilogue from the fp32 tile Ct [BM][CLD] in LDS (scaled, complete), run by
// the NT_ threads of the work-group.
template <int EPI, int BM, int NT_>
__device__ __forceinline__ void epilogue(const GemmParams &p, const float *Ct, int m0, int n0, int t) {
    const EpiArgs &e = p.e;
    if constexpr (EPI == EPI_QKV) {
        const int sel = n0 / e.E + e.sel0;  // 0 = Q, 1 = K, 2 = V (a tile never straddles)
        const int Nw = e.window * e.window;
        const int nwx = e.grid / e.window;
        if (sel == 2) {
            // Vᵀ [b][h][d][slot]: a unit is one column d and 8 consecutive
            // tokens.  Window and image-row boundaries fall on multiples of 8
            // tokens (the model loader checks), so the 8 tokens are positions
            // p..p+7 of one window, p % 8 == 0: two runs of 4 keys, each one
            // 8-byte store per plane at its vt_slot.
            for (int u = t; u < BN * (BM / 8); u += NT_) {
                const int col = u / (BM / 8), r0 = (u % (BM / 8)) * 8;
                const int gm = m0 + r0;
                if (gm >= p.M) continue;
                const int gn = n0 + col;
                const float bv = e.bias[gn];
                const int r2 = gn - (2 - e.sel0) * e.E;
                const int h = r2 / e.HD, d = r2 % e.HD;
                const int py = gm / e.grid, px = gm % e.grid;
                const int b = (py / e.window) * nwx + px / e.window;
                const int pp = (py % e.window) * e.window + px % e.window;
                uint32_t w[4], wl[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float v0 = Ct[(r0 + 2 * j) * CLD + col] + bv;
                    const float v1 = Ct[(r0 + 2 * j + 1) * CLD + col] + bv;
                    const _Float16 h0 = to_half(v0), h1 = to_half(v1);
                    w[j] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                    const _Float16 l0 = (_Float16)(v0 - (float)h0), l1 = (_Float16)(v1 - (float)h1);
                    wl[j] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
                }
                const int64_t row = ((int64_t)(b * e.NH + h) * e.HD + d) * e.vt_ld;
                const int64_t o0 = row + vt_slot(pp), o1 = row + vt_slot(pp + 4);
                *(uint2 *)(e.vt + o0) = make_uint2(w[0], w[1]);
                *(uint2 *)(e.vt + o1) = make_uint2(w[2], w[3]);
                if (e.vt_lo) {
                    *(uint2 *)(e.vt_lo + o0) = make_uint2(wl[0], wl[1]);
                    *(uint2 *)(e.vt_lo + o1) = make_uint2(wl[2], wl[3]);
                }
            }
        } else {
            // Q, K [b][h][p][d] with RoPE: a unit is one token and 16 columns
            for (int u = t; u < BM * (BN / 16); u += NT_) {
                const int row = u / (BN / 16), cc = u % (BN / 16);
                const int gm = m0 + row;
                if (gm >= p.M) continue;
                const int gn0 = n0 + cc * 16;
                float v[16];
#pragma unroll
                for (int j = 0; j < 16; j += 4) {
                    const float4 x = *(const float4 *)(Ct + row * CLD + cc * 16 + j);
                    const float4 bb = *(const float4 *)(e.bias + gn0 + j);
                    v[j] = x.x + bb.x;
                    v[j + 1] = x.y + bb.y;
                    v[j + 2] = x.z + bb.z;
                    v[j + 3] = x.w + bb.w;
                }
                const int py = gm / e.grid, px = gm % e.grid;
                const int b = (py / e.window) * nwx + px / e.window;
                const int pp = (py % e.window) * e.window + px % e.window;
                const int r2 = gn0 - (sel - e.sel0) * e.E;
                const int h = r2 / e.HD, d0 = r2 % e.HD;
                if (e.freqs && (e.rope_rows <= 0 || gm < e.rope_rows)) {
                    // sam3_apply_rope: out_re = re·cos − im·sin, out_im = re·sin + im·cos,
                    // each product rounded on its own (separate ggml ops).
                    const float4 *f4 = (const float4 *)(e.freqs + ((int64_t)pp * (e.HD / 2) + d0 / 2) * 2);
#pragma unroll
                    for (int j = 0; j < 16; j += 4) {
                        const float4 cs = f4[j / 4];  // cos, sin of pairs j/2 and j/2 + 1
                        const float c0 = cs.x, s0 = cs.y, c1 = cs.z, s1 = cs.w;
                        const float re0 = v[j], im0 = v[j + 1], re1 = v[j + 2], im1 = v[j + 3];
                        v[j] = __fsub_rn(__fmul_rn(re0, c0), __fmul_rn(im0, s0));
                        v[j + 1] = __fadd_rn(__fmul_rn(re0, s0), __fmul_rn(im0, c0));
                        v[j + 2] = __fsub_rn(__fmul_rn(re1, c1), __fmul_rn(im1, s1));
                        v[j + 3] = __fadd_rn(__fmul_rn(re1, s1), __fmul_rn(im1, c1));
                    }
                }
                const int64_t o = ((int64_t)(b * e.NH + h) * Nw + pp) * e.HD + d0;
                _Float16 *lo = sel == 0 ? e.q_lo : e.k_lo;
                uint32_t w[8], wl[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
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
                if (lo) {
                    uint4 *l4 = (uint4 *)(lo + o);
                    l4[0] = make_uint4(wl[0], wl[1], wl[2], wl[3]);
                    l4[1] = make_uint4(wl[4], wl[5], wl[6], wl[7]);
                }
            }
        }
    } else if constexpr (EPI == EPI_HQKV) {
        // Hiera (sam2_hiera_block_forward, sam3.cpp:4330-4395): columns [0, C) are Q,
        // [C, 2C) K, [2C, 3C) V of tokens in raster order over a grid_h × grid grid.
        // Windows of wh × ww (window 0: the whole grid) are row-major over nwx per
        // row; heads of HD channels go to rows of hdp (zeros past HD).
        const int C = e.E, HD = e.HD, HDp = e.hdp, W = e.grid;
        const int wh = e.window > 0 ? e.window : e.grid_h, ww = e.window > 0 ? e.window : W;
        const int nwx = (W + ww - 1) / ww, Nkv = wh * ww;
        // Q, K: a unit is one token and 8 columns (one 16-byte store per plane)
        for (int u = t; u < BM * (BN / 8); u += NT_) {
            const int row = u / (BN / 8), cc = u % (BN / 8);
            const int gm = m0 + row, gn0 = n0 + cc * 8;
            if (gm >= p.M || gn0 >= 2 * C) continue;
            float v[8];
            {
                const float4 x0 = *(const float4 *)(Ct + row * CLD + cc * 8);
                const float4 x1 = *(const float4 *)(Ct + row * CLD + cc * 8 + 4);
                const float4 b0 = *(const float4 *)(e.bias + gn0);
                const float4 b1 = *(const float4 *)(e.bias + gn0 + 4);
                v[0] = x0.x + b0.x; v[1] = x0.y + b0.y; v[2] = x0.z + b0.z; v[3] = x0.w + b0.w;
                v[4] = x1.x + b1.x; v[5] = x1.y + b1.y; v[6] = x1.z + b1.z; v[7] = x1.w + b1.w;
            }
            const int sel = gn0 >= C;
            const int r2 = gn0 - sel * C;
            if (sel == 0 && e.qpool) {  // Q rows for the pooling pass
                float4 *dst = (float4 *)(e.y + (int64_t)gm * e.ldy + r2);
                dst[0] = make_float4(v[0], v[1], v[2], v[3]);
                dst[1] = make_float4(v[4], v[5], v[6], v[7]);
                continue;
            }
            const int h = r2 / HD, d0 = r2 % HD;
            const int py = gm / W, px = gm % W;
            const int b = (py / wh) * nwx + px / ww;
            const int pp = (py % wh) * ww + px % ww;
            const int64_t o = ((int64_t)(b * e.NH + h) * Nkv + pp) * HDp + d0;
            _Float16 *hi = sel == 0 ? e.q : e.k;
            _Float16 *lo = sel == 0 ? e.q_lo : e.k_lo;
            uint32_t w[4], wl[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const _Float16 h0 = to_half(v[2 * j]), h1 = to_half(v[2 * j + 1]);
                w[j] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                const _Float16 l0 = (_Float16)(v[2 * j] - (float)h0), l1 = (_Float16)(v[2 * j + 1] - (float)h1);
                wl[j] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
            }
            *(uint4 *)(hi + o) = make_uint4(w[0], w[1], w[2], w[3]);
            if (lo) *(uint4 *)(lo + o) = make_uint4(wl[0], wl[1], wl[2], wl[3]);
            if (d0 + 8 == HD) {  // the head's padding columns
                for (int z = 8; z < HDp - d0; z += 8) {
                    *(uint4 *)(hi + o + z) = make_uint4(0u, 0u, 0u, 0u);
                    if (lo) *(uint4 *)(lo + o + z) = make_uint4(0u, 0u, 0u, 0u);
                }
            }
        }
        // Vᵀ [b][h][d][slot]: lanes run along pairs of tokens of one column, so a
        // store instruction covers runs of consecutive key slots; a pair that
        // stays inside one window row at an even position fills two adjacent
        // slots (vt_slot keeps aligned pairs together) with one 4-byte store
        for (int u = t; u < (BM / 2) * BN; u += NT_) {
            const int rp = u % (BM / 2), col = u / (BM / 2);
            const int gm = m0 + 2 * rp, gn = n0 + col;
            if (gm >= p.M || gn < 2 * C || gn >= 3 * C) continue;
            const float bv = e.bias[gn];
            const float v0 = Ct[(2 * rp) * CLD + col] + bv, v1 = Ct[(2 * rp + 1) * CLD + col] + bv;
            const int r2 = gn - 2 * C;
            const int h = r2 / HD, d = r2 % HD;
            const int py = gm / W, px = gm % W;
            const int b = (py / wh) * nwx + px / ww;
            const int pp = (py % wh) * ww + px % ww;
            const int64_t base = ((int64_t)(b * e.NH + h) * HDp + d) * e.vt_ld;
            const _Float16 h0 = to_half(v0), h1 = to_half(v1);
            const _Float16 l0 = (_Float16)(v0 - (float)h0), l1 = (_Float16)(v1 - (float)h1);
            const bool pair = gm + 1 < p.M && px + 1 < W && (px % ww) + 1 < ww && (pp & 1) == 0;
            if (pair) {
                const int64_t o = base + vt_slot(pp);
                *(uint32_t *)(e.vt + o) =
                    (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                if (e.vt_lo)
                    *(uint32_t *)(e.vt_lo + o) =
                        (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
            } else {
                const int64_t o = base + vt_slot(pp);
                e.vt[o] = h0;
                if (e.vt_lo) e.vt_lo[o] = l0;
                if (gm + 1 < p.M) {
                    const int pyb = (gm + 1) / W, pxb = (gm + 1) % W;
                    const int bb = (pyb / wh) * nwx + pxb / ww;
                    const int ppb = (pyb % wh) * ww + pxb % ww;
                    const int64_t ob = ((int64_t)(bb * e.NH + h) * HDp + d) * e.vt_ld + vt_slot(ppb);
                    e.vt[ob] = h1;
                    if (e.vt_lo) e.vt_lo[ob] = l1;
                }
            }
        }
    } else if constexpr (EPI == EPI_GELU) {
        // full 32-column blocks guaranteed by the launcher (N % 32 == 0)
        for (int ch = t; ch < BM * 4; ch += NT_) {
            const int row = ch >> 2, cc = ch & 3;
            const int gm = m0 + row;
            const int gn0 = n0 + cc * 32;
            if (gm >= p.M || gn0 >= p.N) continue;
            float v[32], bias[32];
            // the bias of the 32 columns is loaded up front: its loads are in
            // flight together instead of each behind the previous group's math
#pragma unroll
            for (int j = 0; j < 32; j += 4) {
                const float4 bb = *(const float4 *)(e.bias + gn0 + j);
                bias[j] = bb.x; bias[j + 1] = bb.y; bias[j + 2] = bb.z; bias[j + 3] = bb.w;
            }
#pragma unroll
            for (int j = 0; j < 32; j += 4) {
                const float4 x = *(const float4 *)(Ct + row * CLD + cc * 32 + j);
                v[j] = x.x; v[j + 1] = x.y; v[j + 2] = x.z; v[j + 3] = x.w;
            }
            if (e.gelu_tab) {
                // ggml_vec_gelu_f32 with GGML_GELU_FP16: x ≤ −10 → 0, x ≥ 10 → x,
                // else the table entry at fp16(x).  All 32 table indices are
                // formed before the first lookup, so the lookups are in flight
                // together (the fp16 rounding's asm fence would otherwise hold
                // each lookup behind the previous one's result).
                uint16_t idx[32];
#pragma unroll
                for (int j = 0; j < 32; j++) {
                    v[j] = __fadd_rn(v[j], bias[j]);
                    idx[j] = half_bits(v[j]);
                }
                uint16_t tv[32];
#pragma unroll
                for (int j = 0; j < 32; j++) tv[j] = e.gelu_tab[idx[j]];
#pragma unroll
                for (int j = 0; j < 32; j++) {
                    const float x = v[j], t = (float)__builtin_bit_cast(_Float16, tv[j]);
                    v[j] = x <= -10.f ? 0.f : (x >= 10.f ? x : t);
                }
            } else if (e.relu) {
                // ggml_relu: x > 0 ? x : 0
#pragma unroll
                for (int j = 0; j < 32; j++) {
                    const float x = __fadd_rn(v[j], bias[j]);
                    v[j] = x > 0.f ? x : 0.f;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 32; j++) v[j] = gelu_erf(__fadd_rn(v[j], bias[j]));
            }
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
            } else if (o.kind == A_F16X2) {
                // fp16 pairs: hi = fp16(v), lo = fp16(v − hi)
                _Float16 *dst = (_Float16 *)o.x + (int64_t)gm * o.ld + gn0;
                _Float16 *dlo = (_Float16 *)o.lo + (int64_t)gm * o.ld + gn0;
                uint32_t w[16], wl[16];
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const _Float16 h0 = to_half(v[2 * j]), h1 = to_half(v[2 * j + 1]);
                    w[j] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                    const _Float16 l0 = (_Float16)(v[2 * j] - (float)h0), l1 = (_Float16)(v[2 * j + 1] - (float)h1);
                    wl[j] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    ((uint4 *)dst)[j] = make_uint4(w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]);
                    ((uint4 *)dlo)[j] = make_uint4(wl[4 * j], wl[4 * j + 1], wl[4 * j + 2], wl[4 * j + 3]);
                }
            } else if (o.kind == A_F32) {
                float4 *dst = (float4 *)((float *)o.x + (int64_t)gm * o.ld + gn0);
#pragma unroll
                for (int j = 0; j < 8; j++) dst[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
            } else if (o.kind == A_F6) {
                quant_block32_f6(v, (uint64_t *)o.x, o.ld / 128, gm, gn0 / QK, o.d + scale_index(o.mp, gm, gn0 / QK));
            } else {
                const int64_t blk = scale_index(o.mp, gm, gn0 / QK);
                quant_block32(v, (int8_t *)o.x + (int64_t)gm * o.ld + gn0, o.d + blk,
                              o.kind == A_Q8_1 ? o.s + blk : nullptr);
            }
        }
    } else if constexpr (EPI == EPI_DECONV) {
        // 2×2 stride-2 transposed convolution: column (2·ky + kx)·Cout + co of
        // input pixel iy·W + ix goes to output pixel (2·iy + ky, 2·ix + kx),
        // channel co.  Lane ↔ 4 consecutive columns (Cout % 4 == 0, so the
        // four share one tap and one output row); + bias, optional gelu_erf,
        // into f32, fp16 or split-fp16 rows.
        const int f = t & 31;
        const int gn = n0 + 4 * f;
        if (gn >= p.N) return;
        const int q = gn / e.dc_cout, co = gn - q * e.dc_cout;
        const float4 bb = *(const float4 *)(e.bias + co);
        const float bj[4] = {bb.x, bb.y, bb.z, bb.w};
        const Act &o = e.out;
        for (int row = t >> 5; row < BM; row += NT_ / 32) {
            const int gm = m0 + row;
            if (gm >= p.M) break;
            const float4 x = *(const float4 *)(Ct + row * CLD + 4 * f);
            float v[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[j] = __fadd_rn(v[j], bj[j]);
                if (e.gelu) v[j] = gelu_erf(v[j]);
            }
            const int iy = gm / e.dc_w, ix = gm - iy * e.dc_w;
            const int64_t orow = (int64_t)(2 * iy + (q >> 1)) * (2 * e.dc_w) + 2 * ix + (q & 1);
            const int64_t i = orow * o.ld + co;
            if (o.kind == A_F32) {
                *(float4 *)((float *)o.x + i) = make_float4(v[0], v[1], v[2], v[3]);
                continue;
            }
            uint32_t w[2], wl[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const _Float16 h0 = to_half(v[2 * j]), h1 = to_half(v[2 * j + 1]);
                w[j] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                const _Float16 l0 = (_Float16)(v[2 * j] - (float)h0), l1 = (_Float16)(v[2 * j + 1] - (float)h1);
                wl[j] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
            }
            *(uint2 *)((_Float16 *)o.x + i) = make_uint2(w[0], w[1]);
            if (o.kind == A_F16X2) *(uint2 *)((_Float16 *)o.lo + i) = make_uint2(wl[0], wl[1]);
        }
    } else {
        // EPI_F32 / EPI_RESID / EPI_POS: lane ↔ 4 consecutive columns, so that one
        // wave store covers 2 rows × 512 contiguous bytes
        const int f = t & 31;
        const int gn = n0 + 4 * f;
        const bool vec = (p.N % 4) == 0 && gn + 3 < p.N;
        constexpr int RPT = BM / (NT_ / 32);  // rows per thread
        if constexpr (EPI == EPI_RESID) {
            if (vec) {
                // the bias, and every residual row of this thread, are loaded
                // before the first store: y and bias may alias as far as the
                // compiler knows, so a load placed after a store would wait
                // for that store
                const float4 bb = e.bias ? *(const float4 *)(e.bias + gn) : make_float4(0.f, 0.f, 0.f, 0.f);
                const float bj[4] = {bb.x, bb.y, bb.z, bb.w};
                float4 res[RPT];
#pragma unroll
                for (int k = 0; k < RPT; k++) {
                    const int gm = m0 + (t >> 5) + k * (NT_ / 32);
                    res[k] = gm < p.M ? *(const float4 *)(e.y + (int64_t)gm * e.ldy + gn)
                                      : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
                for (int k = 0; k < RPT; k++) {
                    const int row = (t >> 5) + k * (NT_ / 32), gm = m0 + row;
                    if (gm >= p.M) continue;
                    const float4 x = *(const float4 *)(Ct + row * CLD + 4 * f);
                    float v[4] = {x.x, x.y, x.z, x.w};
                    if (e.bias) {
#pragma unroll
                        for (int j = 0; j < 4; j++) v[j] = __fadd_rn(v[j], bj[j]);
                    }
                    *(float4 *)(e.y + (int64_t)gm * e.ldy + gn) =
                        make_float4(__fadd_rn(res[k].x, v[0]), __fadd_rn(res[k].y, v[1]),
                                    __fadd_rn(res[k].z, v[2]), __fadd_rn(res[k].w, v[3]));
                }
                return;
            }
        }
        for (int row = t >> 5; row < BM; row += NT_ / 32) {
            const int gm = m0 + row;
            if (gm >= p.M || gn >= p.N) continue;
            const float4 x = *(const float4 *)(Ct + row * CLD + 4 * f);
            float v[4] = {x.x, x.y, x.z, x.w};
            float *y = e.y + (int64_t)gm * e.ldy + gn;
            if constexpr (EPI == EPI_POS) {
                const int py = gm / e.grid, px = gm % e.grid;
                const float *pr = e.pos + ((int64_t)(py % e.pos_grid) * e.pos_grid + (px % e.pos_grid)) * p.N + gn;
                if (e.bias) {
#pragma unroll
                    for (int j = 0; j < 4; j++) v[j] = __fadd_rn(v[j], e.bias[gn + j]);
                }
#pragma unroll
                for (int j = 0; j < 4; j++) v[j] = __fadd_rn(v[j], pr[j]);
            } else {
                if (e.bias) {
#pragma unroll
                    for (int j = 0; j < 4; j++) v[j] = __fadd_rn(v[j], e.bias[gn + j]);
                }
            }
            if (vec) {
                if constexpr (EPI == EPI_RESID) {
                    const float4 o = *(const float4 *)y;
                    v[0] = __fadd_rn(o.x, v[0]);
                    v[1] = __fadd_rn(o.y, v[1]);
                    v[2] = __fadd_rn(o.z, v[2]);
                    v[3] = __fadd_rn(o.w, v[3]);
                }
                *(float4 *)y = make_float4(v[0], v[1], v[2], v[3]);
            } else {
                for (int j = 0; j < 4 && gn + j < p.N; j++) {
                    if constexpr (EPI == EPI_RESID) y[j] = __fadd_rn(y[j], v[j]);
                    else y[j] = v[j];
                }
            }
        }
    }
}

template <int WK, int EPI, int BM, int WAVES>
__global__ __launch_bounds__(64 * WAVES, WAVES == 4 ? 3 : 256 / BM) void k_gemm(GemmParams p) {
    using C = Cfg<WK, BM, WAVES>;
    constexpr int MT = C::MT, NT = C::NT, NBUF = C::NBUF;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[C::LDS];

    // ---- tile of this work-group (and its K range when split) ----
    const int per = gridDim.x >> 3;
    const int logical0 = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (logical0 >= p.ntiles * p.ksplit) return;
    const int kpart = logical0 % p.ksplit, logical = logical0 / p.ksplit;
    constexpr int GROUP = 8;
    const int group = logical / (GROUP * p.tiles_n);
    const int first_m = group * GROUP;
    const int gsz = min(p.tiles_m - first_m, GROUP);
    const int rem = logical - group * GROUP * p.tiles_n;
    const int tm = first_m + rem % gsz, tn = rem / gsz;
    const int m0 = tm * BM, n0 = tn * BN;

    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int lane = t & 63;
    const int wm = wave / C::WN, wn = wave % C::WN;
    const int lr = lane & 31, lh = lane >> 5;

    // ---- per-lane DMA sources: lane writes LDS bytes [16·lane, 16·lane+16) of
    // a 1 KB run = 8 rows, i.e. slot lane & 7 of row lane >> 3 of the run; it
    // fetches the chunk that belongs there
    // Sources are byte offsets into buffer resources (A: M rows of a_ld
    // bytes, B: Np columns of b_ld bytes; the launcher keeps both under 2^31):
    // the stage lives in the uniform soffset, so the DMA of a stage costs no
    // vector ALU work.
    const int dma_row = lane >> 3;
    int a_vo[C::NA], a_cofs[C::NA], b_vo[C::NB];
    // split: a 1 KB run is 16 rows of 64 bytes of one plane (runs of the hi
    // plane first, then the lo plane's, so the run's LDS place is the same
    // formula); lane writes slot lane & 3 of row lane >> 2
    constexpr int AR = BM / 16, BR = BN / 16;  // split: runs per plane
#pragma unroll
    for (int j = 0; j < C::NA; j++) {
        if constexpr (C::split) {
            const int row = 16 * ((wave * C::NA + j) % AR) + (lane >> 2);
            const int gm = min(m0 + row, p.M - 1);
            a_cofs[j] = ((lane & 3) ^ swz64(row)) << 4;
            a_vo[j] = gm * (int)p.a_ld + a_cofs[j];
        } else {
            const int row = 8 * (wave * C::NA + j) + dma_row;
            const int gm = min(m0 + row, p.M - 1);
            a_cofs[j] = ((lane & 7) ^ swz(row)) << 4;
            a_vo[j] = gm * (int)p.a_ld + a_cofs[j];
        }
    }
    const int a_kb = (int)p.a_kbytes, a_last = a_kb - 16;
#pragma unroll
    for (int j = 0; j < C::NB; j++) {
        if constexpr (C::split) {
            const int col = 16 * ((wave * C::NB + j) % BR) + (lane >> 2);
            b_vo[j] = (n0 + col) * (int)p.b_ld + (((lane & 3) ^ swz64(col)) << 4);
        } else {
            const int col = 8 * (wave * C::NB + j) + dma_row;
            b_vo[j] = (n0 + col) * (int)p.b_ld + (((lane & 7) ^ swz(col)) << 4);
        }
    }
    const uint8_t *s_src[C::NS > 0 ? C::NS : 1];
    int64_t s_step[C::NS > 0 ? C::NS : 1];
    int s_dst[C::NS > 0 ? C::NS : 1];
    if constexpr (C::quant) {
#pragma unroll
        for (int j = 0; j < C::NS; j++) {
            // scale run k (256 B); waves past the last run repeat an earlier one
            // (identical bytes to the identical place)
            const int k = (wave + WAVES * j) % C::SC;
            int o = k * 256;
            s_dst[j] = C::OFF_SC + o;
            if (o < BM * 8) {
                s_src[j] = p.a_d + ((int64_t)m0 * 4) * 2 + o;
                s_step[j] = p.a_mp * 8;
            } else if ((o -= BM * 8) < BN * 8) {
                s_src[j] = p.b_d + ((int64_t)n0 * 4) * 2 + o;
                s_step[j] = p.b_np * 8;
            } else if ((o -= BN * 8) < BM * 8) {
                s_src[j] = p.a_s + ((int64_t)m0 * 4) * 2 + o;
                s_step[j] = p.a_mp * 8;
            } else {
                o -= BM * 8;
                s_src[j] = p.b_m + ((int64_t)n0 * 4) * 2 + o;
                s_step[j] = p.b_np * 8;
            }
            s_src[j] += lane * 4;
        }
    }

    // stage s into ring buffer `buf`
    auto issue = [&](int s, int buf) {
        uint8_t *L = lds + buf * C::STAGE;
        if constexpr (C::split) {
            // 32 K (64 bytes) of each plane per stage; the plane is uniform per run
            constexpr int SB = 64;
#pragma unroll
            for (int j = 0; j < C::NA; j++) {
                const uint8_t *base = (wave * C::NA + j) < AR ? p.a : p.a_lo;
                const int vo = (s + 1) * SB <= a_kb ? a_vo[j] + s * SB : min(a_vo[j] + s * SB, a_vo[j] - a_cofs[j] + a_last);
                dma16_buf(base, p.a_rec, L + C::OFF_A + (wave * C::NA + j) * 1024, vo, 0);
            }
#pragma unroll
            for (int j = 0; j < C::NB; j++) {
                const uint8_t *base = (wave * C::NB + j) < BR ? p.b : p.b_lo;
                dma16_buf(base, p.b_rec, L + C::OFF_B + (wave * C::NB + j) * 1024, b_vo[j], s * SB);
            }
            return;
        }
        if ((s + 1) * ROWB <= a_kb) {
#pragma unroll
            for (int j = 0; j < C::NA; j++)
                dma16_buf(p.a, p.a_rec, L + C::OFF_A + (wave * C::NA + j) * 1024, a_vo[j], s * ROWB);
        } else {
            // the stage that reaches past K re-reads the row's last chunk
            // (finite data against zero weight columns)
#pragma unroll
            for (int j = 0; j < C::NA; j++)
                dma16_buf(p.a, p.a_rec, L + C::OFF_A + (wave * C::NA + j) * 1024,
                          min(a_vo[j] + s * ROWB, a_vo[j] - a_cofs[j] + a_last), 0);
        }
#pragma unroll
        for (int j = 0; j < C::NB; j++)
            dma16_buf(p.b, p.b_rec, L + C::OFF_B + (wave * C::NB + j) * 1024, b_vo[j], s * ROWB);
        if constexpr (C::quant) {
#pragma unroll
            for (int j = 0; j < C::NS; j++)
                __builtin_amdgcn_global_load_lds((const void *)(s_src[j] + s * s_step[j]),
                                                 LDS_PTR(L + s_dst[j]), 4, 0, 0);
        }
    };

    // ---- per-lane operand offsets ----
    const int xr = swz(lr);  // tile rows start at multiples of 32
    int a_off[MT], ad_off[MT];
#pragma unroll
    for (int i = 0; i < MT; i++) {
        const int r = wm * (32 * MT) + 32 * i + lr;
        a_off[i] = C::OFF_A + r * ROWB;
        ad_off[i] = r * 8;
    }
    int b_off[NT], bd_off[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int bcol = wn * (32 * NT) + 32 * n + lr;
        b_off[n] = C::OFF_B + bcol * ROWB;
        bd_off[n] = bcol * 8;
    }
    int cofs[4];
#pragma unroll
    for (int q = 0; q < 4; q++) cofs[q] = ((2 * q + lh) ^ xr) << 4;
    if constexpr (C::split) {
        // 64-byte rows; tile rows start at multiples of 32, so the swizzle of
        // row base + lr is swz64(lr); K = 16 step ks reads chunk 2·ks + lh
#pragma unroll
        for (int i = 0; i < MT; i++) a_off[i] = C::OFF_A + (wm * (32 * MT) + 32 * i + lr) * 64;
#pragma unroll
        for (int n = 0; n < NT; n++) b_off[n] = C::OFF_B + (wn * (32 * NT) + 32 * n + lr) * 64;
#pragma unroll
        for (int q = 0; q < 2; q++) cofs[q] = ((2 * q + lh) ^ swz64(lr)) << 4;
    }

    v16f acc[MT][NT], accm[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int r = 0; r < 16; r++) { acc[i][n][r] = 0.f; accm[i][n][r] = 0.f; }

    // one quant block step: integer sums and scale products of MT × NT tiles
    struct QFrag {
        v4i a[MT], b[NT];
        uint32_t da[MT], db[NT];
    };
    auto qread = [&](const uint8_t *L, int blk, QFrag &f) {
#pragma unroll
        for (int i = 0; i < MT; i++) {
            f.a[i] = *(const v4i *)(L + a_off[i] + cofs[blk]);
            f.da[i] = *(const uint16_t *)(L + C::OFF_AD + ad_off[i] + 2 * blk);
        }
#pragma unroll
        for (int n = 0; n < NT; n++) {
            f.b[n] = *(const v4i *)(L + b_off[n] + cofs[blk]);
            f.db[n] = *(const uint16_t *)(L + C::OFF_BD + bd_off[n] + 2 * blk);
        }
    };
    auto qmma = [&](const QFrag &f, v16i (&S)[MT][NT], v16f (&Cs)[MT][NT]) {
        const v16i zi = {};
        const v16f zf = {};
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const v2u hb = {f.db[n], 0u};
#pragma unroll
            for (int i = 0; i < MT; i++) {
                const v2u ha = {f.da[i], 0u};
                S[i][n] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[i], f.b[n], zi, 0, 0, 0);
                Cs[i][n] = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, ha), __builtin_bit_cast(v4h, hb),
                                                                zf, 0, 0, 0);
            }
        }
    };
    auto qvalu = [&](const v16i (&S)[MT][NT], const v16f (&Cs)[MT][NT]) {
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int i = 0; i < MT; i++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    acc[i][n][r] = __builtin_fmaf((float)S[i][n][r], Cs[i][n][r], acc[i][n][r]);
    };

    auto compute = [&](int buf) {
        const uint8_t *L = lds + buf * C::STAGE;
        if constexpr (C::quant) {
            if constexpr (C::PIPE) {
                QFrag f0, f1;
                v16i S0[MT][NT], S1[MT][NT];
                v16f C0[MT][NT], C1[MT][NT];
                qread(L, 0, f0);
                qread(L, 1, f1);
                qmma(f0, S0, C0);
                qread(L, 2, f0);
                qmma(f1, S1, C1);
                qvalu(S0, C0);
                qread(L, 3, f1);
                qmma(f0, S0, C0);
                qvalu(S1, C1);
                qmma(f1, S1, C1);
                qvalu(S0, C0);
                qvalu(S1, C1);
            } else {
#pragma unroll
                for (int blk = 0; blk < 4; blk++) {
                    QFrag f;
                    v16i S[MT][NT];
                    v16f Cs[MT][NT];
                    qread(L, blk, f);
                    qmma(f, S, Cs);
                    qvalu(S, Cs);
                }
            }
            if constexpr (C::q41) {
                // Σ_b s_x[m][b]·m_w[n][b] over the stage's 4 blocks, doubled like
                // the scale products (both lane halves carry the values)
#pragma unroll
                for (int n = 0; n < NT; n++) {
                    const uint2 mb = lds_u2(L + C::OFF_BMIN + bd_off[n]);
                    const v2u hb = {mb.x, mb.y};
#pragma unroll
                    for (int i = 0; i < MT; i++) {
                        const uint2 sa = lds_u2(L + C::OFF_AS + ad_off[i]);
                        const v2u ha = {sa.x, sa.y};
                        accm[i][n] = __builtin_amdgcn_mfma_f32_32x32x8f16(
                            __builtin_bit_cast(v4h, ha), __builtin_bit_cast(v4h, hb), accm[i][n], 0, 0, 0);
                    }
                }
            }
        } else if constexpr (C::split) {
            // x·w = (xh + xl)(wh + wl) ≈ xh·wh + xh·wl + xl·wh: each product
            // exact in fp32 (the dropped xl·wl is ~2^-22 relative)
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                v8h bh[NT], bl[NT], ah[MT], al[MT];
#pragma unroll
                for (int n = 0; n < NT; n++) {
                    bh[n] = *(const v8h *)(L + b_off[n] + cofs[ks]);
                    bl[n] = *(const v8h *)(L + b_off[n] + BN * 64 + cofs[ks]);
                }
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    ah[i] = *(const v8h *)(L + a_off[i] + cofs[ks]);
                    al[i] = *(const v8h *)(L + a_off[i] + BM * 64 + cofs[ks]);
                }
#pragma unroll
                for (int i = 0; i < MT; i++)
#pragma unroll
                    for (int n = 0; n < NT; n++)
                        acc[i][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bh[n], acc[i][n], 0, 0, 0);
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
        } else if constexpr (WK == WK_F16) {
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                v8h bv[NT];
#pragma unroll
                for (int n = 0; n < NT; n++) bv[n] = *(const v8h *)(L + b_off[n] + cofs[ks]);
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    const v8h av = *(const v8h *)(L + a_off[i] + cofs[ks]);
#pragma unroll
                    for (int n = 0; n < NT; n++)
                        acc[i][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv[n], acc[i][n], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < 16; ks++) {
                const int o = ((((ks >> 1) ^ xr)) << 4) + ((2 * (ks & 1) + lh) << 2);
                float bv[NT];
#pragma unroll
                for (int n = 0; n < NT; n++) bv[n] = *(const float *)(L + b_off[n] + o);
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    const float av = *(const float *)(L + a_off[i] + o);
#pragma unroll
                    for (int n = 0; n < NT; n++)
                        acc[i][n] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv[n], acc[i][n], 0, 0, 0);
                }
            }
        }
    };

    // ---- main loop over stages s0 .. s1−1: stage s+NBUF−1 in flight while
    // stage s is consumed ----
    const int kper = (p.nstages + p.ksplit - 1) / p.ksplit;
    const int s0 = kpart * kper, s1 = min(p.nstages, s0 + kper);
    if constexpr (NBUF == 3) {
        issue(s0, 0);
        if (s0 + 1 < s1) issue(s0 + 1, 1);
        for (int s = s0; s < s1; s++) {
            if (s + 1 < s1) wait_and_barrier<C::NLOAD>();
            else wait_and_barrier<0>();
            if (s + 2 < s1) issue(s + 2, (s + 2 - s0) % NBUF);
            compute((s - s0) % NBUF);
        }
    } else {
        issue(s0, 0);
        for (int s = s0; s < s1; s++) {
            wait_and_barrier<0>();  // stage s landed; every wave is done with stage s−1
            if (s + 1 < s1) issue(s + 1, (s + 1 - s0) & 1);
            compute((s - s0) & 1);
        }
    }
    wait_and_barrier<0>();

    // ---- stage the fp32 tile in LDS ----
    float *Ct = (float *)lds;
    constexpr float kScale = C::quant ? 0.5f : 1.0f;  // remove the doubled scale products
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = wm * (32 * MT) + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
                float v = acc[i][n][r];
                if constexpr (C::q41) v += accm[i][n][r];
                Ct[row * CLD + wn * (32 * NT) + 32 * n + lr] = v * (C::split ? p.alpha : kScale);
            }
    __syncthreads();

    if constexpr (EPI == EPI_F32 || EPI == EPI_RESID) {
        if (p.ksplit > 1) {
            // raw partial tile of this K range; the reduction adds bias / residual
            GemmParams q = p;
            q.e.y = p.part + (int64_t)kpart * p.M * p.N;
            q.e.ldy = p.N;
            q.e.bias = nullptr;
            epilogue<EPI_F32, BM, C::NTH>(q, Ct, m0, n0, t);
            return;
        }
    }
    epilogue<EPI, BM, C::NTH>(p, Ct, m0, n0, t);
}

// ---- Q4_0 weights × A_F6 activations --------------------------------------
// The same tile, epilogues and scale products as k_gemm, with the integer
// block sums formed on the fp6 MFMA instead of the int8 one:
// v_mfma_scale_f32_32x32x64_f8f6f4 with E3M2 operands takes K = 64 as two
// halves of 32 (lanes 0-31 and 32-63), each with its own power-of-two scale.
// The activation half carries h (scale 16) and l (scale 1) of q = 16·h + l,
// the weight half carries the Q4_0 code twice, so one instruction returns
//     16·Σ h·qw + Σ l·qw = Σ_{k∈b} qx·qw = S_b
// exactly (integers below 2^24) and already in fp32: the per-block rescale is
// one FMA per element instead of a convert and an FMA, and the fp6 MFMA
// issues at about the int8 one's rate (gfx950 runs fp6 at twice the fp8 /
// int8 rate, so K = 64 of fp6 costs what K = 32 of int8 does).
// Operands stream as they lie in memory: a tile row's stage of A_F6 (12 KB)
// and a tile column's stage of the fp6 weight copy (12 KB) are contiguous,
// laid out so that the 32 rows (columns) of one operand read are 256
// contiguous bytes of LDS.
template <int EPI>
__global__ __launch_bounds__(256, 3) void k_gemm_f6(GemmParams p) {
    constexpr int BM = 64, NTH = 256, WN = 2, NT = 2;
    constexpr int OFF_A = 0, OFF_B = 12288, OFF_AD = 24576, OFF_BD = OFF_AD + BM * 8;
    constexpr int STAGE = OFF_BD + BN * 8;  // 26112
    constexpr int LDSZ = 2 * STAGE > BM * CLD * 4 ? 2 * STAGE : BM * CLD * 4;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDSZ];

    const int per = gridDim.x >> 3;
    const int logical0 = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (logical0 >= p.ntiles * p.ksplit) return;
    const int kpart = logical0 % p.ksplit, logical = logical0 / p.ksplit;
    constexpr int GROUP = 8;
    const int group = logical / (GROUP * p.tiles_n);
    const int first_m = group * GROUP;
    const int gsz = min(p.tiles_m - first_m, GROUP);
    const int rem = logical - group * GROUP * p.tiles_n;
    const int tm = first_m + rem % gsz, tn = rem / gsz;
    const int m0 = tm * BM, n0 = tn * BN;

    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int lane = t & 63;
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, lh = lane >> 5;

    // DMA: wave w copies 1 KB runs 3w .. 3w+2 of the stage's A and of its B,
    // and 256-byte scale runs w and w + 4 (A: runs 0-1, rows m0..; B: runs
    // 2-5, columns n0..)
    const int a_tile = tm * p.nstages * 12288, b_tile = tn * p.nstages * 12288;
    const int a_drec = p.nstages * (int)p.a_mp * 8, b_drec = p.nstages * (int)p.b_np * 8;
    int s_n = 0;
    int s_voff[2], s_dst[2], s_step[2];
    bool s_a[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int k = wave + 4 * j;
        if (k >= 6) break;
        s_n++;
        s_a[j] = k < 2;
        if (k < 2) {
            s_voff[j] = m0 * 8 + k * 256 + lane * 4;
            s_step[j] = (int)p.a_mp * 8;
            s_dst[j] = OFF_AD + k * 256;
        } else {
            s_voff[j] = n0 * 8 + (k - 2) * 256 + lane * 4;
            s_step[j] = (int)p.b_np * 8;
            s_dst[j] = OFF_BD + (k - 2) * 256;
        }
    }
    auto issue = [&](int s, int buf) {
        uint8_t *L = lds + buf * STAGE;
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const int run = 3 * wave + j;
            dma16_buf(p.a, p.a_rec, L + OFF_A + run * 1024, a_tile + run * 1024 + lane * 16, s * 12288);
            dma16_buf(p.b, p.b_rec, L + OFF_B + run * 1024, b_tile + run * 1024 + lane * 16, s * 12288);
        }
#pragma unroll
        for (int j = 0; j < 2; j++)
            if (j < s_n) {
                // the stage offset is wave-uniform: keep it in a scalar register
                const int so = __builtin_amdgcn_readfirstlane(s * s_step[j]);
                if (s_a[j]) dma4_buf(p.a_d, a_drec, L + s_dst[j], s_voff[j], so);
                else dma4_buf(p.b_d, b_drec, L + s_dst[j], s_voff[j], so);
            }
    };

    // per-lane LDS operand offsets: A row wm·32 + lr, part lh; B column
    // wn·64 + 32n + lr (both lane halves read the same B words)
    const int a_row = wm * 32 + lr;
    const int a_off = OFF_A + lh * 3 * 512 + a_row * 8;
    const int ad_off = OFF_AD + a_row * 8;
    int b_off[NT], bd_off[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int col = wn * 64 + 32 * n + lr;
        b_off[n] = OFF_B + col * 8;
        bd_off[n] = OFF_BD + col * 8;
    }
    const int a_scale = lh ? 127 : 131;  // E8M0: 2^0 for l, 2^4 for h

    v16f acc[NT];
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[n][r] = 0.f;

    // scale products on the fp16 MFMA (32×32×8): the A operand carries the
    // stage's four row scales in K slots 0-3 (one 8-byte read per stage; the
    // other lane half holds slots 4-7, the same values), the B operand of
    // block b only its column scale in slots b and 4 + b, so the product is
    // 2·dx[b]·dw[b]
    v2u ha = {0u, 0u};
    struct Ops {
        v8i a, b[NT];
    };
    auto load_ops = [&](const uint8_t *L, int blk, Ops &o) {
        {
            const uint64_t *q = (const uint64_t *)(L + a_off + blk * 6 * 512);
            const v4u64 w = {q[0], q[64], q[128], 0ull};
            o.a = __builtin_bit_cast(v8i, w);
        }
#pragma unroll
        for (int n = 0; n < NT; n++) {
            __asm__ volatile("" ::: "memory");
            const uint64_t *q = (const uint64_t *)(L + b_off[n] + blk * 3 * 1024);
            const v4u64 w = {q[0], q[128], q[256], 0ull};
            o.b[n] = __builtin_bit_cast(v8i, w);
        }
    };
    auto compute = [&](int buf) {
        const uint8_t *L = lds + buf * STAGE;
        {
            const uint2 sa = lds_u2(L + ad_off);
            ha[0] = sa.x;
            ha[1] = sa.y;
        }
        uint2 sb[NT];
#pragma unroll
        for (int n = 0; n < NT; n++) sb[n] = lds_u2(L + bd_off[n]);
#pragma unroll
        for (int blk = 0; blk < 4; blk++) {
            Ops cur;
            load_ops(L, blk, cur);
            const v16f zf = {};
            v16f S[NT], Cs[NT];
#pragma unroll
            for (int n = 0; n < NT; n++) {
                const uint32_t w = blk < 2 ? sb[n].x : sb[n].y;
                const uint32_t m = (blk & 1) ? (w & 0xFFFF0000u) : (w & 0xFFFFu);
                const v2u hb = blk < 2 ? v2u{m, 0u} : v2u{0u, m};
                S[n] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(cur.a, cur.b[n], zf, 3, 3, 0, a_scale, 0, 127);
                Cs[n] = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, ha), __builtin_bit_cast(v4h, hb),
                                                             zf, 0, 0, 0);
            }
#pragma unroll
            for (int n = 0; n < NT; n++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[n][r] = __builtin_fmaf(S[n][r], Cs[n][r], acc[n][r]);
        }
    };

    const int kper = (p.nstages + p.ksplit - 1) / p.ksplit;
    const int s0 = kpart * kper, s1 = min(p.nstages, s0 + kper);
    issue(s0, 0);
    for (int s = s0; s < s1; s++) {
        wait_and_barrier<0>();
        if (s + 1 < s1) issue(s + 1, (s + 1 - s0) & 1);
        compute((s - s0) & 1);
    }
    wait_and_barrier<0>();

    float *Ct = (float *)lds;
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = wm * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
            Ct[row * CLD + wn * 64 + 32 * n + lr] = acc[n][r] * 0.5f;  // the doubled scale products
        }
    __syncthreads();
    if constexpr (EPI == EPI_F32 || EPI == EPI_RESID) {
        if (p.ksplit > 1) {
            GemmParams q = p;
            q.e.y = p.part + (int64_t)kpart * p.M * p.N;
            q.e.ldy = p.N;
            q.e.bias = nullptr;
            epilogue<EPI_F32, BM, NTH>(q, Ct, m0, n0, t);
            return;
        }
    }
    epilogue<EPI, BM, NTH>(p, Ct, m0, n0, t);
}

// y = Σ_k part[k] (+ bias) for EPI_F32, y += Σ_k part[k] (+ bias) for
// EPI_RESID, the ranges summed in order (the result does not depend on the
// schedule).  One thread per 4 consecutive outputs of a row.
__global__ __launch_bounds__(256) void k_gemm_reduce(const float *__restrict__ part, int ks, int M, int N,
                                                     const float *__restrict__ bias, float *y, int64_t ldy,
                                                     int resid) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    const uint32_t n4 = (uint32_t)N / 4;
    if (i >= (uint32_t)M * n4) return;
    const uint32_t r = i / n4;
    const int c = (int)(i - r * n4) * 4;
    const int64_t plane = (int64_t)M * N;
    float4 v = *(const float4 *)(part + (int64_t)r * N + c);
    for (int k = 1; k < ks; k++) {
        const float4 w = *(const float4 *)(part + k * plane + (int64_t)r * N + c);
        v.x = __fadd_rn(v.x, w.x);
        v.y = __fadd_rn(v.y, w.y);
        v.z = __fadd_rn(v.z, w.z);
        v.w = __fadd_rn(v.w, w.w);
    }
    if (bias) {
        v.x = __fadd_rn(v.x, bias[c]);
        v.y = __fadd_rn(v.y, bias[c + 1]);
        v.z = __fadd_rn(v.z, bias[c + 2]);
        v.w = __fadd_rn(v.w, bias[c + 3]);
    }
    float4 *o = (float4 *)(y + (int64_t)r * ldy + c);
    if (resid) {
        const float4 x = *o;
        v = make_float4(__fadd_rn(x.x, v.x), __fadd_rn(x.y, v.y), __fadd_rn(x.z, v.z), __fadd_rn(x.w, v.w));
    }
    *o = v;
}

template <int WK, int EPI, int BM, int WAVES>
hipError_t launch_one(const GemmParams &p, hipStream_t st) {
    const int grid = ((p.ntiles * p.ksplit + 7) / 8) * 8;
    hipLaunchKernelGGL((k_gemm<WK, EPI, BM, WAVES>), dim3(grid), dim3(64 * WAVES), 0, st, p);
    return hipGetLastError();
}

template <int WK, int WAVES>
hipError_t dispatch_epi(Epi epi, const GemmParams &p, hipStream_t st) {
    switch (epi) {
        case EPI_F32: return launch_one<WK, EPI_F32, 64, WAVES>(p, st);
        case EPI_RESID: return launch_one<WK, EPI_RESID, 64, WAVES>(p, st);
        case EPI_POS: return launch_one<WK, EPI_POS, 64, WAVES>(p, st);
        case EPI_GELU: return launch_one<WK, EPI_GELU, 64, WAVES>(p, st);
        case EPI_QKV: return launch_one<WK, EPI_QKV, 64, WAVES>(p, st);
        case EPI_HQKV: return launch_one<WK, EPI_HQKV, 64, WAVES>(p, st);
        case EPI_DECONV:
            // the neck's transposed convolutions (fp16 kernels)
            if constexpr (WK == WK_F16) return launch_one<WK, EPI_DECONV, 64, WAVES>(p, st);
            break;
        default: break;  // EPI_ACT belongs to k_conv
    }
    return hipErrorInvalidValue;
}

// fp16 products with work-groups to spare and a long K run on 128 × 128 tiles
// (each wave 64 × 64: every operand read feeds two MFMAs), two work-groups per
// CU.  fc1 at 5184 rows (1517 such tiles): 85-92 → 73-78 µs; in the banded
// ViT frame (518 per band) and on short K (Hiera's first stages) the 64-row
// tiles' three work-groups per CU measured as fast or faster.
constexpr int64_t F16_WIDE_MIN_TILES = 1200;
constexpr int64_t F16_WIDE_MIN_K = 512;

template <int WK>
hipError_t dispatch_waves(Epi epi, GemmParams &p, hipStream_t st) {
    if constexpr (WK == WK_F16) {
        const int64_t t128 = (int64_t)(p.M + 127) / 128 * p.tiles_n;
        if (p.ksplit == 1 && t128 >= F16_WIDE_MIN_TILES && p.a_kbytes >= 2 * F16_WIDE_MIN_K &&
            (epi == EPI_F32 || epi == EPI_GELU || epi == EPI_QKV || epi == EPI_HQKV || epi == EPI_DECONV)) {
            p.tiles_m = (p.M + 127) / 128;
            p.ntiles = p.tiles_m * p.tiles_n;
            switch (epi) {
                case EPI_F32: return launch_one<WK, EPI_F32, 128, 4>(p, st);
                case EPI_GELU: return launch_one<WK, EPI_GELU, 128, 4>(p, st);
                case EPI_QKV: return launch_one<WK, EPI_QKV, 128, 4>(p, st);
                case EPI_DECONV: return launch_one<WK, EPI_DECONV, 128, 4>(p, st);
                default: return launch_one<WK, EPI_HQKV, 128, 4>(p, st);
            }
        }
    }
    constexpr int BM = 64;
    p.tiles_m = (p.M + BM - 1) / BM;
    p.ntiles = p.tiles_m * p.tiles_n;
    // 4-wave work-groups (three per CU, 4-12% faster on the SAM 3 shapes)
    // except for Q4_1, whose extra minimum term needs more registers than
    // three work-groups per CU leave
    if constexpr (WK == WK_Q4_1) return dispatch_epi<WK, 8>(epi, p, st);
    else return dispatch_epi<WK, 4>(epi, p, st);
}

// K ranges for a product that leaves CUs idle: fewer 64 × 128 tiles than CUs
// and at least 8 stages of K; about 512 work-groups, each range at least four
// stages.
int splitk_of(const Weight &w, int64_t M) {
    const int esize = (w.kind == WK_F16) ? 2 : (w.kind == WK_F32 ? 4 : 1);
    const int64_t ns = w.kind == WK_F16X3 ? w.Kp / 32 : w.Kp * esize / 128, tiles = (M + 63) / 64 * (w.Np / BN);
    if (tiles >= 256 || ns < 8 || w.N % 4 != 0) return 1;
    int64_t ks = std::min<int64_t>((512 + tiles - 1) / tiles, ns / 4);
    const int64_t per = (ns + ks - 1) / ks;
    return (int)((ns + per - 1) / per);
}

}  // namespace

int64_t gemm_splitk_floats(const Weight &w, int64_t M) {
    const int ks = splitk_of(w, M);
    return ks > 1 ? (int64_t)ks * M * w.N : 0;
}

hipError_t launch_gemm(const Weight &w, const Act &a, int64_t M, Epi epi, const EpiArgs &ea,
                       hipStream_t st) {
    if (M <= 0) return hipSuccess;
    GemmParams p{};
    const bool split = w.kind == WK_F16X3;
    // split: fp16 hi / lo planes of the same row layout on both sides, rows
    // whole 16-byte chunks
    if (split && (a.kind != A_F16X2 || !a.lo || !w.lo || w.Kp % 64 != 0 || w.K % 8 != 0)) return hipErrorInvalidValue;
    const int esize = (w.kind == WK_F16 || split) ? 2 : (w.kind == WK_F32 ? 4 : 1);
    p.a = (const uint8_t *)a.x;
    p.a_lo = (const uint8_t *)a.lo;
    p.b_lo = (const uint8_t *)w.lo;
    p.alpha = w.alpha;
    p.a_d = (const uint8_t *)a.d;
    p.a_s = (const uint8_t *)a.s;
    p.a_ld = a.ld * esize;
    p.a_kbytes = w.K * esize;
    p.a_mp = a.mp;
    p.b = (const uint8_t *)w.q;
    p.b_d = (const uint8_t *)w.d;
    p.b_m = (const uint8_t *)w.m;
    p.b_ld = w.Kp * esize;
    p.b_np = w.Np;
    // buffer-load reach: A rows [0, M), B columns [0, Np), byte offsets below 2^31
    if ((int64_t)M * p.a_ld > INT32_MAX || (int64_t)w.Np * p.b_ld > INT32_MAX) return hipErrorInvalidValue;
    p.a_rec = (int)(M * p.a_ld);
    p.b_rec = (int)(w.Np * p.b_ld);
    p.M = (int)M;
    p.N = (int)w.N;
    p.ksplit = 1;
    if ((epi == EPI_F32 || epi == EPI_RESID) && ea.ws && ea.ldy % 4 == 0) {
        const int ks = splitk_of(w, M);
        if (ks > 1 && (int64_t)ks * M * w.N <= ea.ws_cap) {
            p.ksplit = ks;
            p.part = ea.ws;
        }
    }
    p.nstages = (int)(w.Kp / (split ? 32 : stage_k(w.kind)));
    p.tiles_n = (int)(w.Np / BN);
    p.e = ea;
    if (epi == EPI_HQKV) {
        // 8-column units stay inside one head; Q/K rows are 16-byte aligned
        if (ea.E <= 0 || w.N != 3LL * ea.E || ea.HD <= 0 || ea.HD % 8 != 0 || ea.E % ea.HD != 0 ||
            ea.hdp < ea.HD || ea.hdp % 8 != 0 || ea.NH * ea.HD != ea.E || ea.grid <= 0 || ea.grid_h <= 0 ||
            (int64_t)ea.grid * ea.grid_h != M || ea.window < 0 || !ea.bias || !ea.k || !ea.vt || ea.vt_ld <= 0 ||
            (ea.qpool ? (!ea.y || ea.ldy < ea.E) : !ea.q))
            return hipErrorInvalidValue;
    }
    if (epi == EPI_GELU && ea.out.kind == A_F16X2 &&
        (!ea.out.lo || ea.out.ld % 8 != 0 || (uintptr_t)ea.out.x % 16 != 0 || (uintptr_t)ea.out.lo % 16 != 0))
        return hipErrorInvalidValue;  // whole 16-byte stores of both planes
    if (epi == EPI_DECONV) {
        // fp16 kernels on fp16 rows, four taps of Cout columns, whole input rows
        const Act &o = ea.out;
        if (w.kind != WK_F16 || a.kind != A_F16 || ea.dc_w <= 0 || ea.dc_cout <= 0 || ea.dc_cout % 4 != 0 ||
            w.N != 4LL * ea.dc_cout || M % ea.dc_w != 0 || !ea.bias || !o.x || o.ld % 4 != 0 || o.ld < ea.dc_cout ||
            (o.kind != A_F16 && o.kind != A_F16X2 && o.kind != A_F32) || (o.kind == A_F16X2 && !o.lo))
            return hipErrorInvalidValue;
    }
    if (a.kind == A_F6) {
        // Q4_0 weights against fp6 activations (k_gemm_f6)
        if (w.kind != WK_Q4_0 || !w.f6 || w.Kp % 128 != 0 || a.ld != w.Kp || !a.d) return hipErrorInvalidValue;
        p.b = (const uint8_t *)w.f6;
        p.nstages = (int)(w.Kp / 128);
        p.tiles_m = (int)((M + 63) / 64);
        p.ntiles = p.tiles_m * p.tiles_n;
        const int64_t arec = (int64_t)p.tiles_m * p.nstages * 12288, brec = (int64_t)p.tiles_n * p.nstages * 12288;
        if (arec > INT32_MAX || brec > INT32_MAX || (int64_t)p.nstages * a.mp * 8 > INT32_MAX ||
            (int64_t)p.nstages * w.Np * 8 > INT32_MAX)
            return hipErrorInvalidValue;
        p.a_rec = (int)arec;
        p.b_rec = (int)brec;
        const int grid = ((p.ntiles * p.ksplit + 7) / 8) * 8;
        switch (epi) {
            case EPI_F32: hipLaunchKernelGGL(k_gemm_f6<EPI_F32>, dim3(grid), dim3(256), 0, st, p); break;
            case EPI_RESID: hipLaunchKernelGGL(k_gemm_f6<EPI_RESID>, dim3(grid), dim3(256), 0, st, p); break;
            case EPI_GELU: hipLaunchKernelGGL(k_gemm_f6<EPI_GELU>, dim3(grid), dim3(256), 0, st, p); break;
            case EPI_QKV: hipLaunchKernelGGL(k_gemm_f6<EPI_QKV>, dim3(grid), dim3(256), 0, st, p); break;
            default: return hipErrorInvalidValue;
        }
        hipError_t e = hipGetLastError();
        if (e == hipSuccess && p.ksplit > 1) {
            const int64_t n = M * (w.N / 4);
            hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p.part, p.ksplit,
                               (int)M, (int)w.N, ea.bias, ea.y, ea.ldy, epi == EPI_RESID ? 1 : 0);
            e = hipGetLastError();
        }
        return e;
    }
    // 64-row tiles: two or three work-groups share a CU, so one work-group's
    // epilogue overlaps another's main loop; with 128-row tiles (one per CU)
    // every CU alternates between the two phases.
    hipError_t e;
    switch (w.kind) {
        case WK_Q4_0: e = dispatch_waves<WK_Q4_0>(epi, p, st); break;
        case WK_Q4_1: e = dispatch_waves<WK_Q4_1>(epi, p, st); break;
        case WK_Q8_0: e = dispatch_waves<WK_Q8_0>(epi, p, st); break;
        case WK_F16: e = dispatch_waves<WK_F16>(epi, p, st); break;
        case WK_F32: e = dispatch_waves<WK_F32>(epi, p, st); break;
        case WK_F16X3: e = dispatch_waves<WK_F16X3>(epi, p, st); break;
        default: return hipErrorInvalidValue;
    }
    if (e == hipSuccess && p.ksplit > 1) {
        const int64_t n = M * (w.N / 4);
        hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p.part, p.ksplit,
                           (int)M, (int)w.N, ea.bias, ea.y, ea.ldy, epi == EPI_RESID ? 1 : 0);
        e = hipGetLastError();
    }
    return e;
}

}  // namespace s3e
