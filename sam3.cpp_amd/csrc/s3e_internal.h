// s3e_internal.h — shared declarations of the engine's HIP kernels and host
// runtime.  Not part of the public ABI (include/s3e.h is).
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>
#include <exception>
#include <new>
#include <string>

#include "../../include/s3e.h"

namespace s3e {

// ggml block size of the quantized types (QK4_0 = QK4_1 = QK8_0 = QK8_1 = 32).
constexpr int QK = 32;

// Weight kinds as the GEMM kernels see them.  WK_F16X3 holds f32 weights as
// two fp16 planes (w·2^k = hi + lo) and multiplies f32 activations held the
// same way: hi·hi + hi·lo + lo·hi on fp16 MFMA, fp32-accurate products.
enum WKind : int { WK_Q4_0 = 0, WK_Q4_1 = 1, WK_Q8_0 = 2, WK_F16 = 3, WK_F32 = 4, WK_F16X3 = 5 };

// Activation formats (what a producer writes for the next GEMM to read).
//   A_Q8_0 : int8 qs[M][ld] + fp16 d[M][ld/32]          (vec_dot type of Q4_0/Q8_0)
//   A_Q8_1 : as A_Q8_0 + fp16 s[M][ld/32] = fp16(d·Σq)   (vec_dot type of Q4_1)
//   A_F16  : fp16 [M][ld]                                 (vec_dot type of F16)
//   A_F32  : f32  [M][ld]                                 (vec_dot type of F32)
//   A_F16X2: fp16 hi [M][ld] + fp16 lo [M][ld], x = hi + lo  (f32 input of WK_F16X3)
//   A_F6   : the Q8_0 codes q of each 32-element block split as q = 16·h + l
//            (h ∈ [−8, 8], l ∈ [−8, 7], both exact in fp6 E3M2), in the
//            operand order of the fp6 MFMA (f6_word below); fp16 scales d as
//            for A_Q8_0.  Input of Q4_0 weights in the large-M GEMM (ld a
//            multiple of 128).
enum AKind : int { A_Q8_0 = 0, A_Q8_1 = 1, A_F16 = 2, A_F32 = 3, A_F16X2 = 4, A_F6 = 5 };

inline AKind act_kind_for(WKind w) {
    switch (w) {
        case WK_Q4_0: case WK_Q8_0: return A_Q8_0;
        case WK_Q4_1: return A_Q8_1;
        case WK_F16: return A_F16;
        case WK_F16X3: return A_F16X2;
        default: return A_F32;
    }
}

// Rows of every activation buffer are padded to a multiple of this, so the
// GEMM's tile loads never leave the allocation.
constexpr int ROW_PAD = 128;

// A device activation buffer in one of the formats above.
//   x : values, row-major [mp][ld] (int8 codes, fp16 or f32)
//   lo: A_F16X2 only, the fp16 low plane, same shape as x
//   d : fp16 block scales, and s: fp16 block sums (Q8_1), "stage-major":
//       block b of row r at ((b / 4) * mp + r) * 4 + b % 4, so the four
//       blocks one GEMM stage consumes for 128 consecutive rows are 1 KB of
//       contiguous memory.
struct Act {
    AKind kind = A_F32;
    void *x = nullptr;
    uint16_t *d = nullptr;
    uint16_t *s = nullptr;
    void *lo = nullptr;
    int64_t ld = 0;   // elements per row (multiple of 32)
    int64_t mp = 0;   // row pitch of the scale planes (rows rounded up to ROW_PAD)
};

__host__ __device__ inline int64_t scale_index(int64_t mp, int64_t row, int64_t blk) {
    return ((blk >> 2) * mp + row) * 4 + (blk & 3);
}

// fp6 E3M2 (sign, 3 exponent bits with bias 3, 2 mantissa bits): the code of
// an integer v ∈ [−8, 8] (0, ±1, ±2, ±3 = 1.5·2, ±4, ±5 = 1.25·4, ±6, ±7 =
// 1.75·4, ±8).  The magnitudes' 5-bit codes 0, 12, 16, 18, 20, 21, 22, 23, 24
// sit in 6-bit fields of one 64-bit constant.
__host__ __device__ inline uint32_t f6_code(int v) {
    constexpr uint64_t T = (0ull) | (12ull << 6) | (16ull << 12) | (18ull << 18) | (20ull << 24) | (21ull << 30) |
                           (22ull << 36) | (23ull << 42) | (24ull << 48);
    const uint32_t a = (uint32_t)(v < 0 ? -v : v);
    return ((uint32_t)(T >> (6 * a)) & 31u) | (v < 0 ? 32u : 0u);
}
// q = 16·h + l with h = ⌊(q + 8)/16⌋ ∈ [−8, 8] and l ∈ [−8, 7], for |q| ≤ 127.
__host__ __device__ inline int f6_hi(int q) { return (q + 8) >> 4; }

// A fp6 operand is 32 codes of one 32-element block (block order, code j in
// bits [6j, 6j + 6) of a 192-bit string, little endian), stored as three
// 8-byte words t = 0, 1, 2.  Activations (A_F6), in units of 8 bytes: for
// 64-row tile rt, stage s of 4 blocks (K/128 stages), block b of the stage,
// part p (0: h, 1: l), word t, row r % 64:
//     (((rt · nst + s) · 4 + b) · 2 + p) · 3 + t) · 64 + r % 64
// so one tile row's stage is 12 KB of contiguous memory (what the GEMM's DMA
// copies to LDS as it is), and the 32 rows one MFMA operand read touches are
// 256 contiguous bytes.  Weights (Weight::f6), likewise per 128-column tile
// ct:  (((ct · nst + s) · 4 + b) · 3 + t) · 128 + n % 128.
__host__ __device__ inline int64_t f6_act_word(int64_t nst, int64_t r, int64_t blk, int p, int t) {
    return (((((r >> 6) * nst + (blk >> 2)) * 4 + (blk & 3)) * 2 + p) * 3 + t) * 64 + (r & 63);
}
__host__ __device__ inline int64_t f6_weight_word(int64_t nst, int64_t n, int64_t blk, int t) {
    return ((((n >> 7) * nst + (blk >> 2)) * 4 + (blk & 3)) * 3 + t) * 128 + (n & 127);
}

// A weight matrix repacked for the GEMM kernels.  N rows of K, stored as
// column-blocks of the output: row n of the ggml matrix is "column" n here.
//   Q4_0/Q4_1/Q8_0: q8 [Np][Kp] int8 block codes — the file's integers
//              (Q4_0 nibble − 8, Q4_1 nibble 0..15, Q8_0 as stored), held
//              expanded because the weights stay cache-resident in the large-M
//              GEMM; d, m (Q4_1 minimum) fp16 stage-major [Kp/128][Np][4].
//   F16/F32  : values [Np][Kp].
//   F16X3    : q = hi, lo = low plane, both fp16 [Np][Kp], of the f32 weights
//              scaled by 2^k so that the largest is in [2^14, 2^15): the low
//              plane stays out of the fp16 subnormal range; alpha = 2^-k
//              undoes the scale on the accumulator (exactly).
// Kp pads K to the kernel's stage width, Np pads N to the tile width; the
// padding is zero and contributes nothing.
struct Weight {
    WKind kind = WK_F32;
    int ggml_type = 0;
    int64_t K = 0, N = 0, Kp = 0, Np = 0, Kbp = 0;
    void *q = nullptr;
    uint16_t *d = nullptr;
    uint16_t *m = nullptr;
    void *lo = nullptr;
    float alpha = 1.0f;
    size_t bytes = 0;
    // Q4_0: the codes again as fp6 E3M2 words (f6_weight_word) for the GEMM
    // against A_F6 activations
    void *f6 = nullptr;
};

// The activation format the large-M GEMM takes for w: Q4_0 weights with an
// fp6 copy run on the fp6 MFMA (A_F6), everything else as act_kind_for.
inline AKind act_kind_gemm(const Weight &w) { return (w.kind == WK_Q4_0 && w.f6) ? A_F6 : act_kind_for(w.kind); }

// Rows [r0, ...) of an activation as an activation of their own (r0 a
// multiple of 64 for A_F6): codes and values by row (A_F6 by 64-row tile),
// the scale planes by row inside each stage (their stage pitch mp stays the
// buffer's).
inline Act act_rows(const Act &a, int64_t r0) {
    Act o = a;
    switch (a.kind) {
        case A_F6: o.x = (uint8_t *)a.x + (r0 / 64) * (a.ld / 128) * 12288; break;
        case A_Q8_0: case A_Q8_1: o.x = (int8_t *)a.x + r0 * a.ld; break;
        case A_F16: o.x = (_Float16 *)a.x + r0 * a.ld; break;
        case A_F16X2:
            o.x = (_Float16 *)a.x + r0 * a.ld;
            o.lo = (_Float16 *)a.lo + r0 * a.ld;
            break;
        default: o.x = (float *)a.x + r0 * a.ld; break;
    }
    if (a.d) o.d = a.d + r0 * 4;
    if (a.s) o.s = a.s + r0 * 4;
    return o;
}

// GEMM epilogues.
enum Epi : int {
    EPI_F32 = 0,     // y = acc + bias
    EPI_RESID = 1,   // y += acc + bias                    (residual add)
    EPI_POS = 2,     // y = (acc + bias) + pos[tile(token)]  (patch embed + tiled pos_embed; bias optional)
    EPI_GELU = 3,    // act = quant(gelu_erf(acc + bias))   (fc1 → fc2)
    EPI_QKV = 4,     // split Q/K/V, RoPE, fp16, window layout
    EPI_DECONV = 5,  // 2×2 stride-2 transposed conv: (+ bias, GELU) → pixel shuffle into act
    EPI_ACT = 6,     // act = acc + bias                     (conv → next conv)
    EPI_HQKV = 7,    // Hiera: Q/K/Vᵀ in window order (padded grid, heads padded to hdp), fp16
                     // (hi, lo); with qpool, Q as f32 rows into y for the pooling pass
};

struct EpiArgs {
    const float *bias = nullptr;
    float *y = nullptr;          // EPI_F32 / EPI_RESID / EPI_POS
    int64_t ldy = 0;
    // EPI_F32 / EPI_RESID: workspace for a split over K (gemm_splitk_floats
    // floats); null: never split
    float *ws = nullptr;
    int64_t ws_cap = 0;
    Act out;                     // EPI_GELU
    // EPI_POS
    const float *pos = nullptr;  // [pg][pg][E]
    int pos_grid = 0;
    // geometry shared by EPI_POS and EPI_QKV
    int grid = 0;                // tokens per side
    int window = 0;              // window side (== grid for global attention)
    // EPI_QKV
    int E = 0, HD = 0, NH = 0;
    const float *freqs = nullptr;  // [Nw][HD/2][2] or nullptr (no RoPE)
    _Float16 *q = nullptr, *k = nullptr, *vt = nullptr;
    // low halves of the fp16 pairs (x = hi + lo) when attention runs split
    _Float16 *q_lo = nullptr, *k_lo = nullptr, *vt_lo = nullptr;
    int vt_ld = 0;                 // row stride of Vᵀ in keys (vt_ld_for of the window size)
    // EPI_HQKV: grid height (grid = width), padded head dim, Q pooled later
    int grid_h = 0, hdp = 0, qpool = 0;
    // EPI_QKV: the first column block is sel0 (0 Q, 1 K, 2 V) — a product with
    // only K or only V columns; RoPE only on tokens below rope_rows (0: all)
    int sel0 = 0, rope_rows = 0;
    int relu = 0;                  // EPI_GELU: ReLU instead of GELU
    // EPI_DECONV: input width (pixels per row) and output channels; column n
    // of the GEMM is kernel tap q = n / cout (ky = q / 2, kx = q % 2),
    // channel n % cout, written to output pixel (2y + ky, 2x + kx)
    int dc_w = 0, dc_cout = 0;
    int gelu = 0;                  // EPI_DECONV: gelu_erf after the bias
    // EPI_F32 of a 3×3 conv: bias holds 9 rows of N, row 3·cy + cx for an
    // output pixel in image row class cy and column class cx (0: first, 2:
    // last, 1: otherwise)
    int bias_cls = 0;
    // EPI_GELU: ggml_gelu (tanh form) through this fp16 table (65536 entries,
    // ggml_vec_gelu_f32 with GGML_GELU_FP16) instead of gelu_erf
    const uint16_t *gelu_tab = nullptr;
};

// Implicit-GEMM geometry of a 3×3 stride-1 pad-1 convolution over an NHWC
// image: row m of A is output pixel (m / w, m % w); stage s of K reads the
// input pixel shifted by tap s / spt ((dy, dx) = (tap / 3 − 1, tap % 3 − 1))
// at channels [32·(s % spt), +32), or the zero row outside the image.
struct ConvGeom {
    int w = 0, h = 0;
    int spt = 0;                   // stages per tap = Cin / 32
    const void *zero = nullptr;    // ≥ 128 zero bytes, 16-byte aligned
};

// Vᵀ rows (fp16 [BH][64][vt_ld]) hold the keys of each aligned 16-key group
// with the middle two quarters swapped: key q of a group sits at slot
// vt_slot(q).  One 16-byte chunk then holds keys {0-3, 8-11} or {4-7, 12-15}
// of a group, the 8 keys one lane half feeds to a K=16 MFMA step of the
// attention kernel, so that operand is one LDS read.  vt_ld is the key count
// rounded up to 16; keys past the count are zero.
__host__ __device__ inline int64_t vt_slot(int64_t q) {
    return (q & ~(int64_t)15) | (q & 3) | ((q & 4) << 1) | ((q & 8) >> 1);
}
__host__ __device__ inline int64_t vt_ld_for(int64_t nkv) { return (nkv + 15) / 16 * 16; }

// Attention I/O.
struct AttnArgs {
    const _Float16 *q = nullptr;   // [BH][Nq][hd]
    const _Float16 *k = nullptr;   // [BH][Nkv][hd]
    const _Float16 *vt = nullptr;  // [BH][hd][vt_ld_for(Nkv)], keys in vt_slot order
    // V as ggml holds it, fp16 [BH][Nkv][hd] (hd 64 or 128, no lo planes):
    // when set the kernel reads V where it lies (LDS transpose loads) and vt
    // is not used
    const _Float16 *v = nullptr;
    // low halves (x = hi + lo) for split-precision attention, else null
    const _Float16 *q_lo = nullptr, *k_lo = nullptr, *vt_lo = nullptr;
    int Nq = 0, Nkv = 0, NH = 0, BH = 0;
    // elements between the Q rows of consecutive (batch, head) pairs (0:
    // Nq·hd): a band of queries of a longer sequence reads its rows in place
    int64_t q_hs = 0;
    int hd = 64;                   // head dim of the q/k/vt rows: 64, or 128 (narrower heads zero-padded)
    int hd_out = 0;                // real head dim (0: = hd); output columns h·hd_out + d for d < hd_out
    float scale = 0.f;
    // output row of query i of batch b: token(b, i) when grid > 0, else b*Nq + i
    int grid = 0, window = 0;
    // windowed output with cropping (wo > 0): query i of window b = (b / nwx,
    // b % nwx) sits at (y, x) = (wy·wo + i / wo, wx·wo + i % wo) of an
    // out_h × out_w grid, row y·out_w + x; positions outside are dropped
    int wo = 0, nwx = 0, out_h = 0, out_w = 0;
    // split over keys (nsplit > 1): each of nsplit key ranges writes its
    // unnormalised output to part_o [nsplit][BH][Nq][hd] and (m, l) to
    // part_ml [nsplit][BH][Nq][2]; a combining pass then writes out (A_F32,
    // row b·Nq + i, column h·hd + d).  Plain layouts only (no crop, grid 0).
    int nsplit = 1;
    float *part_o = nullptr, *part_ml = nullptr;
    Act out;                       // A_Q8_0 / A_Q8_1 / A_F16 / A_F32, row = token, col = h*64 + d
};

// One product of a small-M launch (k_gemm_sm.hip): weights in the
// block-interleaved copy (block b of column n at (b·np + n)·BB bytes, BB =
// 16 / 32 / 64 for Q4 nibbles / Q8_0 / F16) with the usual stage-major scale
// planes; activations in the weight's vec_dot format.  Work-group w works on
// column group w − wg0 of this product (sm_wgs: 32-column strips, 4 / ks of
// them per work-group).
struct SmGemm {
    const uint8_t *w = nullptr;
    const uint16_t *wd = nullptr, *wm = nullptr;
    const void *x = nullptr;
    const uint16_t *xd = nullptr, *xs = nullptr;
    const float *bias = nullptr;
    float *y = nullptr;
    int64_t ldx = 0, ldy = 0, xmp = 0, np = 0;
    int K = 0, N = 0, nst = 0;   // nst: stages of 4 blocks (Kp rounded up to 128, over 128)
    int wg0 = 0;                 // first work-group of this product
};
struct SmArgs {
    SmGemm one;                  // used when many == nullptr
    const SmGemm *many = nullptr;  // device array of n products
    const uint16_t *wg_gemm = nullptr;  // device: product index of each work-group (with many)
    int n = 1;
    int M = 0;                   // rows, 1..64, shared by the products
    // one product split over K across kg work-groups per column group
    // (k_gemm_sm only): part holds the kg·M·N partial sums
    int kg = 1;
    float *part = nullptr;
    // k_gemm_sm with M > 32: 2 gives each 32-row tile work-groups of its own
    int rt = 1;
};

// ---- kernel launchers (k_*.hip) ----
// Floats of workspace a product of M rows against w would use when split over
// K (0: it runs unsplit): products with fewer tiles than CUs and a long K.
int64_t gemm_splitk_floats(const Weight &w, int64_t M);
// Products against uploaded weights (k_gemm.hip): every epilogue but EPI_ACT;
// EPI_DECONV takes WK_F16 weights and A_F16 rows.
hipError_t launch_gemm(const Weight &w, const Act &a, int64_t M, Epi epi, const EpiArgs &ea,
                       hipStream_t st);
// Small-M products (k_gemm_sm.hip): Q4_0 / Q4_1 / Q8_0 / F16 weights, M ≤ 64.
// ks = 4 (four waves split the K range of one 32-column strip); wgs = total
// of sm_wgs(N, ks) over the products, times a.kg for a split product.
int64_t sm_weight_bytes(const Weight &w);
int sm_wgs(int64_t N, int ks);
constexpr int SM_KG_MAX = 16;  // most work-groups one column group's K range splits over
hipError_t launch_pack_sm(const Weight &w, void *out, hipStream_t st);
hipError_t launch_gemm_sm(WKind kind, const SmArgs &a, int wgs, int ks, hipStream_t st);
// Batched products (many): 4 strips per work-group, activations staged in
// LDS; wgs = total of sm_wgs(N, 1).
hipError_t launch_gemm_smb(WKind kind, const SmArgs &a, int wgs, hipStream_t st);
// Neck GEMMs (k_conv.hip; WK_F16 or WK_F16X3 weights with N padded to
// CONV_BN): EPI_ACT / EPI_F32 on plain rows, or EPI_F32 as a 3×3 implicit
// GEMM when g is given.
hipError_t launch_conv(const Weight &w, const Act &a, int64_t M, Epi epi, const EpiArgs &ea,
                       const ConvGeom *g, hipStream_t st);
// NHWC f32 [h][w][c] → act (A_F16 or A_F16X2) of the same pixels (pool = 1)
// or of the 2×2 stride-2 max pool (pool = 2, floor((h − 2)/2) + 1 rows).
hipError_t launch_pool_act(const float *x, int h, int w, int c, int pool, const Act &out, hipStream_t st);
hipError_t launch_rows_quant(AKind kind, const float *x, int64_t M, int64_t K, const Act &out,
                             hipStream_t st);
hipError_t launch_layernorm(const float *x, int64_t M, int64_t E, float eps, const float *w,
                            const float *b, const Act &out, float *y_f32, hipStream_t st);
hipError_t launch_attn(const AttnArgs &a, hipStream_t st);
hipError_t launch_attn_prep(const float *q, const int64_t q_nb[4], const float *k,
                            const int64_t k_nb[4], const float *v, const int64_t v_nb[4],
                            int64_t Nq, int64_t Nkv, int64_t nh, int64_t B, int D, int hdp, _Float16 *q16,
                            _Float16 *k16, _Float16 *vt16, _Float16 *q_lo, _Float16 *k_lo,
                            _Float16 *vt_lo, int64_t ldv, hipStream_t st);
// fp16 operands of s3e_flash_attn_ext_f16: Q, K and V (when q16 / k16 /
// v16 are given) copied to [BH][N][hdp] with zeros for d ≥ D; when vt16 is
// given V is transposed to Vᵀ [BH][hdp][ldv] in vt_slot order with zeros past
// Nkv (every slot of every row is written).
hipError_t launch_attn_prep16(const _Float16 *q, const int64_t q_nb[4], const _Float16 *k, const int64_t k_nb[4],
                              const _Float16 *v, const int64_t v_nb[4], int64_t Nq, int64_t Nkv, int64_t nh,
                              int64_t B, int D, int hdp, _Float16 *q16, _Float16 *k16, _Float16 *v16,
                              _Float16 *vt16, int64_t ldv, hipStream_t st);
// Measurement kernels (k_probe.hip).  Stream: mode 0 read (sink: blocks·256
// words), 1 copy, 2 write; bytes a multiple of 16.  MFMA: kind 0 i8
// 32×32×32, 1 f16 32×32×16, 2 scaled fp6 32×32×64, 3 f16 32×32×8; iters
// steps of eight MFMAs per wave; sink: blocks·4 words.
hipError_t launch_probe_stream(int mode, void *dst, const void *src, size_t bytes, uint32_t *sink, int blocks,
                               hipStream_t st);
hipError_t launch_probe_mfma(int kind, int64_t iters, int blocks, uint32_t *sink, hipStream_t st);
// Rows of ldk per patch (A_F32, A_F16, or A_F16X2 with the lo plane at lo).
hipError_t launch_im2col(const float *chw, int img, int P, int64_t ldk, AKind kind, void *out,
                         hipStream_t st, void *lo = nullptr);
hipError_t launch_copy(void *dst, const void *src, size_t bytes, hipStream_t st);
// y = a + b·s elementwise (n floats; y may alias a)
hipError_t launch_add_scaled(float *y, const float *a, const float *b, float s, int64_t n, hipStream_t st);
// HWC uint8 image of w × h → CHW f32 of S × S: bilinear resize (skipped when
// w = h = S) and normalisation (norm 0: (v − 0.5)/0.5, 1: ImageNet mean/std).
hipError_t launch_preprocess(const uint8_t *hwc, int w, int h, int S, int norm, float *chw, hipStream_t st);

// ---- sub-stage hooks (k_rows.hip) ----
hipError_t launch_gelu_rows(const float *x, float *y, int64_t n, hipStream_t st);
// ggml_win_part (part = 1: grid rows → window rows, zero-padded) or
// ggml_win_unpart (part = 0) on rows of E floats over a W0 × H0 grid
hipError_t launch_win_perm(const float *x, float *y, int W0, int H0, int WS, int64_t E, int part, hipStream_t st);
// qkv [B·N][3·NH·HD] → RoPE'd Q and K, f32 [2][B][NH][N][HD] (freqs may be null)
hipError_t launch_vit_rope_split(const float *qkv, const float *freqs, float *out, int64_t B, int64_t N, int NH,
                                 int HD, hipStream_t st);
// A_F16 / A_F32 activation rows → f32 [M][K]
hipError_t launch_act_f32(const Act &a, int64_t M, int64_t K, float *y, hipStream_t st);
hipError_t launch_transpose(const float *x, float *y, int64_t R, int64_t C, hipStream_t st);
// y = x + pos tiled over the G × G grid (pos [pg][pg][E]); rows of E
hipError_t launch_add_pos(const float *x, const float *pos, float *y, int G, int pg, int64_t E, int64_t rows,
                          hipStream_t st);

// ---- Hiera (k_hiera.hip) ----
// Patch-embedding im2col: CHW f32 [3][S][S], k×k / stride / pad → rows of ldk.
hipError_t launch_im2col_conv(const float *chw, int S, int k, int stride, int pad, int64_t ldk, AKind kind,
                              void *out, hipStream_t st, void *lo = nullptr);
// Attention operands of a Hiera block from its QKV GEMM output (window
// partition with bias-valued padding, Q max-pool, head split, zero-padded
// head dim, fp16 hi/lo).
struct HieraPrepArgs {
    const float *qkv = nullptr;   // [H·W][3C] f32, bias added
    const float *bias = nullptr;  // [3C]: the value of padded window positions
    int H = 0, W = 0, C = 0, NH = 0, HD = 0, HDp = 0;
    int window = 0;               // 0: one window of the whole grid (global attention)
    int q_stride = 0;
    int qkv_ld = 0;               // row stride of qkv in floats (0: 3C); Q columns start at 0
    _Float16 *q = nullptr, *k = nullptr, *vt = nullptr;
    _Float16 *q_lo = nullptr, *k_lo = nullptr, *vt_lo = nullptr;
};
hipError_t launch_hiera_prep(const HieraPrepArgs &a, hipStream_t st);
// The attention operands that the EPI_HQKV epilogue does not write: window
// positions outside the grid (the QKV bias; zeros past HD), Q only without Q
// stride, and the Vᵀ key slots from the window size up to vt_ld (zeros).
hipError_t launch_hiera_pad(const HieraPrepArgs &a, hipStream_t st);
// dst [side²][D] += nearest-×2 upsampling of src [(side/2)²][D]
hipError_t launch_upsample_add(float *dst, const float *src, int side, int D, hipStream_t st);

// fp32 → fp16 of a value computed in fp32.  The empty asm statement (it emits
// no instruction) pins the fp32 value in a VGPR: without it LLVM folds
// fptrunc(fmul/fadd) into v_fma_mix*, rounding the exact result once instead
// of first to fp32 and then to fp16 as ggml's CPU path does.
__device__ __forceinline__ _Float16 to_half(float x) {
    __asm__ volatile("" : "+v"(x));
    return (_Float16)x;
}
__device__ __forceinline__ uint16_t half_bits(float x) { return __builtin_bit_cast(uint16_t, to_half(x)); }

// gelu_erf(x) = 0.5·x·(1 + erf(x/√2)) (ggml_vec_gelu_erf_f32), branch-free.
// With z = |x|/√2, erfc(z) = t·P(t)·e^(−z²), t = 1/(1 + 0.63·z), P a degree-8
// polynomial fitted by least squares to erfc(z)·e^(z²)/t on z ∈ [0, 6]
// (relative error ≤ 3.1e-7 in float32; beyond z = 6, e^(−z²) < 3e-16 makes
// the product vanish).  1 + erf(x/√2) is 2 − erfc(z) for x ≥ 0 and erfc(z)
// for x < 0, so neither branch cancels.
__device__ __forceinline__ float gelu_erf(float x) {
    const float z = fabsf(x) * 0.70710678118654752440f;
    const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.63f, z, 1.0f));
    float P = 0.06951001286506653f;
    P = __builtin_fmaf(P, t, -0.4178536534309387f);
    P = __builtin_fmaf(P, t, 1.0159318447113037f);
    P = __builtin_fmaf(P, t, -1.1790587902069092f);
    P = __builtin_fmaf(P, t, 0.5140861868858337f);
    P = __builtin_fmaf(P, t, -0.02842715010046959f);
    P = __builtin_fmaf(P, t, 0.3184112310409546f);
    P = __builtin_fmaf(P, t, 0.35179051756858826f);
    P = __builtin_fmaf(P, t, 0.3556097745895386f);
    const float e = __builtin_amdgcn_exp2f(-(z * z) * 1.4426950408889634f);
    const float E = t * P * e;
    const float w = (x >= 0.f) ? 2.0f - E : E;
    return 0.5f * x * w;
}

// ---- fp6 (E3M2) operand strings on the device ----
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x6 __attribute__((ext_vector_type(6)));

// The E3M2 codes of 32 small integers (|v| ≤ 8, exact in E3M2) as the 192-bit
// operand string, code j in bits [6j, 6j + 6): v_cvt_scalef32_2xpk16_bf6_f32
// fills slot 2i from even[i] and slot 2i + 1 from odd[i] (so even / odd are
// the block's even- and odd-indexed values), dividing by the scale (1 here).
// Written as asm with an early-clobber result: through the builtin the
// compiler may give the result registers that overlap the inputs, and the
// instruction then reads inputs it has already overwritten.
__device__ __forceinline__ u32x6 pack_bf6(const f32x16 &even, const f32x16 &odd) {
    u32x6 r;
    __asm__("v_cvt_scalef32_2xpk16_bf6_f32 %0, %1, %2, %3" : "=&v"(r) : "v"(even), "v"(odd), "v"(1.0f));
    return r;
}

// q = round-half-even(v·id) as a float, split q = 16·h + l with
// h = ⌊(q + 8) / 16⌋, l = q − 16·h (f6_hi); every step is exact.
__device__ __forceinline__ void f6_split(float v, float id, float &h, float &l) {
    const float q = __builtin_rintf(v * id);
    h = __builtin_floorf((q + 8.f) * 0.0625f);
    l = __builtin_fmaf(-16.f, h, q);
}

// 16 / 8 bytes loaded through a global-address-space pointer.  A pointer the
// compiler cannot place (one read from memory rather than a kernel argument)
// makes a flat load, which may address LDS, so behind LDS DMA the compiler
// first waits for every DMA in flight.  The loads go through vector types:
// HIP's uint4 / uint2 copy through a generic reference and stay flat.
__device__ __forceinline__ uint4 gload16(const void *p) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
    const u32x4 v = *(g_u32x4 *)p;
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 gload8(const void *p) {
    typedef __attribute__((address_space(1))) const uint64_t g_u64;
    const uint64_t v = *(g_u64 *)p;
    return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}

// An 8-byte LDS word as two 32-bit halves.  Read as uint2, the load makes
// the compiler wait for every LDS DMA in flight (the next stage's included)
// before it; a 64-bit read does not.
__device__ __forceinline__ uint2 lds_u2(const void *p) {
    const uint64_t v = *(const uint64_t *)p;
    return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}

// Wait until at most N of this wave's vector-memory operations are
// outstanding and all its LDS reads have returned, then join the work-group.
// The wait is the builtin (gfx9 s_waitcnt fields: vmcnt [3:0] and [15:14],
// expcnt [6:4] left at 7, lgkmcnt [11:8] at 0) so that the compiler's own
// wait tracking knows those loads completed: behind an opaque asm wait it
// would still treat earlier loads (e.g. fragments loaded before a loop) as
// outstanding and put a vmcnt(0) inside the loop, which also drains the LDS
// DMA of the next stage.  The barrier is asm with a memory clobber, which
// keeps the compiler from moving LDS accesses across it.
template <int N>
__device__ __forceinline__ void wait_and_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
    __asm__ volatile("s_barrier" ::: "memory");
}

// Stage widths (elements of K per pipeline stage) by weight kind.
inline int64_t stage_k(WKind w) {
    switch (w) {
        case WK_Q4_0: case WK_Q4_1: case WK_Q8_0: return 128;
        case WK_F16: case WK_F16X3: return 64;
        default: return 32;
    }
}
constexpr int GEMM_BN = 128;
constexpr int CONV_BN = 256;

// ---- error state (s3e_runtime.cpp) ----
void set_error(const char *fmt, ...);

}  // namespace s3e

// Handlers of the function-try-blocks around the extern "C" entry points
// (`extern "C" int s3e_x(...) try { ... } S3E_CATCH("s3e_x")`): no exception
// leaves the library; a failed host allocation returns S3E_ERR_NOMEM,
// anything else S3E_ERR_IO, with the message set.
#define S3E_CATCH(fn)                                                 \
    catch (const std::bad_alloc &) {                                  \
        s3e::set_error("%s: out of host memory", fn);                 \
        return S3E_ERR_NOMEM;                                         \
    }                                                                 \
    catch (const std::exception &ex_) {                               \
        s3e::set_error("%s: %s", fn, ex_.what());                     \
        return S3E_ERR_IO;                                            \
    }                                                                 \
    catch (...) {                                                     \
        s3e::set_error("%s: unexpected exception", fn);               \
        return S3E_ERR_IO;                                            \
    }
