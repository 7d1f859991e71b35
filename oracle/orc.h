/*
 * orc.h — CPU oracle for the sam3.cpp image-encoder hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the arithmetic
 * that sam3.cpp's encoder graph performs through ggml's CPU backend
 * (ggml_mul_mat, ggml_flash_attn_ext, ggml_norm, ggml_gelu_erf, RoPE,
 * window partition, patch-embed conv).  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it, and only as the reference
 * results to compare against or the timed CPU baseline; the product path
 * never links or calls it.
 *
 * ggml itself is not available in this repository (the submodule referenced by
 * .gitmodules:1-3 is empty), so every ggml-internal behaviour restated here
 * is marked [ext] at its definition, with the public ggml source it follows.
 *
 * Layouts follow ggml's ne order, fastest dimension first.  A matrix that
 * ggml calls [K, M] is stored here as M rows of K contiguous elements.
 *
 * Parity status per function is listed in orc_core.c's header comment.
 */
#ifndef SAM3_ORACLE_ORC_H
#define SAM3_ORACLE_ORC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (sam3.cpp:3242-3248 switch, examples/quantize.cpp:63). */
enum {
    ORC_TYPE_F32  = 0,
    ORC_TYPE_F16  = 1,
    ORC_TYPE_Q4_0 = 2,
    ORC_TYPE_Q4_1 = 3,
    ORC_TYPE_Q8_0 = 8,
    ORC_TYPE_Q8_1 = 9,
};

/* ---- scalar conversions ------------------------------------------------ */
uint16_t orc_fp32_to_fp16(float f);            /* round to nearest even */
float    orc_fp16_to_fp32(uint16_t h);
float    orc_fp16_to_fp32_soft(uint16_t h);
void     orc_fp32_to_fp16_row(const float *x, uint16_t *y, int64_t n);
void     orc_fp16_to_fp32_row(const uint16_t *x, float *y, int64_t n);

/* ---- block formats ------------------------------------------------------ */
int64_t  orc_blck_size(int type);               /* 1 or 32 */
size_t   orc_type_size(int type);               /* bytes per block */
size_t   orc_row_size(int type, int64_t ne0);   /* ggml_row_size */
int      orc_vec_dot_type(int wtype);           /* ggml vec_dot_type */

/* Reference quantizers used by ggml_quantize_chunk (weights). */
void orc_quantize_row_q4_0_ref(const float *x, void *y, int64_t k);
void orc_quantize_row_q4_1_ref(const float *x, void *y, int64_t k);
void orc_quantize_row_q8_0_ref(const float *x, void *y, int64_t k);
void orc_quantize_row_q8_1_ref(const float *x, void *y, int64_t k);
/* from_float of the vec_dot type on x86 SIMD (activations). */
void orc_quantize_row_q8_0(const float *x, void *y, int64_t k);
void orc_quantize_row_q8_1(const float *x, void *y, int64_t k);
/* Convert a row of f32 into `type` the way mul_mat converts src1. */
void orc_from_float(int type, const float *x, void *y, int64_t k);
void orc_dequantize_row(int type, const void *x, float *y, int64_t k);

/* ---- dot products (ggml vec_dot_<wtype>_<vec_dot_type>, AVX2 order) ---- */
float orc_vec_dot(int wtype, int64_t n, const void *w_row, const void *x_row);
/* Which ggml CPU build to restate.  Same block math, different fp32
 * rounding — for measuring the order sensitivity of the reference itself:
 *   ORC_VARIANT_X86 (default) x86 AVX2 dots and quantizers;
 *   ORC_VARIANT_GENERIC       ggml's generic scalar dots;
 *   ORC_VARIANT_ARM           the Apple M4 Pro build of the reference's
 *                             published timings: tinyBLAS_Q0_ARM for Q4_0 /
 *                             Q8_0, the i8mm vec_dot for Q4_1, NEON
 *                             quantizers and f32 dots;
 *   ORC_VARIANT_ARM_DOTPROD   NEON vec_dot with nrc = 1 for every quantized
 *                             type (two alternating float32x4 accumulators);
 *   ORC_VARIANT_ARM_I8MM      NEON vec_dot with nrc = 2 for every quantized
 *                             type (one fp32 fma chain over exact block sums).
 * The ARM variants also switch the Q8_0 / Q8_1 quantizers (id = 1/d) and
 * the f32 dot (NEON order). */
enum { ORC_VARIANT_X86 = 0, ORC_VARIANT_GENERIC = 1, ORC_VARIANT_ARM = 2, ORC_VARIANT_ARM_DOTPROD = 3,
       ORC_VARIANT_ARM_I8MM = 4 };
void  orc_set_variant(int v);
/* Exact per-block integer sums Σ q_w·q_x of one (w row, x row) pair. */
void  orc_block_isums(int wtype, int64_t n, const void *w_row, const void *x_row, int32_t *out);

/* ---- operators ---------------------------------------------------------- */
/* ggml_mul_mat(W, X): W is N rows of K in `wtype`, X is M rows of K f32,
 * Y is M rows of N f32.  X is converted to the vec_dot type first. */
void orc_mul_mat(int wtype, const void *W, int64_t N, int64_t K,
                 const float *X, int64_t M, float *Y, int nthreads);
/* Same, with X already in the vec_dot type (row stride orc_row_size). */
void orc_mul_mat_preq(int wtype, const void *W, int64_t N, int64_t K,
                      const void *Xq, int64_t M, float *Y, int nthreads);

/* ggml_norm(x, eps) then *w then +b (w, b may be NULL). rows of n. */
void orc_layer_norm(const float *x, float *y, int64_t rows, int64_t n, float eps,
                    const float *w, const float *b, int nthreads);
void orc_gelu_erf(float *x, int64_t n);

/* RoPE (sam3.cpp:3667-3706): x is [HD, N, nh] with HD fastest (a row of HD
 * per token per head), freqs is [2, HD/2, N] (cos, sin). In place. */
void orc_rope(float *x, int64_t HD, int64_t N, int64_t nh, const float *freqs);

/* ggml_flash_attn_ext with mask=NULL, max_bias=0, softcap=0, F32 Q/K/V.
 * Q(b,h,i,d) at q[b*qs3 + h*qs2 + i*qs1 + d] (element strides);
 * K, V likewise.  O is [D, nh, Nq, B]: o[((b*Nq + i)*nh + h)*D + d]. */
void orc_flash_attn_ext(const float *q, int64_t qs1, int64_t qs2, int64_t qs3,
                        const float *k, int64_t ks1, int64_t ks2, int64_t ks3,
                        const float *v, int64_t vs1, int64_t vs2, int64_t vs3,
                        int64_t D, int64_t Nq, int64_t Nkv, int64_t nh, int64_t B,
                        float scale, float *o, int nthreads);

/* sam3_compute_axial_cis (sam3.cpp:3555-3586): out [N=end_x*end_y][dim/2][2]. */
void orc_compute_axial_cis(float *out, int dim, int end_x, int end_y,
                           float theta, float scale_pos);

/* sam3_preprocess_image (sam3.cpp:3441-3514): HWC uint8 → CHW f32. */
void orc_preprocess_sam3(const uint8_t *img, int w, int h, int img_size, float *chw);
/* sam3_resize_bilinear (sam3.cpp:3441-3484) alone: HWC uint8 → HWC uint8. */
void orc_resize_bilinear_u8(const uint8_t *img, int w, int h, uint8_t *out, int ow, int oh);
/* sam2_preprocess_image (sam3.cpp:3518-3544): resize + ImageNet mean/std. */
void orc_preprocess_sam2(const uint8_t *img, int w, int h, int img_size, float *chw);

/* ---- SAM 3 ViT encoder (sam3.cpp:3706-3849) ----------------------------- */
typedef struct orc_model orc_model;
/* Hiera / FPN hparams of a SAM 2 file (sam2_load_hparams, sam3.cpp:1564-1626) */
typedef struct {
    int32_t img_size, embed_dim, num_heads, num_stages, stages[4];
    int32_t global_n, global_idx[8], q_pool, window_spec[4], bkg_h, bkg_w, scalp;
    int32_t neck_dim, fpn_td_n, fpn_td[4];
} orc_hiera_hp;
orc_model *orc_model_load(const char *path);      /* NULL on failure */
void       orc_model_free(orc_model *m);
const char *orc_last_error(void);
/* hparams: img_size, patch, E, depth, heads, mlp, window, n_global, g0..g3,
 * ftype, neck_dim, visual_only, necks present (bit 0 trk, bit 1 det) */
void orc_model_hparams(const orc_model *m, int32_t out[16]);
/* A loaded tensor in its registered type (sam3.cpp:2461-2591). */
typedef struct {
    int type;
    int64_t ne[4];
    const void *data;
} orc_tensor_view;
int  orc_model_tensor(const orc_model *m, const char *prefix, const char *suffix, orc_tensor_view *out);
/* NULL unless the model is a SAM 2 (Hiera) file */
const orc_hiera_hp *orc_model_hiera(const orc_model *m);
/* Encode size of the following Hiera calls (0 < img_size, a multiple of 32). */
int orc_hiera_set_img_size(orc_model *m, int img_size);
void orc_set_error(const char *fmt, ...);
/* Prefix (patch embed + tiled pos + ln_pre): chw [3][img][img] → x [T][E]. */
int  orc_vit_prefix(const orc_model *m, const float *chw, float *x, int nthreads);
/* One block in place on x [T][E]. */
int  orc_vit_block(const orc_model *m, int idx, float *x, int nthreads);
/* Whole backbone: chw → vit_output [T][E]. */
int  orc_vit_encode(const orc_model *m, const float *chw, float *out, int nthreads);
/* Sub-stage hooks (sam3_test_run_vit_block_stage / _prefix_stage, stage
 * numbers of sam3.h:112-134) on an f32 input in ggml 4D layout; out_ne gets
 * the output shape, out may be NULL (shape only). */
int  orc_vit_block_stage(const orc_model *m, int idx, int stage, const float *in, const int64_t in_ne[4],
                         float *out, int64_t out_ne[4], int nthreads);
int  orc_vit_prefix_stage(const orc_model *m, int stage, const float *in, const int64_t in_ne[4], float *out,
                          int64_t out_ne[4], int nthreads);

/* ---- SimpleFPN neck (sam3.cpp:3863-3921), NHWC activations --------------- */
/* ggml_conv_transpose_2d_p0 with a 2×2 fp16 kernel ggml [2, 2, Cout, Cin]:
 * x [H][W][Cin] → y [2H][2W][Cout] (no bias). */
void orc_conv_transpose_2x2(const uint16_t *w16, int64_t Cin, int64_t Cout, const float *x, int64_t H,
                            int64_t W, float *y, int nthreads);
/* ggml_conv_2d, stride 1, padding pad: kernel ggml [KW, KH, Cin, Cout] of
 * type ktype (F32 or F16); x [H][W][Cin] → y [OH][OW][Cout] (no bias). */
void orc_conv2d(int ktype, const void *w, int64_t KW, int64_t KH, int64_t Cin, int64_t Cout, int64_t pad,
                const float *x, int64_t H, int64_t W, float *y, int nthreads);
/* ggml_pool_2d MAX 2×2 stride 2: x [H][W][C] → y [H/2][W/2][C]. */
void orc_maxpool2x2(const float *x, int64_t H, int64_t W, int64_t C, float *y);
/* sam3_sinusoidal_pe_2d (sam3.cpp:3597-3633): out [H][W][d_model]. */
void orc_sinusoidal_pe_2d(int H, int W, int d_model, float *out);
/* Sides of the four levels and their width D for neck "trk" or "det". */
int  orc_neck_dims(const orc_model *m, const char *which, int64_t side[4], int64_t *D);
/* The neck on vit_output x [G²][E]: out[i] receives side[i]² rows of D. */
int  orc_neck(const orc_model *m, const char *which, const float *x, float *out[4], int nthreads);

/* ---- SAM 2.x Hiera encoder + FPN (sam3.cpp:4066-4603), NHWC ------------- */
/* ggml_gelu on f32 through ggml's fp16 table; the 65536-entry table itself */
void orc_gelu_tanh(float *x, int64_t n);
void orc_gelu_tanh_table(uint16_t *out);
/* sam2_bicubic_interpolate_cpu: src [C][Hi][Wi] → dst [C][Ho][Wo] */
void orc_bicubic(const float *src, int C, int Hi, int Wi, float *dst, int Ho, int Wo);
int  orc_hiera_num_blocks(const orc_model *m);
/* dim_in, dim_out, heads, window (0 global), q_stride, stage, stage end */
int  orc_hiera_block_info(const orc_model *m, int i, int32_t out[7]);
/* per stage: side and channel width */
int  orc_hiera_dims(const orc_model *m, int side[4], int width[4]);
/* sam2_compute_pos_embed: out [H][W][E] */
int  orc_hiera_pos_embed(const orc_model *m, int H, int W, float *out);
/* patch embed + bias + PE: chw [3][S][S] → x [S/4][S/4][E] */
int  orc_hiera_prefix(const orc_model *m, const float *chw, float *x, int nthreads);
/* one block: x [H][W][Cin] → y [Ho][Wo][Cout] */
int  orc_hiera_block(const orc_model *m, int bi, const float *x, int H, int W, float *y, int *Ho, int *Wo,
                     int nthreads);
/* FPN over the four stage outputs; out[i] NULL skips a level */
int  orc_hiera_fpn(const orc_model *m, float *const stage[4], const int side[4], float *out[4], int nthreads);
/* whole encoder; stage_out may be NULL */
int  orc_hiera_encode(const orc_model *m, const float *chw, float *out[4], float *stage_out[4], int nthreads);

/* ---- memory attention (orc_memattn.c) ----------------------------------- */
/* layers, D (neck_dim), MD (mem_out_dim), FFN of the model's memory attention */
int  orc_mem_attn_dims(const orc_model *m, int32_t out[4]);
/* sam3_build_mem_attn_graph (sam3.cpp:9224-9337): curr, src_pos [N][D];
 * prompt, prompt_pos [M_total][MD], the last n_ptr rows object-pointer
 * tokens; rope_q [N][D/2][2], rope_k [M_total − n_ptr][D/2][2]; out [N][D]. */
int  orc_mem_attn(const orc_model *m, const float *curr, const float *src_pos, int64_t N, const float *prompt,
                  const float *prompt_pos, int64_t M_total, int64_t n_ptr, const float *rope_q,
                  const float *rope_k, float *out, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
