/*
 * s3e.h — C ABI of the MI355X image-encoder engine for sam3.cpp model files.
 *
 * The engine replaces the two ggml operators that dominate sam3.cpp's image
 * encoders (ggml_mul_mat on Q4_0/Q4_1/Q8_0/F16/F32 weights and
 * ggml_flash_attn_ext) and the encoder graph that strings them together,
 * behind plain C entry points: pointers, sizes and status codes, no C++ or
 * torch types.  All calls return 0 (S3E_OK) on success; on failure they
 * return a non-zero status and s3e_last_error() describes the cause.  No
 * exception crosses this boundary.
 *
 * Memory: pointers documented as "device" are HBM addresses on the context's
 * device (from s3e_malloc or any HIP allocator); "host" pointers are ordinary
 * process memory.  Every compute call is asynchronous on the context's HIP
 * stream; s3e_ctx_sync() waits for it.
 *
 * Threading: one caller thread per context at a time, as sam3.cpp allows one
 * caller per sam3_state (sam3.cpp:1015-1026 resets the backend per call).
 * Models are read-only after loading and may be shared by contexts on the
 * same device.
 */
#ifndef S3E_H
#define S3E_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define S3E_ABI_VERSION 6

enum s3e_status {
    S3E_OK = 0,
    S3E_ERR_INVALID = 1,     /* bad argument or shape */
    S3E_ERR_HIP = 2,         /* HIP runtime error */
    S3E_ERR_IO = 3,          /* file missing, truncated or malformed */
    S3E_ERR_UNSUPPORTED = 4, /* valid input this engine does not handle */
    S3E_ERR_NOMEM = 5,       /* allocation failed */
};

/* ggml type ids as stored in sam3.cpp model files (sam3.cpp:3242-3248). */
enum s3e_type {
    S3E_TYPE_F32 = 0,
    S3E_TYPE_F16 = 1,
    S3E_TYPE_Q4_0 = 2,
    S3E_TYPE_Q4_1 = 3,
    S3E_TYPE_Q8_0 = 8,
    S3E_TYPE_Q8_1 = 9,
    /* Not a ggml type: the Q8_0 codes of quantize_row_q8_0, each split
     * q = 16·h + l (h = ⌊(q + 8)/16⌋) into two fp6 E3M2 values, in the tiled
     * layout the engine's Q4_0 kernel streams (s3e_quantize_rows,
     * s3e_mul_mat_q_f6). */
    S3E_TYPE_Q8_0_F6X2 = 64,
};

typedef struct s3e_ctx s3e_ctx;       /* device + HIP stream */
typedef struct s3e_weight s3e_weight; /* one uploaded weight matrix */
typedef struct s3e_model s3e_model;   /* SAM 3 ViT backbone weights */
typedef struct s3e_state s3e_state;   /* per-image activations and outputs */

/* Last error message of the calling thread ("" if none). */
const char *s3e_last_error(void);
int s3e_abi_version(void);

/* ---- context ------------------------------------------------------------
 * Replaces the ggml backend selection of sam3_load_model
 * (sam3.cpp:3274-3288) and the per-call backend setup of sam3_graph_compute
 * (sam3.cpp:1015-1026). */
int s3e_ctx_create(int device, s3e_ctx **out);
void s3e_ctx_destroy(s3e_ctx *ctx);
int s3e_ctx_sync(s3e_ctx *ctx);
/* The context's hipStream_t, for callers that record events on it. */
void *s3e_ctx_stream(s3e_ctx *ctx);

/* Device-memory helpers for FFI callers without their own allocator
 * (the role ggml_backend_alloc_ctx_tensors / ggml_backend_tensor_set/get play
 * in sam3.cpp:3300-3330, 6115). */
int s3e_malloc(s3e_ctx *ctx, size_t bytes, void **out);
int s3e_free(s3e_ctx *ctx, void *ptr);
int s3e_memcpy_h2d(s3e_ctx *ctx, void *dst, const void *src, size_t bytes);
int s3e_memcpy_d2h(s3e_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Device-to-device copy by a plain streaming kernel on the context stream
 * (bytes a multiple of 16, pointers 16-byte aligned).  Asynchronous. */
int s3e_copy(s3e_ctx *ctx, void *dst, const void *src, size_t bytes);

/* ---- ggml_mul_mat --------------------------------------------------------
 * Upload one weight matrix given as ggml bytes: ne0 = K (the contiguous
 * dimension), ne1 = N rows, in `type` (F32, F16, Q4_0, Q4_1 or Q8_0), exactly
 * as a sam3.cpp model file stores it (sam3.cpp:3091-3143).  The engine
 * repacks the blocks into its own HBM layout.  Replaces the weight tensors
 * that sam3_load_tensors fills (sam3.cpp:3145-3150). */
int s3e_weight_upload(s3e_ctx *ctx, int type, int64_t ne0, int64_t ne1,
                      const void *host_data, size_t nbytes, s3e_weight **out);
void s3e_weight_free(s3e_weight *w);
/* out[0]=type, out[1]=K, out[2]=N, out[3]=device bytes held. */
int s3e_weight_info(const s3e_weight *w, int64_t out[4]);

/* Y = ggml_add(ggml_mul_mat(W, X), bias): X is M rows of K f32 (device),
 * Y is M rows of N f32 (device), bias is N f32 (device) or NULL.  X is first
 * converted to W's vec_dot type exactly as ggml's CPU path converts src1
 * (Q8_0 for Q4_0/Q8_0, Q8_1 for Q4_1, F16 for F16, none for F32).
 * Replaces ggml_mul_mat + ggml_add at sam3.cpp:3738-3739, 3779-3780,
 * 3792-3796.  Above 64 rows the converted X (M rows of K bytes for Q8, 2·K
 * for F16, 4·K for F32, padded to 128-byte stages) and the repacked W must
 * each stay below 2 GiB; larger products return S3E_ERR_HIP.  M = 0 (an
 * empty batch) succeeds and writes nothing; M < 0 is S3E_ERR_INVALID. */
int s3e_mul_mat(s3e_ctx *ctx, const s3e_weight *w, const float *X, int64_t M,
                const float *bias, float *Y);

/* No counterpart in the reference: s3e_mul_mat for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid hipMalloc).  Same arguments and results; X is converted into a
 * file-scope device array of S3E_NOALLOC_SCRATCH_BYTES per GPU (64 MiB:
 * every C4 linear at 5184 rows fits, in every weight type) instead of a
 * per-call allocation, and every product runs on the large-M kernel (at 64
 * rows or fewer s3e_mul_mat streams the weight on another kernel: equal up
 * to fp32 summation order).  Calls no hipMalloc / hipFree and does not
 * synchronise.  A product whose conversion exceeds the array returns
 * S3E_ERR_INVALID.  All calls on one GPU share its array and leave their
 * contents in it: calls that overlap on one GPU race. */
#define S3E_NOALLOC_SCRATCH_BYTES (64ull << 20)
int s3e_mul_mat_noalloc(s3e_ctx *ctx, const s3e_weight *w, const float *X, int64_t M, const float *bias,
                        float *Y);

/* Same GEMM with X already in W's vec_dot type (ggml_mul_mat with src1 of
 * that type; ggml skips the conversion then): `xq`, `d`, `s` as written by
 * s3e_quantize_rows for K = W's ne0 (layout there).  Launches the GEMM kernel
 * only, so it is also the entry point to time the kernel alone.  Products of
 * at most 64 rows with Q4_0/Q4_1/Q8_0/F16 weights run on the weight-streaming
 * kernel.  s3e_weight_upload makes everything that kernel needs: the
 * block-interleaved copy of the weight and room in the uploading context's
 * workspace for the partial sums of a K-split product of up to 64 rows.  So
 * s3e_mul_mat_q allocates nothing and does not synchronise; on a context
 * other than the upload's, a small product whose partial sums do not fit
 * that context's workspace runs with K unsplit (same kernel, results equal
 * up to fp32 summation order). */
int s3e_mul_mat_q(s3e_ctx *ctx, const s3e_weight *w, const void *xq, const uint16_t *d,
                  const uint16_t *s, int64_t M, const float *bias, float *Y);
/* No counterpart in the reference: s3e_mul_mat_q for Q4_0 weights with
 * activations in S3E_TYPE_Q8_0_F6X2 (from s3e_quantize_rows), the kernel
 * s3e_mul_mat and the encoder run for Q4_0: each 32-block sum comes from the
 * fp6 MFMA, the same integers as the int8 path, so Y equals s3e_mul_mat_q's
 * bit for bit.  K must be a multiple of 128; any M (no small-M kernel).
 * Launches the GEMM kernel only. */
int s3e_mul_mat_q_f6(s3e_ctx *ctx, const s3e_weight *w, const void *xq, const uint16_t *d, int64_t M,
                     const float *bias, float *Y);

/* Several independent products of one graph level in one launch: Y[i] =
 * ggml_add(ggml_mul_mat(W[i], X[i]), bias[i]) for i < n, each as in
 * s3e_mul_mat_q (activations already in the weight's vec_dot format, device
 * pointers), all weights of one type among Q4_0/Q4_1/Q8_0/F16 and
 * 1 <= M <= 64 rows shared by the products.  ggml evaluates such nodes one
 * by one (ggml_backend_graph_compute over the graph, sam3.cpp:1015-1026);
 * there is no single reference entry point: at a few rows each product is a
 * weight stream too short to fill the GPU, and one launch streams them
 * together.  bias may be NULL, or hold NULL entries. */
int s3e_mul_mat_q_batch(s3e_ctx *ctx, int n, const s3e_weight *const *w, const void *const *xq,
                        const uint16_t *const *d, const uint16_t *const *s, int64_t M,
                        const float *const *bias, float *const *Y);

/* Convert M rows of K f32 (device) into a vec_dot type, as ggml's
 * from_float does for src1 of ggml_mul_mat: `type` is Q8_0, Q8_1 or F16.
 * F16: `qs` receives M*K fp16, row-major; d and s are unused.
 * Q8_0/Q8_1: `qs` receives M*K int8 codes, row-major.  `d` receives the fp16
 * block scales and, for Q8_1, `s` the fp16 block sums fp16(d·Σq), each as a
 * stage-major plane: with Mp = M rounded up to 128 and G = ceil(K/128),
 * block b of row r is element ((b/4)·Mp + r)·4 + b%4 of a plane of G·Mp·4
 * fp16 values (blocks of one row come in groups of 4, and each group is laid
 * out for all rows before the next).  Blocks from K/32 to 4G−1 are written as
 * zero; rows from M to Mp−1 are not written.  All device pointers.
 * S3E_TYPE_Q8_0_F6X2 (K a multiple of 128): the same codes and `d` as Q8_0;
 * `qs` receives 3·Mt·K/2 bytes, Mt = M rounded up to 64: for each 64-row
 * tile t, stage g (128 columns), block b < 4 of the stage, part p (0 h, 1 l)
 * and word w < 3, the 64 rows' 8-byte words of the 192-bit E3M2 strings
 * (code j of the block in bits [6j, 6j + 6)), as word
 * ((((t·G + g)·4 + b)·2 + p)·3 + w)·64 + row % 64.
 * M = 0 (an empty batch) succeeds and writes nothing; M < 0 is
 * S3E_ERR_INVALID. */
int s3e_quantize_rows(s3e_ctx *ctx, int type, const float *X, int64_t M, int64_t K,
                      void *qs, uint16_t *d, uint16_t *s);

/* sam3_layer_norm (sam3.cpp:1037-1047): y = ggml_norm(x, eps)·w + b over rows
 * of n f32 (device), w/b of n f32 or NULL.  Mean and variance accumulate in
 * double as ggml_norm does, so the result is bit-identical to the CPU path.
 * x and y may alias.  n must be a multiple of 32 and at most 4096. */
int s3e_layer_norm(s3e_ctx *ctx, const float *x, int64_t rows, int64_t n, float eps,
                   const float *w, const float *b, float *y);

/* ---- ggml_flash_attn_ext -------------------------------------------------
 * O = softmax(scale·Q·Kᵀ)·V with mask = NULL, max_bias = 0, softcap = 0, as
 * sam3.cpp:3774 and the isolated core at sam3.cpp:6778-6823 call it.
 * Tensors are f32 device memory addressed by ggml-style element strides:
 * Q(b,h,i,d) = q[b*q_nb[3] + h*q_nb[2] + i*q_nb[1] + d] (d contiguous), K and
 * V likewise (V may be the strided view of sam3.cpp:3762-3763).  O follows
 * ggml's output layout [D, nh, Nq, B]: o[((b*Nq + i)*nh + h)*D + d].
 * D: any multiple of 4 up to 128 (the ViT's 64; Hiera's 96, 56, 72, 32 —
 * run zero-padded to 64 or 128 channels, sam3.cpp:4395), or 256 (the
 * memory attention, sam3.cpp:9267, :9312; S3E_PREC_DEFAULT only).  Nq and
 * Nkv may differ (Hiera's pooled queries).  When the query tiles alone
 * would leave the GPU idle the keys are split into ranges whose partial
 * results a second pass combines.  `prec` mirrors ggml_flash_attn_ext_set_prec:
 * S3E_PREC_DEFAULT computes on fp16 MFMA with Q, K, V and the
 * probabilities rounded to fp16 (fp32 accumulation); S3E_PREC_F32 carries
 * each operand as an fp16 pair (hi + lo) and reproduces f32 attention,
 * as ggml's CPU path computes it, to ~1e-7. */
enum s3e_prec { S3E_PREC_DEFAULT = 0, S3E_PREC_F32 = 1 };
int s3e_flash_attn_ext(s3e_ctx *ctx,
                       const float *q, const int64_t q_nb[4],
                       const float *k, const int64_t k_nb[4],
                       const float *v, const int64_t v_nb[4],
                       int64_t D, int64_t Nq, int64_t Nkv, int64_t nh, int64_t B,
                       float scale, int prec, float *o);

/* ggml_flash_attn_ext with F16 Q, K and V (ggml accepts F16 K/V tensors; the
 * isolated attention microbench feeds fp16 operands): the same addressing,
 * shapes and output as s3e_flash_attn_ext, q/k/v as IEEE fp16 bits, computed
 * at S3E_PREC_DEFAULT (fp16 operands and probabilities, fp32 accumulation).
 * Q, K and V are read in place when they are contiguous [B][nh][N][D] with
 * D = 64 or 128 (else copied to that layout, zero-padded to 64 / 128; at
 * D = 256 V is transposed into the engine's layout by one pass).  Asynchronous on the context's stream: O is complete after
 * s3e_ctx_sync.  The copies live in a context-owned workspace that a call
 * grows (synchronising the stream, then hipMalloc) only when it needs more
 * room than every earlier call on the context; calls that fit allocate
 * nothing. */
int s3e_flash_attn_ext_f16(s3e_ctx *ctx,
                           const uint16_t *q, const int64_t q_nb[4],
                           const uint16_t *k, const int64_t k_nb[4],
                           const uint16_t *v, const int64_t v_nb[4],
                           int64_t D, int64_t Nq, int64_t Nkv, int64_t nh, int64_t B,
                           float scale, float *o);

/* ---- measurement ---------------------------------------------------------
 * No counterpart in the reference: the rates this GPU reaches, against which
 * the benchmark reads its roofline fractions next to the published peaks.
 * s3e_probe_stream moves `bytes` (a multiple of 16) through HBM with 64-byte
 * steps per thread and 8 work-groups of 4 waves per CU: mode 0 reads src,
 * 1 copies src to dst, 2 writes dst.  s3e_probe_mfma runs, on every SIMD,
 * waves_per_simd (1-4) waves of `iters` steps of eight independent MFMAs of
 * one form with operands in registers: kind 0 v_mfma_i32_32x32x32_i8
 * (65 536 ops each), 1 v_mfma_f32_32x32x16_f16 (32 768), 2 the scaled
 * 32x32x64 f8f6f4 form on fp6 operands (131 072), 3 v_mfma_f32_32x32x8_f16
 * (16 384).  Both are asynchronous; time them with events on the context's
 * stream.  The first call allocates a small output array on the context. */
int s3e_probe_stream(s3e_ctx *ctx, int mode, void *dst, const void *src, size_t bytes);
int s3e_probe_mfma(s3e_ctx *ctx, int kind, int64_t iters, int waves_per_simd);

/* ---- encoder -------------------------------------------------------------
 * Load the image encoder of a sam3.cpp model file (sam3.cpp:3200-3344):
 * for SAM 3 files (magic "sam3", version 3) the ViT backbone ("vit.") and
 * the SimpleFPN necks ("neck.trk.", and "neck.det." in full files;
 * sam3.cpp:2562-2596); for SAM 2.x files (magic "sam2", version 1) the
 * Hiera backbone ("hiera.") and its FPN ("fpn."; sam3.cpp:1745-1847).
 * Other records are skipped, so full and visual-only
 * files both load; a file without neck records loads as a backbone-only
 * encoder.  Replaces the encoder part of sam3_load_model (sam3.h:184). */
int s3e_model_load(s3e_ctx *ctx, const char *path, s3e_model **out);
void s3e_model_free(s3e_model *m);
/* SAM 3 files: out[0..15] = img_size, patch, E, depth, heads, mlp, window,
 * n_global, global_idx[4], ftype, tokens per side, neck_dim, necks present
 * (bit 0 tracker, bit 1 detector).  SAM 2 files: img_size, −1, embed_dim,
 * blocks, heads, stages[4], q_pool, window_spec[0], scalp, ftype, level-0
 * side, neck_dim, 1. */
int s3e_model_hparams(const s3e_model *m, int32_t out[16]);
/* sam3_get_model_type (sam3.h:194): 0 SAM 3, 1 SAM 3 visual-only, 2 SAM 2. */
int s3e_model_type(const s3e_model *m);

/* Per-image state holding activations and outputs (sam3_create_state,
 * sam3.h:196; outputs of sam3.cpp:896-928). */
int s3e_state_create(s3e_ctx *ctx, const s3e_model *m, s3e_state **out);
/* sam3_create_state with sam3_params::encode_img_size (sam3.cpp:3392-3402,
 * :245-257): the state encodes images of img_size pixels per side (0: the
 * model's own).  For SAM 2.x files any multiple of 32 up to 4096: the token
 * grids follow sam3_effective_feat_size's rule (img / 4, halved at every
 * Q-stride block) and the Hiera positional embedding is recomputed for the
 * new grid by the reference's bicubic resize (sam3.cpp:4114-4171); chw
 * inputs are [3][img_size][img_size] and s3e_encode_image_u8 resizes to
 * img_size.  SAM 3 files encode at their native size only
 * (S3E_ERR_UNSUPPORTED otherwise). */
int s3e_state_create_sized(s3e_ctx *ctx, const s3e_model *m, int img_size, s3e_state **out);
void s3e_state_free(s3e_state *st);

/* Encode a preprocessed CHW f32 image of img_size² (device pointer).
 * Replaces the graph build + compute of sam3_encode_image
 * (sam3.cpp:6051-6131) and sam3_encode_image_from_preprocessed
 * (sam3.cpp:7287-7482): the backbone ("vit_output" [E, W, H] = W*H rows of
 * E f32) and every neck of the model ("neck_trk_0..3", "neck_det_0..3"
 * [D, S, S] with S = 4W, 2W, W, W/2; sam3_build_neck_graph,
 * sam3.cpp:3863-3921). */
int s3e_encode_chw(s3e_state *st, const float *chw_device);
/* Same from host memory (uploads first). */
int s3e_encode_chw_host(s3e_state *st, const float *chw_host);
/* sam3_encode_image (sam3.h:216): HWC RGB uint8 of any size (host memory);
 * uploaded, resized and normalised on the device by s3e_preprocess_image
 * with the model's normalisation (SAM 3: sam3_preprocess_image,
 * sam3.cpp:3441-3514; SAM 2: sam2_preprocess_image, :3518-3544), then
 * encoded.  Returns after the encode has finished. */
int s3e_encode_image_u8(s3e_state *st, const uint8_t *hwc, int width, int height);

#define S3E_NORM_SAM3 0     /* (v/255 − 0.5)/0.5 */
#define S3E_NORM_IMAGENET 1 /* (v/255 − mean[c])/std[c], SAM 2 */
/* Device-side preprocessing, replacing sam3_resize_bilinear + the
 * normalisation loop of sam3_preprocess_image (sam3.cpp:3441-3514) and
 * sam2_preprocess_image (:3518-3544): hwc_device is width × height × 3 uint8
 * (RGB, row-major), chw_device receives 3 × img_size × img_size f32.  The
 * resize (skipped when width = height = img_size) is the reference's
 * half-pixel bilinear in double precision with round-half-up, so the
 * resized bytes, and hence the output, equal the reference's bit for bit.
 * Enqueued on the context's stream; no synchronisation. */
int s3e_preprocess_image(s3e_ctx *ctx, const uint8_t *hwc_device, int width, int height, int img_size, int norm,
                         float *chw_device);

/* Stage hooks (sam3_test_run_vit_block_stage, sam3.h:489 / sam3.cpp:6874):
 * prefix writes x (device, T rows of E f32) from a device CHW image; block
 * runs ViT block idx in place on x. */
int s3e_vit_prefix(s3e_state *st, const float *chw_device, float *x_device);
int s3e_vit_block(s3e_state *st, int idx, float *x_device);
/* Sub-stage hooks, replacing sam3_test_run_vit_block_stage and
 * sam3_test_run_vit_prefix_stage (sam3.h:441-496, sam3.cpp:6390-6520 and
 * :6874-6993; stage builders :6716-6872): one operator group of the graph
 * on an f32 input in ggml 4D layout (in_ne; entries ≤ 0 count as 1), on the
 * device.  out_ne receives the output shape; with out_device NULL only the
 * shape is computed (in_device may then be NULL too).  Stage numbers are
 * the reference's enums (sam3.h:112-134), reproduced below.  Block stages:
 * NORM1 / NORM2 [E,..] → [E,..]; WINDOW_PART [E,W,H,1] → [E,WS,WS,n]
 * (zero-padded); QKV_PROJ [E,..] → [3E,..]; ATTN_CORE [3E,W,H,B] → [E,W,H,B]
 * (q|k|v split, heads, RoPE from the block's table, which must have W·H
 * positions, attention); ATTN_PROJ [E,..]; WINDOW_UNPART [E,WS,WS,n] →
 * [E,G,G,1]; MLP_FC1 [E,..] → [MLP,..]; MLP_GELU; MLP_FC2 [MLP,..] → [E,..];
 * MLP = fc1 + GELU + fc2.  Prefix stages: PATCH_EMBED [img,img,3,1] →
 * [E,G,G,1]; PATCH_IM2COL → [3P²,G,G,1] (in the kernel's type, as f32);
 * PATCH_MULMAT_RAW [3P²,G,G,1] → [G²,E,1,1] and PATCH_MULMAT → [G,G,E,1]
 * (input and kernel rounded to F16, as the reference's F16 input tensor
 * makes ggml do); POS_ADD; LN_PRE_NORM (ggml_norm); LN_PRE.  Inputs and
 * outputs of at most G² rows (the state's buffers).  Asynchronous on the
 * context's stream. */
enum s3e_vit_block_stage {
    S3E_VIT_BLOCK_STAGE_NORM1 = 0,
    S3E_VIT_BLOCK_STAGE_WINDOW_PART,
    S3E_VIT_BLOCK_STAGE_QKV_PROJ,
    S3E_VIT_BLOCK_STAGE_ATTN_CORE,
    S3E_VIT_BLOCK_STAGE_ATTN_PROJ,
    S3E_VIT_BLOCK_STAGE_WINDOW_UNPART,
    S3E_VIT_BLOCK_STAGE_NORM2,
    S3E_VIT_BLOCK_STAGE_MLP_FC1,
    S3E_VIT_BLOCK_STAGE_MLP_GELU,
    S3E_VIT_BLOCK_STAGE_MLP_FC2,
    S3E_VIT_BLOCK_STAGE_MLP
};
enum s3e_vit_prefix_stage {
    S3E_VIT_PREFIX_STAGE_PATCH_EMBED = 0,
    S3E_VIT_PREFIX_STAGE_PATCH_IM2COL,
    S3E_VIT_PREFIX_STAGE_PATCH_MULMAT_RAW,
    S3E_VIT_PREFIX_STAGE_PATCH_MULMAT,
    S3E_VIT_PREFIX_STAGE_POS_ADD,
    S3E_VIT_PREFIX_STAGE_LN_PRE_NORM,
    S3E_VIT_PREFIX_STAGE_LN_PRE
};
int s3e_vit_block_stage(s3e_state *st, int idx, int stage, const float *in_device, const int64_t in_ne[4],
                        float *out_device, int64_t out_ne[4]);
int s3e_vit_prefix_stage(s3e_state *st, int stage, const float *in_device, const int64_t in_ne[4],
                         float *out_device, int64_t out_ne[4]);
/* The backbone alone (prefix + blocks, no neck) into "vit_output": the graph
 * of sam3_encode_vit_from_preprocessed_selective (sam3.cpp:6237-6327). */
int s3e_encode_vit_chw(s3e_state *st, const float *chw_device);
/* A model tensor in its registered type, copied to host memory (the
 * ggml_backend_tensor_get of sam3.cpp:6540, :6637-6641 in the host
 * references): "vit.patch_embed.proj.weight" and the block linears
 * "vit.blocks.<i>.{attn.qkv,attn.proj,mlp.lin1,mlp.lin2}.{weight,bias}".
 * Weights come back only when stored F16 or F32 (quantized ones are
 * repacked on the device: S3E_ERR_UNSUPPORTED, with type and ne still
 * written).  type and ne (ggml order) are written for every tensor found;
 * host may be NULL to query them. */
int s3e_model_tensor_get(const s3e_model *m, const char *name, int *type, int64_t ne[4], void *host, size_t bytes);
/* Neck stage hook: run the model's necks on a backbone output given on the
 * device (W*H rows of E f32), filling the state's neck_* tensors exactly as
 * s3e_encode_chw does after the backbone (the neck part of the encode graph,
 * sam3.cpp:6072-6075). */
int s3e_run_neck(s3e_state *st, const float *x_device);
/* ---- memory attention ---------------------------------------------------
 * The tracker's memory attention (sam3_build_mem_attn_graph,
 * sam3.cpp:9224-9337), loaded from the "mem_attn.*" records of either file
 * type.  out[0..3] = layers, D (neck_dim), MD (mem_out_dim), FFN width; an
 * error if the file has none. */
int s3e_mem_attn_dims(const s3e_model *m, int32_t out[4]);
/* Condition N current-frame tokens on the memory bank, on device f32
 * buffers, with the layouts sam3_propagate_single gives the graph
 * (sam3.cpp:11232-11304): curr and src_pos [N][D]; prompt and prompt_pos
 * [M_total][MD], whose last num_obj_ptr_tokens rows are object-pointer
 * tokens (no RoPE on their keys); rope_q [N][D/2][2] and rope_k
 * [M_total − num_obj_ptr_tokens][D/2][2] (cos, sin; NULL when every memory
 * token is a pointer token); out [N][D].  The state keeps the scratch, grown
 * to the largest sizes seen (allocated on first use).  Asynchronous. */
int s3e_mem_attn(s3e_state *st, const float *curr, const float *src_pos, int64_t N, const float *prompt,
                 const float *prompt_pos, int64_t M_total, int64_t num_obj_ptr_tokens, const float *rope_q,
                 const float *rope_k, float *out);
/* SAM 2 stage hook: Hiera block idx (sam2_hiera_block_forward,
 * sam3.cpp:4295-4457) on x (device, H·W rows of the block's input width,
 * NHWC) into y (H/2·W/2 rows under Q stride, else H·W, of its output
 * width).  x and y may be the same buffer when the block keeps its size. */
int s3e_hiera_block(s3e_state *st, int idx, const float *x_device, int H, int W, float *y_device);

/* State outputs by name (sam3_get_state_tensor_info / sam3_dump_state_tensor,
 * sam3.h:407-414, sam3.cpp:14334-14376).  Names: "vit_output",
 * "neck_trk_<i>", "neck_det_<i>", "neck_det_pe_<i>", "neck_trk_pe_<i>" and
 * "pe_<i>" (i = 0..3; the PEs of sam3_sinusoidal_pe_2d, sam3.cpp:6146-6193).
 * SAM 2 models: "neck_trk_<i>" and "neck_trk_pe_<i>" / "pe_<i>" for the
 * levels kept after scalp (sam3.cpp:5959-6003), and "hiera_stage_<i>", the
 * four stage outputs.  A name the model does not produce is an error.  ne receives the ggml
 * shape; get copies n floats to host memory. */
int s3e_state_tensor_info(const s3e_state *st, const char *name, int64_t ne[4]);
int s3e_state_tensor_get(const s3e_state *st, const char *name, float *host, size_t n);
const float *s3e_state_tensor_device(const s3e_state *st, const char *name);

/* ---- synthetic model files -----------------------------------------------
 * Write a random-init SAM 3 visual-only model file in sam3.cpp's format
 * (header + hparams per convert_sam3_to_ggml.py:27-67, 202-255), with
 * weights N(0, std²) from mt19937_64(seed) via Box-Muller, biases 0,
 * LayerNorm γ=1 β=0, freqs_cis from sam3_compute_axial_cis
 * (sam3.cpp:3555-3586; windows scale 1, global scale window/grid), and
 * linear weights quantized by the reference quantizers the way
 * examples/quantize.cpp:195-266 decides (ftype 0, 1, 2, 3 or 8).
 * Replaces the converter + quantize tool for synthetic-weight runs. */
typedef struct s3e_synth_cfg {
    int32_t img_size, patch, embed_dim, depth, heads, mlp_ratio_x1000, window;
    int32_t n_global, global_idx[4];
    int32_t ftype;
    uint64_t seed;
    float std;
    /* necks (sam3.cpp:2562-2591): 0 none, 1 tracker only (visual-only
     * file), 2 detector and tracker; neck_dim 0 means 256 */
    int32_t neck, neck_dim;
    /* memory-attention layers to write (0: none; the reference has 4):
     * "mem_attn.layers.<l>.*" and "mem_attn.norm.*" of sam3.cpp:3034-3060,
     * D = neck_dim, mem_out_dim 64, FFN 2048 */
    int32_t mem_attn_layers;
} s3e_synth_cfg;
int s3e_synth_write(const char *path, const s3e_synth_cfg *cfg);

/* Write a random-init SAM 2.x model file's image encoder (Hiera backbone +
 * FPN neck) in sam3.cpp's SAM 2 format (magic "sam2", version 1; header and
 * 57 hparams per convert_sam2_to_ggml.py:205-277, tensors per
 * sam2_register_tensors, sam3.cpp:1745-1847), weights N(0, std²) as above,
 * stored and quantized by the same rules.  Hiera-T: embed 96, heads 1,
 * stages {1,2,7,2}, global {5,7,9}, windows {8,4,14,7}, bkg 7×7; Hiera-B+:
 * 112, 2, {2,3,16,3}, {12,16,20}, {8,4,14,7}, 14×14 (convert_sam2_to_ggml.py:
 * 79-106).  Replaces the SAM 2 converter for synthetic-weight runs. */
typedef struct s3e_synth_sam2_cfg {
    int32_t img_size, embed_dim, num_heads, stages[4];
    int32_t global_n, global_idx[8], q_pool, window_spec[4], bkg_h, bkg_w, scalp;
    int32_t neck_dim, fpn_td_n, fpn_td[4];
    int32_t ftype;
    uint64_t seed;
    float std;  /* negative: also randomise biases and LayerNorm affine */
    int32_t mem_attn_layers;  /* as in s3e_synth_cfg (sam3.cpp:2004-2040) */
} s3e_synth_sam2_cfg;
int s3e_synth_write_sam2(const char *path, const s3e_synth_sam2_cfg *cfg);

#ifdef __cplusplus
}
#endif
#endif /* S3E_H */
