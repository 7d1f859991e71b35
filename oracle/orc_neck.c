/*
 * orc_neck.c — CPU oracle: the SAM 3 SimpleFPN neck and the sinusoidal
 * position encodings stored beside its outputs.  TEST INFRASTRUCTURE ONLY
 * (see orc.h).
 *
 * Graph: sam3_build_neck_graph (sam3.cpp:3863-3921), weights registered at
 * sam3.cpp:2562-2591, deconvolution kernels cast to F16 by
 * sam3_conv_transpose_weight (sam3.cpp:1083-1086).  PEs:
 * sam3_sinusoidal_pe_2d (sam3.cpp:3597-3633), one per level
 * (sam3.cpp:6146-6193).
 *
 * ggml CPU semantics restated here [ext] (ggml-cpu ops.cpp):
 *   conv_transpose_2d, F16 kernel and F32 input: the kernel is permuted to
 *     [Cout][kH][kW][Cin] and the input converted to fp16 as [H][W][Cin]
 *     (round to nearest even); each output element (y·s + ky, x·s + kx, co)
 *     accumulates ggml_vec_dot_f16 over Cin into a zeroed destination.  With
 *     kernel 2 and stride 2 every output receives exactly one dot.
 *   conv_2d = im2col + mul_mat: im2col writes the input in the kernel's type
 *     with K ordered [Cin][kH][kW] (kW fastest) and zeros outside the image;
 *     mul_mat(im2col, kernel) takes one vec_dot of the kernel's type per
 *     (pixel, output channel).  The kernel's ggml layout [kW, kH, Cin, Cout]
 *     makes each output channel's row exactly that K order.
 *   pool_2d MAX: maximum over the window, starting from -FLT_MAX; output
 *     size (in - k)/s + 1.
 *   add (bias broadcast over pixels) and gelu_erf in f32.
 *
 * Activations here are NHWC: pixel (y, x) is a row of C contiguous floats,
 * which is the memory order of the neck's outputs after their final permute
 * ([C, W, H] in ggml's ne order).
 *
 * Parity: conv_transpose / conv_2d / pool / the neck composition are pinned
 * by float64 torch.nn.functional restatements on the same rounded operands
 * (tests/test_oracle_neck.py); the PE by its closed form in float64.
 */
#include "orc.h"

#include <float.h>
#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ggml_conv_transpose_2d_p0(kernel, x, 2) with a 2×2 kernel. */
void orc_conv_transpose_2x2(const uint16_t *w16, int64_t Cin, int64_t Cout, const float *x, int64_t H,
                            int64_t W, float *y, int nthreads) {
    if (nthreads <= 0) nthreads = omp_get_max_threads();
    /* kernel element (kx, ky, co, ci) sits at ((ci·Cout + co)·2 + ky)·2 + kx */
    uint16_t *kp = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(4 * Cout * Cin));
    for (int64_t ci = 0; ci < Cin; ci++)
        for (int64_t co = 0; co < Cout; co++)
            for (int ky = 0; ky < 2; ky++)
                for (int kx = 0; kx < 2; kx++)
                    kp[((co * 2 + ky) * 2 + kx) * Cin + ci] = w16[((ci * Cout + co) * 2 + ky) * 2 + kx];
    uint16_t *xh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(H * W * Cin));
#pragma omp parallel for num_threads(nthreads)
    for (int64_t p = 0; p < H * W; p++) orc_fp32_to_fp16_row(x + p * Cin, xh + p * Cin, Cin);
    const int64_t OW = 2 * W;
#pragma omp parallel for schedule(dynamic, 4) num_threads(nthreads)
    for (int64_t p = 0; p < H * W; p++) {
        const int64_t iy = p / W, ix = p % W;
        for (int ky = 0; ky < 2; ky++)
            for (int kx = 0; kx < 2; kx++) {
                float *yr = y + ((2 * iy + ky) * OW + 2 * ix + kx) * Cout;
                for (int64_t co = 0; co < Cout; co++)
                    yr[co] = 0.0f + orc_vec_dot(ORC_TYPE_F16, Cin, kp + ((co * 2 + ky) * 2 + kx) * Cin,
                                                xh + p * Cin);
            }
    }
    free(kp);
    free(xh);
}

/* ggml_conv_2d(kernel, x, 1, 1, pad, pad, 1, 1): stride 1, dilation 1.
 * ktype is the kernel's type (F32 or F16); kernel ggml [KW, KH, Cin, Cout]. */
void orc_conv2d(int ktype, const void *w, int64_t KW, int64_t KH, int64_t Cin, int64_t Cout, int64_t pad,
                const float *x, int64_t H, int64_t W, float *y, int nthreads) {
    if (nthreads <= 0) nthreads = omp_get_max_threads();
    const int64_t OH = H + 2 * pad - KH + 1, OW = W + 2 * pad - KW + 1;
    const int64_t K = Cin * KH * KW;
    const size_t rs = orc_row_size(ktype, K);
#pragma omp parallel num_threads(nthreads)
    {
        float *col = (float *)malloc(sizeof(float) * (size_t)K);
        char *colt = (char *)malloc(rs);
#pragma omp for schedule(dynamic, 16)
        for (int64_t p = 0; p < OH * OW; p++) {
            const int64_t oy = p / OW, ox = p % OW;
            for (int64_t ic = 0; ic < Cin; ic++)
                for (int64_t kh = 0; kh < KH; kh++)
                    for (int64_t kw = 0; kw < KW; kw++) {
                        const int64_t iy = oy + kh - pad, ix = ox + kw - pad;
                        const int in = iy >= 0 && iy < H && ix >= 0 && ix < W;
                        col[(ic * KH + kh) * KW + kw] = in ? x[(iy * W + ix) * Cin + ic] : 0.0f;
                    }
            orc_from_float(ktype, col, colt, K);
            float *yr = y + p * Cout;
            for (int64_t oc = 0; oc < Cout; oc++)
                yr[oc] = orc_vec_dot(ktype, K, colt, (const char *)w + (size_t)oc * rs);
        }
        free(col);
        free(colt);
    }
}

/* ggml_pool_2d(x, MAX, 2, 2, 2, 2, 0, 0) on NHWC. */
void orc_maxpool2x2(const float *x, int64_t H, int64_t W, int64_t C, float *y) {
    const int64_t OH = (H - 2) / 2 + 1, OW = (W - 2) / 2 + 1;
    for (int64_t oy = 0; oy < OH; oy++)
        for (int64_t ox = 0; ox < OW; ox++)
            for (int64_t c = 0; c < C; c++) {
                float m = -FLT_MAX;
                for (int ky = 0; ky < 2; ky++)
                    for (int kx = 0; kx < 2; kx++) {
                        const float v = x[((2 * oy + ky) * W + 2 * ox + kx) * C + c];
                        if (v > m) m = v;
                    }
                y[(oy * OW + ox) * C + c] = m;
            }
}

/* sam3_sinusoidal_pe_2d (sam3.cpp:3597-3633): out [H][W][d_model]; channels
 * [0, d/2) encode y, [d/2, d) encode x; even channels sin, odd cos. */
void orc_sinusoidal_pe_2d(int H, int W, int d_model, float *out) {
    const int half = d_model / 2;
    const float scale = 2.0f * (float)M_PI;
    for (int y = 0; y < H; ++y)
        for (int x = 0; x < W; ++x) {
            const float pos_y = ((float)(y + 1) / (float)H) * scale;
            const float pos_x = ((float)(x + 1) / (float)W) * scale;
            float *o = out + ((size_t)y * W + x) * d_model;
            for (int i = 0; i < half; ++i) {
                const int paired = i & ~1;
                const float dim_t = powf(10000.0f, (float)paired / (float)half);
                o[i] = (i % 2 == 0) ? sinf(pos_y / dim_t) : cosf(pos_y / dim_t);
                o[i + half] = (i % 2 == 0) ? sinf(pos_x / dim_t) : cosf(pos_x / dim_t);
            }
        }
}

static void add_bias(float *y, int64_t rows, int64_t C, const float *b) {
    for (int64_t r = 0; r < rows; r++)
        for (int64_t c = 0; c < C; c++) y[r * C + c] = y[r * C + c] + b[c];
}

/* The kernel of a deconvolution as fp16 (ggml_cast to F16 unless F16). */
static uint16_t *as_f16(const orc_tensor_view *t) {
    const int64_t n = t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3];
    uint16_t *h = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)n);
    if (t->type == ORC_TYPE_F16) memcpy(h, t->data, sizeof(uint16_t) * (size_t)n);
    else orc_fp32_to_fp16_row((const float *)t->data, h, n);
    return h;
}

#define NECK_T(var, suffix)                                                        \
    orc_tensor_view var;                                                           \
    if (orc_model_tensor(m, prefix, suffix, &var) != 0) return -1;
/* the same inside orc_neck, which frees its buffers on the way out */
#define NECK_TG(var, suffix)                                                       \
    orc_tensor_view var;                                                           \
    if (orc_model_tensor(m, prefix, suffix, &var) != 0) goto done;

/* Deconvolution + bias (sam3.cpp:3880-3881, 3883-3884, 3894-3895). */
static int deconv(const orc_model *m, const char *prefix, const char *wname, const char *bname, const float *x,
                  int64_t H, int64_t W, int64_t Cin, float *y, int64_t *Cout, int nthreads) {
    NECK_T(w, wname);
    NECK_T(b, bname);
    if (w.ne[0] != 2 || w.ne[1] != 2 || w.ne[3] != Cin || b.ne[0] != w.ne[2]) {
        orc_set_error("%s%s: unexpected shape", prefix, wname);
        return -1;
    }
    *Cout = w.ne[2];
    uint16_t *w16 = as_f16(&w);
    orc_conv_transpose_2x2(w16, Cin, *Cout, x, H, W, y, nthreads);
    free(w16);
    add_bias(y, 4 * H * W, *Cout, (const float *)b.data);
    return 0;
}

/* Convolution (stride 1, pad k/2) + bias (ggml_conv_2d_sk_p0 for 1×1,
 * ggml_conv_2d_s1_ph for 3×3). */
static int conv(const orc_model *m, const char *prefix, const char *wname, const char *bname, const float *x,
                int64_t H, int64_t W, int64_t Cin, float *y, int64_t *Cout, int nthreads) {
    NECK_T(w, wname);
    NECK_T(b, bname);
    if (w.ne[2] != Cin || b.ne[0] != w.ne[3] || w.ne[0] != w.ne[1]) {
        orc_set_error("%s%s: unexpected shape", prefix, wname);
        return -1;
    }
    *Cout = w.ne[3];
    orc_conv2d(w.type, w.data, w.ne[0], w.ne[1], Cin, *Cout, w.ne[0] / 2, x, H, W, y, nthreads);
    add_bias(y, H * W, *Cout, (const float *)b.data);
    return 0;
}

int orc_neck_dims(const orc_model *m, const char *which, int64_t side[4], int64_t *D) {
    char prefix[32];
    snprintf(prefix, sizeof prefix, "neck.%s.", which);
    NECK_T(w, "0.conv_3x3.weight");
    int32_t hp[16];
    orc_model_hparams(m, hp);
    const int64_t G = hp[0] / hp[1];
    side[0] = 4 * G; side[1] = 2 * G; side[2] = G; side[3] = (G - 2) / 2 + 1;
    *D = w.ne[3];
    return 0;
}

/* sam3_build_neck_graph (sam3.cpp:3863-3921) for neck "trk" or "det".
 * x: vit_output, G² rows of E.  out[i]: side[i]² rows of D (orc_neck_dims). */
int orc_neck(const orc_model *m, const char *which, const float *x, float *out[4], int nthreads) {
    char prefix[32];
    snprintf(prefix, sizeof prefix, "neck.%s.", which);
    int32_t hp[16];
    orc_model_hparams(m, hp);
    const int64_t G = hp[0] / hp[1], E = hp[2], Gh = (G - 2) / 2 + 1;
    int64_t c1 = 0, c2 = 0, c3 = 0, c4 = 0;
    int rc = -1;
    float *t1 = NULL, *t2 = NULL, *t3 = NULL;
#define NEWBUF(p, n) do { free(p); (p) = (float *)malloc(sizeof(float) * (size_t)(n)); } while (0)
    /* scale 0 (4×): deconv, gelu_erf, deconv, 1×1, 3×3 */
    {
        NECK_TG(w1, "0.dconv_2x2_0.weight");
        NECK_TG(w2, "0.dconv_2x2_1.weight");
        NECK_TG(w3, "0.conv_1x1.weight");
        NEWBUF(t1, 4 * G * G * w1.ne[2]);
        NEWBUF(t2, 16 * G * G * w2.ne[2]);
        NEWBUF(t3, 16 * G * G * w3.ne[3]);
        if (deconv(m, prefix, "0.dconv_2x2_0.weight", "0.dconv_2x2_0.bias", x, G, G, E, t1, &c1, nthreads)) goto done;
        orc_gelu_erf(t1, 4 * G * G * c1);
        if (deconv(m, prefix, "0.dconv_2x2_1.weight", "0.dconv_2x2_1.bias", t1, 2 * G, 2 * G, c1, t2, &c2, nthreads)) goto done;
        if (conv(m, prefix, "0.conv_1x1.weight", "0.conv_1x1.bias", t2, 4 * G, 4 * G, c2, t3, &c3, nthreads)) goto done;
        if (conv(m, prefix, "0.conv_3x3.weight", "0.conv_3x3.bias", t3, 4 * G, 4 * G, c3, out[0], &c4, nthreads)) goto done;
    }
    /* scale 1 (2×): deconv, 1×1, 3×3 */
    {
        NECK_TG(w1, "1.dconv_2x2.weight");
        NECK_TG(w2, "1.conv_1x1.weight");
        NEWBUF(t1, 4 * G * G * w1.ne[2]);
        NEWBUF(t2, 4 * G * G * w2.ne[3]);
        if (deconv(m, prefix, "1.dconv_2x2.weight", "1.dconv_2x2.bias", x, G, G, E, t1, &c1, nthreads)) goto done;
        if (conv(m, prefix, "1.conv_1x1.weight", "1.conv_1x1.bias", t1, 2 * G, 2 * G, c1, t2, &c2, nthreads)) goto done;
        if (conv(m, prefix, "1.conv_3x3.weight", "1.conv_3x3.bias", t2, 2 * G, 2 * G, c2, out[1], &c3, nthreads)) goto done;
    }
    /* scale 2 (1×): 1×1, 3×3 */
    {
        NECK_TG(w1, "2.conv_1x1.weight");
        NEWBUF(t1, G * G * w1.ne[3]);
        if (conv(m, prefix, "2.conv_1x1.weight", "2.conv_1x1.bias", x, G, G, E, t1, &c1, nthreads)) goto done;
        if (conv(m, prefix, "2.conv_3x3.weight", "2.conv_3x3.bias", t1, G, G, c1, out[2], &c2, nthreads)) goto done;
    }
    /* scale 3 (0.5×): maxpool 2×2, 1×1, 3×3 */
    {
        NECK_TG(w1, "3.conv_1x1.weight");
        NEWBUF(t3, Gh * Gh * E);
        NEWBUF(t1, Gh * Gh * w1.ne[3]);
        orc_maxpool2x2(x, G, G, E, t3);
        if (conv(m, prefix, "3.conv_1x1.weight", "3.conv_1x1.bias", t3, Gh, Gh, E, t1, &c1, nthreads)) goto done;
        if (conv(m, prefix, "3.conv_3x3.weight", "3.conv_3x3.bias", t1, Gh, Gh, c1, out[3], &c2, nthreads)) goto done;
    }
    rc = 0;
done:
#undef NEWBUF
    free(t1);
    free(t2);
    free(t3);
    return rc;
}
