/*
 * orc_hiera.c — CPU oracle: the SAM 2.x Hiera image encoder and its FPN
 * neck.  TEST INFRASTRUCTURE ONLY (see orc.h).
 *
 * Graph: sam2_build_hiera_graph (sam3.cpp:4462-4527),
 * sam2_hiera_block_forward (sam3.cpp:4295-4457), sam2_window_partition /
 * unpartition (sam3.cpp:4190-4277), sam2_maxpool_2d (sam3.cpp:4283-4292),
 * sam2_compute_pos_embed + sam2_bicubic_interpolate_cpu
 * (sam3.cpp:4072-4171), sam2_build_fpn_neck_graph (sam3.cpp:4532-4603);
 * block metadata sam2_precompute_hiera_metadata (sam3.cpp:1676-1742);
 * preprocessing sam2_preprocess_image (sam3.cpp:3518-3544).
 *
 * Activations are NHWC: token (y, x) is a row of C floats (ggml [C, W, H]).
 * Windows are visited row-major; the reference's own window order
 * (sam3.cpp:4188) is internal to partition/unpartition, which invert each
 * other, so it does not change any result.  Padded window positions hold
 * zero rows of the normalised input (ggml_pad), so their queries, keys and
 * values are the QKV bias and take part in attention as real keys.
 *
 * ggml CPU semantics restated here [ext]:
 *   ggml_gelu on f32 with GGML_GELU_FP16 (ggml_vec_gelu_f32): x ≤ −10 → 0,
 *     x ≥ 10 → x, otherwise table[fp16(x)] with
 *     table[h] = fp16(0.5·v·(1 + tanhf(√(2/π)·v·(1 + 0.044715·v²)))),
 *     v = fp32(h) — every result is an fp16 value.
 *   ggml_upscale NEAREST ×2: out[y][x] = in[y/2][x/2].
 *   ggml_norm with eps 1e-6 (orc_layer_norm), conv_2d = im2col in the
 *     kernel's type + mul_mat, flash_attn_ext on F32 operands — as for SAM 3.
 *
 * Parity: pinned by tests/test_oracle_hiera.py against float64 torch
 * restatements of the block, the patch embedding, the positional embedding
 * (torch bicubic, a = −0.75) and the FPN; the GELU table against float64
 * tanh-GELU within one fp16 rounding.
 */
#include "orc.h"

#include <float.h>
#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---- ggml_gelu (tanh form) through the fp16 table ----------------------- */
static uint16_t g_gelu_tab[65536];
static int g_gelu_init = 0;

static void gelu_table_init(void) {
    if (g_gelu_init) return;
    const float SQRT_2_OVER_PI = 0.79788456080286535587989211986876f;
    const float GELU_COEF_A = 0.044715f;
    for (int i = 0; i < 65536; i++) {
        const float v = orc_fp16_to_fp32((uint16_t)i);
        const float y = 0.5f * v * (1.0f + tanhf(SQRT_2_OVER_PI * v * (1.0f + GELU_COEF_A * v * v)));
        g_gelu_tab[i] = orc_fp32_to_fp16(y);
    }
    g_gelu_init = 1;
}

void orc_gelu_tanh_table(uint16_t *out) {
    gelu_table_init();
    memcpy(out, g_gelu_tab, sizeof g_gelu_tab);
}

void orc_gelu_tanh(float *x, int64_t n) {
    gelu_table_init();
    for (int64_t i = 0; i < n; i++) {
        const float v = x[i];
        if (v <= -10.0f) x[i] = 0.0f;
        else if (v >= 10.0f) x[i] = v;
        else x[i] = orc_fp16_to_fp32(g_gelu_tab[orc_fp32_to_fp16(v)]);
    }
}

/* ---- block metadata (sam3.cpp:1676-1742) -------------------------------- */
/* out: dim_in, dim_out, heads, window (0 = global), q_stride, stage, is stage end */
int orc_hiera_block_info(const orc_model *m, int i, int32_t out[7]) {
    const orc_hiera_hp *h = orc_model_hiera(m);
    if (!h) { orc_set_error("not a SAM 2 model"); return -1; }
    int stage_ends[4], cum = 0, total = 0;
    for (int s = 0; s < 4; s++) { cum += h->stages[s]; stage_ends[s] = cum - 1; total += h->stages[s]; }
    if (i < 0 || i >= total) { orc_set_error("block %d out of range", i); return -1; }
    int q_pool_blocks[4], nq = 0;
    for (int s = 0; s < 3 && nq < h->q_pool; s++) q_pool_blocks[nq++] = stage_ends[s] + 1;
    int cur = 0, dim = h->embed_dim, heads = h->num_heads;
    for (int b = 0; b <= i; b++) {
        /* the window size lags a block: the first block of a stage still uses
         * the previous stage's window */
        int ws = h->window_spec[cur];
        for (int g = 0; g < h->global_n; g++)
            if (h->global_idx[g] == b) ws = 0;
        int dim_out = dim;
        if (b > 0 && b - 1 == stage_ends[cur]) {
            dim_out = dim * 2;
            heads *= 2;
            cur++;
        }
        int qs = 0;
        for (int k = 0; k < nq; k++)
            if (q_pool_blocks[k] == b) qs = 1;
        if (b == i) {
            out[0] = dim; out[1] = dim_out; out[2] = heads; out[3] = ws; out[4] = qs; out[5] = cur;
            out[6] = (b == stage_ends[cur]);
        }
        dim = dim_out;
    }
    return 0;
}

int orc_hiera_num_blocks(const orc_model *m) {
    const orc_hiera_hp *h = orc_model_hiera(m);
    return h ? h->stages[0] + h->stages[1] + h->stages[2] + h->stages[3] : 0;
}

/* ---- positional embedding (sam3.cpp:4072-4171) --------------------------- */
/* sam2_bicubic_interpolate_cpu: src [C][Hi][Wi] → dst [C][Ho][Wo], Keys cubic
 * a = −0.75, half-pixel centres, clamped taps, float arithmetic in the
 * reference's order. */
void orc_bicubic(const float *src, int C, int Hi, int Wi, float *dst, int Ho, int Wo) {
    for (int c = 0; c < C; ++c)
        for (int y = 0; y < Ho; ++y) {
            const float fy = ((float)y + 0.5f) * (float)Hi / (float)Ho - 0.5f;
            const int iy = (int)floorf(fy);
            const float dy = fy - iy;
            for (int x = 0; x < Wo; ++x) {
                const float fx = ((float)x + 0.5f) * (float)Wi / (float)Wo - 0.5f;
                const int ix = (int)floorf(fx);
                const float dx = fx - ix;
                float val = 0.0f;
                for (int jj = -1; jj <= 2; ++jj) {
                    float t = fabsf(dy - jj);
                    const float wy = t < 1.0f ? (1.25f * t - 2.25f) * t * t + 1.0f
                                              : (t < 2.0f ? ((-0.75f * t + 3.75f) * t - 6.0f) * t + 3.0f : 0.0f);
                    int sy = iy + jj;
                    sy = sy < 0 ? 0 : (sy > Hi - 1 ? Hi - 1 : sy);
                    for (int ii = -1; ii <= 2; ++ii) {
                        float u = fabsf(dx - ii);
                        const float wx = u < 1.0f ? (1.25f * u - 2.25f) * u * u + 1.0f
                                                  : (u < 2.0f ? ((-0.75f * u + 3.75f) * u - 6.0f) * u + 3.0f : 0.0f);
                        int sx = ix + ii;
                        sx = sx < 0 ? 0 : (sx > Wi - 1 ? Wi - 1 : sx);
                        val += wy * wx * src[(size_t)c * Hi * Wi + sy * Wi + sx];
                    }
                }
                dst[(size_t)c * Ho * Wo + y * Wo + x] = val;
            }
        }
}

/* PE [H][W][E] = bicubic(pos_embed) + tile(pos_embed_window) */
int orc_hiera_pos_embed(const orc_model *m, int H, int W, float *out) {
    const orc_hiera_hp *h = orc_model_hiera(m);
    if (!h) { orc_set_error("not a SAM 2 model"); return -1; }
    orc_tensor_view bkg, win;
    if (orc_model_tensor(m, "hiera.", "pos_embed", &bkg) || orc_model_tensor(m, "hiera.", "pos_embed_window", &win))
        return -1;
    const int E = h->embed_dim, bh = (int)bkg.ne[1], bw = (int)bkg.ne[0], ws = (int)win.ne[0];
    /* registered [bkg_w, bkg_h, E, 1]: the bytes are CHW [E][bkg_h][bkg_w] */
    float *interp = (float *)malloc(sizeof(float) * (size_t)E * H * W);
    orc_bicubic((const float *)bkg.data, E, bh, bw, interp, H, W);
    const float *wd = (const float *)win.data;
    for (int y = 0; y < H; ++y)
        for (int x = 0; x < W; ++x)
            for (int e = 0; e < E; ++e)
                out[((size_t)y * W + x) * E + e] =
                    interp[(size_t)e * H * W + y * W + x] + wd[(size_t)e * ws * ws + (y % ws) * ws + (x % ws)];
    free(interp);
    return 0;
}

/* sam2_preprocess_image normalisation (sam3.cpp:3518-3544) after the same
 * bilinear resize as SAM 3: HWC uint8 → CHW f32. */
void orc_preprocess_sam2(const uint8_t *img, int w, int h, int img_size, float *chw) {
    static const float mean[3] = {0.485f, 0.456f, 0.406f};
    static const float stdv[3] = {0.229f, 0.224f, 0.225f};
    uint8_t *rs = (uint8_t *)malloc((size_t)img_size * img_size * 3);
    if (w != img_size || h != img_size) orc_resize_bilinear_u8(img, w, h, rs, img_size, img_size);
    else memcpy(rs, img, (size_t)img_size * img_size * 3);
    for (int c = 0; c < 3; ++c)
        for (int y = 0; y < img_size; ++y)
            for (int x = 0; x < img_size; ++x) {
                const float v = rs[((size_t)y * img_size + x) * 3 + c] / 255.0f;
                chw[(size_t)c * img_size * img_size + (size_t)y * img_size + x] = (v - mean[c]) / stdv[c];
            }
    free(rs);
}

/* ---- convolution with stride (ggml_conv_2d via im2col) ------------------- */
/* x NHWC [H][W][Cin] → y [OH][OW][Cout], kernel ggml [KW, KH, Cin, Cout] */
static void conv2d_strided(int ktype, const void *w, int KW, int KH, int Cin, int Cout, int stride, int pad,
                           const float *x, int H, int W, float *y, int nthreads) {
    const int OH = (H + 2 * pad - KH) / stride + 1, OW = (W + 2 * pad - KW) / stride + 1;
    const int64_t K = (int64_t)Cin * KH * KW;
    const size_t rs = orc_row_size(ktype, K);
#pragma omp parallel num_threads(nthreads)
    {
        float *col = (float *)malloc(sizeof(float) * (size_t)K);
        char *colt = (char *)malloc(rs);
#pragma omp for schedule(dynamic, 16)
        for (int64_t p = 0; p < (int64_t)OH * OW; p++) {
            const int oy = (int)(p / OW), ox = (int)(p % OW);
            for (int ic = 0; ic < Cin; ic++)
                for (int kh = 0; kh < KH; kh++)
                    for (int kw = 0; kw < KW; kw++) {
                        const int iy = oy * stride + kh - pad, ix = ox * stride + kw - pad;
                        const int in = iy >= 0 && iy < H && ix >= 0 && ix < W;
                        col[((int64_t)ic * KH + kh) * KW + kw] = in ? x[((int64_t)iy * W + ix) * Cin + ic] : 0.0f;
                    }
            orc_from_float(ktype, col, colt, K);
            for (int oc = 0; oc < Cout; oc++)
                y[p * Cout + oc] = orc_vec_dot(ktype, K, colt, (const char *)w + (size_t)oc * rs);
        }
        free(col);
        free(colt);
    }
}

/* Patch embedding 7×7 / stride 4 / pad 3 + bias + positional embedding:
 * chw [3][S][S] → x [S/4][S/4][E] (sam3.cpp:4469-4490). */
int orc_hiera_prefix(const orc_model *m, const float *chw, float *x, int nthreads) {
    const orc_hiera_hp *h = orc_model_hiera(m);
    if (!h) { orc_set_error("not a SAM 2 model"); return -1; }
    if (nthreads <= 0) nthreads = omp_get_max_threads();
    orc_tensor_view pw, pb;
    if (orc_model_tensor(m, "hiera.", "patch_embed.weight", &pw) || orc_model_tensor(m, "hiera.", "patch_embed.bias", &pb))
        return -1;
    const int S = h->img_size, E = h->embed_dim, G = S / 4;
    float *hwc = (float *)malloc(sizeof(float) * (size_t)S * S * 3);
    for (int c = 0; c < 3; c++)
        for (int64_t i = 0; i < (int64_t)S * S; i++) hwc[i * 3 + c] = chw[(int64_t)c * S * S + i];
    conv2d_strided(pw.type, pw.data, 7, 7, 3, E, 4, 3, hwc, S, S, x, nthreads);
    free(hwc);
    float *pe = (float *)malloc(sizeof(float) * (size_t)G * G * E);
    if (orc_hiera_pos_embed(m, G, G, pe) != 0) { free(pe); return -1; }
    const float *b = (const float *)pb.data;
    for (int64_t t = 0; t < (int64_t)G * G; t++)
        for (int e = 0; e < E; e++) x[t * E + e] = (x[t * E + e] + b[e]) + pe[t * E + e];
    free(pe);
    return 0;
}

static void add_bias_rows(float *y, int64_t rows, int64_t C, const float *b) {
    for (int64_t r = 0; r < rows; r++)
        for (int64_t c = 0; c < C; c++) y[r * C + c] = y[r * C + c] + b[c];
}

/* One MultiScaleBlock (sam3.cpp:4295-4457): x [H][W][Cin] → y [Ho][Wo][Cout]
 * with (Ho, Wo) = (H/2, W/2) under Q pooling.  Ho_out, Wo_out receive the output
 * size; y must hold Ho·Wo·Cout floats. */
int orc_hiera_block(const orc_model *m, int bi, const float *x, int H, int W, float *y, int *Ho_out, int *Wo_out,
                    int nthreads) {
    int32_t info[7];
    if (orc_hiera_block_info(m, bi, info) != 0) return -1;
    if (nthreads <= 0) nthreads = omp_get_max_threads();
    const int Cin = info[0], Cout = info[1], NH = info[2], ws = info[3], qs = info[4];
    const int HD = Cout / NH;
    char p[48];
    snprintf(p, sizeof p, "hiera.blocks.%d.", bi);
    orc_tensor_view n1w, n1b, qw, qb, pjw, pjb, n2w, n2b, f1w, f1b, f2w, f2b, dpw, dpb;
    if (orc_model_tensor(m, p, "norm1.weight", &n1w) || orc_model_tensor(m, p, "norm1.bias", &n1b) ||
        orc_model_tensor(m, p, "attn.qkv.weight", &qw) || orc_model_tensor(m, p, "attn.qkv.bias", &qb) ||
        orc_model_tensor(m, p, "attn.proj.weight", &pjw) || orc_model_tensor(m, p, "attn.proj.bias", &pjb) ||
        orc_model_tensor(m, p, "norm2.weight", &n2w) || orc_model_tensor(m, p, "norm2.bias", &n2b) ||
        orc_model_tensor(m, p, "mlp.fc1.weight", &f1w) || orc_model_tensor(m, p, "mlp.fc1.bias", &f1b) ||
        orc_model_tensor(m, p, "mlp.fc2.weight", &f2w) || orc_model_tensor(m, p, "mlp.fc2.bias", &f2b))
        return -1;
    if (Cin != Cout && (orc_model_tensor(m, p, "proj.weight", &dpw) || orc_model_tensor(m, p, "proj.bias", &dpb)))
        return -1;
    const int64_t T = (int64_t)H * W;
    const int Ht = qs ? H / 2 : H, Wt = qs ? W / 2 : W;
    const int64_t Tt = (int64_t)Ht * Wt;
    /* 1. pre-norm */
    float *normed = (float *)malloc(sizeof(float) * (size_t)T * Cin);
    orc_layer_norm(x, normed, T, Cin, 1e-6f, (const float *)n1w.data, (const float *)n1b.data, nthreads);
    /* 2. shortcut: dim projection of the normed input, max-pooled under Q stride */
    float *sc = (float *)malloc(sizeof(float) * (size_t)Tt * Cout);
    if (Cin != Cout) {
        float *pr = (float *)malloc(sizeof(float) * (size_t)T * Cout);
        orc_mul_mat(dpw.type, dpw.data, Cout, Cin, normed, T, pr, nthreads);
        add_bias_rows(pr, T, Cout, (const float *)dpb.data);
        if (qs) orc_maxpool2x2(pr, H, W, Cout, sc);
        else memcpy(sc, pr, sizeof(float) * (size_t)T * Cout);
        free(pr);
    } else if (qs) {
        orc_maxpool2x2(x, H, W, Cin, sc);
    } else {
        memcpy(sc, x, sizeof(float) * (size_t)T * Cin);
    }
    /* 3. windows (row-major), padded with zero rows */
    int wh, ww, nwh, nww;
    if (ws > 0) {
        wh = ww = ws;
        nwh = (H + ws - 1) / ws;
        nww = (W + ws - 1) / ws;
    } else {
        wh = H; ww = W; nwh = nww = 1;
    }
    const int NW = nwh * nww, Nkv = wh * ww;
    float *A = (float *)calloc((size_t)NW * Nkv * Cin, sizeof(float));
    for (int w = 0; w < NW; w++)
        for (int iy = 0; iy < wh; iy++)
            for (int ix = 0; ix < ww; ix++) {
                const int ty = (w / nww) * wh + iy, tx = (w % nww) * ww + ix;
                if (ty < H && tx < W)
                    memcpy(A + ((int64_t)w * Nkv + iy * ww + ix) * Cin, normed + ((int64_t)ty * W + tx) * Cin,
                           sizeof(float) * Cin);
            }
    free(normed);
    /* 4. QKV + bias, Q pooled inside each window, attention */
    float *qkv = (float *)malloc(sizeof(float) * (size_t)NW * Nkv * 3 * Cout);
    orc_mul_mat(qw.type, qw.data, 3 * Cout, Cin, A, (int64_t)NW * Nkv, qkv, nthreads);
    free(A);
    add_bias_rows(qkv, (int64_t)NW * Nkv, 3 * Cout, (const float *)qb.data);
    const int qh = qs ? wh / 2 : wh, qw_ = qs ? ww / 2 : ww, Nq = qh * qw_;
    float *Q = (float *)malloc(sizeof(float) * (size_t)NW * Nq * Cout);
    for (int w = 0; w < NW; w++)
        for (int py = 0; py < qh; py++)
            for (int px = 0; px < qw_; px++)
                for (int c = 0; c < Cout; c++) {
                    float v;
                    if (qs) {
                        v = -FLT_MAX;
                        for (int dy = 0; dy < 2; dy++)
                            for (int dx = 0; dx < 2; dx++) {
                                const float u = qkv[((int64_t)w * Nkv + (2 * py + dy) * ww + 2 * px + dx) * 3 * Cout + c];
                                if (u > v) v = u;
                            }
                    } else {
                        v = qkv[((int64_t)w * Nkv + py * ww + px) * 3 * Cout + c];
                    }
                    Q[((int64_t)w * Nq + py * qw_ + px) * Cout + c] = v;
                }
    float *O = (float *)malloc(sizeof(float) * (size_t)NW * Nq * Cout);
    orc_flash_attn_ext(Q, Cout, HD, (int64_t)Nq * Cout,
                       qkv + Cout, 3 * Cout, HD, (int64_t)Nkv * 3 * Cout,
                       qkv + 2 * Cout, 3 * Cout, HD, (int64_t)Nkv * 3 * Cout,
                       HD, Nq, Nkv, NH, NW, 1.0f / sqrtf((float)HD), O, nthreads);
    free(Q);
    free(qkv);
    float *PJ = (float *)malloc(sizeof(float) * (size_t)NW * Nq * Cout);
    orc_mul_mat(pjw.type, pjw.data, Cout, Cout, O, (int64_t)NW * Nq, PJ, nthreads);
    free(O);
    add_bias_rows(PJ, (int64_t)NW * Nq, Cout, (const float *)pjb.data);
    /* 5. un-partition (crop) + 6. residual */
    float *r1 = sc;  /* res1 = shortcut + attention, in place */
    for (int w = 0; w < NW; w++)
        for (int py = 0; py < qh; py++)
            for (int px = 0; px < qw_; px++) {
                const int ty = (w / nww) * qh + py, tx = (w % nww) * qw_ + px;
                if (ty >= Ht || tx >= Wt) continue;
                float *dst = r1 + ((int64_t)ty * Wt + tx) * Cout;
                const float *src = PJ + ((int64_t)w * Nq + py * qw_ + px) * Cout;
                for (int c = 0; c < Cout; c++) dst[c] = dst[c] + src[c];
            }
    free(PJ);
    /* 7. MLP + residual */
    const int MLP = (int)f1w.ne[1];
    float *n2 = (float *)malloc(sizeof(float) * (size_t)Tt * Cout);
    orc_layer_norm(r1, n2, Tt, Cout, 1e-6f, (const float *)n2w.data, (const float *)n2b.data, nthreads);
    float *h1 = (float *)malloc(sizeof(float) * (size_t)Tt * MLP);
    orc_mul_mat(f1w.type, f1w.data, MLP, Cout, n2, Tt, h1, nthreads);
    add_bias_rows(h1, Tt, MLP, (const float *)f1b.data);
    orc_gelu_tanh(h1, Tt * MLP);
    orc_mul_mat(f2w.type, f2w.data, Cout, MLP, h1, Tt, n2, nthreads);
    const float *b2 = (const float *)f2b.data;
    for (int64_t t = 0; t < Tt; t++)
        for (int c = 0; c < Cout; c++) y[t * Cout + c] = r1[t * Cout + c] + (n2[t * Cout + c] + b2[c]);
    free(h1);
    free(n2);
    free(sc);
    *Ho_out = Ht;
    *Wo_out = Wt;
    return 0;
}

/* sam2_build_fpn_neck_graph (sam3.cpp:4532-4603): stage outputs (NHWC, side
 * s[i], width C[i]) → FPN levels 0 .. 3 − scalp, each [s[i]²][D].  out[3]
 * may be NULL when scalp ≥ 1 (the level is still formed for the top-down
 * path). */
int orc_hiera_fpn(const orc_model *m, float *const stage[4], const int side[4], float *out[4], int nthreads) {
    const orc_hiera_hp *h = orc_model_hiera(m);
    if (!h) { orc_set_error("not a SAM 2 model"); return -1; }
    if (nthreads <= 0) nthreads = omp_get_max_threads();
    const int D = h->neck_dim;
    float *lat[4] = {NULL, NULL, NULL, NULL};
    int rc = -1;
    for (int i = 0; i < 4; i++) {
        char p[32];
        snprintf(p, sizeof p, "fpn.convs.%d.", 3 - i);
        orc_tensor_view w, b;
        if (orc_model_tensor(m, p, "weight", &w) || orc_model_tensor(m, p, "bias", &b)) goto done;
        const int ch = (int)w.ne[2];
        lat[i] = (float *)malloc(sizeof(float) * (size_t)side[i] * side[i] * D);
        orc_conv2d(w.type, w.data, 1, 1, ch, D, 0, stage[i], side[i], side[i], lat[i], nthreads);
        add_bias_rows(lat[i], (int64_t)side[i] * side[i], D, (const float *)b.data);
    }
    {
        const float *prev = NULL;
        int prev_side = 0;
        for (int i = 3; i >= 0; i--) {
            int td = 0;
            for (int j = 0; j < h->fpn_td_n; j++)
                if (h->fpn_td[j] == i) td = 1;
            if (td && prev) {
                for (int y = 0; y < side[i]; y++)
                    for (int x = 0; x < side[i]; x++) {
                        float *d = lat[i] + ((int64_t)y * side[i] + x) * D;
                        const float *u = prev + ((int64_t)(y / 2) * prev_side + x / 2) * D;
                        for (int c = 0; c < D; c++) d[c] = d[c] + u[c];
                    }
                prev = lat[i];
                prev_side = side[i];
            } else if (td || !prev) {
                prev = lat[i];
                prev_side = side[i];
            }
        }
    }
    for (int i = 0; i < 4; i++)
        if (out[i]) memcpy(out[i], lat[i], sizeof(float) * (size_t)side[i] * side[i] * D);
    rc = 0;
done:
    for (int i = 0; i < 4; i++) free(lat[i]);
    return rc;
}

/* Stage sides and widths of the encoder for img_size (stage i: side, width). */
int orc_hiera_dims(const orc_model *m, int side[4], int width[4]) {
    const orc_hiera_hp *h = orc_model_hiera(m);
    if (!h) { orc_set_error("not a SAM 2 model"); return -1; }
    int s = h->img_size / 4, d = h->embed_dim;
    for (int i = 0; i < 4; i++) {
        if (i > 0 && i <= h->q_pool) s /= 2;
        side[i] = s;
        width[i] = d;
        d *= 2;
    }
    return 0;
}

/* Whole encoder: chw → FPN levels out[0 .. 3 − scalp] (others may be NULL),
 * optionally the four stage outputs. */
int orc_hiera_encode(const orc_model *m, const float *chw, float *out[4], float *stage_out[4], int nthreads) {
    const orc_hiera_hp *h = orc_model_hiera(m);
    if (!h) { orc_set_error("not a SAM 2 model"); return -1; }
    int side[4], width[4];
    orc_hiera_dims(m, side, width);
    const int G = h->img_size / 4;
    float *x = (float *)malloc(sizeof(float) * (size_t)G * G * h->embed_dim);
    float *st[4] = {NULL, NULL, NULL, NULL};
    int rc = -1;
    if (orc_hiera_prefix(m, chw, x, nthreads) != 0) goto done;
    {
        int H = G, W = G, stage = 0;
        const int nb = orc_hiera_num_blocks(m);
        for (int b = 0; b < nb; b++) {
            int32_t info[7];
            orc_hiera_block_info(m, b, info);
            const int Ho = info[4] ? H / 2 : H, Wo = info[4] ? W / 2 : W;
            float *y = (float *)malloc(sizeof(float) * (size_t)Ho * Wo * info[1]);
            int ho, wo;
            if (orc_hiera_block(m, b, x, H, W, y, &ho, &wo, nthreads) != 0) { free(y); goto done; }
            free(x);
            x = y;
            H = ho;
            W = wo;
            if (info[6]) {
                st[stage] = (float *)malloc(sizeof(float) * (size_t)H * W * info[1]);
                memcpy(st[stage], x, sizeof(float) * (size_t)H * W * info[1]);
                if (stage_out && stage_out[stage]) memcpy(stage_out[stage], x, sizeof(float) * (size_t)H * W * info[1]);
                stage++;
            }
        }
        if (stage != 4) { orc_set_error("found %d stage ends", stage); goto done; }
    }
    {
        float *lv[4];
        for (int i = 0; i < 4; i++) lv[i] = out[i];
        rc = orc_hiera_fpn(m, st, side, lv, nthreads);
    }
done:
    free(x);
    for (int i = 0; i < 4; i++) free(st[i]);
    return rc;
}
