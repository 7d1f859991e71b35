/*
 * asan_check.c — drives every entry point of the CPU oracle once on small,
 * odd-sized inputs, for the AddressSanitizer / UndefinedBehaviorSanitizer
 * build (`make -C oracle asan`).  TEST INFRASTRUCTURE ONLY, like the rest of
 * oracle/: the sanitizers do the checking here; the program itself only
 * checks that every output is finite.
 *
 *     asan_check                      formats, products and operators
 *     asan_check MODEL.ggml [...]     also load each model and run its
 *                                     encoder (ViT + necks, or Hiera + FPN)
 *                                     and its memory attention, if present
 *     asan_check --load-only FILE...  only load (and free) each file: for
 *                                     damaged copies of a model
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "orc.h"

static int failures = 0;

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static float frand(void) {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (float)((rng_state >> 40) & 0xFFFFFF) / (float)0x800000 - 1.0f;  /* [-1, 1) */
}
static float *frand_buf(size_t n, float scale) {
    float *p = malloc(n * sizeof(float));
    for (size_t i = 0; i < n; i++) p[i] = frand() * scale;
    return p;
}
static void check_finite(const char *what, const float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (!isfinite(x[i])) {
            fprintf(stderr, "asan_check: %s: non-finite value at %zu\n", what, i);
            failures++;
            return;
        }
}

static void formats(void) {
    const int types[] = {ORC_TYPE_F32, ORC_TYPE_F16, ORC_TYPE_Q4_0, ORC_TYPE_Q4_1, ORC_TYPE_Q8_0, ORC_TYPE_Q8_1};
    const int64_t k = 32 * 7;
    float *x = frand_buf((size_t)k, 3.0f), *y = malloc((size_t)k * sizeof(float));
    for (size_t t = 0; t < sizeof(types) / sizeof(types[0]); t++) {
        void *q = malloc(orc_row_size(types[t], k));
        orc_from_float(types[t], x, q, k);
        orc_dequantize_row(types[t], q, y, k);
        check_finite("dequantize_row", y, (size_t)k);
        free(q);
    }
    uint16_t h[7];
    const float f[7] = {0.f, -0.f, 65504.f, 1e-8f, -3.5f, 70000.f, 0.33333f};
    for (int i = 0; i < 7; i++) h[i] = orc_fp32_to_fp16(f[i]);
    float back[7];
    orc_fp16_to_fp32_row(h, back, 7);
    for (int i = 0; i < 7; i++) back[i] = orc_fp16_to_fp32_soft(h[i]) - back[i];
    free(x);
    free(y);
}

static void products(void) {
    const int wtypes[] = {ORC_TYPE_F32, ORC_TYPE_F16, ORC_TYPE_Q4_0, ORC_TYPE_Q4_1, ORC_TYPE_Q8_0};
    const int64_t N = 40, K = 96, M = 5;
    float *W = frand_buf((size_t)(N * K), 0.1f), *X = frand_buf((size_t)(M * K), 1.0f);
    float *Y = malloc((size_t)(M * N) * sizeof(float));
    for (size_t t = 0; t < sizeof(wtypes) / sizeof(wtypes[0]); t++) {
        const size_t rs = orc_row_size(wtypes[t], K);
        uint8_t *wb = malloc(rs * (size_t)N);
        for (int64_t n = 0; n < N; n++) orc_from_float(wtypes[t], W + n * K, wb + rs * (size_t)n, K);
        orc_mul_mat(wtypes[t], wb, N, K, X, M, Y, 2);
        check_finite("mul_mat", Y, (size_t)(M * N));
        const int vt = orc_vec_dot_type(wtypes[t]);
        void *xq = malloc(orc_row_size(vt, K));
        orc_from_float(vt, X, xq, K);
        (void)orc_vec_dot(wtypes[t], K, wb, xq);
        if (wtypes[t] != ORC_TYPE_F32 && wtypes[t] != ORC_TYPE_F16) {
            int32_t isums[3];
            orc_block_isums(wtypes[t], K, wb, xq, isums);
        }
        free(xq);
        free(wb);
    }
    free(W);
    free(X);
    free(Y);
}

static void operators(void) {
    /* LayerNorm, GELUs */
    const int64_t rows = 7, n = 96;
    float *x = frand_buf((size_t)(rows * n), 4.0f), *y = malloc((size_t)(rows * n) * sizeof(float));
    float *w = frand_buf((size_t)n, 1.0f), *b = frand_buf((size_t)n, 1.0f);
    orc_layer_norm(x, y, rows, n, 1e-6f, w, b, 2);
    check_finite("layer_norm", y, (size_t)(rows * n));
    orc_gelu_erf(y, rows * n);
    orc_gelu_tanh(x, rows * n);
    check_finite("gelu", y, (size_t)(rows * n));
    uint16_t *tab = malloc(65536 * sizeof(uint16_t));
    orc_gelu_tanh_table(tab);
    free(tab);
    free(x);
    free(y);
    free(w);
    free(b);

    /* RoPE + axial table */
    const int HD = 16, side = 3, NT = side * side, nh = 2;
    float *cis = malloc((size_t)(NT * HD) * sizeof(float));
    orc_compute_axial_cis(cis, HD, side, side, 10000.f, 1.0f);
    float *r = frand_buf((size_t)(HD * NT * nh), 1.0f);
    orc_rope(r, HD, NT, nh, cis);
    check_finite("rope", r, (size_t)(HD * NT * nh));
    free(cis);
    free(r);

    /* attention, Nq != Nkv, strided like the encoder's views */
    const int64_t D = 24, Nq = 13, Nkv = 37, H = 3, B = 2;
    float *q = frand_buf((size_t)(D * Nq * H * B), 1.0f), *k = frand_buf((size_t)(D * Nkv * H * B), 1.0f);
    float *v = frand_buf((size_t)(D * Nkv * H * B), 1.0f), *o = malloc((size_t)(D * Nq * H * B) * sizeof(float));
    orc_flash_attn_ext(q, D, Nq * D, H * Nq * D, k, D, Nkv * D, H * Nkv * D, v, H * D, D, Nkv * H * D, D, Nq, Nkv, H,
                       B, 0.2f, o, 2);
    check_finite("flash_attn_ext", o, (size_t)(D * Nq * H * B));
    free(q);
    free(k);
    free(v);
    free(o);

    /* image preprocessing and resize */
    const int iw = 37, ih = 23, S = 32;
    uint8_t *img = malloc((size_t)(iw * ih * 3)), *rs = malloc((size_t)(S * S * 3));
    for (int i = 0; i < iw * ih * 3; i++) img[i] = (uint8_t)(i * 37 + 11);
    float *chw = malloc((size_t)(3 * S * S) * sizeof(float));
    orc_preprocess_sam3(img, iw, ih, S, chw);
    check_finite("preprocess_sam3", chw, (size_t)(3 * S * S));
    orc_preprocess_sam2(img, iw, ih, S, chw);
    orc_resize_bilinear_u8(img, iw, ih, rs, S, S);
    free(img);
    free(rs);
    free(chw);

    /* neck operators */
    const int64_t C = 8, Co = 6, Hh = 5, Ww = 7;
    float *xi = frand_buf((size_t)(Hh * Ww * C), 1.0f);
    uint16_t *w16 = malloc((size_t)(4 * C * Co) * sizeof(uint16_t));
    for (int64_t i = 0; i < 4 * C * Co; i++) w16[i] = orc_fp32_to_fp16(frand() * 0.5f);
    float *yd = malloc((size_t)(4 * Hh * Ww * Co) * sizeof(float));
    orc_conv_transpose_2x2(w16, C, Co, xi, Hh, Ww, yd, 2);
    check_finite("conv_transpose_2x2", yd, (size_t)(4 * Hh * Ww * Co));
    float *w3 = frand_buf((size_t)(9 * C * Co), 0.3f), *y3 = malloc((size_t)(Hh * Ww * Co) * sizeof(float));
    orc_conv2d(ORC_TYPE_F32, w3, 3, 3, C, Co, 1, xi, Hh, Ww, y3, 2);
    uint16_t *w3h = malloc((size_t)(9 * C * Co) * sizeof(uint16_t));
    orc_fp32_to_fp16_row(w3, w3h, 9 * C * Co);
    orc_conv2d(ORC_TYPE_F16, w3h, 3, 3, C, Co, 1, xi, Hh, Ww, y3, 2);
    check_finite("conv2d", y3, (size_t)(Hh * Ww * Co));
    float *yp = malloc((size_t)((Hh / 2) * (Ww / 2) * C) * sizeof(float));
    orc_maxpool2x2(xi, Hh - 1, Ww - 1, C, yp);
    float *pe = malloc((size_t)(Hh * Ww * 16) * sizeof(float));
    orc_sinusoidal_pe_2d((int)Hh, (int)Ww, 16, pe);
    check_finite("sinusoidal_pe_2d", pe, (size_t)(Hh * Ww * 16));
    float *bi = malloc((size_t)(C * 9 * 11) * sizeof(float));
    orc_bicubic(xi, (int)C, (int)Hh, (int)Ww, bi, 9, 11);
    check_finite("bicubic", bi, (size_t)(C * 9 * 11));
    free(xi);
    free(w16);
    free(yd);
    free(w3);
    free(y3);
    free(w3h);
    free(yp);
    free(pe);
    free(bi);
}

static void mem_attn(const orc_model *m) {
    int32_t dims[4];
    if (orc_mem_attn_dims(m, dims) != 0) return;  /* no memory attention in this file */
    const int64_t D = dims[1], MD = dims[2], N = 16, n_ptr = 4, M_total = 2 * N + n_ptr;
    float *curr = frand_buf((size_t)(N * D), 1.0f), *pos = frand_buf((size_t)(N * D), 1.0f);
    float *prompt = frand_buf((size_t)(M_total * MD), 1.0f), *ppos = frand_buf((size_t)(M_total * MD), 1.0f);
    float *rq = frand_buf((size_t)(N * D), 1.0f), *rk = frand_buf((size_t)((M_total - n_ptr) * D), 1.0f);
    float *out = malloc((size_t)(N * D) * sizeof(float));
    if (orc_mem_attn(m, curr, pos, N, prompt, ppos, M_total, n_ptr, rq, rk, out, 2) != 0) {
        fprintf(stderr, "asan_check: mem_attn: %s\n", orc_last_error());
        failures++;
    } else {
        check_finite("mem_attn", out, (size_t)(N * D));
        printf("asan_check: memory attention, %d layer(s)\n", dims[0]);
    }
    free(curr);
    free(pos);
    free(prompt);
    free(ppos);
    free(rq);
    free(rk);
    free(out);
}

static void model(const char *path) {
    orc_model *m = orc_model_load(path);
    if (!m) {
        fprintf(stderr, "asan_check: %s: %s\n", path, orc_last_error());
        failures++;
        return;
    }
    const orc_hiera_hp *hp = orc_model_hiera(m);
    if (hp) {
        const int S = hp->img_size;
        float *chw = frand_buf((size_t)(3 * S * S), 1.0f);
        int side[4], width[4];
        orc_hiera_dims(m, side, width);
        float *out[4], *stage[4];
        for (int i = 0; i < 4; i++) {
            out[i] = malloc((size_t)side[i] * side[i] * (size_t)hp->neck_dim * sizeof(float));
            stage[i] = malloc((size_t)side[i] * side[i] * (size_t)width[i] * sizeof(float));
        }
        if (orc_hiera_encode(m, chw, out, stage, 2) != 0) {
            fprintf(stderr, "asan_check: hiera_encode: %s\n", orc_last_error());
            failures++;
        } else {
            for (int i = 0; i < 4; i++)
                check_finite("hiera_encode", out[i], (size_t)side[i] * side[i] * (size_t)hp->neck_dim);
            printf("asan_check: %s: Hiera encoder + FPN\n", path);
        }
        for (int i = 0; i < 4; i++) {
            free(out[i]);
            free(stage[i]);
        }
        free(chw);
    } else {
        int32_t h[16];
        orc_model_hparams(m, h);
        const int S = h[0], G = h[0] / h[1], E = h[2];
        float *chw = frand_buf((size_t)(3 * S * S), 1.0f), *x = malloc((size_t)G * G * (size_t)E * sizeof(float));
        if (orc_vit_encode(m, chw, x, 2) != 0) {
            fprintf(stderr, "asan_check: vit_encode: %s\n", orc_last_error());
            failures++;
        } else {
            check_finite("vit_encode", x, (size_t)G * G * (size_t)E);
            const char *which[2] = {"trk", "det"};
            for (int wi = 0; wi < 2; wi++) {
                int64_t side[4], D;
                if (orc_neck_dims(m, which[wi], side, &D) != 0) continue;
                float *out[4];
                for (int i = 0; i < 4; i++) out[i] = malloc((size_t)(side[i] * side[i] * D) * sizeof(float));
                if (orc_neck(m, which[wi], x, out, 2) != 0) {
                    fprintf(stderr, "asan_check: neck %s: %s\n", which[wi], orc_last_error());
                    failures++;
                } else {
                    for (int i = 0; i < 4; i++) check_finite("neck", out[i], (size_t)(side[i] * side[i] * D));
                    printf("asan_check: %s: ViT encoder + %s neck\n", path, which[wi]);
                }
                for (int i = 0; i < 4; i++) free(out[i]);
            }
        }
        free(chw);
        free(x);
    }
    mem_attn(m);
    orc_model_free(m);
}

int main(int argc, char **argv) {
    if (argc > 1 && strcmp(argv[1], "--load-only") == 0) {
        /* damaged files: loading must end in a clean refusal or a model that
           frees cleanly, with no sanitizer report either way */
        int refused = 0;
        for (int i = 2; i < argc; i++) {
            orc_model *m = orc_model_load(argv[i]);
            if (m) orc_model_free(m);
            else refused++;
        }
        printf("asan_check: load-only ok (%d of %d refused)\n", refused, argc - 2);
        return 0;
    }
    formats();
    products();
    operators();
    for (int i = 1; i < argc; i++) model(argv[i]);
    if (failures) {
        fprintf(stderr, "asan_check: %d failure(s)\n", failures);
        return 1;
    }
    printf("asan_check: ok (%d model file(s))\n", argc - 1);
    return 0;
}
