/*
 * orc_memattn.c — CPU oracle: the tracker's memory attention, the
 * transformer that conditions the current frame's image tokens on the
 * memory bank.  TEST INFRASTRUCTURE ONLY (see orc.h).
 *
 * Graph: sam3_build_mem_attn_graph (sam3.cpp:9224-9337), shared by SAM 3 and
 * SAM 2 models; weights registered at sam3.cpp:2004-2040 / :3034-3060
 * ("mem_attn.layers.<l>.{sa,ca}.{q,k,v,out}_proj", ".linear1/2", ".norm1-3",
 * "mem_attn.norm"); inputs as sam3_propagate_single builds them
 * (sam3.cpp:11232-11304).
 *
 *   x = curr + 0.1·src_pos                       (ggml_scale, then ggml_add)
 *   per layer:
 *     self-attention: LN1 → q, k, v (D → D, + bias); RoPE on q and k
 *       (rope_q, [2, D/2, N]); one head of D channels, scale 1/√D;
 *       out_proj + bias; residual
 *     cross-attention: LN2 → q (+ bias), RoPE(rope_q); k from prompt +
 *       prompt_pos (MD → D, + bias), RoPE on the first M_spatial keys only
 *       (rope_k, [2, D/2, M_spatial]); v from prompt (MD → D, + bias); one
 *       head, scale 1/√D; out_proj + bias; residual
 *     FFN: LN3 → linear1 (+ bias) → ReLU → linear2 (+ bias); residual
 *   final LN (mem_attn.norm)
 * LayerNorm eps 1e-5 (sam3_layer_norm, sam3.cpp:1037-1047); every
 * ggml_mul_mat converts its input to the weight's vec_dot type and
 * flash_attn_ext runs on F32 operands, as in the rest of the oracle.
 *
 * Parity: pinned by tests/test_oracle_memattn.py against a float64 torch
 * restatement of the same layers built from the weights read back from the
 * model file (F32 file: every operation but the evaluation order is the
 * same), with RoPE and LayerNorm pinned separately in tests/test_oracle.py.
 */
#include "orc.h"

#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    orc_tensor_view w, b;
} lin_t;

static int get(const orc_model *m, const char *pre, const char *suf, orc_tensor_view *v) {
    return orc_model_tensor(m, pre, suf, v);
}

static int get_lin(const orc_model *m, const char *pre, const char *name, lin_t *l) {
    char s[64];
    snprintf(s, sizeof s, "%s.weight", name);
    if (get(m, pre, s, &l->w)) return -1;
    snprintf(s, sizeof s, "%s.bias", name);
    return get(m, pre, s, &l->b);
}

/* y[M][N] = x[M][K]·Wᵀ + b (ggml_add(ggml_mul_mat(W, x), b)) */
static void linear(const lin_t *l, const float *x, int64_t M, float *y, int nth) {
    const int64_t K = l->w.ne[0], N = l->w.ne[1];
    orc_mul_mat(l->w.type, l->w.data, N, K, x, M, y, nth);
    const float *b = (const float *)l->b.data;
#pragma omp parallel for num_threads(nth)
    for (int64_t r = 0; r < M; r++)
        for (int64_t c = 0; c < N; c++) y[r * N + c] += b[c];
}

static void add_into(float *x, const float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] += y[i];
}

/* one head of D channels: q [Nq][D], k [Nkv][D], v [Nkv][D] → o [Nq][D] */
static void attend(const float *q, int64_t Nq, const float *k, const float *v, int64_t Nkv, int64_t D, float *o,
                   int nth) {
    orc_flash_attn_ext(q, D, Nq * D, Nq * D, k, D, Nkv * D, Nkv * D, v, D, Nkv * D, Nkv * D, D, Nq, Nkv, 1, 1,
                       1.0f / sqrtf((float)D), o, nth);
}

int orc_mem_attn_dims(const orc_model *m, int32_t out[4]) {
    orc_tensor_view t;
    int L = 0;
    char pre[48];
    for (;;) {
        snprintf(pre, sizeof pre, "mem_attn.layers.%d.", L);
        if (get(m, pre, "sa.q_proj.weight", &t)) break;
        L++;
    }
    if (L == 0) {
        orc_set_error("the model has no memory attention");
        return -1;
    }
    if (get(m, "mem_attn.layers.0.", "ca.k_proj.weight", &t)) return -1;
    out[0] = L;
    out[1] = (int32_t)t.ne[1];  /* D */
    out[2] = (int32_t)t.ne[0];  /* MD */
    if (get(m, "mem_attn.layers.0.", "linear1.weight", &t)) return -1;
    out[3] = (int32_t)t.ne[1];  /* FFN */
    return 0;
}

int orc_mem_attn(const orc_model *m, const float *curr, const float *src_pos, int64_t N, const float *prompt,
                 const float *prompt_pos, int64_t M_total, int64_t n_ptr, const float *rope_q,
                 const float *rope_k, float *out, int nth) {
    int32_t dims[4];
    if (orc_mem_attn_dims(m, dims)) return -1;
    const int L = dims[0];
    const int64_t D = dims[1], MD = dims[2], FFN = dims[3];
    const int64_t M_sp = M_total - n_ptr;
    if (nth <= 0) nth = omp_get_max_threads();
    if (N <= 0 || M_total <= 0 || n_ptr < 0 || M_sp < 0 || (M_sp > 0 && !rope_k)) {
        orc_set_error("orc_mem_attn: bad sizes");
        return -1;
    }
    float *x = (float *)malloc(sizeof(float) * (size_t)(N * D));
    float *xn = (float *)malloc(sizeof(float) * (size_t)(N * D));
    float *q = (float *)malloc(sizeof(float) * (size_t)(N * D));
    float *kk = (float *)malloc(sizeof(float) * (size_t)((N > M_total ? N : M_total) * D));
    float *vv = (float *)malloc(sizeof(float) * (size_t)((N > M_total ? N : M_total) * D));
    float *o = (float *)malloc(sizeof(float) * (size_t)(N * D));
    float *t2 = (float *)malloc(sizeof(float) * (size_t)(N * D));
    float *h = (float *)malloc(sizeof(float) * (size_t)(N * FFN));
    float *kvp = (float *)malloc(sizeof(float) * (size_t)(M_total * MD));
    int rc = -1;
    /* pos_enc_at_input: x = curr + 0.1·src_pos */
    for (int64_t i = 0; i < N * D; i++) x[i] = curr[i] + src_pos[i] * 0.1f;
    for (int64_t i = 0; i < M_total * MD; i++) kvp[i] = prompt[i] + prompt_pos[i];
    for (int l = 0; l < L; l++) {
        char pre[48];
        snprintf(pre, sizeof pre, "mem_attn.layers.%d.", l);
        orc_tensor_view n1w, n1b, n2w, n2b, n3w, n3b;
        lin_t sq, sk, sv, so, cq, ck, cv, co, f1, f2;
        if (get(m, pre, "norm1.weight", &n1w) || get(m, pre, "norm1.bias", &n1b) ||
            get(m, pre, "norm2.weight", &n2w) || get(m, pre, "norm2.bias", &n2b) ||
            get(m, pre, "norm3.weight", &n3w) || get(m, pre, "norm3.bias", &n3b) ||
            get_lin(m, pre, "sa.q_proj", &sq) || get_lin(m, pre, "sa.k_proj", &sk) ||
            get_lin(m, pre, "sa.v_proj", &sv) || get_lin(m, pre, "sa.out_proj", &so) ||
            get_lin(m, pre, "ca.q_proj", &cq) || get_lin(m, pre, "ca.k_proj", &ck) ||
            get_lin(m, pre, "ca.v_proj", &cv) || get_lin(m, pre, "ca.out_proj", &co) ||
            get_lin(m, pre, "linear1", &f1) || get_lin(m, pre, "linear2", &f2))
            goto done;
        /* self-attention with RoPE */
        orc_layer_norm(x, xn, N, D, 1e-5f, (const float *)n1w.data, (const float *)n1b.data, nth);
        linear(&sq, xn, N, q, nth);
        linear(&sk, xn, N, kk, nth);
        linear(&sv, xn, N, vv, nth);
        orc_rope(q, D, N, 1, rope_q);
        orc_rope(kk, D, N, 1, rope_q);
        attend(q, N, kk, vv, N, D, o, nth);
        linear(&so, o, N, t2, nth);
        add_into(x, t2, N * D);
        /* cross-attention to the memory */
        orc_layer_norm(x, xn, N, D, 1e-5f, (const float *)n2w.data, (const float *)n2b.data, nth);
        linear(&cq, xn, N, q, nth);
        linear(&ck, kvp, M_total, kk, nth);
        linear(&cv, prompt, M_total, vv, nth);
        orc_rope(q, D, N, 1, rope_q);
        if (M_sp > 0) orc_rope(kk, D, M_sp, 1, rope_k);  /* pointer tokens keep no RoPE */
        attend(q, N, kk, vv, M_total, D, o, nth);
        linear(&co, o, N, t2, nth);
        add_into(x, t2, N * D);
        /* FFN */
        orc_layer_norm(x, xn, N, D, 1e-5f, (const float *)n3w.data, (const float *)n3b.data, nth);
        linear(&f1, xn, N, h, nth);
        for (int64_t i = 0; i < N * FFN; i++) h[i] = h[i] > 0.f ? h[i] : 0.f;
        linear(&f2, h, N, t2, nth);
        add_into(x, t2, N * D);
    }
    {
        orc_tensor_view nw, nb;
        if (get(m, "mem_attn.", "norm.weight", &nw) || get(m, "mem_attn.", "norm.bias", &nb)) goto done;
        orc_layer_norm(x, out, N, D, 1e-5f, (const float *)nw.data, (const float *)nb.data, nth);
    }
    rc = 0;
done:
    free(x); free(xn); free(q); free(kk); free(vv); free(o); free(t2); free(h); free(kvp);
    return rc;
}
