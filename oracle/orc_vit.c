/*
 * orc_vit.c — CPU oracle: GGML model-file reader and the SAM 3 ViT backbone.
 * TEST INFRASTRUCTURE ONLY (see orc.h).
 *
 * File format: sam3.cpp:3200-3344 (header), :1477-1520 (SAM3 hparams),
 * :3091-3194 (tensor records, 32-byte aligned data, dtype coercion to the
 * registered type).  Registered types: sam3.cpp:2461-2557 (T2/T4 use the
 * file's weight type when ne[0] is a multiple of the block size, F32
 * otherwise; T1f/T3f/T4f are always F32).
 *
 * Backbone graph: sam3_build_vit_prefix_graph (sam3.cpp:3806-3830) and
 * sam3_vit_block_forward (sam3.cpp:3710-3801).
 */
#define _GNU_SOURCE
#include "orc.h"

#include <fcntl.h>
#include <math.h>
#include <omp.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

static __thread char g_err[512];
const char *orc_last_error(void) { return g_err; }
void orc_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
#define ORC_FAIL(...) do { snprintf(g_err, sizeof g_err, __VA_ARGS__); goto fail; } while (0)

typedef struct {
    char name[96];
    int type;        /* registered (in-memory) type */
    int64_t ne[4];
    void *data;      /* owned */
} orc_tensor;

typedef struct {
    int32_t img_size, patch, E, depth, heads, mlp, window, n_global, gidx[4];
    int32_t neck_dim, visual_only;
} orc_hp;

struct orc_model {
    orc_hp hp;
    int is_sam2;
    orc_hiera_hp h2;  /* SAM 2 files (sam2_load_hparams, sam3.cpp:1564-1626) */
    int ftype, wtype;
    int n_tensors;
    orc_tensor *t;
};

static const orc_tensor *find(const orc_model *m, const char *name) {
    for (int i = 0; i < m->n_tensors; i++) {
        if (strcmp(m->t[i].name, name) == 0) return &m->t[i];
    }
    return NULL;
}

static const orc_tensor *findf(const orc_model *m, const char *fmt, int i) {
    char buf[96];
    snprintf(buf, sizeof buf, fmt, i);
    return find(m, buf);
}

static int is_global(const orc_hp *hp, int idx) {
    for (int i = 0; i < hp->n_global && i < 4; i++) {
        if (hp->gidx[i] == idx) return 1;
    }
    return 0;
}

/* Names registered with T1f/T3f/T4f (always F32) among the encoder's tensors
 * (sam3.cpp:2527-2557). Everything else 2D+ follows the T2/T4 rule. */
static int registered_type(const char *name, int n_dims, int64_t ne0, int wtype) {
    if (n_dims < 2) return ORC_TYPE_F32;
    if (strstr(name, "pos_embed") || strstr(name, "freqs_cis")) return ORC_TYPE_F32;
    const int64_t blk = orc_blck_size(wtype);
    return (ne0 % blk == 0) ? wtype : ORC_TYPE_F32;
}

static int ftype_to_wtype(int ftype) {
    switch (ftype) {
        case 0: return ORC_TYPE_F32;
        case 1: return ORC_TYPE_F16;
        case 2: return ORC_TYPE_Q4_0;
        case 3: return ORC_TYPE_Q4_1;
        case 8: return ORC_TYPE_Q8_0;
        default: return -1;
    }
}

orc_model *orc_model_load(const char *path) {
    orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
    int fd = -1;
    uint8_t *map = NULL;
    size_t fsize = 0;
    fd = open(path, O_RDONLY);
    if (fd < 0) ORC_FAIL("cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0) ORC_FAIL("stat failed");
    fsize = (size_t)st.st_size;
    map = (uint8_t *)mmap(NULL, fsize, PROT_READ, MAP_PRIVATE, fd, 0);
    if (map == MAP_FAILED) { map = NULL; ORC_FAIL("mmap failed"); }
    size_t off = 0;
#define RD32(dst) do { if (off + 4 > fsize) ORC_FAIL("truncated file"); memcpy(&(dst), map + off, 4); off += 4; } while (0)
    uint32_t magic; int32_t version, ftype, n_tensors;
    RD32(magic); RD32(version); RD32(ftype); RD32(n_tensors);
    if (magic == 0x73616D32u) { /* "sam2" */
        if (version != 1) ORC_FAIL("unsupported SAM2 version %d", version);
        m->is_sam2 = 1;
    } else {
        if (magic != 0x73616D33u) ORC_FAIL("bad magic 0x%08x (expected sam3 or sam2)", magic);
        if (version != 3) ORC_FAIL("unsupported version %d", version);
    }
    m->ftype = ftype;
    m->wtype = ftype_to_wtype(ftype);
    if (m->wtype < 0) ORC_FAIL("unsupported ftype %d", ftype);
    if (m->is_sam2) {
        /* 57 int32 fields in sam2_load_hparams order; the encoder keeps the
         * Hiera and FPN ones */
        int32_t v[57];
        for (int i = 0; i < 57; i++) RD32(v[i]);
        orc_hiera_hp *h = &m->h2;
        h->img_size = v[0];
        if (v[1] != 1) ORC_FAIL("backbone type %d is not Hiera", v[1]);
        h->embed_dim = v[2]; h->num_heads = v[3]; h->num_stages = v[4];
        for (int i = 0; i < 4; i++) h->stages[i] = v[5 + i];
        h->global_n = v[9];
        for (int i = 0; i < 8; i++) h->global_idx[i] = v[10 + i];
        h->q_pool = v[18];
        for (int i = 0; i < 4; i++) h->window_spec[i] = v[19 + i];
        h->bkg_h = v[23]; h->bkg_w = v[24]; h->scalp = v[25];
        h->neck_dim = v[26]; h->fpn_td_n = v[27];
        for (int i = 0; i < 4; i++) h->fpn_td[i] = v[28 + i];
        if (h->num_stages != 4 || h->global_n > 8 || h->embed_dim <= 0 || h->img_size % 4 != 0)
            ORC_FAIL("inconsistent Hiera hparams");
        goto tensors;
    }
    /* SAM3 hparams: 39 int32 fields in the order of sam3_load_hparams. */
    int32_t hpv[39];
    {
        int32_t v[10];
        for (int i = 0; i < 8; i++) RD32(v[i]);
        m->hp.img_size = v[0]; m->hp.patch = v[1]; m->hp.E = v[2]; m->hp.depth = v[3];
        m->hp.heads = v[4];
        m->hp.mlp = (int32_t)(v[2] * (v[5] / 1000.0f));
        m->hp.window = v[6];
        m->hp.n_global = v[7];
        for (int i = 0; i < m->hp.n_global && i < 4; i++) RD32(m->hp.gidx[i]);
        /* remaining 27 fields (text .. visual_only); the neck width and
         * visual_only are kept */
        for (int i = 0; i < 27; i++) RD32(hpv[i]);
        m->hp.neck_dim = hpv[6];
        m->hp.visual_only = hpv[26];
    }
tensors:
    /* every record takes at least its 16-byte header: a count the file
       cannot hold is refused before anything is allocated for it */
    if (n_tensors < 0 || (size_t)n_tensors > (fsize - off) / 16) ORC_FAIL("bad tensor count %d", n_tensors);
    m->t = (orc_tensor *)calloc((size_t)(n_tensors > 0 ? n_tensors : 1), sizeof(orc_tensor));
    if (!m->t) ORC_FAIL("out of memory");
    for (int ti = 0; ti < n_tensors; ti++) {
        int32_t n_dims, name_len, dtype;
        RD32(n_dims); RD32(name_len); RD32(dtype);
        if (n_dims < 1 || n_dims > 4) ORC_FAIL("bad n_dims %d", n_dims);
        if (orc_type_size(dtype) == 0) ORC_FAIL("tensor %d: unsupported dtype %d", ti, dtype);
        orc_tensor *t = &m->t[m->n_tensors];
        int64_t n_el = 1;
        for (int i = 0; i < 4; i++) t->ne[i] = 1;
        for (int i = 0; i < n_dims; i++) {
            int32_t d;
            RD32(d);
            /* positive, and no more elements than the file has bits (so the
               products below cannot overflow) */
            if (d <= 0 || n_el > (int64_t)(8 * fsize) / d) ORC_FAIL("tensor %d: bad dimension %d", ti, d);
            t->ne[i] = d;
            n_el *= d;
        }
        if (t->ne[0] % orc_blck_size(dtype) != 0) ORC_FAIL("tensor %d: ne0 %lld not a block multiple", ti, (long long)t->ne[0]);
        if (name_len <= 0 || name_len >= (int)sizeof t->name || (size_t)name_len > fsize - off) ORC_FAIL("bad name length");
        memcpy(t->name, map + off, (size_t)name_len);
        t->name[name_len] = 0;
        off += (size_t)name_len;
        off += (32 - off % 32) % 32;
        const size_t bytes = orc_row_size(dtype, t->ne[0]) * (size_t)(n_el / t->ne[0]);
        if (off > fsize || bytes > fsize - off) ORC_FAIL("tensor %s: truncated data", t->name);
        const uint8_t *src = map + off;
        off += bytes;
        /* encoder backbones, necks and the memory attention only */
        if (strncmp(t->name, "vit.", 4) != 0 && strncmp(t->name, "neck.", 5) != 0 &&
            strncmp(t->name, "hiera.", 6) != 0 && strncmp(t->name, "fpn.", 4) != 0 &&
            strncmp(t->name, "mem_attn.", 9) != 0)
            continue;
        const int rt = registered_type(t->name, n_dims, t->ne[0], m->wtype);
        t->type = rt;
        const size_t out_bytes = orc_row_size(rt, t->ne[0]) * (size_t)(n_el / t->ne[0]);
        t->data = malloc(out_bytes);
        if (!t->data) ORC_FAIL("out of memory");
        if (rt == dtype) {
            memcpy(t->data, src, bytes);
        } else if (rt == ORC_TYPE_F32) {
            /* F16 → F32 or dequantize → F32 (sam3.cpp:3151-3172) */
            const int64_t rows = n_el / t->ne[0];
            const size_t rs = orc_row_size(dtype, t->ne[0]);
            for (int64_t r = 0; r < rows; r++) {
                orc_dequantize_row(dtype, src + r * rs, (float *)t->data + r * t->ne[0], t->ne[0]);
            }
        } else if (rt == ORC_TYPE_F16 && dtype == ORC_TYPE_F32) {
            orc_fp32_to_fp16_row((const float *)src, (uint16_t *)t->data, n_el);
        } else {
            free(t->data);
            t->data = NULL;
            ORC_FAIL("tensor %s: unsupported conversion %d -> %d", t->name, dtype, rt);
        }
        m->n_tensors++;
    }
    munmap(map, fsize);
    close(fd);
    return m;
fail:
    if (map) munmap(map, fsize);
    if (fd >= 0) close(fd);
    orc_model_free(m);
    return NULL;
#undef RD32
}

void orc_model_free(orc_model *m) {
    if (!m) return;
    for (int i = 0; i < m->n_tensors; i++) free(m->t[i].data);
    free(m->t);
    free(m);
}

void orc_model_hparams(const orc_model *m, int32_t out[16]) {
    memset(out, 0, 16 * sizeof(int32_t));
    out[0] = m->hp.img_size; out[1] = m->hp.patch; out[2] = m->hp.E; out[3] = m->hp.depth;
    out[4] = m->hp.heads; out[5] = m->hp.mlp; out[6] = m->hp.window; out[7] = m->hp.n_global;
    for (int i = 0; i < 4; i++) out[8 + i] = m->hp.gidx[i];
    out[12] = m->ftype;
    out[13] = m->hp.neck_dim;
    out[14] = m->hp.visual_only;
    out[15] = (find(m, "neck.trk.0.conv_3x3.weight") ? 1 : 0) | (find(m, "neck.det.0.conv_3x3.weight") ? 2 : 0);
}

const orc_hiera_hp *orc_model_hiera(const orc_model *m) { return m->is_sam2 ? &m->h2 : NULL; }

/* sam3_create_state's encode_img_size for a SAM 2 file (sam3.cpp:3392-3402):
 * every later Hiera call builds its grids and positional embedding for
 * img_size pixels per side (sam2_encode_image_hiera, :5862, uses the state's
 * size; the PE is the bicubic resize for that grid, :4114-4171). */
int orc_hiera_set_img_size(orc_model *m, int img_size) {
    if (!m->is_sam2) { snprintf(g_err, sizeof g_err, "not a SAM 2 model"); return -1; }
    if (img_size <= 0 || img_size % 32 != 0) {
        snprintf(g_err, sizeof g_err, "image size %d is not a positive multiple of 32", img_size);
        return -1;
    }
    m->h2.img_size = img_size;
    return 0;
}

int orc_model_tensor(const orc_model *m, const char *prefix, const char *suffix, orc_tensor_view *out) {
    char buf[96];
    snprintf(buf, sizeof buf, "%s%s", prefix, suffix);
    const orc_tensor *t = find(m, buf);
    if (!t) {
        snprintf(g_err, sizeof g_err, "tensor %s not in the model", buf);
        return -1;
    }
    out->type = t->type;
    for (int i = 0; i < 4; i++) out->ne[i] = t->ne[i];
    out->data = t->data;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Prefix: ggml_conv_2d_sk_p0 (im2col in the kernel's type, then mul_mat with
 * the im2col matrix as src0 and the kernel as src1), permute, + tiled
 * pos_embed (ggml_repeat), ggml_norm(1e-5)·w + b.  sam3.cpp:3806-3830. */
int orc_vit_prefix(const orc_model *m, const float *chw, float *x, int nthreads) {
    const orc_hp *hp = &m->hp;
    const int P = hp->patch, G = hp->img_size / P, E = hp->E, T = G * G;
    const int64_t Kp = (int64_t)P * P * 3;
    const orc_tensor *pw = find(m, "vit.patch_embed.proj.weight");
    const orc_tensor *pos = find(m, "vit.pos_embed");
    const orc_tensor *lw = find(m, "vit.ln_pre.weight");
    const orc_tensor *lb = find(m, "vit.ln_pre.bias");
    if (!pw || !pos || !lw || !lb) { snprintf(g_err, sizeof g_err, "missing prefix tensors"); return -1; }
    const int pg = (int)pos->ne[1];
    if (nthreads <= 0) nthreads = omp_get_max_threads();
    const int ptype = pw->type; /* F32 or F16 */
    const size_t rs = orc_row_size(ptype, Kp);
    char *cols = (char *)malloc(rs * (size_t)T);
    const size_t plane = (size_t)hp->img_size * hp->img_size;
#pragma omp parallel for num_threads(nthreads)
    for (int t = 0; t < T; t++) {
        const int py = t / G, px = t % G;
        float tmp[3 * 64 * 64];
        int64_t k = 0;
        for (int c = 0; c < 3; c++)
            for (int ky = 0; ky < P; ky++)
                for (int kx = 0; kx < P; kx++)
                    tmp[k++] = chw[c * plane + (size_t)(py * P + ky) * hp->img_size + px * P + kx];
        orc_from_float(ptype, tmp, cols + (size_t)t * rs, Kp);
    }
    /* result[t][e] = vec_dot(im2col row t, kernel row e) */
#pragma omp parallel for num_threads(nthreads)
    for (int t = 0; t < T; t++) {
        const int py = t / G, px = t % G;
        const float *pr = (const float *)pos->data + ((size_t)(py % pg) * pg + (px % pg)) * E;
        for (int e = 0; e < E; e++) {
            const float conv = orc_vec_dot(ptype, Kp, cols + (size_t)t * rs, (const char *)pw->data + (size_t)e * rs);
            x[(size_t)t * E + e] = conv + pr[e];
        }
    }
    free(cols);
    orc_layer_norm(x, x, T, E, 1e-5f, (const float *)lw->data, (const float *)lb->data, nthreads);
    return 0;
}

/* One ViT block, in place on x [T][E] (natural token order).  Windowed blocks
 * gather tokens in ggml_win_part order: window index py*nwx + px, position
 * (iy*WS + ix) inside the window. */
int orc_vit_block(const orc_model *m, int bi, float *x, int nthreads) {
    const orc_hp *hp = &m->hp;
    const int G = hp->img_size / hp->patch, E = hp->E, T = G * G, NH = hp->heads, HD = E / NH;
    const int glob = is_global(hp, bi);
    const int WS = glob ? G : hp->window;
    if (G % WS != 0) { snprintf(g_err, sizeof g_err, "grid %d not a multiple of window %d", G, WS); return -1; }
    const int nw1 = G / WS, NW = nw1 * nw1, N = WS * WS;
    const orc_tensor *n1w = findf(m, "vit.blocks.%d.norm1.weight", bi), *n1b = findf(m, "vit.blocks.%d.norm1.bias", bi);
    const orc_tensor *qw = findf(m, "vit.blocks.%d.attn.qkv.weight", bi), *qb = findf(m, "vit.blocks.%d.attn.qkv.bias", bi);
    const orc_tensor *pjw = findf(m, "vit.blocks.%d.attn.proj.weight", bi), *pjb = findf(m, "vit.blocks.%d.attn.proj.bias", bi);
    const orc_tensor *n2w = findf(m, "vit.blocks.%d.norm2.weight", bi), *n2b = findf(m, "vit.blocks.%d.norm2.bias", bi);
    const orc_tensor *f1w = findf(m, "vit.blocks.%d.mlp.lin1.weight", bi), *f1b = findf(m, "vit.blocks.%d.mlp.lin1.bias", bi);
    const orc_tensor *f2w = findf(m, "vit.blocks.%d.mlp.lin2.weight", bi), *f2b = findf(m, "vit.blocks.%d.mlp.lin2.bias", bi);
    const orc_tensor *fc = findf(m, "vit.blocks.%d.attn.freqs_cis", bi);
    if (!n1w || !n1b || !qw || !qb || !pjw || !pjb || !n2w || !n2b || !f1w || !f1b || !f2w || !f2b) {
        snprintf(g_err, sizeof g_err, "block %d: missing tensors", bi);
        return -1;
    }
    if (fc && fc->ne[2] != N) { snprintf(g_err, sizeof g_err, "block %d: freqs_cis has %lld positions, need %d", bi, (long long)fc->ne[2], N); return -1; }
    const int MLP = (int)f1w->ne[1];
    if (nthreads <= 0) nthreads = omp_get_max_threads();

    float *h = (float *)malloc(sizeof(float) * (size_t)T * E);
    float *hp_ = (float *)malloc(sizeof(float) * (size_t)T * E);
    int *perm = (int *)malloc(sizeof(int) * (size_t)T); /* partition row → token */
    for (int w = 0; w < NW; w++) {
        const int wy = w / nw1, wx = w % nw1;
        for (int p = 0; p < N; p++) {
            const int iy = p / WS, ix = p % WS;
            perm[w * N + p] = (wy * WS + iy) * G + wx * WS + ix;
        }
    }
    /* attention branch */
    orc_layer_norm(x, h, T, E, 1e-5f, (const float *)n1w->data, (const float *)n1b->data, nthreads);
    for (int r = 0; r < T; r++) memcpy(hp_ + (size_t)r * E, h + (size_t)perm[r] * E, sizeof(float) * E);
    float *qkv = (float *)malloc(sizeof(float) * (size_t)T * 3 * E);
    orc_mul_mat(qw->type, qw->data, 3 * E, E, hp_, T, qkv, nthreads);
    const float *qbias = (const float *)qb->data;
    for (int64_t r = 0; r < T; r++)
        for (int c = 0; c < 3 * E; c++) qkv[r * 3 * E + c] = qkv[r * 3 * E + c] + qbias[c];
    /* split into Q, K [HD, N, NH*NW] contiguous, V read through strides */
    float *Q = (float *)malloc(sizeof(float) * (size_t)T * E);
    float *K = (float *)malloc(sizeof(float) * (size_t)T * E);
    for (int w = 0; w < NW; w++)
        for (int hh = 0; hh < NH; hh++)
            for (int p = 0; p < N; p++) {
                const float *src = qkv + ((size_t)(w * N + p)) * 3 * E;
                float *dq = Q + (((size_t)w * NH + hh) * N + p) * HD;
                float *dk = K + (((size_t)w * NH + hh) * N + p) * HD;
                memcpy(dq, src + 0 * E + hh * HD, sizeof(float) * HD);
                memcpy(dk, src + 1 * E + hh * HD, sizeof(float) * HD);
            }
    if (fc) {
        orc_rope(Q, HD, N, (int64_t)NH * NW, (const float *)fc->data);
        orc_rope(K, HD, N, (int64_t)NH * NW, (const float *)fc->data);
    }
    float *O = (float *)malloc(sizeof(float) * (size_t)T * E);
    /* Q(b,h,i,d): b*NH*N*HD + h*N*HD + i*HD + d; V(b,h,j,d) in qkv rows */
    orc_flash_attn_ext(Q, HD, (int64_t)N * HD, (int64_t)NH * N * HD,
                       K, HD, (int64_t)N * HD, (int64_t)NH * N * HD,
                       qkv + 2 * E, 3 * E, HD, (int64_t)N * 3 * E,
                       HD, N, N, NH, NW, 1.0f / sqrtf((float)HD), O, nthreads);
    /* O rows are in partition order, [E] = [NH][HD] per row */
    float *proj = (float *)malloc(sizeof(float) * (size_t)T * E);
    orc_mul_mat(pjw->type, pjw->data, E, E, O, T, proj, nthreads);
    const float *pbias = (const float *)pjb->data;
    for (int r = 0; r < T; r++) {
        float *xr = x + (size_t)perm[r] * E;
        const float *pr = proj + (size_t)r * E;
        for (int c = 0; c < E; c++) xr[c] = xr[c] + (pr[c] + pbias[c]);
    }
    free(Q); free(K); free(O); free(proj); free(qkv);
    /* MLP branch */
    orc_layer_norm(x, h, T, E, 1e-5f, (const float *)n2w->data, (const float *)n2b->data, nthreads);
    float *f1 = (float *)malloc(sizeof(float) * (size_t)T * MLP);
    orc_mul_mat(f1w->type, f1w->data, MLP, E, h, T, f1, nthreads);
    const float *b1 = (const float *)f1b->data;
#pragma omp parallel for num_threads(nthreads)
    for (int r = 0; r < T; r++) {
        float *fr = f1 + (size_t)r * MLP;
        for (int c = 0; c < MLP; c++) fr[c] = fr[c] + b1[c];
        orc_gelu_erf(fr, MLP);
    }
    orc_mul_mat(f2w->type, f2w->data, E, MLP, f1, T, hp_, nthreads);
    const float *b2 = (const float *)f2b->data;
    for (int64_t r = 0; r < T; r++)
        for (int c = 0; c < E; c++) x[r * E + c] = x[r * E + c] + (hp_[r * E + c] + b2[c]);
    free(f1); free(h); free(hp_); free(perm);
    return 0;
}

int orc_vit_encode(const orc_model *m, const float *chw, float *out, int nthreads) {
    if (orc_vit_prefix(m, chw, out, nthreads) != 0) return -1;
    for (int i = 0; i < m->hp.depth; i++) {
        if (orc_vit_block(m, i, out, nthreads) != 0) return -1;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Sub-stage hooks: sam3_test_run_vit_block_stage and
 * sam3_test_run_vit_prefix_stage (sam3.cpp:6390-6520, :6874-6993), one
 * ggml operator group of the graph at a time on an f32 input in ggml 4D
 * layout; the stage builders are sam3.cpp:6716-6872.  Stage numbers follow
 * the enums of sam3.h:112-134.  out may be NULL: only out_ne is produced. */
enum {
    BS_NORM1 = 0, BS_WINDOW_PART, BS_QKV_PROJ, BS_ATTN_CORE, BS_ATTN_PROJ, BS_WINDOW_UNPART, BS_NORM2,
    BS_MLP_FC1, BS_MLP_GELU, BS_MLP_FC2, BS_MLP
};
enum { PS_PATCH_EMBED = 0, PS_PATCH_IM2COL, PS_PATCH_MULMAT_RAW, PS_PATCH_MULMAT, PS_POS_ADD, PS_LN_PRE_NORM, PS_LN_PRE };

static void norm_ne(const int64_t in[4], int64_t ne[4]) {
    for (int i = 0; i < 4; i++) ne[i] = (in && in[i] > 0) ? in[i] : 1;
}

/* y = W·x + bias over rows of K (ggml_add(ggml_mul_mat(w, x), b)). */
static void linear_bias(const orc_tensor *w, const orc_tensor *b, const float *x, int64_t M, float *y,
                        int nthreads) {
    const int64_t K = w->ne[0], N = w->ne[1];
    orc_mul_mat(w->type, w->data, N, K, x, M, y, nthreads);
    const float *bb = (const float *)b->data;
    for (int64_t r = 0; r < M; r++)
        for (int64_t c = 0; c < N; c++) y[r * N + c] = y[r * N + c] + bb[c];
}

int orc_vit_block_stage(const orc_model *m, int bi, int stage, const float *in, const int64_t in_ne[4],
                        float *out, int64_t out_ne[4], int nthreads) {
    const orc_hp *hp = &m->hp;
    if (m->is_sam2) { snprintf(g_err, sizeof g_err, "not a SAM 3 model"); return -1; }
    if (bi < 0 || bi >= hp->depth) { snprintf(g_err, sizeof g_err, "invalid block_idx=%d", bi); return -1; }
    if (stage < BS_NORM1 || stage > BS_MLP) { snprintf(g_err, sizeof g_err, "unknown block stage %d", stage); return -1; }
    const int E = hp->E, G = hp->img_size / hp->patch, NH = hp->heads, HD = E / NH, WS = hp->window;
    const orc_tensor *f1w = findf(m, "vit.blocks.%d.mlp.lin1.weight", bi);
    if (!f1w) { snprintf(g_err, sizeof g_err, "block %d: missing tensors", bi); return -1; }
    const int MLP = (int)f1w->ne[1];
    int64_t ne[4];
    norm_ne(in_ne, ne);
    const int64_t want0 = stage == BS_ATTN_CORE ? 3 * E : ((stage == BS_MLP_GELU || stage == BS_MLP_FC2) ? MLP : E);
    if (ne[0] != want0) {
        snprintf(g_err, sizeof g_err, "stage %d input ne0=%lld expected %lld", stage, (long long)ne[0], (long long)want0);
        return -1;
    }
    const int64_t rows = ne[1] * ne[2] * ne[3];
    int64_t o[4] = {ne[0], ne[1], ne[2], ne[3]};
    switch (stage) {
        case BS_WINDOW_PART: {
            if (ne[3] != 1) { snprintf(g_err, sizeof g_err, "window partition needs ne3 = 1"); return -1; }
            const int64_t npx = (ne[1] + WS - 1) / WS, npy = (ne[2] + WS - 1) / WS;
            o[1] = WS; o[2] = WS; o[3] = npx * npy;
        } break;
        case BS_WINDOW_UNPART:
            if (ne[1] != WS || ne[2] != WS) { snprintf(g_err, sizeof g_err, "window unpartition needs [E, %d, %d, n]", WS, WS); return -1; }
            if (ne[3] != (int64_t)((G + WS - 1) / WS) * ((G + WS - 1) / WS)) { snprintf(g_err, sizeof g_err, "window count %lld does not tile the %dx%d grid", (long long)ne[3], G, G); return -1; }
            o[1] = G; o[2] = G; o[3] = 1;
            break;
        case BS_QKV_PROJ: o[0] = 3 * E; break;
        case BS_ATTN_CORE: o[0] = E; break;
        case BS_MLP_FC1: o[0] = MLP; break;
        case BS_MLP_FC2: o[0] = E; break;
        default: break;
    }
    for (int i = 0; i < 4; i++) out_ne[i] = o[i];
    if (!out) return 0;
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#define T_(s) findf(m, "vit.blocks.%d." s, bi)
    switch (stage) {
        case BS_NORM1:
        case BS_NORM2: {
            const orc_tensor *w = stage == BS_NORM1 ? T_("norm1.weight") : T_("norm2.weight");
            const orc_tensor *b = stage == BS_NORM1 ? T_("norm1.bias") : T_("norm2.bias");
            orc_layer_norm(in, out, rows, E, 1e-5f, (const float *)w->data, (const float *)b->data, nthreads);
        } break;
        case BS_WINDOW_PART: /* ggml_win_part: window py*npx + px, zero padding */
        case BS_WINDOW_UNPART: {
            const int part = stage == BS_WINDOW_PART;
            const int64_t W0 = part ? ne[1] : G, H0 = part ? ne[2] : G;
            const int64_t npx = (W0 + WS - 1) / WS, npy = (H0 + WS - 1) / WS;
            for (int64_t w = 0; w < npx * npy; w++)
                for (int64_t p = 0; p < (int64_t)WS * WS; p++) {
                    const int64_t x = (w % npx) * WS + p % WS, y = (w / npx) * WS + p / WS;
                    const int64_t wr = w * WS * WS + p, tr = y * W0 + x;
                    const int inside = x < W0 && y < H0;
                    if (part) {
                        if (inside) memcpy(out + wr * E, in + tr * E, sizeof(float) * E);
                        else memset(out + wr * E, 0, sizeof(float) * E);
                    } else if (inside) {
                        memcpy(out + tr * E, in + wr * E, sizeof(float) * E);
                    }
                }
        } break;
        case BS_QKV_PROJ: linear_bias(T_("attn.qkv.weight"), T_("attn.qkv.bias"), in, rows, out, nthreads); break;
        case BS_ATTN_PROJ: linear_bias(T_("attn.proj.weight"), T_("attn.proj.bias"), in, rows, out, nthreads); break;
        case BS_MLP_FC1: linear_bias(f1w, T_("mlp.lin1.bias"), in, rows, out, nthreads); break;
        case BS_MLP_FC2: linear_bias(T_("mlp.lin2.weight"), T_("mlp.lin2.bias"), in, rows, out, nthreads); break;
        case BS_MLP_GELU:
            memcpy(out, in, sizeof(float) * (size_t)(rows * MLP));
            orc_gelu_erf(out, rows * MLP);
            break;
        case BS_MLP: {
            float *h = (float *)malloc(sizeof(float) * (size_t)(rows * MLP));
            linear_bias(f1w, T_("mlp.lin1.bias"), in, rows, h, nthreads);
            orc_gelu_erf(h, rows * MLP);
            linear_bias(T_("mlp.lin2.weight"), T_("mlp.lin2.bias"), h, rows, out, nthreads);
            free(h);
        } break;
        case BS_ATTN_CORE: {
            /* sam3_build_vit_attn_core_from_qkv (sam3.cpp:6778-6823): q|k|v
             * column thirds, heads of HD, RoPE on Q and K, flash attention,
             * output [E, W, H, B] with heads adjacent. */
            const int64_t N = ne[1] * ne[2], B = ne[3];
            const orc_tensor *fc = T_("attn.freqs_cis");
            if (fc && fc->ne[2] != N) {
                snprintf(g_err, sizeof g_err, "freqs_cis has %lld positions, attention has %lld", (long long)fc->ne[2], (long long)N);
                return -1;
            }
            float *Q = (float *)malloc(sizeof(float) * (size_t)(B * N * E));
            float *K = (float *)malloc(sizeof(float) * (size_t)(B * N * E));
            for (int64_t b = 0; b < B; b++)
                for (int h = 0; h < NH; h++)
                    for (int64_t p = 0; p < N; p++) {
                        const float *src = in + (b * N + p) * 3 * E;
                        memcpy(Q + ((b * NH + h) * N + p) * HD, src + h * HD, sizeof(float) * HD);
                        memcpy(K + ((b * NH + h) * N + p) * HD, src + E + h * HD, sizeof(float) * HD);
                    }
            if (fc) {
                orc_rope(Q, HD, N, (int64_t)NH * B, (const float *)fc->data);
                orc_rope(K, HD, N, (int64_t)NH * B, (const float *)fc->data);
            }
            orc_flash_attn_ext(Q, HD, N * HD, (int64_t)NH * N * HD, K, HD, N * HD, (int64_t)NH * N * HD,
                               in + 2 * E, 3 * E, HD, N * 3 * E, HD, N, N, NH, B, 1.0f / sqrtf((float)HD), out,
                               nthreads);
            free(Q);
            free(K);
        } break;
        default: break;
    }
#undef T_
    return 0;
}

int orc_vit_prefix_stage(const orc_model *m, int stage, const float *in, const int64_t in_ne[4], float *out,
                         int64_t out_ne[4], int nthreads) {
    const orc_hp *hp = &m->hp;
    if (m->is_sam2) { snprintf(g_err, sizeof g_err, "not a SAM 3 model"); return -1; }
    if (stage < PS_PATCH_EMBED || stage > PS_LN_PRE) { snprintf(g_err, sizeof g_err, "unknown prefix stage %d", stage); return -1; }
    const int P = hp->patch, G = hp->img_size / P, E = hp->E, T = G * G;
    const int64_t Kp = (int64_t)P * P * 3;
    const orc_tensor *pw = find(m, "vit.patch_embed.proj.weight");
    const orc_tensor *pos = find(m, "vit.pos_embed");
    const orc_tensor *lw = find(m, "vit.ln_pre.weight"), *lb = find(m, "vit.ln_pre.bias");
    if (!pw || !pos || !lw || !lb) { snprintf(g_err, sizeof g_err, "missing prefix tensors"); return -1; }
    int64_t ne[4];
    norm_ne(in_ne, ne);
    int64_t o[4] = {ne[0], ne[1], ne[2], ne[3]};
    switch (stage) {
        case PS_PATCH_EMBED:
        case PS_PATCH_IM2COL:
            if (ne[0] != hp->img_size || ne[1] != hp->img_size || ne[2] != 3 || ne[3] != 1) {
                snprintf(g_err, sizeof g_err, "patch_embed input shape mismatch");
                return -1;
            }
            o[0] = stage == PS_PATCH_EMBED ? E : Kp; o[1] = G; o[2] = G; o[3] = 1;
            break;
        case PS_PATCH_MULMAT_RAW:
        case PS_PATCH_MULMAT:
            if (ne[0] != Kp || ne[1] != G || ne[2] != G || ne[3] != 1) {
                snprintf(g_err, sizeof g_err, "patch_mulmat input shape mismatch");
                return -1;
            }
            if (stage == PS_PATCH_MULMAT_RAW) { o[0] = T; o[1] = E; o[2] = 1; o[3] = 1; }
            else { o[0] = G; o[1] = G; o[2] = E; o[3] = 1; }
            break;
        default:
            if (ne[0] != E || ne[1] != G || ne[2] != G) {
                snprintf(g_err, sizeof g_err, "prefix feature input shape mismatch");
                return -1;
            }
            break;
    }
    for (int i = 0; i < 4; i++) out_ne[i] = o[i];
    if (!out) return 0;
    if (nthreads <= 0) nthreads = omp_get_max_threads();
    const int64_t rows = ne[1] * ne[2] * ne[3];
    switch (stage) {
        case PS_PATCH_EMBED:
            /* the conv without position embedding and norm: the prefix on a
             * zero position table would add zeros, so compute it directly */
        case PS_PATCH_IM2COL: {
            const int ptype = pw->type;
            const size_t rs = orc_row_size(ptype, Kp);
            char *cols = (char *)malloc(rs * (size_t)T);
            const size_t plane = (size_t)hp->img_size * hp->img_size;
#pragma omp parallel for num_threads(nthreads)
            for (int t = 0; t < T; t++) {
                const int py = t / G, px = t % G;
                float tmp[3 * 64 * 64];
                int64_t k = 0;
                for (int c = 0; c < 3; c++)
                    for (int ky = 0; ky < P; ky++)
                        for (int kx = 0; kx < P; kx++)
                            tmp[k++] = in[c * plane + (size_t)(py * P + ky) * hp->img_size + px * P + kx];
                orc_from_float(ptype, tmp, cols + (size_t)t * rs, Kp);
            }
            if (stage == PS_PATCH_IM2COL) {
                for (int t = 0; t < T; t++) {
                    if (ptype == ORC_TYPE_F16) orc_fp16_to_fp32_row((const uint16_t *)(cols + (size_t)t * rs), out + (size_t)t * Kp, Kp);
                    else memcpy(out + (size_t)t * Kp, cols + (size_t)t * rs, sizeof(float) * Kp);
                }
            } else {
#pragma omp parallel for num_threads(nthreads)
                for (int t = 0; t < T; t++)
                    for (int e = 0; e < E; e++)
                        out[(size_t)t * E + e] = orc_vec_dot(ptype, Kp, cols + (size_t)t * rs, (const char *)pw->data + (size_t)e * rs);
            }
            free(cols);
        } break;
        case PS_PATCH_MULMAT_RAW:
        case PS_PATCH_MULMAT: {
            /* the stage's input tensor is F16 (sam3.cpp:6463-6464); mul_mat(im2col,
             * kernel) converts the kernel to F16 too; result[e][t] */
            uint16_t *a = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(T * Kp));
            uint16_t *kw = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(E * Kp));
            orc_fp32_to_fp16_row(in, a, T * Kp);
            if (pw->type == ORC_TYPE_F16) memcpy(kw, pw->data, sizeof(uint16_t) * (size_t)(E * Kp));
            else orc_fp32_to_fp16_row((const float *)pw->data, kw, E * Kp);
#pragma omp parallel for num_threads(nthreads)
            for (int e = 0; e < E; e++)
                for (int t = 0; t < T; t++)
                    out[(size_t)e * T + t] = orc_vec_dot(ORC_TYPE_F16, Kp, a + (size_t)t * Kp, kw + (size_t)e * Kp);
            free(a);
            free(kw);
        } break;
        case PS_POS_ADD: {
            const int pg = (int)pos->ne[1];
            for (int64_t r = 0; r < rows; r++) {
                const int64_t t = r % T, py = t / G, px = t % G;
                const float *pr = (const float *)pos->data + ((size_t)(py % pg) * pg + (px % pg)) * E;
                for (int e = 0; e < E; e++) out[r * E + e] = in[r * E + e] + pr[e];
            }
        } break;
        case PS_LN_PRE_NORM: orc_layer_norm(in, out, rows, E, 1e-5f, NULL, NULL, nthreads); break;
        case PS_LN_PRE:
            orc_layer_norm(in, out, rows, E, 1e-5f, (const float *)lw->data, (const float *)lb->data, nthreads);
            break;
        default: break;
    }
    return 0;
}
