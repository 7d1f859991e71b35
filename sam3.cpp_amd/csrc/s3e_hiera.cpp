// s3e_hiera.cpp — the SAM 2.x Hiera image encoder and its FPN neck on the
// engine's kernels: model loading from sam3.cpp's SAM 2 files, per-image
// buffers and the encode schedule.
//
// Reference: sam2_load_hparams (sam3.cpp:1564-1626), sam2_precompute_
// hiera_metadata (:1676-1742), sam2_register_tensors (:1745-1847),
// sam2_build_hiera_graph (:4462-4527), sam2_hiera_block_forward
// (:4295-4457), sam2_compute_pos_embed (:4114-4171),
// sam2_build_fpn_neck_graph (:4532-4603), sam2_encode_image_hiera
// (:5857-6018).
//
// Schedule of one block (activations NHWC, a token is a row of channels):
//   LayerNorm(1e-6) → the QKV weight's activation format
//   shortcut: dim projection GEMM (+ bias) and 2×2 max pool under Q stride,
//             written into the block's output buffer (the residual stream)
//   QKV GEMM (+ bias) whose epilogue writes Q, K, Vᵀ in window order as
//             fp16 (hi, lo) planes, heads zero-padded to 64/128; a small
//             pass fills window padding with the bias; under Q stride Q goes
//             out as f32 rows and k_hiera_prep max-pools it inside windows
//   attention (k_attn, head dim 64 or 128) → proj input, written at the
//             un-partitioned, cropped token rows
//   proj GEMM + bias + residual; LayerNorm; fc1 + bias + ggml_gelu (fp16
//             table) → fc2 input; fc2 + bias + residual.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "s3e_hiera.h"
#include "s3e_memattn.h"
#include "s3e_rt.h"

namespace s3e {

struct HBlock {
    int din = 0, dout = 0, heads = 0, ws = 0, qs = 0, stage = 0, stage_end = 0;
    int in_side = 0;  // tokens per side of the block's input in the encoder
    float *n1w = nullptr, *n1b = nullptr, *n2w = nullptr, *n2b = nullptr;
    float *qkv_b = nullptr, *proj_b = nullptr, *fc1_b = nullptr, *fc2_b = nullptr, *dp_b = nullptr;
    Weight qkv, proj, fc1, fc2, dp;
    int found = 0;
};

struct HieraModel {
    int ftype = 0, wtype = 0;
    int32_t img = 0, E0 = 0, heads0 = 0, stages[4] = {}, gn = 0, gidx[8] = {}, q_pool = 0, wspec[4] = {};
    int32_t bkg_h = 0, bkg_w = 0, scalp = 0, D = 0, td_n = 0, td[4] = {};
    int G = 0;                      // tokens per side after the patch embedding (img / 4)
    int side[4] = {}, width[4] = {};  // per stage
    int64_t patch_k = 0;            // 3·7·7 padded to a multiple of 32
    Weight patch;
    float *patch_b = nullptr, *pe = nullptr;  // pe: [G][G][E0], bicubic background + tiled window
    // the registered PE tensors as CHW on the host, for states encoding at
    // another image size (the PE is recomputed for their grid)
    std::vector<float> bkg_chw, win_chw;
    int win_side = 0;
    std::vector<HBlock> blocks;
    Weight fpn[4];                  // fpn.convs.i, which maps stage 3 − i
    float *fpn_b[4] = {};
    uint16_t *gelu_tab = nullptr;   // 65536 fp16 entries
    std::vector<void *> owned;
    int found_misc = 0;
    ~HieraModel() {
        free_weight(patch);
        for (auto &b : blocks) {
            free_weight(b.qkv);
            free_weight(b.proj);
            free_weight(b.fc1);
            free_weight(b.fc2);
            free_weight(b.dp);
        }
        for (auto &w : fpn) free_weight(w);
        for (void *p : owned) (void)hipFree(p);
    }
};

struct HieraState {
    // geometry of the image size this state encodes (sam3_effective_feat_size
    // and the per-stage grids of sam2_build_hiera_graph for that size)
    int img = 0, G = 0, side[4] = {};
    std::vector<int> in_side;       // per block: tokens per side of its input
    const float *pos = nullptr;     // [G][G][E0] PE: the model's, or pe_own
    float *pe_own = nullptr;        // PE recomputed for a non-native size
    ActBuf col, a1, a2;             // im2col rows; GEMM inputs (E-wide, MLP-wide)
    float *xs[4] = {};              // stage residual streams = stage outputs
    float *qkv = nullptr, *dp = nullptr, *attn_f32 = nullptr;  // qkv: Q rows of Q-stride blocks
    _Float16 *q16 = nullptr, *k16 = nullptr, *vt16 = nullptr;  // [hi | lo] planes
    int64_t q_cap = 0, k_cap = 0, v_cap = 0;
    _Float16 *fin = nullptr;        // FPN inputs as fp16 planes [hi | lo]
    int64_t fin_cap = 0;
    float *part = nullptr;          // key-split partials of global attention: outputs | (m, l)
    int64_t part_cap = 0;
    float *gws = nullptr;           // K-split partials of the small-grid residual GEMMs
    int64_t gws_cap = 0;
    float *lat[4] = {};             // FPN levels, f32 [side²][D]
    float *pe[4] = {};              // sinusoidal PEs of the output levels
    ~HieraState() {
        col.release();
        a1.release();
        a2.release();
        for (void *p : {(void *)qkv, (void *)dp, (void *)attn_f32, (void *)q16, (void *)k16, (void *)vt16,
                        (void *)fin, (void *)part, (void *)gws, (void *)pe_own})
            if (p) (void)hipFree(p);
        for (int i = 0; i < 4; i++)
            for (void *p : {(void *)xs[i], (void *)lat[i], (void *)pe[i]})
                if (p) (void)hipFree(p);
    }
};

namespace {

// Key ranges for a global block's attention: enough work-groups (about 512)
// when the query tiles alone would leave CUs idle, each range at least four
// 32-key tiles.
int attn_splits(int64_t nq, int64_t nkv, int64_t bh) {
    const int64_t groups = (nq + 127) / 128 * bh, ktiles = (nkv + 31) / 32;
    if (groups >= 512) return 1;
    int64_t ns = std::min<int64_t>((512 + groups - 1) / groups, std::max<int64_t>(1, ktiles / 4));
    const int64_t per = (ktiles + ns - 1) / ns;
    return (int)((ktiles + per - 1) / per);
}

int upload_f32(HieraModel *m, const RawTensor &t, int64_t expect, float **dst) {
    const int64_t n = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
    if (n != expect) { set_error("tensor has %lld elements, expected %lld", (long long)n, (long long)expect); return S3E_ERR_IO; }
    void *p = nullptr;
    if (hipMalloc(&p, (size_t)n * 4) != hipSuccess) { set_error("hipMalloc failed"); return S3E_ERR_NOMEM; }
    m->owned.push_back(p);
    if (hipMemcpy(p, t.data.data(), (size_t)n * 4, hipMemcpyHostToDevice) != hipSuccess) {
        set_error("hipMemcpy failed");
        return S3E_ERR_HIP;
    }
    *dst = (float *)p;
    return S3E_OK;
}

// sam2_precompute_hiera_metadata (sam3.cpp:1676-1742): the window size lags
// a block (a stage's first block keeps the previous stage's window); global
// blocks have window 0; Q stride at the first block of stages 1..q_pool.
// Grids for an image of img pixels per side: the patch embedding (7×7,
// stride 4, pad 3) gives img / 4 tokens per side, every Q-stride block halves
// it (sam3_effective_feat_size, sam3.cpp:245-257).  side[i]: stage i's grid;
// in_side[b]: block b's input grid.
void geometry(const HieraModel *m, int img, int side[4], std::vector<int> &in_side) {
    int g = img / 4;
    in_side.assign(m->blocks.size(), 0);
    for (size_t i = 0; i < m->blocks.size(); i++) {
        in_side[i] = g;
        if (m->blocks[i].qs) g /= 2;
    }
    int s = img / 4;
    for (int i = 0; i < 4; i++) {
        if (i > 0 && i <= m->q_pool) s /= 2;
        side[i] = s;
    }
}

void block_metadata(HieraModel *m) {
    int total = 0, ends[4], cum = 0;
    for (int s = 0; s < 4; s++) { cum += m->stages[s]; ends[s] = cum - 1; total += m->stages[s]; }
    m->blocks.assign((size_t)total, HBlock{});
    std::vector<int> qblocks;
    for (int s = 0; s < 3 && (int)qblocks.size() < m->q_pool; s++) qblocks.push_back(ends[s] + 1);
    int cur = 0, dim = m->E0, heads = m->heads0;
    for (int i = 0; i < total; i++) {
        HBlock &b = m->blocks[(size_t)i];
        int ws = m->wspec[cur];
        for (int g = 0; g < m->gn && g < 8; g++)
            if (m->gidx[g] == i) ws = 0;
        int dout = dim;
        if (i > 0 && i - 1 == ends[cur]) { dout = dim * 2; heads *= 2; cur++; }
        b.ws = ws;
        b.din = dim;
        b.dout = dout;
        b.heads = heads;
        b.stage = cur;
        b.stage_end = (i == ends[cur]);
        b.qs = std::find(qblocks.begin(), qblocks.end(), i) != qblocks.end();
        dim = dout;
    }
    std::vector<int> in_side;
    geometry(m, m->img, m->side, in_side);
    for (size_t i = 0; i < m->blocks.size(); i++) m->blocks[i].in_side = in_side[i];
    for (int i = 0, d = m->E0; i < 4; i++, d *= 2) m->width[i] = d;
}

// sam2_bicubic_interpolate_cpu (sam3.cpp:4072-4107): Keys cubic a = −0.75,
// half-pixel centres, clamped taps; float arithmetic in the reference's order.
void bicubic(const float *src, int C, int Hi, int Wi, float *dst, int Ho, int Wo) {
    auto cubic = [](float x) -> float {
        x = std::fabs(x);
        if (x < 1.0f) return (1.25f * x - 2.25f) * x * x + 1.0f;
        if (x < 2.0f) return ((-0.75f * x + 3.75f) * x - 6.0f) * x + 3.0f;
        return 0.0f;
    };
    for (int c = 0; c < C; ++c)
        for (int y = 0; y < Ho; ++y) {
            const float fy = ((float)y + 0.5f) * (float)Hi / (float)Ho - 0.5f;
            const int iy = (int)std::floor(fy);
            const float dy = fy - iy;
            for (int x = 0; x < Wo; ++x) {
                const float fx = ((float)x + 0.5f) * (float)Wi / (float)Wo - 0.5f;
                const int ix = (int)std::floor(fx);
                const float dx = fx - ix;
                float val = 0.0f;
                for (int jj = -1; jj <= 2; ++jj) {
                    const float wy = cubic(dy - jj);
                    const int sy = std::min(std::max(iy + jj, 0), Hi - 1);
                    for (int ii = -1; ii <= 2; ++ii) {
                        const float wx = cubic(dx - ii);
                        const int sx = std::min(std::max(ix + ii, 0), Wi - 1);
                        val += wy * wx * src[(size_t)c * Hi * Wi + sy * Wi + sx];
                    }
                }
                dst[(size_t)c * Ho * Wo + y * Wo + x] = val;
            }
        }
}

// ggml_gelu's fp16 table (ggml_vec_gelu_f32 with GGML_GELU_FP16):
// fp16(0.5·v·(1 + tanhf(√(2/π)·v·(1 + 0.044715·v²)))) for every fp16 v.
// sam2_compute_pos_embed (sam3.cpp:4114-4171) for a G × G token grid:
// bicubic background + the window PE tiled, as [G][G][E0]
std::vector<float> pos_embed(const HieraModel *m, int G) {
    const int E = m->E0, ws = m->win_side;
    std::vector<float> interp((size_t)E * G * G), pe((size_t)E * G * G);
    bicubic(m->bkg_chw.data(), E, m->bkg_h, m->bkg_w, interp.data(), G, G);
    for (int y = 0; y < G; ++y)
        for (int x = 0; x < G; ++x)
            for (int e = 0; e < E; ++e)
                pe[((size_t)y * G + x) * E + e] = interp[(size_t)e * G * G + (size_t)y * G + x] +
                                                  m->win_chw[(size_t)e * ws * ws + (y % ws) * ws + (x % ws)];
    return pe;
}

std::vector<uint16_t> gelu_table() {
    std::vector<uint16_t> t(65536);
    const float SQRT_2_OVER_PI = 0.79788456080286535587989211986876f, A = 0.044715f;
    for (int i = 0; i < 65536; i++) {
        const float v = host_h2f((uint16_t)i);
        t[(size_t)i] = host_f2h(0.5f * v * (1.0f + std::tanh(SQRT_2_OVER_PI * v * (1.0f + A * v * v))));
    }
    return t;
}

Act plane_act(AKind kind, void *base, int64_t cap, int64_t ld) {
    Act a;
    a.kind = kind;
    a.x = base;
    a.lo = (_Float16 *)base + cap;
    a.ld = ld;
    return a;
}

int hd_pad(int hd) { return hd <= 64 ? 64 : 128; }

}  // namespace

int hiera_load(int device, std::ifstream &fin, int ftype, int32_t n_tensors, HieraModel **out, MemAttnModel **ma) {
    (void)device;
    *out = nullptr;
    std::unique_ptr<HieraModel> m(new HieraModel);
    int32_t v[57];
    if (!fin.read((char *)v, sizeof v)) { set_error("s3e_model_load: truncated SAM2 hparams"); return S3E_ERR_IO; }
    if (v[1] != 1) { set_error("s3e_model_load: backbone type %d is not Hiera (EdgeTAM is not supported)", v[1]); return S3E_ERR_UNSUPPORTED; }
    m->ftype = ftype;
    switch (ftype) {
        case 0: case 1: case 2: case 3: case 8: m->wtype = ftype; break;
        default: set_error("s3e_model_load: unsupported ftype %d", ftype); return S3E_ERR_UNSUPPORTED;
    }
    m->img = v[0]; m->E0 = v[2]; m->heads0 = v[3];
    for (int i = 0; i < 4; i++) m->stages[i] = v[5 + i];
    m->gn = v[9];
    for (int i = 0; i < 8; i++) m->gidx[i] = v[10 + i];
    m->q_pool = v[18];
    for (int i = 0; i < 4; i++) m->wspec[i] = v[19 + i];
    m->bkg_h = v[23]; m->bkg_w = v[24]; m->scalp = v[25];
    m->D = v[26]; m->td_n = v[27];
    for (int i = 0; i < 4; i++) m->td[i] = v[28 + i];
    if (v[4] != 4 || m->img <= 0 || m->img % 32 != 0 || m->E0 <= 0 || m->heads0 <= 0 || m->E0 % m->heads0 != 0 ||
        m->gn < 0 || m->gn > 8 || m->q_pool < 0 || m->q_pool > 3 || m->scalp < 0 || m->scalp > 3 || m->D <= 0 ||
        m->td_n < 0 || m->td_n > 4 || m->bkg_h <= 0 || m->bkg_w <= 0) {
        set_error("s3e_model_load: inconsistent Hiera hparams");
        return S3E_ERR_IO;
    }
    for (int i = 0; i < 4; i++)
        if (m->stages[i] <= 0 || m->wspec[i] <= 0) { set_error("s3e_model_load: inconsistent Hiera stages"); return S3E_ERR_IO; }
    m->G = m->img / 4;
    block_metadata(m.get());
    // what the kernels need: heads of at most 128 channels, float4 rows, 32-wide
    // K blocks where a layer is quantized (checked below per weight)
    for (const HBlock &b : m->blocks) {
        if (b.dout % b.heads != 0 || b.dout / b.heads > 128 || (b.dout / b.heads) % 8 != 0 || b.din % 4 != 0) {
            set_error("s3e_model_load: Hiera block with width %d and %d heads is not supported", b.dout, b.heads);
            return S3E_ERR_UNSUPPORTED;
        }
        // un-partition after Q pooling must meet the partition's window count
        if (b.qs && b.ws > 0 && (b.ws % 2 != 0)) { set_error("s3e_model_load: odd window %d at a Q-stride block", b.ws); return S3E_ERR_UNSUPPORTED; }
    }
    if (m->D % 32 != 0) { set_error("s3e_model_load: neck_dim %d must be a multiple of 32", m->D); return S3E_ERR_UNSUPPORTED; }
    const int wtype = m->wtype;
    std::vector<float> bkg, win;
    int64_t win_side = 0;
    for (int ti = 0; ti < n_tensors; ti++) {
        int32_t hdr[3];
        if (!fin.read((char *)hdr, 12)) { set_error("s3e_model_load: truncated tensor header %d", ti); return S3E_ERR_IO; }
        RawTensor t;
        t.n_dims = hdr[0];
        const int32_t name_len = hdr[1];
        t.type = hdr[2];
        if (t.n_dims < 1 || t.n_dims > 4 || name_len <= 0 || name_len > 256 || ggml_tsize(t.type) == 0) {
            set_error("s3e_model_load: malformed tensor record %d", ti);
            return S3E_ERR_IO;
        }
        for (int i = 0; i < t.n_dims; i++) {
            int32_t dd;
            if (!fin.read((char *)&dd, 4) || dd <= 0) { set_error("s3e_model_load: bad dims in record %d", ti); return S3E_ERR_IO; }
            t.ne[i] = dd;
        }
        std::string name((size_t)name_len, '\0');
        if (!fin.read(&name[0], name_len)) { set_error("s3e_model_load: truncated name"); return S3E_ERR_IO; }
        const std::streamoff pos = fin.tellg();
        fin.seekg((32 - pos % 32) % 32, std::ios::cur);
        if (t.ne[0] % ggml_blck(t.type) != 0) { set_error("s3e_model_load: '%s' ne0 not a block multiple", name.c_str()); return S3E_ERR_IO; }
        size_t bytes = 0;
        if (!fin || !record_bytes(t.type, t.ne, stream_left(fin), &bytes)) {
            set_error("s3e_model_load: data of '%s' oversized or past the end of the file", name.c_str());
            return S3E_ERR_IO;
        }
        const int64_t n_el = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
        if (memattn_wants(name)) {
            t.data.resize(bytes);
            if (!fin.read((char *)t.data.data(), (std::streamsize)bytes)) { set_error("s3e_model_load: truncated data of '%s'", name.c_str()); return S3E_ERR_IO; }
            const int rc = memattn_take(ma, name, std::move(t), wtype);
            if (rc != S3E_OK) return rc;
            continue;
        }
        if (name.compare(0, 6, "hiera.") != 0 && name.compare(0, 4, "fpn.") != 0) {
            fin.seekg((std::streamoff)bytes, std::ios::cur);
            if (!fin) { set_error("s3e_model_load: truncated data of '%s'", name.c_str()); return S3E_ERR_IO; }
            continue;
        }
        t.data.resize(bytes);
        if (!fin.read((char *)t.data.data(), (std::streamsize)bytes)) { set_error("s3e_model_load: truncated data of '%s'", name.c_str()); return S3E_ERR_IO; }
        // registered type: T1f/T4f → F32; T2/T4 → weight type iff ne0 % block == 0
        int want = 0;
        if (t.n_dims >= 2 && name.find("pos_embed") == std::string::npos)
            want = (t.ne[0] % ggml_blck(wtype) == 0) ? wtype : 0;
        if (!coerce(t, want)) { set_error("s3e_model_load: cannot convert '%s' from type %d to %d", name.c_str(), t.type, want); return S3E_ERR_IO; }
        int rc = S3E_OK;
        if (name == "hiera.patch_embed.weight") {
            if (t.ne[0] != 7 || t.ne[1] != 7 || t.ne[2] != 3 || t.ne[3] != m->E0) { set_error("patch_embed shape mismatch"); return S3E_ERR_IO; }
            // K = 147 padded with zero columns to a multiple of 32 (the im2col rows are padded the same way)
            const int64_t K = 147, Kp = round_up(K, 32);
            const int es = (t.type == 1) ? 2 : 4;
            std::vector<uint8_t> padded((size_t)(m->E0 * Kp * es), 0);
            for (int64_t n = 0; n < m->E0; n++)
                std::memcpy(&padded[(size_t)(n * Kp * es)], &t.data[(size_t)(n * K * es)], (size_t)(K * es));
            m->patch_k = Kp;
            // an F32 kernel runs as split fp16 pairs on the fp16 MFMA
            if (t.type == 0) rc = upload_weight_split((const float *)padded.data(), Kp, m->E0, m->patch, GEMM_BN);
            else rc = upload_weight(0, t.type, Kp, m->E0, padded.data(), padded.size(), m->patch);
            m->found_misc++;
        } else if (name == "hiera.patch_embed.bias") {
            rc = upload_f32(m.get(), t, m->E0, &m->patch_b);
            m->found_misc++;
        } else if (name == "hiera.pos_embed") {
            if (t.ne[0] != m->bkg_w || t.ne[1] != m->bkg_h || t.ne[2] != m->E0) { set_error("pos_embed shape mismatch"); return S3E_ERR_IO; }
            bkg.assign((const float *)t.data.data(), (const float *)t.data.data() + n_el);
            m->found_misc++;
        } else if (name == "hiera.pos_embed_window") {
            if (t.ne[0] != t.ne[1] || t.ne[2] != m->E0) { set_error("pos_embed_window shape mismatch"); return S3E_ERR_IO; }
            win_side = t.ne[0];
            win.assign((const float *)t.data.data(), (const float *)t.data.data() + n_el);
            m->found_misc++;
        } else if (name.compare(0, 13, "hiera.blocks.") == 0) {
            const size_t dot = name.find('.', 13);
            const int bi = std::atoi(name.substr(13, dot - 13).c_str());
            if (dot == std::string::npos || bi < 0 || bi >= (int)m->blocks.size()) { set_error("tensor '%s' has a bad block index", name.c_str()); return S3E_ERR_IO; }
            HBlock &b = m->blocks[(size_t)bi];
            const std::string f = name.substr(dot + 1);
            // F32 linears (the first stage's, whose width is no Q8 block
            // multiple) run as split fp16 pairs on the fp16 MFMA
            auto lin = [&](Weight &w, int64_t K, int64_t N) {
                if (t.ne[0] != K || t.ne[1] != N) { set_error("'%s': expected [%lld, %lld]", name.c_str(), (long long)K, (long long)N); return (int)S3E_ERR_IO; }
                if (t.type == 0 && K % 8 == 0) return upload_weight_split((const float *)t.data.data(), K, N, w, GEMM_BN);
                return upload_weight(0, t.type, K, N, t.data.data(), t.data.size(), w);
            };
            if (f == "norm1.weight") rc = upload_f32(m.get(), t, b.din, &b.n1w);
            else if (f == "norm1.bias") rc = upload_f32(m.get(), t, b.din, &b.n1b);
            else if (f == "norm2.weight") rc = upload_f32(m.get(), t, b.dout, &b.n2w);
            else if (f == "norm2.bias") rc = upload_f32(m.get(), t, b.dout, &b.n2b);
            else if (f == "attn.qkv.weight") rc = lin(b.qkv, b.din, 3LL * b.dout);
            else if (f == "attn.qkv.bias") rc = upload_f32(m.get(), t, 3LL * b.dout, &b.qkv_b);
            else if (f == "attn.proj.weight") rc = lin(b.proj, b.dout, b.dout);
            else if (f == "attn.proj.bias") rc = upload_f32(m.get(), t, b.dout, &b.proj_b);
            else if (f == "mlp.fc1.weight") rc = lin(b.fc1, b.dout, 4LL * b.dout);
            else if (f == "mlp.fc1.bias") rc = upload_f32(m.get(), t, 4LL * b.dout, &b.fc1_b);
            else if (f == "mlp.fc2.weight") rc = lin(b.fc2, 4LL * b.dout, b.dout);
            else if (f == "mlp.fc2.bias") rc = upload_f32(m.get(), t, b.dout, &b.fc2_b);
            else if (f == "proj.weight" && b.din != b.dout) rc = lin(b.dp, b.din, b.dout);
            else if (f == "proj.bias" && b.din != b.dout) rc = upload_f32(m.get(), t, b.dout, &b.dp_b);
            else continue;
            if (rc == S3E_OK) b.found++;
        } else if (name.compare(0, 10, "fpn.convs.") == 0 && name.size() > 11) {
            const int i = name[10] - '0';
            const std::string f = name.substr(11);
            if (i < 0 || i > 3 || name[11] != '.') continue;
            const int stage = 3 - i;
            if (f == ".weight") {
                if (t.ne[0] != 1 || t.ne[1] != 1 || t.ne[2] != m->width[stage] || t.ne[3] != m->D) { set_error("'%s': unexpected shape", name.c_str()); return S3E_ERR_IO; }
                // [1, 1, Cin, Cout]: rows of Cin per output channel; fp16 in F16 files, split planes otherwise
                if (t.type == 1) rc = upload_weight(0, 1, t.ne[2], t.ne[3], t.data.data(), t.data.size(), m->fpn[i], CONV_BN);
                else rc = upload_weight_split((const float *)t.data.data(), t.ne[2], t.ne[3], m->fpn[i], CONV_BN);
            } else if (f == ".bias") {
                rc = upload_f32(m.get(), t, m->D, &m->fpn_b[i]);
            } else {
                continue;
            }
            m->found_misc++;
        } else {
            continue;
        }
        if (rc != S3E_OK) return rc;
    }
    // completeness
    if (m->found_misc != 4 + 8) { set_error("s3e_model_load: found %d of 12 Hiera embedding/FPN tensors", m->found_misc); return S3E_ERR_IO; }
    for (size_t i = 0; i < m->blocks.size(); i++) {
        const HBlock &b = m->blocks[i];
        const int need = b.din != b.dout ? 14 : 12;
        if (b.found != need) { set_error("s3e_model_load: Hiera block %zu: found %d of %d tensors", i, b.found, need); return S3E_ERR_IO; }
        // fc1 feeds its GELU epilogue in 32-column blocks
        if ((4 * b.dout) % 32 != 0) { set_error("s3e_model_load: MLP width %d not a multiple of 32", 4 * b.dout); return S3E_ERR_UNSUPPORTED; }
    }
    // positional embedding (sam2_compute_pos_embed, sam3.cpp:4114-4171): the
    // registered [bkg_w, bkg_h, E, 1] bytes are CHW [E][bkg_h][bkg_w]
    m->bkg_chw = std::move(bkg);
    m->win_chw = std::move(win);
    m->win_side = (int)win_side;
    {
        const std::vector<float> pe = pos_embed(m.get(), m->G);
        void *p = nullptr;
        if (hipMalloc(&p, pe.size() * 4) != hipSuccess || hipMemcpy(p, pe.data(), pe.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
            set_error("s3e_model_load: positional embedding upload failed");
            return S3E_ERR_HIP;
        }
        m->owned.push_back(p);
        m->pe = (float *)p;
    }
    {
        const std::vector<uint16_t> tab = gelu_table();
        void *p = nullptr;
        if (hipMalloc(&p, tab.size() * 2) != hipSuccess || hipMemcpy(p, tab.data(), tab.size() * 2, hipMemcpyHostToDevice) != hipSuccess) {
            set_error("s3e_model_load: GELU table upload failed");
            return S3E_ERR_HIP;
        }
        m->owned.push_back(p);
        m->gelu_tab = (uint16_t *)p;
    }
    *out = m.release();
    return S3E_OK;
}

void hiera_free(HieraModel *m) { delete m; }

int hiera_img_size(const HieraModel *m) { return m->img; }

void hiera_hparams(const HieraModel *m, int32_t out[16]) {
    std::memset(out, 0, 16 * sizeof(int32_t));
    out[0] = m->img;
    out[1] = -1;
    out[2] = m->E0;
    out[3] = (int32_t)m->blocks.size();
    out[4] = m->heads0;
    for (int i = 0; i < 4; i++) out[5 + i] = m->stages[i];
    out[9] = m->q_pool;
    out[10] = m->wspec[0];
    out[11] = m->scalp;
    out[12] = m->ftype;
    out[13] = m->side[0];
    out[14] = m->D;
    out[15] = 1;
}

int hiera_state_create(const HieraModel *m, int img, hipStream_t st, HieraState **out) {
    *out = nullptr;
    if (img == 0) img = m->img;
    // the patch grid must halve evenly at every Q-stride block and at the
    // FPN's top-down steps, as at the native size (a multiple of 32)
    if (img < 32 || img % 32 != 0 || img > 4096) {
        set_error("s3e_state_create: encode image size %d is not a multiple of 32 in [32, 4096]", img);
        return S3E_ERR_UNSUPPORTED;
    }
    std::unique_ptr<HieraState> s(new HieraState);
    s->img = img;
    s->G = img / 4;
    geometry(m, img, s->side, s->in_side);
    if (img == m->img) {
        s->pos = m->pe;
    } else {
        const std::vector<float> pe = pos_embed(m, s->G);
        if (hipMalloc(&s->pe_own, pe.size() * 4) != hipSuccess ||
            hipMemcpy(s->pe_own, pe.data(), pe.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
            set_error("s3e_state_create: positional embedding upload failed");
            return S3E_ERR_NOMEM;
        }
        s->pos = s->pe_own;
    }
    const int64_t G = s->G, T0 = G * G;
    hipError_t e = s->col.alloc(T0, m->patch_k, st);
    int64_t emax = 0, qkv_cap = 0, dp_cap = 0, q_cap = 0, k_cap = 0, v_cap = 0, attn_cap = 0, part_cap = 0;
    int64_t gws_cap = 0;
    {
        int H = (int)G, W = (int)G;
        for (const HBlock &b : m->blocks) {
            const int64_t T = (int64_t)H * W;
            const int Ht = b.qs ? H / 2 : H, Wt = b.qs ? W / 2 : W;
            emax = std::max<int64_t>({emax, b.din, b.dout});
            if (b.qs) qkv_cap = std::max(qkv_cap, T * b.dout);  // Q rows before pooling
            dp_cap = std::max(dp_cap, T * b.dout);
            attn_cap = std::max(attn_cap, (int64_t)Ht * Wt * b.dout);
            gws_cap = std::max({gws_cap, gemm_splitk_floats(b.proj, (int64_t)Ht * Wt),
                                gemm_splitk_floats(b.fc2, (int64_t)Ht * Wt)});
            int wh = b.ws > 0 ? b.ws : H, ww = b.ws > 0 ? b.ws : W;
            const int64_t NW = b.ws > 0 ? (int64_t)((H + b.ws - 1) / b.ws) * ((W + b.ws - 1) / b.ws) : 1;
            const int64_t nkv = (int64_t)wh * ww, nq = b.qs ? (int64_t)(wh / 2) * (ww / 2) : nkv;
            const int64_t hdp = hd_pad(b.dout / b.heads);
            q_cap = std::max(q_cap, NW * b.heads * nq * hdp);
            if (b.ws == 0 && !b.qs) {
                const int ns = attn_splits(nq, nkv, b.heads);
                if (ns > 1) part_cap = std::max(part_cap, (int64_t)ns * b.heads * nq * (hdp + 2));
            }
            k_cap = std::max(k_cap, NW * b.heads * nkv * hdp);
            v_cap = std::max(v_cap, NW * b.heads * vt_ld_for(nkv) * hdp);
            H = Ht;
            W = Wt;
        }
    }
    if (e == hipSuccess) e = s->a1.alloc(T0, emax, st);
    if (e == hipSuccess) e = s->a2.alloc(T0, 4 * emax, st);
    for (int i = 0; i < 4 && e == hipSuccess; i++)
        e = hipMalloc(&s->xs[i], (size_t)s->side[i] * s->side[i] * m->width[i] * 4);
    if (e == hipSuccess) e = hipMalloc(&s->qkv, (size_t)std::max<int64_t>(qkv_cap, 1) * 4);
    if (e == hipSuccess) e = hipMalloc(&s->dp, (size_t)dp_cap * 4);
    if (e == hipSuccess) e = hipMalloc(&s->attn_f32, (size_t)attn_cap * 4);
    if (e == hipSuccess && part_cap > 0) e = hipMalloc(&s->part, (size_t)part_cap * 4);
    s->part_cap = part_cap;
    if (e == hipSuccess && gws_cap > 0) e = hipMalloc(&s->gws, (size_t)gws_cap * 4);
    s->gws_cap = gws_cap;
    s->q_cap = q_cap;
    s->k_cap = k_cap;
    s->v_cap = v_cap;
    if (e == hipSuccess) e = hipMalloc(&s->q16, (size_t)q_cap * 2 * 2);
    if (e == hipSuccess) e = hipMalloc(&s->k16, (size_t)k_cap * 2 * 2);
    if (e == hipSuccess) e = hipMalloc(&s->vt16, (size_t)v_cap * 2 * 2);
    s->fin_cap = 0;
    for (int i = 0; i < 4; i++) s->fin_cap = std::max<int64_t>(s->fin_cap, (int64_t)s->side[i] * s->side[i] * m->width[i]);
    if (e == hipSuccess) e = hipMalloc(&s->fin, (size_t)s->fin_cap * 2 * 2);
    for (int i = 0; i < 4 && e == hipSuccess; i++) e = hipMalloc(&s->lat[i], (size_t)s->side[i] * s->side[i] * m->D * 4);
    for (int i = 0; i < 4 - m->scalp && e == hipSuccess; i++) {
        const std::vector<float> pe = sinusoidal_pe_2d(s->side[i], s->side[i], m->D);
        e = hipMalloc(&s->pe[i], pe.size() * 4);
        if (e == hipSuccess) e = hipMemcpy(s->pe[i], pe.data(), pe.size() * 4, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        set_error("s3e_state_create: %s", hipGetErrorString(e));
        return S3E_ERR_NOMEM;
    }
    *out = s.release();
    return S3E_OK;
}

void hiera_state_free(HieraState *s) { delete s; }

int hiera_state_img(const HieraState *s) { return s->img; }

hipError_t hiera_block(const HieraModel *m, HieraState *s, int bi, const float *x, int H, int W, float *y,
                       hipStream_t st) {
    if (bi < 0 || bi >= (int)m->blocks.size()) return hipErrorInvalidValue;
    const HBlock &b = m->blocks[(size_t)bi];
    // the state's buffers are sized for the encoder's grids; a block that
    // changes size cannot run in place
    const int in_side = s->in_side[(size_t)bi];
    if (H <= 0 || W <= 0 || H > in_side || W > in_side || (b.qs && (H % 2 || W % 2)) ||
        (x == y && (b.qs || b.din != b.dout)))
        return hipErrorInvalidValue;
    const int64_t T = (int64_t)H * W;
    const int Ht = b.qs ? H / 2 : H, Wt = b.qs ? W / 2 : W;
    const int64_t Tt = (int64_t)Ht * Wt;
    const int C = b.dout, NH = b.heads, HD = C / NH, HDp = hd_pad(HD);
    hipError_t e;
    // 1. pre-norm → the QKV (and dim-projection) weight's activation format
    const Act a_in = s->a1.as(act_kind_for(b.qkv.kind), b.din);
    if ((e = launch_layernorm(x, T, b.din, 1e-6f, b.n1w, b.n1b, a_in, nullptr, st)) != hipSuccess) return e;
    // 2. shortcut, written into y (the block's residual stream)
    auto f32_act = [](float *p, int64_t ld) {
        Act a;
        a.kind = A_F32;
        a.x = p;
        a.ld = ld;
        return a;
    };
    if (b.din != b.dout) {
        EpiArgs ed;
        ed.bias = b.dp_b;
        ed.y = b.qs ? s->dp : y;
        ed.ldy = C;
        if ((e = launch_gemm(b.dp, a_in, T, EPI_F32, ed, st)) != hipSuccess) return e;
        if (b.qs && (e = launch_pool_act(s->dp, H, W, C, 2, f32_act(y, C), st)) != hipSuccess) return e;
    } else if (b.qs) {
        if ((e = launch_pool_act(x, H, W, C, 2, f32_act(y, C), st)) != hipSuccess) return e;
    } else if (y != x) {
        if ((e = hipMemcpyAsync(y, x, (size_t)T * C * 4, hipMemcpyDeviceToDevice, st)) != hipSuccess) return e;
    }
    // 3. QKV + bias straight into the attention operands (window order, fp16
    // planes); Q of a Q-stride block goes out as f32 rows for the pooling pass.
    // Quantized and F32 projections re-quantize the attention output: split
    // fp16 pairs keep attention at f32 accuracy; F16 models use plain fp16.
    const bool split = b.proj.kind != WK_F16;
    const int wh = b.ws > 0 ? b.ws : H, ww = b.ws > 0 ? b.ws : W;
    HieraPrepArgs pa;
    pa.qkv = s->qkv;
    pa.qkv_ld = C;
    pa.bias = b.qkv_b;
    pa.H = H; pa.W = W; pa.C = C; pa.NH = NH; pa.HD = HD; pa.HDp = HDp;
    pa.window = b.ws;
    pa.q_stride = b.qs;
    pa.q = s->q16; pa.k = s->k16; pa.vt = s->vt16;
    if (split) {
        pa.q_lo = s->q16 + s->q_cap;
        pa.k_lo = s->k16 + s->k_cap;
        pa.vt_lo = s->vt16 + s->v_cap;
    }
    EpiArgs eq;
    eq.bias = b.qkv_b;
    eq.E = C; eq.HD = HD; eq.NH = NH; eq.hdp = HDp;
    eq.grid = W; eq.grid_h = H; eq.window = b.ws;
    eq.vt_ld = (int)vt_ld_for((int64_t)wh * ww);
    eq.q = pa.q; eq.k = pa.k; eq.vt = pa.vt;
    eq.q_lo = pa.q_lo; eq.k_lo = pa.k_lo; eq.vt_lo = pa.vt_lo;
    eq.qpool = b.qs;
    eq.y = s->qkv;
    eq.ldy = C;
    if ((e = launch_gemm(b.qkv, a_in, T, EPI_HQKV, eq, st)) != hipSuccess) return e;
    if ((e = launch_hiera_pad(pa, st)) != hipSuccess) return e;
    if (b.qs && (e = launch_hiera_prep(pa, st)) != hipSuccess) return e;
    // 4. attention → the proj input at the un-partitioned, cropped token rows
    const int nwx = b.ws > 0 ? (W + b.ws - 1) / b.ws : 1, nwy = b.ws > 0 ? (H + b.ws - 1) / b.ws : 1;
    AttnArgs aa;
    aa.q = s->q16; aa.k = s->k16; aa.vt = s->vt16;
    aa.q_lo = pa.q_lo; aa.k_lo = pa.k_lo; aa.vt_lo = pa.vt_lo;
    aa.Nkv = wh * ww;
    aa.Nq = b.qs ? (wh / 2) * (ww / 2) : aa.Nkv;
    aa.NH = NH;
    aa.BH = nwx * nwy * NH;
    aa.hd = HDp;
    aa.hd_out = HD;
    aa.scale = 1.0f / std::sqrt((float)HD);
    aa.wo = b.qs ? ww / 2 : ww;
    aa.nwx = nwx;
    aa.out_h = Ht;
    aa.out_w = Wt;
    const AKind kp = act_kind_for(b.proj.kind);
    const bool q8 = kp == A_Q8_0 || kp == A_Q8_1;
    // A global block whose query tiles leave CUs idle splits its keys into
    // ranges (partials merged by a second pass, f32 or fp16 output); its
    // single window is the grid, so the output rows need no mapping.
    const int ns = (b.ws == 0 && !b.qs) ? attn_splits(aa.Nq, aa.Nkv, aa.BH) : 1;
    if (ns > 1) {
        const int64_t po = (int64_t)ns * aa.BH * aa.Nq * HDp;
        if (!s->part || po + (int64_t)ns * aa.BH * aa.Nq * 2 > s->part_cap) return hipErrorInvalidValue;
        aa.wo = 0;
        aa.nsplit = ns;
        aa.part_o = s->part;
        aa.part_ml = s->part + po;
    }
    // a Q8 block must lie inside one head; a key-split attention into a Q8
    // format or fp16 pairs goes through f32
    const bool direct = (!q8 || HD % 32 == 0) && (ns == 1 || kp == A_F16);
    const Act a_proj = s->a1.as(kp, C);
    aa.out = direct ? a_proj : f32_act(s->attn_f32, C);
    if ((e = launch_attn(aa, st)) != hipSuccess) return e;
    if (!direct && (e = launch_rows_quant(kp, s->attn_f32, Tt, C, a_proj, st)) != hipSuccess) return e;
    // 5. proj + bias + residual
    EpiArgs ep;
    ep.bias = b.proj_b;
    ep.y = y;
    ep.ldy = C;
    ep.ws = s->gws;
    ep.ws_cap = s->gws_cap;
    if ((e = launch_gemm(b.proj, a_proj, Tt, EPI_RESID, ep, st)) != hipSuccess) return e;
    // 6. MLP: norm2 → fc1 + bias + ggml_gelu → fc2 + bias + residual
    const Act a_fc1 = s->a1.as(act_kind_for(b.fc1.kind), C);
    if ((e = launch_layernorm(y, Tt, C, 1e-6f, b.n2w, b.n2b, a_fc1, nullptr, st)) != hipSuccess) return e;
    EpiArgs e1;
    e1.bias = b.fc1_b;
    e1.out = s->a2.as(act_kind_for(b.fc2.kind), 4 * C);
    e1.gelu_tab = m->gelu_tab;
    if ((e = launch_gemm(b.fc1, a_fc1, Tt, EPI_GELU, e1, st)) != hipSuccess) return e;
    EpiArgs e2;
    e2.bias = b.fc2_b;
    e2.y = y;
    e2.ldy = C;
    e2.ws = s->gws;
    e2.ws_cap = s->gws_cap;
    return launch_gemm(b.fc2, e1.out, Tt, EPI_RESID, e2, st);
}

hipError_t hiera_encode(const HieraModel *m, HieraState *s, const float *chw, hipStream_t st) {
    const int G = s->G;
    // patch embedding 7×7 / 4 / 3 + bias + positional embedding
    const AKind pk = act_kind_for(m->patch.kind);
    const Act col = s->col.as(pk, m->patch_k);
    hipError_t e = launch_im2col_conv(chw, s->img, 7, 4, 3, m->patch_k, pk, col.x, st, col.lo);
    if (e != hipSuccess) return e;
    EpiArgs ea;
    ea.bias = m->patch_b;
    ea.y = s->xs[0];
    ea.ldy = m->E0;
    ea.pos = s->pos;
    ea.pos_grid = G;
    ea.grid = G;
    if ((e = launch_gemm(m->patch, col, (int64_t)G * G, EPI_POS, ea, st)) != hipSuccess) return e;
    // blocks: a stage's first block writes the stage's own buffer
    int H = G, W = G;
    float *x = s->xs[0];
    for (size_t i = 0; i < m->blocks.size(); i++) {
        const HBlock &b = m->blocks[i];
        float *y = (i > 0 && b.stage != m->blocks[i - 1].stage) ? s->xs[b.stage] : x;
        if ((e = hiera_block(m, s, (int)i, x, H, W, y, st)) != hipSuccess) return e;
        x = y;
        if (b.qs) { H /= 2; W /= 2; }
    }
    // FPN: lateral 1×1 (+ bias) per stage, then nearest ×2 top-down adds
    for (int i = 0; i < 4; i++) {
        const Weight &w = m->fpn[3 - i];
        const int sd = s->side[i], ch = m->width[i];
        const Act in = plane_act(act_kind_for(w.kind), s->fin, s->fin_cap, ch);
        if ((e = launch_pool_act(s->xs[i], sd, sd, ch, 1, in, st)) != hipSuccess) return e;
        EpiArgs el;
        el.bias = m->fpn_b[3 - i];
        el.y = s->lat[i];
        el.ldy = m->D;
        if ((e = launch_conv(w, in, (int64_t)sd * sd, EPI_F32, el, nullptr, st)) != hipSuccess) return e;
    }
    int prev = -1;
    for (int i = 3; i >= 0; i--) {
        bool td = false;
        for (int j = 0; j < m->td_n; j++)
            if (m->td[j] == i) td = true;
        if (td && prev >= 0) {
            if (s->side[i] != 2 * s->side[prev]) return hipErrorInvalidValue;
            if ((e = launch_upsample_add(s->lat[i], s->lat[prev], s->side[i], m->D, st)) != hipSuccess) return e;
            prev = i;
        } else if (td || prev < 0) {
            prev = i;
        }
    }
    return hipSuccess;
}

const float *hiera_find_tensor(const HieraModel *m, const HieraState *s, const char *name, int64_t ne[4]) {
    auto level = [&](const char *prefix, int *i) {
        const size_t n = std::strlen(prefix);
        if (std::strncmp(name, prefix, n) == 0 && name[n] >= '0' && name[n] <= '3' && name[n + 1] == 0) {
            *i = name[n] - '0';
            return true;
        }
        return false;
    };
    int i = -1;
    const int n_out = 4 - m->scalp;
    if (level("neck_trk_pe_", &i) || level("pe_", &i)) {
        if (i >= n_out) return nullptr;
        ne[0] = m->D; ne[1] = s->side[i]; ne[2] = s->side[i]; ne[3] = 1;
        return s->pe[i];
    }
    if (level("neck_trk_", &i)) {
        if (i >= n_out) return nullptr;
        ne[0] = m->D; ne[1] = s->side[i]; ne[2] = s->side[i]; ne[3] = 1;
        return s->lat[i];
    }
    if (level("hiera_stage_", &i)) {
        ne[0] = m->width[i]; ne[1] = s->side[i]; ne[2] = s->side[i]; ne[3] = 1;
        return s->xs[i];
    }
    return nullptr;
}

}  // namespace s3e
