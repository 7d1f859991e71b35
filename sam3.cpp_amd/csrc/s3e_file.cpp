// s3e_file.cpp — sam3.cpp model-file support on the host: the reference
// weight quantizers, row dequantization, and the synthetic random-init model
// writer (the converter + quantize tool for synthetic-weight runs).
//
// File layout (sam3.cpp:3200-3344, :1477-1520, :3091-3143;
// convert_sam3_to_ggml.py:27-67, 202-255):
//   u32 magic "sam3" | i32 version 3 | i32 ftype | i32 n_tensors
//   39 × i32 hparams
//   per tensor: i32 n_dims, i32 name_len, i32 dtype, i32 ne[n_dims] (ggml
//   order), name bytes, zero pad to a 32-byte file offset, raw data.
#include <algorithm>
#include <atomic>
#include <cstdio>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "s3e_host.h"
#include "s3e_internal.h"

namespace s3e {

// ---- reference quantizers (ggml quantize_row_*_ref) -----------------------
void quantize_q4_0(const float *x, uint8_t *y, int64_t k) {
    for (int64_t i = 0; i < k / 32; i++) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; j++) {
            const float v = x[i * 32 + j];
            if (amax < std::fabs(v)) { amax = std::fabs(v); max = v; }
        }
        const float d = max / -8;
        const float id = d ? 1.0f / d : 0.0f;
        uint8_t *blk = y + i * 18;
        const uint16_t dh = host_f2h(d);
        std::memcpy(blk, &dh, 2);
        for (int j = 0; j < 16; ++j) {
            const float x0 = x[i * 32 + j] * id;
            const float x1 = x[i * 32 + 16 + j] * id;
            const int8_t t0 = (int8_t)(x0 + 8.5f), t1 = (int8_t)(x1 + 8.5f);
            const uint8_t a = (uint8_t)std::min<int>(15, t0), b = (uint8_t)std::min<int>(15, t1);
            blk[2 + j] = (uint8_t)(a | (b << 4));
        }
    }
}

void quantize_q4_1(const float *x, uint8_t *y, int64_t k) {
    for (int64_t i = 0; i < k / 32; i++) {
        float min = 3.402823466e+38f, max = -3.402823466e+38f;
        for (int j = 0; j < 32; j++) {
            const float v = x[i * 32 + j];
            if (v < min) min = v;
            if (v > max) max = v;
        }
        const float d = (max - min) / 15;
        const float id = d ? 1.0f / d : 0.0f;
        uint8_t *blk = y + i * 20;
        const uint16_t dh = host_f2h(d), mh = host_f2h(min);
        std::memcpy(blk, &dh, 2);
        std::memcpy(blk + 2, &mh, 2);
        for (int j = 0; j < 16; ++j) {
            const float x0 = (x[i * 32 + j] - min) * id;
            const float x1 = (x[i * 32 + 16 + j] - min) * id;
            const int8_t t0 = (int8_t)(x0 + 0.5f), t1 = (int8_t)(x1 + 0.5f);
            const uint8_t a = (uint8_t)std::min<int>(15, t0), b = (uint8_t)std::min<int>(15, t1);
            blk[4 + j] = (uint8_t)(a | (b << 4));
        }
    }
}

void quantize_q8_0(const float *x, uint8_t *y, int64_t k) {
    for (int64_t i = 0; i < k / 32; i++) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(x[i * 32 + j]));
        const float d = amax / 127;
        const float id = d ? 1.0f / d : 0.0f;
        uint8_t *blk = y + i * 34;
        const uint16_t dh = host_f2h(d);
        std::memcpy(blk, &dh, 2);
        for (int j = 0; j < 32; ++j) blk[2 + j] = (uint8_t)(int8_t)std::round(x[i * 32 + j] * id);
    }
}

void dequantize_row(int type, const uint8_t *x, float *y, int64_t k) {
    switch (type) {
        case 0: std::memcpy(y, x, (size_t)k * 4); break;
        case 1:
            for (int64_t i = 0; i < k; i++) {
                uint16_t h;
                std::memcpy(&h, x + 2 * i, 2);
                y[i] = host_h2f(h);
            }
            break;
        case 2:
            for (int64_t i = 0; i < k / 32; i++) {
                const uint8_t *b = x + i * 18;
                uint16_t dh;
                std::memcpy(&dh, b, 2);
                const float d = host_h2f(dh);
                for (int j = 0; j < 16; j++) {
                    y[i * 32 + j] = (float)((b[2 + j] & 15) - 8) * d;
                    y[i * 32 + 16 + j] = (float)((b[2 + j] >> 4) - 8) * d;
                }
            }
            break;
        case 3:
            for (int64_t i = 0; i < k / 32; i++) {
                const uint8_t *b = x + i * 20;
                uint16_t dh, mh;
                std::memcpy(&dh, b, 2);
                std::memcpy(&mh, b + 2, 2);
                const float d = host_h2f(dh), m = host_h2f(mh);
                for (int j = 0; j < 16; j++) {
                    y[i * 32 + j] = (float)(b[4 + j] & 15) * d + m;
                    y[i * 32 + 16 + j] = (float)(b[4 + j] >> 4) * d + m;
                }
            }
            break;
        case 8:
            for (int64_t i = 0; i < k / 32; i++) {
                const uint8_t *b = x + i * 34;
                uint16_t dh;
                std::memcpy(&dh, b, 2);
                const float d = host_h2f(dh);
                for (int j = 0; j < 32; j++) y[i * 32 + j] = (float)(int8_t)b[2 + j] * d;
            }
            break;
        default: break;
    }
}

namespace {

struct SynthTensor {
    std::string name;
    std::vector<int64_t> ne;  // ggml order
    int kind;                 // 0 = random weight, 1 = ones, 2 = zeros/bias, 3 = freqs
    bool quantizable;         // ne0 % 32 == 0 and a linear/conv weight
    bool pos;                 // F32-registered (pos_embed)
    int freq_side = 0;
    float freq_scale = 1.f;
};

// sam3_compute_axial_cis (sam3.cpp:3555-3586).
void axial_cis(float *out, int dim, int end_x, int end_y, float theta, float scale_pos) {
    const int half_dim = dim / 4;
    std::vector<float> freqs(half_dim);
    for (int i = 0; i < half_dim; ++i) freqs[i] = 1.0f / std::pow(theta, (float)(i * 4) / (float)dim);
    const int N = end_x * end_y;
    for (int idx = 0; idx < N; ++idx) {
        const float tx = (float)(idx % end_x) * scale_pos;
        const float ty = (float)(idx / end_x) * scale_pos;
        for (int i = 0; i < half_dim; ++i) {
            out[idx * dim + i * 2 + 0] = std::cos(tx * freqs[i]);
            out[idx * dim + i * 2 + 1] = std::sin(tx * freqs[i]);
        }
        for (int i = 0; i < half_dim; ++i) {
            out[idx * dim + half_dim * 2 + i * 2 + 0] = std::cos(ty * freqs[i]);
            out[idx * dim + half_dim * 2 + i * 2 + 1] = std::sin(ty * freqs[i]);
        }
    }
}

// N(0, std²) by Box-Muller on mt19937_64 uniform doubles.
void fill_normal(float *x, int64_t n, uint64_t seed, float stdv) {
    std::mt19937_64 rng(seed);
    const double two_pi = 6.283185307179586476925286766559;
    const double inv = 1.0 / 18446744073709551616.0;  // 2^-64
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = ((double)rng() + 0.5) * inv;
        double u2 = ((double)rng() + 0.5) * inv;
        const double r = std::sqrt(-2.0 * std::log(u1));
        x[i] = (float)(r * std::cos(two_pi * u2) * stdv);
        if (i + 1 < n) x[i + 1] = (float)(r * std::sin(two_pi * u2) * stdv);
    }
}

}  // namespace

}  // namespace s3e

namespace s3e {
namespace {

// Generate every tensor of ts (in parallel: each has its own seed) and write
// the file: header, hparams, records.  Stored dtypes follow the converters
// and the quantize tool: 1-D, pos_embed and freqs tensors F32; in F16 files
// every other 2-D+ tensor F16 unless its name contains "embed"
// (convert_sam3_to_ggml.py:220-232, convert_sam2_to_ggml.py:281-293); in
// quantized files 2-D+ tensors whose ne0 is a multiple of 32 are quantized
// (examples/quantize.cpp:195-223).
int write_model(const char *path, uint32_t magic, int32_t version, int ftype, int wtype,
                const std::vector<int32_t> &hp, const std::vector<SynthTensor> &ts, uint64_t seed, float sd,
                bool rnd_affine, int freq_dim) {
    std::vector<std::vector<uint8_t>> data(ts.size());
    std::vector<int> dtypes(ts.size());
    auto work = [&](size_t idx) {
        const SynthTensor &t = ts[idx];
        int64_t n = 1;
        for (auto d : t.ne) n *= d;
        std::vector<float> v((size_t)n);
        const uint64_t sseed = seed * 0x9E3779B97F4A7C15ull + (uint64_t)idx * 0xBF58476D1CE4E5B9ull + 1;
        if (t.kind == 0) {
            fill_normal(v.data(), n, sseed, sd);
        } else if (t.kind == 1) {
            if (rnd_affine) { fill_normal(v.data(), n, sseed, sd); for (auto &x : v) x += 1.0f; }
            else std::fill(v.begin(), v.end(), 1.0f);
        } else if (t.kind == 2) {
            if (rnd_affine) fill_normal(v.data(), n, sseed, sd);
            else std::fill(v.begin(), v.end(), 0.0f);
        } else {
            axial_cis(v.data(), freq_dim, t.freq_side, t.freq_side, 10000.0f, t.freq_scale);
        }
        int dt = 0;
        if (t.ne.size() >= 2 && !t.pos) {
            if (wtype == 1) dt = (t.name.find("embed") == std::string::npos) ? 1 : 0;
            else if (wtype >= 2 && t.ne[0] % 32 == 0) dt = wtype;
        }
        dtypes[idx] = dt;
        const int64_t rows = n / t.ne[0];
        std::vector<uint8_t> &out = data[idx];
        out.resize(ggml_rowsize(dt, t.ne[0]) * (size_t)rows);
        if (dt == 0) {
            std::memcpy(out.data(), v.data(), out.size());
        } else if (dt == 1) {
            for (int64_t i = 0; i < n; i++) {
                const uint16_t h = host_f2h(v[(size_t)i]);
                std::memcpy(out.data() + 2 * i, &h, 2);
            }
        } else {
            const size_t rs = ggml_rowsize(dt, t.ne[0]);
            for (int64_t r = 0; r < rows; r++) {
                const float *src = v.data() + r * t.ne[0];
                uint8_t *dst = out.data() + (size_t)r * rs;
                if (dt == 2) quantize_q4_0(src, dst, t.ne[0]);
                else if (dt == 3) quantize_q4_1(src, dst, t.ne[0]);
                else quantize_q8_0(src, dst, t.ne[0]);
            }
        }
    };
    {
        const unsigned nth = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
        std::vector<std::thread> pool;
        std::atomic_size_t next{0};
        for (unsigned i = 0; i < nth; i++) {
            pool.emplace_back([&]() {
                for (size_t idx = next++; idx < ts.size(); idx = next++) work(idx);
            });
        }
        for (auto &th : pool) th.join();
    }

    FILE *f = std::fopen(path, "wb");
    if (!f) { set_error("s3e_synth_write: cannot open %s", path); return S3E_ERR_IO; }
    auto w32 = [&](int32_t v) { std::fwrite(&v, 4, 1, f); };
    std::fwrite(&magic, 4, 1, f);
    w32(version);
    w32(ftype);
    w32((int32_t)ts.size());
    for (int32_t v : hp) w32(v);
    long pos = 16 + 4 * (long)hp.size();
    for (size_t i = 0; i < ts.size(); i++) {
        const SynthTensor &t = ts[i];
        w32((int32_t)t.ne.size());
        w32((int32_t)t.name.size());
        w32(dtypes[i]);
        for (auto d : t.ne) w32((int32_t)d);
        std::fwrite(t.name.data(), 1, t.name.size(), f);
        pos += 12 + 4 * (long)t.ne.size() + (long)t.name.size();
        const long pad = (32 - pos % 32) % 32;
        static const char zeros[32] = {0};
        std::fwrite(zeros, 1, (size_t)pad, f);
        pos += pad;
        std::fwrite(data[i].data(), 1, data[i].size(), f);
        pos += (long)data[i].size();
    }
    const bool ok = std::ferror(f) == 0;
    std::fclose(f);
    if (!ok) { set_error("s3e_synth_write: write error on %s", path); return S3E_ERR_IO; }
    return S3E_OK;
}

}  // namespace
}  // namespace s3e

using namespace s3e;

namespace {

// Memory attention (sam3.cpp:3034-3060, :2004-2040): D = neck_dim, MD = 64,
// FFN 2048; appended after the encoder's tensors.
void add_mem_attn(std::vector<SynthTensor> &ts, int layers, int D) {
    const int MD = 64, FFN = 2048;
    for (int l = 0; l < layers; l++) {
        const std::string p = "mem_attn.layers." + std::to_string(l);
        for (const char *a : {".sa.q_proj", ".sa.k_proj", ".sa.v_proj", ".sa.out_proj"}) {
            ts.push_back({p + a + ".weight", {D, D}, 0, true, false});
            ts.push_back({p + a + ".bias", {D}, 2, false, false});
        }
        ts.push_back({p + ".norm1.weight", {D}, 1, false, false});
        ts.push_back({p + ".norm1.bias", {D}, 2, false, false});
        ts.push_back({p + ".ca.q_proj.weight", {D, D}, 0, true, false});
        ts.push_back({p + ".ca.q_proj.bias", {D}, 2, false, false});
        ts.push_back({p + ".ca.k_proj.weight", {MD, D}, 0, true, false});
        ts.push_back({p + ".ca.k_proj.bias", {D}, 2, false, false});
        ts.push_back({p + ".ca.v_proj.weight", {MD, D}, 0, true, false});
        ts.push_back({p + ".ca.v_proj.bias", {D}, 2, false, false});
        ts.push_back({p + ".ca.out_proj.weight", {D, D}, 0, true, false});
        ts.push_back({p + ".ca.out_proj.bias", {D}, 2, false, false});
        ts.push_back({p + ".norm2.weight", {D}, 1, false, false});
        ts.push_back({p + ".norm2.bias", {D}, 2, false, false});
        ts.push_back({p + ".linear1.weight", {D, FFN}, 0, true, false});
        ts.push_back({p + ".linear1.bias", {FFN}, 2, false, false});
        ts.push_back({p + ".linear2.weight", {FFN, D}, 0, true, false});
        ts.push_back({p + ".linear2.bias", {D}, 2, false, false});
        ts.push_back({p + ".norm3.weight", {D}, 1, false, false});
        ts.push_back({p + ".norm3.bias", {D}, 2, false, false});
    }
    if (layers > 0) {
        ts.push_back({"mem_attn.norm.weight", {D}, 1, false, false});
        ts.push_back({"mem_attn.norm.bias", {D}, 2, false, false});
    }
}

}  // namespace

extern "C" int s3e_synth_write(const char *path, const s3e_synth_cfg *cfg) try {
    if (!path || !cfg) { set_error("s3e_synth_write: null argument"); return S3E_ERR_INVALID; }
    const int ftype = cfg->ftype;
    int wtype;
    switch (ftype) {
        case 0: wtype = 0; break;
        case 1: wtype = 1; break;
        case 2: wtype = 2; break;
        case 3: wtype = 3; break;
        case 8: wtype = 8; break;
        default: set_error("s3e_synth_write: unsupported ftype %d", ftype); return S3E_ERR_UNSUPPORTED;
    }
    const int E = cfg->embed_dim, P = cfg->patch, img = cfg->img_size, WS = cfg->window;
    if (E <= 0 || P <= 0 || img % P != 0 || cfg->heads <= 0 || E % cfg->heads != 0 || E % 32 != 0 ||
        cfg->depth <= 0 || WS <= 0 || (img / P) % WS != 0 || (img / P) % 3 != 0 || cfg->neck < 0 ||
        cfg->neck > 2 || cfg->neck_dim < 0) {
        set_error("s3e_synth_write: inconsistent hparams");
        return S3E_ERR_INVALID;
    }
    const int G = img / P, HD = E / cfg->heads;
    const int MLP = (int)(E * (cfg->mlp_ratio_x1000 / 1000.0f));
    const int pg = G / 3;  // pretrained grid tiled 3×3 (sam3.cpp:2529-2535)
    auto is_glob = [&](int i) {
        for (int j = 0; j < cfg->n_global && j < 4; j++)
            if (cfg->global_idx[j] == i) return true;
        return false;
    };
    const bool rnd_affine = cfg->std < 0;  // negative std: also randomise biases and LN affine
    const float sd = std::fabs(cfg->std);

    std::vector<SynthTensor> ts;
    ts.push_back({"vit.patch_embed.proj.weight", {P, P, 3, E}, 0, false, false});
    ts.push_back({"vit.pos_embed", {E, pg, pg, 1}, 0, false, true});
    ts.push_back({"vit.ln_pre.weight", {E}, 1, false, false});
    ts.push_back({"vit.ln_pre.bias", {E}, 2, false, false});
    for (int i = 0; i < cfg->depth; i++) {
        const std::string p = "vit.blocks." + std::to_string(i);
        ts.push_back({p + ".norm1.weight", {E}, 1, false, false});
        ts.push_back({p + ".norm1.bias", {E}, 2, false, false});
        ts.push_back({p + ".attn.qkv.weight", {E, 3 * E}, 0, true, false});
        ts.push_back({p + ".attn.qkv.bias", {3 * E}, 2, false, false});
        ts.push_back({p + ".attn.proj.weight", {E, E}, 0, true, false});
        ts.push_back({p + ".attn.proj.bias", {E}, 2, false, false});
        ts.push_back({p + ".norm2.weight", {E}, 1, false, false});
        ts.push_back({p + ".norm2.bias", {E}, 2, false, false});
        ts.push_back({p + ".mlp.lin1.weight", {E, MLP}, 0, true, false});
        ts.push_back({p + ".mlp.lin1.bias", {MLP}, 2, false, false});
        ts.push_back({p + ".mlp.lin2.weight", {MLP, E}, 0, true, false});
        ts.push_back({p + ".mlp.lin2.bias", {E}, 2, false, false});
        SynthTensor f{p + ".attn.freqs_cis", {2, HD / 2, is_glob(i) ? G * G : WS * WS}, 3, false, true};
        f.freq_side = is_glob(i) ? G : WS;
        f.freq_scale = is_glob(i) ? (float)WS / (float)G : 1.0f;
        ts.push_back(f);
    }
    // SimpleFPN necks (sam3.cpp:2562-2591): ggml conv kernels [kW, kH, Cin, Cout],
    // deconvolution kernels [kW, kH, Cout, Cin]; 512 is the reference's
    // fixed intermediate width.
    const int D = cfg->neck_dim > 0 ? cfg->neck_dim : 256;
    const int MID = 512;
    auto add_neck = [&](const std::string &p) {
        ts.push_back({p + "0.dconv_2x2_0.weight", {2, 2, MID, E}, 0, false, false});
        ts.push_back({p + "0.dconv_2x2_0.bias", {MID}, 2, false, false});
        ts.push_back({p + "0.dconv_2x2_1.weight", {2, 2, D, MID}, 0, false, false});
        ts.push_back({p + "0.dconv_2x2_1.bias", {D}, 2, false, false});
        ts.push_back({p + "0.conv_1x1.weight", {1, 1, D, D}, 0, false, false});
        ts.push_back({p + "0.conv_1x1.bias", {D}, 2, false, false});
        ts.push_back({p + "0.conv_3x3.weight", {3, 3, D, D}, 0, false, false});
        ts.push_back({p + "0.conv_3x3.bias", {D}, 2, false, false});
        ts.push_back({p + "1.dconv_2x2.weight", {2, 2, MID, E}, 0, false, false});
        ts.push_back({p + "1.dconv_2x2.bias", {MID}, 2, false, false});
        ts.push_back({p + "1.conv_1x1.weight", {1, 1, MID, D}, 0, false, false});
        ts.push_back({p + "1.conv_1x1.bias", {D}, 2, false, false});
        ts.push_back({p + "1.conv_3x3.weight", {3, 3, D, D}, 0, false, false});
        ts.push_back({p + "1.conv_3x3.bias", {D}, 2, false, false});
        for (int sc = 2; sc < 4; sc++) {
            const std::string q = p + std::to_string(sc);
            ts.push_back({q + ".conv_1x1.weight", {1, 1, E, D}, 0, false, false});
            ts.push_back({q + ".conv_1x1.bias", {D}, 2, false, false});
            ts.push_back({q + ".conv_3x3.weight", {3, 3, D, D}, 0, false, false});
            ts.push_back({q + ".conv_3x3.bias", {D}, 2, false, false});
        }
    };
    if (cfg->neck == 2) add_neck("neck.det.");
    if (cfg->neck >= 1) add_neck("neck.trk.");
    if (cfg->mem_attn_layers < 0 || cfg->mem_attn_layers > 16) {
        set_error("s3e_synth_write: mem_attn_layers %d out of range", cfg->mem_attn_layers);
        return S3E_ERR_INVALID;
    }
    add_mem_attn(ts, cfg->mem_attn_layers, D);

    // hparams in sam3_load_hparams order (sam3.cpp:1477-1520)
    const std::vector<int32_t> hp = {img, P, E, cfg->depth, cfg->heads, cfg->mlp_ratio_x1000, WS, 4,
                                     cfg->n_global > 0 ? cfg->global_idx[0] : -1,
                                     cfg->n_global > 1 ? cfg->global_idx[1] : -1,
                                     cfg->n_global > 2 ? cfg->global_idx[2] : -1,
                                     cfg->n_global > 3 ? cfg->global_idx[3] : -1,
                                     1024, 16, 24, 32, 49408, 256,  // text
                                     D,                             // neck_dim
                                     6, 8, 2048, 6, 8, 2048, 200, 3, 1, 4,
                                     256, 2, 3, 3, 64, cfg->mem_attn_layers > 0 ? cfg->mem_attn_layers : 4, 7, 16, 2,
                                     cfg->neck == 2 ? 0 : 1};       // visual_only
    return write_model(path, 0x73616D33u, 3, ftype, wtype, hp, ts, cfg->seed, sd, rnd_affine, HD);
} S3E_CATCH("s3e_synth_write")

// SAM 2.x (Hiera) encoder file: convert_sam2_to_ggml.py:205-277 header (magic
// "sam2", version 1, 57 hparams), the Hiera and FPN tensors of
// sam2_register_tensors (sam3.cpp:1745-1847), block dimensions from
// sam2_precompute_hiera_metadata (sam3.cpp:1676-1742).
extern "C" int s3e_synth_write_sam2(const char *path, const s3e_synth_sam2_cfg *cfg) try {
    if (!path || !cfg) { set_error("s3e_synth_write_sam2: null argument"); return S3E_ERR_INVALID; }
    const int ftype = cfg->ftype;
    if (ftype != 0 && ftype != 1 && ftype != 2 && ftype != 3 && ftype != 8) {
        set_error("s3e_synth_write_sam2: unsupported ftype %d", ftype);
        return S3E_ERR_UNSUPPORTED;
    }
    const int E0 = cfg->embed_dim, S = cfg->img_size, D = cfg->neck_dim > 0 ? cfg->neck_dim : 256;
    int total = 0;
    for (int i = 0; i < 4; i++) total += cfg->stages[i];
    if (E0 <= 0 || cfg->num_heads <= 0 || S <= 0 || S % 4 != 0 || total <= 0 || cfg->global_n < 0 ||
        cfg->global_n > 8 || cfg->q_pool < 0 || cfg->q_pool > 3 || cfg->bkg_h <= 0 || cfg->bkg_w <= 0 ||
        cfg->window_spec[0] <= 0 || cfg->fpn_td_n < 0 || cfg->fpn_td_n > 4 || cfg->scalp < 0 || cfg->scalp > 3) {
        set_error("s3e_synth_write_sam2: inconsistent hparams");
        return S3E_ERR_INVALID;
    }
    for (int i = 0; i < 4; i++)
        if (cfg->stages[i] <= 0) { set_error("s3e_synth_write_sam2: every stage needs a block"); return S3E_ERR_INVALID; }
    const bool rnd_affine = cfg->std < 0;
    const float sd = std::fabs(cfg->std);
    std::vector<SynthTensor> ts;
    ts.push_back({"hiera.patch_embed.weight", {7, 7, 3, E0}, 0, false, false});
    ts.push_back({"hiera.patch_embed.bias", {E0}, 2, false, false});
    ts.push_back({"hiera.pos_embed", {cfg->bkg_w, cfg->bkg_h, E0, 1}, 0, false, true});
    ts.push_back({"hiera.pos_embed_window", {cfg->window_spec[0], cfg->window_spec[0], E0, 1}, 0, false, true});
    int stage_end[4], cum = 0;
    for (int i = 0; i < 4; i++) { cum += cfg->stages[i]; stage_end[i] = cum - 1; }
    int dim = E0, cur = 0;
    for (int b = 0; b < total; b++) {
        int dout = dim;
        if (b > 0 && b - 1 == stage_end[cur]) { dout = dim * 2; cur++; }
        const std::string p = "hiera.blocks." + std::to_string(b);
        ts.push_back({p + ".norm1.weight", {dim}, 1, false, false});
        ts.push_back({p + ".norm1.bias", {dim}, 2, false, false});
        ts.push_back({p + ".attn.qkv.weight", {dim, 3 * dout}, 0, true, false});
        ts.push_back({p + ".attn.qkv.bias", {3 * dout}, 2, false, false});
        ts.push_back({p + ".attn.proj.weight", {dout, dout}, 0, true, false});
        ts.push_back({p + ".attn.proj.bias", {dout}, 2, false, false});
        ts.push_back({p + ".norm2.weight", {dout}, 1, false, false});
        ts.push_back({p + ".norm2.bias", {dout}, 2, false, false});
        ts.push_back({p + ".mlp.fc1.weight", {dout, 4 * dout}, 0, true, false});
        ts.push_back({p + ".mlp.fc1.bias", {4 * dout}, 2, false, false});
        ts.push_back({p + ".mlp.fc2.weight", {4 * dout, dout}, 0, true, false});
        ts.push_back({p + ".mlp.fc2.bias", {dout}, 2, false, false});
        if (dout != dim) {
            ts.push_back({p + ".proj.weight", {dim, dout}, 0, true, false});
            ts.push_back({p + ".proj.bias", {dout}, 2, false, false});
        }
        dim = dout;
    }
    for (int i = 0; i < 4; i++) {
        const int stage = 3 - i;  // convs[0] maps the widest stage
        const int ch = E0 << stage;
        const std::string p = "fpn.convs." + std::to_string(i);
        ts.push_back({p + ".weight", {1, 1, ch, D}, 0, false, false});
        ts.push_back({p + ".bias", {D}, 2, false, false});
    }
    if (cfg->mem_attn_layers < 0 || cfg->mem_attn_layers > 16) {
        set_error("s3e_synth_write_sam2: mem_attn_layers %d out of range", cfg->mem_attn_layers);
        return S3E_ERR_INVALID;
    }
    add_mem_attn(ts, cfg->mem_attn_layers, D);
    std::vector<int32_t> hp = {S, 1, E0, cfg->num_heads, 4};
    for (int i = 0; i < 4; i++) hp.push_back(cfg->stages[i]);
    hp.push_back(cfg->global_n);
    for (int i = 0; i < 8; i++) hp.push_back(i < cfg->global_n ? cfg->global_idx[i] : 0);
    hp.push_back(cfg->q_pool);
    for (int i = 0; i < 4; i++) hp.push_back(cfg->window_spec[i]);
    hp.push_back(cfg->bkg_h);
    hp.push_back(cfg->bkg_w);
    hp.push_back(cfg->scalp);
    hp.push_back(D);
    hp.push_back(cfg->fpn_td_n);
    for (int i = 0; i < 4; i++) hp.push_back(i < cfg->fpn_td_n ? cfg->fpn_td[i] : 0);
    // SAM decoder, memory, sigmoid scale/bias and flags: SAM 2.1 defaults
    // (convert_sam2_to_ggml.py:44-75)
    for (int32_t v : {256, 2, 3, 3, 64, 4, 7, 16, 2000, -1000, 1, 1, 1, 1, 1, 1, 0, 1, 0, 1, 1, 1, 1, 1, 1})
        hp.push_back(v);
    if (cfg->mem_attn_layers > 0) hp[32 + 5] = cfg->mem_attn_layers;  // mem_attn_layers
    if (hp.size() != 57) { set_error("s3e_synth_write_sam2: internal hparams count"); return S3E_ERR_INVALID; }
    const int wtype = ftype;  // ggml type ids equal the ftype codes used here
    return write_model(path, 0x73616D32u, 1, ftype, wtype, hp, ts, cfg->seed, sd, rnd_affine, 0);
} S3E_CATCH("s3e_synth_write_sam2")
