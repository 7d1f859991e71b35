// sam3_encoder.cpp — sam3.h's image-encoder entry points (include/sam3_encoder.h)
// on top of the engine's C ABI (include/s3e.h).
//
// Each function keeps the reference's contract: sam3_load_model returns
// nullptr and sam3_encode_image false on failure with a message on stderr
// (sam3.cpp:3200-3344, :6024-6212, :6997-7008); no exception leaves the
// library.  The preprocessing is the engine's, on the device
// (s3e_encode_image_u8: sam3_resize_bilinear + sam3_preprocess_image,
// sam3.cpp:3441-3514, or sam2_preprocess_image, :3518-3544, for SAM 2 files,
// with the same resized bytes).
#include <cstdio>
#include <cstring>
#include <exception>
#include <fstream>
#include <new>

#include "../../include/s3e.h"
#include "../../include/sam3_encoder.h"
#include "s3e_host.h"

struct sam3_model {
    s3e_ctx *ctx = nullptr;
    s3e_model *enc = nullptr;
    int32_t hp[16] = {};
    // scratch state of the test-only stage hooks, made on first use (the
    // reference builds a throw-away graph per call on the model's backend)
    mutable s3e_state *hook = nullptr;
    ~sam3_model() { sam3_free_model(*this); }
};

struct sam3_state {
    const sam3_model *model = nullptr;
    s3e_state *st = nullptr;
    bool vit_only = false;  // after sam3_encode_vit_from_preprocessed_selective
    ~sam3_state() { sam3_free_state(*this); }
};

// Handlers of the function-try-blocks around the sam3.h entry points: no
// exception (a failed host allocation, a stream error) leaves the library.
#define SAM3_CATCH(ret)                                                   \
    catch (const std::exception &ex_) {                                   \
        fprintf(stderr, "%s: %s\n", __func__, ex_.what());                \
        return ret;                                                       \
    }                                                                     \
    catch (...) {                                                         \
        fprintf(stderr, "%s: unexpected exception\n", __func__);          \
        return ret;                                                       \
    }

namespace {

// hparams slots of s3e_model_hparams
constexpr int HP_IMG = 0;

bool read_magic(const std::string &path, uint32_t *magic) {
    std::ifstream f(path, std::ios::binary);
    return f && f.read(reinterpret_cast<char *>(magic), 4);
}

}  // namespace

std::shared_ptr<sam3_model> sam3_load_model(const sam3_params &params) try {
    if (!params.use_gpu) {
        fprintf(stderr, "%s: this encoder runs on the MI355X only (use_gpu = false)\n", __func__);
        return nullptr;
    }
    uint32_t magic = 0;
    if (!read_magic(params.model_path, &magic)) {
        fprintf(stderr, "%s: failed to open '%s'\n", __func__, params.model_path.c_str());
        return nullptr;
    }
    if (magic != 0x73616D33u && magic != 0x73616D32u) {  // "sam3", "sam2"
        fprintf(stderr, "%s: '%s' is not a SAM 3 or SAM 2 model file (magic 0x%08x)\n", __func__,
                params.model_path.c_str(), magic);
        return nullptr;
    }
    std::shared_ptr<sam3_model> m(new (std::nothrow) sam3_model);
    if (!m) return nullptr;
    if (s3e_ctx_create(0, &m->ctx) != S3E_OK || s3e_model_load(m->ctx, params.model_path.c_str(), &m->enc) != S3E_OK ||
        s3e_model_hparams(m->enc, m->hp) != S3E_OK) {
        fprintf(stderr, "%s: %s\n", __func__, s3e_last_error());
        return nullptr;
    }
    return m;
} SAM3_CATCH(nullptr)

void sam3_free_model(sam3_model &model) {
    if (model.hook) s3e_state_free(model.hook);
    model.hook = nullptr;
    if (model.enc) s3e_model_free(model.enc);
    if (model.ctx) s3e_ctx_destroy(model.ctx);
    model.enc = nullptr;
    model.ctx = nullptr;
}

// sam3.cpp:3361-3367: SAM 2 models, and SAM 3 files without the detector
// neck, are visual-only
bool sam3_is_visual_only(const sam3_model &model) { return sam3_get_model_type(model) != SAM3_MODEL_SAM3; }

sam3_model_type sam3_get_model_type(const sam3_model &model) {
    const int t = model.enc ? s3e_model_type(model.enc) : 0;
    return t == 2 ? SAM3_MODEL_SAM2 : (t == 1 ? SAM3_MODEL_SAM3_VISUAL : SAM3_MODEL_SAM3);
}

void sam3_state_deleter::operator()(sam3_state *p) const { delete p; }

sam3_state_ptr sam3_create_state(const sam3_model &model, const sam3_params &params) try {
    if (!model.enc) {
        fprintf(stderr, "%s: model is not loaded\n", __func__);
        return nullptr;
    }
    if (params.encode_img_size != 0 && params.encode_img_size != model.hp[HP_IMG]) {
        fprintf(stderr, "%s: encode_img_size %d is not supported (the model's grid is fixed at %d)\n", __func__,
                params.encode_img_size, model.hp[HP_IMG]);
        return nullptr;
    }
    sam3_state_ptr st(new (std::nothrow) sam3_state);
    if (!st) return nullptr;
    st->model = &model;
    if (s3e_state_create(model.ctx, model.enc, &st->st) != S3E_OK) {
        fprintf(stderr, "%s: %s\n", __func__, s3e_last_error());
        return nullptr;
    }
    return st;
} SAM3_CATCH(nullptr)

void sam3_free_state(sam3_state &state) {
    if (state.st) s3e_state_free(state.st);
    state.st = nullptr;
}

bool sam3_encode_image(sam3_state &state, const sam3_model &model, const sam3_image &image) try {
    if (!state.st || state.model != &model) {
        fprintf(stderr, "%s: state was not created for this model\n", __func__);
        return false;
    }
    if (image.width <= 0 || image.height <= 0 ||
        image.data.size() < (size_t)image.width * (size_t)image.height * 3) {
        fprintf(stderr, "%s: image %dx%d holds %zu bytes, need HWC RGB\n", __func__, image.width, image.height,
                image.data.size());
        return false;
    }
    if (s3e_encode_image_u8(state.st, image.data.data(), image.width, image.height) != S3E_OK) {
        fprintf(stderr, "%s: %s\n", __func__, s3e_last_error());
        return false;
    }
    state.vit_only = false;
    return true;
} SAM3_CATCH(false)

bool sam3_encode_image_from_preprocessed(sam3_state &state, const sam3_model &model, const float *chw_data,
                                         int img_size) try {
    if (!state.st || state.model != &model || !chw_data) {
        fprintf(stderr, "%s: bad argument\n", __func__);
        return false;
    }
    if (img_size != model.hp[HP_IMG]) {
        fprintf(stderr, "%s: img_size mismatch: got %d, expected %d\n", __func__, img_size, model.hp[HP_IMG]);
        return false;
    }
    if (s3e_encode_chw_host(state.st, chw_data) != S3E_OK || s3e_ctx_sync(model.ctx) != S3E_OK) {
        fprintf(stderr, "%s: %s\n", __func__, s3e_last_error());
        return false;
    }
    state.vit_only = false;
    return true;
} SAM3_CATCH(false)

bool sam3_get_state_tensor_info(const sam3_state &state, const std::string &tensor_name, sam3_tensor_info &info) try {
    int64_t ne[4];
    if (!state.st || (state.vit_only && tensor_name != "vit_output") ||
        s3e_state_tensor_info(state.st, tensor_name.c_str(), ne) != S3E_OK) {
        fprintf(stderr, "%s: tensor '%s' not found in state\n", __func__, tensor_name.c_str());
        return false;
    }
    uint64_t nb = 4;
    for (int i = 0; i < 4; i++) {
        info.ne[i] = ne[i];
        info.nb[i] = nb;
        nb *= (uint64_t)ne[i];
    }
    info.type = 0;  // F32
    info.op = 0;
    info.is_contiguous = true;
    return true;
} SAM3_CATCH(false)

bool sam3_dump_state_tensor(const sam3_state &state, const std::string &tensor_name, const std::string &output_path) try {
    sam3_tensor_info info;
    if (!sam3_get_state_tensor_info(state, tensor_name, info)) return false;
    const size_t n = (size_t)(info.ne[0] * info.ne[1] * info.ne[2] * info.ne[3]);
    std::vector<float> data(n);
    if (s3e_state_tensor_get(state.st, tensor_name.c_str(), data.data(), n) != S3E_OK) {
        fprintf(stderr, "%s: %s\n", __func__, s3e_last_error());
        return false;
    }
    {
        std::ofstream f(output_path + ".bin", std::ios::binary);
        if (!f || !f.write(reinterpret_cast<const char *>(data.data()), (std::streamsize)(n * sizeof(float)))) {
            fprintf(stderr, "%s: cannot write '%s.bin'\n", __func__, output_path.c_str());
            return false;
        }
    }
    {
        // ggml_n_dims: up to the last dimension above 1 (at least one)
        int nd = 1;
        for (int i = 1; i < 4; i++)
            if (info.ne[i] > 1) nd = i + 1;
        std::ofstream f(output_path + ".shape");
        if (!f) {
            fprintf(stderr, "%s: cannot write '%s.shape'\n", __func__, output_path.c_str());
            return false;
        }
        for (int i = 0; i < nd; i++) f << (i ? "," : "") << info.ne[i];
        f << "\n";
    }
    fprintf(stderr, "%s: dumped '%s' [%lld, %lld, %lld, %lld] to %s\n", __func__, tensor_name.c_str(),
            (long long)info.ne[0], (long long)info.ne[1], (long long)info.ne[2], (long long)info.ne[3],
            output_path.c_str());
    return true;
} SAM3_CATCH(false)

// ---- test-only entry points (sam3.h:436-496) --------------------------------
namespace {

using s3e::host_f2h;
using s3e::host_h2f;

s3e_state *hook_state(const sam3_model &model, const char *fn) {
    if (!model.enc) {
        fprintf(stderr, "%s: model is not loaded\n", fn);
        return nullptr;
    }
    if (!model.hook && s3e_state_create(model.ctx, model.enc, &model.hook) != S3E_OK) {
        fprintf(stderr, "%s: %s\n", fn, s3e_last_error());
        model.hook = nullptr;
    }
    return model.hook;
}

// Device round trip of one stage call: upload the input, query the output
// shape, run, download.  fn(in, in_ne, out, out_ne) is the s3e stage entry.
template <typename F>
bool run_stage(const sam3_model &model, const char *name, const float *input, const int64_t input_ne[4],
               std::vector<float> &output, int64_t output_ne[4], F fn) {
    if (!input || !output_ne) {
        fprintf(stderr, "%s: input_data is null\n", name);
        return false;
    }
    int64_t ne[4];
    for (int i = 0; i < 4; i++) ne[i] = (input_ne && input_ne[i] > 0) ? input_ne[i] : 1;
    if (fn(nullptr, ne, nullptr, output_ne) != S3E_OK) {
        fprintf(stderr, "%s: %s\n", name, s3e_last_error());
        return false;
    }
    const size_t nin = (size_t)(ne[0] * ne[1] * ne[2] * ne[3]);
    const size_t nout = (size_t)(output_ne[0] * output_ne[1] * output_ne[2] * output_ne[3]);
    void *din = nullptr, *dout = nullptr;
    bool ok = s3e_malloc(model.ctx, nin * 4, &din) == S3E_OK && s3e_malloc(model.ctx, nout * 4, &dout) == S3E_OK &&
              s3e_memcpy_h2d(model.ctx, din, input, nin * 4) == S3E_OK &&
              fn((const float *)din, ne, (float *)dout, output_ne) == S3E_OK;
    if (ok) {
        output.resize(nout);
        ok = s3e_memcpy_d2h(model.ctx, output.data(), dout, nout * 4) == S3E_OK;
    }
    if (!ok) fprintf(stderr, "%s: %s\n", name, s3e_last_error());
    if (din) (void)s3e_free(model.ctx, din);
    if (dout) (void)s3e_free(model.ctx, dout);
    return ok;
}

// A model tensor in its registered type, on the host.
bool model_tensor(const sam3_model &model, const std::string &name, int want, std::vector<uint8_t> &data,
                  int64_t ne[4], const char *fn) {
    int type = -1;
    if (s3e_model_tensor_get(model.enc, name.c_str(), &type, ne, nullptr, 0) != S3E_OK) {
        fprintf(stderr, "%s: %s\n", fn, s3e_last_error());
        return false;
    }
    if (type != want) {
        fprintf(stderr, "%s: unsupported tensor type %d for %s\n", fn, type, name.c_str());
        return false;
    }
    data.resize((size_t)(ne[0] * ne[1] * ne[2] * ne[3]) * (want == S3E_TYPE_F16 ? 2 : 4));
    if (s3e_model_tensor_get(model.enc, name.c_str(), &type, ne, data.data(), data.size()) != S3E_OK) {
        fprintf(stderr, "%s: %s\n", fn, s3e_last_error());
        return false;
    }
    return true;
}

}  // namespace

bool sam3_encode_vit_from_preprocessed_selective(sam3_state &state, const sam3_model &model, const float *chw_data,
                                                 int img_size, const std::vector<std::string> &output_tensors) try {
    if (!state.st || state.model != &model || !chw_data) {
        fprintf(stderr, "%s: bad argument\n", __func__);
        return false;
    }
    if (img_size != model.hp[HP_IMG]) {
        fprintf(stderr, "%s: img_size mismatch: got %d, expected %d\n", __func__, img_size, model.hp[HP_IMG]);
        return false;
    }
    for (const auto &name : output_tensors) {
        if (name != "vit_output") {
            fprintf(stderr, "%s: requested tensor '%s' was not found\n", __func__, name.c_str());
            return false;
        }
    }
    const size_t n = (size_t)3 * img_size * img_size;
    void *d = nullptr;
    bool ok = s3e_malloc(model.ctx, n * 4, &d) == S3E_OK && s3e_memcpy_h2d(model.ctx, d, chw_data, n * 4) == S3E_OK &&
              s3e_encode_vit_chw(state.st, (const float *)d) == S3E_OK && s3e_ctx_sync(model.ctx) == S3E_OK;
    if (!ok) fprintf(stderr, "%s: %s\n", __func__, s3e_last_error());
    if (d) (void)s3e_free(model.ctx, d);
    if (ok) state.vit_only = true;
    return ok;
} SAM3_CATCH(false)

bool sam3_test_run_vit_block0_input(const sam3_model &model, const float *chw_data, int img_size,
                                    std::vector<float> &output_data, int64_t output_ne[4], int n_threads) try {
    (void)n_threads;
    if (!chw_data) {
        fprintf(stderr, "%s: chw_data is null\n", __func__);
        return false;
    }
    if (img_size != model.hp[HP_IMG]) {
        fprintf(stderr, "%s: img_size mismatch: got %d, expected %d\n", __func__, img_size, model.hp[HP_IMG]);
        return false;
    }
    s3e_state *st = hook_state(model, __func__);
    if (!st) return false;
    const int64_t G = model.hp[0] / model.hp[1], E = model.hp[2];
    const size_t nin = (size_t)3 * img_size * img_size, nout = (size_t)(G * G * E);
    void *din = nullptr, *dout = nullptr;
    bool ok = s3e_malloc(model.ctx, nin * 4, &din) == S3E_OK && s3e_malloc(model.ctx, nout * 4, &dout) == S3E_OK &&
              s3e_memcpy_h2d(model.ctx, din, chw_data, nin * 4) == S3E_OK &&
              s3e_vit_prefix(st, (const float *)din, (float *)dout) == S3E_OK;
    if (ok) {
        output_data.resize(nout);
        ok = s3e_memcpy_d2h(model.ctx, output_data.data(), dout, nout * 4) == S3E_OK;
        output_ne[0] = E;
        output_ne[1] = G;
        output_ne[2] = G;
        output_ne[3] = 1;
    }
    if (!ok) fprintf(stderr, "%s: %s\n", __func__, s3e_last_error());
    if (din) (void)s3e_free(model.ctx, din);
    if (dout) (void)s3e_free(model.ctx, dout);
    return ok;
} SAM3_CATCH(false)

bool sam3_test_run_vit_prefix_stage(const sam3_model &model, sam3_vit_prefix_stage stage, const float *input_data,
                                    const int64_t input_ne[4], std::vector<float> &output_data, int64_t output_ne[4],
                                    int n_threads) try {
    (void)n_threads;
    s3e_state *st = hook_state(model, __func__);
    if (!st) return false;
    return run_stage(model, __func__, input_data, input_ne, output_data, output_ne,
                     [&](const float *in, const int64_t *ne, float *out, int64_t *one) {
                         return s3e_vit_prefix_stage(st, (int)stage, in, ne, out, one);
                     });
} SAM3_CATCH(false)

bool sam3_test_run_vit_block_stage(const sam3_model &model, int block_idx, sam3_vit_block_stage stage,
                                   const float *input_data, const int64_t input_ne[4], std::vector<float> &output_data,
                                   int64_t output_ne[4], int n_threads) try {
    (void)n_threads;
    s3e_state *st = hook_state(model, __func__);
    if (!st) return false;
    return run_stage(model, __func__, input_data, input_ne, output_data, output_ne,
                     [&](const float *in, const int64_t *ne, float *out, int64_t *one) {
                         return s3e_vit_block_stage(st, block_idx, (int)stage, in, ne, out, one);
                     });
} SAM3_CATCH(false)

// sam3.cpp:6512-6574: fp16 input and kernel, one f32 (or double) sum per output
bool sam3_test_run_patch_mulmat_host_ref(const sam3_model &model, const float *input_data, const int64_t input_ne[4],
                                         bool use_double_accum, std::vector<float> &output_data,
                                         int64_t output_ne[4]) try {
    if (!input_data || !model.enc) return false;
    int64_t ne[4];
    for (int i = 0; i < 4; i++) ne[i] = (input_ne && input_ne[i] > 0) ? input_ne[i] : 1;
    std::vector<uint8_t> w;
    int64_t wne[4];
    if (!model_tensor(model, "vit.patch_embed.proj.weight", S3E_TYPE_F16, w, wne, __func__)) return false;
    const int64_t patch_k = wne[0] * wne[1] * wne[2], n_out = wne[3], n_img = model.hp[0] / model.hp[1];
    if (ne[0] != patch_k || ne[1] != n_img || ne[2] != n_img) {
        fprintf(stderr, "%s: patch_mulmat input shape mismatch [%lld,%lld,%lld,%lld]\n", __func__, (long long)ne[0],
                (long long)ne[1], (long long)ne[2], (long long)ne[3]);
        return false;
    }
    const int64_t n_patch = ne[1] * ne[2] * ne[3];
    std::vector<float> x((size_t)(patch_k * n_patch));
    for (size_t i = 0; i < x.size(); i++) x[i] = host_h2f(host_f2h(input_data[i]));
    const uint16_t *w16 = (const uint16_t *)w.data();
    output_data.resize((size_t)(n_patch * n_out));
    output_ne[0] = n_patch;
    output_ne[1] = n_out;
    output_ne[2] = 1;
    output_ne[3] = 1;
    for (int64_t oc = 0; oc < n_out; ++oc) {
        const uint16_t *wr = w16 + oc * patch_k;
        float *dst = output_data.data() + oc * n_patch;
        for (int64_t p = 0; p < n_patch; ++p) {
            const float *xr = x.data() + p * patch_k;
            if (use_double_accum) {
                double acc = 0.0;
                for (int64_t k = 0; k < patch_k; ++k) acc += (double)xr[k] * (double)host_h2f(wr[k]);
                dst[p] = (float)acc;
            } else {
                float acc = 0.0f;
                for (int64_t k = 0; k < patch_k; ++k) acc += xr[k] * host_h2f(wr[k]);
                dst[p] = acc;
            }
        }
    }
    return true;
} SAM3_CATCH(false)

// sam3.cpp:6576-6674: bias + Σ fp16(w)·fp16(x), f32 (or double) accumulation
bool sam3_test_run_vit_block_linear_host_ref(const sam3_model &model, int block_idx, sam3_vit_block_stage stage,
                                             const float *input_data, const int64_t input_ne[4], bool use_double_accum,
                                             std::vector<float> &output_data, int64_t output_ne[4]) try {
    if (!input_data || !model.enc || block_idx < 0 || block_idx >= model.hp[3]) return false;
    const char *lin = nullptr;
    switch (stage) {
        case SAM3_VIT_BLOCK_STAGE_QKV_PROJ: lin = "attn.qkv"; break;
        case SAM3_VIT_BLOCK_STAGE_ATTN_PROJ: lin = "attn.proj"; break;
        case SAM3_VIT_BLOCK_STAGE_MLP_FC1: lin = "mlp.lin1"; break;
        case SAM3_VIT_BLOCK_STAGE_MLP_FC2: lin = "mlp.lin2"; break;
        default:
            fprintf(stderr, "%s: unsupported stage %d\n", __func__, (int)stage);
            return false;
    }
    const std::string base = "vit.blocks." + std::to_string(block_idx) + "." + lin;
    std::vector<uint8_t> w, b;
    int64_t wne[4], bne[4];
    if (!model_tensor(model, base + ".weight", S3E_TYPE_F16, w, wne, __func__) ||
        !model_tensor(model, base + ".bias", S3E_TYPE_F32, b, bne, __func__))
        return false;
    int64_t ne[4];
    for (int i = 0; i < 4; i++) ne[i] = (input_ne && input_ne[i] > 0) ? input_ne[i] : 1;
    const int64_t k = wne[0], out_dim = wne[1], n_col = ne[1] * ne[2] * ne[3];
    if (ne[0] != k) {
        fprintf(stderr, "%s: linear input shape mismatch [%lld,%lld,%lld,%lld] for K=%lld\n", __func__,
                (long long)ne[0], (long long)ne[1], (long long)ne[2], (long long)ne[3], (long long)k);
        return false;
    }
    const uint16_t *w16 = (const uint16_t *)w.data();
    const float *bias = (const float *)b.data();
    std::vector<float> x((size_t)(k * n_col));
    for (size_t i = 0; i < x.size(); i++) x[i] = host_h2f(host_f2h(input_data[i]));
    output_data.resize((size_t)(out_dim * n_col));
    output_ne[0] = out_dim;
    output_ne[1] = ne[1];
    output_ne[2] = ne[2];
    output_ne[3] = ne[3];
    for (int64_t col = 0; col < n_col; ++col) {
        const float *xc = x.data() + col * k;
        float *dst = output_data.data() + col * out_dim;
        for (int64_t oc = 0; oc < out_dim; ++oc) {
            const uint16_t *wr = w16 + oc * k;
            if (use_double_accum) {
                double acc = (double)bias[oc];
                for (int64_t i = 0; i < k; ++i) acc += (double)host_h2f(wr[i]) * (double)xc[i];
                dst[oc] = (float)acc;
            } else {
                float acc = bias[oc];
                for (int64_t i = 0; i < k; ++i) acc += host_h2f(wr[i]) * xc[i];
                dst[oc] = acc;
            }
        }
    }
    return true;
} SAM3_CATCH(false)
