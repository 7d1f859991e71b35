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
    int img = 0;            // image size this state encodes (encode_img_size or the model's)
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
    sam3_state_ptr st(new (std::nothrow) sam3_state);
    if (!st) return nullptr;
    st->model = &model;
    st->img = params.encode_img_size > 0 ? params.encode_img_size : model.hp[HP_IMG];
    if (st->img != model.hp[HP_IMG])
        fprintf(stderr, "%s: encode_img_size=%d (model native=%d)\n", __func__, st->img, model.hp[HP_IMG]);
    if (s3e_state_create_sized(model.ctx, model.enc, params.encode_img_size > 0 ? params.encode_img_size : 0,
                               &st->st) != S3E_OK) {
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
    if (state.img != img_size) {
        fprintf(stderr, "%s: the state encodes %d px images (encode_img_size); use sam3_encode_image\n", __func__,
                state.img);
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

// sam3.cpp:6512-6574: the patch embedding as a plain product on the host —
// input and kernel rounded to fp16, one f32 (or double) sum per output
bool sam3_test_run_patch_mulmat_host_ref(const sam3_model &model, const float *input_data, const int64_t input_ne[4],
                                         bool use_double_accum, std::vector<float> &output_data,
                                         int64_t output_ne[4]) try {
    if (!input_data || !model.enc) return false;
    int64_t dims[4];
    for (int i = 0; i < 4; i++) dims[i] = (input_ne && input_ne[i] > 0) ? input_ne[i] : 1;
    std::vector<uint8_t> kern;
    int64_t kne[4];
    if (!model_tensor(model, "vit.patch_embed.proj.weight", S3E_TYPE_F16, kern, kne, __func__)) return false;
    const int64_t kdim = kne[0] * kne[1] * kne[2], cout = kne[3], grid = model.hp[0] / model.hp[1];
    if (dims[0] != kdim || dims[1] != grid || dims[2] != grid) {
        fprintf(stderr, "%s: expected im2col rows of %lld values on a %lldx%lld grid, got dims %lld/%lld/%lld/%lld\n",
                __func__, (long long)kdim, (long long)grid, (long long)grid, (long long)dims[0], (long long)dims[1],
                (long long)dims[2], (long long)dims[3]);
        return false;
    }
    const int64_t npix = dims[1] * dims[2] * dims[3];
    std::vector<float> xr((size_t)(kdim * npix));
    for (size_t i = 0; i < xr.size(); i++) xr[i] = host_h2f(host_f2h(input_data[i]));
    const uint16_t *kh = (const uint16_t *)kern.data();
    output_data.resize((size_t)(npix * cout));
    output_ne[0] = npix;
    output_ne[1] = cout;
    output_ne[2] = 1;
    output_ne[3] = 1;
    // output channel-major: channel c holds npix values
    for (int64_t c = 0; c < cout; ++c) {
        const uint16_t *krow = kh + c * kdim;
        float *o = output_data.data() + c * npix;
        for (int64_t px = 0; px < npix; ++px) {
            const float *v = xr.data() + px * kdim;
            if (use_double_accum) {
                double sum = 0.0;
                for (int64_t j = 0; j < kdim; ++j) sum += (double)v[j] * (double)host_h2f(krow[j]);
                o[px] = (float)sum;
            } else {
                float sum = 0.0f;
                for (int64_t j = 0; j < kdim; ++j) sum += v[j] * host_h2f(krow[j]);
                o[px] = sum;
            }
        }
    }
    return true;
} SAM3_CATCH(false)

// sam3.cpp:6576-6674: one block linear on the host — bias plus the sum of
// fp16(w)·fp16(x), accumulated in f32 (or double) from the bias
bool sam3_test_run_vit_block_linear_host_ref(const sam3_model &model, int block_idx, sam3_vit_block_stage stage,
                                             const float *input_data, const int64_t input_ne[4], bool use_double_accum,
                                             std::vector<float> &output_data, int64_t output_ne[4]) try {
    if (!input_data || !model.enc || block_idx < 0 || block_idx >= model.hp[3]) return false;
    const char *layer = nullptr;
    switch (stage) {
        case SAM3_VIT_BLOCK_STAGE_QKV_PROJ: layer = "attn.qkv"; break;
        case SAM3_VIT_BLOCK_STAGE_ATTN_PROJ: layer = "attn.proj"; break;
        case SAM3_VIT_BLOCK_STAGE_MLP_FC1: layer = "mlp.lin1"; break;
        case SAM3_VIT_BLOCK_STAGE_MLP_FC2: layer = "mlp.lin2"; break;
        default:
            fprintf(stderr, "%s: stage %d is not one of the four block linears\n", __func__, (int)stage);
            return false;
    }
    const std::string base = "vit.blocks." + std::to_string(block_idx) + "." + layer;
    std::vector<uint8_t> wt, bs;
    int64_t wne[4], bne[4];
    if (!model_tensor(model, base + ".weight", S3E_TYPE_F16, wt, wne, __func__) ||
        !model_tensor(model, base + ".bias", S3E_TYPE_F32, bs, bne, __func__))
        return false;
    int64_t dims[4];
    for (int i = 0; i < 4; i++) dims[i] = (input_ne && input_ne[i] > 0) ? input_ne[i] : 1;
    const int64_t kdim = wne[0], nout = wne[1], ntok = dims[1] * dims[2] * dims[3];
    if (dims[0] != kdim) {
        fprintf(stderr, "%s: %s takes rows of %lld values, got dims %lld/%lld/%lld/%lld\n", __func__, base.c_str(),
                (long long)kdim, (long long)dims[0], (long long)dims[1], (long long)dims[2], (long long)dims[3]);
        return false;
    }
    const uint16_t *wh = (const uint16_t *)wt.data();
    const float *bias = (const float *)bs.data();
    std::vector<float> xr((size_t)(kdim * ntok));
    for (size_t i = 0; i < xr.size(); i++) xr[i] = host_h2f(host_f2h(input_data[i]));
    output_data.resize((size_t)(nout * ntok));
    output_ne[0] = nout;
    output_ne[1] = dims[1];
    output_ne[2] = dims[2];
    output_ne[3] = dims[3];
    // token-major output: token t holds nout values
    for (int64_t t = 0; t < ntok; ++t) {
        const float *v = xr.data() + t * kdim;
        float *o = output_data.data() + t * nout;
        for (int64_t c = 0; c < nout; ++c) {
            const uint16_t *wrow = wh + c * kdim;
            if (use_double_accum) {
                double sum = (double)bias[c];
                for (int64_t j = 0; j < kdim; ++j) sum += (double)host_h2f(wrow[j]) * (double)v[j];
                o[c] = (float)sum;
            } else {
                float sum = bias[c];
                for (int64_t j = 0; j < kdim; ++j) sum += host_h2f(wrow[j]) * v[j];
                o[c] = sum;
            }
        }
    }
    return true;
} SAM3_CATCH(false)
