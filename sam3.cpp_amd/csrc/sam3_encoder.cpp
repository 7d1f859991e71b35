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
#include <fstream>
#include <new>

#include "../../include/s3e.h"
#include "../../include/sam3_encoder.h"

struct sam3_model {
    s3e_ctx *ctx = nullptr;
    s3e_model *enc = nullptr;
    int32_t hp[16] = {};
    ~sam3_model() { sam3_free_model(*this); }
};

struct sam3_state {
    const sam3_model *model = nullptr;
    s3e_state *st = nullptr;
    ~sam3_state() { sam3_free_state(*this); }
};

namespace {

// hparams slots of s3e_model_hparams
constexpr int HP_IMG = 0;

bool read_magic(const std::string &path, uint32_t *magic) {
    std::ifstream f(path, std::ios::binary);
    return f && f.read(reinterpret_cast<char *>(magic), 4);
}

}  // namespace

std::shared_ptr<sam3_model> sam3_load_model(const sam3_params &params) {
    if (!params.use_gpu) {
        fprintf(stderr, "%s: this build encodes on the MI355X only (use_gpu = false)\n", __func__);
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
}

void sam3_free_model(sam3_model &model) {
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

sam3_state_ptr sam3_create_state(const sam3_model &model, const sam3_params &params) {
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
}

void sam3_free_state(sam3_state &state) {
    if (state.st) s3e_state_free(state.st);
    state.st = nullptr;
}

bool sam3_encode_image(sam3_state &state, const sam3_model &model, const sam3_image &image) {
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
    return true;
}

bool sam3_encode_image_from_preprocessed(sam3_state &state, const sam3_model &model, const float *chw_data,
                                         int img_size) {
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
    return true;
}

bool sam3_get_state_tensor_info(const sam3_state &state, const std::string &tensor_name, sam3_tensor_info &info) {
    int64_t ne[4];
    if (!state.st || s3e_state_tensor_info(state.st, tensor_name.c_str(), ne) != S3E_OK) {
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
}

bool sam3_dump_state_tensor(const sam3_state &state, const std::string &tensor_name, const std::string &output_path) {
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
}
