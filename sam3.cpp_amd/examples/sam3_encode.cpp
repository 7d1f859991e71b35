// sam3_encode — encode one image with a SAM 3 or SAM 2 model file through the sam3.h
// encoder API (include/sam3_encoder.h, libs3e.so) and dump state tensors in
// sam3_dump_state_tensor's format (<prefix><name>.bin / .shape).
//
//   sam3_encode -m model.ggml -i image.ppm -o out/ [-t name,name,...] [-r repeats]
//   sam3_encode -m model.ggml -p image.chw.f32 -s img_size -o out/ [...]
//   sam3_encode -m model.ggml -p image.chw.f32 -s img_size -o out/ (-b | -B) block
//
// -b (a windowed block) or -B (a global block: no window stages) runs the
// test-only entry points instead of an encode: the prefix
// (sam3_test_run_vit_block0_input), every prefix stage on the image, and
// block `block`'s stage chain (sam3_test_run_vit_block_stage, each stage fed
// the previous stage's output, residuals added here), dumping each output as
// <out>stage_<name>; for F16 files also the host references of the four
// linears on the same inputs (<out>host_<name>), and finally the backbone alone
// (sam3_encode_vit_from_preprocessed_selective → <out>vit_output).
//
// -i takes a binary PPM (P6, maxval 255): RGB bytes in HWC order, which is
// sam3_image's layout.  -p takes a preprocessed CHW float32 image
// (sam3_encode_image_from_preprocessed).  Default tensors: vit_output and
// the tracker levels neck_trk_0..3 for SAM 3 files; the FPN levels
// neck_trk_0..2 and the Hiera stage outputs hiera_stage_0..3 for SAM 2
// files.  Exit status 0 on success, 1 on failure.
#include <array>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/sam3_encoder.h"

namespace {

bool read_ppm(const std::string &path, sam3_image &img) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::string magic;
    int w = 0, h = 0, maxval = 0;
    f >> magic;
    auto skip_comments = [&]() {
        f >> std::ws;
        while (f.peek() == '#') {
            std::string line;
            std::getline(f, line);
            f >> std::ws;
        }
    };
    skip_comments();
    f >> w;
    skip_comments();
    f >> h;
    skip_comments();
    f >> maxval;
    if (magic != "P6" || w <= 0 || h <= 0 || maxval != 255) return false;
    f.get();  // the single whitespace byte before the raster
    img.width = w;
    img.height = h;
    img.channels = 3;
    img.data.resize((size_t)w * h * 3);
    return (bool)f.read(reinterpret_cast<char *>(img.data.data()), (std::streamsize)img.data.size());
}

bool read_f32(const std::string &path, std::vector<float> &v, size_t n) {
    std::ifstream f(path, std::ios::binary);
    v.resize(n);
    return f && f.read(reinterpret_cast<char *>(v.data()), (std::streamsize)(n * sizeof(float)));
}

bool write_dump(const std::string &prefix, const std::vector<float> &v, const int64_t ne[4]) {
    std::ofstream f(prefix + ".bin", std::ios::binary);
    if (!f || !f.write(reinterpret_cast<const char *>(v.data()), (std::streamsize)(v.size() * sizeof(float)))) return false;
    std::ofstream sh(prefix + ".shape");
    sh << ne[0] << "," << ne[1] << "," << ne[2] << "," << ne[3] << "\n";
    return (bool)sh;
}

// Prefix stages on the image and block `bi`'s stage chain.
int run_stages(const sam3_model &model, sam3_state &state, const std::vector<float> &chw, int img_size, int bi,
               bool global, const std::string &out) {
    std::vector<float> x0, h, x1;
    int64_t ne0[4], ne[4], one[4];
    if (!sam3_test_run_vit_block0_input(model, chw.data(), img_size, x0, ne0)) return 1;
    if (!write_dump(out + "block0_input", x0, ne0)) return 1;
    const char *pnames[] = {"PATCH_EMBED", "PATCH_IM2COL"};
    const int64_t img_ne[4] = {img_size, img_size, 3, 1};
    std::vector<float> cols;
    int64_t cne[4];
    for (int s = 0; s < 2; s++) {
        if (!sam3_test_run_vit_prefix_stage(model, (sam3_vit_prefix_stage)s, chw.data(), img_ne, h, one)) return 1;
        if (!write_dump(out + "stage_" + pnames[s], h, one)) return 1;
        if (s == 1) { cols = h; for (int i = 0; i < 4; i++) cne[i] = one[i]; }
    }
    if (!sam3_test_run_vit_prefix_stage(model, SAM3_VIT_PREFIX_STAGE_PATCH_MULMAT, cols.data(), cne, h, one) ||
        !write_dump(out + "stage_PATCH_MULMAT", h, one))
        return 1;
    const char *bnames[] = {"NORM1", "WINDOW_PART", "QKV_PROJ", "ATTN_CORE", "ATTN_PROJ", "WINDOW_UNPART",
                            "NORM2", "MLP_FC1", "MLP_GELU", "MLP_FC2", "MLP"};
    // each stage's input, kept for the host references
    std::vector<std::vector<float>> in(11);
    std::vector<std::array<int64_t, 4>> in_ne(11);
    auto stage = [&](int s, const std::vector<float> &x, const int64_t *xne, std::vector<float> &y) {
        in[s] = x;
        for (int i = 0; i < 4; i++) in_ne[s][i] = xne[i];
        return sam3_test_run_vit_block_stage(model, bi, (sam3_vit_block_stage)s, x.data(), xne, y, one) &&
               write_dump(out + "stage_" + bnames[s], y, one);
    };
    // attention branch: NORM1 → WINDOW_PART → QKV → ATTN_CORE → ATTN_PROJ → WINDOW_UNPART
    std::vector<float> cur = x0;
    for (int i = 0; i < 4; i++) ne[i] = ne0[i];
    for (int s = SAM3_VIT_BLOCK_STAGE_NORM1; s <= SAM3_VIT_BLOCK_STAGE_WINDOW_UNPART; s++) {
        if (global && (s == SAM3_VIT_BLOCK_STAGE_WINDOW_PART || s == SAM3_VIT_BLOCK_STAGE_WINDOW_UNPART)) continue;
        if (!stage(s, cur, ne, h)) return 1;
        cur.swap(h);
        for (int i = 0; i < 4; i++) ne[i] = one[i];
    }
    x1.resize(x0.size());
    for (size_t i = 0; i < x0.size(); i++) x1[i] = x0[i] + cur[i];
    // MLP branch on LN2(x1): FC1 → GELU → FC2, and MLP in one call
    std::vector<float> n2;
    if (!stage(SAM3_VIT_BLOCK_STAGE_NORM2, x1, ne0, n2)) return 1;
    cur = n2;
    for (int i = 0; i < 4; i++) ne[i] = one[i];
    for (int s = SAM3_VIT_BLOCK_STAGE_MLP_FC1; s <= SAM3_VIT_BLOCK_STAGE_MLP_FC2; s++) {
        if (!stage(s, cur, ne, h)) return 1;
        cur.swap(h);
        for (int i = 0; i < 4; i++) ne[i] = one[i];
    }
    if (!stage(SAM3_VIT_BLOCK_STAGE_MLP, n2, ne0, h)) return 1;
    // host references of the four linears on their stage inputs (F16 weights
    // only: other files make them fail, as the reference's do)
    const int lin[4] = {SAM3_VIT_BLOCK_STAGE_QKV_PROJ, SAM3_VIT_BLOCK_STAGE_ATTN_PROJ, SAM3_VIT_BLOCK_STAGE_MLP_FC1,
                        SAM3_VIT_BLOCK_STAGE_MLP_FC2};
    for (int s : lin) {
        if (!sam3_test_run_vit_block_linear_host_ref(model, bi, (sam3_vit_block_stage)s, in[s].data(),
                                                     in_ne[s].data(), false, h, one))
            break;
        if (!write_dump(out + "host_" + bnames[s], h, one)) return 1;
    }
    const std::vector<std::string> names = {"vit_output"};
    if (!sam3_encode_vit_from_preprocessed_selective(state, model, chw.data(), img_size, names)) return 1;
    if (!sam3_dump_state_tensor(state, "vit_output", out + "vit_output")) return 1;
    sam3_tensor_info info;
    if (sam3_get_state_tensor_info(state, "neck_trk_0", info)) {
        fprintf(stderr, "neck levels must not be readable after a backbone-only encode\n");
        return 1;
    }
    return 0;
}

int usage() {
    fprintf(stderr,
            "usage: sam3_encode -m model.ggml (-i image.ppm | -p chw.f32 -s img_size) -o out_prefix\n"
            "                   [-t name,name,...] [-r repeats] [(-b | -B) block] [-e encode_img_size]\n");
    return 1;
}

}  // namespace

int main(int argc, char **argv) {
    std::string model_path, image_path, chw_path, out = "./", tensors;
    int img_size = 0, repeats = 1, stage_block = -1, encode_img_size = 0;
    bool stage_global = false;
    for (int i = 1; i < argc; i++) {
        const std::string a = argv[i];
        if (i + 1 >= argc) return usage();
        const std::string v = argv[++i];
        if (a == "-m") model_path = v;
        else if (a == "-i") image_path = v;
        else if (a == "-p") chw_path = v;
        else if (a == "-s") img_size = std::atoi(v.c_str());
        else if (a == "-o") out = v;
        else if (a == "-t") tensors = v;
        else if (a == "-r") repeats = std::atoi(v.c_str());
        else if (a == "-e") encode_img_size = std::atoi(v.c_str());
        else if (a == "-b" || a == "-B") {
            stage_block = std::atoi(v.c_str());
            stage_global = a == "-B";
        }
        else return usage();
    }
    if (model_path.empty() || (image_path.empty() == chw_path.empty()) || repeats < 1) return usage();

    sam3_params params;
    params.model_path = model_path;
    params.encode_img_size = encode_img_size;
    auto model = sam3_load_model(params);
    if (!model) return 1;
    auto state = sam3_create_state(*model, params);
    if (!state) return 1;
    const sam3_model_type type = sam3_get_model_type(*model);
    printf("model: %s, visual_only=%d\n",
           type == SAM3_MODEL_SAM3 ? "SAM3" : (type == SAM3_MODEL_SAM2 ? "SAM2" : "SAM3 visual"),
           (int)sam3_is_visual_only(*model));
    if (tensors.empty())
        tensors = type == SAM3_MODEL_SAM2
                      ? "neck_trk_0,neck_trk_1,neck_trk_2,hiera_stage_0,hiera_stage_1,hiera_stage_2,hiera_stage_3"
                      : "vit_output,neck_trk_0,neck_trk_1,neck_trk_2,neck_trk_3";

    sam3_image img;
    std::vector<float> chw;
    if (!image_path.empty()) {
        if (!read_ppm(image_path, img)) {
            fprintf(stderr, "cannot read PPM image '%s'\n", image_path.c_str());
            return 1;
        }
    } else if (img_size <= 0 || !read_f32(chw_path, chw, (size_t)3 * img_size * img_size)) {
        fprintf(stderr, "cannot read %d x %d CHW image '%s'\n", img_size, img_size, chw_path.c_str());
        return 1;
    }
    if (stage_block >= 0) {
        if (chw.empty()) return usage();
        return run_stages(*model, *state, chw, img_size, stage_block, stage_global, out);
    }
    for (int r = 0; r < repeats; r++) {
        const auto t0 = std::chrono::steady_clock::now();
        const bool ok = image_path.empty() ? sam3_encode_image_from_preprocessed(*state, *model, chw.data(), img_size)
                                           : sam3_encode_image(*state, *model, img);
        const auto t1 = std::chrono::steady_clock::now();
        if (!ok) return 1;
        printf("encode %d: %.2f ms (host preprocessing and copies included)\n", r,
               std::chrono::duration<double, std::milli>(t1 - t0).count());
    }
    std::stringstream ss(tensors);
    std::string name;
    while (std::getline(ss, name, ',')) {
        if (name.empty()) continue;
        sam3_tensor_info info;
        if (!sam3_get_state_tensor_info(*state, name, info)) return 1;
        if (!sam3_dump_state_tensor(*state, name, out + name)) return 1;
        printf("%s: [%lld, %lld, %lld, %lld]\n", name.c_str(), (long long)info.ne[0], (long long)info.ne[1],
               (long long)info.ne[2], (long long)info.ne[3]);
    }
    return 0;
}
