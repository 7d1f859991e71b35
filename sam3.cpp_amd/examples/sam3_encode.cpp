// sam3_encode — encode one image with a SAM 3 or SAM 2 model file through the sam3.h
// encoder API (include/sam3_encoder.h, libs3e.so) and dump state tensors in
// sam3_dump_state_tensor's format (<prefix><name>.bin / .shape).
//
//   sam3_encode -m model.ggml -i image.ppm -o out/ [-t name,name,...] [-r repeats]
//   sam3_encode -m model.ggml -p image.chw.f32 -s img_size -o out/ [...]
//
// -i takes a binary PPM (P6, maxval 255): RGB bytes in HWC order, which is
// sam3_image's layout.  -p takes a preprocessed CHW float32 image
// (sam3_encode_image_from_preprocessed).  Default tensors: vit_output and
// the tracker levels neck_trk_0..3 for SAM 3 files; the FPN levels
// neck_trk_0..2 and the Hiera stage outputs hiera_stage_0..3 for SAM 2
// files.  Exit status 0 on success, 1 on failure.
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

int usage() {
    fprintf(stderr,
            "usage: sam3_encode -m model.ggml (-i image.ppm | -p chw.f32 -s img_size) -o out_prefix\n"
            "                   [-t name,name,...] [-r repeats]\n");
    return 1;
}

}  // namespace

int main(int argc, char **argv) {
    std::string model_path, image_path, chw_path, out = "./", tensors;
    int img_size = 0, repeats = 1;
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
        else return usage();
    }
    if (model_path.empty() || (image_path.empty() == chw_path.empty()) || repeats < 1) return usage();

    sam3_params params;
    params.model_path = model_path;
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
