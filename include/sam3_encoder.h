/*
 * sam3_encoder.h — the image-encoder part of sam3.cpp's public C++ API
 * (sam3.h), implemented on the MI355X engine (s3e.h).
 *
 * A program that uses sam3.cpp only to load a model, encode images and read
 * the encoder's outputs compiles unchanged against this header and links
 * libs3e.so instead of sam3 + ggml.  Every declaration below has the name,
 * signature, argument meaning and failure behaviour of the sam3.h entry
 * point cited beside it (nullptr / false plus a message on stderr, no
 * exceptions).  The structs repeat sam3.h's field names, types, order and
 * defaults so that code written against sam3.h keeps compiling.
 *
 * Differences, all reported as failures rather than silently changed:
 *   - params.use_gpu == false is refused (the engine encodes on the GPU);
 *   - params.encode_img_size is honoured for SAM 2 files (any multiple of
 *     32; the Hiera grids and positional embedding follow it, as in
 *     sam3_create_state); SAM 3 files accept 0 or the model's img_size
 *     only.  sam3_encode_image_from_preprocessed refuses a state whose
 *     encode size is not the model's (it takes native-size input);
 *   - SAM 2 (Hiera) files are accepted and encoded; EdgeTAM files are
 *     refused;
 *   - the test-only stage hooks take inputs of at most the model's token
 *     count (G² rows), and n_threads is ignored (the work runs on the GPU).
 * The segmentation, tracking and text entry points of sam3.h are not part
 * of the encoder and are not declared here.
 */
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

struct sam3_model;
struct sam3_state;

/* sam3.h:27-30 */
struct sam3_state_deleter { void operator()(sam3_state * p) const; };
using sam3_state_ptr = std::unique_ptr<sam3_state, sam3_state_deleter>;

/* sam3.h:36-41 */
enum sam3_model_type {
    SAM3_MODEL_SAM3        = 0,
    SAM3_MODEL_SAM3_VISUAL = 1,
    SAM3_MODEL_SAM2        = 2,
    SAM3_MODEL_EDGETAM     = 3,
};

/* sam3.h:61-66: HWC RGB uint8 */
struct sam3_image {
    int width    = 0;
    int height   = 0;
    int channels = 3;
    std::vector<uint8_t> data;
};

/* sam3.h:96-102 */
struct sam3_params {
    std::string model_path;
    int         n_threads       = 4;
    bool        use_gpu         = true;
    int         seed            = 42;
    int         encode_img_size = 0;
};

/* sam3.h:112-124 */
enum sam3_vit_block_stage {
    SAM3_VIT_BLOCK_STAGE_NORM1 = 0,
    SAM3_VIT_BLOCK_STAGE_WINDOW_PART,
    SAM3_VIT_BLOCK_STAGE_QKV_PROJ,
    SAM3_VIT_BLOCK_STAGE_ATTN_CORE,
    SAM3_VIT_BLOCK_STAGE_ATTN_PROJ,
    SAM3_VIT_BLOCK_STAGE_WINDOW_UNPART,
    SAM3_VIT_BLOCK_STAGE_NORM2,
    SAM3_VIT_BLOCK_STAGE_MLP_FC1,
    SAM3_VIT_BLOCK_STAGE_MLP_GELU,
    SAM3_VIT_BLOCK_STAGE_MLP_FC2,
    SAM3_VIT_BLOCK_STAGE_MLP,
};

/* sam3.h:126-134 */
enum sam3_vit_prefix_stage {
    SAM3_VIT_PREFIX_STAGE_PATCH_EMBED = 0,
    SAM3_VIT_PREFIX_STAGE_PATCH_IM2COL,
    SAM3_VIT_PREFIX_STAGE_PATCH_MULMAT_RAW,
    SAM3_VIT_PREFIX_STAGE_PATCH_MULMAT,
    SAM3_VIT_PREFIX_STAGE_POS_ADD,
    SAM3_VIT_PREFIX_STAGE_LN_PRE_NORM,
    SAM3_VIT_PREFIX_STAGE_LN_PRE,
};

/* sam3.h:104-110: ne/nb in ggml order; the engine's state tensors are
 * contiguous f32 (type 0) */
struct sam3_tensor_info {
    int64_t  ne[4] = {0, 0, 0, 0};
    uint64_t nb[4] = {0, 0, 0, 0};
    int  type = 0;
    int  op = 0;
    bool is_contiguous = false;
};

/* sam3.h:184: load the encoder of a SAM 3 model file; nullptr on failure */
std::shared_ptr<sam3_model> sam3_load_model(const sam3_params & params);
/* sam3.h:187 */
void sam3_free_model(sam3_model & model);
/* sam3.h:191 */
bool sam3_is_visual_only(const sam3_model & model);
/* sam3.h:194 */
sam3_model_type sam3_get_model_type(const sam3_model & model);

/* sam3.h:201: state holding the encoder outputs; nullptr on failure */
sam3_state_ptr sam3_create_state(const sam3_model & model, const sam3_params & params);
/* sam3.h:205 */
void sam3_free_state(sam3_state & state);

/* sam3.h:216: resize + normalise as sam3.cpp:3441-3514 does (on the device), then the
 * ViT backbone and every FPN neck of the model on the GPU */
bool sam3_encode_image(sam3_state & state, const sam3_model & model, const sam3_image & image);
/* sam3.h:432: CHW f32 already resized and normalised; img_size must equal
 * the model's (sam3.cpp:7004-7008) */
bool sam3_encode_image_from_preprocessed(sam3_state & state, const sam3_model & model,
                                         const float * chw_data, int img_size);

/* sam3.h:407-414: names of sam3.cpp:14334-14376 (vit_output, neck_trk_<i>,
 * neck_det_<i>, neck_det_pe_<i>, pe_<i>).  The dump writes
 * <output_path>.bin (f32, ggml order) and <output_path>.shape (ne up to the
 * last dimension above 1, comma separated), as sam3.cpp:12429-12520 does. */
bool sam3_dump_state_tensor(const sam3_state & state, const std::string & tensor_name,
                            const std::string & output_path);
bool sam3_get_state_tensor_info(const sam3_state & state, const std::string & tensor_name,
                                sam3_tensor_info & info);

/* ---- test-only entry points (sam3.h:436-496) ---- */

/* sam3.h:441: the ViT backbone alone (no neck); output_tensors may name
 * "vit_output" (the only named tensor of the reference's ViT graph,
 * sam3.cpp:6237-6327); afterwards the state holds vit_output only. */
bool sam3_encode_vit_from_preprocessed_selective(sam3_state & state, const sam3_model & model,
                                                 const float * chw_data, int img_size,
                                                 const std::vector<std::string> & output_tensors);
/* sam3.h:451: the prefix (patch embed + pos embed + ln_pre) */
bool sam3_test_run_vit_block0_input(const sam3_model & model, const float * chw_data, int img_size,
                                    std::vector<float> & output_data, int64_t output_ne[4], int n_threads = 4);
/* sam3.h:463: one prefix sub-stage on the GPU */
bool sam3_test_run_vit_prefix_stage(const sam3_model & model, sam3_vit_prefix_stage stage,
                                    const float * input_data, const int64_t input_ne[4],
                                    std::vector<float> & output_data, int64_t output_ne[4], int n_threads = 4);
/* sam3.h:470, :476: host (CPU) references of the patch mul_mat and the
 * block linears for F16 weights: fp16 operands, f32 (or double) sums */
bool sam3_test_run_patch_mulmat_host_ref(const sam3_model & model, const float * input_data,
                                         const int64_t input_ne[4], bool use_double_accum,
                                         std::vector<float> & output_data, int64_t output_ne[4]);
bool sam3_test_run_vit_block_linear_host_ref(const sam3_model & model, int block_idx, sam3_vit_block_stage stage,
                                             const float * input_data, const int64_t input_ne[4],
                                             bool use_double_accum, std::vector<float> & output_data,
                                             int64_t output_ne[4]);
/* sam3.h:489: one block sub-stage on the GPU */
bool sam3_test_run_vit_block_stage(const sam3_model & model, int block_idx, sam3_vit_block_stage stage,
                                   const float * input_data, const int64_t input_ne[4],
                                   std::vector<float> & output_data, int64_t output_ne[4], int n_threads = 4);
