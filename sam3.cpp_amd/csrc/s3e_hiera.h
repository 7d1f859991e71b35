// s3e_hiera.h — the SAM 2.x Hiera encoder inside the engine (s3e_hiera.cpp):
// model loading, per-image state and the encode schedule, reached from the
// public entry points in s3e_runtime.cpp.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <fstream>

namespace s3e {

struct HieraModel;
struct HieraState;

// Read the SAM 2 hparams and tensor records that follow the 16-byte header
// (sam2_load_hparams + sam3_load_tensors, sam3.cpp:1564-1626, :3091-3194).
struct MemAttnModel;
// "mem_attn.*" records go to *ma (s3e_memattn.h), created when present.
int hiera_load(int device, std::ifstream &fin, int ftype, int32_t n_tensors, HieraModel **out, MemAttnModel **ma);
void hiera_free(HieraModel *m);
// img_size, −1 (marks a Hiera model), embed_dim, blocks, heads, stages[4],
// q_pool, window_spec[0], scalp, ftype, level-0 side, neck_dim, 1 (tracker FPN)
void hiera_hparams(const HieraModel *m, int32_t out[16]);
int hiera_img_size(const HieraModel *m);

// img: the image size this state encodes (0: the model's own); the token
// grids, buffers and positional embedding follow it
int hiera_state_create(const HieraModel *m, int img, hipStream_t st, HieraState **out);
void hiera_state_free(HieraState *s);
int hiera_state_img(const HieraState *s);
// chw: preprocessed image on the device ([3][S][S] f32)
hipError_t hiera_encode(const HieraModel *m, HieraState *s, const float *chw, hipStream_t st);
// Block idx on x ([H·W][dim_in] f32, device) into y ([Ho·Wo][dim_out]).
hipError_t hiera_block(const HieraModel *m, HieraState *s, int idx, const float *x, int H, int W, float *y,
                       hipStream_t st);
// neck_trk_<i>, neck_trk_pe_<i> / pe_<i> (levels below 4 − scalp) and
// hiera_stage_<i>; nullptr if the name does not resolve
const float *hiera_find_tensor(const HieraModel *m, const HieraState *s, const char *name, int64_t ne[4]);

}  // namespace s3e
