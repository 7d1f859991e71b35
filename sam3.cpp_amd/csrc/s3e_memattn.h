// s3e_memattn.h — the tracker's memory attention inside the engine
// (s3e_memattn.cpp): weights taken from either model loader, per-state
// scratch, and the layer schedule.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "s3e_rt.h"

namespace s3e {

struct MemAttnModel;
struct MemAttnState;

// Tensors named "mem_attn.*" belong here (sam3.cpp:2004-2040, :3034-3060).
bool memattn_wants(const std::string &name);
// Keep one record (coerced to its registered type); *m is created on first use.
int memattn_take(MemAttnModel **m, const std::string &name, RawTensor &&t, int wtype);
// Check completeness and upload; a model without records stays nullptr.
int memattn_finish(MemAttnModel *m);
void memattn_free(MemAttnModel *m);
// layers, D, MD, FFN
void memattn_dims(const MemAttnModel *m, int32_t out[4]);

void memattn_state_free(MemAttnState *s);
// sam3_build_mem_attn_graph (sam3.cpp:9224-9337) on device buffers; the
// state's scratch grows to the largest (N, M_total) seen.
int memattn_run(const MemAttnModel *m, MemAttnState **s, const float *curr, const float *src_pos, int64_t N,
                const float *prompt, const float *prompt_pos, int64_t M_total, int64_t n_ptr, const float *rope_q,
                const float *rope_k, float *out, hipStream_t st);

}  // namespace s3e
