// s3e_rt.h — host-side helpers shared by the runtime translation units
// (s3e_runtime.cpp: contexts, weights, SAM 3 model and state; s3e_hiera.cpp:
// the SAM 2.x Hiera model and state).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <vector>

#include "s3e_host.h"
#include "s3e_internal.h"

// A context: one device and one stream of work (s3e.h).
struct s3e_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    // descriptors of the last batched small-M launch (device copy + host copy,
    // reused while a caller repeats the same batch)
    void *sm_dev = nullptr;
    size_t sm_cap = 0;
    std::vector<uint8_t> sm_last;
    // this device's copy of the allocation-free entry points' scratch array
    void *scratch = nullptr;
    // partial sums of small-M products split over K across work-groups
    float *sk_part = nullptr;
    int64_t sk_part_cap = 0;
    // s3e_flash_attn_ext_f16's operand copies and key-split partials
    void *attn_ws = nullptr;
    size_t attn_ws_cap = 0;
    // the measurement kernels' output words (made at first use)
    uint32_t *probe_sink = nullptr;
    int64_t probe_sink_cap = 0;
};

struct s3e_weight {
    s3e_ctx *ctx = nullptr;
    s3e::Weight w;
    // the small-M kernel's block-interleaved copy, made at first use
    mutable std::mutex mu;
    mutable void *sm = nullptr;
};

namespace s3e {

// Address of the allocation-free entry points' scratch array on `device`
// (which must be current), looked up once per device (s3e_noalloc.cpp).
int noalloc_init(int device, void **scratch);

int64_t round_up(int64_t x, int64_t m);
WKind wkind_of(int type);
void free_weight(Weight &w);
// Repack ggml bytes (N rows of K in `type`) into the GEMM layout and upload;
// N is padded to npad.
int upload_weight(int device, int type, int64_t K, int64_t N, const uint8_t *src, size_t nbytes, Weight &w,
                  int64_t npad = GEMM_BN);
// f32 weights as the two fp16 planes of WK_F16X3, N padded to npad.
int upload_weight_split(const float *src, int64_t K, int64_t N, Weight &w, int64_t npad);

// A tensor record as read from a model file.
struct RawTensor {
    int type = 0;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    std::vector<uint8_t> data;
};

// Convert to the registered type (F32, or F16 from F32); false if impossible.
bool coerce(RawTensor &t, int want);

// sam3_sinusoidal_pe_2d (sam3.cpp:3597-3633): [H][W][d].
std::vector<float> sinusoidal_pe_2d(int H, int W, int d);

// Device activation buffer able to hold M rows of up to K elements in any
// format.  The scale planes are stage-major with a row pitch of M rounded up
// to ROW_PAD and K rounded up to 128 (4 blocks); they are zeroed on the
// stream that will use the buffer, so blocks past K and rows past M hold zero
// scales.
struct ActBuf {
    void *x = nullptr;
    uint16_t *d = nullptr, *s = nullptr;
    int64_t cap_rows = 0, cap_k = 0, mp = 0;
    hipError_t alloc(int64_t M, int64_t K, hipStream_t st) {
        cap_rows = M;
        cap_k = K;
        mp = round_up(M, ROW_PAD);
        const size_t sbytes = (size_t)(mp * (round_up(K, 128) / 32) * 2);
        hipError_t e = hipMalloc(&x, (size_t)(M * K * 4));
        if (e == hipSuccess) e = hipMalloc(&d, sbytes);
        if (e == hipSuccess) e = hipMalloc(&s, sbytes);
        if (e == hipSuccess) e = hipMemsetAsync(d, 0, sbytes, st);
        if (e == hipSuccess) e = hipMemsetAsync(s, 0, sbytes, st);
        return e;
    }
    void release() {
        if (x) (void)hipFree(x);
        if (d) (void)hipFree(d);
        if (s) (void)hipFree(s);
        x = nullptr;
        d = s = nullptr;
    }
    Act as(AKind kind, int64_t ld) const {
        Act a;
        a.kind = kind;
        a.x = x;
        a.d = d;
        a.s = s;
        a.ld = ld;
        a.mp = mp;
        // split fp16 pairs: the low plane fills the second half of the buffer
        if (kind == A_F16X2) a.lo = (void *)((_Float16 *)x + cap_rows * cap_k);
        return a;
    }
};

}  // namespace s3e
