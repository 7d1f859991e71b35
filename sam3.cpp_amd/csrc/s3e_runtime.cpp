// s3e_runtime.cpp — host runtime behind include/s3e.h: contexts, weight
// upload and repacking, the operator entry points (mul_mat, flash attention,
// activation conversion), the SAM 3 ViT model loader and the encoder
// schedule.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdlib>
#include <cstring>
#include <cstdio>
#include <fstream>
#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "s3e_host.h"
#include "s3e_internal.h"
#include "s3e_rt.h"
#include "s3e_hiera.h"
#include "s3e_memattn.h"

namespace s3e {

static thread_local std::string g_err;

void set_error(const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
}

}  // namespace s3e

using namespace s3e;

#define HIP_TRY(expr)                                                                   \
    do {                                                                                \
        hipError_t _e = (expr);                                                         \
        if (_e != hipSuccess) {                                                         \
            set_error("%s: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, __LINE__); \
            return S3E_ERR_HIP;                                                         \
        }                                                                               \
    } while (0)

// ---- host helpers shared with s3e_hiera.cpp (declared in s3e_rt.h) ----
namespace s3e {

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

WKind wkind_of(int type) {
    switch (type) {
        case S3E_TYPE_Q4_0: return WK_Q4_0;
        case S3E_TYPE_Q4_1: return WK_Q4_1;
        case S3E_TYPE_Q8_0: return WK_Q8_0;
        case S3E_TYPE_F16: return WK_F16;
        default: return WK_F32;
    }
}

void free_weight(Weight &w) {
    if (w.q) (void)hipFree(w.q);
    if (w.d) (void)hipFree(w.d);
    if (w.m) (void)hipFree(w.m);
    if (w.lo) (void)hipFree(w.lo);
    if (w.f6) (void)hipFree(w.f6);
    w.q = nullptr;
    w.d = w.m = nullptr;
    w.lo = nullptr;
    w.f6 = nullptr;
}

// f32 weights (N rows of K) as two fp16 planes for the split-precision GEMM:
// w·2^k = hi + lo with hi = fp16(w·2^k) and lo = fp16(w·2^k − hi), k chosen
// so that the largest |w|·2^k lies in [2^14, 2^15); alpha = 2^-k.
int upload_weight_split(const float *src, int64_t K, int64_t N, Weight &w, int64_t npad) {
    w = Weight{};
    w.kind = WK_F16X3;
    w.ggml_type = S3E_TYPE_F32;
    w.K = K;
    w.N = N;
    w.Kp = round_up(K, stage_k(WK_F16X3));
    w.Np = round_up(N, npad);
    float amax = 0.f;
    for (int64_t i = 0; i < K * N; i++) amax = std::max(amax, std::fabs(src[i]));
    int k = 0;
    if (amax > 0.f && std::isfinite(amax)) {
        int e = 0;
        (void)std::frexp(amax, &e);  // amax = f·2^e, f in [0.5, 1)
        k = std::min(100, std::max(-100, 15 - e));
    }
    w.alpha = std::ldexp(1.0f, -k);
    std::vector<uint16_t> hi((size_t)(w.Np * w.Kp), 0), lo((size_t)(w.Np * w.Kp), 0);
    for (int64_t n = 0; n < N; n++)
        for (int64_t i = 0; i < K; i++) {
            const float v = std::ldexp(src[n * K + i], k);
            const uint16_t h = host_f2h(v);
            hi[(size_t)(n * w.Kp + i)] = h;
            lo[(size_t)(n * w.Kp + i)] = host_f2h(v - host_h2f(h));
        }
    const size_t bytes = hi.size() * 2;
    hipError_t e = hipMalloc(&w.q, bytes);
    if (e == hipSuccess) e = hipMemcpy(w.q, hi.data(), bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMalloc(&w.lo, bytes);
    if (e == hipSuccess) e = hipMemcpy(w.lo, lo.data(), bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        free_weight(w);
        set_error("weight upload: %s", hipGetErrorString(e));
        return S3E_ERR_HIP;
    }
    w.bytes = 2 * bytes;
    return S3E_OK;
}

// Repack ggml bytes (N rows of K in `type`) into the GEMM layout and upload.
int upload_weight(int device, int type, int64_t K, int64_t N, const uint8_t *src, size_t nbytes,
                  Weight &w, int64_t npad) {
    (void)device;
    if (type != S3E_TYPE_F32 && type != S3E_TYPE_F16 && type != S3E_TYPE_Q4_0 && type != S3E_TYPE_Q4_1 &&
        type != S3E_TYPE_Q8_0) {
        set_error("weight type %d is not supported", type);
        return S3E_ERR_UNSUPPORTED;
    }
    if (K <= 0 || N <= 0 || K % ggml_blck(type) != 0) {
        set_error("weight shape [%lld, %lld] invalid for type %d", (long long)K, (long long)N, type);
        return S3E_ERR_INVALID;
    }
    const size_t rs = ggml_rowsize(type, K);
    if (nbytes < rs * (size_t)N) {
        set_error("weight data holds %zu bytes, need %zu", nbytes, rs * (size_t)N);
        return S3E_ERR_INVALID;
    }
    w = Weight{};
    w.kind = wkind_of(type);
    w.ggml_type = type;
    w.K = K;
    w.N = N;
    w.Kp = round_up(K, stage_k(w.kind));
    w.Np = round_up(N, npad);
    w.Kbp = w.Kp / 32;
    const int64_t Kb = K / 32;
    std::vector<uint8_t> q;
    std::vector<uint16_t> d, m;
    // stage-major scale planes: block b of column n at ((b / 4) * Np + n) * 4 + b % 4
    auto sidx = [&](int64_t n, int64_t b) { return (size_t)(((b >> 2) * w.Np + n) * 4 + (b & 3)); };
    switch (w.kind) {
        case WK_Q4_0:
        case WK_Q4_1:
        case WK_Q8_0: {
            const bool q4 = (w.kind != WK_Q8_0);
            const int bs = (w.kind == WK_Q4_0) ? 18 : (w.kind == WK_Q4_1 ? 20 : 34);
            const int qo = (w.kind == WK_Q4_1) ? 4 : 2;
            q.assign((size_t)(w.Np * w.Kp), 0);
            d.assign((size_t)(w.Np * w.Kbp), 0);
            if (w.kind == WK_Q4_1) m.assign((size_t)(w.Np * w.Kbp), 0);
            for (int64_t n = 0; n < N; n++)
                for (int64_t b = 0; b < Kb; b++) {
                    const uint8_t *blk = src + (size_t)n * rs + (size_t)b * bs;
                    std::memcpy(&d[sidx(n, b)], blk, 2);
                    if (w.kind == WK_Q4_1) std::memcpy(&m[sidx(n, b)], blk + 2, 2);
                    int8_t *dst = (int8_t *)&q[(size_t)(n * w.Kp + b * 32)];
                    if (q4) {
                        // byte j holds element j (low nibble) and element j + 16 (high nibble)
                        const int off = (w.kind == WK_Q4_0) ? 8 : 0;
                        for (int j = 0; j < 16; j++) {
                            dst[j] = (int8_t)((blk[qo + j] & 0x0F) - off);
                            dst[j + 16] = (int8_t)((blk[qo + j] >> 4) - off);
                        }
                    } else {
                        std::memcpy(dst, blk + qo, 32);
                    }
                }
        } break;
        case WK_F16:
        case WK_F32: {
            const int es = (w.kind == WK_F16) ? 2 : 4;
            q.assign((size_t)(w.Np * w.Kp * es), 0);
            for (int64_t n = 0; n < N; n++) std::memcpy(&q[(size_t)(n * w.Kp * es)], src + (size_t)n * rs, (size_t)K * es);
        } break;
        default: break;  // WK_F16X3 comes from upload_weight_split
    }
    // Q4_0 with K a multiple of 128: the codes also as fp6 E3M2 operand words
    std::vector<uint64_t> f6;
    if (w.kind == WK_Q4_0 && K % 128 == 0) {
        const int64_t nst = w.Kp / 128;
        f6.assign((size_t)(w.Np * (w.Kp / 32) * 3), 0);
        for (int64_t n = 0; n < N; n++)
            for (int64_t b = 0; b < Kb; b++) {
                const int8_t *c = (const int8_t *)&q[(size_t)(n * w.Kp + b * 32)];
                uint64_t bits[3] = {0, 0, 0};
                for (int j = 0; j < 32; j++) {
                    const uint64_t v = f6_code(c[j]);
                    const int at = 6 * j;
                    bits[at / 64] |= v << (at % 64);
                    if (at % 64 > 58) bits[at / 64 + 1] |= v >> (64 - at % 64);
                }
                for (int t = 0; t < 3; t++) f6[(size_t)f6_weight_word(nst, n, b, t)] = bits[t];
            }
    }
    hipError_t e = hipMalloc(&w.q, q.size());
    if (e == hipSuccess) e = hipMemcpy(w.q, q.data(), q.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess && !f6.empty()) {
        e = hipMalloc(&w.f6, f6.size() * 8);
        if (e == hipSuccess) e = hipMemcpy(w.f6, f6.data(), f6.size() * 8, hipMemcpyHostToDevice);
    }
    if (e == hipSuccess && !d.empty()) {
        e = hipMalloc(&w.d, d.size() * 2);
        if (e == hipSuccess) e = hipMemcpy(w.d, d.data(), d.size() * 2, hipMemcpyHostToDevice);
    }
    if (e == hipSuccess && !m.empty()) {
        e = hipMalloc(&w.m, m.size() * 2);
        if (e == hipSuccess) e = hipMemcpy(w.m, m.data(), m.size() * 2, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        free_weight(w);
        set_error("weight upload: %s", hipGetErrorString(e));
        return S3E_ERR_HIP;
    }
    w.bytes = q.size() + d.size() * 2 + m.size() * 2 + f6.size() * 8;
    return S3E_OK;
}

// Convert file bytes to the type sam3.cpp registers for the tensor
// (sam3.cpp:2461-2557 registration, :3145-3178 conversion).
bool coerce(RawTensor &t, int want) {
    if (t.type == want) return true;
    int64_t n = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
    if (want == 0) {
        std::vector<uint8_t> out((size_t)n * 4);
        const size_t rs = ggml_rowsize(t.type, t.ne[0]);
        for (int64_t r = 0; r < n / t.ne[0]; r++)
            dequantize_row(t.type, t.data.data() + r * rs, (float *)out.data() + r * t.ne[0], t.ne[0]);
        t.data.swap(out);
        t.type = 0;
        return true;
    }
    if (want == 1 && t.type == 0) {
        std::vector<uint8_t> out((size_t)n * 2);
        const float *src = (const float *)t.data.data();
        for (int64_t i = 0; i < n; i++) {
            const uint16_t h = host_f2h(src[i]);
            std::memcpy(out.data() + 2 * i, &h, 2);
        }
        t.data.swap(out);
        t.type = 1;
        return true;
    }
    return false;
}

// sam3_sinusoidal_pe_2d (sam3.cpp:3597-3633): [H][W][d] with channels
// [0, d/2) following y and [d/2, d) following x, even channels sin, odd cos.
std::vector<float> sinusoidal_pe_2d(int H, int W, int d) {
    const int half = d / 2;
    const float scale = 2.0f * (float)M_PI;
    std::vector<float> pe((size_t)d * H * W);
    for (int y = 0; y < H; ++y)
        for (int x = 0; x < W; ++x) {
            const float py = ((float)(y + 1) / (float)H) * scale;
            const float px = ((float)(x + 1) / (float)W) * scale;
            float *o = pe.data() + ((size_t)y * W + x) * d;
            for (int i = 0; i < half; ++i) {
                const float dim_t = std::pow(10000.0f, (float)(i & ~1) / (float)half);
                o[i] = (i % 2 == 0) ? std::sin(py / dim_t) : std::cos(py / dim_t);
                o[i + half] = (i % 2 == 0) ? std::sin(px / dim_t) : std::cos(px / dim_t);
            }
        }
    return pe;
}

}  // namespace s3e
// ---- end of shared host helpers ----

// ---------------------------------------------------------------------------
extern "C" const char *s3e_last_error(void) { return g_err.c_str(); }
extern "C" int s3e_abi_version(void) { return S3E_ABI_VERSION; }

extern "C" int s3e_ctx_create(int device, s3e_ctx **out) try {
    if (!out) { set_error("s3e_ctx_create: out is NULL"); return S3E_ERR_INVALID; }
    *out = nullptr;
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) {
        set_error("s3e_ctx_create: device %d out of range (%d devices)", device, n);
        return S3E_ERR_INVALID;
    }
    HIP_TRY(hipSetDevice(device));
    // the allocation-free entry points' scratch address on this device
    void *scratch = nullptr;
    const int rc = noalloc_init(device, &scratch);
    if (rc != S3E_OK) return rc;
    auto *c = new s3e_ctx;
    c->device = device;
    c->scratch = scratch;
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        set_error("hipStreamCreate: %s", hipGetErrorString(e));
        return S3E_ERR_HIP;
    }
    *out = c;
    return S3E_OK;
} S3E_CATCH("s3e_ctx_create")

extern "C" void s3e_ctx_destroy(s3e_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipStreamDestroy(ctx->stream);
    if (ctx->sm_dev) (void)hipFree(ctx->sm_dev);
    if (ctx->sk_part) (void)hipFree(ctx->sk_part);
    if (ctx->attn_ws) (void)hipFree(ctx->attn_ws);
    if (ctx->probe_sink) (void)hipFree(ctx->probe_sink);
    delete ctx;
}

extern "C" int s3e_ctx_sync(s3e_ctx *ctx) try {
    if (!ctx) { set_error("s3e_ctx_sync: NULL context"); return S3E_ERR_INVALID; }
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return S3E_OK;
} S3E_CATCH("s3e_ctx_sync")

extern "C" void *s3e_ctx_stream(s3e_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

extern "C" int s3e_malloc(s3e_ctx *ctx, size_t bytes, void **out) try {
    if (!ctx || !out) { set_error("s3e_malloc: NULL argument"); return S3E_ERR_INVALID; }
    HIP_TRY(hipSetDevice(ctx->device));
    if (hipMalloc(out, bytes) != hipSuccess) {
        set_error("s3e_malloc: cannot allocate %zu bytes", bytes);
        return S3E_ERR_NOMEM;
    }
    return S3E_OK;
} S3E_CATCH("s3e_malloc")

extern "C" int s3e_free(s3e_ctx *ctx, void *ptr) try {
    if (!ctx) { set_error("s3e_free: NULL context"); return S3E_ERR_INVALID; }
    if (ptr) HIP_TRY(hipFree(ptr));
    return S3E_OK;
} S3E_CATCH("s3e_free")

extern "C" int s3e_memcpy_h2d(s3e_ctx *ctx, void *dst, const void *src, size_t bytes) try {
    if (!ctx) { set_error("s3e_memcpy_h2d: NULL context"); return S3E_ERR_INVALID; }
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return S3E_OK;
} S3E_CATCH("s3e_memcpy_h2d")

extern "C" int s3e_copy(s3e_ctx *ctx, void *dst, const void *src, size_t bytes) try {
    if (!ctx || !dst || !src) { set_error("s3e_copy: NULL argument"); return S3E_ERR_INVALID; }
    if (bytes % 16 != 0 || ((uintptr_t)dst | (uintptr_t)src) % 16 != 0) {
        set_error("s3e_copy: size and pointers must be 16-byte multiples");
        return S3E_ERR_INVALID;
    }
    HIP_TRY(hipSetDevice(ctx->device));
    HIP_TRY(launch_copy(dst, src, bytes, ctx->stream));
    return S3E_OK;
} S3E_CATCH("s3e_copy")

extern "C" int s3e_memcpy_d2h(s3e_ctx *ctx, void *dst, const void *src, size_t bytes) try {
    if (!ctx) { set_error("s3e_memcpy_d2h: NULL context"); return S3E_ERR_INVALID; }
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return S3E_OK;
} S3E_CATCH("s3e_memcpy_d2h")

// ---- ggml_mul_mat ---------------------------------------------------------
namespace {
hipError_t sm_prepare(s3e_ctx *ctx, const s3e_weight *w);
}  // namespace

extern "C" int s3e_weight_upload(s3e_ctx *ctx, int type, int64_t ne0, int64_t ne1, const void *host_data,
                                 size_t nbytes, s3e_weight **out) try {
    if (!ctx || !host_data || !out) { set_error("s3e_weight_upload: NULL argument"); return S3E_ERR_INVALID; }
    *out = nullptr;
    HIP_TRY(hipSetDevice(ctx->device));
    auto *w = new s3e_weight;
    w->ctx = ctx;
    const int rc = upload_weight(ctx->device, type, ne0, ne1, (const uint8_t *)host_data, nbytes, w->w);
    if (rc != S3E_OK) {
        delete w;
        return rc;
    }
    // everything a product of at most 64 rows needs is made here, so that
    // later products on this weight and context allocate nothing
    const hipError_t e = sm_prepare(ctx, w);
    if (e != hipSuccess) {
        s3e_weight_free(w);
        set_error("s3e_weight_upload: %s", hipGetErrorString(e));
        return S3E_ERR_HIP;
    }
    *out = w;
    return S3E_OK;
} S3E_CATCH("s3e_weight_upload")

extern "C" void s3e_weight_free(s3e_weight *w) {
    if (!w) return;
    free_weight(w->w);
    if (w->sm) (void)hipFree(w->sm);
    delete w;
}

namespace {

// Products of at most 64 rows stream their weights: they run on the small-M
// kernel (k_gemm_sm.hip) from its block-interleaved weight copy.
bool sm_eligible(const Weight &W, int64_t M) {
    return M >= 1 && M <= 64 &&
           (W.kind == WK_Q4_0 || W.kind == WK_Q4_1 || W.kind == WK_Q8_0 || W.kind == WK_F16);
}

hipError_t sm_weights(const s3e_weight *w, hipStream_t st, const uint8_t **out) {
    std::lock_guard<std::mutex> lock(w->mu);
    if (!w->sm) {
        void *p = nullptr;
        hipError_t e = hipMalloc(&p, (size_t)sm_weight_bytes(w->w));
        if (e != hipSuccess) return e;
        e = launch_pack_sm(w->w, p, st);
        // finished before another context's stream may read it
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) {
            (void)hipFree(p);
            return e;
        }
        w->sm = p;
    }
    *out = (const uint8_t *)w->sm;
    return hipSuccess;
}

SmGemm sm_desc(const Weight &W, const uint8_t *wsm, const Act &a, const float *bias, float *Y, int wg0) {
    SmGemm g;
    g.w = wsm;
    g.wd = W.d;
    g.wm = W.m;
    g.x = a.x;
    g.xd = a.d;
    g.xs = a.s;
    g.bias = bias;
    g.y = Y;
    g.ldx = a.ld;
    g.ldy = W.N;
    g.xmp = a.mp;
    g.np = W.Np;
    g.K = (int)W.K;
    g.N = (int)W.N;
    g.nst = (int)((W.Kp + 127) / 128);
    g.wg0 = wg0;
    return g;
}

// Four waves share each 32-column strip's K range.
constexpr int SM_KS = 4;
// A lone small-M product splits K across work-groups until about SM_WG_GOAL
// column-group × K-range work-groups run, keeping at least SM_MIN_STAGES
// stages of 128 K per wave, and over 32 rows runs each 32-row tile in
// work-groups of its own (half the dependent MFMA/VALU chain per wave; the
// second read of each weight mostly hits the Infinity Cache).  At 64 rows
// this measured fc2 (N 1024, K 4736, Q4_0) 21.3 → 8.4 µs and fc1 (N 4736,
// K 1024) 7.3 → 6.8 µs.
constexpr int SM_WG_GOAL = 128;
constexpr int SM_MIN_STAGES = 1;
constexpr bool SM_ROW_TILES = true;

int sm_kgroups(const Weight &W) {
    const int cgs = sm_wgs(W.N, SM_KS);
    const int nst = (int)((W.Kp + 127) / 128);
    return std::max(1, std::min({SM_WG_GOAL / cgs, nst / (SM_KS * SM_MIN_STAGES), SM_KG_MAX}));
}

// Grow the context's split workspace to hold `parts` partial sums.
hipError_t sk_workspace(s3e_ctx *ctx, int64_t parts) {
    if (parts <= ctx->sk_part_cap) return hipSuccess;
    hipError_t e = hipStreamSynchronize(ctx->stream);  // earlier launches may still read it
    if (e != hipSuccess) return e;
    if (ctx->sk_part) (void)hipFree(ctx->sk_part);
    ctx->sk_part = nullptr;
    ctx->sk_part_cap = 0;
    e = hipMalloc(&ctx->sk_part, (size_t)parts * sizeof(float));
    if (e != hipSuccess) return e;
    ctx->sk_part_cap = parts;
    return hipSuccess;
}

hipError_t run_mul_mat(s3e_ctx *ctx, const s3e_weight *w, const Act &a, int64_t M, const EpiArgs &ea) {
    const Weight &W = w->w;
    hipStream_t st = ctx->stream;
    if (!sm_eligible(W, M)) return launch_gemm(W, a, M, EPI_F32, ea, st);
    const uint8_t *wsm = nullptr;
    hipError_t e = sm_weights(w, st, &wsm);
    if (e != hipSuccess) return e;
    SmArgs sa;
    sa.one = sm_desc(W, wsm, a, ea.bias, ea.y, 0);
    sa.M = (int)M;
    const int cgs = sm_wgs(W.N, SM_KS);
    sa.kg = sm_kgroups(W);
    sa.rt = (SM_ROW_TILES && M > 32) ? 2 : 1;
    // the workspace was sized when the weight was uploaded on this context;
    // a context that has not seen the weight before runs it unsplit rather
    // than allocating inside the call
    if (sa.kg > 1 && (int64_t)sa.kg * M * W.N > ctx->sk_part_cap) sa.kg = 1;
    if (sa.kg > 1) sa.part = ctx->sk_part;
    return launch_gemm_sm(W.kind, sa, cgs * sa.kg * sa.rt, SM_KS, st);
}

// Called once per uploaded weight of a small-M type: the weight's
// block-interleaved copy and room in the context's split workspace for the
// partial sums of its largest small-M product (64 rows).
hipError_t sm_prepare(s3e_ctx *ctx, const s3e_weight *w) {
    const Weight &W = w->w;
    if (!sm_eligible(W, 64)) return hipSuccess;
    const uint8_t *wsm = nullptr;
    hipError_t e = sm_weights(w, ctx->stream, &wsm);
    if (e != hipSuccess) return e;
    const int kg = sm_kgroups(W);
    return kg > 1 ? sk_workspace(ctx, (int64_t)kg * 64 * W.N) : hipSuccess;
}

}  // namespace

extern "C" int s3e_weight_info(const s3e_weight *w, int64_t out[4]) try {
    if (!w || !out) { set_error("s3e_weight_info: NULL argument"); return S3E_ERR_INVALID; }
    out[0] = w->w.ggml_type;
    out[1] = w->w.K;
    out[2] = w->w.N;
    out[3] = (int64_t)w->w.bytes;
    return S3E_OK;
} S3E_CATCH("s3e_weight_info")

extern "C" int s3e_quantize_rows(s3e_ctx *ctx, int type, const float *X, int64_t M, int64_t K, void *qs,
                                 uint16_t *d, uint16_t *s) try {
    if (!ctx || !X || !qs) { set_error("s3e_quantize_rows: NULL argument"); return S3E_ERR_INVALID; }
    if (M < 0) { set_error("s3e_quantize_rows: negative M"); return S3E_ERR_INVALID; }
    if (K % 32 != 0) { set_error("s3e_quantize_rows: K=%lld must be a multiple of 32", (long long)K); return S3E_ERR_INVALID; }
    Act a;
    a.x = qs;
    a.d = d;
    a.s = s;
    a.ld = K;
    a.mp = round_up(M, ROW_PAD);
    if (type == S3E_TYPE_Q8_0) a.kind = A_Q8_0;
    else if (type == S3E_TYPE_Q8_1) a.kind = A_Q8_1;
    else if (type == S3E_TYPE_F16) a.kind = A_F16;
    else if (type == S3E_TYPE_Q8_0_F6X2) a.kind = A_F6;
    else { set_error("s3e_quantize_rows: type %d is not a vec_dot type", type); return S3E_ERR_UNSUPPORTED; }
    if (a.kind == A_F6 && K % 128 != 0) {
        set_error("s3e_quantize_rows: K=%lld must be a multiple of 128 for the fp6 split", (long long)K);
        return S3E_ERR_INVALID;
    }
    if ((a.kind != A_F16 && !d) || (a.kind == A_Q8_1 && !s)) { set_error("s3e_quantize_rows: missing scale buffer"); return S3E_ERR_INVALID; }
    if (M == 0) return S3E_OK;  // an empty batch: nothing to convert
    HIP_TRY(hipSetDevice(ctx->device));
    HIP_TRY(launch_rows_quant(a.kind, X, M, K, a, ctx->stream));
    return S3E_OK;
} S3E_CATCH("s3e_quantize_rows")

extern "C" int s3e_mul_mat(s3e_ctx *ctx, const s3e_weight *w, const float *X, int64_t M, const float *bias,
                           float *Y) try {
    if (!ctx || !w || !X || !Y) { set_error("s3e_mul_mat: NULL argument"); return S3E_ERR_INVALID; }
    if (M < 0) { set_error("s3e_mul_mat: negative M"); return S3E_ERR_INVALID; }
    const Weight &W = w->w;
    if (W.K % 32 != 0) {
        set_error("s3e_mul_mat: K=%lld is not a multiple of 32", (long long)W.K);
        return S3E_ERR_UNSUPPORTED;
    }
    if (M == 0) return S3E_OK;
    HIP_TRY(hipSetDevice(ctx->device));
    const AKind ak = act_kind_for(W.kind);
    EpiArgs ea;
    ea.bias = bias;
    ea.y = Y;
    ea.ldy = W.N;
    if (ak == A_F32) {
        Act a;
        a.kind = A_F32;
        a.x = (void *)X;
        a.ld = W.K;
        HIP_TRY(launch_gemm(W, a, M, EPI_F32, ea, ctx->stream));
        return S3E_OK;
    }
    ActBuf buf;
    HIP_TRY(buf.alloc(std::max<int64_t>(M, 64), W.K, ctx->stream));
    const Act a = buf.as(sm_eligible(W, M) ? ak : act_kind_gemm(W), W.K);
    hipError_t e = launch_rows_quant(a.kind, X, M, W.K, a, ctx->stream);
    if (e == hipSuccess) e = run_mul_mat(ctx, w, a, M, ea);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    buf.release();
    if (e != hipSuccess) { set_error("s3e_mul_mat: %s", hipGetErrorString(e)); return S3E_ERR_HIP; }
    return S3E_OK;
} S3E_CATCH("s3e_mul_mat")

extern "C" int s3e_mul_mat_q_f6(s3e_ctx *ctx, const s3e_weight *w, const void *xq, const uint16_t *d, int64_t M,
                                const float *bias, float *Y) try {
    if (!ctx || !w || !xq || !d || !Y) { set_error("s3e_mul_mat_q_f6: NULL argument"); return S3E_ERR_INVALID; }
    const Weight &W = w->w;
    if (W.kind != WK_Q4_0 || !W.f6) {
        set_error("s3e_mul_mat_q_f6: needs Q4_0 weights with K a multiple of 128");
        return S3E_ERR_UNSUPPORTED;
    }
    if (M < 0) { set_error("s3e_mul_mat_q_f6: negative M"); return S3E_ERR_INVALID; }
    if (M == 0) return S3E_OK;
    HIP_TRY(hipSetDevice(ctx->device));
    Act a;
    a.kind = A_F6;
    a.x = (void *)xq;
    a.d = (uint16_t *)d;
    a.ld = W.K;
    a.mp = round_up(M, ROW_PAD);
    EpiArgs ea;
    ea.bias = bias;
    ea.y = Y;
    ea.ldy = W.N;
    HIP_TRY(launch_gemm(W, a, M, EPI_F32, ea, ctx->stream));
    return S3E_OK;
} S3E_CATCH("s3e_mul_mat_q_f6")

extern "C" int s3e_mul_mat_q(s3e_ctx *ctx, const s3e_weight *w, const void *xq, const uint16_t *d,
                             const uint16_t *s, int64_t M, const float *bias, float *Y) try {
    if (!ctx || !w || !xq || !Y) { set_error("s3e_mul_mat_q: NULL argument"); return S3E_ERR_INVALID; }
    const Weight &W = w->w;
    const AKind ak = act_kind_for(W.kind);
    if ((ak == A_Q8_0 || ak == A_Q8_1) && !d) { set_error("s3e_mul_mat_q: missing scales"); return S3E_ERR_INVALID; }
    if (ak == A_Q8_1 && !s) { set_error("s3e_mul_mat_q: missing block sums"); return S3E_ERR_INVALID; }
    if (W.K % 32 != 0 || M < 0) { set_error("s3e_mul_mat_q: K=%lld must be a multiple of 32", (long long)W.K); return S3E_ERR_UNSUPPORTED; }
    if (M == 0) return S3E_OK;
    HIP_TRY(hipSetDevice(ctx->device));
    Act a;
    a.kind = ak;
    a.x = (void *)xq;
    a.d = (uint16_t *)d;
    a.s = (uint16_t *)s;
    a.ld = W.K;
    a.mp = round_up(M, ROW_PAD);
    EpiArgs ea;
    ea.bias = bias;
    ea.y = Y;
    ea.ldy = W.N;
    HIP_TRY(run_mul_mat(ctx, w, a, M, ea));
    return S3E_OK;
} S3E_CATCH("s3e_mul_mat_q")

extern "C" int s3e_mul_mat_q_batch(s3e_ctx *ctx, int n, const s3e_weight *const *w, const void *const *xq,
                                   const uint16_t *const *d, const uint16_t *const *s, int64_t M,
                                   const float *const *bias, float *const *Y) try {
    if (!ctx || n <= 0 || !w || !xq || !Y) { set_error("s3e_mul_mat_q_batch: NULL argument or n <= 0"); return S3E_ERR_INVALID; }
    if (M < 1 || M > 64) { set_error("s3e_mul_mat_q_batch: M=%lld is outside 1..64", (long long)M); return S3E_ERR_UNSUPPORTED; }
    const WKind kind = w[0] ? w[0]->w.kind : WK_F32;
    std::vector<SmGemm> g((size_t)n);
    // batches: four strips per work-group, activations shared through LDS
    const int ks = 1;
    int wgs = 0;
    HIP_TRY(hipSetDevice(ctx->device));
    for (int i = 0; i < n; i++) {
        if (!w[i] || !xq[i] || !Y[i]) { set_error("s3e_mul_mat_q_batch: NULL entry %d", i); return S3E_ERR_INVALID; }
        const Weight &W = w[i]->w;
        if (W.kind != kind || !sm_eligible(W, M)) {
            set_error("s3e_mul_mat_q_batch: product %d: all weights must share one of Q4_0/Q4_1/Q8_0/F16", i);
            return S3E_ERR_UNSUPPORTED;
        }
        const AKind ak = act_kind_for(W.kind);
        if ((ak == A_Q8_0 || ak == A_Q8_1) && (!d || !d[i])) { set_error("s3e_mul_mat_q_batch: missing scales of %d", i); return S3E_ERR_INVALID; }
        if (ak == A_Q8_1 && (!s || !s[i])) { set_error("s3e_mul_mat_q_batch: missing block sums of %d", i); return S3E_ERR_INVALID; }
        const uint8_t *wsm = nullptr;
        HIP_TRY(sm_weights(w[i], ctx->stream, &wsm));
        Act a;
        a.kind = ak;
        a.x = (void *)xq[i];
        a.d = d ? (uint16_t *)d[i] : nullptr;
        a.s = s ? (uint16_t *)s[i] : nullptr;
        a.ld = W.K;
        a.mp = round_up(M, ROW_PAD);
        g[(size_t)i] = sm_desc(W, wsm, a, bias ? bias[i] : nullptr, Y[i], wgs);
        wgs += sm_wgs(W.N, ks);
        if (n > 65535 || wgs > (1 << 30)) { set_error("s3e_mul_mat_q_batch: batch too large"); return S3E_ERR_UNSUPPORTED; }
    }
    // descriptors, then the product index of every work-group
    const size_t desc_bytes = sizeof(SmGemm) * (size_t)n;
    std::vector<uint8_t> blob(desc_bytes + sizeof(uint16_t) * (size_t)wgs);
    std::memcpy(blob.data(), g.data(), desc_bytes);
    uint16_t *tab = (uint16_t *)(blob.data() + desc_bytes);
    for (int i = 0; i < n; i++) {
        const int end = i + 1 < n ? g[(size_t)i + 1].wg0 : wgs;
        for (int b = g[(size_t)i].wg0; b < end; b++) tab[b] = (uint16_t)i;
    }
    // the descriptors go to the device once per distinct batch, after every
    // launch that still reads the previous ones
    if (ctx->sm_last != blob) {
        HIP_TRY(hipStreamSynchronize(ctx->stream));
        ctx->sm_last.clear();
        if (blob.size() > ctx->sm_cap) {
            if (ctx->sm_dev) (void)hipFree(ctx->sm_dev);
            ctx->sm_dev = nullptr;
            ctx->sm_cap = 0;
            HIP_TRY(hipMalloc(&ctx->sm_dev, blob.size()));
            ctx->sm_cap = blob.size();
        }
        HIP_TRY(hipMemcpy(ctx->sm_dev, blob.data(), blob.size(), hipMemcpyHostToDevice));
        ctx->sm_last = blob;
    }
    SmArgs sa;
    sa.many = (const SmGemm *)ctx->sm_dev;
    sa.wg_gemm = (const uint16_t *)((const uint8_t *)ctx->sm_dev + desc_bytes);
    sa.n = n;
    sa.M = (int)M;
    HIP_TRY(launch_gemm_smb(kind, sa, wgs, ctx->stream));
    return S3E_OK;
} S3E_CATCH("s3e_mul_mat_q_batch")

extern "C" int s3e_layer_norm(s3e_ctx *ctx, const float *x, int64_t rows, int64_t n, float eps, const float *w,
                              const float *b, float *y) try {
    if (!ctx || !x || !y) { set_error("s3e_layer_norm: NULL argument"); return S3E_ERR_INVALID; }
    if (rows < 0 || n <= 0 || n % 32 != 0 || n > 4096) {
        set_error("s3e_layer_norm: row length %lld must be a positive multiple of 32 up to 4096", (long long)n);
        return S3E_ERR_UNSUPPORTED;
    }
    if (rows == 0) return S3E_OK;
    HIP_TRY(hipSetDevice(ctx->device));
    Act none;
    HIP_TRY(launch_layernorm(x, rows, n, eps, w, b, none, y, ctx->stream));
    return S3E_OK;
} S3E_CATCH("s3e_layer_norm")

// ---- ggml_flash_attn_ext --------------------------------------------------
extern "C" int s3e_flash_attn_ext(s3e_ctx *ctx, const float *q, const int64_t q_nb[4], const float *k,
                                  const int64_t k_nb[4], const float *v, const int64_t v_nb[4], int64_t D,
                                  int64_t Nq, int64_t Nkv, int64_t nh, int64_t B, float scale, int prec,
                                  float *o) try {
    if (!ctx || !q || !k || !v || !o || !q_nb || !k_nb || !v_nb) {
        set_error("s3e_flash_attn_ext: NULL argument");
        return S3E_ERR_INVALID;
    }
    if (Nq <= 0 || Nkv <= 0 || nh <= 0 || B <= 0 || D <= 0) { set_error("s3e_flash_attn_ext: empty shape"); return S3E_ERR_INVALID; }
    if (prec != S3E_PREC_DEFAULT && prec != S3E_PREC_F32) { set_error("s3e_flash_attn_ext: unknown precision %d", prec); return S3E_ERR_INVALID; }
    // head dims up to 128 run zero-padded to 64 or 128 channels (ViT 64; Hiera 96, 56, 32, 72); 256 (memory
    // attention) runs as is, on fp16 operands only
    const int hdp = D <= 64 ? 64 : (D <= 128 ? 128 : 256);
    if (D % 4 != 0 || (D > 128 && D != 256)) {
        set_error("s3e_flash_attn_ext: head dim %lld not supported (multiples of 4 up to 128, or 256)", (long long)D);
        return S3E_ERR_UNSUPPORTED;
    }
    if (D == 256 && prec == S3E_PREC_F32) {
        set_error("s3e_flash_attn_ext: head dim 256 runs on fp16 operands only (S3E_PREC_DEFAULT)");
        return S3E_ERR_UNSUPPORTED;
    }
    if (B * nh > 65535 || Nq > (1 << 24) || Nkv > (1 << 24)) { set_error("s3e_flash_attn_ext: shape too large"); return S3E_ERR_INVALID; }
    HIP_TRY(hipSetDevice(ctx->device));
    const int64_t ldv = vt_ld_for(Nkv);
    const int np = (prec == S3E_PREC_F32) ? 2 : 1;  // hi (+ lo) planes
    const size_t qn = (size_t)(B * nh * Nq * hdp), kn = (size_t)(B * nh * Nkv * hdp), vn = (size_t)(B * nh * ldv * hdp);
    // split the keys when the query tiles alone leave the chip idle (plain layouts only)
    const int64_t BH = B * nh, qtiles = (Nq + 127) / 128, ktiles = (Nkv + 31) / 32;
    int nsplit = 1;
    // about one round of work-groups: 512 (two or three fit a CU), 256 at head dim 256 (one fits)
    const int64_t target = hdp == 256 ? 256 : 512;
    if (D == hdp && qtiles * BH < target) {
        int64_t ns = std::min<int64_t>((target + qtiles * BH - 1) / (qtiles * BH), std::max<int64_t>(1, ktiles / 4));
        const int64_t per = (ktiles + ns - 1) / ns;
        nsplit = (int)((ktiles + per - 1) / per);
    }
    _Float16 *q16 = nullptr, *k16 = nullptr, *vt16 = nullptr;
    float *part = nullptr;
    hipError_t e = hipMalloc(&q16, qn * 2 * np);
    if (e == hipSuccess) e = hipMalloc(&k16, kn * 2 * np);
    if (e == hipSuccess) e = hipMalloc(&vt16, vn * 2 * np);
    if (e == hipSuccess) e = hipMemsetAsync(vt16, 0, vn * 2 * np, ctx->stream);
    const size_t po = (size_t)nsplit * BH * Nq * hdp, pml = (size_t)nsplit * BH * Nq * 2;
    if (e == hipSuccess && nsplit > 1) e = hipMalloc(&part, (po + pml) * 4);
    AttnArgs a;
    a.q = q16;
    a.k = k16;
    a.vt = vt16;
    if (np == 2) {
        a.q_lo = q16 + qn;
        a.k_lo = k16 + kn;
        a.vt_lo = vt16 + vn;
    }
    if (e == hipSuccess)
        e = launch_attn_prep(q, q_nb, k, k_nb, v, v_nb, Nq, Nkv, nh, B, (int)D, hdp, q16, k16, vt16,
                             (_Float16 *)a.q_lo, (_Float16 *)a.k_lo, (_Float16 *)a.vt_lo, ldv, ctx->stream);
    if (e == hipSuccess) {
        a.Nq = (int)Nq;
        a.Nkv = (int)Nkv;
        a.NH = (int)nh;
        a.BH = (int)BH;
        a.hd = hdp;
        a.hd_out = D == hdp ? 0 : (int)D;
        a.scale = scale;
        a.grid = 0;
        a.nsplit = nsplit;
        if (nsplit > 1) {
            a.part_o = part;
            a.part_ml = part + po;
        }
        a.out.kind = A_F32;
        a.out.x = o;
        a.out.ld = nh * D;
        e = launch_attn(a, ctx->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (q16) (void)hipFree(q16);
    if (k16) (void)hipFree(k16);
    if (vt16) (void)hipFree(vt16);
    if (part) (void)hipFree(part);
    if (e != hipSuccess) { set_error("s3e_flash_attn_ext: %s", hipGetErrorString(e)); return S3E_ERR_HIP; }
    return S3E_OK;
} S3E_CATCH("s3e_flash_attn_ext")

extern "C" int s3e_flash_attn_ext_f16(s3e_ctx *ctx, const uint16_t *q, const int64_t q_nb[4], const uint16_t *k,
                                      const int64_t k_nb[4], const uint16_t *v, const int64_t v_nb[4], int64_t D,
                                      int64_t Nq, int64_t Nkv, int64_t nh, int64_t B, float scale, float *o) try {
    if (!ctx || !q || !k || !v || !o || !q_nb || !k_nb || !v_nb) {
        set_error("s3e_flash_attn_ext_f16: NULL argument");
        return S3E_ERR_INVALID;
    }
    if (Nq <= 0 || Nkv <= 0 || nh <= 0 || B <= 0 || D <= 0) { set_error("s3e_flash_attn_ext_f16: empty shape"); return S3E_ERR_INVALID; }
    if (D % 4 != 0 || (D > 128 && D != 256)) {
        set_error("s3e_flash_attn_ext_f16: head dim %lld not supported (multiples of 4 up to 128, or 256)", (long long)D);
        return S3E_ERR_UNSUPPORTED;
    }
    if (B * nh > 65535 || Nq > (1 << 24) || Nkv > (1 << 24)) { set_error("s3e_flash_attn_ext_f16: shape too large"); return S3E_ERR_INVALID; }
    for (int i = 1; i < 4; i++)
        if (q_nb[i] < 0 || k_nb[i] < 0 || v_nb[i] < 0) { set_error("s3e_flash_attn_ext_f16: negative stride"); return S3E_ERR_INVALID; }
    if (q_nb[0] != 1 || k_nb[0] != 1 || v_nb[0] != 1) {
        set_error("s3e_flash_attn_ext_f16: the head dimension must be contiguous (nb[0] = 1)");
        return S3E_ERR_INVALID;
    }
    HIP_TRY(hipSetDevice(ctx->device));
    const int hdp = D <= 64 ? 64 : (D <= 128 ? 128 : 256);
    const int64_t ldv = vt_ld_for(Nkv);
    const int64_t BH = B * nh, qtiles = (Nq + 127) / 128, ktiles = (Nkv + 31) / 32;
    // Q and K are read where they lie when they already are [B][nh][N][hdp]
    auto plain = [&](const int64_t nb[4], int64_t N) {
        return D == hdp && nb[1] == hdp && nb[2] == N * hdp && nb[3] == nh * N * hdp;
    };
    const bool q_in = plain(q_nb, Nq), k_in = plain(k_nb, Nkv);
    // V: read where it lies as well (head dims up to 128), else copied to the
    // plain layout; head dim 256 goes through the Vᵀ layout
    const bool vnat = hdp <= 128, v_in = vnat && plain(v_nb, Nkv);
    int nsplit = 1;
    const int64_t target = hdp == 256 ? 256 : 512;
    if (D == hdp && qtiles * BH < target) {
        const int64_t ns = std::min<int64_t>((target + qtiles * BH - 1) / (qtiles * BH), std::max<int64_t>(1, ktiles / 4));
        const int64_t per = (ktiles + ns - 1) / ns;
        nsplit = (int)((ktiles + per - 1) / per);
    }
    // workspace: [V copy or Vᵀ][Q copy][K copy][partials], 256-byte aligned pieces
    auto al = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t vb = vnat ? (v_in ? 0 : al((size_t)(BH * Nkv * hdp) * 2)) : al((size_t)(BH * hdp * ldv) * 2), qb = q_in ? 0 : al((size_t)(BH * Nq * hdp) * 2),
                 kb = k_in ? 0 : al((size_t)(BH * Nkv * hdp) * 2);
    const size_t po = (size_t)nsplit * BH * Nq * hdp, pml = (size_t)nsplit * BH * Nq * 2;
    const size_t pb = nsplit > 1 ? (po + pml) * 4 : 0;
    const size_t need = vb + qb + kb + pb;
    if (need > ctx->attn_ws_cap) {
        HIP_TRY(hipStreamSynchronize(ctx->stream));  // earlier calls may still read it
        if (ctx->attn_ws) (void)hipFree(ctx->attn_ws);
        ctx->attn_ws = nullptr;
        ctx->attn_ws_cap = 0;
        HIP_TRY(hipMalloc(&ctx->attn_ws, need));
        ctx->attn_ws_cap = need;
    }
    uint8_t *ws = (uint8_t *)ctx->attn_ws;
    _Float16 *vt16 = vnat ? nullptr : (_Float16 *)ws;
    _Float16 *v16 = (vnat && !v_in) ? (_Float16 *)ws : nullptr;
    _Float16 *q16 = q_in ? nullptr : (_Float16 *)(ws + vb);
    _Float16 *k16 = k_in ? nullptr : (_Float16 *)(ws + vb + qb);
    hipError_t e = hipSuccess;
    if (!q_in || !k_in || !v_in)
        e = launch_attn_prep16((const _Float16 *)q, q_nb, (const _Float16 *)k, k_nb, (const _Float16 *)v, v_nb, Nq,
                               Nkv, nh, B, (int)D, hdp, q16, k16, v16, vt16, ldv, ctx->stream);
    if (e == hipSuccess) {
        AttnArgs a;
        a.q = q_in ? (const _Float16 *)q : q16;
        a.k = k_in ? (const _Float16 *)k : k16;
        if (vnat) a.v = v_in ? (const _Float16 *)v : v16;
        else a.vt = vt16;
        a.Nq = (int)Nq;
        a.Nkv = (int)Nkv;
        a.NH = (int)nh;
        a.BH = (int)BH;
        a.hd = hdp;
        a.hd_out = D == hdp ? 0 : (int)D;
        a.scale = scale;
        a.nsplit = nsplit;
        if (nsplit > 1) {
            a.part_o = (float *)(ws + vb + qb + kb);
            a.part_ml = a.part_o + po;
        }
        a.out.kind = A_F32;
        a.out.x = o;
        a.out.ld = nh * D;
        e = launch_attn(a, ctx->stream);
    }
    if (e != hipSuccess) { set_error("s3e_flash_attn_ext_f16: %s", hipGetErrorString(e)); return S3E_ERR_HIP; }
    return S3E_OK;
} S3E_CATCH("s3e_flash_attn_ext_f16")

// ---- measurement ---------------------------------------------------------
namespace {

// The measurement kernels' sink (one word per thread or per wave), grown on
// the first calls.
hipError_t probe_setup(s3e_ctx *ctx, int64_t words) {
    if (words <= ctx->probe_sink_cap) return hipSuccess;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return e;
    if (ctx->probe_sink) (void)hipFree(ctx->probe_sink);
    ctx->probe_sink = nullptr;
    ctx->probe_sink_cap = 0;
    e = hipMalloc(&ctx->probe_sink, (size_t)words * 4);
    if (e == hipSuccess) ctx->probe_sink_cap = words;
    return e;
}

}  // namespace

extern "C" int s3e_probe_stream(s3e_ctx *ctx, int mode, void *dst, const void *src, size_t bytes) try {
    if (!ctx || (mode != 0 && !dst) || (mode != 2 && !src)) { set_error("s3e_probe_stream: NULL argument"); return S3E_ERR_INVALID; }
    if (mode < 0 || mode > 2 || bytes == 0 || bytes % 16 != 0) {
        set_error("s3e_probe_stream: mode %d / %zu bytes (modes 0-2, a multiple of 16 bytes)", mode, bytes);
        return S3E_ERR_INVALID;
    }
    HIP_TRY(hipSetDevice(ctx->device));
    int cus = 0;
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device));
    const int blocks = 8 * cus;  // 8 work-groups of 4 waves per CU
    hipError_t e = probe_setup(ctx, (int64_t)blocks * 256);
    if (e == hipSuccess) e = launch_probe_stream(mode, dst, src, bytes, ctx->probe_sink, blocks, ctx->stream);
    if (e != hipSuccess) { set_error("s3e_probe_stream: %s", hipGetErrorString(e)); return S3E_ERR_HIP; }
    return S3E_OK;
} S3E_CATCH("s3e_probe_stream")

extern "C" int s3e_probe_mfma(s3e_ctx *ctx, int kind, int64_t iters, int waves_per_simd) try {
    if (!ctx) { set_error("s3e_probe_mfma: NULL context"); return S3E_ERR_INVALID; }
    if (kind < 0 || kind > 3 || iters <= 0 || iters > (1 << 24) || waves_per_simd < 1 || waves_per_simd > 4) {
        set_error("s3e_probe_mfma: kind %d (0-3), %lld steps, %d waves per SIMD (1-4)", kind, (long long)iters,
                  waves_per_simd);
        return S3E_ERR_INVALID;
    }
    HIP_TRY(hipSetDevice(ctx->device));
    int cus = 0;
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device));
    const int blocks = cus * waves_per_simd;  // 4 waves (one per SIMD) per work-group
    hipError_t e = probe_setup(ctx, (int64_t)blocks * 4);
    if (e == hipSuccess) e = launch_probe_mfma(kind, iters, blocks, ctx->probe_sink, ctx->stream);
    if (e != hipSuccess) { set_error("s3e_probe_mfma: %s", hipGetErrorString(e)); return S3E_ERR_HIP; }
    return S3E_OK;
} S3E_CATCH("s3e_probe_mfma")

// ---- SAM 3 ViT model -------------------------------------------------------
namespace {

struct Block {
    float *n1w = nullptr, *n1b = nullptr, *n2w = nullptr, *n2b = nullptr;
    float *qkv_b = nullptr, *proj_b = nullptr, *fc1_b = nullptr, *fc2_b = nullptr;
    float *freqs = nullptr;  // [Nw][HD/2][2] or null
    int64_t freqs_n = 0;
    Weight qkv, proj, fc1, fc2;
    bool global = false;
};

// One level of a SimpleFPN neck (sam3.cpp:2562-2591).  dc[0], dc[1]: the
// 2×2 stride-2 deconvolutions (scale 0 has two, scale 1 one) as fp16 GEMM
// weights N = 4·Cout, K = Cin with column (2·ky + kx)·Cout + co; c1: the 1×1
// conv, c3: the 3×3 conv with K ordered [ky][kx][Cin]; both fp16 in F16
// files, split fp16 (WK_F16X3) otherwise.
struct NeckScale {
    Weight dc[2], c1, c3;
    float *dc_b[2] = {nullptr, nullptr}, *c1_b = nullptr, *c3_b = nullptr;
    int64_t dc_b_n[2] = {0, 0}, c1_b_n = 0, c3_b_n = 0;
    // scale 0 of files with F32 convs: the 1×1 folded into the 3×3 (c3f,
    // weights W3·W1 per tap; c3f_b: 9 bias rows by border class), and the
    // host f32 records it is computed from until the neck is complete
    Weight c3f;
    float *c3f_b = nullptr;
    std::vector<float> h_c1, h_c1_b, h_c3, h_c3_b;
};

struct Neck {
    NeckScale s[4];
    int found = 0;  // tensors read
};

}  // namespace

struct s3e_model {
    s3e_ctx *ctx = nullptr;
    int ftype = 0, wtype = 0;
    int32_t img = 0, patch = 0, E = 0, depth = 0, heads = 0, mlp = 0, window = 0, n_global = 0, gidx[4] = {0, 0, 0, 0};
    int grid = 0, pos_grid = 0;
    Weight patch_w;  // K = 3·P², N = E
    // an F32 patch kernel again as split fp16 pairs (K padded like patch_w),
    // the form the encoder's patch GEMM runs; patch_w serves the readers
    Weight patch_split;
    float *pos = nullptr, *ln_pre_w = nullptr, *ln_pre_b = nullptr;
    std::vector<Block> blocks;
    Neck necks[2];              // 0 = "neck.det.", 1 = "neck.trk."
    int necks_present = 0;      // bit 0 trk, bit 1 det
    int32_t neck_dim = 0, visual_only = 1;
    std::vector<void *> owned;  // device f32 arrays
    HieraModel *hiera = nullptr;  // SAM 2.x files: the Hiera encoder instead of the ViT
    MemAttnModel *ma = nullptr;   // the tracker's memory attention, when the file has it
};

namespace {

int ftype_wtype(int ftype) {
    switch (ftype) {
        case 0: return 0;
        case 1: return 1;
        case 2: return 2;
        case 3: return 3;
        case 8: return 8;
        default: return -1;
    }
}

int upload_f32(s3e_model *m, const RawTensor &t, int64_t expect, float **dst) {
    int64_t n = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
    if (n != expect) { set_error("tensor has %lld elements, expected %lld", (long long)n, (long long)expect); return S3E_ERR_IO; }
    void *p = nullptr;
    HIP_TRY(hipMalloc(&p, (size_t)n * 4));
    m->owned.push_back(p);
    HIP_TRY(hipMemcpy(p, t.data.data(), (size_t)n * 4, hipMemcpyHostToDevice));
    *dst = (float *)p;
    return S3E_OK;
}

}  // namespace

namespace {

// One "neck.{det,trk}.<scale>.<layer>.{weight,bias}" record, already in its
// registered type (F32, or F16 in F16 files).  Shapes are checked across the
// neck once every record is in (check_neck).
int load_neck_tensor(s3e_model *m, const std::string &name, const RawTensor &t) {
    const int which = name.compare(0, 9, "neck.det.") == 0 ? 0 : 1;
    Neck &nk = m->necks[which];
    if (name.size() < 12 || name[9] < '0' || name[9] > '3' || name[10] != '.') return S3E_OK;  // not ours
    NeckScale &sc = nk.s[name[9] - '0'];
    const std::string f = name.substr(11);
    const int64_t n_el = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
    int rc = S3E_OK;
    auto bias = [&](float **dst, int64_t *len) {
        if (t.n_dims != 1) { set_error("'%s': expected a 1-D bias", name.c_str()); return (int)S3E_ERR_IO; }
        *len = t.ne[0];
        return upload_f32(m, t, t.ne[0], dst);
    };
    const bool scale0 = name[9] == '0';
    auto keep = [&](std::vector<float> &h) {  // scale-0 f32 record for the 1×1 → 3×3 fold
        if (scale0 && t.type == 0) {
            const float *src = (const float *)t.data.data();
            h.assign(src, src + n_el);
        }
    };
    if (f == "dconv_2x2_0.bias" || f == "dconv_2x2.bias") rc = bias(&sc.dc_b[0], &sc.dc_b_n[0]);
    else if (f == "dconv_2x2_1.bias") rc = bias(&sc.dc_b[1], &sc.dc_b_n[1]);
    else if (f == "conv_1x1.bias") { rc = bias(&sc.c1_b, &sc.c1_b_n); keep(sc.h_c1_b); }
    else if (f == "conv_3x3.bias") { rc = bias(&sc.c3_b, &sc.c3_b_n); keep(sc.h_c3_b); }
    else if (f == "dconv_2x2_0.weight" || f == "dconv_2x2.weight" || f == "dconv_2x2_1.weight") {
        // ggml [kW=2, kH=2, Cout, Cin]: element (kx, ky, co, ci) at ((ci·Cout + co)·2 + ky)·2 + kx;
        // cast to fp16 as sam3_conv_transpose_weight does (sam3.cpp:1083-1086)
        if (t.ne[0] != 2 || t.ne[1] != 2) { set_error("'%s': expected a 2x2 kernel", name.c_str()); return S3E_ERR_IO; }
        const int64_t Cout = t.ne[2], Cin = t.ne[3];
        std::vector<uint16_t> w((size_t)(4 * Cout * Cin));
        for (int64_t ci = 0; ci < Cin; ci++)
            for (int64_t co = 0; co < Cout; co++)
                for (int q = 0; q < 4; q++) {
                    const int64_t src = (ci * Cout + co) * 4 + q;  // q = 2·ky + kx
                    uint16_t h;
                    if (t.type == 1) std::memcpy(&h, t.data.data() + 2 * src, 2);
                    else h = host_f2h(((const float *)t.data.data())[src]);
                    w[(size_t)((q * Cout + co) * Cin + ci)] = h;
                }
        Weight &dst = sc.dc[f == "dconv_2x2_1.weight" ? 1 : 0];
        rc = upload_weight(m->ctx->device, S3E_TYPE_F16, Cin, 4 * Cout, (const uint8_t *)w.data(), w.size() * 2, dst,
                           CONV_BN);
    } else if (f == "conv_1x1.weight" || f == "conv_3x3.weight") {
        // ggml [kW, kH, Cin, Cout]: element (kx, ky, ci, co) at ((co·Cin + ci)·kH + ky)·kW + kx;
        // the GEMM's K order is [ky][kx][Cin] so that one stage stays inside one tap
        const int64_t k = (f == "conv_1x1.weight") ? 1 : 3;
        if (t.ne[0] != k || t.ne[1] != k) { set_error("'%s': expected a %lldx%lld kernel", name.c_str(), (long long)k, (long long)k); return S3E_ERR_IO; }
        const int64_t Cin = t.ne[2], Cout = t.ne[3], K = k * k * Cin;
        Weight &dst = (k == 1) ? sc.c1 : sc.c3;
        std::vector<float> wf((size_t)(K * Cout));
        std::vector<uint16_t> wh(t.type == 1 ? (size_t)(K * Cout) : 0);
        for (int64_t co = 0; co < Cout; co++)
            for (int64_t ci = 0; ci < Cin; ci++)
                for (int64_t ky = 0; ky < k; ky++)
                    for (int64_t kx = 0; kx < k; kx++) {
                        const int64_t src = ((co * Cin + ci) * k + ky) * k + kx;
                        const size_t d = (size_t)(co * K + (ky * k + kx) * Cin + ci);
                        if (t.type == 1) std::memcpy(&wh[d], t.data.data() + 2 * src, 2);
                        else wf[d] = ((const float *)t.data.data())[src];
                    }
        if (t.type == 1)
            rc = upload_weight(m->ctx->device, S3E_TYPE_F16, K, Cout, (const uint8_t *)wh.data(), wh.size() * 2, dst,
                               CONV_BN);
        else
            rc = upload_weight_split(wf.data(), K, Cout, dst, CONV_BN);
        if (rc == S3E_OK && scale0 && t.type == 0) (k == 1 ? sc.h_c1 : sc.h_c3) = std::move(wf);
    } else {
        return S3E_OK;
    }
    (void)n_el;
    if (rc == S3E_OK) nk.found++;
    return rc;
}

// Shapes of a complete neck: the graph of sam3.cpp:3863-3921 on E channels.
int check_neck(const s3e_model *m, int which) {
    const Neck &nk = m->necks[which];
    const char *nm = which == 0 ? "neck.det" : "neck.trk";
    if (nk.found != 22) { set_error("%s: found %d of 22 tensors", nm, nk.found); return S3E_ERR_IO; }
    const int64_t E = m->E;
    const NeckScale &s0 = nk.s[0], &s1 = nk.s[1], &s2 = nk.s[2], &s3 = nk.s[3];
    const int64_t mid0 = s0.dc[0].N / 4, D = s0.dc[1].N / 4, mid1 = s1.dc[0].N / 4;
    bool ok = s0.dc[0].K == E && s0.dc[1].K == mid0 && s1.dc[0].K == E && s0.dc_b_n[0] == mid0 &&
              s0.dc_b_n[1] == D && s1.dc_b_n[0] == mid1 && s0.c1.K == D && s1.c1.K == mid1 && s2.c1.K == E &&
              s3.c1.K == E;
    for (int i = 0; i < 4; i++) {
        const NeckScale &sc = nk.s[i];
        ok = ok && sc.c1.N == D && sc.c3.N == D && sc.c3.K == 9 * D && sc.c1_b_n == D && sc.c3_b_n == D &&
             sc.c1.q && sc.c3.q && sc.c1_b && sc.c3_b;
    }
    if (!ok) { set_error("%s: tensor shapes do not form the SimpleFPN graph", nm); return S3E_ERR_IO; }
    // fp16 GEMM rows are read 64 channels per stage; the 3×3 needs whole stages per tap
    if (D % 64 != 0 || mid0 % 64 != 0 || mid1 % 64 != 0) {
        set_error("%s: channel counts (%lld, %lld, %lld) must be multiples of 64", nm, (long long)D, (long long)mid0, (long long)mid1);
        return S3E_ERR_UNSUPPORTED;
    }
    if (D != m->neck_dim) { set_error("%s: width %lld differs from neck_dim %d", nm, (long long)D, m->neck_dim); return S3E_ERR_IO; }
    return S3E_OK;
}

// Scale 0 of a neck with F32 convs: its 1×1 (W1 [D][D], b1) feeds the 3×3
// (W3 [D][9][D], b3) with nothing between them (sam3.cpp:3863-3921), so
//     3×3(pad(1×1(y))) = Σ_taps y_shifted·(W3_tap·W1) + b3 + Σ_{taps inside} W3_tap·b1:
// one 3×3 with weights W3_tap·W1 over the deconvolution's output, whose bias
// depends only on which taps fall outside the image (zero padding), i.e. on
// the pixel's border class (first / inner / last row × column).  Products
// and sums in double, rounded once to f32 and split to fp16 pairs as any F32
// conv weight; the 1×1 pass over 16·G² pixels disappears.
int fold_neck0(s3e_model *m, int which) {
    NeckScale &sc = m->necks[which].s[0];
    const int64_t D = sc.c1.N;
    if (sc.h_c1.size() != (size_t)(D * D) || sc.h_c1_b.size() != (size_t)D || sc.h_c3.size() != (size_t)(9 * D * D) ||
        sc.h_c3_b.size() != (size_t)D)
        return S3E_OK;  // F16 convs: the reference rounds the 1×1 output to fp16 first; keep both passes
    std::vector<float> wf((size_t)(9 * D * D));
    std::vector<double> acc((size_t)D), bt((size_t)(9 * D));
    for (int64_t co = 0; co < D; co++)
        for (int tap = 0; tap < 9; tap++) {
            std::fill(acc.begin(), acc.end(), 0.0);
            const float *w3 = sc.h_c3.data() + (size_t)(co * 9 * D + tap * D);
            double b = 0.0;
            for (int64_t c = 0; c < D; c++) {
                const double w = w3[c];
                const float *w1 = sc.h_c1.data() + (size_t)(c * D);
                for (int64_t ci = 0; ci < D; ci++) acc[(size_t)ci] += w * (double)w1[ci];
                b += w * (double)sc.h_c1_b[(size_t)c];
            }
            for (int64_t ci = 0; ci < D; ci++) wf[(size_t)(co * 9 * D + tap * D + ci)] = (float)acc[(size_t)ci];
            bt[(size_t)(tap * D + co)] = b;
        }
    std::vector<float> b9((size_t)(9 * D));
    for (int cy = 0; cy < 3; cy++)
        for (int cx = 0; cx < 3; cx++)
            for (int64_t co = 0; co < D; co++) {
                double b = sc.h_c3_b[(size_t)co];
                for (int ky = 0; ky < 3; ky++)
                    for (int kx = 0; kx < 3; kx++) {
                        const bool out = (cy == 0 && ky == 0) || (cy == 2 && ky == 2) || (cx == 0 && kx == 0) ||
                                         (cx == 2 && kx == 2);
                        if (!out) b += bt[(size_t)((ky * 3 + kx) * D + co)];
                    }
                b9[(size_t)((cy * 3 + cx) * D + co)] = (float)b;
            }
    int rc = upload_weight_split(wf.data(), 9 * D, D, sc.c3f, CONV_BN);
    if (rc != S3E_OK) return rc;
    void *p = nullptr;
    HIP_TRY(hipMalloc(&p, b9.size() * 4));
    m->owned.push_back(p);
    HIP_TRY(hipMemcpy(p, b9.data(), b9.size() * 4, hipMemcpyHostToDevice));
    sc.c3f_b = (float *)p;
    std::vector<float>().swap(sc.h_c1);
    std::vector<float>().swap(sc.h_c1_b);
    std::vector<float>().swap(sc.h_c3);
    std::vector<float>().swap(sc.h_c3_b);
    return S3E_OK;
}

}  // namespace

extern "C" void s3e_model_free(s3e_model *m) {
    if (!m) return;
    if (m->hiera) hiera_free(m->hiera);
    if (m->ma) memattn_free(m->ma);
    free_weight(m->patch_w);
    free_weight(m->patch_split);
    for (auto &nk : m->necks)
        for (auto &sc : nk.s) {
            free_weight(sc.dc[0]);
            free_weight(sc.dc[1]);
            free_weight(sc.c1);
            free_weight(sc.c3);
            free_weight(sc.c3f);
        }
    for (auto &b : m->blocks) {
        free_weight(b.qkv);
        free_weight(b.proj);
        free_weight(b.fc1);
        free_weight(b.fc2);
    }
    for (void *p : m->owned) (void)hipFree(p);
    delete m;
}

extern "C" int s3e_model_load(s3e_ctx *ctx, const char *path, s3e_model **out) try {
    if (!ctx || !path || !out) { set_error("s3e_model_load: NULL argument"); return S3E_ERR_INVALID; }
    *out = nullptr;
    HIP_TRY(hipSetDevice(ctx->device));
    std::ifstream fin(path, std::ios::binary);
    if (!fin) { set_error("s3e_model_load: cannot open '%s'", path); return S3E_ERR_IO; }
    auto rd = [&](void *dst, size_t n) { fin.read((char *)dst, (std::streamsize)n); return (bool)fin; };
    uint32_t magic = 0;
    int32_t version = 0, ftype = 0, n_tensors = 0;
    if (!rd(&magic, 4) || !rd(&version, 4) || !rd(&ftype, 4) || !rd(&n_tensors, 4)) {
        set_error("s3e_model_load: truncated header");
        return S3E_ERR_IO;
    }
    if (magic == 0x73616D32u) {  // "sam2": Hiera backbone + FPN (sam3.cpp:3224-3231)
        if (version != 1) { set_error("s3e_model_load: unsupported SAM2 version %d", version); return S3E_ERR_IO; }
        std::unique_ptr<s3e_model, void (*)(s3e_model *)> m2(new s3e_model, s3e_model_free);
        m2->ctx = ctx;
        m2->ftype = ftype;
        int rc = hiera_load(ctx->device, fin, ftype, n_tensors, &m2->hiera, &m2->ma);
        if (rc == S3E_OK) rc = memattn_finish(m2->ma);
        if (rc != S3E_OK) return rc;
        m2->img = hiera_img_size(m2->hiera);
        m2->necks_present = 1;
        *out = m2.release();
        return S3E_OK;
    }
    if (magic != 0x73616D33u) { set_error("s3e_model_load: unknown magic 0x%08x (expected sam3 or sam2)", magic); return S3E_ERR_IO; }
    if (version != 3) { set_error("s3e_model_load: unsupported SAM3 version %d", version); return S3E_ERR_IO; }
    const int wtype = ftype_wtype(ftype);
    if (wtype < 0) { set_error("s3e_model_load: unsupported ftype %d", ftype); return S3E_ERR_UNSUPPORTED; }
    std::unique_ptr<s3e_model, void (*)(s3e_model *)> m(new s3e_model, s3e_model_free);
    m->ctx = ctx;
    m->ftype = ftype;
    m->wtype = wtype;
    int32_t hv[8];
    if (!rd(hv, 32)) { set_error("s3e_model_load: truncated hparams"); return S3E_ERR_IO; }
    m->img = hv[0]; m->patch = hv[1]; m->E = hv[2]; m->depth = hv[3]; m->heads = hv[4];
    m->mlp = (int32_t)(hv[2] * (hv[5] / 1000.0f));
    m->window = hv[6];
    m->n_global = hv[7];
    for (int i = 0; i < m->n_global && i < 4; i++)
        if (!rd(&m->gidx[i], 4)) { set_error("s3e_model_load: truncated hparams"); return S3E_ERR_IO; }
    int32_t rest[27];
    if (!rd(rest, sizeof rest)) { set_error("s3e_model_load: truncated hparams"); return S3E_ERR_IO; }
    m->neck_dim = rest[6];
    m->visual_only = rest[26];
    if (m->patch <= 0 || m->img % m->patch != 0 || m->E <= 0 || m->heads <= 0 || m->E % m->heads != 0 ||
        m->depth <= 0 || m->depth > 256 || m->window <= 0) {
        set_error("s3e_model_load: inconsistent hparams");
        return S3E_ERR_IO;
    }
    m->grid = m->img / m->patch;
    if (m->E / m->heads != 64) { set_error("s3e_model_load: head dim %d not supported (64 only)", m->E / m->heads); return S3E_ERR_UNSUPPORTED; }
    if (m->E % 128 != 0) { set_error("s3e_model_load: embed dim %d must be a multiple of 128", m->E); return S3E_ERR_UNSUPPORTED; }
    if (m->grid % m->window != 0) { set_error("s3e_model_load: grid %d is not a multiple of the window %d", m->grid, m->window); return S3E_ERR_UNSUPPORTED; }
    // the QKV epilogue moves 8 consecutive tokens of one window row at a time
    if (m->window % 8 != 0) { set_error("s3e_model_load: window %d must be a multiple of 8", m->window); return S3E_ERR_UNSUPPORTED; }
    m->blocks.resize((size_t)m->depth);
    for (int i = 0; i < m->depth; i++) {
        for (int j = 0; j < m->n_global && j < 4; j++)
            if (m->gidx[j] == i) m->blocks[(size_t)i].global = true;
    }
    const int64_t E = m->E, MLP = m->mlp;
    int seen = 0;
    const int expected = 4 + 13 * m->depth;
    for (int ti = 0; ti < n_tensors; ti++) {
        int32_t hdr[3];
        if (!rd(hdr, 12)) { set_error("s3e_model_load: truncated tensor header %d", ti); return S3E_ERR_IO; }
        RawTensor t;
        t.n_dims = hdr[0];
        const int32_t name_len = hdr[1];
        t.type = hdr[2];
        if (t.n_dims < 1 || t.n_dims > 4 || name_len <= 0 || name_len > 256 || ggml_tsize(t.type) == 0) {
            set_error("s3e_model_load: malformed tensor record %d", ti);
            return S3E_ERR_IO;
        }
        for (int i = 0; i < t.n_dims; i++) {
            int32_t dd;
            if (!rd(&dd, 4) || dd <= 0) { set_error("s3e_model_load: bad dims in record %d", ti); return S3E_ERR_IO; }
            t.ne[i] = dd;
        }
        std::string name((size_t)name_len, '\0');
        if (!rd(&name[0], (size_t)name_len)) { set_error("s3e_model_load: truncated name"); return S3E_ERR_IO; }
        const std::streamoff pos = fin.tellg();
        fin.seekg((32 - pos % 32) % 32, std::ios::cur);
        if (t.ne[0] % ggml_blck(t.type) != 0) { set_error("s3e_model_load: '%s' ne0 not a block multiple", name.c_str()); return S3E_ERR_IO; }
        size_t bytes = 0;
        if (!fin || !record_bytes(t.type, t.ne, stream_left(fin), &bytes)) {
            set_error("s3e_model_load: data of '%s' oversized or past the end of the file", name.c_str());
            return S3E_ERR_IO;
        }
        const bool is_neck = name.compare(0, 9, "neck.det.") == 0 || name.compare(0, 9, "neck.trk.") == 0;
        if (memattn_wants(name)) {
            t.data.resize(bytes);
            if (!rd(t.data.data(), bytes)) { set_error("s3e_model_load: truncated data of '%s'", name.c_str()); return S3E_ERR_IO; }
            const int rc = memattn_take(&m->ma, name, std::move(t), wtype);
            if (rc != S3E_OK) return rc;
            continue;
        }
        if (name.compare(0, 4, "vit.") != 0 && !is_neck) {  // not part of the encoder: skip
            fin.seekg((std::streamoff)bytes, std::ios::cur);
            if (!fin) { set_error("s3e_model_load: truncated data of '%s'", name.c_str()); return S3E_ERR_IO; }
            continue;
        }
        t.data.resize(bytes);
        if (!rd(t.data.data(), bytes)) { set_error("s3e_model_load: truncated data of '%s'", name.c_str()); return S3E_ERR_IO; }
        // registered type (T1f/T3f/T4f → F32; T2/T4 → weight type iff ne0 % block == 0)
        int want = 0;
        const bool f32_reg = t.n_dims < 2 || name.find("pos_embed") != std::string::npos || name.find("freqs_cis") != std::string::npos;
        if (!f32_reg) want = (t.ne[0] % ggml_blck(wtype) == 0) ? wtype : 0;
        if (!coerce(t, want)) { set_error("s3e_model_load: cannot convert '%s' from type %d to %d", name.c_str(), t.type, want); return S3E_ERR_IO; }
        if (is_neck) {
            const int rc = load_neck_tensor(m.get(), name, t);
            if (rc != S3E_OK) return rc;
            continue;
        }
        int rc = S3E_OK;
        if (name == "vit.patch_embed.proj.weight") {
            if (t.ne[0] != m->patch || t.ne[1] != m->patch || t.ne[2] != 3 || t.ne[3] != E) { set_error("patch_embed shape mismatch"); return S3E_ERR_IO; }
            const int64_t K = 3LL * m->patch * m->patch;
            // pad K to a multiple of 32 with zero columns (the im2col rows are padded the same way)
            const int64_t Kp = round_up(K, 32);
            const int es = (t.type == 1) ? 2 : 4;
            std::vector<uint8_t> padded((size_t)(E * Kp * es), 0);
            for (int64_t n = 0; n < E; n++) std::memcpy(&padded[(size_t)(n * Kp * es)], &t.data[(size_t)(n * K * es)], (size_t)(K * es));
            rc = upload_weight(ctx->device, t.type, Kp, E, padded.data(), padded.size(), m->patch_w);
            if (rc == S3E_OK && t.type == 0)
                rc = upload_weight_split((const float *)padded.data(), Kp, E, m->patch_split, GEMM_BN);
        } else if (name == "vit.pos_embed") {
            m->pos_grid = (int)t.ne[1];
            if (t.ne[0] != E || t.ne[1] != t.ne[2] || m->pos_grid <= 0) { set_error("pos_embed shape mismatch"); return S3E_ERR_IO; }
            rc = upload_f32(m.get(), t, E * t.ne[1] * t.ne[2], &m->pos);
        } else if (name == "vit.ln_pre.weight") {
            rc = upload_f32(m.get(), t, E, &m->ln_pre_w);
        } else if (name == "vit.ln_pre.bias") {
            rc = upload_f32(m.get(), t, E, &m->ln_pre_b);
        } else if (name.compare(0, 11, "vit.blocks.") == 0) {
            const size_t dot = name.find('.', 11);
            const int bi = std::atoi(name.substr(11, dot - 11).c_str());
            if (bi < 0 || bi >= m->depth || dot == std::string::npos) { set_error("tensor '%s' has a bad block index", name.c_str()); return S3E_ERR_IO; }
            Block &b = m->blocks[(size_t)bi];
            const std::string f = name.substr(dot + 1);
            const int64_t Nw = b.global ? (int64_t)m->grid * m->grid : (int64_t)m->window * m->window;
            if (f == "norm1.weight") rc = upload_f32(m.get(), t, E, &b.n1w);
            else if (f == "norm1.bias") rc = upload_f32(m.get(), t, E, &b.n1b);
            else if (f == "norm2.weight") rc = upload_f32(m.get(), t, E, &b.n2w);
            else if (f == "norm2.bias") rc = upload_f32(m.get(), t, E, &b.n2b);
            else if (f == "attn.qkv.bias") rc = upload_f32(m.get(), t, 3 * E, &b.qkv_b);
            else if (f == "attn.proj.bias") rc = upload_f32(m.get(), t, E, &b.proj_b);
            else if (f == "mlp.lin1.bias") rc = upload_f32(m.get(), t, MLP, &b.fc1_b);
            else if (f == "mlp.lin2.bias") rc = upload_f32(m.get(), t, E, &b.fc2_b);
            else if (f == "attn.freqs_cis") {
                if (t.ne[0] != 2 || t.ne[1] != 32 || t.ne[2] != Nw) { set_error("'%s': expected [2, 32, %lld]", name.c_str(), (long long)Nw); return S3E_ERR_IO; }
                rc = upload_f32(m.get(), t, 64 * Nw, &b.freqs);
                b.freqs_n = Nw;
            } else if (f == "attn.qkv.weight" || f == "attn.proj.weight" || f == "mlp.lin1.weight" || f == "mlp.lin2.weight") {
                Weight &w = (f == "attn.qkv.weight") ? b.qkv : (f == "attn.proj.weight") ? b.proj : (f == "mlp.lin1.weight") ? b.fc1 : b.fc2;
                const int64_t eK = (f == "mlp.lin2.weight") ? MLP : E;
                const int64_t eN = (f == "attn.qkv.weight") ? 3 * E : (f == "mlp.lin1.weight") ? MLP : E;
                if (t.ne[0] != eK || t.ne[1] != eN) { set_error("'%s': expected [%lld, %lld]", name.c_str(), (long long)eK, (long long)eN); return S3E_ERR_IO; }
                rc = upload_weight(ctx->device, t.type, eK, eN, t.data.data(), t.data.size(), w);
            } else {
                continue;  // unknown per-block tensor: not used by the backbone
            }
        } else {
            continue;
        }
        if (rc != S3E_OK) return rc;
        seen++;
    }
    if (seen != expected) {
        set_error("s3e_model_load: found %d of %d backbone tensors", seen, expected);
        return S3E_ERR_IO;
    }
    if (m->mlp % 128 != 0) { set_error("s3e_model_load: MLP width %d must be a multiple of 128", m->mlp); return S3E_ERR_UNSUPPORTED; }
    // necks: optional (an encoder-only file has none); a partial one is an error
    for (int which = 0; which < 2; which++) {
        if (m->necks[which].found == 0) continue;
        int rc = check_neck(m.get(), which);
        if (rc == S3E_OK) rc = fold_neck0(m.get(), which);
        if (rc != S3E_OK) return rc;
        m->necks_present |= which == 1 ? 1 : 2;
    }
    *out = m.release();
    return S3E_OK;
} S3E_CATCH("s3e_model_load")

extern "C" int s3e_model_type(const s3e_model *m) try {
    if (!m) return -1;
    if (m->hiera) return 2;           // SAM3_MODEL_SAM2
    return m->necks_present & 2 ? 0   // SAM3_MODEL_SAM3
                                : 1;  // SAM3_MODEL_SAM3_VISUAL
} S3E_CATCH("s3e_model_type")

extern "C" int s3e_model_hparams(const s3e_model *m, int32_t out[16]) try {
    if (!m || !out) { set_error("s3e_model_hparams: NULL argument"); return S3E_ERR_INVALID; }
    if (m->hiera) {
        hiera_hparams(m->hiera, out);
        return S3E_OK;
    }
    std::memset(out, 0, 16 * sizeof(int32_t));
    out[0] = m->img; out[1] = m->patch; out[2] = m->E; out[3] = m->depth; out[4] = m->heads;
    out[5] = m->mlp; out[6] = m->window; out[7] = m->n_global;
    for (int i = 0; i < 4; i++) out[8 + i] = m->gidx[i];
    out[12] = m->ftype;
    out[13] = m->grid;
    out[14] = m->neck_dim;
    out[15] = m->necks_present;
    return S3E_OK;
} S3E_CATCH("s3e_model_hparams")

// ---- state + encoder --------------------------------------------------------
struct s3e_state {
    s3e_ctx *ctx = nullptr;
    const s3e_model *m = nullptr;
    int img = 0;                  // image size this state encodes (the model's, or a SAM 2 override)
    MemAttnState *mas = nullptr;  // memory-attention scratch, made at first use
    int64_t T = 0;
    float *x = nullptr;       // residual stream, T × E f32 ("vit_output" after encode)
    float *chw = nullptr;     // uploaded image for the host-pointer entry points
    uint8_t *img8 = nullptr;  // uint8 image of s3e_encode_image_u8, grown to the largest seen
    size_t img8_cap = 0;
    ActBuf a1, a2, col;       // E-wide, MLP-wide and im2col activations
    _Float16 *q16 = nullptr, *k16 = nullptr, *vt16 = nullptr;  // [hi plane | lo plane]
    int64_t vt_elems = 0;
    // Q, K, Vᵀ (hi + lo planes) of the global blocks when the blocks run in
    // bands: two sets used in turn, apart from the windowed blocks' q16 / k16 /
    // vt16, because a band that moves on to the next block writes its rows of
    // that block's layout while the other bands may still read theirs
    _Float16 *gq16[2] = {nullptr, nullptr}, *gk16[2] = {nullptr, nullptr}, *gvt16[2] = {nullptr, nullptr};
    int64_t gvt_elems = 0;
    // necks: level sides, outputs (f32 [side²][D]) per neck, the shared PEs,
    // and fp16 work planes, each [hi | lo] of cap halves
    int64_t side[4] = {0, 0, 0, 0};
    float *neck_out[2][4] = {{nullptr, nullptr, nullptr, nullptr}, {nullptr, nullptr, nullptr, nullptr}};
    float *pe[4] = {nullptr, nullptr, nullptr, nullptr};
    // fp16 planes of vit_output (nx), the scale-0 first deconvolution output
    // (n_dc), and per level the 1×1 input (lv_a) and 3×3 input (lv_b)
    _Float16 *nx = nullptr, *n_dc = nullptr, *lv_a[4] = {}, *lv_b[4] = {};
    int64_t nx_cap = 0, lv_a_cap[4] = {}, lv_b_cap[4] = {};
    void *zero = nullptr;
    // the four levels are independent after the shared conversion: levels 1
    // and 2-3 run on two more streams (default priority) joined back into
    // the context stream by events
    hipStream_t aux[2] = {nullptr, nullptr};
    hipEvent_t ev_fork = nullptr, ev_join[2] = {nullptr, nullptr};
    HieraState *hst = nullptr;  // SAM 2.x models
    // sub-stage hooks: f32 scratch grown on demand, and an F16 copy of an
    // F32 patch kernel (the mul_mat stages convert the kernel to F16)
    float *stg = nullptr;
    int64_t stg_cap = 0;
    Weight patch16;
};

extern "C" void s3e_state_free(s3e_state *st) {
    if (!st) return;
    (void)hipSetDevice(st->ctx->device);
    (void)hipStreamSynchronize(st->ctx->stream);
    if (st->mas) memattn_state_free(st->mas);
    if (st->x) (void)hipFree(st->x);
    if (st->chw) (void)hipFree(st->chw);
    if (st->img8) (void)hipFree(st->img8);
    st->a1.release();
    st->a2.release();
    st->col.release();
    if (st->q16) (void)hipFree(st->q16);
    if (st->k16) (void)hipFree(st->k16);
    if (st->vt16) (void)hipFree(st->vt16);
    for (int i = 0; i < 2; i++) {
        if (st->gq16[i]) (void)hipFree(st->gq16[i]);
        if (st->gk16[i]) (void)hipFree(st->gk16[i]);
        if (st->gvt16[i]) (void)hipFree(st->gvt16[i]);
    }
    for (auto &lv : st->neck_out)
        for (float *p : lv)
            if (p) (void)hipFree(p);
    for (float *p : st->pe)
        if (p) (void)hipFree(p);
    for (void *p : {(void *)st->nx, (void *)st->n_dc, st->zero})
        if (p) (void)hipFree(p);
    for (int i = 0; i < 4; i++) {
        if (st->lv_a[i]) (void)hipFree(st->lv_a[i]);
        if (st->lv_b[i]) (void)hipFree(st->lv_b[i]);
    }
    for (int i = 0; i < 2; i++) {
        if (st->aux[i]) (void)hipStreamDestroy(st->aux[i]);
        if (st->ev_join[i]) (void)hipEventDestroy(st->ev_join[i]);
    }
    if (st->ev_fork) (void)hipEventDestroy(st->ev_fork);
    if (st->hst) hiera_state_free(st->hst);
    if (st->stg) (void)hipFree(st->stg);
    free_weight(st->patch16);
    delete st;
}

namespace {

// Neck buffers and PEs of a state (sizes from the loaded necks).
hipError_t alloc_neck(s3e_state *st) {
    const s3e_model *m = st->m;
    if (!m->necks_present) return hipSuccess;
    const int64_t G = m->grid, T = G * G, E = m->E;
    st->side[0] = 4 * G;
    st->side[1] = 2 * G;
    st->side[2] = G;
    st->side[3] = (G - 2) / 2 + 1;
    int64_t D = m->neck_dim, mid0 = 0, mid1 = 0;
    for (const Neck &nk : m->necks) {
        if (!nk.found) continue;
        mid0 = std::max(mid0, nk.s[0].dc[0].N / 4);
        mid1 = std::max(mid1, nk.s[1].dc[0].N / 4);
    }
    const int64_t S3 = st->side[3] * st->side[3];
    st->nx_cap = T * E;
    const int64_t a_cap[4] = {16 * T * D, 4 * T * mid1, 0, S3 * E};
    hipError_t e = hipMalloc(&st->nx, (size_t)st->nx_cap * 2 * 2);
    if (e == hipSuccess) e = hipMalloc(&st->n_dc, (size_t)(4 * T * mid0) * 2);
    for (int i = 0; i < 4 && e == hipSuccess; i++) {
        st->lv_a_cap[i] = a_cap[i];
        st->lv_b_cap[i] = st->side[i] * st->side[i] * D;
        if (a_cap[i]) e = hipMalloc(&st->lv_a[i], (size_t)a_cap[i] * 2 * 2);
        if (e == hipSuccess) e = hipMalloc(&st->lv_b[i], (size_t)st->lv_b_cap[i] * 2 * 2);
    }
    if (e == hipSuccess) e = hipMalloc(&st->zero, 256);
    if (e == hipSuccess) e = hipMemsetAsync(st->zero, 0, 256, st->ctx->stream);
    for (int which = 0; which < 2 && e == hipSuccess; which++) {
        if (!m->necks[which].found) continue;
        for (int i = 0; i < 4 && e == hipSuccess; i++)
            e = hipMalloc(&st->neck_out[which][i], (size_t)(st->side[i] * st->side[i] * D) * 4);
    }
    for (int i = 0; i < 4 && e == hipSuccess; i++) {
        const std::vector<float> pe = sinusoidal_pe_2d((int)st->side[i], (int)st->side[i], (int)D);
        e = hipMalloc(&st->pe[i], pe.size() * 4);
        if (e == hipSuccess) e = hipMemcpy(st->pe[i], pe.data(), pe.size() * 4, hipMemcpyHostToDevice);
    }
    return e;
}

}  // namespace

namespace {
int vit_bands(const s3e_state *st);
}  // namespace

extern "C" int s3e_state_create(s3e_ctx *ctx, const s3e_model *m, s3e_state **out) {
    return s3e_state_create_sized(ctx, m, 0, out);
}

extern "C" int s3e_state_create_sized(s3e_ctx *ctx, const s3e_model *m, int img_size, s3e_state **out) try {
    if (!ctx || !m || !out) { set_error("s3e_state_create: NULL argument"); return S3E_ERR_INVALID; }
    *out = nullptr;
    if (img_size < 0) { set_error("s3e_state_create: negative image size"); return S3E_ERR_INVALID; }
    // sam3_create_state (sam3.cpp:3392-3402): a state may encode at another
    // image size than the model's; the engine builds SAM 2.x (Hiera)
    // encoders for any multiple of 32 and the SAM 3 ViT at its native grid
    if (!m->hiera && img_size != 0 && img_size != m->img) {
        set_error("s3e_state_create: a SAM 3 file encodes at its native %d px (asked %d)", m->img, img_size);
        return S3E_ERR_UNSUPPORTED;
    }
    HIP_TRY(hipSetDevice(ctx->device));
    auto *st = new s3e_state;
    st->ctx = ctx;
    st->m = m;
    st->img = img_size > 0 ? img_size : m->img;
    if (m->hiera) {
        hipError_t e = hipMalloc(&st->chw, (size_t)3 * st->img * st->img * 4);
        const int rc = e == hipSuccess ? hiera_state_create(m->hiera, st->img, ctx->stream, &st->hst) : (int)S3E_ERR_NOMEM;
        if (rc != S3E_OK) {
            if (e != hipSuccess) set_error("s3e_state_create: %s", hipGetErrorString(e));
            s3e_state_free(st);
            return rc;
        }
        *out = st;
        return S3E_OK;
    }
    st->T = (int64_t)m->grid * m->grid;
    const int64_t T = st->T, E = m->E;
    hipError_t e = hipMalloc(&st->x, (size_t)(T * E * 4));
    if (e == hipSuccess) e = hipMalloc(&st->chw, (size_t)3 * m->img * m->img * 4);
    if (e == hipSuccess) e = st->a1.alloc(T, E, ctx->stream);
    if (e == hipSuccess) e = st->a2.alloc(T, m->mlp, ctx->stream);
    if (e == hipSuccess) e = st->col.alloc(T, round_up(3LL * m->patch * m->patch, 32), ctx->stream);
    // Q, K, Vᵀ hold two fp16 planes each (hi, lo) for split-precision attention
    if (e == hipSuccess) e = hipMalloc(&st->q16, (size_t)(T * E * 2 * 2));
    if (e == hipSuccess) e = hipMalloc(&st->k16, (size_t)(T * E * 2 * 2));
    // Vᵀ rows are padded to a multiple of 16 keys: size for the widest block.
    int64_t vt_elems = T * E;
    for (const Block &b : m->blocks) {
        const int64_t WS = b.global ? m->grid : m->window;
        const int64_t NW = (m->grid / WS) * (m->grid / WS);
        vt_elems = std::max<int64_t>(vt_elems, NW * m->heads * 64 * vt_ld_for(WS * WS));
    }
    st->vt_elems = vt_elems;
    if (e == hipSuccess) e = hipMalloc(&st->vt16, (size_t)(vt_elems * 2 * 2));
    // two side streams (default priority) and their events: the windowed
    // blocks' row bands and the neck levels run on them
    for (int i = 0; i < 2 && e == hipSuccess; i++) {
        e = hipStreamCreateWithFlags(&st->aux[i], hipStreamNonBlocking);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&st->ev_join[i], hipEventDisableTiming);
    }
    if (e == hipSuccess) e = hipEventCreateWithFlags(&st->ev_fork, hipEventDisableTiming);
    if (e == hipSuccess && vit_bands(st) > 1) {
        bool any_global = false;
        for (const Block &b : m->blocks) any_global = any_global || b.global;
        st->gvt_elems = m->heads * 64 * vt_ld_for(T);
        for (int i = 0; i < 2 && any_global && e == hipSuccess; i++) {
            e = hipMalloc(&st->gq16[i], (size_t)(T * E * 2 * 2));
            if (e == hipSuccess) e = hipMalloc(&st->gk16[i], (size_t)(T * E * 2 * 2));
            if (e == hipSuccess) e = hipMalloc(&st->gvt16[i], (size_t)(st->gvt_elems * 2 * 2));
        }
    }
    if (e == hipSuccess) e = alloc_neck(st);
    if (e != hipSuccess) {
        s3e_state_free(st);
        set_error("s3e_state_create: %s", hipGetErrorString(e));
        return S3E_ERR_NOMEM;
    }
    *out = st;
    return S3E_OK;
} S3E_CATCH("s3e_state_create")

namespace {

// The patch embedding's im2col and GEMM into y with epilogue epi (EPI_POS
// or EPI_F32): an F32 kernel runs as split fp16 pairs on the fp16 MFMA.
hipError_t patch_gemm(s3e_state *st, const float *chw, Epi epi, const EpiArgs &ea, hipStream_t s) {
    const s3e_model *m = st->m;
    const Weight &w = m->patch_split.q ? m->patch_split : m->patch_w;
    const int64_t ldk = m->patch_w.K;  // 3·P² padded to 32
    const Act col = st->col.as(act_kind_for(w.kind), ldk);
    hipError_t e = launch_im2col(chw, m->img, m->patch, ldk, col.kind, col.x, s, col.lo);
    if (e == hipSuccess) e = launch_gemm(w, col, st->T, epi, ea, s);
    return e;
}

hipError_t run_prefix(s3e_state *st, const float *chw, float *x) {
    const s3e_model *m = st->m;
    hipStream_t s = st->ctx->stream;
    EpiArgs ea;
    ea.y = x;
    ea.ldy = m->E;
    ea.pos = m->pos;
    ea.pos_grid = m->pos_grid;
    ea.grid = m->grid;
    hipError_t e = patch_gemm(st, chw, EPI_POS, ea, s);
    if (e != hipSuccess) return e;
    Act none;
    return launch_layernorm(x, st->T, m->E, 1e-5f, m->ln_pre_w, m->ln_pre_b, none, x, s);
}

// The launches of a block, one bit each, and its phases: A = LN1 + QKV,
// B = attention, C = proj + LN2 + fc1 + fc2.
enum : int {
    ST_LN1 = 1, ST_QKV = 2, ST_ATTN = 4, ST_PROJ = 8, ST_LN2 = 16, ST_FC1 = 32, ST_FC2 = 64,
    PH_A = ST_LN1 | ST_QKV, PH_B = ST_ATTN, PH_C = ST_PROJ | ST_LN2 | ST_FC1 | ST_FC2, PH_ALL = PH_A | PH_B | PH_C
};

// sam3_vit_block_forward (sam3.cpp:3710-3801) as 7 launches on stream s, for
// the token rows [r0, r0 + rows) (r0 and rows multiples of 64).  Phases A and
// C work token by token, and a windowed block's attention stays inside its
// windows, so a band of whole window rows is a block of its own: its
// activations, Q/K/Vᵀ windows and residual rows are disjoint parts of the
// state's buffers.  A global block's attention (phase B) needs every row;
// its phases A and C take any band, with the band's rows at their positions
// in the one window; its attention takes a band of queries too, against
// all keys, once every band's phase A is done.
hipError_t run_block_rows(s3e_state *st, int bi, float *x, int64_t r0, int64_t rows, hipStream_t s,
                          int phases = PH_ALL, int gset = -1) {
    const s3e_model *m = st->m;
    const Block &b = m->blocks[(size_t)bi];
    const int64_t T = rows, E = m->E;
    const int WS = b.global ? m->grid : m->window;
    const int Nw = WS * WS;
    // the band's Q/K/Vᵀ: windowed blocks from its first window on (windows
    // row-major over the grid); the global block's one window from position
    // r0 on (r0 a multiple of 16 keeps Vᵀ's slot groups whole)
    int64_t qoff, voff, foff = 0, NW;
    if (b.global) {
        qoff = r0 * 64;
        voff = r0;
        foff = r0 * 64;
        NW = 1;
    } else {
        const int64_t w0 = r0 / ((int64_t)WS * m->grid) * (m->grid / WS);
        qoff = w0 * m->heads * Nw * 64;
        voff = w0 * m->heads * 64 * vt_ld_for(Nw);
        NW = rows / ((int64_t)WS * m->grid) * (m->grid / WS);
    }
    float *xb = x + r0 * E;
    // Quantized (and F32) projections re-quantize the attention output: run
    // attention split so it matches f32 attention; F16 models use plain fp16.
    const bool split = b.proj.kind != WK_F16;
    // Q/K/Vᵀ planes: the state's own, or global set gset (banded runs)
    _Float16 *Q = gset >= 0 ? st->gq16[gset] : st->q16, *K = gset >= 0 ? st->gk16[gset] : st->k16;
    _Float16 *VT = gset >= 0 ? st->gvt16[gset] : st->vt16;
    const int64_t vte = gset >= 0 ? st->gvt_elems : st->vt_elems;
    _Float16 *q = Q + qoff, *k = K + qoff, *vt = VT + voff;
    _Float16 *q_lo = split ? Q + st->T * E + qoff : nullptr, *k_lo = split ? K + st->T * E + qoff : nullptr;
    _Float16 *vt_lo = split ? VT + vte + voff : nullptr;
    const Act a_proj = act_rows(st->a1.as(act_kind_gemm(b.proj), E), r0);
    const Act a_qkv = act_rows(st->a1.as(act_kind_gemm(b.qkv), E), r0);
    const Act a_fc1 = act_rows(st->a1.as(act_kind_gemm(b.fc1), E), r0);
    const Act a_fc2 = act_rows(st->a2.as(act_kind_gemm(b.fc2), m->mlp), r0);
    hipError_t e = hipSuccess;
    if (phases & ST_LN1) {
        // LN1 → activation for the QKV weight
        e = launch_layernorm(xb, T, E, 1e-5f, b.n1w, b.n1b, a_qkv, nullptr, s);
        if (e != hipSuccess) return e;
    }
    if (phases & ST_QKV) {
        // QKV GEMM + bias + RoPE → fp16 Q, K, Vᵀ in window layout
        EpiArgs eq;
        eq.bias = b.qkv_b;
        eq.grid = m->grid;
        eq.window = WS;
        eq.E = (int)E;
        eq.HD = 64;
        eq.NH = m->heads;
        eq.freqs = b.freqs ? b.freqs + foff : nullptr;
        eq.q = q;
        eq.k = k;
        eq.vt = vt;
        eq.q_lo = q_lo;
        eq.k_lo = k_lo;
        eq.vt_lo = vt_lo;
        eq.vt_ld = (int)vt_ld_for(Nw);
        e = launch_gemm(b.qkv, a_qkv, T, EPI_QKV, eq, s);
        if (e != hipSuccess) return e;
    }
    if (phases & ST_ATTN) {
        // attention → activation for the proj weight, un-partitioned
        AttnArgs aa;
        aa.q = q;
        aa.q_lo = q_lo;
        aa.Nq = (int)(b.global ? rows : Nw);
        aa.Nkv = Nw;
        if (b.global) {
            // the band's queries (rows of the one window, heads Nw rows apart)
            // against every key
            aa.q_hs = (int64_t)Nw * 64;
            aa.k = K;
            aa.vt = VT;
            aa.k_lo = split ? K + st->T * E : nullptr;
            aa.vt_lo = split ? VT + vte : nullptr;
        } else {
            aa.k = k;
            aa.vt = vt;
            aa.k_lo = k_lo;
            aa.vt_lo = vt_lo;
        }
        aa.NH = m->heads;
        aa.BH = (int)NW * m->heads;
        aa.scale = 1.0f / std::sqrt(64.0f);
        aa.grid = m->grid;
        aa.window = WS;
        aa.out = a_proj;
        e = launch_attn(aa, s);
        if (e != hipSuccess) return e;
    }
    if (phases & ST_PROJ) {
        // proj + bias + residual
        EpiArgs ep;
        ep.bias = b.proj_b;
        ep.y = xb;
        ep.ldy = E;
        e = launch_gemm(b.proj, a_proj, T, EPI_RESID, ep, s);
        if (e != hipSuccess) return e;
    }
    // LN2 → fc1 + bias + GELU(erf) → activation for fc2 → fc2 + bias + residual
    if (phases & ST_LN2) {
        e = launch_layernorm(xb, T, E, 1e-5f, b.n2w, b.n2b, a_fc1, nullptr, s);
        if (e != hipSuccess) return e;
    }
    if (phases & ST_FC1) {
        EpiArgs e1;
        e1.bias = b.fc1_b;
        e1.out = a_fc2;
        e = launch_gemm(b.fc1, a_fc1, T, EPI_GELU, e1, s);
        if (e != hipSuccess) return e;
    }
    if (phases & ST_FC2) {
        EpiArgs e2;
        e2.bias = b.fc2_b;
        e2.y = xb;
        e2.ldy = E;
        e = launch_gemm(b.fc2, a_fc2, T, EPI_RESID, e2, s);
    }
    return e;
}

hipError_t run_block(s3e_state *st, int bi, float *x) {
    return run_block_rows(st, bi, x, 0, st->T, st->ctx->stream);
}

// Bands of window rows: up to three, each on its own stream (the context's
// and the state's two side streams).  Each stream runs its band through the
// blocks while the others do the same, joined only around the global blocks'
// attention, so one band's single-round kernel tails, epilogue bursts and
// short LayerNorm passes overlap the other bands' main loops.  1 when the grid
// has fewer than two window rows, a window row is not a multiple of 64
// tokens, or the linears of the blocks read an activation buffer in more than
// one format (the formats' rows differ in bytes — fp6 tiles, Q8, fp16, f32 —
// so one band's rows in one format would overlap another band's in another).
int vit_bands(const s3e_state *st) {
    const s3e_model *m = st->m;
    const int nwr = m->grid / m->window;
    if (nwr < 2 || ((int64_t)m->window * m->grid) % 64 != 0 || !st->aux[0] || !st->aux[1] || m->blocks.empty())
        return 1;
    const AKind k1 = act_kind_gemm(m->blocks[0].qkv), k2 = act_kind_gemm(m->blocks[0].fc2);
    for (const Block &b : m->blocks)
        if (act_kind_gemm(b.qkv) != k1 || act_kind_gemm(b.proj) != k1 || act_kind_gemm(b.fc1) != k1 ||
            act_kind_gemm(b.fc2) != k2)
            return 1;
    return std::min(nwr, 3);
}

// The side streams wait for the context stream's work so far.
hipError_t fork_bands(s3e_state *st, int nb) {
    hipError_t e = hipEventRecord(st->ev_fork, st->ctx->stream);
    for (int k = 0; k < nb - 1 && e == hipSuccess; k++) e = hipStreamWaitEvent(st->aux[k], st->ev_fork, 0);
    return e;
}

// The context stream waits for the side streams' work so far (recorded also
// after an error, so that the context stream never runs ahead of work already
// queued on the side streams).
hipError_t join_bands(s3e_state *st, int nb, hipError_t e) {
    for (int k = 0; k < nb - 1; k++) {
        const hipError_t r = hipEventRecord(st->ev_join[k], st->aux[k]);
        const hipError_t w = r == hipSuccess ? hipStreamWaitEvent(st->ctx->stream, st->ev_join[k], 0) : r;
        if (e == hipSuccess) e = w;
    }
    return e;
}

// The backbone's blocks on x, in vit_bands() bands.
hipError_t run_blocks(s3e_state *st, float *x) {
    const s3e_model *m = st->m;
    const int nb = vit_bands(st);
    if (nb == 1) {
        for (int i = 0; i < m->depth; i++) {
            const hipError_t e = run_block(st, i, x);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const int nwr = m->grid / m->window;
    const int64_t wrow = (int64_t)m->window * m->grid;
    // the launches of the bands are enqueued step by step (each band's LN1,
    // then each band's QKV, ...), in the order the bands will need them
    auto bands = [&](int bi, int phases, int gset) {
        hipError_t e = hipSuccess;
        for (int step = ST_LN1; step <= ST_FC2 && e == hipSuccess; step <<= 1) {
            if (!(phases & step)) continue;
            for (int band = 0; band < nb && e == hipSuccess; band++) {
                const int64_t wr0 = (int64_t)nwr * band / nb, wr1 = (int64_t)nwr * (band + 1) / nb;
                e = run_block_rows(st, bi, x, wr0 * wrow, (wr1 - wr0) * wrow,
                                   band == 0 ? st->ctx->stream : st->aux[band - 1], step, gset);
            }
        }
        return e;
    };
    hipStream_t bs[3] = {st->ctx->stream, st->aux[0], st->aux[1]};
    hipEvent_t done_a[3] = {st->ev_fork, st->ev_join[0], st->ev_join[1]};
    // Hazards between bands.  Consecutive windowed blocks: each band writes
    // and reads only its own windows.  A global block: each band writes its
    // rows of a global Q/K/Vᵀ set and reads all of them only after the other
    // bands' phase A (the cross waits below), and the windowed blocks keep
    // their own planes, so a band entering or leaving a global block never
    // writes what another band may still read.  Global blocks use the two
    // sets in turn: a band rewrites a set only after the cross waits of the
    // global block in between, which every band passes after finishing the
    // attention that read that set.
    int nglobal = 0;
    hipError_t e = fork_bands(st, nb);
    for (int i = 0; i < m->depth && e == hipSuccess; i++) {
        if (!m->blocks[(size_t)i].global) {
            e = bands(i, PH_ALL, -1);
            continue;
        }
        // a global block: every band's QKV, then each band waits for the
        // others' and runs the attention of its own queries and its phase C
        const int gset = nglobal++ & 1;
        e = bands(i, PH_A, gset);
        for (int band = 0; band < nb && e == hipSuccess; band++) e = hipEventRecord(done_a[band], bs[band]);
        for (int band = 0; band < nb && e == hipSuccess; band++)
            for (int o = 0; o < nb && e == hipSuccess; o++)
                if (o != band) e = hipStreamWaitEvent(bs[band], done_a[o], 0);
        if (e == hipSuccess) e = bands(i, PH_B | PH_C, gset);
    }
    return join_bands(st, nb, e);
}

Act plane_act(AKind kind, _Float16 *base, int64_t cap, int64_t ld) {
    Act a;
    a.kind = kind;
    a.x = base;
    a.lo = base + cap;
    a.ld = ld;
    return a;
}

// One level of sam3_build_neck_graph (sam3.cpp:3863-3921) for one neck on
// vit_output x (G² rows of E f32), into st->neck_out[which][lvl], on stream
// s.  NHWC throughout: a pixel is a row of channels, so a 1×1 conv is a plain
// GEMM, a 2×2 stride-2 deconvolution is a GEMM with N = 4·Cout whose
// epilogue scatters each tap to its output pixel, and the 3×3 conv is an
// implicit GEMM over shifted pixel rows.  nx (the fp16 planes of x) is
// written by the caller before any level runs.
hipError_t run_level(s3e_state *st, int which, int lvl, const float *x, hipStream_t s) {
    const s3e_model *m = st->m;
    const NeckScale &sc = m->necks[which].s[lvl];
    const int G = m->grid;
    const int64_t T = (int64_t)G * G, E = m->E, D = m->neck_dim;
    const int side = (int)st->side[lvl];
    const Act a_3 = plane_act(act_kind_for(sc.c3.kind), st->lv_b[lvl], st->lv_b_cap[lvl], D);
    auto conv1 = [&](const Act &in, int64_t M) {
        EpiArgs e;
        e.bias = sc.c1_b;
        e.out = a_3;
        return launch_conv(sc.c1, in, M, EPI_ACT, e, nullptr, s);
    };
    auto deconv = [&](const Weight &w, const float *b, const Act &in, int in_side, int gelu, const Act &o) {
        EpiArgs e;
        e.bias = b;
        e.dc_w = in_side;
        e.dc_cout = (int)(w.N / 4);
        e.gelu = gelu;
        e.out = o;
        return launch_gemm(w, in, (int64_t)in_side * in_side, EPI_DECONV, e, s);
    };
    const Act x16 = plane_act(A_F16, st->nx, st->nx_cap, E);  // fp16(x): the deconvolutions' input
    hipError_t err = hipSuccess;
    if (lvl == 0) {
        // 4×: deconv + bias + gelu_erf (fp16: the next deconv's input), deconv + bias, 1×1
        const Act a_dc = plane_act(A_F16, st->n_dc, 0, sc.dc[0].N / 4);
        const Act a_1 = plane_act(act_kind_for(sc.c1.kind), st->lv_a[0], st->lv_a_cap[0], D);
        if ((err = deconv(sc.dc[0], sc.dc_b[0], x16, G, 1, a_dc)) != hipSuccess) return err;
        if ((err = deconv(sc.dc[1], sc.dc_b[1], a_dc, 2 * G, 0, a_1)) != hipSuccess) return err;
        if (sc.c3f.q) {
            // the 1×1 folded into the 3×3 (fold_neck0): straight from the deconvolution
            EpiArgs e;
            e.bias = sc.c3f_b;
            e.bias_cls = 1;
            e.y = st->neck_out[which][0];
            e.ldy = D;
            ConvGeom g;
            g.w = g.h = side;
            g.spt = (int)(D / 32);
            g.zero = st->zero;
            return launch_conv(sc.c3f, a_1, (int64_t)side * side, EPI_F32, e, &g, s);
        }
        err = conv1(a_1, 16 * T);
    } else if (lvl == 1) {
        // 2×: deconv + bias, 1×1
        const Act a_1 = plane_act(act_kind_for(sc.c1.kind), st->lv_a[1], st->lv_a_cap[1], sc.dc[0].N / 4);
        if ((err = deconv(sc.dc[0], sc.dc_b[0], x16, G, 0, a_1)) != hipSuccess) return err;
        err = conv1(a_1, 4 * T);
    } else if (lvl == 2) {
        // 1×: 1×1 on x itself
        err = conv1(plane_act(act_kind_for(sc.c1.kind), st->nx, st->nx_cap, E), T);
    } else {
        // 0.5×: 2×2 max pool, 1×1
        const Act a_1 = plane_act(act_kind_for(sc.c1.kind), st->lv_a[3], st->lv_a_cap[3], E);
        if ((err = launch_pool_act(x, G, G, (int)E, 2, a_1, s)) != hipSuccess) return err;
        err = conv1(a_1, (int64_t)side * side);
    }
    if (err != hipSuccess) return err;
    // 3×3 + bias → the level's f32 output
    EpiArgs e;
    e.bias = sc.c3_b;
    e.y = st->neck_out[which][lvl];
    e.ldy = D;
    ConvGeom g;
    g.w = g.h = side;
    g.spt = (int)(D / 32);
    g.zero = st->zero;
    return launch_conv(sc.c3, a_3, (int64_t)side * side, EPI_F32, e, &g, s);
}

// Both necks (detector first, as sam3.cpp:6072-6075 builds them) on x.
// Level 0 runs on the context stream, level 1 on aux[0], levels 2 and 3 on
// aux[1]; a level's buffers are its own, so the streams share nothing but
// the read-only nx and x.
hipError_t run_necks(s3e_state *st, const float *x) {
    const s3e_model *m = st->m;
    if (!m->necks_present) return hipSuccess;
    hipStream_t s = st->ctx->stream;
    // fp16 planes of x: hi feeds the deconvolutions, hi + lo the scale-2 1×1
    bool split = false;
    for (const Neck &nk : m->necks)
        if (nk.found && nk.s[2].c1.kind == WK_F16X3) split = true;
    hipError_t e = launch_pool_act(x, m->grid, m->grid, m->E, 1,
                                   plane_act(split ? A_F16X2 : A_F16, st->nx, st->nx_cap, m->E), s);
    if (e == hipSuccess) e = hipEventRecord(st->ev_fork, s);
    for (int i = 0; i < 2 && e == hipSuccess; i++) e = hipStreamWaitEvent(st->aux[i], st->ev_fork, 0);
    for (int which = 0; which < 2 && e == hipSuccess; which++) {
        if (!m->necks[which].found) continue;
        e = run_level(st, which, 0, x, s);
        if (e == hipSuccess) e = run_level(st, which, 1, x, st->aux[0]);
        if (e == hipSuccess) e = run_level(st, which, 2, x, st->aux[1]);
        if (e == hipSuccess) e = run_level(st, which, 3, x, st->aux[1]);
    }
    // join (also on error, so that the context stream never runs ahead of work
    // already queued on the side streams)
    for (int i = 0; i < 2; i++) {
        const hipError_t r = hipEventRecord(st->ev_join[i], st->aux[i]);
        const hipError_t w = r == hipSuccess ? hipStreamWaitEvent(s, st->ev_join[i], 0) : r;
        if (e == hipSuccess) e = w;
    }
    return e;
}

}  // namespace

extern "C" int s3e_vit_prefix(s3e_state *st, const float *chw_device, float *x_device) try {
    if (!st || !chw_device || !x_device) { set_error("s3e_vit_prefix: NULL argument"); return S3E_ERR_INVALID; }
    if (st->m->hiera) { set_error("s3e_vit_prefix: the model is a SAM 2 (Hiera) encoder"); return S3E_ERR_INVALID; }
    HIP_TRY(hipSetDevice(st->ctx->device));
    HIP_TRY(run_prefix(st, chw_device, x_device));
    return S3E_OK;
} S3E_CATCH("s3e_vit_prefix")

extern "C" int s3e_vit_block(s3e_state *st, int idx, float *x_device) try {
    if (!st || !x_device) { set_error("s3e_vit_block: NULL argument"); return S3E_ERR_INVALID; }
    if (st->m->hiera) { set_error("s3e_vit_block: the model is a SAM 2 (Hiera) encoder"); return S3E_ERR_INVALID; }
    if (idx < 0 || idx >= st->m->depth) { set_error("s3e_vit_block: block %d out of range", idx); return S3E_ERR_INVALID; }
    HIP_TRY(hipSetDevice(st->ctx->device));
    HIP_TRY(run_block(st, idx, x_device));
    return S3E_OK;
} S3E_CATCH("s3e_vit_block")

// ---- sub-stage hooks --------------------------------------------------------
// sam3_test_run_vit_block_stage / sam3_test_run_vit_prefix_stage
// (sam3.cpp:6390-6520, :6874-6993; stage builders :6716-6872): one operator
// group of the graph on an f32 input in ggml 4D layout, through the kernels
// the encoder uses for it.  Where the encoder fuses a stage into a
// neighbour's epilogue (window partition into the QKV store, RoPE into the
// QKV epilogue, GELU into fc1's, the position table into the patch GEMM's),
// the hook runs the same device arithmetic as a stand-alone pass.
namespace {

enum : int {
    BS_NORM1 = 0, BS_WINDOW_PART, BS_QKV_PROJ, BS_ATTN_CORE, BS_ATTN_PROJ, BS_WINDOW_UNPART, BS_NORM2,
    BS_MLP_FC1, BS_MLP_GELU, BS_MLP_FC2, BS_MLP
};
enum : int { PS_PATCH_EMBED = 0, PS_PATCH_IM2COL, PS_PATCH_MULMAT_RAW, PS_PATCH_MULMAT, PS_POS_ADD, PS_LN_PRE_NORM, PS_LN_PRE };

void norm_ne4(const int64_t *in, int64_t ne[4]) {
    for (int i = 0; i < 4; i++) ne[i] = (in && in[i] > 0) ? in[i] : 1;
}

hipError_t stage_scratch(s3e_state *st, int64_t floats) {
    if (floats <= st->stg_cap) return hipSuccess;
    if (st->stg) {
        hipError_t e = hipStreamSynchronize(st->ctx->stream);
        if (e != hipSuccess) return e;
        (void)hipFree(st->stg);
        st->stg = nullptr;
        st->stg_cap = 0;
    }
    hipError_t e = hipMalloc(&st->stg, (size_t)floats * 4);
    if (e == hipSuccess) st->stg_cap = floats;
    return e;
}

// y = W·x + b on M rows: x converted to W's activation format in buf, then
// the encoder's GEMM with an f32 output.
hipError_t stage_linear(s3e_state *st, const Weight &w, const float *bias, const ActBuf &buf, const float *x,
                        int64_t M, float *y) {
    hipStream_t s = st->ctx->stream;
    const Act a = buf.as(act_kind_gemm(w), w.K);
    hipError_t e = launch_rows_quant(a.kind, x, M, w.K, a, s);
    if (e != hipSuccess) return e;
    EpiArgs ea;
    ea.bias = bias;
    ea.y = y;
    ea.ldy = w.N;
    return launch_gemm(w, a, M, EPI_F32, ea, s);
}

// The F16 patch kernel the mul_mat stages multiply by.
int patch_f16(s3e_state *st, const Weight **out) {
    const s3e_model *m = st->m;
    if (m->patch_w.kind == WK_F16) { *out = &m->patch_w; return S3E_OK; }
    if (!st->patch16.q) {
        const Weight &w = m->patch_w;  // WK_F32 [Np][Kp]
        std::vector<float> f((size_t)(w.Np * w.Kp));
        HIP_TRY(hipMemcpy(f.data(), w.q, f.size() * 4, hipMemcpyDeviceToHost));
        std::vector<uint16_t> h((size_t)(w.N * w.K));
        for (int64_t n = 0; n < w.N; n++)
            for (int64_t k = 0; k < w.K; k++) h[(size_t)(n * w.K + k)] = host_f2h(f[(size_t)(n * w.Kp + k)]);
        const int rc = upload_weight(st->ctx->device, S3E_TYPE_F16, w.K, w.N, (const uint8_t *)h.data(),
                                     h.size() * 2, st->patch16);
        if (rc != S3E_OK) return rc;
    }
    *out = &st->patch16;
    return S3E_OK;
}

}  // namespace

extern "C" int s3e_vit_block_stage(s3e_state *st, int idx, int stage, const float *in_device, const int64_t in_ne[4],
                                   float *out_device, int64_t out_ne[4]) try {
    if (!st || !in_ne || !out_ne) { set_error("s3e_vit_block_stage: NULL argument"); return S3E_ERR_INVALID; }
    const s3e_model *m = st->m;
    if (m->hiera) { set_error("s3e_vit_block_stage: the model is a SAM 2 (Hiera) encoder"); return S3E_ERR_INVALID; }
    if (idx < 0 || idx >= m->depth) { set_error("s3e_vit_block_stage: invalid block_idx=%d", idx); return S3E_ERR_INVALID; }
    if (stage < BS_NORM1 || stage > BS_MLP) { set_error("s3e_vit_block_stage: unknown stage %d", stage); return S3E_ERR_INVALID; }
    const Block &b = m->blocks[(size_t)idx];
    const int64_t E = m->E, MLP = m->mlp, G = m->grid, WS = m->window, NH = m->heads, HD = E / NH;
    int64_t ne[4];
    norm_ne4(in_ne, ne);
    const int64_t want0 = stage == BS_ATTN_CORE ? 3 * E : ((stage == BS_MLP_GELU || stage == BS_MLP_FC2) ? MLP : E);
    if (ne[0] != want0) {
        set_error("s3e_vit_block_stage: stage %d input ne0=%lld expected %lld", stage, (long long)ne[0], (long long)want0);
        return S3E_ERR_INVALID;
    }
    int64_t o[4] = {ne[0], ne[1], ne[2], ne[3]};
    const int64_t npx = (ne[1] + WS - 1) / WS, npy = (ne[2] + WS - 1) / WS;
    switch (stage) {
        case BS_WINDOW_PART:
            if (ne[3] != 1) { set_error("s3e_vit_block_stage: window partition needs ne3 = 1"); return S3E_ERR_INVALID; }
            o[1] = WS; o[2] = WS; o[3] = npx * npy;
            break;
        case BS_WINDOW_UNPART: {
            const int64_t nw = ((G + WS - 1) / WS) * ((G + WS - 1) / WS);
            if (ne[1] != WS || ne[2] != WS || ne[3] != nw) {
                set_error("s3e_vit_block_stage: window unpartition needs [E, %lld, %lld, %lld]", (long long)WS, (long long)WS, (long long)nw);
                return S3E_ERR_INVALID;
            }
            o[1] = G; o[2] = G; o[3] = 1;
        } break;
        case BS_QKV_PROJ: o[0] = 3 * E; break;
        case BS_ATTN_CORE: o[0] = E; break;
        case BS_MLP_FC1: o[0] = MLP; break;
        case BS_MLP_FC2: o[0] = E; break;
        default: break;
    }
    for (int i = 0; i < 4; i++) out_ne[i] = o[i];
    if (!out_device) return S3E_OK;
    if (!in_device) { set_error("s3e_vit_block_stage: NULL input"); return S3E_ERR_INVALID; }
    const int64_t rows = ne[1] * ne[2] * ne[3];
    const int64_t orows = o[1] * o[2] * o[3];
    // the state's activation buffers hold T rows
    if (rows > st->T || orows > st->T) {
        set_error("s3e_vit_block_stage: %lld rows exceed the state's %lld", (long long)std::max(rows, orows), (long long)st->T);
        return S3E_ERR_INVALID;
    }
    HIP_TRY(hipSetDevice(st->ctx->device));
    hipStream_t s = st->ctx->stream;
    Act none;
    switch (stage) {
        case BS_NORM1:
        case BS_NORM2:
            HIP_TRY(launch_layernorm(in_device, rows, E, 1e-5f, stage == BS_NORM1 ? b.n1w : b.n2w,
                                     stage == BS_NORM1 ? b.n1b : b.n2b, none, out_device, s));
            break;
        case BS_WINDOW_PART:
            HIP_TRY(launch_win_perm(in_device, out_device, (int)ne[1], (int)ne[2], (int)WS, E, 1, s));
            break;
        case BS_WINDOW_UNPART:
            HIP_TRY(launch_win_perm(in_device, out_device, (int)G, (int)G, (int)WS, E, 0, s));
            break;
        case BS_QKV_PROJ: HIP_TRY(stage_linear(st, b.qkv, b.qkv_b, st->a1, in_device, rows, out_device)); break;
        case BS_ATTN_PROJ: HIP_TRY(stage_linear(st, b.proj, b.proj_b, st->a1, in_device, rows, out_device)); break;
        case BS_MLP_FC1: HIP_TRY(stage_linear(st, b.fc1, b.fc1_b, st->a1, in_device, rows, out_device)); break;
        case BS_MLP_FC2: HIP_TRY(stage_linear(st, b.fc2, b.fc2_b, st->a2, in_device, rows, out_device)); break;
        case BS_MLP_GELU: HIP_TRY(launch_gelu_rows(in_device, out_device, rows * MLP, s)); break;
        case BS_MLP: {
            // fc1 with the encoder's fused bias + GELU + conversion epilogue, then fc2
            const Act a1 = st->a1.as(act_kind_gemm(b.fc1), E);
            HIP_TRY(launch_rows_quant(a1.kind, in_device, rows, E, a1, s));
            EpiArgs e1;
            e1.bias = b.fc1_b;
            e1.out = st->a2.as(act_kind_gemm(b.fc2), MLP);
            HIP_TRY(launch_gemm(b.fc1, a1, rows, EPI_GELU, e1, s));
            EpiArgs e2;
            e2.bias = b.fc2_b;
            e2.y = out_device;
            e2.ldy = E;
            HIP_TRY(launch_gemm(b.fc2, e1.out, rows, EPI_F32, e2, s));
        } break;
        case BS_ATTN_CORE: {
            const int64_t N = ne[1] * ne[2], B = ne[3];
            if (b.freqs && b.freqs_n != N) {
                set_error("s3e_vit_block_stage: freqs_cis has %lld positions, attention has %lld", (long long)b.freqs_n, (long long)N);
                return S3E_ERR_INVALID;
            }
            const int64_t ldv = vt_ld_for(N);
            if (HD != 64 || B * NH * HD * ldv > st->vt_elems || B * NH > 65535) {
                set_error("s3e_vit_block_stage: attention shape [%lld tokens x %lld windows] not supported", (long long)N, (long long)B);
                return S3E_ERR_UNSUPPORTED;
            }
            HIP_TRY(stage_scratch(st, 2 * rows * E));
            float *rq = st->stg, *rk = st->stg + rows * E;
            HIP_TRY(launch_vit_rope_split(in_device, b.freqs, st->stg, B, N, (int)NH, (int)HD, s));
            // the encoder's rule: split fp16 pairs unless the projection is F16
            const bool split = b.proj.kind != WK_F16;
            _Float16 *q_lo = split ? st->q16 + st->T * E : nullptr;
            _Float16 *k_lo = split ? st->k16 + st->T * E : nullptr;
            _Float16 *vt_lo = split ? st->vt16 + st->vt_elems : nullptr;
            HIP_TRY(hipMemsetAsync(st->vt16, 0, (size_t)(B * NH * HD * ldv) * 2, s));
            if (split) HIP_TRY(hipMemsetAsync(vt_lo, 0, (size_t)(B * NH * HD * ldv) * 2, s));
            const int64_t qk_nb[4] = {1, HD, N * HD, NH * N * HD};
            const int64_t v_nb[4] = {1, 3 * E, HD, N * 3 * E};
            HIP_TRY(launch_attn_prep(rq, qk_nb, rk, qk_nb, in_device + 2 * E, v_nb, N, N, NH, B, (int)HD, 64,
                                     st->q16, st->k16, st->vt16, q_lo, k_lo, vt_lo, ldv, s));
            AttnArgs a;
            a.q = st->q16;
            a.k = st->k16;
            a.vt = st->vt16;
            a.q_lo = q_lo;
            a.k_lo = k_lo;
            a.vt_lo = vt_lo;
            a.Nq = (int)N;
            a.Nkv = (int)N;
            a.NH = (int)NH;
            a.BH = (int)(B * NH);
            a.scale = 1.0f / std::sqrt((float)HD);
            a.out.kind = A_F32;
            a.out.x = out_device;
            a.out.ld = E;
            HIP_TRY(launch_attn(a, s));
        } break;
        default: break;
    }
    return S3E_OK;
} S3E_CATCH("s3e_vit_block_stage")

extern "C" int s3e_vit_prefix_stage(s3e_state *st, int stage, const float *in_device, const int64_t in_ne[4],
                                    float *out_device, int64_t out_ne[4]) try {
    if (!st || !in_ne || !out_ne) { set_error("s3e_vit_prefix_stage: NULL argument"); return S3E_ERR_INVALID; }
    const s3e_model *m = st->m;
    if (m->hiera) { set_error("s3e_vit_prefix_stage: the model is a SAM 2 (Hiera) encoder"); return S3E_ERR_INVALID; }
    if (stage < PS_PATCH_EMBED || stage > PS_LN_PRE) { set_error("s3e_vit_prefix_stage: unknown stage %d", stage); return S3E_ERR_INVALID; }
    const int64_t P = m->patch, G = m->grid, E = m->E, T = st->T, K = 3 * P * P;
    int64_t ne[4];
    norm_ne4(in_ne, ne);
    int64_t o[4] = {ne[0], ne[1], ne[2], ne[3]};
    switch (stage) {
        case PS_PATCH_EMBED:
        case PS_PATCH_IM2COL:
            if (ne[0] != m->img || ne[1] != m->img || ne[2] != 3 || ne[3] != 1) {
                set_error("s3e_vit_prefix_stage: patch_embed input shape mismatch");
                return S3E_ERR_INVALID;
            }
            o[0] = stage == PS_PATCH_EMBED ? E : K; o[1] = G; o[2] = G; o[3] = 1;
            break;
        case PS_PATCH_MULMAT_RAW:
        case PS_PATCH_MULMAT:
            if (ne[0] != K || ne[1] != G || ne[2] != G || ne[3] != 1) {
                set_error("s3e_vit_prefix_stage: patch_mulmat input shape mismatch");
                return S3E_ERR_INVALID;
            }
            if (stage == PS_PATCH_MULMAT_RAW) { o[0] = T; o[1] = E; o[2] = 1; o[3] = 1; }
            else { o[0] = G; o[1] = G; o[2] = E; o[3] = 1; }
            break;
        default:
            if (ne[0] != E || ne[1] != G || ne[2] != G) {
                set_error("s3e_vit_prefix_stage: prefix feature input shape mismatch");
                return S3E_ERR_INVALID;
            }
            break;
    }
    for (int i = 0; i < 4; i++) out_ne[i] = o[i];
    if (!out_device) return S3E_OK;
    if (!in_device) { set_error("s3e_vit_prefix_stage: NULL input"); return S3E_ERR_INVALID; }
    const int64_t rows = ne[1] * ne[2] * ne[3];
    HIP_TRY(hipSetDevice(st->ctx->device));
    hipStream_t s = st->ctx->stream;
    const AKind pk = (m->patch_w.kind == WK_F16) ? A_F16 : A_F32;
    const int64_t ldk = m->patch_w.K;  // 3·P² padded to 32
    switch (stage) {
        case PS_PATCH_EMBED: {
            EpiArgs ea;
            ea.y = out_device;
            ea.ldy = E;
            HIP_TRY(patch_gemm(st, in_device, EPI_F32, ea, s));
        } break;
        case PS_PATCH_IM2COL:
            HIP_TRY(launch_im2col(in_device, m->img, m->patch, ldk, pk, st->col.x, s));
            HIP_TRY(launch_act_f32(st->col.as(pk, ldk), T, K, out_device, s));
            break;
        case PS_PATCH_MULMAT_RAW:
        case PS_PATCH_MULMAT: {
            // the stage's input is F16 (sam3.cpp:6463-6464) and mul_mat converts
            // the kernel to F16: fp16 × fp16 products, f32 sums, result [E][T]
            const Weight *w16 = nullptr;
            const int rc = patch_f16(st, &w16);
            if (rc != S3E_OK) return rc;
            const Act a = st->col.as(A_F16, ldk);
            HIP_TRY(hipMemsetAsync(a.x, 0, (size_t)(T * ldk) * 2, s));  // zero columns past K
            HIP_TRY(launch_rows_quant(A_F16, in_device, T, K, a, s));
            HIP_TRY(stage_scratch(st, T * E));
            EpiArgs ea;
            ea.y = st->stg;
            ea.ldy = E;
            HIP_TRY(launch_gemm(*w16, a, T, EPI_F32, ea, s));
            HIP_TRY(launch_transpose(st->stg, out_device, T, E, s));
        } break;
        case PS_POS_ADD:
            HIP_TRY(launch_add_pos(in_device, m->pos, out_device, (int)G, m->pos_grid, E, rows, s));
            break;
        case PS_LN_PRE_NORM:
        case PS_LN_PRE: {
            Act none;
            const bool aff = stage == PS_LN_PRE;
            HIP_TRY(launch_layernorm(in_device, rows, E, 1e-5f, aff ? m->ln_pre_w : nullptr, aff ? m->ln_pre_b : nullptr,
                                     none, out_device, s));
        } break;
        default: break;
    }
    return S3E_OK;
} S3E_CATCH("s3e_vit_prefix_stage")

extern "C" int s3e_encode_vit_chw(s3e_state *st, const float *chw_device) try {
    if (!st || !chw_device) { set_error("s3e_encode_vit_chw: NULL argument"); return S3E_ERR_INVALID; }
    if (st->m->hiera) { set_error("s3e_encode_vit_chw: the model is a SAM 2 (Hiera) encoder"); return S3E_ERR_INVALID; }
    HIP_TRY(hipSetDevice(st->ctx->device));
    HIP_TRY(run_prefix(st, chw_device, st->x));
    HIP_TRY(run_blocks(st, st->x));
    return S3E_OK;
} S3E_CATCH("s3e_encode_vit_chw")

extern "C" int s3e_model_tensor_get(const s3e_model *m, const char *name, int *type, int64_t ne[4], void *host,
                                    size_t bytes) try {
    if (!m || !name || !type || !ne) { set_error("s3e_model_tensor_get: NULL argument"); return S3E_ERR_INVALID; }
    if (m->hiera) { set_error("s3e_model_tensor_get: the model is a SAM 2 (Hiera) encoder"); return S3E_ERR_UNSUPPORTED; }
    const std::string n(name);
    const Weight *w = nullptr;
    const float *vec = nullptr;
    int64_t vlen = 0;
    int64_t K = 0;
    for (int i = 0; i < 4; i++) ne[i] = 1;
    if (n == "vit.patch_embed.proj.weight") {
        w = &m->patch_w;
        K = 3LL * m->patch * m->patch;
        ne[0] = m->patch; ne[1] = m->patch; ne[2] = 3; ne[3] = m->E;
    } else if (n.compare(0, 11, "vit.blocks.") == 0) {
        const size_t dot = n.find('.', 11);
        const int bi = dot == std::string::npos ? -1 : std::atoi(n.substr(11, dot - 11).c_str());
        if (bi < 0 || bi >= m->depth) { set_error("s3e_model_tensor_get: no tensor '%s'", name); return S3E_ERR_INVALID; }
        const Block &b = m->blocks[(size_t)bi];
        const std::string rest = n.substr(dot + 1);
        const struct { const char *w, *b; const Weight *wt; const float *bias; } lin[4] = {
            {"attn.qkv.weight", "attn.qkv.bias", &b.qkv, b.qkv_b}, {"attn.proj.weight", "attn.proj.bias", &b.proj, b.proj_b},
            {"mlp.lin1.weight", "mlp.lin1.bias", &b.fc1, b.fc1_b}, {"mlp.lin2.weight", "mlp.lin2.bias", &b.fc2, b.fc2_b}};
        for (const auto &l : lin) {
            if (rest == l.w) { w = l.wt; K = w->K; ne[0] = w->K; ne[1] = w->N; }
            if (rest == l.b) { vec = l.bias; vlen = l.wt->N; ne[0] = vlen; }
        }
    }
    if (!w && !vec) { set_error("s3e_model_tensor_get: no tensor '%s' (linear and patch weights and biases only)", name); return S3E_ERR_INVALID; }
    if (vec) {
        *type = S3E_TYPE_F32;
        if (!host) return S3E_OK;
        if (bytes < (size_t)vlen * 4) { set_error("s3e_model_tensor_get: buffer too small"); return S3E_ERR_INVALID; }
        HIP_TRY(hipSetDevice(m->ctx->device));
        HIP_TRY(hipMemcpy(host, vec, (size_t)vlen * 4, hipMemcpyDeviceToHost));
        return S3E_OK;
    }
    if (w->kind != WK_F16 && w->kind != WK_F32) {
        *type = w->ggml_type;  // the S3E_TYPE_* values are ggml's type ids
        set_error("s3e_model_tensor_get: '%s' is quantized; only F16 and F32 weights are returned", name);
        return S3E_ERR_UNSUPPORTED;
    }
    *type = w->kind == WK_F16 ? S3E_TYPE_F16 : S3E_TYPE_F32;
    if (!host) return S3E_OK;
    const size_t es = w->kind == WK_F16 ? 2 : 4;
    if (bytes < (size_t)(K * w->N) * es) { set_error("s3e_model_tensor_get: buffer too small"); return S3E_ERR_INVALID; }
    HIP_TRY(hipSetDevice(m->ctx->device));
    HIP_TRY(hipMemcpy2D(host, (size_t)K * es, w->q, (size_t)w->Kp * es, (size_t)K * es, (size_t)w->N, hipMemcpyDeviceToHost));
    return S3E_OK;
} S3E_CATCH("s3e_model_tensor_get")

extern "C" int s3e_encode_chw(s3e_state *st, const float *chw_device) try {
    if (!st || !chw_device) { set_error("s3e_encode_chw: NULL argument"); return S3E_ERR_INVALID; }
    HIP_TRY(hipSetDevice(st->ctx->device));
    if (st->m->hiera) {
        HIP_TRY(hiera_encode(st->m->hiera, st->hst, chw_device, st->ctx->stream));
        return S3E_OK;
    }
    HIP_TRY(run_prefix(st, chw_device, st->x));
    HIP_TRY(run_blocks(st, st->x));
    HIP_TRY(run_necks(st, st->x));
    return S3E_OK;
} S3E_CATCH("s3e_encode_chw")

extern "C" int s3e_run_neck(s3e_state *st, const float *x_device) try {
    if (!st || !x_device) { set_error("s3e_run_neck: NULL argument"); return S3E_ERR_INVALID; }
    if (!st->m->necks_present || st->m->hiera) { set_error("s3e_run_neck: the model has no SimpleFPN neck"); return S3E_ERR_INVALID; }
    HIP_TRY(hipSetDevice(st->ctx->device));
    HIP_TRY(run_necks(st, x_device));
    return S3E_OK;
} S3E_CATCH("s3e_run_neck")

extern "C" int s3e_mem_attn_dims(const s3e_model *m, int32_t out[4]) try {
    if (!m || !out) { set_error("s3e_mem_attn_dims: NULL argument"); return S3E_ERR_INVALID; }
    if (!m->ma) { set_error("s3e_mem_attn_dims: the model file has no memory attention"); return S3E_ERR_UNSUPPORTED; }
    memattn_dims(m->ma, out);
    return S3E_OK;
} S3E_CATCH("s3e_mem_attn_dims")

extern "C" int s3e_mem_attn(s3e_state *st, const float *curr, const float *src_pos, int64_t N, const float *prompt,
                            const float *prompt_pos, int64_t M_total, int64_t num_obj_ptr_tokens, const float *rope_q,
                            const float *rope_k, float *out) try {
    if (!st) { set_error("s3e_mem_attn: NULL state"); return S3E_ERR_INVALID; }
    if (!st->m->ma) { set_error("s3e_mem_attn: the model file has no memory attention"); return S3E_ERR_UNSUPPORTED; }
    HIP_TRY(hipSetDevice(st->ctx->device));
    return memattn_run(st->m->ma, &st->mas, curr, src_pos, N, prompt, prompt_pos, M_total, num_obj_ptr_tokens, rope_q,
                       rope_k, out, st->ctx->stream);
} S3E_CATCH("s3e_mem_attn")

extern "C" int s3e_hiera_block(s3e_state *st, int idx, const float *x_device, int H, int W, float *y_device) try {
    if (!st || !x_device || !y_device) { set_error("s3e_hiera_block: NULL argument"); return S3E_ERR_INVALID; }
    if (!st->m->hiera) { set_error("s3e_hiera_block: the model is not a SAM 2 (Hiera) encoder"); return S3E_ERR_INVALID; }
    int32_t hp[16];
    hiera_hparams(st->m->hiera, hp);
    if (idx < 0 || idx >= hp[3] || H <= 0 || W <= 0 || H > hp[13] || W > hp[13]) {
        set_error("s3e_hiera_block: block %d on %dx%d is out of range", idx, H, W);
        return S3E_ERR_INVALID;
    }
    HIP_TRY(hipSetDevice(st->ctx->device));
    const hipError_t e = hiera_block(st->m->hiera, st->hst, idx, x_device, H, W, y_device, st->ctx->stream);
    if (e == hipErrorInvalidValue) {
        set_error("s3e_hiera_block: block %d cannot run on a %dx%d input%s (larger than its encoder grid, odd "
                  "under Q stride, or in place across a size change)", idx, H, W, x_device == y_device ? " in place" : "");
        return S3E_ERR_INVALID;
    }
    HIP_TRY(e);
    return S3E_OK;
} S3E_CATCH("s3e_hiera_block")

extern "C" int s3e_encode_chw_host(s3e_state *st, const float *chw_host) try {
    if (!st || !chw_host) { set_error("s3e_encode_chw_host: NULL argument"); return S3E_ERR_INVALID; }
    HIP_TRY(hipSetDevice(st->ctx->device));
    HIP_TRY(hipMemcpyAsync(st->chw, chw_host, (size_t)3 * st->img * st->img * 4, hipMemcpyHostToDevice,
                           st->ctx->stream));
    return s3e_encode_chw(st, st->chw);
} S3E_CATCH("s3e_encode_chw_host")

extern "C" int s3e_preprocess_image(s3e_ctx *ctx, const uint8_t *hwc_device, int width, int height, int img_size,
                                    int norm, float *chw_device) try {
    if (!ctx || !hwc_device || !chw_device || width <= 0 || height <= 0 || img_size <= 0 ||
        (norm != S3E_NORM_SAM3 && norm != S3E_NORM_IMAGENET)) {
        set_error("s3e_preprocess_image: bad argument");
        return S3E_ERR_INVALID;
    }
    HIP_TRY(hipSetDevice(ctx->device));
    HIP_TRY(launch_preprocess(hwc_device, width, height, img_size, norm, chw_device, ctx->stream));
    return S3E_OK;
} S3E_CATCH("s3e_preprocess_image")

// sam3_encode_image's preprocessing (sam3_resize_bilinear +
// sam3_preprocess_image, sam3.cpp:3441-3514, or sam2_preprocess_image,
// :3518-3544, for SAM 2 models) on the device, then the encode.
extern "C" int s3e_encode_image_u8(s3e_state *st, const uint8_t *hwc, int width, int height) try {
    if (!st || !hwc || width <= 0 || height <= 0) { set_error("s3e_encode_image_u8: bad argument"); return S3E_ERR_INVALID; }
    HIP_TRY(hipSetDevice(st->ctx->device));
    const size_t bytes = (size_t)width * height * 3;
    if (bytes > st->img8_cap) {
        HIP_TRY(hipStreamSynchronize(st->ctx->stream));
        if (st->img8) (void)hipFree(st->img8);
        st->img8 = nullptr;
        st->img8_cap = 0;
        HIP_TRY(hipMalloc(&st->img8, bytes));
        st->img8_cap = bytes;
    }
    HIP_TRY(hipMemcpyAsync(st->img8, hwc, bytes, hipMemcpyHostToDevice, st->ctx->stream));
    const int norm = st->m->hiera ? S3E_NORM_IMAGENET : S3E_NORM_SAM3;
    int rc = s3e_preprocess_image(st->ctx, st->img8, width, height, st->img, norm, st->chw);
    if (rc == S3E_OK) rc = s3e_encode_chw(st, st->chw);
    if (rc != S3E_OK) return rc;
    return s3e_ctx_sync(st->ctx);
} S3E_CATCH("s3e_encode_image_u8")

namespace {

// Names of sam3_find_state_tensor (sam3.cpp:14334-14376): vit_output,
// neck_{det,trk}_<i>, neck_det_pe_<i> and the PE tensors pe_<i>, plus
// neck_trk_pe_<i> (the same PEs: sam3.cpp:6190-6192).  A tensor the model
// does not produce (neck_det_* of a visual-only model) does not resolve.
const float *find_tensor(const s3e_state *st, const char *name, int64_t ne[4]) {
    const s3e_model *m = st->m;
    if (m->hiera) return hiera_find_tensor(m->hiera, st->hst, name, ne);
    if (std::strcmp(name, "vit_output") == 0) {
        ne[0] = m->E; ne[1] = m->grid; ne[2] = m->grid; ne[3] = 1;
        return st->x;
    }
    int i = -1;
    const float *p = nullptr;
    auto level = [&](const char *prefix) {
        const size_t n = std::strlen(prefix);
        if (std::strncmp(name, prefix, n) == 0 && name[n] >= '0' && name[n] <= '3' && name[n + 1] == 0) {
            i = name[n] - '0';
            return true;
        }
        return false;
    };
    if (level("neck_det_pe_") || level("neck_trk_pe_") || level("pe_")) p = st->pe[i];
    else if (level("neck_det_")) p = st->neck_out[0][i];
    else if (level("neck_trk_")) p = st->neck_out[1][i];
    if (!p) return nullptr;
    ne[0] = m->neck_dim; ne[1] = st->side[i]; ne[2] = st->side[i]; ne[3] = 1;
    return p;
}

}  // namespace

extern "C" int s3e_state_tensor_info(const s3e_state *st, const char *name, int64_t ne[4]) try {
    if (!st || !name || !ne) { set_error("s3e_state_tensor_info: NULL argument"); return S3E_ERR_INVALID; }
    if (!find_tensor(st, name, ne)) { set_error("s3e_state_tensor_info: unknown tensor '%s'", name); return S3E_ERR_INVALID; }
    return S3E_OK;
} S3E_CATCH("s3e_state_tensor_info")

extern "C" const float *s3e_state_tensor_device(const s3e_state *st, const char *name) {
    int64_t ne[4];
    if (!st || !name) return nullptr;
    return find_tensor(st, name, ne);
}

extern "C" int s3e_state_tensor_get(const s3e_state *st, const char *name, float *host, size_t n) try {
    int64_t ne[4];
    if (!st || !name) { set_error("s3e_state_tensor_get: NULL argument"); return S3E_ERR_INVALID; }
    const float *src = find_tensor(st, name, ne);
    if (!src) { set_error("s3e_state_tensor_get: unknown tensor '%s'", name); return S3E_ERR_INVALID; }
    const size_t need = (size_t)(ne[0] * ne[1] * ne[2] * ne[3]);
    if (!host || n < need) { set_error("s3e_state_tensor_get: buffer holds %zu floats, need %zu", n, need); return S3E_ERR_INVALID; }
    HIP_TRY(hipSetDevice(st->ctx->device));
    HIP_TRY(hipMemcpyAsync(host, src, need * 4, hipMemcpyDeviceToHost, st->ctx->stream));
    HIP_TRY(hipStreamSynchronize(st->ctx->stream));
    return S3E_OK;
} S3E_CATCH("s3e_state_tensor_get")
