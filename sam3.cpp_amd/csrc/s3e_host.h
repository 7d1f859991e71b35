// s3e_host.h — host-side helpers shared by the runtime and the model-file
// code: fp16 conversion, ggml block formats and the reference quantizers.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>
#include <istream>

namespace s3e {

// IEEE binary16 round-to-nearest-even (ggml's fp32→fp16 on F16C hosts).
inline uint16_t host_f2h(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        float a;
        std::memcpy(&a, &ax, 4);
        return (uint16_t)(sign | (uint32_t)std::nearbyint(a * 16777216.0f));
    }
    const uint32_t mant = ax & 0x7fffffu;
    uint32_t h = (((ax >> 23) - 112u) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

inline float host_h2f(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            float v = (float)m * (1.0f / 16777216.0f);
            std::memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

inline int64_t ggml_blck(int type) { return (type == 2 || type == 3 || type == 8 || type == 9) ? 32 : 1; }
inline size_t ggml_tsize(int type) {
    switch (type) {
        case 0: return 4;
        case 1: return 2;
        case 2: return 18;
        case 3: return 20;
        case 8: return 34;
        case 9: return 36;
        default: return 0;
    }
}
inline size_t ggml_rowsize(int type, int64_t ne0) { return ggml_tsize(type) * (size_t)(ne0 / ggml_blck(type)); }

// Data bytes of a tensor record with dims ne[0..3] (positive, unused ones 1)
// of ggml type `type`, if that size is representable and at most `left`
// (the bytes remaining in the file): a malformed or truncated record is
// refused before anything is allocated for it.
inline bool record_bytes(int type, const int64_t ne[4], int64_t left, size_t *bytes) {
    const int64_t lim = (int64_t)1 << 62;
    int64_t rows = 1;
    for (int i = 1; i < 4; i++) {
        if (ne[i] <= 0 || rows > lim / ne[i]) return false;
        rows *= ne[i];
    }
    if (ne[0] <= 0 || ggml_tsize(type) == 0 || ne[0] % ggml_blck(type) != 0) return false;
    const int64_t rb = (int64_t)ggml_rowsize(type, ne[0]);
    if (rb > lim / rows) return false;
    const int64_t b = rb * rows;
    if (b > left) return false;
    *bytes = (size_t)b;
    return true;
}

// Bytes between the read position of `f` and its end.
inline int64_t stream_left(std::istream &f) {
    const std::streamoff cur = f.tellg();
    f.seekg(0, std::ios::end);
    const std::streamoff end = f.tellg();
    f.seekg(cur, std::ios::beg);
    return cur < 0 || end < cur ? 0 : (int64_t)(end - cur);
}

// ggml reference quantizers (ggml_quantize_chunk with no importance matrix),
// the ones examples/quantize.cpp:244-245 runs on model weights.
void quantize_q4_0(const float *x, uint8_t *y, int64_t k);
void quantize_q4_1(const float *x, uint8_t *y, int64_t k);
void quantize_q8_0(const float *x, uint8_t *y, int64_t k);
// ggml to_float of a row.
void dequantize_row(int type, const uint8_t *x, float *y, int64_t k);

}  // namespace s3e
