// k_rows.hip — row kernels: LayerNorm fused with the conversion of its output
// into the next GEMM's activation format, plain activation quantization, the
// patch-embed im2col, and the f32→fp16 repack used by the stand-alone
// flash-attention entry point.
#include "s3e_internal.h"

namespace s3e {
namespace {

__device__ __forceinline__ uint16_t f2h_bits(float v) { return half_bits(v); }

// A double moved by a DPP pattern within 16-lane rows (both 32-bit halves).
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, (uint64_t)lo | ((uint64_t)hi << 32));
}
__device__ __forceinline__ double swz16_d(double v) {  // lane ^ 16 within each 32-lane half
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_swizzle((int)(uint32_t)u, 0x401F);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_swizzle((int)(uint32_t)(u >> 32), 0x401F);
    return __builtin_bit_cast(double, (uint64_t)lo | ((uint64_t)hi << 32));
}

// Sum over the wave's 64 lanes, in every lane: DPP within rows of 16 (quad
// xor 1, quad xor 2, half-row mirror, row mirror), a swizzle across the rows
// of each half, a permute across the halves.  Only the last two wait on LDS.
__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_d<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_d<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_d<0x141>(v);  // row_half_mirror
    v += dpp_d<0x140>(v);  // row_mirror
    v += swz16_d(v);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// Write 4 consecutive values (columns col..col+3, col % 4 == 0) in the
// activation format.  For the Q8 formats the 8 lanes 8k..8k+7 of the wave
// must hold the 8 float4 of one 32-element block, in order.
__device__ __forceinline__ void emit4(const float *v, const Act &o, int64_t row, int64_t col, int lane) {
    if (o.kind == A_F32) {
        *(float4 *)((float *)o.x + row * o.ld + col) = make_float4(v[0], v[1], v[2], v[3]);
        return;
    }
    if (o.kind == A_F16 || o.kind == A_F16X2) {
        _Float16 h[4];
#pragma unroll
        for (int i = 0; i < 4; i++) h[i] = to_half(v[i]);
        auto pack = [](_Float16 a, _Float16 b) {
            return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
        };
        *(uint2 *)((_Float16 *)o.x + row * o.ld + col) = make_uint2(pack(h[0], h[1]), pack(h[2], h[3]));
        if (o.kind == A_F16X2) {
            // low half: fp16 of the exact fp32 difference
            _Float16 l[4];
#pragma unroll
            for (int i = 0; i < 4; i++) l[i] = (_Float16)(v[i] - (float)h[i]);
            *(uint2 *)((_Float16 *)o.lo + row * o.ld + col) = make_uint2(pack(l[0], l[1]), pack(l[2], l[3]));
        }
        return;
    }
    // Q8_0 / Q8_1 as ggml's x86 quantize_row_q8_0 / q8_1: d = amax/127,
    // id = 127/amax, q = round-half-even(v·id), s = fp16(d·Σq).
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const float d = amax / 127.f;
    const float id = (amax != 0.f) ? 127.f / amax : 0.f;
    if (o.kind == A_F6) {
        // the same codes, split q = 16·h + l; lane k of the block's 8 holds
        // bits [24k, 24k + 24) of each part's 192-bit operand string, and
        // lanes 0-5 of the 8 each assemble and store one 8-byte word
        uint32_t ph = 0, pl = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = (int)__builtin_rintf(v[i] * id);
            const int h = f6_hi(q);
            ph |= f6_code(h) << (6 * i);
            pl |= f6_code(q - 16 * h) << (6 * i);
        }
        const int g = lane & ~7, k = lane & 7;
        uint32_t x[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t a = __shfl(ph, g + j, 64), b = __shfl(pl, g + j, 64);
            x[j] = k < 3 ? a : b;
        }
        if (k < 6) {
            const int t = k % 3;
            uint64_t w;
            if (t == 0) w = (uint64_t)x[0] | ((uint64_t)x[1] << 24) | ((uint64_t)(x[2] & 0xFFFFu) << 48);
            else if (t == 1) w = (uint64_t)(x[2] >> 16) | ((uint64_t)x[3] << 8) | ((uint64_t)x[4] << 32) | ((uint64_t)(x[5] & 0xFFu) << 56);
            else w = (uint64_t)(x[5] >> 8) | ((uint64_t)x[6] << 16) | ((uint64_t)x[7] << 40);
            ((uint64_t *)o.x)[f6_act_word(o.ld / 128, row, col / QK, k / 3, t)] = w;
        }
        if (k == 0) o.d[scale_index(o.mp, row, col / QK)] = f2h_bits(d);
        return;
    }
    int sum = 0;
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = (int)__builtin_rintf(v[i] * id);
        sum += q;
        packed |= ((uint32_t)(q & 0xff)) << (8 * i);
    }
    *(uint32_t *)((int8_t *)o.x + row * o.ld + col) = packed;
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    if ((lane & 7) == 0) {
        const int64_t blk = scale_index(o.mp, row, col / QK);
        o.d[blk] = f2h_bits(d);
        // s = fp16(fp32(d·Σq)): f2h_bits keeps the fp32 rounding of the product
        if (o.kind == A_Q8_1) o.s[blk] = f2h_bits(d * (float)sum);
    }
}

// One wave per row; lane L holds float4 number L + 64·it of the row
// (it < NIT = ceil(E / 256)), so every load and store of the wave is one
// contiguous run.
template <int NIT>
__global__ __launch_bounds__(256) void k_layernorm(const float *__restrict__ x, int64_t M, int64_t E,
                                                   float eps, const float *__restrict__ w,
                                                   const float *__restrict__ b, Act o,
                                                   float *__restrict__ y32) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const int nf4 = (int)(E / 4);
    const float4 *xr = (const float4 *)(x + row * E);
    float v[NIT][4];
    // ggml_norm: mean and variance accumulated in double, each rounded to
    // float once; centred values and squares in float.  With double sums the
    // summation order no longer shows in the float results, so the output
    // matches the CPU path bit for bit.
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int f = lane + 64 * it;
        const float4 q = (f < nf4) ? xr[f] : make_float4(0.f, 0.f, 0.f, 0.f);
        v[it][0] = q.x; v[it][1] = q.y; v[it][2] = q.z; v[it][3] = q.w;
    }
    double s = 0.0;
#pragma unroll
    for (int it = 0; it < NIT; it++)
#pragma unroll
        for (int j = 0; j < 4; j++) s += (double)v[it][j];
    s = wave_sum_d(s);
    const float mean = (float)(s / (double)E);
    double s2 = 0.0;
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const bool ok = lane + 64 * it < nf4;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float c = __fsub_rn(v[it][j], mean);
            v[it][j] = c;
            if (ok) s2 += (double)__fmul_rn(c, c);
        }
    }
    s2 = wave_sum_d(s2);
    const float var = (float)(s2 / (double)E);
    const float scale = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int f = lane + 64 * it;
        if (64 * it >= nf4) break;  // whole wave past the row (nf4 is a multiple of 8)
        if (f < nf4) {
            const float4 wf = w ? ((const float4 *)w)[f] : make_float4(1.f, 1.f, 1.f, 1.f);
            const float4 bf = b ? ((const float4 *)b)[f] : make_float4(0.f, 0.f, 0.f, 0.f);
            const float wv[4] = {wf.x, wf.y, wf.z, wf.w}, bv[4] = {bf.x, bf.y, bf.z, bf.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float t = __fmul_rn(v[it][j], scale);
                if (w) t = __fmul_rn(t, wv[j]);
                if (b) t = __fadd_rn(t, bv[j]);
                v[it][j] = t;
            }
        }
        // the 8 lanes of a Q8 block are all inside or all past the row
        if (f < nf4) {
            if (y32) *(float4 *)(y32 + row * E + 4 * f) = make_float4(v[it][0], v[it][1], v[it][2], v[it][3]);
            else emit4(v[it], o, row, 4 * (int64_t)f, lane);
        }
    }
}

// LayerNorm straight into A_F6 (E % 128 == 0, E ≤ 1024·NIT): a work-group
// normalizes 16 consecutive rows (each wave LNF6_ROWS / LNF6_WAVES of them, the
// next row's values loaded while one is converted), lane L of a wave holding the
// 16 consecutive
// values [16·(L + 64·it), +16), half L & 1 of one 32-element block.  Each
// lane converts its half with one fp6 pack instruction (h codes in slots
// 0-15, l codes in 16-31) and leaves its bits in LDS in the output's order;
// the work-group then writes every (block, part, word) run of its 16 rows
// (128 contiguous bytes in A_F6) and every stage's 16 rows of block scales
// as whole lines.  The same statistics and per-element operations as
// k_layernorm, so the same codes.
constexpr int LNF6_ROWS = 16;
// waves per work-group, LNF6_ROWS / LNF6_WAVES rows each: one row per wave
// (no chain of dependent row loads; 5184 rows: 11.42 → 11.33 ms per ViT frame
// against four rows per wave)
constexpr int LNF6_WAVES = 16;
constexpr int LNF6_BSTRIDE = 98;  // 8-byte LDS words per block: 6 runs of 16 rows, padded (bank spread, 16 B aligned)

template <int NIT, bool WB, int LNW>
__global__ __launch_bounds__(64 * LNW) void k_layernorm_f6(const float *__restrict__ x, int64_t M, int64_t E,
                                                      float eps, const float *__restrict__ w,
                                                      const float *__restrict__ b, Act o) {
    __shared__ __attribute__((aligned(16))) uint64_t stg[32 * NIT * LNF6_BSTRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t stgd[8 * NIT][LNF6_ROWS][4];
    // gamma and beta, read once per work-group (every wave's row uses all of them)
    __shared__ __attribute__((aligned(16))) float swb[WB ? 2 * 1024 * NIT : 4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nseg = (int)(E / 16), nblk = (int)(E / 32);
    const int64_t r0 = (int64_t)blockIdx.x * LNF6_ROWS;
    uint32_t *stg32 = (uint32_t *)stg;
    // pairwise sums in double (exact enough that the order never shows in
    // the float results)
    auto dsum16 = [](const float *a) {
        double t[8];
#pragma unroll
        for (int j = 0; j < 8; j++) t[j] = (double)a[2 * j] + (double)a[2 * j + 1];
#pragma unroll
        for (int j = 0; j < 4; j++) t[j] += t[j + 4];
        return (t[0] + t[2]) + (t[1] + t[3]);
    };
    float nx[NIT][16];
    auto load_row = [&](int64_t r) {
        const float4 *xr = (const float4 *)(x + r * E);
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int seg = lane + 64 * it;
            if (seg < nseg) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float4 q = xr[4 * seg + j];
                    nx[it][4 * j] = q.x; nx[it][4 * j + 1] = q.y; nx[it][4 * j + 2] = q.z; nx[it][4 * j + 3] = q.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 16; j++) nx[it][j] = 0.f;
            }
        }
    };
    constexpr int RPW = LNF6_ROWS / LNW;  // rows per wave
    if (r0 + wave * RPW < M) load_row(r0 + wave * RPW);
    if constexpr (WB) {
        for (int i = threadIdx.x; i < (int)E / 4; i += 64 * LNW) {
            ((float4 *)swb)[i] = ((const float4 *)w)[i];
            ((float4 *)swb)[256 * NIT + i] = ((const float4 *)b)[i];
        }
        __syncthreads();
    }
    for (int k = 0; k < RPW; k++) {
        const int rr = wave * RPW + k;  // row within the group
        const int64_t row = r0 + rr;
        if (row >= M) break;
        float v[NIT][16];
#pragma unroll
        for (int it = 0; it < NIT; it++)
#pragma unroll
            for (int j = 0; j < 16; j++) v[it][j] = nx[it][j];
        if (k + 1 < RPW && row + 1 < M) load_row(row + 1);
        double s = 0.0;
#pragma unroll
        for (int it = 0; it < NIT; it++) s += dsum16(v[it]);
        s = wave_sum_d(s);
        const float mean = (float)(s / (double)E);
        double s2 = 0.0;
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            float sq[16];
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const float c = __fsub_rn(v[it][j], mean);
                v[it][j] = c;
                sq[j] = __fmul_rn(c, c);
            }
            if (lane + 64 * it < nseg) s2 += dsum16(sq);
        }
        s2 = wave_sum_d(s2);
        const float var = (float)(s2 / (double)E);
        const float scale = 1.0f / sqrtf(var + eps);
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int seg = lane + 64 * it;
            if (64 * it >= nseg) break;  // whole wave past the row
            // both lanes of a block are inside the row or both past it (nseg is even)
            if (seg >= nseg) continue;
            float amax = 0.f;
#pragma unroll
            for (int j4 = 0; j4 < 4; j4++) {
                float wv[4] = {1.f, 1.f, 1.f, 1.f}, bv[4] = {0.f, 0.f, 0.f, 0.f};
                if constexpr (WB) {
                    const float4 wf = ((const float4 *)swb)[4 * seg + j4];
                    const float4 bf = ((const float4 *)swb)[256 * NIT + 4 * seg + j4];
                    wv[0] = wf.x; wv[1] = wf.y; wv[2] = wf.z; wv[3] = wf.w;
                    bv[0] = bf.x; bv[1] = bf.y; bv[2] = bf.z; bv[3] = bf.w;
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float t = __fmul_rn(v[it][4 * j4 + j], scale);
                    if constexpr (WB) t = __fadd_rn(__fmul_rn(t, wv[j]), bv[j]);
                    v[it][4 * j4 + j] = t;
                    amax = fmaxf(amax, fabsf(t));
                }
            }
            amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                              0, __builtin_bit_cast(int, amax), 0xB1, 0xF, 0xF, false)));
            const float id = (amax != 0.f) ? 127.f / amax : 0.f;
            // one conversion for both parts: slots 0-15 take this lane's h
            // codes, slots 16-31 its l codes, so result dwords 0-2 are its 96
            // bits of the h string and dwords 3-5 its 96 bits of the l string
            f32x16 ev, od;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float a, c, e, g;
                f6_split(v[it][2 * i], id, a, c);
                f6_split(v[it][2 * i + 1], id, e, g);
                ev[i] = a;
                od[i] = e;
                ev[8 + i] = c;
                od[8 + i] = g;
            }
            const u32x6 r6 = pack_bf6(ev, od);
            const int blk = seg >> 1;
            // LDS word of (block, part p, word t, row rr): blk·98 + (3p + t)·16 + rr
            const int wb = blk * LNF6_BSTRIDE + rr;
            if ((seg & 1) == 0) {
                // bits [0, 96) of the block string: word 0 and the low half of word 1
                stg[wb] = (uint64_t)r6[0] | ((uint64_t)r6[1] << 32);
                stg32[2 * (wb + 16)] = r6[2];
                stg[wb + 48] = (uint64_t)r6[3] | ((uint64_t)r6[4] << 32);
                stg32[2 * (wb + 64)] = r6[5];
                stgd[blk >> 2][rr][blk & 3] = f2h_bits(amax / 127.f);
            } else {
                // bits [96, 192): the high half of word 1 and word 2
                stg32[2 * (wb + 16) + 1] = r6[0];
                stg[wb + 32] = (uint64_t)r6[1] | ((uint64_t)r6[2] << 32);
                stg32[2 * (wb + 64) + 1] = r6[3];
                stg[wb + 80] = (uint64_t)r6[4] | ((uint64_t)r6[5] << 32);
            }
        }
    }
    __syncthreads();
    // (block, part, word) runs: 16 rows × 8 bytes at f6_act_word(.., r0, ..);
    // 16-byte pieces of rows 2q, 2q + 1 (rows past M land in the padded rows
    // of the 64-row tile, which no product stores)
    const int64_t nst = o.ld / 128;
    const int npieces = nblk * 6 * 8;
    for (int pc = threadIdx.x; pc < npieces; pc += 64 * LNW) {
        const int run = pc >> 3, q = pc & 7;
        const int blk = run / 6, pt = run % 6;
        if (r0 + 2 * q >= M) continue;
        const uint4 val = *(const uint4 *)(stg + blk * LNF6_BSTRIDE + pt * 16 + 2 * q);
        *(uint4 *)((uint64_t *)o.x + f6_act_word(nst, r0, blk, pt / 3, pt % 3) + 2 * q) = val;
    }
    // block scales: per stage, 16 rows × 4 fp16 = 128 contiguous bytes
    for (int pc = threadIdx.x; pc < (nblk / 4) * 8; pc += 64 * LNW) {
        const int sg = pc >> 3, q = pc & 7;
        if (r0 + 2 * q >= M) continue;
        *(uint4 *)(o.d + scale_index(o.mp, r0 + 2 * q, 4 * sg)) = *(const uint4 *)&stgd[sg][2 * q][0];
    }
}

// Plain conversion of f32 rows into an activation format (ggml from_float):
// lane L of a wave converts float4 number 64·blockIdx.x + L of its row.
__global__ __launch_bounds__(256) void k_rows_quant(const float *__restrict__ x, int64_t M, int64_t K, Act o) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.y * 4 + (threadIdx.x >> 6);
    const int64_t f = (int64_t)blockIdx.x * 64 + lane;
    if (row >= M) return;
    // Q8: K % 32 == 0, so the 8 lanes of a block are all inside or all past the row
    if (f >= K / 4) {
        // blocks between K and the next multiple of 128 get zero scales: the
        // GEMM reads whole groups of four blocks
        const int64_t f4 = (K + 127) / 128 * 32;
        if (f < f4 && (lane & 7) == 0 && (o.kind == A_Q8_0 || o.kind == A_Q8_1)) {
            const int64_t blk = scale_index(o.mp, row, f / 8);
            o.d[blk] = 0;
            if (o.kind == A_Q8_1) o.s[blk] = 0;
        }
        return;
    }
    const float4 q = ((const float4 *)(x + row * K))[f];
    const float v[4] = {q.x, q.y, q.z, q.w};
    emit4(v, o, row, 4 * f, lane);
}

// im2col for ggml_conv_2d_sk_p0 with a P×P kernel and stride P on a CHW image:
// row t = py*G + px, column k = (c*P + ky)*P + kx, zero for k >= 3·P².
__global__ void k_im2col(const float *__restrict__ chw, int img, int P, int64_t ldk, int kind,
                         void *out, _Float16 *lo) {
    // 32-bit index arithmetic (the launcher keeps G²·ldk below 2^31)
    const int G = img / P;
    const uint32_t T = (uint32_t)(G * G);
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= T * (uint32_t)ldk) return;
    const uint32_t t = idx / (uint32_t)ldk;
    const int k = (int)(idx - t * (uint32_t)ldk);
    float val = 0.f;
    if (k < 3 * P * P) {
        const int c = k / (P * P), r = k % (P * P), ky = r / P, kx = r % P;
        const int py = (int)(t / (uint32_t)G), px = (int)(t - (uint32_t)py * G);
        val = chw[(int64_t)c * img * img + (int64_t)(py * P + ky) * img + px * P + kx];
    }
    if (kind == A_F16 || kind == A_F16X2) {
        const _Float16 h = to_half(val);
        ((_Float16 *)out)[idx] = h;
        if (kind == A_F16X2) lo[idx] = (_Float16)(val - (float)h);  // fp16 of the exact difference
    } else {
        ((float *)out)[idx] = val;
    }
}

// f32 strided Q/K/V (head dim D) → fp16 [BH][N][hdp] for Q and K,
// [BH][hdp][ldt] for V (keys in vt_slot order), channels D..hdp−1 zero.
// With lo != null the value is stored as the pair hi = fp16(v),
// lo = fp16(v − hi) for split-precision attention.
__global__ void k_attn_prep(const float *__restrict__ src, int64_t s1, int64_t s2, int64_t s3,
                            int64_t N, int64_t nh, int64_t B, int D, int hdp, _Float16 *__restrict__ dst,
                            _Float16 *__restrict__ lo, int64_t ldt, int transpose) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = B * nh * N * hdp;
    if (idx >= total) return;
    const int64_t d = idx % hdp;
    const int64_t i = (idx / hdp) % N;
    const int64_t h = (idx / (hdp * N)) % nh;
    const int64_t b = idx / (hdp * N * nh);
    const float v = d < D ? src[b * s3 + h * s2 + i * s1 + d] : 0.f;
    const int64_t bh = b * nh + h;
    const int64_t o = transpose ? (bh * hdp + d) * ldt + vt_slot(i) : (bh * N + i) * hdp + d;
    const _Float16 hv = to_half(v);
    dst[o] = hv;
    if (lo) lo[o] = (_Float16)(v - (float)hv);
}

// fp16 strided rows (head dim D) → fp16 [BH][N][hdp], channels D..hdp−1 zero
// (Q or K of s3e_flash_attn_ext_f16 when they are not already in that
// layout).  One thread per output element.
__global__ void k_attn_prep16(const _Float16 *__restrict__ src, int64_t s1, int64_t s2, int64_t s3, int64_t N,
                              int64_t nh, int64_t B, int D, int hdp, _Float16 *__restrict__ dst) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= B * nh * N * hdp) return;
    const int64_t d = idx % hdp, i = (idx / hdp) % N, h = (idx / (hdp * N)) % nh, b = idx / (hdp * N * nh);
    dst[idx] = d < D ? src[b * s3 + h * s2 + i * s1 + d] : (_Float16)0.f;
}

// fp16 V (key j of head h of batch b at v[b*s3 + h*s2 + j*s1 + d]) → Vᵀ
// [BH][hdp][ldv], keys in vt_slot order, zero past Nkv and for d ≥ D.  One
// thread per 8 slots × 8 channels: it reads the 8 keys those slots hold (16
// bytes of channels each; VEC: one 16-byte load per key, else element by
// element) and writes the 8 channel rows' 16-byte runs, transposing in
// registers.  Slots 8c .. 8c + 7 of a 16-key group hold keys {0-3, 8-11}
// (c even) or {4-7, 12-15} (c odd) of it.
template <bool VEC>
__global__ __launch_bounds__(256) void k_vt16(const _Float16 *__restrict__ v, int64_t s1, int64_t s2, int64_t s3,
                                              int64_t Nkv, int64_t nh, int D, int hdp, int64_t ldv,
                                              _Float16 *__restrict__ vt, int64_t total) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int dch = hdp / 8;
    const int64_t nsc = ldv / 8;
    const int d0 = (int)(t % dch) * 8;
    const int64_t sc = (t / dch) % nsc, bh = t / (dch * nsc);
    const _Float16 *vb = v + (bh / nh) * s3 + (bh % nh) * s2;
    const int64_t kbase = (sc >> 1) * 16 + (sc & 1) * 4;
    _Float16 x[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int64_t key = kbase + (i & 3) + (i >> 2) * 8;
        if (VEC && key < Nkv && d0 + 8 <= D) {
            *(uint4 *)x[i] = *(const uint4 *)(vb + key * s1 + d0);
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) x[i][j] = (key < Nkv && d0 + j < D) ? vb[key * s1 + d0 + j] : (_Float16)0.f;
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        _Float16 run[8];
#pragma unroll
        for (int i = 0; i < 8; i++) run[i] = x[i][j];
        *(uint4 *)(vt + (bh * hdp + d0 + j) * ldv + 8 * sc) = *(const uint4 *)run;
    }
}

// NHWC f32 pixels → fp16 / split-fp16 activation rows, optionally through
// the 2×2 stride-2 max pool (ggml_pool_2d MAX, sam3.cpp:3914): one thread per
// 4 channels of an output pixel.
__global__ __launch_bounds__(256) void k_pool_act(const float *__restrict__ x, int w, int c, int pool, int ow,
                                                  int64_t n4, Act o) {
    // 32-bit index arithmetic (the launcher keeps n4 below 2^31)
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint32_t)n4) return;
    const uint32_t c4 = c / 4;
    const uint32_t pix32 = i / c4;
    const int64_t pix = pix32;
    const int cc = (int)(i - pix32 * c4) * 4;
    float4 v;
    if (pool == 1) {
        v = *(const float4 *)(x + pix * c + cc);
    } else {
        const int64_t oy = pix32 / (uint32_t)ow, ox = pix - oy * ow;
        const float *p0 = x + ((2 * oy) * w + 2 * ox) * c + cc;
        const float4 a = *(const float4 *)p0, b = *(const float4 *)(p0 + c);
        const float4 d = *(const float4 *)(p0 + (int64_t)w * c), e = *(const float4 *)(p0 + (int64_t)w * c + c);
        v.x = fmaxf(fmaxf(a.x, b.x), fmaxf(d.x, e.x));
        v.y = fmaxf(fmaxf(a.y, b.y), fmaxf(d.y, e.y));
        v.z = fmaxf(fmaxf(a.z, b.z), fmaxf(d.z, e.z));
        v.w = fmaxf(fmaxf(a.w, b.w), fmaxf(d.w, e.w));
    }
    const float vv[4] = {v.x, v.y, v.z, v.w};
    emit4(vv, o, pix, cc, 0);
}

}  // namespace

hipError_t launch_pool_act(const float *x, int h, int w, int c, int pool, const Act &out, hipStream_t st) {
    if ((pool != 1 && pool != 2) || c % 4 != 0 || (out.kind != A_F16 && out.kind != A_F16X2 && out.kind != A_F32) ||
        out.ld != c || h < pool || w < pool)
        return hipErrorInvalidValue;
    const int oh = pool == 1 ? h : (h - 2) / 2 + 1, ow = pool == 1 ? w : (w - 2) / 2 + 1;
    const int64_t n4 = (int64_t)oh * ow * (c / 4);
    if (n4 >= INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pool_act, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, x, w, c, pool, ow, n4, out);
    return hipGetLastError();
}

hipError_t launch_layernorm(const float *x, int64_t M, int64_t E, float eps, const float *w,
                            const float *b, const Act &out, float *y_f32, hipStream_t st) {
    // float4 lanes; a Q8 block must be whole inside the row
    const bool q8 = !y_f32 && (out.kind == A_Q8_0 || out.kind == A_Q8_1);
    const bool f6 = !y_f32 && out.kind == A_F6;
    if (E % 4 != 0 || E > 4096 || (q8 && E % 32 != 0) || (f6 && (E % 128 != 0 || out.ld != E))) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((M + 3) / 4));
    if (f6 && E <= 1024 && (w != nullptr) == (b != nullptr)) {
        // rows of up to 1024 (the ViT's); the ViT's norms carry both gamma and
        // beta (sam3_layer_norm, sam3.cpp:1037-1046)
        const dim3 gf((unsigned)((M + LNF6_ROWS - 1) / LNF6_ROWS));
        constexpr int W = LNF6_WAVES;
        if (w) hipLaunchKernelGGL((k_layernorm_f6<1, true, W>), gf, dim3(64 * W), 0, st, x, M, E, eps, w, b, out);
        else hipLaunchKernelGGL((k_layernorm_f6<1, false, W>), gf, dim3(64 * W), 0, st, x, M, E, eps, w, b, out);
        return hipGetLastError();
    }
    if (E <= 256) hipLaunchKernelGGL(k_layernorm<1>, grid, dim3(256), 0, st, x, M, E, eps, w, b, out, y_f32);
    else if (E <= 512) hipLaunchKernelGGL(k_layernorm<2>, grid, dim3(256), 0, st, x, M, E, eps, w, b, out, y_f32);
    else if (E <= 1024) hipLaunchKernelGGL(k_layernorm<4>, grid, dim3(256), 0, st, x, M, E, eps, w, b, out, y_f32);
    else if (E <= 2048) hipLaunchKernelGGL(k_layernorm<8>, grid, dim3(256), 0, st, x, M, E, eps, w, b, out, y_f32);
    else hipLaunchKernelGGL(k_layernorm<16>, grid, dim3(256), 0, st, x, M, E, eps, w, b, out, y_f32);
    return hipGetLastError();
}

hipError_t launch_rows_quant(AKind kind, const float *x, int64_t M, int64_t K, const Act &out,
                             hipStream_t st) {
    (void)kind;
    // a Q8 block must be whole inside the row; other formats go by float4
    const bool q8 = out.kind == A_Q8_0 || out.kind == A_Q8_1;
    if ((q8 && K % 32 != 0) || K % 4 != 0 || (out.kind == A_F6 && (K % 128 != 0 || out.ld != K)))
        return hipErrorInvalidValue;
    if (M <= 0) return hipSuccess;  // no rows: a launch would have an empty grid
    const int64_t nf4 = (K + 127) / 128 * 32;  // float4 up to the 128-element group
    const dim3 grid((unsigned)((nf4 + 63) / 64), (unsigned)((M + 3) / 4));
    hipLaunchKernelGGL(k_rows_quant, grid, dim3(256), 0, st, x, M, K, out);
    return hipGetLastError();
}

hipError_t launch_im2col(const float *chw, int img, int P, int64_t ldk, AKind kind, void *out,
                         hipStream_t st, void *lo) {
    if (kind == A_F16X2 && !lo) return hipErrorInvalidValue;
    const int G = img / P;
    const int64_t total = (int64_t)G * G * ldk;
    if (total >= INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_im2col, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, chw, img, P,
                       ldk, (int)kind, out, (_Float16 *)lo);
    return hipGetLastError();
}

hipError_t launch_attn_prep(const float *q, const int64_t q_nb[4], const float *k,
                            const int64_t k_nb[4], const float *v, const int64_t v_nb[4],
                            int64_t Nq, int64_t Nkv, int64_t nh, int64_t B, int D, int hdp, _Float16 *q16,
                            _Float16 *k16, _Float16 *vt16, _Float16 *q_lo, _Float16 *k_lo,
                            _Float16 *vt_lo, int64_t ldv, hipStream_t st) {
    if (D <= 0 || D > hdp) return hipErrorInvalidValue;
    const int64_t tq = B * nh * Nq * hdp, tk = B * nh * Nkv * hdp;
    hipLaunchKernelGGL(k_attn_prep, dim3((unsigned)((tq + 255) / 256)), dim3(256), 0, st, q, q_nb[1],
                       q_nb[2], q_nb[3], Nq, nh, B, D, hdp, q16, q_lo, (int64_t)0, 0);
    hipLaunchKernelGGL(k_attn_prep, dim3((unsigned)((tk + 255) / 256)), dim3(256), 0, st, k, k_nb[1],
                       k_nb[2], k_nb[3], Nkv, nh, B, D, hdp, k16, k_lo, (int64_t)0, 0);
    hipLaunchKernelGGL(k_attn_prep, dim3((unsigned)((tk + 255) / 256)), dim3(256), 0, st, v, v_nb[1],
                       v_nb[2], v_nb[3], Nkv, nh, B, D, hdp, vt16, vt_lo, ldv, 1);
    return hipGetLastError();
}

hipError_t launch_attn_prep16(const _Float16 *q, const int64_t q_nb[4], const _Float16 *k, const int64_t k_nb[4],
                              const _Float16 *v, const int64_t v_nb[4], int64_t Nq, int64_t Nkv, int64_t nh,
                              int64_t B, int D, int hdp, _Float16 *q16, _Float16 *k16, _Float16 *v16,
                              _Float16 *vt16, int64_t ldv, hipStream_t st) {
    if (D <= 0 || D > hdp || hdp > 256 || (vt16 && (ldv % 16 != 0 || ldv < Nkv))) return hipErrorInvalidValue;
    if (q16) {
        const int64_t t = B * nh * Nq * hdp;
        hipLaunchKernelGGL(k_attn_prep16, dim3((unsigned)((t + 255) / 256)), dim3(256), 0, st, q, q_nb[1], q_nb[2],
                           q_nb[3], Nq, nh, B, D, hdp, q16);
    }
    if (k16) {
        const int64_t t = B * nh * Nkv * hdp;
        hipLaunchKernelGGL(k_attn_prep16, dim3((unsigned)((t + 255) / 256)), dim3(256), 0, st, k, k_nb[1], k_nb[2],
                           k_nb[3], Nkv, nh, B, D, hdp, k16);
    }
    if (v16) {
        const int64_t t = B * nh * Nkv * hdp;
        hipLaunchKernelGGL(k_attn_prep16, dim3((unsigned)((t + 255) / 256)), dim3(256), 0, st, v, v_nb[1], v_nb[2],
                           v_nb[3], Nkv, nh, B, D, hdp, v16);
    }
    if (!vt16) return hipGetLastError();
    const int64_t total = B * nh * (ldv / 8) * (hdp / 8);
    const bool vec = ((uintptr_t)v % 16 == 0) && v_nb[1] % 8 == 0 && v_nb[2] % 8 == 0 && v_nb[3] % 8 == 0;
    const dim3 grid((unsigned)((total + 255) / 256));
    if (vec)
        hipLaunchKernelGGL(k_vt16<true>, grid, dim3(256), 0, st, v, v_nb[1], v_nb[2], v_nb[3], Nkv, nh, D, hdp, ldv,
                           vt16, total);
    else
        hipLaunchKernelGGL(k_vt16<false>, grid, dim3(256), 0, st, v, v_nb[1], v_nb[2], v_nb[3], Nkv, nh, D, hdp, ldv,
                           vt16, total);
    return hipGetLastError();
}

}  // namespace s3e

namespace s3e {
namespace {

// Streaming 16-byte copy, grid-stride (used to calibrate HBM byte counters).
__global__ __launch_bounds__(256) void k_copy(uint4 *__restrict__ dst, const uint4 *__restrict__ src, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

// y = a + b·s (ggml_scale, then ggml_add: the product is rounded first)
__global__ __launch_bounds__(256) void k_add_scaled(float *__restrict__ y, const float *__restrict__ a,
                                                    const float *__restrict__ b, float s, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = __fadd_rn(a[i], __fmul_rn(b[i], s));
}

}  // namespace

hipError_t launch_add_scaled(float *y, const float *a, const float *b, float s, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_add_scaled, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, y, a, b, s, n);
    return hipGetLastError();
}

hipError_t launch_copy(void *dst, const void *src, size_t bytes, hipStream_t st) {
    const int64_t n = (int64_t)(bytes / 16);
    const int64_t blocks = n / 256 + 1 < 8192 ? n / 256 + 1 : 8192;
    hipLaunchKernelGGL(k_copy, dim3((unsigned)blocks), dim3(256), 0, st, (uint4 *)dst, (const uint4 *)src, n);
    return hipGetLastError();
}

}  // namespace s3e

// ---- sub-stage hooks (sam3_test_run_vit_block_stage / _prefix_stage) ----------
// The fused encoder never materialises these intermediates; the hooks do,
// with the same device arithmetic the fused epilogues use.
namespace s3e {
namespace {

// ggml_gelu_erf on f32, the device gelu_erf of the fc1 epilogue.
__global__ __launch_bounds__(256) void k_gelu_rows(const float *__restrict__ x, float *__restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = gelu_erf(x[i]);
}

// ggml_win_part / ggml_win_unpart on rows of E (E % 4 == 0): window
// w = wy·npx + wx of WS×WS positions, zero rows where a window leaves the
// W0×H0 grid (partition only).  One thread per float4.
__global__ __launch_bounds__(256) void k_win_perm(const float4 *__restrict__ x, float4 *__restrict__ y, int W0,
                                                  int H0, int WS, int64_t e4, int64_t n, int part) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t r = i / e4, c = i - r * e4;  // window row r = w·WS² + p
    const int64_t npx = (W0 + WS - 1) / WS;
    const int64_t w = r / ((int64_t)WS * WS), p = r - w * WS * WS;
    const int64_t gx = (w % npx) * WS + p % WS, gy = (w / npx) * WS + p / WS;
    const bool inside = gx < W0 && gy < H0;
    const int64_t t = gy * W0 + gx;
    if (part) y[i] = inside ? x[t * e4 + c] : make_float4(0.f, 0.f, 0.f, 0.f);
    else if (inside) y[t * e4 + c] = x[i];
}

// Q and K of the ViT attention core from qkv rows [B·N][3E] (bias added):
// q|k column thirds, heads of HD; RoPE as sam3_apply_rope (each product
// rounded, then the difference / sum, as the EPI_QKV epilogue computes it);
// out [2][B][NH][N][HD] f32.  One thread per (re, im) pair.
__global__ __launch_bounds__(256) void k_vit_rope_split(const float *__restrict__ qkv, const float *__restrict__ freqs,
                                                        float *__restrict__ out, int64_t B, int64_t N, int NH, int HD,
                                                        int64_t npairs) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= npairs) return;
    const int half = HD / 2;
    const int64_t E = (int64_t)NH * HD;
    const int j = (int)(i % half);
    const int64_t p = (i / half) % N, h = (i / ((int64_t)half * N)) % NH;
    const int64_t b = (i / ((int64_t)half * N * NH)) % B, sel = i / ((int64_t)half * N * NH * B);
    const float *src = qkv + (b * N + p) * 3 * E + sel * E + h * HD + 2 * j;
    float re = src[0], im = src[1];
    if (freqs) {
        const float c = freqs[(p * half + j) * 2], s = freqs[(p * half + j) * 2 + 1];
        const float r2 = __fsub_rn(__fmul_rn(re, c), __fmul_rn(im, s));
        const float i2 = __fadd_rn(__fmul_rn(re, s), __fmul_rn(im, c));
        re = r2;
        im = i2;
    }
    float *dst = out + (((sel * B + b) * NH + h) * N + p) * HD + 2 * j;
    dst[0] = re;
    dst[1] = im;
}

// Activation rows (A_F16 or A_F32, row stride ld) → f32 [M][K].
__global__ __launch_bounds__(256) void k_act_f32(const void *__restrict__ x, int kind, int64_t ld, int64_t K,
                                                 int64_t n, float *__restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t r = i / K, c = i - r * K;
    y[i] = kind == A_F16 ? (float)((const _Float16 *)x)[r * ld + c] : ((const float *)x)[r * ld + c];
}

// [R][C] → [C][R] through a 32×33 LDS tile.
__global__ __launch_bounds__(256) void k_transpose(const float *__restrict__ x, float *__restrict__ y, int64_t R,
                                                   int64_t C) {
    __shared__ float tile[32][33];
    const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int k = ty; k < 32; k += 8) {
        const int64_t r = r0 + k, c = c0 + tx;
        if (r < R && c < C) tile[k][tx] = x[r * C + c];
    }
    __syncthreads();
    for (int k = ty; k < 32; k += 8) {
        const int64_t c = c0 + k, r = r0 + tx;
        if (r < R && c < C) y[c * R + r] = tile[tx][k];
    }
}

// ggml_add(x, ggml_repeat(pos [pg][pg][E], [E, G, G])): rows of E, token
// t = row % G² at (t / G, t % G).
__global__ __launch_bounds__(256) void k_add_pos(const float *__restrict__ x, const float *__restrict__ pos,
                                                 float *__restrict__ y, int G, int pg, int64_t E, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t r = i / E, e = i - r * E, t = r % ((int64_t)G * G);
    const int64_t py = t / G, px = t % G;
    y[i] = __fadd_rn(x[i], pos[((py % pg) * pg + px % pg) * E + e]);
}

inline dim3 blocks_for(int64_t n) { return dim3((unsigned)((n + 255) / 256)); }

}  // namespace

hipError_t launch_gelu_rows(const float *x, float *y, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_gelu_rows, blocks_for(n), dim3(256), 0, st, x, y, n);
    return hipGetLastError();
}

hipError_t launch_win_perm(const float *x, float *y, int W0, int H0, int WS, int64_t E, int part, hipStream_t st) {
    if (E % 4 != 0 || WS <= 0 || W0 <= 0 || H0 <= 0) return hipErrorInvalidValue;
    const int64_t nw = (int64_t)((W0 + WS - 1) / WS) * ((H0 + WS - 1) / WS);
    const int64_t n = nw * WS * WS * (E / 4);
    hipLaunchKernelGGL(k_win_perm, blocks_for(n), dim3(256), 0, st, (const float4 *)x, (float4 *)y, W0, H0, WS,
                       E / 4, n, part);
    return hipGetLastError();
}

hipError_t launch_vit_rope_split(const float *qkv, const float *freqs, float *out, int64_t B, int64_t N, int NH,
                                 int HD, hipStream_t st) {
    if (HD % 2 != 0 || B <= 0 || N <= 0) return hipErrorInvalidValue;
    const int64_t np = 2 * B * NH * N * (HD / 2);
    hipLaunchKernelGGL(k_vit_rope_split, blocks_for(np), dim3(256), 0, st, qkv, freqs, out, B, N, NH, HD, np);
    return hipGetLastError();
}

hipError_t launch_act_f32(const Act &a, int64_t M, int64_t K, float *y, hipStream_t st) {
    if (a.kind != A_F16 && a.kind != A_F32) return hipErrorInvalidValue;
    const int64_t n = M * K;
    hipLaunchKernelGGL(k_act_f32, blocks_for(n), dim3(256), 0, st, (const void *)a.x, (int)a.kind, a.ld, K, n, y);
    return hipGetLastError();
}

hipError_t launch_transpose(const float *x, float *y, int64_t R, int64_t C, hipStream_t st) {
    const dim3 grid((unsigned)((C + 31) / 32), (unsigned)((R + 31) / 32));
    hipLaunchKernelGGL(k_transpose, grid, dim3(256), 0, st, x, y, R, C);
    return hipGetLastError();
}

hipError_t launch_add_pos(const float *x, const float *pos, float *y, int G, int pg, int64_t E, int64_t rows,
                          hipStream_t st) {
    const int64_t n = rows * E;
    hipLaunchKernelGGL(k_add_pos, blocks_for(n), dim3(256), 0, st, x, pos, y, G, pg, E, n);
    return hipGetLastError();
}


}  // namespace s3e
