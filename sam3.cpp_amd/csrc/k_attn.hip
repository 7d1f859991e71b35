// k_attn.hip — fused flash attention on gfx950 fp16 MFMA, the engine's
// replacement for ggml_flash_attn_ext (sam3.cpp:3774; isolated core at
// sam3.cpp:6778-6823): O = softmax(scale·QKᵀ)·V, no mask, head dim 64.
//
// Layout: Q, K are fp16 [BH][N][64]; V arrives transposed, fp16
// [BH][64][vt_ld] with keys in vt_slot order, which the QKV GEMM epilogue
// writes directly.  One work-group = 4 waves (one per SIMD) = 128 queries
// of one (batch, head); each wave owns 32 queries, and waves past the last
// query only help move tiles.  The scores are computed
// transposed, Sᵀ = K·Qᵀ (v_mfma_f32_32x32x16_f16, A = 32 keys × 16 d from
// LDS, B = Qᵀ held in registers for the whole kernel), so that in the
// accumulator every lane holds 16 keys of ONE query (column = lane % 32) and
// the softmax statistics are per-lane scalars.  The output is formed
// transposed too, Oᵀ = Vᵀ·Pᵀ: the probabilities go from the Sᵀ accumulator
// registers straight into the B operand (fp16) with no data movement, and the
// keys of each K=16 MFMA step are the ones that lane already holds; thanks to
// the vt_slot order the matching Vᵀ A-operand is one 16-byte LDS read.
// The VN variant (fp16 operands, head dims 64 / 128) reads V as ggml holds
// it, [BH][Nkv][hd]: its tiles are laid out like K tiles, and each Vᵀ
// A-operand is two LDS transpose loads (ds_read_b64_tr_b16), which hand every
// lane one channel of four keys.
//
// K and Vᵀ tiles of 32 keys stream through a 2-deep LDS ring filled by
// buffer_load_dwordx4 ... lds (rows of 128 bytes, 16-byte chunks
// XOR-swizzled by row for the 64-bank LDS): tile j+1 is in flight while tile
// j is used, one barrier per tile.  The tile's position lives in the
// buffer descriptor (scalar registers), so issuing a tile costs no vector
// address arithmetic.
//
// Precision.  SPLIT = false rounds Q, K, V and P to fp16 (fp32 accumulate).
// SPLIT = true carries every operand as an fp16 pair x = hi + lo (hi =
// fp16(x), lo = fp16(x − hi): 22 significant bits) and forms each product
// as hi·hi + hi·lo + lo·hi on MFMA, which reproduces fp32 attention to
// ~1e-7.  Quantized models need SPLIT: the attention output is re-quantized
// to Q8 for the projection GEMM, and an fp16-level error there flips
// rounding decisions, turning a 1e-4 difference into whole quantization
// steps.
//
// Online softmax in the exp2 domain: x = s·scale·log2(e), per-lane running
// reference m and partial sum l.  m is only raised when a tile's maximum
// exceeds it by more than 8 (p ≤ 2^8 meanwhile, well inside fp16 and fp32),
// so the rescale of Oᵀ by exp2(m_old − m_new) is rare; the result is the
// same quotient.  The two lanes sharing a query (l, l^32) agree on m through
// one lane-half swap per tile and add their partial l at the end.
//
// The result leaves the kernel already in the next GEMM's activation format
// (Q8_0 / Q8_1 per 32-d block exactly as ggml quantizes a row, fp16, or
// f32), at row token(b, i) — the window un-partition of sam3.cpp:3784 folded
// into the store address.
#include <type_traits>

#include "s3e_internal.h"

namespace s3e {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

#define LDS_PTR(p) ((__attribute__((address_space(3))) void *)(p))

constexpr int AW = 4;             // waves per work-group (one per SIMD)
constexpr int NTHR = 64 * AW;
constexpr int QT = 32 * AW;       // queries per work-group
constexpr int KT = 32;            // keys per tile

// Geometry by head dimension (64, or 128 for wider heads zero-padded to it).
template <int HD>
struct AG {
    static constexpr int ROWK = HD * 2;        // bytes of one K row
    static constexpr int KPL = KT * ROWK;      // bytes of one K plane of a tile
    static constexpr int VPL = HD * KT * 2;    // bytes of one Vᵀ plane of a tile: HD rows × 32 keys
    static constexpr int KRUNS = KPL / 1024 / AW;  // 1 KB DMA runs per wave per K plane
    static constexpr int VRUNS = VPL / 1024 / AW;  // ... per Vᵀ plane
    static constexpr int DS = HD / 16;         // K=16 steps of Sᵀ
    static constexpr int DT = HD / 32;         // 32-row tiles of Oᵀ
};

__device__ __forceinline__ uint16_t f2h_bits(float v) { return half_bits(v); }

__device__ __forceinline__ v16f mfma(const v8h &a, const v8h &b, const v16f &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// 16-byte chunk c of LDS row r sits at slot c ^ swz(r).  With 64 banks of 4
// bytes, 128-byte K rows r and r+2 share banks (swzk), and 64-byte Vᵀ rows
// r, r+4, r+8, r+12 do (swzv); either way the 16 rows one ds_read_b128 phase
// touches land on distinct banks.
__device__ __forceinline__ int swzk(int r) { return (r >> 1) & 7; }
// 256-byte K rows (HD = 128) each span all 64 banks: 16 consecutive rows need
// 16 distinct slots
__device__ __forceinline__ int swzk256(int r) { return r & 15; }
template <int HD>
__device__ __forceinline__ int swzk_hd(int r) { return HD == 64 ? swzk(r) : swzk256(r); }
__device__ __forceinline__ int swzv(int r) { return (r >> 2) & 3; }
// Natural V tiles (VN): a transpose load reads 64 bytes of each of four
// consecutive rows per lane half, so those rows must land in distinct bank
// groups, and the DMA and the rows' 16-byte chunks stay a bijection.  HD 64
// (128-byte rows, r and r + 2 share banks): the three bits of (r >> 1)
// reversed, which puts rows 4i and 4i + 2 in different 64-byte halves of the
// bank space; HD 128 (256-byte rows): the two low row bits pick the 64-byte
// group.
template <int HD>
__device__ __forceinline__ int swzvn(int r) {
    if constexpr (HD == 64) {
        const int x = (r >> 1) & 7;
        return ((x & 1) << 2) | (x & 2) | (x >> 2);
    } else {
        return ((r & 3) << 2) | ((r >> 2) & 3);
    }
}

typedef __fp16 v4fp16 __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives element
// i % 4 of the 8 bytes addressed by lanes 4j + i / 4, j = 0..3
__device__ __forceinline__ v4h lds_tr16(const uint8_t *p) {
    const v4fp16 r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) v4fp16 *)(p));
    return __builtin_bit_cast(v4h, r);
}

// p − h for the fp16 value h in the low or high half of h2, exact, in one
// v_fma_mix_f32 (h2·(−1) + p with h2 read as fp16)
__device__ __forceinline__ float sub_lo_half(float p, uint32_t h2) {
    float r;
    __asm__("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(p));
    return r;
}
__device__ __forceinline__ float sub_hi_half(float p, uint32_t h2) {
    float r;
    __asm__("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(p));
    return r;
}

// CROP: the windowed, cropped output mapping and narrower real heads
// (a.wo, a.hd_out; the Hiera layouts), kept out of the plain variants.
template <bool SPLIT, int HD, bool CROP, bool VN = false>
__global__ __launch_bounds__(NTHR, HD == 64 ? 3 : (HD == 128 ? 2 : 1)) void k_attn(AttnArgs a, int ldv) {
    static_assert(!VN || (!SPLIT && HD <= 128), "natural V: fp16 operands, head dim 64 or 128");
    using G = AG<HD>;
    constexpr int NP = SPLIT ? 2 : 1;  // planes: hi (and lo)
    constexpr int KPL = G::KPL, VPL = G::VPL;
    constexpr int KBUF = NP * KPL, VBUF = NP * VPL;
    // K ring (2 tiles) then Vᵀ ring (2 tiles)
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * KBUF + 2 * VBUF];

    const int bh = blockIdx.y;
    const int q0 = blockIdx.x * QT;
    const int t = threadIdx.x, lane = t & 63, lr = lane & 31, lh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int qi = q0 + wave * 32 + lr;
    const bool qvalid = qi < a.Nq;

    v8h qf[NP][G::DS];
    {
        const int64_t off = (int64_t)bh * (a.q_hs > 0 ? a.q_hs : (int64_t)a.Nq * HD) + (int64_t)(qvalid ? qi : 0) * HD;
#pragma unroll
        for (int pl = 0; pl < NP; pl++) {
            const _Float16 *qrow = (pl == 0 ? a.q : a.q_lo) + off;
#pragma unroll
            for (int ds = 0; ds < G::DS; ds++) {
                v8h z = {};
                qf[pl][ds] = qvalid ? *(const v8h *)(qrow + ds * 16 + lh * 8) : z;
            }
        }
    }
    const float c = a.scale * 1.44269504088896340736f;
    float mrun = -INFINITY, lsum = 0.f;
    v16f o[G::DT];
#pragma unroll
    for (int dt = 0; dt < G::DT; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.f;

    const int64_t koff = (int64_t)bh * a.Nkv * HD, voff = (int64_t)bh * HD * ldv;
    // key tiles of this work-group: all, or with nsplit > 1 the blockIdx.z-th
    // of nsplit consecutive ranges (each holds at least one tile)
    const int ntiles_all = (a.Nkv + KT - 1) / KT;
    const int per = (ntiles_all + a.nsplit - 1) / a.nsplit;
    const int t0 = (int)blockIdx.z * per;
    const int ntiles = min(ntiles_all, t0 + per) - t0;
    uint8_t *const Kring = lds, *const Vring = lds + 2 * KBUF;

    // DMA: per plane, a K tile is runs of 1 KB (8 rows of 128 B, or 4 of 256 B)
    // and a Vᵀ tile runs of 1 KB (16 rows of 64 B); wave w moves runs
    // w·RUNS .. w·RUNS + RUNS − 1.  A lane writes the 16 bytes at 16·lane of its
    // run and fetches the chunk that belongs there.  The loads go through
    // buffer descriptors whose base and record count carry the tile's
    // position (scalar arithmetic), so each lane's offset is a constant and
    // reads past the record count return zeros: K rows past the keys (their
    // scores are masked).  In a tile that reaches past a Vᵀ row's vt_ld keys
    // those chunks are clamped onto the row's last 8 keys (finite, and their
    // probabilities are 0), never into the next row, which may be an
    // unwritten padding row.
    auto dma = [&](const void *base, uint32_t nrec, uint8_t *ldsp, int lane_off) {
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)nrec, 0x00020000);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, LDS_PTR(ldsp), 16, lane_off, 0, 0, 0);
    };
    int k_lane[G::KRUNS], v_lane[G::VRUNS];
#pragma unroll
    for (int j = 0; j < G::KRUNS; j++) {
        constexpr int RPR = 1024 / G::ROWK;      // rows per run
        constexpr int CPR = G::ROWK / 16;        // chunks per row
        const int r = RPR * (wave * G::KRUNS + j) + lane / CPR;
        k_lane[j] = r * G::ROWK + (((lane % CPR) ^ swzk_hd<HD>(r)) << 4);
    }
    int vn_lane[G::KRUNS];  // VN: V tiles as K tiles, own swizzle
#pragma unroll
    for (int j = 0; j < G::KRUNS; j++) {
        constexpr int RPR = 1024 / G::ROWK;
        constexpr int CPR = G::ROWK / 16;
        const int r = RPR * (wave * G::KRUNS + j) + lane / CPR;
        vn_lane[j] = r * G::ROWK + (((lane % CPR) ^ swzvn<HD>(r)) << 4);
    }
    int v_row[G::VRUNS], v_ch[G::VRUNS];
#pragma unroll
    for (int j = 0; j < G::VRUNS; j++) {
        const int r = 16 * (wave * G::VRUNS + j) + (lane >> 2);
        v_row[j] = r * ldv * 2;
        v_ch[j] = (lane & 3) ^ swzv(r);
        v_lane[j] = v_row[j] + (v_ch[j] << 4);
    }
    auto issue_k = [&](int tt) {
        uint8_t *L = Kring + (tt & 1) * KBUF;
        const int tile = t0 + tt;
        const uint32_t nrec = (uint32_t)min(a.Nkv - tile * KT, KT) * G::ROWK;
#pragma unroll
        for (int pl = 0; pl < NP; pl++) {
            const _Float16 *base = (pl == 0 ? a.k : a.k_lo) + koff + (int64_t)tile * KT * HD;
#pragma unroll
            for (int j = 0; j < G::KRUNS; j++) dma(base, nrec, L + pl * KPL + (wave * G::KRUNS + j) * 1024, k_lane[j]);
        }
    };
    auto issue_v = [&](int tt) {
        uint8_t *L = Vring + (tt & 1) * VBUF;
        const int tile = t0 + tt;
        if constexpr (VN) {
            // rows past the keys read as zeros (their probabilities are 0)
            const uint32_t nk = (uint32_t)min(a.Nkv - tile * KT, KT) * G::ROWK;
            const _Float16 *base = a.v + koff + (int64_t)tile * KT * HD;
#pragma unroll
            for (int j = 0; j < G::KRUNS; j++) dma(base, nk, L + (wave * G::KRUNS + j) * 1024, vn_lane[j]);
            return;
        }
        const uint32_t nrec = (uint32_t)(HD * ldv - tile * KT) * 2;
        int off[G::VRUNS];
#pragma unroll
        for (int j = 0; j < G::VRUNS; j++) off[j] = v_lane[j];
        if (tile * KT + KT > ldv) {  // the row's end falls inside this tile
#pragma unroll
            for (int j = 0; j < G::VRUNS; j++) off[j] = v_row[j] + 2 * min(8 * v_ch[j], ldv - 8 - tile * KT);
        }
#pragma unroll
        for (int pl = 0; pl < NP; pl++) {
            const _Float16 *base = (pl == 0 ? a.vt : a.vt_lo) + voff + (int64_t)tile * KT;
#pragma unroll
            for (int j = 0; j < G::VRUNS; j++) dma(base, nrec, L + pl * VPL + (wave * G::VRUNS + j) * 1024, off[j]);
        }
    };

    const int xk = swzk_hd<HD>(lr), xv = swzv(lr);  // operand rows start at multiples of 32

    // Sᵀ = K·Qᵀ for the 32 keys of tile tt × 32 queries
    auto qk = [&](int tt) {
        const uint8_t *L = Kring + (tt & 1) * KBUF;
        v16f acc = {};
#pragma unroll
        for (int ds = 0; ds < G::DS; ds++) {
            const int o_ = lr * G::ROWK + (((2 * ds + lh) ^ xk) << 4);
            const v8h kh = *(const v8h *)(L + o_);
            if constexpr (SPLIT) {
                const v8h kl = *(const v8h *)(L + KPL + o_);
                acc = mfma(kl, qf[0][ds], acc);
                acc = mfma(kh, qf[1][ds], acc);
            }
            acc = mfma(kh, qf[0][ds], acc);
        }
        return acc;
    };
    // Oᵀ += Vᵀ·Pᵀ for the 32 keys of tile tt
    // VN: lane L = 16g + 4j + q (g = 2·lh + gc) addresses key row
    // 16·jj + 4·lh + j (+ 8 for the second load) at channels dt·32 + 16·gc +
    // 4q .. + 3, so each lane receives channel dt·32 + L % 32 of keys
    // 16·jj + 4·lh + 0..3 and + 8..11: the keys its K slots hold
    const int tr_j = (lane & 15) >> 2, tr_q = lane & 3, tr_gc = (lane >> 4) & 1;
    auto tr_off = [&](int dt, int jj, int half) {
        const int row = 16 * jj + 8 * half + 4 * lh + tr_j;
        const int chunk = 4 * dt + 2 * tr_gc + (tr_q >> 1);
        return row * G::ROWK + ((chunk ^ swzvn<HD>(row)) << 4) + 8 * (tr_q & 1);
    };
    auto pv = [&](int tt, const v8h (&ph)[2], const v8h (&pl)[2]) {
        const uint8_t *L = Vring + (tt & 1) * VBUF;
        if constexpr (VN) {
#pragma unroll
            for (int dt = 0; dt < G::DT; dt++)
#pragma unroll
                for (int jj = 0; jj < 2; jj++) {
                    const v4h v0 = lds_tr16(L + tr_off(dt, jj, 0)), v1 = lds_tr16(L + tr_off(dt, jj, 1));
                    const v8h vh = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
                    o[dt] = mfma(vh, ph[jj], o[dt]);
                }
            return;
        }
#pragma unroll
        for (int dt = 0; dt < G::DT; dt++)
#pragma unroll
            for (int jj = 0; jj < 2; jj++) {
                const int o_ = (dt * 32 + lr) * 64 + (((2 * jj + lh) ^ xv) << 4);
                const v8h vh = *(const v8h *)(L + o_);
                if constexpr (SPLIT) {
                    const v8h vl = *(const v8h *)(L + VPL + o_);
                    o[dt] = mfma(vl, ph[jj], o[dt]);
                    o[dt] = mfma(vh, pl[jj], o[dt]);
                }
                o[dt] = mfma(vh, ph[jj], o[dt]);
            }
    };
    // scaled maximum over the tile's 32 keys (both lane halves): one lane-half
    // swap leaves every lane with {own, partner} in some order, no LDS trip
    auto tmax = [&](const v16f &sv) {
        float m = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) m = fmaxf(m, sv[r]);
        const uint32_t mb = __builtin_bit_cast(uint32_t, m);
        const auto sw = __builtin_amdgcn_permlane32_swap(mb, mb, false, false);
        return fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]), __builtin_bit_cast(float, (uint32_t)sw[1])) * c;
    };
    // keys past Nkv score −inf (only the last, partial tile)
    auto mask = [&](v16f &sv, int tt) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = (t0 + tt) * KT + 8 * (r >> 2) + 4 * lh + (r & 3);
            if (key >= a.Nkv) sv[r] = -INFINITY;
        }
    };
    // P = exp2(s·c − m) as fp16 hi (+ lo) B operands; returns Σp
    auto softmax = [&](const v16f &sv, float m, v8h (&ph)[2], v8h (&pl)[2]) {
        const float nm = -m;
        float ps = 0.f;
#pragma unroll
        for (int jj = 0; jj < 2; jj++) {
            v4u hw, lw;
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[8 * jj + i], c, nm));
                const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[8 * jj + i + 1], c, nm));
                ps += p0;
                ps += p1;
                const uint32_t h2 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p0, p1));
                hw[i / 2] = h2;
                if constexpr (SPLIT)
                    lw[i / 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(sub_lo_half(p0, h2), sub_hi_half(p1, h2)));
            }
            ph[jj] = __builtin_bit_cast(v8h, hw);
            if constexpr (SPLIT) pl[jj] = __builtin_bit_cast(v8h, lw);
        }
        return ps;
    };
    // Issue is in order within a wave: the scheduling barriers interleave the
    // MFMA stream (Sᵀ of the next tile, Oᵀ of the previous) with the softmax
    // VALU of the current tile, which then runs in the MFMA shadow.
    auto interleave = [&]() {
#pragma unroll
        for (int i = 0; i < 24; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // VALU
        }
    };

    // Software pipeline over tiles: iteration j forms Sᵀ(j+1) and Oᵀ += P(j−1)
    // on MFMA while the VALU turns Sᵀ(j) into P(j).  The K ring holds tiles
    // j+1 (read) and j+2 (in flight), the Vᵀ ring j−1 (read) and j (in
    // flight).  The running reference m is raised only when a tile's maximum
    // exceeds it by more than 8 (p ≤ 2^8 meanwhile); then Oᵀ, which then
    // holds P(j−1) terms under the old m, is rescaled after this iteration's
    // MFMAs.  (Two alternating register sets instead of the copies at the end
    // of an iteration need more VGPRs than 3 waves per SIMD allow; the
    // occupancy is worth more.)
    const bool wave_live = q0 + wave * 32 < a.Nq;  // waves past the queries only move tiles
    v16f s_cur = {}, s_next = {};
    v8h ph_prev[2], pl_prev[2], ph_cur[2], pl_cur[2];
    auto iter = [&](int j, auto has_qk, auto has_sm, auto masked, auto has_pv) {
        wait_and_barrier<0>();  // K(j+1), Vᵀ(j−1) landed; tiles of j−1 released
        if (j + 2 < ntiles) issue_k(j + 2);
        if (j < ntiles) issue_v(j);
        if (!wave_live) return;
        bool raise = false;
        float mnew = mrun, alpha = 1.f, ps = 0.f;
        if constexpr (decltype(has_sm)::value) {
            if constexpr (decltype(masked)::value) mask(s_cur, j);
            const float mt = tmax(s_cur);
            raise = mt > mrun + 8.f;
            mnew = raise ? mt : mrun;
            alpha = __builtin_amdgcn_exp2f(mrun - mnew);
        }
        if constexpr (decltype(has_qk)::value) s_next = qk(j + 1);
        if constexpr (decltype(has_pv)::value) pv(j - 1, ph_prev, pl_prev);
        if constexpr (decltype(has_sm)::value) ps = softmax(s_cur, mnew, ph_cur, pl_cur);
        interleave();
        if constexpr (decltype(has_sm)::value) {
            lsum = lsum * alpha + ps;
            if (__any(raise)) {
#pragma unroll
                for (int dt = 0; dt < G::DT; dt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) o[dt][r] *= alpha;
            }
            mrun = mnew;
        }
        if constexpr (decltype(has_qk)::value) s_cur = s_next;
        if constexpr (decltype(has_sm)::value) {
#pragma unroll
            for (int jj = 0; jj < 2; jj++) { ph_prev[jj] = ph_cur[jj]; pl_prev[jj] = pl_cur[jj]; }
        }
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    const bool partial = (a.Nkv % KT) != 0 && t0 + ntiles == ntiles_all;

    issue_k(0);
    if (ntiles > 1) issue_k(1);
    wait_and_barrier<0>();
    if (wave_live) s_cur = qk(0);
    // j = 0 .. ntiles: Sᵀ(j+1) while j+1 < ntiles, P(j) while j < ntiles
    // (masked on a partial last tile), Oᵀ += P(j−1) from j = 1
    if (ntiles == 1) {
        if (partial) iter(0, F_{}, T_{}, T_{}, F_{});
        else iter(0, F_{}, T_{}, F_{}, F_{});
    } else {
        iter(0, T_{}, T_{}, F_{}, F_{});
        for (int j = 1; j + 1 < ntiles; j++) iter(j, T_{}, T_{}, F_{}, T_{});
        if (partial) iter(ntiles - 1, F_{}, T_{}, T_{}, T_{});
        else iter(ntiles - 1, F_{}, T_{}, F_{}, T_{});
    }
    iter(ntiles, F_{}, F_{}, F_{}, T_{});

    lsum += __shfl_xor(lsum, 32, 64);
    if (a.nsplit > 1) {
        // unnormalised partial output and its statistics (exp2 domain) for
        // the combining pass
        if (qvalid) {
            const int64_t prow = ((int64_t)blockIdx.z * a.BH + bh) * a.Nq + qi;
#pragma unroll
            for (int dt = 0; dt < G::DT; dt++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                    *(float4 *)(a.part_o + prow * HD + dt * 32 + 8 * g + 4 * lh) =
                        make_float4(o[dt][4 * g], o[dt][4 * g + 1], o[dt][4 * g + 2], o[dt][4 * g + 3]);
            if (lh == 0) *(float2 *)(a.part_ml + prow * 2) = make_float2(mrun, lsum);
        }
        return;
    }
    const float inv = (lsum == 0.f) ? 0.f : 1.0f / lsum;
#pragma unroll
    for (int dt = 0; dt < G::DT; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] *= inv;

    // output row for (batch b, query qi)
    const int b = bh / a.NH, h = bh % a.NH;
    int64_t orow;
    bool ovalid = qvalid;
    if (CROP && a.wo > 0) {
        // windows of wo×wo queries, row-major over nwx windows per row, on an
        // out_h × out_w grid; positions past it (window padding) are dropped
        const int wy = b / a.nwx, wx = b % a.nwx;
        const int qq = qvalid ? qi : 0;
        const int y = wy * a.wo + qq / a.wo, x = wx * a.wo + qq % a.wo;
        ovalid = ovalid && y < a.out_h && x < a.out_w;
        orow = (int64_t)y * a.out_w + x;
    } else if (a.grid > 0) {
        const int nwx = a.grid / a.window;
        const int wy = b / nwx, wx = b % nwx;
        const int iy = (qvalid ? qi : 0) / a.window, ix = (qvalid ? qi : 0) % a.window;
        orow = (int64_t)(wy * a.window + iy) * a.grid + wx * a.window + ix;
    } else {
        orow = (int64_t)b * a.Nq + qi;
    }
    const Act &out = a.out;
    const int hdo = (CROP && a.hd_out > 0) ? a.hd_out : HD;  // real head dim: padded columns are not stored
    const int64_t colbase = (int64_t)h * hdo;
#pragma unroll
    for (int dt = 0; dt < G::DT; dt++) {
        if (CROP && dt * 32 >= hdo) break;
        if (out.kind == A_F6) {
            // the same Q8_0 codes in the A_F6 layout: this lane holds block
            // positions 8g + 4·lh + i (i < 4), lane l ^ 32 the others.  Each
            // value splits as q = 16h + l; one lane-half swap per pair leaves
            // lanes 0-31 with the block's 32 h values (own in slots 8g + i,
            // the partner's in 8g + 4 + i) and lanes 32-63 with its 32 l
            // values, which one fp6 conversion packs into the 192-bit string
            // of part lh
            float amax = 0.f;
#pragma unroll
            for (int r = 0; r < 16; r++) amax = fmaxf(amax, fabsf(o[dt][r]));
            amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
            const float d = amax / 127.f;
            const float id = (amax != 0.f) ? 127.f / amax : 0.f;
            f32x16 ev, od;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                float a[4], b[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float hv, lv;
                    f6_split(o[dt][4 * g + i], id, hv, lv);
                    // lanes 0-31 keep hv and receive the partner's hv; lanes
                    // 32-63 receive the partner's lv and keep lv
                    const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, hv),
                                                                     __builtin_bit_cast(uint32_t, lv), false, false);
                    a[i] = __builtin_bit_cast(float, (uint32_t)sw[0]);
                    b[i] = __builtin_bit_cast(float, (uint32_t)sw[1]);
                }
                // slot 2k from ev[k], 2k + 1 from od[k]: slots 8g .. 8g + 3 ← a, 8g + 4 .. 8g + 7 ← b
                ev[4 * g] = a[0];
                od[4 * g] = a[1];
                ev[4 * g + 1] = a[2];
                od[4 * g + 1] = a[3];
                ev[4 * g + 2] = b[0];
                od[4 * g + 2] = b[1];
                ev[4 * g + 3] = b[2];
                od[4 * g + 3] = b[3];
            }
            const u32x6 mine = pack_bf6(ev, od);
            if (ovalid) {
                const int64_t blk = (colbase + dt * 32) / QK;
                uint64_t *base = (uint64_t *)out.x;
#pragma unroll
                for (int tw = 0; tw < 3; tw++)
                    base[f6_act_word(out.ld / 128, orow, blk, lh, tw)] =
                        (uint64_t)mine[2 * tw] | ((uint64_t)mine[2 * tw + 1] << 32);
                if (lh == 0) out.d[scale_index(out.mp, orow, blk)] = f2h_bits(d);
            }
        } else if (out.kind == A_Q8_0 || out.kind == A_Q8_1) {
            // ggml quantize_row_q8_0/q8_1 of the 32 values d = dt*32 .. dt*32+31,
            // split 16/16 between lanes l and l^32
            float amax = 0.f;
#pragma unroll
            for (int r = 0; r < 16; r++) amax = fmaxf(amax, fabsf(o[dt][r]));
            amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
            const float d = amax / 127.f;
            const float id = (amax != 0.f) ? 127.f / amax : 0.f;
            int sum = 0;
            uint32_t w[4];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                uint32_t packed = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int q = (int)__builtin_rintf(o[dt][4 * g + i] * id);
                    sum += q;
                    packed |= ((uint32_t)(q & 0xff)) << (8 * i);
                }
                w[g] = packed;
            }
            sum += __shfl_xor(sum, 32, 64);
            if (ovalid) {
                int8_t *dst = (int8_t *)out.x + orow * out.ld + colbase + dt * 32 + 4 * lh;
#pragma unroll
                for (int g = 0; g < 4; g++) *(uint32_t *)(dst + 8 * g) = w[g];
                if (lh == 0) {
                    const int64_t blk = scale_index(out.mp, orow, (colbase + dt * 32) / QK);
                    out.d[blk] = f2h_bits(d);
                    if (out.kind == A_Q8_1) out.s[blk] = f2h_bits(d * (float)sum);
                }
            }
        } else if (ovalid) {
#pragma unroll
            for (int g = 0; g < 4; g++) {
                if (CROP && dt * 32 + 8 * g + 4 * lh >= hdo) continue;  // zero-padded head dims
                const int64_t col = colbase + dt * 32 + 8 * g + 4 * lh;
                if (out.kind == A_F32) {
                    *(float4 *)((float *)out.x + orow * out.ld + col) =
                        make_float4(o[dt][4 * g], o[dt][4 * g + 1], o[dt][4 * g + 2], o[dt][4 * g + 3]);
                } else {
                    const uint32_t w0 = (uint32_t)f2h_bits(o[dt][4 * g]) | ((uint32_t)f2h_bits(o[dt][4 * g + 1]) << 16);
                    const uint32_t w1 = (uint32_t)f2h_bits(o[dt][4 * g + 2]) | ((uint32_t)f2h_bits(o[dt][4 * g + 3]) << 16);
                    *(uint2 *)((_Float16 *)out.x + orow * out.ld + col) = make_uint2(w0, w1);
                    if (out.kind == A_F16X2) {
                        // the pair's low half: fp16 of the exact difference
                        uint32_t l[4];
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const float v = o[dt][4 * g + i];
                            const _Float16 hv = __builtin_bit_cast(_Float16, (uint16_t)f2h_bits(v));
                            l[i] = __builtin_bit_cast(uint16_t, (_Float16)(v - (float)hv));
                        }
                        *(uint2 *)((_Float16 *)out.lo + orow * out.ld + col) =
                            make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
                    }
                }
            }
        }
    }
}

// Combine the key-range partials: O = Σ_s 2^(m_s − M)·O_s / Σ_s 2^(m_s − M)·l_s.
// One thread per (batch·head, query, 4 channels); channels past the real
// head dim (zero-padded heads) are not stored.  f32 or fp16 output, row
// b·Nq + q, column h·hd_out + d.
__global__ void k_attn_combine(AttnArgs a, int hd, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int d = (int)(i % (hd / 4)) * 4;
    const int hdo = a.hd_out > 0 ? a.hd_out : hd;
    if (d >= hdo) return;
    const int64_t r = i / (hd / 4);  // bh·Nq + q
    const int64_t plane = (int64_t)a.BH * a.Nq;
    float M = -INFINITY;
    for (int s = 0; s < a.nsplit; s++) M = fmaxf(M, a.part_ml[(s * plane + r) * 2]);
    float den = 0.f;
    float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < a.nsplit; s++) {
        const float2 ml = *(const float2 *)(a.part_ml + (s * plane + r) * 2);
        const float w = __builtin_amdgcn_exp2f(ml.x - M);
        den = __builtin_fmaf(w, ml.y, den);
        const float4 o = *(const float4 *)(a.part_o + (s * plane + r) * hd + d);
        num.x = __builtin_fmaf(w, o.x, num.x);
        num.y = __builtin_fmaf(w, o.y, num.y);
        num.z = __builtin_fmaf(w, o.z, num.z);
        num.w = __builtin_fmaf(w, o.w, num.w);
    }
    const float inv = den == 0.f ? 0.f : 1.0f / den;
    const int64_t bh = r / a.Nq, q = r % a.Nq;
    const int64_t b = bh / a.NH, h = bh % a.NH;
    const int64_t off = (b * a.Nq + q) * a.out.ld + h * hdo + d;
    if (a.out.kind == A_F16) {
        const uint32_t w0 = (uint32_t)f2h_bits(num.x * inv) | ((uint32_t)f2h_bits(num.y * inv) << 16);
        const uint32_t w1 = (uint32_t)f2h_bits(num.z * inv) | ((uint32_t)f2h_bits(num.w * inv) << 16);
        *(uint2 *)((_Float16 *)a.out.x + off) = make_uint2(w0, w1);
    } else {
        *(float4 *)((float *)a.out.x + off) = make_float4(num.x * inv, num.y * inv, num.z * inv, num.w * inv);
    }
}

}  // namespace

hipError_t launch_attn(const AttnArgs &a, hipStream_t st) {
    // Vᵀ rows hold vt_ld_for(Nkv) keys (zero past Nkv, in vt_slot order)
    const int ldv = (int)vt_ld_for(a.Nkv);
    const int hd = a.hd > 0 ? a.hd : 64;
    if ((hd != 64 && hd != 128 && hd != 256) || a.BH <= 0 || a.BH > 65535 || a.Nq <= 0 || a.Nkv <= 0)
        return hipErrorInvalidValue;
    const int ntiles = (a.Nkv + 31) / 32;
    if (a.nsplit < 1 || a.nsplit > ntiles) return hipErrorInvalidValue;
    if (a.q_hs != 0 && a.q_hs < (int64_t)a.Nq * hd) return hipErrorInvalidValue;
    if (a.nsplit > 1) {
        // every range must hold a tile; plain layouts (narrower heads allowed),
        // f32 or fp16 output
        const int per = (ntiles + a.nsplit - 1) / a.nsplit;
        if ((int64_t)per * (a.nsplit - 1) >= ntiles || !a.part_o || !a.part_ml ||
            (a.out.kind != A_F32 && a.out.kind != A_F16) || a.wo > 0 || a.grid > 0 ||
            (a.hd_out > 0 && (a.hd_out > hd || a.hd_out % 4 != 0)))
            return hipErrorInvalidValue;
    }
    // head dim 256: fp16 operands only
    if (hd == 256 && (a.q_lo || a.wo > 0 || (a.hd_out > 0 && a.hd_out != hd))) return hipErrorInvalidValue;
    // a Q8 output block must lie inside one head
    if (a.out.kind == A_F6 && (a.out.ld % 128 != 0 || (a.hd_out > 0 && a.hd_out % 32 != 0)))
        return hipErrorInvalidValue;
    if ((a.out.kind == A_Q8_0 || a.out.kind == A_Q8_1) && a.hd_out > 0 && a.hd_out % 32 != 0)
        return hipErrorInvalidValue;
    if (a.out.kind == A_F16X2 && (!a.out.lo || a.out.ld % 4 != 0)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((a.Nq + QT - 1) / QT), (unsigned)a.BH, (unsigned)a.nsplit);
    const bool crop = a.wo > 0 || (a.hd_out > 0 && a.hd_out != hd);
    if (a.v) {
        // natural V: fp16 operands, head dim 64 or 128
        if (a.q_lo || a.k_lo || hd == 256) return hipErrorInvalidValue;
        if (hd == 64 && !crop) hipLaunchKernelGGL((k_attn<false, 64, false, true>), grid, dim3(NTHR), 0, st, a, ldv);
        else if (hd == 64) hipLaunchKernelGGL((k_attn<false, 64, true, true>), grid, dim3(NTHR), 0, st, a, ldv);
        else hipLaunchKernelGGL((k_attn<false, 128, true, true>), grid, dim3(NTHR), 0, st, a, ldv);
    } else if (hd == 256) {
        hipLaunchKernelGGL((k_attn<false, 256, false>), grid, dim3(NTHR), 0, st, a, ldv);
    } else if (hd == 64 && !crop) {
        if (a.q_lo) hipLaunchKernelGGL((k_attn<true, 64, false>), grid, dim3(NTHR), 0, st, a, ldv);
        else hipLaunchKernelGGL((k_attn<false, 64, false>), grid, dim3(NTHR), 0, st, a, ldv);
    } else if (hd == 64) {
        if (a.q_lo) hipLaunchKernelGGL((k_attn<true, 64, true>), grid, dim3(NTHR), 0, st, a, ldv);
        else hipLaunchKernelGGL((k_attn<false, 64, true>), grid, dim3(NTHR), 0, st, a, ldv);
    } else {
        if (a.q_lo) hipLaunchKernelGGL((k_attn<true, 128, true>), grid, dim3(NTHR), 0, st, a, ldv);
        else hipLaunchKernelGGL((k_attn<false, 128, true>), grid, dim3(NTHR), 0, st, a, ldv);
    }
    if (a.nsplit > 1) {
        const int64_t total = (int64_t)a.BH * a.Nq * (hd / 4);
        hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, a, hd, total);
    }
    return hipGetLastError();
}

}  // namespace s3e
