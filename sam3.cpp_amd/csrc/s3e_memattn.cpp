// s3e_memattn.cpp — the tracker's memory attention on the engine's kernels:
// the transformer that conditions the current frame's image tokens on the
// memory bank before the mask decoder (sam3_build_mem_attn_graph,
// sam3.cpp:9224-9337; inputs as sam3_propagate_single builds them,
// sam3.cpp:11232-11304).
//
// Per layer (D = neck_dim channels, one attention head of D channels):
//   self-attention   LN1 → one GEMM for q|k|v (the three weights concatenated
//                    at load) whose epilogue applies RoPE to q and k and
//                    writes fp16 Q, K and Vᵀ → attention (head dim 256,
//                    split over keys) → out_proj + bias + residual
//   cross-attention  LN2 → q GEMM (+ RoPE); k GEMM on memory + memory
//                    positions (RoPE on the spatial keys only: the trailing
//                    object-pointer tokens keep none) and v GEMM on the memory,
//                    both MD → D → attention → out_proj + bias + residual
//   FFN              LN3 → linear1 + bias + ReLU → linear2 + bias + residual
// then the final LayerNorm.  The input is curr + 0.1·src_pos.  LayerNorm eps
// 1e-5 (sam3_layer_norm, sam3.cpp:1037-1047); GEMM inputs are converted to
// the weight's vec_dot type as everywhere in the engine; attention runs on
// fp16 operands with fp32 accumulation.
#include "s3e_memattn.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <vector>

namespace s3e {

struct MemAttnLayer {
    Weight sa_qkv, sa_out, ca_q, ca_k, ca_v, ca_out, fc1, fc2;
    float *sa_qkv_b = nullptr, *sa_out_b = nullptr, *ca_q_b = nullptr, *ca_k_b = nullptr, *ca_v_b = nullptr,
          *ca_out_b = nullptr, *fc1_b = nullptr, *fc2_b = nullptr;
    float *n1w = nullptr, *n1b = nullptr, *n2w = nullptr, *n2b = nullptr, *n3w = nullptr, *n3b = nullptr;
};

struct MemAttnModel {
    int L = 0, D = 0, MD = 0, FFN = 0;
    std::vector<MemAttnLayer> layers;
    float *nw = nullptr, *nb = nullptr;
    std::map<std::string, RawTensor> raw;  // host records until memattn_finish
    std::vector<void *> owned;
    ~MemAttnModel() {
        for (auto &l : layers)
            for (Weight *w : {&l.sa_qkv, &l.sa_out, &l.ca_q, &l.ca_k, &l.ca_v, &l.ca_out, &l.fc1, &l.fc2})
                free_weight(*w);
        for (void *p : owned) (void)hipFree(p);
    }
};

struct MemAttnState {
    int64_t capN = 0, capM = 0;
    int D = 0, MD = 0, FFN = 0;
    float *x = nullptr, *att = nullptr, *kvp = nullptr, *part_o = nullptr, *part_ml = nullptr;
    int64_t part_cap = 0;           // rows of part_ml (and of part_o at D floats each)
    int64_t part_o_floats = 0;      // part_o also serves the K-split residual GEMMs
    ActBuf an, ah, am1, am2;
    _Float16 *q16 = nullptr, *k16 = nullptr, *vt16 = nullptr;
    void release() {
        an.release();
        ah.release();
        am1.release();
        am2.release();
        for (void *p : {(void *)x, (void *)att, (void *)kvp, (void *)part_o, (void *)part_ml, (void *)q16, (void *)k16,
                        (void *)vt16})
            if (p) (void)hipFree(p);
        x = att = kvp = part_o = part_ml = nullptr;
        q16 = k16 = vt16 = nullptr;
        capN = capM = part_cap = part_o_floats = 0;
    }
    ~MemAttnState() { release(); }
};

bool memattn_wants(const std::string &name) { return name.compare(0, 9, "mem_attn.") == 0; }

int memattn_take(MemAttnModel **m, const std::string &name, RawTensor &&t, int wtype) {
    // registered types: T2 weights take the file's weight type when ne0 is a
    // block multiple, T1f vectors F32 (sam3.cpp:2004-2040)
    int want = 0;
    if (t.n_dims >= 2) want = (t.ne[0] % ggml_blck(wtype) == 0) ? wtype : 0;
    if (!coerce(t, want)) {
        set_error("s3e_model_load: cannot convert '%s' from type %d to %d", name.c_str(), t.type, want);
        return S3E_ERR_IO;
    }
    if (!*m) *m = new MemAttnModel;
    (*m)->raw[name] = std::move(t);
    return S3E_OK;
}

namespace {

int upload_vec(MemAttnModel *m, const RawTensor &t, int64_t n, float **dst) {
    const int64_t have = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
    if (have != n || t.type != 0) {
        set_error("memory attention: vector of %lld floats expected", (long long)n);
        return S3E_ERR_IO;
    }
    void *p = nullptr;
    if (hipMalloc(&p, (size_t)n * 4) != hipSuccess) { set_error("hipMalloc failed"); return S3E_ERR_NOMEM; }
    m->owned.push_back(p);
    if (hipMemcpy(p, t.data.data(), (size_t)n * 4, hipMemcpyHostToDevice) != hipSuccess) {
        set_error("hipMemcpy failed");
        return S3E_ERR_HIP;
    }
    *dst = (float *)p;
    return S3E_OK;
}

}  // namespace

int memattn_finish(MemAttnModel *m) {
    if (!m) return S3E_OK;
    auto find = [&](const std::string &n) -> const RawTensor * {
        auto it = m->raw.find(n);
        return it == m->raw.end() ? nullptr : &it->second;
    };
    int L = 0;
    while (find("mem_attn.layers." + std::to_string(L) + ".sa.q_proj.weight")) L++;
    const RawTensor *ck = find("mem_attn.layers.0.ca.k_proj.weight"), *f1 = find("mem_attn.layers.0.linear1.weight");
    if (L == 0 || !ck || !f1) { set_error("s3e_model_load: incomplete memory attention"); return S3E_ERR_IO; }
    m->L = L;
    m->D = (int)ck->ne[1];
    m->MD = (int)ck->ne[0];
    m->FFN = (int)f1->ne[1];
    const int D = m->D, MD = m->MD, FFN = m->FFN;
    if (D != 256 || MD % 32 != 0 || FFN % 32 != 0) {
        set_error("s3e_model_load: memory attention with D=%d MD=%d FFN=%d is not supported (D must be 256)", D, MD, FFN);
        return S3E_ERR_UNSUPPORTED;
    }
    m->layers.resize((size_t)L);
    int rc = S3E_OK;
    for (int l = 0; l < L && rc == S3E_OK; l++) {
        MemAttnLayer &ly = m->layers[(size_t)l];
        const std::string p = "mem_attn.layers." + std::to_string(l) + ".";
        auto need = [&](const std::string &s) -> const RawTensor * {
            const RawTensor *t = find(p + s);
            if (!t) set_error("s3e_model_load: missing tensor %s%s", p.c_str(), s.c_str());
            return t;
        };
        auto lin = [&](const char *name, int64_t K, int64_t N, Weight &w, float **b) {
            const RawTensor *tw = need(std::string(name) + ".weight"), *tb = need(std::string(name) + ".bias");
            if (!tw || !tb) return (int)S3E_ERR_IO;
            if (tw->ne[0] != K || tw->ne[1] != N) { set_error("memory attention %s%s: bad shape", p.c_str(), name); return (int)S3E_ERR_IO; }
            const int r = upload_weight(0, tw->type, K, N, tw->data.data(), tw->data.size(), w);
            return r != S3E_OK ? r : upload_vec(m, *tb, N, b);
        };
        // q | k | v of the self-attention as one [3D][D] weight
        {
            const RawTensor *q = need("sa.q_proj.weight"), *k = need("sa.k_proj.weight"), *v = need("sa.v_proj.weight");
            const RawTensor *qb = need("sa.q_proj.bias"), *kb = need("sa.k_proj.bias"), *vb = need("sa.v_proj.bias");
            if (!q || !k || !v || !qb || !kb || !vb) return S3E_ERR_IO;
            for (const RawTensor *t : {q, k, v})
                if (t->ne[0] != D || t->ne[1] != D || t->type != q->type) { set_error("memory attention: bad sa weights"); return S3E_ERR_IO; }
            std::vector<uint8_t> cat;
            for (const RawTensor *t : {q, k, v}) cat.insert(cat.end(), t->data.begin(), t->data.end());
            rc = upload_weight(0, q->type, D, 3LL * D, cat.data(), cat.size(), ly.sa_qkv);
            if (rc != S3E_OK) return rc;
            RawTensor bcat;
            bcat.type = 0;
            bcat.n_dims = 1;
            bcat.ne[0] = 3LL * D;
            for (const RawTensor *t : {qb, kb, vb}) bcat.data.insert(bcat.data.end(), t->data.begin(), t->data.end());
            rc = upload_vec(m, bcat, 3LL * D, &ly.sa_qkv_b);
            if (rc != S3E_OK) return rc;
        }
        if ((rc = lin("sa.out_proj", D, D, ly.sa_out, &ly.sa_out_b)) != S3E_OK) return rc;
        if ((rc = lin("ca.q_proj", D, D, ly.ca_q, &ly.ca_q_b)) != S3E_OK) return rc;
        if ((rc = lin("ca.k_proj", MD, D, ly.ca_k, &ly.ca_k_b)) != S3E_OK) return rc;
        if ((rc = lin("ca.v_proj", MD, D, ly.ca_v, &ly.ca_v_b)) != S3E_OK) return rc;
        if ((rc = lin("ca.out_proj", D, D, ly.ca_out, &ly.ca_out_b)) != S3E_OK) return rc;
        if ((rc = lin("linear1", D, FFN, ly.fc1, &ly.fc1_b)) != S3E_OK) return rc;
        if ((rc = lin("linear2", FFN, D, ly.fc2, &ly.fc2_b)) != S3E_OK) return rc;
        const char *ln[6] = {"norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias", "norm3.weight", "norm3.bias"};
        float **dst[6] = {&ly.n1w, &ly.n1b, &ly.n2w, &ly.n2b, &ly.n3w, &ly.n3b};
        for (int i = 0; i < 6; i++) {
            const RawTensor *t = need(ln[i]);
            if (!t) return S3E_ERR_IO;
            if ((rc = upload_vec(m, *t, D, dst[i])) != S3E_OK) return rc;
        }
    }
    const RawTensor *nw = find("mem_attn.norm.weight"), *nb = find("mem_attn.norm.bias");
    if (!nw || !nb) { set_error("s3e_model_load: missing mem_attn.norm"); return S3E_ERR_IO; }
    if ((rc = upload_vec(m, *nw, D, &m->nw)) != S3E_OK) return rc;
    if ((rc = upload_vec(m, *nb, D, &m->nb)) != S3E_OK) return rc;
    m->raw.clear();
    return S3E_OK;
}

void memattn_free(MemAttnModel *m) { delete m; }

void memattn_dims(const MemAttnModel *m, int32_t out[4]) {
    out[0] = m->L;
    out[1] = m->D;
    out[2] = m->MD;
    out[3] = m->FFN;
}

void memattn_state_free(MemAttnState *s) { delete s; }

namespace {

hipError_t grow(const MemAttnModel *m, MemAttnState *s, int64_t N, int64_t M, hipStream_t st) {
    if (N <= s->capN && M <= s->capM) return hipSuccess;
    const int64_t cN = std::max(N, s->capN), cM = std::max(M, s->capM);
    (void)hipStreamSynchronize(st);
    s->release();
    s->D = m->D;
    s->MD = m->MD;
    s->FFN = m->FFN;
    const int64_t D = m->D, MD = m->MD, NK = std::max(cN, cM);
    hipError_t e = hipMalloc(&s->x, (size_t)(cN * D * 4));
    if (e == hipSuccess) e = hipMalloc(&s->att, (size_t)(cN * D * 4));
    if (e == hipSuccess) e = hipMalloc(&s->kvp, (size_t)(cM * MD * 4));
    if (e == hipSuccess) e = s->an.alloc(cN, D, st);
    if (e == hipSuccess) e = s->ah.alloc(cN, m->FFN, st);
    if (e == hipSuccess) e = s->am1.alloc(cM, MD, st);
    if (e == hipSuccess) e = s->am2.alloc(cM, MD, st);
    if (e == hipSuccess) e = hipMalloc(&s->q16, (size_t)(cN * D * 2));
    if (e == hipSuccess) e = hipMalloc(&s->k16, (size_t)(NK * D * 2));
    const int64_t vbytes = (int64_t)D * vt_ld_for(NK) * 2;
    // key slots past a window's keys are read (and multiplied by zero
    // probabilities), so they must hold finite values: zero once
    if (e == hipSuccess) e = hipMalloc(&s->vt16, (size_t)vbytes);
    if (e == hipSuccess) e = hipMemsetAsync(s->vt16, 0, (size_t)vbytes, st);
    if (e != hipSuccess) return e;
    s->capN = cN;
    s->capM = cM;
    return hipSuccess;
}

// split the keys so that query tiles × splits give each CU one work-group
// (head dim 256 holds one work-group per CU)
int pick_splits(int64_t Nq, int64_t Nkv) {
    const int64_t qtiles = (Nq + 127) / 128, ktiles = (Nkv + 31) / 32;
    int64_t ns = std::max<int64_t>(1, (256 + qtiles - 1) / qtiles);
    ns = std::min(ns, std::max<int64_t>(1, ktiles / 4));  // at least 4 tiles per range
    const int64_t per = (ktiles + ns - 1) / ns;
    return (int)((ktiles + per - 1) / per);
}

}  // namespace

int memattn_run(const MemAttnModel *m, MemAttnState **sp, const float *curr, const float *src_pos, int64_t N,
                const float *prompt, const float *prompt_pos, int64_t M, int64_t n_ptr, const float *rope_q,
                const float *rope_k, float *out, hipStream_t st) {
    const int D = m->D, MD = m->MD, FFN = m->FFN;
    const int64_t Msp = M - n_ptr;
    if (N <= 0 || M <= 0 || n_ptr < 0 || Msp < 0 || !curr || !src_pos || !prompt || !prompt_pos || !rope_q ||
        !out || (Msp > 0 && !rope_k) || N > (1 << 20) || M > 46000) {
        set_error("s3e_mem_attn: bad arguments (N=%lld, M_total=%lld, pointer tokens=%lld)", (long long)N,
                  (long long)M, (long long)n_ptr);
        return S3E_ERR_INVALID;
    }
    if (!*sp) *sp = new MemAttnState;
    MemAttnState *s = *sp;
    hipError_t e = grow(m, s, N, M, st);
    const int nsS = pick_splits(N, N), nsC = pick_splits(N, M);
    const int64_t part = (int64_t)std::max(nsS, nsC) * N;
    // the residual GEMMs (N rows, D outputs) may split K through part_o: the
    // attention partials are merged before each of them on the same stream
    int64_t gws = 0;
    for (const MemAttnLayer &ly : m->layers)
        gws = std::max({gws, gemm_splitk_floats(ly.sa_out, N), gemm_splitk_floats(ly.ca_out, N),
                        gemm_splitk_floats(ly.fc2, N)});
    const int64_t need_o = std::max(part * D, gws);
    if (e == hipSuccess && (part > s->part_cap || need_o > s->part_o_floats)) {
        if (s->part_o) (void)hipFree(s->part_o);
        if (s->part_ml) (void)hipFree(s->part_ml);
        s->part_o = s->part_ml = nullptr;
        s->part_cap = s->part_o_floats = 0;
        e = hipMalloc(&s->part_o, (size_t)(need_o * 4));
        if (e == hipSuccess) e = hipMalloc(&s->part_ml, (size_t)(part * 2 * 4));
        if (e == hipSuccess) {
            s->part_cap = part;
            s->part_o_floats = need_o;
        }
    }
    if (e != hipSuccess) { set_error("s3e_mem_attn: %s", hipGetErrorString(e)); return S3E_ERR_NOMEM; }
#define MA_TRY(x)                                                                  \
    do {                                                                           \
        const hipError_t e_ = (x);                                                 \
        if (e_ != hipSuccess) {                                                    \
            set_error("s3e_mem_attn: %s (%s)", hipGetErrorString(e_), #x);         \
            return S3E_ERR_HIP;                                                    \
        }                                                                          \
    } while (0)
    // x = curr + 0.1·src_pos; memory + positions for the keys
    MA_TRY(launch_add_scaled(s->x, curr, src_pos, 0.1f, N * D, st));
    MA_TRY(launch_add_scaled(s->kvp, prompt, prompt_pos, 1.0f, M * MD, st));
    const float scale = 1.0f / std::sqrt((float)D);
    auto f32_act = [](float *p, int64_t ld) {
        Act a;
        a.kind = A_F32;
        a.x = p;
        a.ld = ld;
        return a;
    };
    auto attend = [&](int64_t Nkv, int ns) {
        AttnArgs aa;
        aa.q = s->q16;
        aa.k = s->k16;
        aa.vt = s->vt16;
        aa.Nq = (int)N;
        aa.Nkv = (int)Nkv;
        aa.NH = 1;
        aa.BH = 1;
        aa.hd = D;
        aa.scale = scale;
        aa.nsplit = ns;
        aa.part_o = s->part_o;
        aa.part_ml = s->part_ml;
        aa.out = f32_act(s->att, D);
        return launch_attn(aa, st);
    };
    auto qkv_args = [&](const float *bias, int64_t rows, int sel0, const float *freqs, int64_t rope_rows) {
        EpiArgs e3;
        e3.bias = bias;
        e3.E = D;
        e3.HD = D;
        e3.NH = 1;
        e3.grid = (int)rows;  // one window holding the whole sequence: position = token
        e3.window = (int)rows;
        e3.freqs = freqs;
        e3.rope_rows = (int)rope_rows;
        e3.sel0 = sel0;
        e3.q = s->q16;
        e3.k = s->k16;
        e3.vt = s->vt16;
        e3.vt_ld = (int)vt_ld_for(rows);
        return e3;
    };
    MA_TRY(launch_rows_quant(act_kind_for(m->layers[0].ca_k.kind), s->kvp, M, MD,
                             s->am1.as(act_kind_for(m->layers[0].ca_k.kind), MD), st));
    MA_TRY(launch_rows_quant(act_kind_for(m->layers[0].ca_v.kind), prompt, M, MD,
                             s->am2.as(act_kind_for(m->layers[0].ca_v.kind), MD), st));
    for (const MemAttnLayer &ly : m->layers) {
        // self-attention with RoPE on q and k
        const Act aq = s->an.as(act_kind_for(ly.sa_qkv.kind), D);
        MA_TRY(launch_layernorm(s->x, N, D, 1e-5f, ly.n1w, ly.n1b, aq, nullptr, st));
        MA_TRY(launch_gemm(ly.sa_qkv, aq, N, EPI_QKV, qkv_args(ly.sa_qkv_b, N, 0, rope_q, 0), st));
        MA_TRY(attend(N, nsS));
        const Act ao = s->an.as(act_kind_for(ly.sa_out.kind), D);
        MA_TRY(launch_rows_quant(ao.kind, s->att, N, D, ao, st));
        EpiArgs er;
        er.bias = ly.sa_out_b;
        er.y = s->x;
        er.ldy = D;
        er.ws = s->part_o;
        er.ws_cap = s->part_o_floats;
        MA_TRY(launch_gemm(ly.sa_out, ao, N, EPI_RESID, er, st));
        // cross-attention: keys from memory + positions, RoPE on the spatial ones
        const Act ac = s->an.as(act_kind_for(ly.ca_q.kind), D);
        MA_TRY(launch_layernorm(s->x, N, D, 1e-5f, ly.n2w, ly.n2b, ac, nullptr, st));
        MA_TRY(launch_gemm(ly.ca_q, ac, N, EPI_QKV, qkv_args(ly.ca_q_b, N, 0, rope_q, 0), st));
        MA_TRY(launch_gemm(ly.ca_k, s->am1.as(act_kind_for(ly.ca_k.kind), MD), M, EPI_QKV,
                           qkv_args(ly.ca_k_b, M, 1, Msp > 0 ? rope_k : nullptr, Msp), st));
        MA_TRY(launch_gemm(ly.ca_v, s->am2.as(act_kind_for(ly.ca_v.kind), MD), M, EPI_QKV,
                           qkv_args(ly.ca_v_b, M, 2, nullptr, 0), st));
        MA_TRY(attend(M, nsC));
        const Act ao2 = s->an.as(act_kind_for(ly.ca_out.kind), D);
        MA_TRY(launch_rows_quant(ao2.kind, s->att, N, D, ao2, st));
        er.bias = ly.ca_out_b;
        MA_TRY(launch_gemm(ly.ca_out, ao2, N, EPI_RESID, er, st));
        // FFN with ReLU
        const Act af = s->an.as(act_kind_for(ly.fc1.kind), D);
        MA_TRY(launch_layernorm(s->x, N, D, 1e-5f, ly.n3w, ly.n3b, af, nullptr, st));
        EpiArgs e1;
        e1.bias = ly.fc1_b;
        e1.relu = 1;
        e1.out = s->ah.as(act_kind_for(ly.fc2.kind), FFN);
        MA_TRY(launch_gemm(ly.fc1, af, N, EPI_GELU, e1, st));
        er.bias = ly.fc2_b;
        MA_TRY(launch_gemm(ly.fc2, e1.out, N, EPI_RESID, er, st));
    }
    MA_TRY(launch_layernorm(s->x, N, D, 1e-5f, m->nw, m->nb, f32_act(out, D), nullptr, st));
#undef MA_TRY
    return S3E_OK;
}

}  // namespace s3e
