"""GPU parity of every ViT sub-stage (s3e_vit_block_stage /
s3e_vit_prefix_stage, the engine's sam3_test_run_vit_block_stage and
sam3_test_run_vit_prefix_stage) against the oracle's stage functions, each
stage fed the same input: the oracle's own chain of stages from one image.

A quantized model re-quantizes each linear's input to Q8 per 32-block, so
a last-bit difference in a stage output can flip a code of the next
quantization.  For the stages that feed a quantization (the attention core
→ proj, GELU → fc2, the linears → the next stage) the test reports how many
Q8 codes differ when both outputs are quantized the oracle's way: that is
where the GPU's end-to-end distance from the CPU path starts.

Bounds: LayerNorm, window partition / unpartition, im2col, position add:
bit-exact.  Linears: relative L2 ≤ 1e-6 (only fp32 accumulation order
differs), or twice ggml's own AVX2-vs-generic distance where that is larger
(Q4_1 fc2: its input is the positive-biased GELU output, so the minimum term
m·s and the scaled block sums are large and cancel, and ggml's two orders
are 9.4e-6 apart).  Attention core: ≤ 2e-6 with the split-fp16 operands of
quantized models, ≤ 2e-3 with the fp16 operands of F16 models.  MLP (fc1 →
GELU → re-quantization → fc2): at most twice ggml's own order distance on
the same input — a last-bit difference of fc1 flips a few Q8 codes of fc2's
input.  GELU: the engine's erf is a float approximation (relative error
3.1e-7 in erfc) where the oracle calls glibc's erff; each output may differ
by what those errors move 0.5·x·(1 + erf) by, plus two roundings.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle_lib as orc

pytestmark = pytest.mark.gpu
orc.LIB.orc_set_variant.argtypes = [ctypes.c_int]

BS = {n: i for i, n in enumerate(orc.BLOCK_STAGES)}
PS = {n: i for i, n in enumerate(orc.PREFIX_STAGES)}
IMG, P, E, WS = 336, 14, 1024, 8
G = IMG // P
FTYPES = ["q4_0", "q8_0", "q4_1", "f16"]


@pytest.fixture(scope="module", params=FTYPES)
def small(request, tmpdir_session, ctx):
    import s3e

    ft = request.param
    path = os.path.join(str(tmpdir_session), f"stages_{ft}.ggml")
    s3e.synth_write(path, img_size=IMG, patch=P, embed_dim=E, depth=2, heads=16, window=WS, global_idx=(1,),
                    ftype=ft, seed=5, std=0.02, random_affine=True, neck=0)
    om = orc.OracleModel(path)
    gm = s3e.Model(ctx, path)
    st = s3e.State(ctx, gm)
    img = np.random.default_rng(3).integers(0, 256, (IMG, IMG, 3), dtype=np.uint8)
    chw = orc.preprocess_sam3(img, IMG)
    yield ft, om, st, chw
    st.free()
    gm.free()


def _q8_flips(vdt, got, ref, k):
    """Q8 codes (and block scales) that differ when both rows are quantized."""
    rows = got.size // k
    a = orc.split_q8(vdt, orc.from_float(vdt, got.reshape(rows, k)), rows, k)
    b = orc.split_q8(vdt, orc.from_float(vdt, ref.reshape(rows, k)), rows, k)
    return int(np.count_nonzero(a[0] != b[0])), int(np.count_nonzero(a[1] != b[1])), a[0].size


def _ulps(got, ref):
    g = got.astype(np.float32).view(np.int32).astype(np.int64)
    r = ref.astype(np.float32).view(np.int32).astype(np.int64)
    g = np.where(g < 0, -(g & 0x7FFFFFFF), g)
    r = np.where(r < 0, -(r & 0x7FFFFFFF), r)
    return np.abs(g - r)


def _order_gap(fn, ref):
    """Distance of ggml's generic evaluation order from the AVX2 one."""
    orc.LIB.orc_set_variant(1)
    try:
        alt = fn()
    finally:
        orc.LIB.orc_set_variant(0)
    return orc.rel_l2(alt, ref)


def _chain(om, bi, x0, glob):
    """Oracle inputs of every stage of block bi."""
    ins = {}
    ne = (E, G, G, 1)
    ins["NORM1"] = (x0, ne)
    h, ne_h = om.block_stage(bi, BS["NORM1"], x0, ne)
    if not glob:
        ins["WINDOW_PART"] = (h, ne_h)
        h, ne_h = om.block_stage(bi, BS["WINDOW_PART"], h, ne_h)
    ins["QKV_PROJ"] = (h, ne_h)
    h, ne_h = om.block_stage(bi, BS["QKV_PROJ"], h, ne_h)
    ins["ATTN_CORE"] = (h, ne_h)
    h, ne_h = om.block_stage(bi, BS["ATTN_CORE"], h, ne_h)
    ins["ATTN_PROJ"] = (h, ne_h)
    h, ne_h = om.block_stage(bi, BS["ATTN_PROJ"], h, ne_h)
    if not glob:
        ins["WINDOW_UNPART"] = (h, ne_h)
        h, ne_h = om.block_stage(bi, BS["WINDOW_UNPART"], h, ne_h)
    x1 = (x0.ravel() + h).astype(np.float32)
    ins["NORM2"] = (x1, ne)
    h, _ = om.block_stage(bi, BS["NORM2"], x1, ne)
    ins["MLP_FC1"] = (h, ne)
    ins["MLP"] = (h, ne)
    f, ne_f = om.block_stage(bi, BS["MLP_FC1"], h, ne)
    ins["MLP_GELU"] = (f, ne_f)
    g, _ = om.block_stage(bi, BS["MLP_GELU"], f, ne_f)
    ins["MLP_FC2"] = (g, ne_f)
    return ins


@pytest.mark.parametrize("bi", [0, 1])
def test_block_stages(small, bi):
    ft, om, st, chw = small
    glob = bi == 1
    x0 = om.prefix(chw)
    ins = _chain(om, bi, x0, glob)
    vdt = orc.VEC_DOT[{"q4_0": orc.Q4_0, "q8_0": orc.Q8_0, "q4_1": orc.Q4_1, "f16": orc.F16}[ft]]
    bad = []
    for name, (x, ne) in ins.items():
        stage = BS[name]
        ref, one = om.block_stage(bi, stage, x, ne)
        got, gne = st.block_stage(bi, stage, x, ne)
        assert gne == one, name
        rl, ma = orc.rel_l2(got, ref), orc.max_abs(got, ref)
        msg = f"{ft} block {bi} {name}: rel_l2={rl:.3e} max_abs={ma:.3e}"
        gap = 0.0
        if name in ("MLP_FC2", "MLP"):
            gap = _order_gap(lambda: om.block_stage(bi, stage, x, ne)[0], ref)
            msg += f" | ggml order gap {gap:.3e} (x{rl / max(gap, 1e-30):.2f})"
        if name in ("ATTN_CORE", "MLP_GELU") and vdt in (orc.Q8_0, orc.Q8_1):
            fq, fd, n = _q8_flips(vdt, got, ref, one[0])
            msg += f" | Q8 codes differing {fq}/{n} ({fq / n:.2e}), scales {fd}"
        if name == "MLP_GELU":
            msg += f" | outputs differing {np.count_nonzero(got != ref)}/{got.size}"
            xa = np.abs(x.astype(np.float64))
            w = np.where(xa > 0, 2 * np.abs(ref.astype(np.float64)) / np.maximum(xa, 1e-30), 1.0)
            lim = 0.5 * xa * (2.4e-7 + 6e-7 * w) + 2 * np.spacing(np.abs(ref))
            excess = np.abs(got.astype(np.float64) - ref) - lim
        print(msg, flush=True)
        if name in ("NORM1", "NORM2", "WINDOW_PART", "WINDOW_UNPART"):
            ok = np.array_equal(got, ref)
        elif name in ("QKV_PROJ", "ATTN_PROJ", "MLP_FC1", "MLP_FC2"):
            ok = rl <= max(1e-6, 2 * gap)
        elif name == "ATTN_CORE":
            ok = rl <= (2e-3 if ft == "f16" else 2e-6)
        elif name == "MLP_GELU":
            ok = excess.max() <= 0
        else:  # MLP
            ok = rl <= 2 * gap
        if not ok:
            bad.append(name)
    assert not bad, bad


def test_prefix_stages(small):
    ft, om, st, chw = small
    ne = (IMG, IMG, 3, 1)
    ins = {"PATCH_EMBED": (chw, ne), "PATCH_IM2COL": (chw, ne)}
    cols, cne = om.prefix_stage(PS["PATCH_IM2COL"], chw, ne)
    ins["PATCH_MULMAT_RAW"] = ins["PATCH_MULMAT"] = (cols, cne)
    p, pne = om.prefix_stage(PS["PATCH_EMBED"], chw, ne)
    ins["POS_ADD"] = (p, pne)
    p, _ = om.prefix_stage(PS["POS_ADD"], p, pne)
    ins["LN_PRE_NORM"] = ins["LN_PRE"] = (p, pne)
    for name, (x, xne) in ins.items():
        ref, one = om.prefix_stage(PS[name], x, xne)
        got, gne = st.prefix_stage(PS[name], x, xne)
        assert gne == one, name
        rl = orc.rel_l2(got, ref)
        print(f"{ft} prefix {name}: rel_l2={rl:.3e} max_abs={orc.max_abs(got, ref):.3e}", flush=True)
        if name in ("PATCH_IM2COL", "POS_ADD", "LN_PRE_NORM", "LN_PRE"):
            assert np.array_equal(got, ref), name
        else:
            assert rl <= 1e-6, name


def test_stage_rejects(small):
    import s3e

    ft, om, st, chw = small
    x = np.zeros(E * 4, np.float32)
    with pytest.raises(s3e.S3EError):
        st.block_stage(0, BS["QKV_PROJ"], x, (E + 32, 4, 1, 1))  # wrong ne0
    with pytest.raises(s3e.S3EError):
        st.block_stage(0, 11, x, (E, 4, 1, 1))  # no such stage
    with pytest.raises(s3e.S3EError):
        st.block_stage(2, BS["NORM1"], x, (E, 4, 1, 1))  # no such block
    with pytest.raises(s3e.S3EError):
        st.block_stage(0, BS["ATTN_CORE"], np.zeros(3 * E * 10, np.float32), (3 * E, 10, 1, 1))  # RoPE table length
    with pytest.raises(s3e.S3EError):
        st.prefix_stage(PS["PATCH_EMBED"], x, (E, 4, 1, 1))
