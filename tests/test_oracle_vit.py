"""Pins the oracle's SAM 3 ViT composition (oracle/orc_vit.c) independently.

The oracle strings ggml's operators together the way sam3_build_vit_prefix_graph
and sam3_vit_block_forward do (sam3.cpp:3710-3830).  This file restates the
same backbone in float64 torch, following the PyTorch side of the model
(tests/dump_vit_reference.py:26-102, 177-242 in the reference: F.conv2d patch
embedding, tiled absolute position embedding, F.layer_norm, the qkv reshape to
(L, 3, NH, HD), view_as_complex RoPE on q and k, softmax attention,
window_partition / window_unpartition, erf GELU), with the weights read back
out of the model file.  Nothing here calls the oracle's own kernels, so a
swapped q/k split, a transposed head split, a wrong window order, RoPE on V or
a dropped residual shows up as a distance far above the tolerance.  The
mutation tests plant exactly those mistakes in the torch restatement (on the
CPU) and check that each one is detected.  No GPU.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle_lib as orc

# 168 px / 14 = 12×12 tokens; window 4 → 3×3 windows of 16 tokens; E = 128 with
# two heads of the reference's head dim 64; block 1 is global.
IMG, P, E, NH, WS = 168, 14, 128, 2, 4
G, HD = IMG // P, E // NH


@pytest.fixture(scope="module")
def s3e_mod():
    import s3e

    return s3e


def _model(s3e_mod, tmp_path_factory, ftype):
    p = str(tmp_path_factory.mktemp("vit") / f"vit_{ftype}.ggml")
    s3e_mod.synth_write(p, img_size=IMG, embed_dim=E, heads=NH, depth=2, window=WS, global_idx=(1,),
                        ftype=ftype, seed=11, std=0.05, random_affine=True, neck=0)
    return p, orc.read_model_file(p)


@pytest.fixture(scope="module")
def f32_model(s3e_mod, tmp_path_factory):
    return _model(s3e_mod, tmp_path_factory, "f32")


@pytest.fixture(scope="module")
def f16_model(s3e_mod, tmp_path_factory):
    return _model(s3e_mod, tmp_path_factory, "f16")


def _t(tensors, name):
    return torch.from_numpy(np.asarray(tensors[name][2], np.float64).copy())


def _r16(t, on):
    """ggml's F16 vec_dot rounds the activation operand to fp16 first."""
    return torch.from_numpy(t.numpy().astype(np.float32).astype(np.float16).astype(np.float64)) if on else t


# ---- the PyTorch semantics (dump_vit_reference.py:26-102) ----------------------
def axial_cis(dim, end_x, end_y, scale=1.0, theta=10000.0):
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 4, dtype=torch.float64)[: dim // 4] / dim))
    t = torch.arange(end_x * end_y, dtype=torch.float64)
    tx, ty = (t % end_x) * scale, torch.div(t, end_x, rounding_mode="floor") * scale
    fx, fy = torch.outer(tx, freqs), torch.outer(ty, freqs)
    return torch.cat([torch.polar(torch.ones_like(fx), fx), torch.polar(torch.ones_like(fy), fy)], dim=-1)


def apply_rotary(x, freqs_cis):
    xc = torch.view_as_complex(x.reshape(*x.shape[:-1], -1, 2).contiguous())
    return torch.view_as_real(xc * freqs_cis).flatten(3)


def window_partition(x, ws):
    B, H, W, C = x.shape
    x = x.view(B, H // ws, ws, W // ws, ws, C)
    return x.permute(0, 1, 3, 2, 4, 5).reshape(-1, ws, ws, C)


def window_unpartition(w, ws, H, W):
    B = w.shape[0] // (H * W // ws // ws)
    x = w.reshape(B, H // ws, W // ws, ws, ws, -1)
    return x.permute(0, 1, 3, 2, 4, 5).reshape(B, H, W, -1)


def torch_prefix(tensors, chw, f16=False):
    # ne [P,P,3,E] → [E,3,P,P]; stored F32 in F16 files ("embed" names), the
    # loader coerces it to the registered F16 type (sam3.cpp:3091-3194, :2528)
    w = _r16(_t(tensors, "vit.patch_embed.proj.weight"), f16)
    img = _r16(torch.from_numpy(chw.astype(np.float64)), f16)[None]
    x = F.conv2d(img, w, stride=P).permute(0, 2, 3, 1)  # [1,G,G,E]
    pos = _t(tensors, "vit.pos_embed")  # ne [E,pg,pg,1] → [1,pg,pg,E]
    pg = pos.shape[1]
    tiled = pos.permute(0, 3, 1, 2).tile([1, 1, G // pg + 1, G // pg + 1])[:, :, :G, :G].permute(0, 2, 3, 1)
    x = x + tiled
    return F.layer_norm(x, [E], _t(tensors, "vit.ln_pre.weight"), _t(tensors, "vit.ln_pre.bias"), eps=1e-5)


def torch_block(tensors, i, x, glob, f16=False, mutate=None):
    p = f"vit.blocks.{i}."
    shortcut = x
    xn = F.layer_norm(x, [E], _t(tensors, p + "norm1.weight"), _t(tensors, p + "norm1.bias"), eps=1e-5)
    if not glob:
        if mutate == "window_transpose":  # windows and in-window positions taken column-major
            xn = xn.transpose(1, 2)
        xn = window_partition(xn, WS)
    B, Hc, Wc, _ = xn.shape
    L = Hc * Wc
    qkv = F.linear(_r16(xn, f16), _t(tensors, p + "attn.qkv.weight"), _t(tensors, p + "attn.qkv.bias"))
    if mutate == "head_split":  # (HD, NH) instead of (NH, HD) inside each of q, k, v
        qkv = qkv.reshape(B, L, 3, HD, NH).transpose(3, 4)
    qkv = qkv.reshape(B, L, 3, NH, HD)
    q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)  # [B, NH, L, HD]
    if mutate == "swap_qk":
        q, k = k, q
    fc = _t(tensors, p + "attn.freqs_cis")  # ne [2, HD/2, N] → [N, HD/2, 2]
    freqs = torch.complex(fc[..., 0], fc[..., 1])
    if mutate != "no_rope":
        q, k = apply_rotary(q, freqs), apply_rotary(k, freqs)
    if mutate == "rope_v":
        v = apply_rotary(v, freqs)
    s = torch.matmul(q, k.transpose(-1, -2)) / math.sqrt(HD)
    o = torch.matmul(torch.softmax(s, dim=-1), v)
    o = o.view(B, NH, Hc, Wc, HD).permute(0, 2, 3, 1, 4).reshape(B, Hc, Wc, E)
    o = F.linear(_r16(o, f16), _t(tensors, p + "attn.proj.weight"), _t(tensors, p + "attn.proj.bias"))
    if not glob:
        o = window_unpartition(o, WS, G, G)
        if mutate == "window_transpose":
            o = o.transpose(1, 2)
    x = o if mutate == "no_residual" else shortcut + o
    shortcut = x
    xn = F.layer_norm(x, [E], _t(tensors, p + "norm2.weight"), _t(tensors, p + "norm2.bias"), eps=1e-5)
    h = F.linear(_r16(xn, f16), _t(tensors, p + "mlp.lin1.weight"), _t(tensors, p + "mlp.lin1.bias"))
    h = F.gelu(h, approximate="tanh") if mutate == "gelu_tanh" else F.gelu(h)
    h = F.linear(_r16(h, f16), _t(tensors, p + "mlp.lin2.weight"), _t(tensors, p + "mlp.lin2.bias"))
    return shortcut + h


def _image(seed=5):
    img = np.random.default_rng(seed).integers(0, 256, (IMG, IMG, 3), dtype=np.uint8)
    return orc.preprocess_sam3(img, IMG)


def _tok(x):
    return x.reshape(G * G, E).numpy() if isinstance(x, torch.Tensor) else x


def _grid(x):
    return torch.from_numpy(np.asarray(x, np.float64).reshape(1, G, G, E))


# ---- the tests -------------------------------------------------------------------
def test_freqs_cis_closed_form(f32_model):
    """The file's tables equal compute_axial_cis (window: 4×4 grid, scale 1;
    global: 12×12 grid, scale window/grid) — test_phase3.cpp:118-178's
    known-answer rule, at its 1e-5 tolerance."""
    _, tensors = f32_model
    for i, (side, scale) in ((0, (WS, 1.0)), (1, (G, WS / G))):
        fc = np.asarray(tensors[f"vit.blocks.{i}.attn.freqs_cis"][2], np.float64)
        ref = axial_cis(HD, side, side, scale)
        assert fc.shape == (side * side, HD // 2, 2)
        assert np.max(np.abs(fc[..., 0] - ref.real.numpy())) < 1e-5
        assert np.max(np.abs(fc[..., 1] - ref.imag.numpy())) < 1e-5


def test_prefix_vs_torch(f32_model):
    path, tensors = f32_model
    om = orc.OracleModel(path)
    chw = _image()
    got = om.prefix(chw)
    ref = _tok(torch_prefix(tensors, chw))
    assert orc.rel_l2(got, ref) < 1e-6


@pytest.mark.parametrize("bi,glob", [(0, False), (1, True)])
def test_block_vs_torch(f32_model, bi, glob):
    path, tensors = f32_model
    om = orc.OracleModel(path)
    x = np.random.default_rng(bi).standard_normal((G * G, E)).astype(np.float32)
    got = om.block(bi, x)
    ref = _tok(torch_block(tensors, bi, _grid(x), glob))
    assert orc.rel_l2(got, ref) < 1e-6
    # the block changed its input substantially, so the bound says something
    assert orc.rel_l2(got, x) > 0.05


def test_encode_vs_torch(f32_model):
    path, tensors = f32_model
    om = orc.OracleModel(path)
    chw = _image(9)
    x = torch_prefix(tensors, chw)
    x = torch_block(tensors, 0, x, False)
    x = torch_block(tensors, 1, x, True)
    assert orc.rel_l2(om.encode(chw), _tok(x)) < 1e-6


def test_f16_file_vs_torch(f16_model):
    """F16 weights: ggml rounds each linear's (and the im2col's) activation
    operand to fp16; the restatement rounds at the same places.  A value
    computed in f32 by the oracle and in f64 here can round to neighbouring
    fp16 values, one ulp (4.9e-4 relative) apart: the restatement evaluated
    in float32 is itself 1-2e-5 from its float64 evaluation on these blocks,
    so the bound is 5e-5.  Leaving the roundings out moves the result by
    about 1.2e-4, beyond that bound."""
    path, tensors = f16_model
    om = orc.OracleModel(path)
    chw = _image(3)
    x = torch_prefix(tensors, chw, f16=True)
    assert orc.rel_l2(om.prefix(chw), _tok(x)) < 1e-5
    for bi, glob in ((0, False), (1, True)):
        xin = np.random.default_rng(20 + bi).standard_normal((G * G, E)).astype(np.float32)
        got = om.block(bi, xin)
        assert orc.rel_l2(got, _tok(torch_block(tensors, bi, _grid(xin), glob, f16=True))) < 5e-5, bi
        assert orc.rel_l2(got, _tok(torch_block(tensors, bi, _grid(xin), glob, f16=False))) > 8e-5, bi


@pytest.mark.parametrize("mutation", ["swap_qk", "head_split", "window_transpose", "no_rope", "rope_v",
                                      "no_residual", "gelu_tanh"])
def test_planted_mistakes_are_detected(f32_model, mutation):
    """Each plausible composition mistake, planted in the torch restatement,
    moves the result at least ten times beyond the 1e-6 bound the oracle
    meets (the oracle sits at 7e-8; tanh-GELU for erf-GELU, the smallest
    mistake, moves it by 8e-5)."""
    path, tensors = f32_model
    om = orc.OracleModel(path)
    x = np.random.default_rng(0).standard_normal((G * G, E)).astype(np.float32)
    got = om.block(0, x)
    bad = _tok(torch_block(tensors, 0, _grid(x), False, mutate=mutation))
    assert orc.rel_l2(got, bad) > 1e-5, (mutation, orc.rel_l2(got, bad))


# ---- sub-stage hooks (sam3_test_run_vit_block_stage / _prefix_stage) ---------------
BS = {n: i for i, n in enumerate(orc.BLOCK_STAGES)}
PS = {n: i for i, n in enumerate(orc.PREFIX_STAGES)}


def _stages_block(om, bi, x, glob):
    """The block as the reference's stage sequence: each stage fed the previous
    stage's output, residual adds in float32 as ggml_add does."""
    nw = (G // WS) ** 2
    h, ne = om.block_stage(bi, BS["NORM1"], x, (E, G, G, 1))
    if not glob:
        h, ne = om.block_stage(bi, BS["WINDOW_PART"], h, ne)
        assert ne == (E, WS, WS, nw)
    h, ne = om.block_stage(bi, BS["QKV_PROJ"], h, ne)
    assert ne[0] == 3 * E
    h, ne = om.block_stage(bi, BS["ATTN_CORE"], h, ne)
    assert ne[0] == E
    h, ne = om.block_stage(bi, BS["ATTN_PROJ"], h, ne)
    if not glob:
        h, ne = om.block_stage(bi, BS["WINDOW_UNPART"], h, ne)
    assert ne == (E, G, G, 1)
    x1 = (x.ravel() + h).astype(np.float32)
    h, _ = om.block_stage(bi, BS["NORM2"], x1, ne)
    y, _ = om.block_stage(bi, BS["MLP"], h, ne)
    return (x1 + y).astype(np.float32)


@pytest.mark.parametrize("bi,glob", [(0, False), (1, True)])
def test_block_stages_compose_to_block(f32_model, f16_model, bi, glob):
    """Chaining the stage hooks reproduces the block bit for bit, and MLP is
    MLP_FC1 → MLP_GELU → MLP_FC2."""
    for path, _ in (f32_model, f16_model):
        om = orc.OracleModel(path)
        x = np.random.default_rng(30 + bi).standard_normal((G * G, E)).astype(np.float32)
        assert np.array_equal(_stages_block(om, bi, x, glob), om.block(bi, x).ravel())
        h, ne = om.block_stage(bi, BS["NORM2"], x, (E, G, G, 1))
        a, ne1 = om.block_stage(bi, BS["MLP_FC1"], h, ne)
        a, _ = om.block_stage(bi, BS["MLP_GELU"], a, ne1)
        a, ne2 = om.block_stage(bi, BS["MLP_FC2"], a, ne1)
        assert ne2 == ne and np.array_equal(a, om.block_stage(bi, BS["MLP"], h, ne)[0])


def test_stages_vs_torch(f32_model):
    """Each stage against its torch restatement: the window operators against
    window_partition / window_unpartition, the attention core against RoPE +
    softmax attention, GELU against erf-GELU."""
    path, tensors = f32_model
    om = orc.OracleModel(path)
    rng = np.random.default_rng(7)
    x = rng.standard_normal((G * G, E)).astype(np.float32)
    w, ne = om.block_stage(0, BS["WINDOW_PART"], x, (E, G, G, 1))
    ref = window_partition(_grid(x), WS).numpy()
    assert np.array_equal(w, ref.ravel().astype(np.float32))
    back, ne2 = om.block_stage(0, BS["WINDOW_UNPART"], w, ne)
    assert ne2 == (E, G, G, 1) and np.array_equal(back, x.ravel())
    nw = (G // WS) ** 2
    qkv = rng.standard_normal((nw, WS * WS, 3 * E)).astype(np.float32)
    got, one = om.block_stage(0, BS["ATTN_CORE"], qkv, (3 * E, WS, WS, nw))
    assert one == (E, WS, WS, nw)
    t = torch.from_numpy(qkv.astype(np.float64)).reshape(nw, WS * WS, 3, NH, HD)
    q, k, v = t.permute(2, 0, 3, 1, 4).unbind(0)
    fc = _t(tensors, "vit.blocks.0.attn.freqs_cis")
    freqs = torch.complex(fc[..., 0], fc[..., 1])
    q, k = apply_rotary(q, freqs), apply_rotary(k, freqs)
    o = torch.matmul(torch.softmax(torch.matmul(q, k.transpose(-1, -2)) / math.sqrt(HD), dim=-1), v)
    ref = o.permute(0, 2, 1, 3).reshape(-1).numpy()  # [B][N][NH][HD]
    assert orc.rel_l2(got, ref) < 1e-6
    a = rng.standard_normal((16, 592)).astype(np.float32) * 3
    g, _ = om.block_stage(0, BS["MLP_GELU"], a, (592, 16, 1, 1))
    ref = torch.nn.functional.gelu(torch.from_numpy(a.astype(np.float64))).numpy()
    assert np.max(np.abs(g - ref.ravel())) < 1e-6


def test_prefix_stages_compose(f32_model, f16_model):
    for path, tensors in (f32_model, f16_model):
        om = orc.OracleModel(path)
        chw = _image(13)
        p, ne = om.prefix_stage(PS["PATCH_EMBED"], chw, (IMG, IMG, 3, 1))
        assert ne == (E, G, G, 1)
        p, ne = om.prefix_stage(PS["POS_ADD"], p, ne)
        p, ne = om.prefix_stage(PS["LN_PRE"], p, ne)
        assert np.array_equal(p, om.prefix(chw).ravel())
        # ln_pre = ggml_norm, then ·w + b
        n, _ = om.prefix_stage(PS["LN_PRE_NORM"], p, ne)
        ref = F.layer_norm(torch.from_numpy(p.astype(np.float64)).reshape(-1, E), [E], eps=1e-5).numpy()
        assert orc.rel_l2(n, ref.ravel()) < 1e-6
        # im2col rows are the image patches in (c, ky, kx) order, in the kernel's type
        cols, cne = om.prefix_stage(PS["PATCH_IM2COL"], chw, (IMG, IMG, 3, 1))
        assert cne == (3 * P * P, G, G, 1)
        ref = chw.reshape(3, G, P, G, P).transpose(1, 3, 0, 2, 4).reshape(G * G, 3 * P * P)
        f16 = tensors["vit.patch_embed.proj.weight"][0] == orc.F16 or path.endswith("f16.ggml")
        if f16:
            ref = ref.astype(np.float16).astype(np.float32)
        assert np.array_equal(cols, ref.ravel())
        # the mul_mat stages take an F16 input and convert the kernel to F16
        raw, rne = om.prefix_stage(PS["PATCH_MULMAT_RAW"], cols, cne)
        assert rne == (G * G, E, 1, 1)
        mm, mne = om.prefix_stage(PS["PATCH_MULMAT"], cols, cne)
        assert mne == (G, G, E, 1) and np.array_equal(mm, raw)
        w16 = np.asarray(tensors["vit.patch_embed.proj.weight"][2], np.float32).reshape(E, -1)
        w16 = w16.astype(np.float16).astype(np.float64)
        a16 = cols.reshape(G * G, -1).astype(np.float16).astype(np.float64)
        assert orc.rel_l2(raw, (w16 @ a16.T).ravel()) < 1e-6
        if f16:  # the same products as the conv itself: equal up to the transpose
            conv, _ = om.prefix_stage(PS["PATCH_EMBED"], chw, (IMG, IMG, 3, 1))
            assert np.array_equal(raw.reshape(E, G * G).T.ravel(), conv)
