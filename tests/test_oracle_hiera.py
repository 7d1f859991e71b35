"""Pins the oracle's SAM 2.x encoder (oracle/orc_hiera.c) before it is trusted.

Independent checks, all on the CPU:
* the tanh-GELU table against float64 tanh-GELU (every fp16 input in
  (−10, 10) within one fp16 rounding of the exact value) and its ±10 clamps;
* the background positional-embedding resize against torch's bicubic
  interpolation (a = −0.75, align_corners=False) in float64;
* the patch embedding (7×7, stride 4, pad 3) against torch conv2d, plus the
  window-tiled positional embedding;
* every block of a small Hiera (padded windows, Q pooling inside windows and
  at a stage change, a global block, dimension projection) against a float64
  torch restatement of the PyTorch MultiScaleBlock semantics the reference
  graph follows (window_partition / unpartition with F.pad, max_pool2d on Q,
  scaled-dot-product attention), with exact tanh-GELU: the oracle's fp16
  GELU table is the only intended difference;
* the FPN (lateral 1×1, nearest ×2 top-down on the listed levels, scalp)
  against torch;
* the SAM 2 normalisation against its closed form.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle_lib as orc


def t64(a):
    return torch.from_numpy(np.asarray(a, np.float64))


def test_gelu_table_vs_f64():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = h.view(np.float16).astype(np.float32)
    ok = np.isfinite(x) & (x > -10) & (x < 10)
    xs = x[ok]
    got = orc.gelu_tanh(xs)
    xd = xs.astype(np.float64)
    ref = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * xd * (1 + 0.044715 * xd * xd)))
    # the table holds fp16 values: within one fp16 rounding (half an ulp of the
    # result) of the exact tanh-GELU, plus the fp32 evaluation error of
    # 0.5·x·(1 + tanh(·)), which cancels for negative x (a few ulp of 1, times |x|/2)
    assert np.all(got.astype(np.float16).astype(np.float32) == got)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    err = np.abs(got - ref)
    assert np.all(err <= 0.5 * ulp + 3e-7 * np.abs(xd) + 1e-12)
    assert np.mean(err <= 0.5 * ulp + 1e-12) > 0.99  # almost all are the correctly rounded value
    # clamps
    edge = np.array([-10.0, -11.5, -1e4, 10.0, 12.25, 3e4], np.float32)
    assert np.array_equal(orc.gelu_tanh(edge), np.array([0, 0, 0, 10.0, 12.25, 3e4], np.float32))


@pytest.mark.parametrize("hi,wi,ho,wo", [(7, 7, 64, 64), (14, 14, 256, 256), (5, 9, 12, 7)])
def test_bicubic_vs_torch(hi, wi, ho, wo):
    rng = np.random.default_rng(hi * wi)
    src = rng.standard_normal((3, hi, wi)).astype(np.float32)
    dst = np.empty((3, ho, wo), np.float32)
    orc.LIB.orc_bicubic(orc.ptr(src), 3, hi, wi, orc.ptr(dst), ho, wo)
    ref = F.interpolate(t64(src)[None], size=(ho, wo), mode="bicubic", align_corners=False)[0].numpy()
    assert np.max(np.abs(dst - ref)) < 2e-5 * max(1.0, np.abs(ref).max())


def test_preprocess_sam2_closed_form():
    rng = np.random.default_rng(1)
    img = rng.integers(0, 256, (32, 32, 3), dtype=np.uint8)
    chw = orc.preprocess_sam2(img, 32)
    mean = np.array([0.485, 0.456, 0.406], np.float32)[:, None, None]
    std = np.array([0.229, 0.224, 0.225], np.float32)[:, None, None]
    ref = ((img.astype(np.float32) / np.float32(255)).transpose(2, 0, 1) - mean) / std
    assert np.array_equal(chw, ref.astype(np.float32))


# ---- a small Hiera: padding, Q pooling in windows, a global block -----------
SMALL = dict(embed_dim=32, num_heads=1, stages=(1, 2, 3, 2), global_idx=(4,), window_spec=(8, 6, 4, 4), bkg=(5, 5))


@pytest.fixture(scope="module")
def small_hiera(tmp_path_factory):
    import s3e

    p = str(tmp_path_factory.mktemp("hiera") / "small_f32.ggml")
    s3e.synth_write_sam2(p, "hiera_t", img_size=192, ftype="f32", seed=3, std=0.08, random_affine=True,
                         neck_dim=64, **SMALL)
    return p, orc.OracleHiera(p), orc.read_model_file(p)


def _w(tensors, name):
    return t64(tensors[name][2])


def _table_gelu(h):
    """ggml's fp16-table GELU (pinned by test_gelu_table_vs_f64) on float64 data."""
    return t64(orc.gelu_tanh(h.numpy().astype(np.float32)))


def _torch_block(x, H, W, tensors, bi, info, gelu=lambda h: F.gelu(h, approximate="tanh")):
    """PyTorch MultiScaleBlock semantics in float64 (x: [H, W, Cin])."""
    p = f"hiera.blocks.{bi}."
    Cin, Cout, NH, ws, qs = info["dim_in"], info["dim_out"], info["heads"], info["window"], info["q_stride"]
    HD = Cout // NH
    x = t64(x).reshape(H, W, Cin)
    normed = F.layer_norm(x, (Cin,), _w(tensors, p + "norm1.weight"), _w(tensors, p + "norm1.bias"), eps=1e-6)

    def pool(t):  # [h, w, C] → max 2×2
        return F.max_pool2d(t.permute(2, 0, 1)[None], 2, 2)[0].permute(1, 2, 0)

    if Cin != Cout:
        sc = normed @ _w(tensors, p + "proj.weight").T + _w(tensors, p + "proj.bias")
        if qs:
            sc = pool(sc)
    elif qs:
        sc = pool(x)
    else:
        sc = x
    if ws > 0:
        ph, pw = (ws - H % ws) % ws, (ws - W % ws) % ws
        xp = F.pad(normed, (0, 0, 0, pw, 0, ph))
        Hp, Wp = H + ph, W + pw
        win = xp.view(Hp // ws, ws, Wp // ws, ws, Cin).permute(0, 2, 1, 3, 4).reshape(-1, ws, ws, Cin)
    else:
        win = normed[None]
    nW, wh, ww = win.shape[0], win.shape[1], win.shape[2]
    qkv = win.reshape(nW, wh * ww, Cin) @ _w(tensors, p + "attn.qkv.weight").T + _w(tensors, p + "attn.qkv.bias")
    qkv = qkv.reshape(nW, wh * ww, 3, NH, HD)
    q, k, v = qkv.unbind(2)
    if qs:
        q = q.reshape(nW, wh, ww, Cout).permute(0, 3, 1, 2)
        q = F.max_pool2d(q, 2, 2).permute(0, 2, 3, 1)
        qh, qw = q.shape[1], q.shape[2]
        q = q.reshape(nW, qh * qw, NH, HD)
    else:
        qh, qw = wh, ww
    att = torch.softmax(torch.einsum("bqhd,bkhd->bhqk", q, k) / math.sqrt(HD), dim=-1)
    o = torch.einsum("bhqk,bkhd->bqhd", att, v).reshape(nW, qh * qw, Cout)
    o = o @ _w(tensors, p + "attn.proj.weight").T + _w(tensors, p + "attn.proj.bias")
    Ht, Wt = (H // 2, W // 2) if qs else (H, W)
    if ws > 0:
        wo = qh
        nh, nw = (Ht + wo - 1) // wo, (Wt + wo - 1) // wo
        assert nh * nw == nW
        o = o.reshape(nh, nw, wo, wo, Cout).permute(0, 2, 1, 3, 4).reshape(nh * wo, nw * wo, Cout)[:Ht, :Wt]
    else:
        o = o.reshape(Ht, Wt, Cout)
    r1 = sc + o
    n2 = F.layer_norm(r1, (Cout,), _w(tensors, p + "norm2.weight"), _w(tensors, p + "norm2.bias"), eps=1e-6)
    h = n2 @ _w(tensors, p + "mlp.fc1.weight").T + _w(tensors, p + "mlp.fc1.bias")
    h = gelu(h)
    y = r1 + (h @ _w(tensors, p + "mlp.fc2.weight").T + _w(tensors, p + "mlp.fc2.bias"))
    return y.reshape(Ht * Wt, Cout).numpy(), Ht, Wt


def test_small_hiera_metadata(small_hiera):
    _, om, _ = small_hiera
    infos = [om.block_info(i) for i in range(om.nblocks)]
    assert [i["window"] for i in infos] == [8, 8, 6, 6, 0, 4, 4, 4]
    assert [i["q_stride"] for i in infos] == [0, 1, 0, 1, 0, 0, 1, 0]
    assert [i["dim_out"] for i in infos] == [32, 64, 64, 128, 128, 128, 256, 256]
    assert om.side == [48, 24, 12, 6] and om.width == [32, 64, 128, 256]


def test_patch_embed_and_pos_embed_vs_torch(small_hiera):
    p, om, tensors = small_hiera
    rng = np.random.default_rng(5)
    chw = rng.standard_normal((3, 192, 192)).astype(np.float32)
    got = om.prefix(chw)
    w = _w(tensors, "hiera.patch_embed.weight")  # [E, 3, 7, 7]
    conv = F.conv2d(t64(chw)[None], w, _w(tensors, "hiera.patch_embed.bias"), stride=4, padding=3)[0]
    bkg = _w(tensors, "hiera.pos_embed")[0]  # [E, bkg_h, bkg_w]
    win = _w(tensors, "hiera.pos_embed_window")[0]  # [E, ws, ws]
    pe = F.interpolate(bkg[None], size=(48, 48), mode="bicubic", align_corners=False)[0] + win.repeat(1, 6, 6)
    ref = (conv + pe).permute(1, 2, 0).reshape(48 * 48, 32).numpy()
    assert orc.rel_l2(got, ref) < 1e-6


def test_blocks_vs_torch(small_hiera):
    p, om, tensors = small_hiera
    rng = np.random.default_rng(6)
    H = W = 48
    x = rng.standard_normal((H * W, 32)).astype(np.float32)
    for bi in range(om.nblocks):
        info = om.block_info(bi)
        got, Ho, Wo = om.block(bi, x, H, W)
        ref, Hr, Wr = _torch_block(x, H, W, tensors, bi, info)
        assert (Ho, Wo) == (Hr, Wr)
        # exact tanh-GELU: the fp16 table (relative rounding ≤ 2^-11 per hidden
        # unit) is the only intended difference
        rl = orc.rel_l2(got, ref)
        assert rl < 5e-4, (bi, info, rl)
        # with ggml's table in the restatement too, only f32-vs-f64 evaluation
        # (and the odd one-ulp table flip it causes) remains
        ref_t, _, _ = _torch_block(x, H, W, tensors, bi, info, gelu=_table_gelu)
        assert orc.rel_l2(got, ref_t) < 3e-5, (bi, info)
        x, H, W = got, Ho, Wo


def test_fpn_vs_torch(small_hiera):
    p, om, tensors = small_hiera
    rng = np.random.default_rng(7)
    stages = [rng.standard_normal((s * s, w)).astype(np.float32) for s, w in zip(om.side, om.width)]
    got = om.fpn(stages)
    lat = []
    for i in range(4):
        c = 3 - i
        w = _w(tensors, f"fpn.convs.{c}.weight")
        s = om.side[i]
        xi = t64(stages[i]).reshape(s, s, -1).permute(2, 0, 1)[None]
        lat.append(F.conv2d(xi, w, _w(tensors, f"fpn.convs.{c}.bias"))[0])
    # top-down levels {2, 3}: level 2 += nearest ×2 of level 3; levels 0, 1 lateral only
    lat[2] = lat[2] + F.interpolate(lat[3][None], scale_factor=2, mode="nearest")[0]
    for i in range(4):
        ref = lat[i].permute(1, 2, 0).reshape(-1, 64).numpy()
        assert orc.rel_l2(got[i], ref) < 1e-6, i


def test_encode_composes_the_stages(small_hiera):
    p, om, tensors = small_hiera
    rng = np.random.default_rng(8)
    img = rng.integers(0, 256, (200, 170, 3), dtype=np.uint8)
    chw = orc.preprocess_sam2(img, 192)
    outs, stages = om.encode(chw)
    assert len(outs) == 3 and [o.shape[0] for o in outs] == [48 * 48, 24 * 24, 12 * 12]
    x, H, W = om.prefix(chw), 48, 48
    st = []
    for bi in range(om.nblocks):
        x, H, W = om.block(bi, x, H, W)
        if om.block_info(bi)["stage_end"]:
            st.append(x)
    for a, b in zip(st, stages):
        assert np.array_equal(a, b)
    lv = om.fpn(st)
    for a, b in zip(outs, lv):
        assert np.array_equal(a, b)


def test_encode_at_another_image_size(small_hiera):
    """sam3_create_state's encode_img_size on a SAM 2 file (sam3.cpp:3392-3402,
    :245-257, :5862): the same model encoding 128 px images instead of its
    native 192 — a 32 × 32 patch grid, stage grids 32/16/8/4, the positional
    embedding bicubic-resized to 32 × 32 plus the window PE tiled, and every
    block on the smaller grid (windows now padded differently) — against the
    float64 torch restatement."""
    p, _, tensors = small_hiera
    om = orc.OracleHiera(p)
    om.set_img_size(128)
    assert om.side == [32, 16, 8, 4]
    rng = np.random.default_rng(9)
    chw = rng.standard_normal((3, 128, 128)).astype(np.float32)
    x = om.prefix(chw)
    w = _w(tensors, "hiera.patch_embed.weight")
    conv = F.conv2d(t64(chw)[None], w, _w(tensors, "hiera.patch_embed.bias"), stride=4, padding=3)[0]
    bkg = _w(tensors, "hiera.pos_embed")[0]
    win = _w(tensors, "hiera.pos_embed_window")[0]
    pe = F.interpolate(bkg[None], size=(32, 32), mode="bicubic", align_corners=False)[0] + win.repeat(1, 4, 4)
    assert orc.rel_l2(x, (conv + pe).permute(1, 2, 0).reshape(32 * 32, 32).numpy()) < 1e-6
    H = W = 32
    stages = []
    for bi in range(om.nblocks):
        info = om.block_info(bi)
        got, Ho, Wo = om.block(bi, x, H, W)
        ref, Hr, Wr = _torch_block(x, H, W, tensors, bi, info, gelu=_table_gelu)
        assert (Ho, Wo) == (Hr, Wr)
        assert orc.rel_l2(got, ref) < 3e-5, (bi, info)
        x, H, W = got, Ho, Wo
        if info["stage_end"]:
            stages.append(x)
    outs, st = om.encode(chw)
    assert [o.shape[0] for o in outs] == [32 * 32, 16 * 16, 8 * 8]
    for a, b in zip(stages, st):
        assert np.array_equal(a, b)
    with pytest.raises(AssertionError):
        om.set_img_size(100)  # not a multiple of 32
