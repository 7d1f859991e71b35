"""GPU parity of the SAM 3 ViT encoder at its real size: 1008×1008 input,
72×72 tokens, 32 blocks of width 1024 with 16 heads and MLP 4736, 24×24
windows (9 windows of 576 tokens) and global blocks 7/15/23/31 over 5184
tokens with the 72×72 / scale-1/3 RoPE table, and the tracker neck's four
levels at 288², 144², 72² and 36² — the backend acceptance comparison of
the reference (tests/test_metal_vit.cpp:33-162: vit_output and the neck
levels of a backend against the CPU path).

Random-init weights N(0, 0.02) with random biases and LayerNorm affine,
seed 0; a uniform random uint8 image, seed 0.

* F16 end to end (vit_output and neck_trk_0..3): relative L2 ≤ 2e-3.
* Q4_0 / Q8_0 block 0 (windowed) and block 7 (global), each fed the
  oracle's own input: relative L2 ≤ 1e-3.  The max-abs distance is reported
  next to ggml's own AVX2-vs-generic distance on the same block: ggml's two
  evaluation orders are already 9e-3 apart in max-abs after one block at
  this size, above the nominal 5e-3.
* Q4_0 end to end: reported against that distance on the whole encoder
  (tests/golden/c4_order_gap.json, written by tests/golden/make_c4_gap.py:
  ggml's generic order takes minutes on the whole encoder).
"""
import ctypes
import json
import os

import numpy as np
import pytest

import oracle_lib as orc

pytestmark = pytest.mark.gpu

orc.LIB.orc_set_variant.argtypes = [ctypes.c_int]
GOLD = os.path.join(os.path.dirname(__file__), "golden", "c4_order_gap.json")
IMG = 1008


def c4_model(path, ft):
    import s3e

    s3e.synth_write(path, img_size=IMG, ftype=ft, seed=0, random_affine=True)


def c4_image():
    return np.random.default_rng(0).integers(0, 256, (IMG, IMG, 3), dtype=np.uint8)


@pytest.fixture(scope="module", params=["f16", "q4_0", "q8_0"])
def c4(request, tmpdir_session, ctx):
    import s3e

    ft = request.param
    path = os.path.join(str(tmpdir_session), f"c4_{ft}.ggml")
    print(f"C4 {ft}: writing the model", flush=True)
    c4_model(path, ft)
    om = orc.OracleModel(path)
    gm = s3e.Model(ctx, path)
    st = s3e.State(ctx, gm)
    img = c4_image()
    chw = orc.preprocess_sam3(img, IMG)
    x0 = om.prefix(chw)
    yield ft, om, gm, st, img, chw, x0
    st.free()
    gm.free()
    os.remove(path)


def _report(tag, got, ref, gap=None):
    rl, ma = orc.rel_l2(got, ref), orc.max_abs(got, ref)
    g = "" if gap is None else f" | ggml order gap rel_l2={gap[0]:.3e} max_abs={gap[1]:.3e}"
    print(f"{tag}: rel_l2={rl:.3e} max_abs={ma:.3e} |ref|max={np.abs(ref).max():.3f}{g}", flush=True)
    return rl, ma


def test_c4_prefix(c4, ctx):
    ft, om, gm, st, img, chw, x0 = c4
    chw_d = ctx.to_device(chw)
    xd = ctx.buffer(x0.nbytes)
    st.prefix(chw_d, xd)
    ctx.sync()
    rl, _ = _report(f"C4 {ft} prefix", xd.download(np.float32, x0.shape), x0)
    assert rl <= 1e-5


@pytest.mark.parametrize("bi", [0, 7])
def test_c4_block(c4, ctx, bi):
    ft, om, gm, st, img, chw, x0 = c4
    print(f"C4 {ft} block {bi}: oracle", flush=True)
    ref = om.block(bi, x0)
    gap = None
    if ft != "f16":
        orc.LIB.orc_set_variant(1)
        try:
            alt = om.block(bi, x0)
        finally:
            orc.LIB.orc_set_variant(0)
        gap = (orc.rel_l2(alt, ref), orc.max_abs(alt, ref))
    xd = ctx.to_device(x0)
    st.block(bi, xd)
    ctx.sync()
    rl, ma = _report(f"C4 {ft} block {bi}", xd.download(np.float32, x0.shape), ref, gap)
    assert rl <= (2e-3 if ft == "f16" else 1e-3)


def test_c4_neck_on_oracle_input(c4, ctx):
    """The tracker neck at its real size on a given backbone output (72² tokens
    of 1024), against the oracle's neck on the same input: levels of 288²,
    144², 72² and 36².  Quantized files hold the neck in F32, computed on split
    fp16 pairs (the 288² level's 3×3 in 256-pixel tiles, the others in 128);
    F16 files in fp16."""
    ft, om, gm, st, img, chw, x0 = c4
    G, E = IMG // 14, 1024
    x = np.random.default_rng(5).standard_normal((G * G, E)).astype(np.float32)
    print(f"C4 {ft} neck on the oracle's input", flush=True)
    xd = ctx.to_device(x)
    st.run_neck(xd)
    ctx.sync()
    ref = om.neck(x, "trk")
    tol = 2e-3 if ft == "f16" else 1e-4
    for lvl in range(4):
        got = st.tensor(f"neck_trk_{lvl}")
        assert got.shape == ref[lvl].shape, lvl
        rl, ma = _report(f"C4 {ft} neck_trk_{lvl} (oracle input)", got, ref[lvl])
        assert rl <= tol, lvl
        if ft != "f16":
            assert ma <= 5e-3, lvl
    xd.free()


def test_c4_encode(c4, ctx):
    """F16: the specification end to end.  Quantized: Q4_0 only (the oracle's
    whole encoder takes about a minute per weight type on the host), against
    the committed order gap of the same model and image."""
    ft, om, gm, st, img, chw, x0 = c4
    if ft == "q8_0":
        pytest.skip("end to end runs for F16 and Q4_0; Q8_0 is covered block by block")
    print(f"C4 {ft} encode: oracle", flush=True)
    ref = om.encode(chw)
    st.encode_image_u8(img)
    got = st.tensor("vit_output")
    gap = None
    if ft == "q4_0":
        g = json.load(open(GOLD))["q4_0"]
        gap = (g["vit_output"]["rel_l2"], g["vit_output"]["max_abs"])
    rl, ma = _report(f"C4 {ft} vit_output", got, ref, gap)
    if ft == "f16":
        assert rl <= 2e-3
    else:
        assert rl <= max(1e-3, 1.5 * gap[0])
    levels = om.neck(ref, "trk")
    for i, lv in enumerate(levels):
        g = st.tensor(f"neck_trk_{i}")
        assert g.shape == lv.shape
        lgap = None
        if ft == "q4_0":
            e = json.load(open(GOLD))["q4_0"][f"neck_trk_{i}"]
            lgap = (e["rel_l2"], e["max_abs"])
        rl, ma = _report(f"C4 {ft} neck_trk_{i}", g, lv, lgap)
        if ft == "f16":
            assert rl <= 2e-3
        else:
            assert rl <= max(1e-3, 1.5 * lgap[0])
