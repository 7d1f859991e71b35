"""GPU parity of the SAM 3 ViT backbone against the CPU oracle.

A small random-init model in sam3.cpp's file format (img 336 → 24×24 tokens,
width 1024, 16 heads, MLP 4736, window 8 → 9 windows, block 1 global,
random biases and LayerNorm affine) is run stage by stage on identical
inputs (prefix, each block) and end to end, for every weight type.

Tolerances.  The prefix (patch GEMM + tiled pos-embed + ln_pre) must match
to fp32 order noise (relative L2 ≤ 1e-5).  F16 models must meet the F16
specification end to end: relative L2 ≤ 2e-3.  Quantized models re-quantize
every GEMM input to Q8 per 32-block; a difference in the last fp32 bit ahead
of such a rounding flips it, and each flip perturbs the next quantizer's
inputs, so any two implementations whose fp32 evaluation order differs end
up apart by about the quantization noise.  The reference is no exception:
ggml's own AVX2 and generic-C dot-product orders (both restated in the
oracle, orc_set_variant) disagree by more than the nominal 1e-3 / 5e-3 after
a single block.  Quantized blocks therefore must meet relative L2 ≤ 1e-3,
and quantized outputs must stay within 2× the distance between those two
ggml evaluation orders, measured here on the same model and image.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle_lib as orc

pytestmark = pytest.mark.gpu

FTYPES = ["q4_0", "q8_0", "q4_1", "f16"]
orc.LIB.orc_set_variant.argtypes = [ctypes.c_int]
# Measured: the engine's quantized outputs sit at 0.9-1.9x ggml's own
# AVX2-vs-generic distance (1.0x for the 32-block encoder at 1008 px, where
# both saturate at the quantization noise).  The two ggml orders share
# ggml's f32 attention; the engine's split-fp16 attention is one more
# independent source of last-bit differences (it flips 1e-5-3e-5 of the proj
# input's Q8 codes per block), so small models sit above 1x.
FLOOR_FACTOR = 2.0


def _variant_gap(fn):
    """Distance between ggml's AVX2 and generic evaluation orders for fn()."""
    orc.LIB.orc_set_variant(0)
    a = fn()
    orc.LIB.orc_set_variant(1)
    try:
        b = fn()
    finally:
        orc.LIB.orc_set_variant(0)
    return a, orc.rel_l2(b, a), orc.max_abs(b, a)


@pytest.fixture(scope="module", params=FTYPES)
def small(request, tmpdir_session, ctx):
    import s3e

    ft = request.param
    path = os.path.join(str(tmpdir_session), f"vit_small_{ft}.ggml")
    s3e.synth_write(path, img_size=336, patch=14, embed_dim=1024, depth=2, heads=16, window=8,
                    global_idx=(1,), ftype=ft, seed=5, std=0.02, random_affine=True)
    om = orc.OracleModel(path)
    gm = s3e.Model(ctx, path)
    st = s3e.State(ctx, gm)
    rng = np.random.default_rng(3)
    img = rng.integers(0, 256, (336, 336, 3), dtype=np.uint8)
    chw = orc.preprocess_sam3(img, 336)
    yield ft, om, gm, st, img, chw
    st.free()
    gm.free()


def _report(ft, what, got, ref, floor=None):
    rl, ma = orc.rel_l2(got, ref), orc.max_abs(got, ref)
    fl = "" if floor is None else f" | ggml order gap rel_l2={floor[0]:.3e} max_abs={floor[1]:.3e}"
    print(f"{ft} {what}: rel_l2={rl:.3e} max_abs={ma:.3e} |ref|max={np.abs(ref).max():.3f}{fl}")
    return rl, ma


def test_prefix(small, ctx):
    ft, om, gm, st, img, chw = small
    ref = om.prefix(chw)
    chw_d = ctx.to_device(chw)
    xd = ctx.buffer(ref.nbytes)
    st.prefix(chw_d, xd)
    ctx.sync()
    rl, _ = _report(ft, "prefix", xd.download(np.float32, ref.shape), ref)
    assert rl <= 1e-5


@pytest.mark.parametrize("bi", [0, 1])
def test_block(small, ctx, bi):
    ft, om, gm, st, img, chw = small
    x0 = om.prefix(chw)
    if bi == 1:
        x0 = om.block(0, x0)
    ref, frl, fma = _variant_gap(lambda: om.block(bi, x0))
    xd = ctx.to_device(x0)
    st.block(bi, xd)
    ctx.sync()
    rl, ma = _report(ft, f"block{bi}", xd.download(np.float32, ref.shape), ref, (frl, fma))
    if ft == "f16":
        assert rl <= 2e-3
    else:
        assert rl <= 1e-3
        assert ma <= max(5e-3, FLOOR_FACTOR * fma)


def test_encode_image(small, ctx):
    ft, om, gm, st, img, chw = small
    ref, frl, fma = _variant_gap(lambda: om.encode(chw))
    st.encode_image_u8(img)
    rl, ma = _report(ft, "vit_output", st.tensor("vit_output"), ref, (frl, fma))
    if ft == "f16":
        assert rl <= 2e-3
    else:
        assert rl <= max(1e-3, FLOOR_FACTOR * frl)
        assert ma <= max(5e-3, FLOOR_FACTOR * fma)


def test_banded_encode_equals_block_chain(small, ctx):
    """The encoder runs each run of windowed blocks as bands of window rows
    on three streams (24×24 tokens, window 8: three bands of 192 rows).
    Every element is computed as in the one-stream chain of s3e_vit_prefix +
    s3e_vit_block, so vit_output must equal that chain bit for bit, for each
    activation format (fp6 split, Q8_0, Q8_1, fp16).

    First the blocks run one at a time on another input, so that the state's
    Q/K/Vᵀ planes hold other values in both layouts: a band that overwrote
    planes another band still reads (a windowed block's windows and a global
    block's rows alias in one buffer) showed up here as a different result."""
    ft, om, gm, st, img, chw = small
    other = ctx.to_device(np.random.default_rng(11).standard_normal((576, 1024)).astype(np.float32))
    for i in range(om.depth):
        st.block(i, other)
    ctx.sync()
    other.free()
    chw_d = ctx.to_device(chw)
    st.encode_chw(chw_d)
    banded = st.tensor("vit_output")
    xd = ctx.buffer(banded.nbytes)
    st.prefix(chw_d, xd)
    for i in range(om.depth):
        st.block(i, xd)
    ctx.sync()
    chain = xd.download(np.float32, banded.shape)
    ndiff = int(np.count_nonzero(banded != chain))
    print(f"{ft} banded vs chain: {ndiff} differing elements")
    assert ndiff == 0
    for b in (chw_d, xd):
        b.free()


@pytest.mark.parametrize("ft", ["q4_0", "q8_0", "f16"])
def test_two_bands_and_both_global_plane_sets(tmpdir_session, ctx, ft):
    """A grid of two window rows (48×48 tokens, window 24) runs in two bands,
    and two global blocks (1 and 3) use the two global Q/K/Vᵀ plane sets in
    turn: the banded encode equals the one-stream chain bit for bit, with the
    planes first filled from another input as in the three-band test."""
    import s3e

    path = os.path.join(str(tmpdir_session), f"vit_two_bands_{ft}.ggml")
    s3e.synth_write(path, img_size=672, patch=14, embed_dim=512, depth=5, heads=8, window=24, mlp_ratio_x1000=4500,
                    global_idx=(1, 3), ftype=ft, seed=9, std=0.02, random_affine=True, neck=0)
    gm = s3e.Model(ctx, path)
    st = s3e.State(ctx, gm)
    try:
        rng = np.random.default_rng(12)
        other = ctx.to_device(rng.standard_normal((2304, 512)).astype(np.float32))
        for i in range(5):
            st.block(i, other)
        ctx.sync()
        other.free()
        chw = orc.preprocess_sam3(rng.integers(0, 256, (672, 672, 3), dtype=np.uint8), 672)
        chw_d = ctx.to_device(chw)
        st.encode_chw(chw_d)
        banded = st.tensor("vit_output")
        xd = ctx.buffer(banded.nbytes)
        st.prefix(chw_d, xd)
        for i in range(5):
            st.block(i, xd)
        ctx.sync()
        chain = xd.download(np.float32, banded.shape)
        ndiff = int(np.count_nonzero(banded != chain))
        print(f"{ft} two bands vs chain: {ndiff} differing elements, |x|max={np.abs(chain).max():.3f}", flush=True)
        assert np.all(np.isfinite(chain))
        assert ndiff == 0
        for b in (chw_d, xd):
            b.free()
    finally:
        st.free()
        gm.free()
