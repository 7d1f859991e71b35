"""GPU parity of the SimpleFPN neck (sam3_build_neck_graph, sam3.cpp:3863-3921)
against the CPU oracle.

Stage parity: the engine's neck runs on the same vit_output the oracle
gets (s3e_run_neck), so only the neck's own arithmetic differs.  In
quantized files the neck's conv kernels are F32 (their ne0 of 1, 2 or 3 is
not a block multiple, sam3.cpp:2473-2494): the engine runs them as split
fp16 (x = hi + lo, three fp16 products) with fp32 accumulation, and the
deconvolutions in fp16 exactly as ggml's conv_transpose_2d does, so the
levels agree to fp32 accumulation-order noise plus the rare one-ulp fp16
rounding flips of intermediates that ggml itself rounds to fp16.  F16 files
round every conv input to fp16 (ggml's im2col in the kernel type) and are
held to the F16 specification.

End to end: the tracker levels after encoding an image are compared with
the oracle's backbone + neck on the same image, to the specification
(relative L2 ≤ 1e-3 and max-abs ≤ 5e-3 for quantized files, relative L2 ≤
2e-3 for F16), with the same allowance for ggml's own evaluation-order gap
as the backbone tests.
"""
import os

import numpy as np
import pytest

import oracle_lib as orc

pytestmark = pytest.mark.gpu


def _report(what, got, ref):
    rl, ma = orc.rel_l2(got, ref), orc.max_abs(got, ref)
    print(f"{what}: rel_l2={rl:.3e} max_abs={ma:.3e} |ref|max={np.abs(ref).max():.3f}", flush=True)
    return rl, ma


@pytest.fixture(scope="module", params=["q8_0", "f16"])
def neck_model(request, tmpdir_session, ctx):
    import s3e

    ft = request.param
    path = os.path.join(str(tmpdir_session), f"neck_{ft}.ggml")
    # 24×24 tokens of width 128, both necks (a full, not visual-only, file)
    s3e.synth_write(path, img_size=336, patch=14, embed_dim=128, depth=1, heads=2, mlp_ratio_x1000=4000,
                    window=8, global_idx=(), ftype=ft, seed=11, std=0.05, random_affine=True, neck=2,
                    neck_dim=128)
    om = orc.OracleModel(path)
    gm = s3e.Model(ctx, path)
    st = s3e.State(ctx, gm)
    yield ft, om, gm, st
    st.free()
    gm.free()


def test_neck_levels_match_oracle(neck_model, ctx):
    ft, om, gm, st = neck_model
    assert gm.necks == 3 and gm.neck_dim == 128
    G, E = 24, 128
    x = (np.random.default_rng(4).standard_normal((G * G, E)) * 2.0).astype(np.float32)
    print(f"neck stage {ft}: G={G} E={E}", flush=True)
    xd = ctx.to_device(x)
    st.run_neck(xd)
    ctx.sync()
    tol = 2e-3 if ft == "f16" else 1e-4
    for which in ("trk", "det"):
        ref = om.neck(x, which)
        for lvl in range(4):
            got = st.tensor(f"neck_{which}_{lvl}")
            assert got.shape == ref[lvl].shape, (which, lvl)
            rl, ma = _report(f"{ft} neck_{which}_{lvl}", got, ref[lvl])
            assert rl <= tol, (which, lvl)
            if ft != "f16":
                assert ma <= 5e-3, (which, lvl)


def test_neck_is_deterministic_and_repeatable(neck_model, ctx):
    ft, om, gm, st = neck_model
    x = np.random.default_rng(8).standard_normal((576, 128)).astype(np.float32)
    xd = ctx.to_device(x)
    st.run_neck(xd)
    a = [st.tensor(f"neck_trk_{i}") for i in range(4)]
    st.run_neck(xd)
    b = [st.tensor(f"neck_trk_{i}") for i in range(4)]
    for u, v in zip(a, b):
        assert np.array_equal(u, v)


def test_pe_tensors(neck_model, ctx):
    ft, om, gm, st = neck_model
    sides = [96, 48, 24, 12]
    for i, sd in enumerate(sides):
        ref = orc.sinusoidal_pe_2d(sd, sd, 128).reshape(sd * sd, 128)
        for name in (f"pe_{i}", f"neck_det_pe_{i}", f"neck_trk_pe_{i}"):
            got = st.tensor(name)
            assert got.shape == ref.shape
            assert np.max(np.abs(got - ref)) <= 1e-6, name


@pytest.fixture(scope="module", params=["q4_0", "f16"])
def full_model(request, tmpdir_session, ctx):
    import s3e

    ft = request.param
    path = os.path.join(str(tmpdir_session), f"enc_neck_{ft}.ggml")
    s3e.synth_write(path, img_size=336, patch=14, embed_dim=1024, depth=2, heads=16, window=8,
                    global_idx=(1,), ftype=ft, seed=5, std=0.02, random_affine=True, neck=1)
    om = orc.OracleModel(path)
    gm = s3e.Model(ctx, path)
    st = s3e.State(ctx, gm)
    yield ft, om, gm, st
    st.free()
    gm.free()


def test_encode_image_neck_levels(full_model, ctx):
    import ctypes

    ft, om, gm, st = full_model
    assert gm.necks == 1
    rng = np.random.default_rng(3)
    img = rng.integers(0, 256, (336, 336, 3), dtype=np.uint8)
    chw = orc.preprocess_sam3(img, 336)
    print(f"encode + neck {ft}", flush=True)
    st.encode_image_u8(img)
    orc.LIB.orc_set_variant.argtypes = [ctypes.c_int]
    refs, gaps = [], []
    for variant in (0, 1):  # ggml's AVX2 and generic evaluation orders
        orc.LIB.orc_set_variant(variant)
        try:
            refs.append(om.neck(om.encode(chw), "trk"))
        finally:
            orc.LIB.orc_set_variant(0)
    with pytest.raises(Exception):
        st.tensor("neck_det_0")  # visual-only file: no detector neck
    for lvl in range(4):
        ref = refs[0][lvl]
        grl, gma = orc.rel_l2(refs[1][lvl], ref), orc.max_abs(refs[1][lvl], ref)
        got = st.tensor(f"neck_trk_{lvl}")
        rl, ma = _report(f"{ft} neck_trk_{lvl} (order gap {grl:.2e}/{gma:.2e})", got, ref)
        if ft == "f16":
            assert rl <= 2e-3
        else:
            assert rl <= max(1e-3, 2.0 * grl)
            assert ma <= max(5e-3, 2.0 * gma)
