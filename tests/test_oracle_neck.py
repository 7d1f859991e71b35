"""Pins the oracle's SimpleFPN neck (oracle/orc_neck.c) before it is trusted.

Each function is compared with torch.nn.functional evaluated in float64 on
the same operands, rounded where ggml rounds them (fp16 input and kernel of
the deconvolutions; fp16 im2col for F16 kernels).  torch's conv_transpose2d,
conv2d and max_pool2d are library routines that fix the index conventions
independently: a transposed kernel, a swapped (ky, kx), a wrong padding side
or a mis-ordered K would fail them.  The composite neck is checked against a
torch restatement of sam3_build_neck_graph (sam3.cpp:3863-3921) built from
the weights read back from the model file, and the PEs against the closed
form of sam3_sinusoidal_pe_2d (sam3.cpp:3597-3633) in float64.  No GPU.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle_lib as orc


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16)


def nchw(x_hwc):
    return torch.from_numpy(np.ascontiguousarray(np.asarray(x_hwc, np.float64).transpose(2, 0, 1)))[None]


def hwc(t):
    return t[0].permute(1, 2, 0).numpy()


@pytest.mark.parametrize("Cin,Cout,H,W", [(64, 32, 5, 7), (96, 40, 3, 2)])
def test_conv_transpose_2x2_vs_torch(Cin, Cout, H, W):
    rng = np.random.default_rng(Cin + W)
    w = f16(rng.standard_normal((Cin, Cout, 2, 2)) * 0.1)  # ggml ne [kW, kH, Cout, Cin]
    x = rng.standard_normal((H, W, Cin)).astype(np.float32)
    got = orc.conv_transpose_2x2(w.view(np.uint16), x)
    # torch weight [Cin, Cout, kH, kW] is ggml's [kW, kH, Cout, Cin] in row-major order
    ref = F.conv_transpose2d(nchw(f16(x).astype(np.float32)), torch.from_numpy(w.astype(np.float64)), stride=2)
    ref = hwc(ref)
    assert got.shape == ref.shape
    assert orc.rel_l2(got, ref) < 1e-6


@pytest.mark.parametrize("k,pad", [(1, 0), (3, 1)])
@pytest.mark.parametrize("ktype", [orc.F32, orc.F16])
def test_conv2d_vs_torch(k, pad, ktype):
    rng = np.random.default_rng(10 * k + ktype)
    Cin, Cout, H, W = 48, 24, 6, 9
    w = (rng.standard_normal((Cout, Cin, k, k)) * 0.1).astype(np.float32)  # ggml ne [kW, kH, Cin, Cout]
    x = rng.standard_normal((H, W, Cin)).astype(np.float32)
    if ktype == orc.F16:
        wk = f16(w)
        got = orc.conv2d(ktype, wk.view(np.uint16), x, pad)
        wt, xt = wk.astype(np.float64), f16(x).astype(np.float64)
    else:
        got = orc.conv2d(ktype, w, x, pad)
        wt, xt = w.astype(np.float64), x.astype(np.float64)
    ref = hwc(F.conv2d(nchw(xt), torch.from_numpy(wt), padding=pad))
    assert got.shape == ref.shape == (H, W, Cout)
    assert orc.rel_l2(got, ref) < 1e-6


def test_conv2d_padding_sees_zeros():
    """A 3×3 all-ones kernel over an all-ones image counts the in-image taps:
    4 at corners, 6 on edges, 9 inside."""
    x = np.ones((5, 4, 1), np.float32)
    got = orc.conv2d(orc.F32, np.ones((1, 1, 3, 3), np.float32), x, 1)[..., 0]
    rows = np.array([2, 3, 3, 3, 2])[:, None]
    cols = np.array([2, 3, 3, 2])[None, :]
    assert np.array_equal(got, (rows * cols).astype(np.float32))


def test_maxpool_vs_torch():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 6, 5)).astype(np.float32)
    ref = hwc(F.max_pool2d(nchw(x), 2, 2))
    assert np.array_equal(orc.maxpool2x2(x), ref.astype(np.float32))
    x7 = rng.standard_normal((7, 7, 3)).astype(np.float32)  # odd sides drop the last row/column
    assert orc.maxpool2x2(x7).shape == (3, 3, 3)


@pytest.mark.parametrize("side", [36, 9])
def test_sinusoidal_pe_closed_form(side):
    d = 256
    got = orc.sinusoidal_pe_2d(side, side, d)
    half = d // 2
    pos = (np.arange(side, dtype=np.float64) + 1) / side * 2 * math.pi
    i = np.arange(half)
    dim_t = 10000.0 ** ((i & ~1) / half)
    ang = pos[:, None] / dim_t[None, :]  # [side, half]
    enc = np.where(i % 2 == 0, np.sin(ang), np.cos(ang))
    ref = np.empty((side, side, d))
    ref[:, :, :half] = enc[:, None, :]   # channels [0, half) follow y
    ref[:, :, half:] = enc[None, :, :]   # channels [half, d) follow x
    assert np.max(np.abs(got - ref)) < 4e-6


def _torch_neck(tensors, prefix, x, G, E):
    """sam3_build_neck_graph restated with torch float64 ops, rounding to fp16
    where ggml's conv_transpose_2d does (input and kernel)."""

    def t(name):
        dt, ne, arr = tensors[prefix + name]
        return torch.from_numpy(np.asarray(arr, np.float64))

    def deconv(inp, wname, bname):
        w = torch.from_numpy(t(wname).numpy().astype(np.float16).astype(np.float64))  # ggml_cast to F16
        xi = torch.from_numpy(inp.numpy().astype(np.float32).astype(np.float16).astype(np.float64))
        return F.conv_transpose2d(xi, w, stride=2) + t(bname)[None, :, None, None]

    def conv(inp, wname, bname):
        w = t(wname)
        if tensors[prefix + wname][0] == orc.F16:  # im2col in fp16
            inp = torch.from_numpy(inp.numpy().astype(np.float32).astype(np.float16).astype(np.float64))
        return F.conv2d(inp, w, padding=w.shape[-1] // 2) + t(bname)[None, :, None, None]

    xin = torch.from_numpy(x.astype(np.float64).reshape(G, G, E).transpose(2, 0, 1).copy())[None]
    s0 = deconv(xin, "0.dconv_2x2_0.weight", "0.dconv_2x2_0.bias")
    s0 = 0.5 * s0 * (1.0 + torch.erf(s0 / math.sqrt(2.0)))
    s0 = deconv(s0, "0.dconv_2x2_1.weight", "0.dconv_2x2_1.bias")
    s0 = conv(s0, "0.conv_1x1.weight", "0.conv_1x1.bias")
    s0 = conv(s0, "0.conv_3x3.weight", "0.conv_3x3.bias")
    s1 = deconv(xin, "1.dconv_2x2.weight", "1.dconv_2x2.bias")
    s1 = conv(s1, "1.conv_1x1.weight", "1.conv_1x1.bias")
    s1 = conv(s1, "1.conv_3x3.weight", "1.conv_3x3.bias")
    s2 = conv(xin, "2.conv_1x1.weight", "2.conv_1x1.bias")
    s2 = conv(s2, "2.conv_3x3.weight", "2.conv_3x3.bias")
    s3 = F.max_pool2d(xin, 2, 2)
    s3 = conv(s3, "3.conv_1x1.weight", "3.conv_1x1.bias")
    s3 = conv(s3, "3.conv_3x3.weight", "3.conv_3x3.bias")
    return [hwc(s).reshape(-1, s.shape[1]) for s in (s0, s1, s2, s3)]


@pytest.fixture(scope="module")
def s3e_mod():
    import s3e

    return s3e


@pytest.mark.parametrize("ft", ["q8_0", "f16"])
def test_neck_vs_torch(s3e_mod, tmp_path, ft):
    p = str(tmp_path / f"neck_{ft}.ggml")
    s3e_mod.synth_write(p, img_size=168, embed_dim=128, heads=2, depth=1, window=4, global_idx=(),
                        ftype=ft, seed=7, std=0.05, random_affine=True, neck=2, neck_dim=64)
    om = orc.OracleModel(p)
    G, E = 12, 128
    x = np.random.default_rng(2).standard_normal((G * G, E)).astype(np.float32)
    tensors = orc.read_model_file(p)
    assert tensors["neck.trk.0.conv_3x3.weight"][0] == (orc.F16 if ft == "f16" else orc.F32)
    for which in ("trk", "det"):
        side, D = om.neck_dims(which)
        assert side == [48, 24, 12, 6] and D == 64
        got = om.neck(x, which)
        ref = _torch_neck(tensors, f"neck.{which}.", x, G, E)
        for lvl in range(4):
            assert got[lvl].shape == ref[lvl].shape
            # fp16 roundings of intermediates can land one ulp apart between
            # f32 and f64 evaluation: a few elements differ by ~1e-3 relative
            assert orc.rel_l2(got[lvl], ref[lvl]) < 1e-4, (which, lvl)
    # the two necks have different weights
    assert not np.allclose(om.neck(x, "trk")[2], om.neck(x, "det")[2])
