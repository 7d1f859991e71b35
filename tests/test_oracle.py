"""Pins the CPU oracle (oracle/) before the GPU results are compared against it.

Each oracle function is checked against something it does not compute itself:
hand-derived golden vectors (tests/golden/quant_golden.json), numpy's IEEE
float16, closed forms evaluated in float64, exact integer brute force, the
reference's own known-answer formulas (RoPE tables, tests/test_phase3.cpp:
118-178), and invariants that a dropped term, wrong sign or wrong index would
break.  No GPU needed.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle_lib as orc

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "quant_golden.json")))
L = orc.LIB


# ---- fp16 ---------------------------------------------------------------------
def test_fp16_decode_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    soft = np.array([L.orc_fp16_to_fp32_soft(int(v)) for v in h], dtype=np.float32)
    hw = np.empty(65536, np.float32)
    L.orc_fp16_to_fp32_row(orc.ptr(h), orc.ptr(hw), 65536)
    fin = np.isfinite(ref)
    assert np.array_equal(soft[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.array_equal(hw[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(soft[np.isnan(ref)])) and np.all(np.isinf(soft[np.isinf(ref)]))


def test_fp16_encode_matches_ieee_rne():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(400_000) * np.exp2(rng.integers(-30, 17, 400_000))).astype(np.float32)
    # every midpoint between adjacent binary16 values in [2^-14, 2^15]: exact ties
    hs = np.arange(0x0400, 0x7BFF, dtype=np.uint16)
    a = hs.view(np.float16).astype(np.float64)
    b = (hs + 1).view(np.float16).astype(np.float64)
    mids = ((a + b) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids])
    out = np.empty(x.size, np.uint16)
    L.orc_fp32_to_fp16_row(orc.ptr(x), orc.ptr(out), x.size)
    assert np.array_equal(out, x.astype(np.float16).view(np.uint16))


def test_fp16_golden():
    for c in GOLD["fp16"]:
        assert L.orc_fp32_to_fp16(c["x"]) == c["bits"], c


# ---- weight quantizers (ggml_quantize_chunk reference) --------------------------
def _blocks(t, data, n):
    return np.frombuffer(data.tobytes(), np.uint8).reshape(n, orc.BLOCK_BYTES[t])


def test_q4_0_golden():
    g = GOLD["q4_0"]
    out = orc.quantize_ref(orc.Q4_0, np.array([g["x"]], np.float32))
    b = _blocks(orc.Q4_0, out, 1)[0]
    assert np.frombuffer(b[:2].tobytes(), np.float16)[0] == g["d"]
    q = np.concatenate([b[2:] & 15, b[2:] >> 4])
    assert q.tolist() == g["q"]


def test_q4_1_golden_ends():
    g = GOLD["q4_1_ends"]
    out = orc.quantize_ref(orc.Q4_1, np.array([g["x"]], np.float32))
    b = _blocks(orc.Q4_1, out, 1)[0]
    q = np.concatenate([b[4:] & 15, b[4:] >> 4])
    assert q[0] == g["q_first"] and q[-1] == g["q_last"]
    assert np.frombuffer(b[2:4].tobytes(), np.float16)[0] == np.float16(g["m"])
    assert np.frombuffer(b[0:2].tobytes(), np.float16)[0] == np.float16(g["d"])


def test_q8_tie_rounding():
    """Weights use roundf (half away), activations the x86 RNE path; the
    fixture's k+0.5 values tell them apart."""
    g = GOLD["q8_ties"]
    x = np.array([g["x"]], np.float32)
    w = _blocks(orc.Q8_0, orc.quantize_ref(orc.Q8_0, x), 1)[0]
    a = _blocks(orc.Q8_0, orc.from_float(orc.Q8_0, x), 1)[0]
    assert w[2:].view(np.int8).tolist() == g["q_weights_round_half_away"]
    assert a[2:].view(np.int8).tolist() == g["q_activations_round_half_even"]
    a1 = orc.split_q8(orc.Q8_1, orc.from_float(orc.Q8_1, x), 1, 32)
    assert a1[0][0].tolist() == g["q_activations_round_half_even"]
    s = np.frombuffer(a1[2].tobytes(), np.float16)[0]
    assert s == np.float16(sum(g["q_activations_round_half_even"]))  # d = 1


@pytest.mark.parametrize("t", [orc.Q4_0, orc.Q4_1, orc.Q8_0])
def test_quantizer_reconstruction_bounds(t):
    rng = np.random.default_rng(t)
    x = (rng.standard_normal((64, 256)) * rng.uniform(1e-3, 10, (64, 1))).astype(np.float32)
    q = orc.quantize_ref(t, x)
    y = orc.dequantize(t, q, 64, 256).astype(np.float64)
    xb = x.reshape(64, 8, 32).astype(np.float64)
    yb = y.reshape(64, 8, 32)
    amax = np.abs(xb).max(axis=2, keepdims=True)
    # fp16 storage of d (and m) moves every reconstructed value by at most
    # |q|·|d − fp16(d)| ≤ amax·2^-11 (plus |m|·2^-11 for Q4_1)
    if t == orc.Q8_0:
        bound = amax / 127 * 0.5 + amax * 2 ** -11  # half a step
    elif t == orc.Q4_0:
        bound = amax / 8 + amax * 2 ** -11  # the clamp at code 15 costs up to one step
    else:
        rngb = xb.max(axis=2, keepdims=True) - xb.min(axis=2, keepdims=True)
        bound = rngb / 15 * 0.5 + (rngb + 2 * amax) * 2 ** -11
    assert np.all(np.abs(yb - xb) <= bound + 1e-12)


# ---- dot products ------------------------------------------------------------
def _unpack(t, wb, N, K):
    blocks = np.frombuffer(wb.tobytes(), np.uint8).reshape(N, K // 32, orc.BLOCK_BYTES[t])
    d = blocks[:, :, 0:2].copy().view(np.float16).reshape(N, K // 32).astype(np.float64)
    if t == orc.Q8_0:
        return blocks[:, :, 2:].copy().view(np.int8).astype(np.int64), d, None
    off = 2 if t == orc.Q4_0 else 4
    nib = blocks[:, :, off:].astype(np.int64)
    q = np.concatenate([nib & 15, nib >> 4], axis=2)
    if t == orc.Q4_0:
        return q - 8, d, None
    m = blocks[:, :, 2:4].copy().view(np.float16).reshape(N, K // 32).astype(np.float64)
    return q, d, m


@pytest.mark.parametrize("t", [orc.Q4_0, orc.Q4_1, orc.Q8_0])
def test_block_sums_and_dot(t):
    rng = np.random.default_rng(7 + t)
    N, M, K = 6, 5, 320
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    wb = orc.to_weight_bytes(t, W)
    vdt = orc.VEC_DOT[t]
    xq = orc.from_float(vdt, X)
    qw, dw, mw = _unpack(t, wb, N, K)
    qx, dx, sx = orc.split_q8(vdt, xq, M, K)
    qx = qx.reshape(M, K // 32, 32).astype(np.int64)
    dx = dx.view(np.float16).astype(np.float64)
    rs, xs = orc.row_size(t, K), orc.row_size(vdt, K)
    sums = np.empty(K // 32, np.int32)
    for n in range(N):
        for m in range(M):
            L.orc_block_isums(t, K, orc.ptr(wb) + n * rs, orc.ptr(xq) + m * xs, orc.ptr(sums))
            exact = (qw[n] * qx[m]).sum(axis=1)
            assert np.array_equal(sums, exact)
            want = (dw[n] * dx[m] * exact).sum()
            if t == orc.Q4_1:
                want += (mw[n] * sx[m].view(np.float16).astype(np.float64)).sum()
            got = L.orc_vec_dot(t, K, orc.ptr(wb) + n * rs, orc.ptr(xq) + m * xs)
            assert abs(got - want) <= 1e-6 * max(1.0, abs(want)), (n, m, got, want)


@pytest.mark.parametrize("t", [orc.Q4_0, orc.Q4_1, orc.Q8_0, orc.F16, orc.F32])
def test_mul_mat_vs_f64(t):
    rng = np.random.default_rng(3 + t)
    M, N, K = 37, 70, 256
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    wb = orc.to_weight_bytes(t, W)
    Y = orc.mul_mat(t, wb, N, K, X)
    vdt = orc.VEC_DOT[t]
    Wd = orc.dequantize(t, wb, N, K).astype(np.float64) if t != orc.F32 else W.astype(np.float64)
    if t == orc.F32:
        Xd = X.astype(np.float64)
    elif t == orc.F16:
        Xd = X.astype(np.float16).astype(np.float64)
    else:
        Xd = orc.dequantize(vdt, orc.from_float(vdt, X), M, K).astype(np.float64)
    ref = Xd @ Wd.T
    if t == orc.Q4_1:  # ggml uses s = fp16(d·Σq) in place of the exact block sum
        qx, dx, sx = orc.split_q8(vdt, orc.from_float(vdt, X), M, K)
        _, _, mw = _unpack(t, wb, N, K)
        exact_s = dx.view(np.float16).astype(np.float64) * qx.reshape(M, K // 32, 32).sum(axis=2)
        ref += (sx.view(np.float16).astype(np.float64) - exact_s) @ mw.T
    assert orc.rel_l2(Y, ref) <= 2e-7


@pytest.mark.parametrize("t", [orc.Q4_0, orc.Q4_1, orc.Q8_0])
def test_blocked_mul_mat_is_bit_identical_to_vec_dot(t):
    rng = np.random.default_rng(11)
    M, N, K = 38, 71, 128
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    wb = orc.to_weight_bytes(t, W)
    Y = orc.mul_mat(t, wb, N, K, X)
    xq = orc.from_float(orc.VEC_DOT[t], X)
    rs, xs = orc.row_size(t, K), orc.row_size(orc.VEC_DOT[t], K)
    ref = np.array([[L.orc_vec_dot(t, K, orc.ptr(wb) + n * rs, orc.ptr(xq) + m * xs) for n in range(N)]
                    for m in range(M)], np.float32)
    assert np.array_equal(Y.view(np.uint32), ref.view(np.uint32))


# ---- norm, gelu, rope, attention ------------------------------------------------
def test_layer_norm_vs_f64():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((50, 1024)) * 3 + 2).astype(np.float32)
    w = rng.normal(1, 0.1, 1024).astype(np.float32)
    b = rng.normal(0, 0.1, 1024).astype(np.float32)
    y = orc.layer_norm(x, 1e-5, w, b)
    xd = x.astype(np.float64)
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * w + b
    assert orc.rel_l2(y, ref) <= 1e-6
    y0 = orc.layer_norm(x, 1e-5).astype(np.float64)
    assert np.abs(y0.mean(1)).max() < 1e-5 and np.abs(y0.var(1) - 1).max() < 1e-4


def test_gelu_erf_vs_f64():
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    y = x.copy()
    L.orc_gelu_erf(orc.ptr(y), y.size)
    ref = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)])
    assert np.max(np.abs(y - ref)) <= 2e-6 * np.maximum(1, np.abs(ref)).max()


@pytest.mark.parametrize("end,scale", [(24, 1.0), (72, 24.0 / 72.0)])
def test_axial_cis_known_answer(end, scale):
    """tests/test_phase3.cpp:118-178 known answers: window 24² scale 1, global
    72² scale 24/72; tolerance 1e-5 as there."""
    out = np.empty((end * end, 64), np.float32)
    L.orc_compute_axial_cis(orc.ptr(out), 64, end, end, 10000.0, scale)
    idx = np.arange(end * end)
    tx, ty = (idx % end) * scale, (idx // end) * scale
    freqs = 1.0 / 10000.0 ** (np.arange(16) * 4 / 64.0)
    ax, ay = np.outer(tx, freqs), np.outer(ty, freqs)
    ref = np.empty((end * end, 64))
    ref[:, 0:32:2], ref[:, 1:32:2] = np.cos(ax), np.sin(ax)
    ref[:, 32::2], ref[:, 33::2] = np.cos(ay), np.sin(ay)
    assert np.max(np.abs(out - ref)) <= 1e-5


def test_rope_is_complex_multiplication():
    rng = np.random.default_rng(9)
    HD, N, nh = 64, 50, 3
    x = rng.standard_normal((nh, N, HD)).astype(np.float32)
    f = np.empty((N, 64), np.float32)
    L.orc_compute_axial_cis(orc.ptr(f), 64, 10, 5, 10000.0, 1.0)
    y = x.copy()
    L.orc_rope(orc.ptr(y), HD, N, nh, orc.ptr(f))
    z = x[..., 0::2].astype(np.float64) + 1j * x[..., 1::2]
    c = f[:, 0::2].astype(np.float64) + 1j * f[:, 1::2]
    r = z * c[None]
    assert np.max(np.abs(y[..., 0::2] - r.real)) < 1e-5 and np.max(np.abs(y[..., 1::2] - r.imag)) < 1e-5


def _attn_f64(q, k, v, scale):
    s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), k.astype(np.float64)) * scale
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhij,bhjd->bihd", p, v.astype(np.float64))


@pytest.mark.parametrize("B,nh,Nq,Nkv", [(1, 1, 7, 9), (2, 3, 33, 65), (1, 2, 64, 200)])
def test_flash_attn_vs_f64(B, nh, Nq, Nkv):
    rng = np.random.default_rng(Nq)
    q = rng.standard_normal((B, nh, Nq, 64)).astype(np.float32) * 2
    k = rng.standard_normal((B, nh, Nkv, 64)).astype(np.float32)
    v = rng.standard_normal((B, nh, Nkv, 64)).astype(np.float32)
    o = np.empty((B, Nq, nh, 64), np.float32)
    L.orc_flash_attn_ext(orc.ptr(q), 64, Nq * 64, nh * Nq * 64, orc.ptr(k), 64, Nkv * 64, nh * Nkv * 64,
                         orc.ptr(v), 64, Nkv * 64, nh * Nkv * 64, 64, Nq, Nkv, nh, B, 0.125, orc.ptr(o), 0)
    assert orc.rel_l2(o, _attn_f64(q, k, v, 0.125)) <= 2e-6


def test_flash_attn_invariants():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 2, 40, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, 90, 64)).astype(np.float32)
    ones = np.ones((1, 2, 90, 64), np.float32)
    # V = 1 → O = 1 (rows of P sum to one)
    o = np.empty((1, 40, 2, 64), np.float32)
    L.orc_flash_attn_ext(orc.ptr(q), 64, 40 * 64, 2 * 40 * 64, orc.ptr(k), 64, 90 * 64, 2 * 90 * 64,
                         orc.ptr(ones), 64, 90 * 64, 2 * 90 * 64, 64, 40, 90, 2, 1, 0.125, orc.ptr(o), 0)
    assert np.max(np.abs(o - 1)) < 1e-6
    # permuting keys together with their values leaves the output unchanged
    v = rng.standard_normal((1, 2, 90, 64)).astype(np.float32)
    perm = rng.permutation(90)
    o1 = np.empty_like(o)
    o2 = np.empty_like(o)
    kp, vp = np.ascontiguousarray(k[:, :, perm]), np.ascontiguousarray(v[:, :, perm])
    for src_k, src_v, dst in ((k, v, o1), (kp, vp, o2)):
        L.orc_flash_attn_ext(orc.ptr(q), 64, 40 * 64, 2 * 40 * 64, orc.ptr(src_k), 64, 90 * 64, 2 * 90 * 64,
                             orc.ptr(src_v), 64, 90 * 64, 2 * 90 * 64, 64, 40, 90, 2, 1, 0.125, orc.ptr(dst), 0)
    assert orc.rel_l2(o2, o1) < 1e-6


# ---- preprocessing, encoder structure -----------------------------------------
def test_preprocess_identity_and_constant():
    rng = np.random.default_rng(4)
    img = rng.integers(0, 256, (28, 28, 3), dtype=np.uint8)
    chw = orc.preprocess_sam3(img, 28)
    ref = ((img.astype(np.float32) / np.float32(255) - np.float32(0.5)) / np.float32(0.5)).transpose(2, 0, 1)
    assert np.array_equal(chw, ref)
    const = np.full((50, 70, 3), 77, np.uint8)
    out = orc.preprocess_sam3(const, 28)
    assert np.all(out == np.float32((np.float32(77) / np.float32(255) - np.float32(0.5)) / np.float32(0.5)))


def _resize_u8(img, ow, oh):
    h, w, _ = img.shape
    out = np.empty((oh, ow, 3), np.uint8)
    orc.LIB.orc_resize_bilinear_u8(orc.ptr(np.ascontiguousarray(img)), w, h, orc.ptr(out), ow, oh)
    return out


def test_resize_exact_2x_downscale():
    """Halving: every output pixel sits at the centre of a 2×2 source block
    (half-pixel centres), so the result is the block mean rounded half up."""
    img = np.random.default_rng(8).integers(0, 256, (64, 96, 3), dtype=np.uint8)
    got = _resize_u8(img, 48, 32)
    s = img.astype(np.int64).reshape(32, 2, 48, 2, 3).sum(axis=(1, 3))
    assert np.array_equal(got, ((s * 2 + 4) // 8).astype(np.uint8))  # floor(s/4 + 0.5)


@pytest.mark.parametrize("w,h,ow,oh", [(1920, 1080, 1008, 1008), (640, 480, 336, 336), (100, 50, 336, 336),
                                       (7, 3, 64, 64), (1, 1, 16, 16), (1007, 1009, 1008, 1008),
                                       (333, 777, 1024, 1024)])
def test_resize_matches_torch_bilinear(w, h, ow, oh):
    """sam3_resize_bilinear against torch's bilinear interpolation
    (align_corners=False: half-pixel centres, source clamped at 0, edge
    replication) in float64, rounded half up.  The two evaluation orders may
    differ in the last bit of a value that is exactly half-way (an integer
    + 0.5 in exact arithmetic), so those ties — and only those — may round
    apart, by 1."""
    import torch
    import torch.nn.functional as F

    img = np.random.default_rng(w + h).integers(0, 256, (h, w, 3), dtype=np.uint8)
    got = _resize_u8(img, ow, oh)
    t = torch.from_numpy(img.astype(np.float64)).permute(2, 0, 1)[None]
    r = F.interpolate(t, size=(oh, ow), mode="bilinear", align_corners=False)[0].permute(1, 2, 0).numpy()
    ref = np.clip(np.floor(r + 0.5), 0, 255).astype(np.uint8)
    bad = got != ref
    assert np.abs(got.astype(int) - ref.astype(int)).max() <= 1
    assert bad.sum() <= 1e-4 * got.size
    assert np.all(np.abs(r[bad] - np.floor(r[bad]) - 0.5) < 1e-9)


@pytest.fixture(scope="module")
def s3e_mod():
    import s3e

    return s3e


def test_block_with_zero_weights_is_identity(s3e_mod, tmp_path):
    """All linear weights and biases zero: attention output and MLP output are
    zero, so each block returns its input unchanged (bit for bit)."""
    p = str(tmp_path / "zero.ggml")
    s3e_mod.synth_write(p, img_size=168, depth=2, window=4, global_idx=(1,), ftype="q4_0", seed=1, std=0.0)
    om = orc.OracleModel(p)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((144, 1024)).astype(np.float32)
    for bi in (0, 1):
        assert np.array_equal(om.block(bi, x), x)


def test_single_window_equals_global(s3e_mod, tmp_path):
    """A windowed block whose window covers the whole grid computes exactly the
    global block (same RoPE table, identity partition)."""
    pw, pg = str(tmp_path / "w.ggml"), str(tmp_path / "g.ggml")
    s3e_mod.synth_write(pw, img_size=168, depth=1, window=12, global_idx=(), ftype="q8_0", seed=3,
                        random_affine=True)
    s3e_mod.synth_write(pg, img_size=168, depth=1, window=12, global_idx=(0,), ftype="q8_0", seed=3,
                        random_affine=True)
    a, b = orc.OracleModel(pw), orc.OracleModel(pg)
    x = np.random.default_rng(1).standard_normal((144, 1024)).astype(np.float32)
    assert np.array_equal(a.block(0, x), b.block(0, x))


# ---- ggml's ARM NEON evaluation orders (orc_set_variant 2, 3, 4) ----------------
ARM_VARIANTS = [2, 3, 4]  # M4 Pro build (tinyBLAS for Q4_0/Q8_0), vec_dot nrc = 1, vec_dot nrc = 2


@pytest.mark.parametrize("v", ARM_VARIANTS)
@pytest.mark.parametrize("t", [orc.Q4_0, orc.Q4_1, orc.Q8_0])
def test_arm_orders_vs_f64(t, v):
    """Each ARM order, with its own (NEON) activation quantizer, against the
    float64 product of the same dequantized operands: K = 288 (nine blocks:
    an odd last block takes the nrc = 1 path's scalar tail)."""
    rng = np.random.default_rng(31 + t + v)
    M, N, K = 21, 40, 288
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    wb = orc.to_weight_bytes(t, W)
    vdt = orc.VEC_DOT[t]
    L.orc_set_variant(v)
    try:
        Y = orc.mul_mat(t, wb, N, K, X)
        xq = orc.from_float(vdt, X)
    finally:
        L.orc_set_variant(0)
    ref = orc.dequantize(vdt, xq, M, K).astype(np.float64) @ orc.dequantize(t, wb, N, K).astype(np.float64).T
    if t == orc.Q4_1:  # s = fp16(d·Σq) stands in for the exact block sum, as in every ggml order
        qx, dx, sx = orc.split_q8(vdt, xq, M, K)
        _, _, mw = _unpack(t, wb, N, K)
        exact_s = dx.view(np.float16).astype(np.float64) * qx.reshape(M, K // 32, 32).sum(axis=2)
        ref += (sx.view(np.float16).astype(np.float64) - exact_s) @ mw.T
    assert orc.rel_l2(Y, ref) <= 2e-7


@pytest.mark.parametrize("v", [0, 1] + ARM_VARIANTS)
def test_orders_exact_on_integer_data(v):
    """Q8_0 weights and activations whose scales are exactly 1 and whose
    codes are small integers: every product and partial sum is an exact
    integer in fp32, so every order must return the exact integer dot — a
    lane partition that dropped or repeated a group of four, or a block
    counted twice, would not."""
    rng = np.random.default_rng(40 + v)
    N, M, K = 7, 5, 320  # ten blocks
    qw = rng.integers(-9, 10, (N, K)).astype(np.int8)
    qx = rng.integers(-9, 10, (M, K)).astype(np.int8)
    one = np.uint16(0x3C00)  # fp16 1.0
    def blocks(q):
        R = q.shape[0]
        b = np.empty((R, K // 32, 34), np.uint8)
        b[:, :, :2] = np.full((R, K // 32), one, np.uint16).view(np.uint8).reshape(R, K // 32, 2)
        b[:, :, 2:] = q.reshape(R, K // 32, 32).view(np.uint8)
        return b.reshape(R, -1)
    wb, xb = blocks(qw), blocks(qx)
    Y = np.empty((M, N), np.float32)
    L.orc_set_variant(v)
    try:
        L.orc_mul_mat_preq(orc.Q8_0, orc.ptr(wb), N, K, orc.ptr(xb), M, orc.ptr(Y), 1)
    finally:
        L.orc_set_variant(0)
    assert np.array_equal(Y, (qx.astype(np.int64) @ qw.astype(np.int64).T).astype(np.float32))


def test_arm_quantizer_is_the_reference_quantizer_on_non_ties():
    """ggml's NEON quantize_row_q8_0 takes id = 1/d like the generic
    quantize_row_q8_0_ref (pinned by the golden fixtures) and differs from it
    only in rounding exact .5 ties (half to even instead of away), which
    random data does not hit; the x86 quantizer (id = 127/amax) lands on the
    other side of some rounding boundaries."""
    rng = np.random.default_rng(12)
    X = (rng.standard_normal((400, 1024)) * rng.uniform(0.1, 5, (400, 1))).astype(np.float32)
    ref = orc.quantize_ref(orc.Q8_0, X)
    L.orc_set_variant(2)
    try:
        arm = orc.from_float(orc.Q8_0, X)
    finally:
        L.orc_set_variant(0)
    assert np.array_equal(arm, ref)
    # known answer: amax = 1.4442534 (0x3fb8dd4c), x = 0.017058112
    # (0x3c8bbd74).  x86: id = fp32(127/amax) = 87.93471, x·id rounds to
    # 1.5000001 → code 2; NEON: id = fp32(1/fp32(amax/127)) = 87.9347, x·id
    # rounds to 1.4999999 → code 1 (the generic reference quantizer agrees)
    blk = np.zeros((1, 32), np.float32)
    blk[0, :2] = np.array([0x3FB8DD4C, 0x3C8BBD74], np.uint32).view(np.float32)
    x86 = orc.from_float(orc.Q8_0, blk)
    L.orc_set_variant(2)
    try:
        arm = orc.from_float(orc.Q8_0, blk)
    finally:
        L.orc_set_variant(0)
    ref = orc.quantize_ref(orc.Q8_0, blk)
    assert (x86[2:4].view(np.int8).tolist(), arm[2:4].view(np.int8).tolist()) == ([127, 2], [127, 1])
    assert np.array_equal(arm, ref)
