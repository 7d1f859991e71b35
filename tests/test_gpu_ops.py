"""GPU parity of the operator entry points against the CPU oracle.

- s3e_quantize_rows: bit-exact with ggml's x86 from_float (Q8_0, Q8_1, F16),
  including rows built so that x·127/amax lands exactly on k + 0.5.
- s3e_mul_mat: every weight type at small, ragged and SAM 3 ViT MLP shapes
  (fc1 N=4736 K=1024, fc2 N=1024 K=4736, M = 5184 and 64), and the
  weight-streaming kernel of products with at most 64 rows (M = 1 .. 64,
  ragged N and K).  Both sides use the same quantized activations, so only
  fp32 accumulation order differs: relative L2 ≤ 1e-5.
- s3e_mul_mat_q_batch: several products in one launch, equal to one
  s3e_mul_mat_q call each up to the order of the K-range accumulation
  (relative L2 ≤ 1e-6), and deterministic.
- s3e_flash_attn_ext: windowed (9 × 576) and global (5184) shapes, head dim
  64.  Default precision rounds Q, K, V and P to fp16 (fp32 accumulation):
  the F16 tolerance, relative L2 ≤ 2e-3.  F32 precision (fp16 hi/lo pairs)
  must match f32 attention: relative L2 ≤ 1e-5.
"""
import numpy as np
import pytest

import oracle_lib as orc
import s3e

pytestmark = pytest.mark.gpu


def _tie_rows(K):
    """Rows whose scaled values sit exactly on k + 0.5 (amax = 127 → id = 1,
    amax = 63.5 → id = 2), so round-half-even and round-half-away differ."""
    r0 = np.zeros(K, np.float32)
    r0[0::32] = 127.0
    base = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, -3.5, 100.5, -100.5, 126.5, -126.5], np.float32)
    for b in range(K // 32):
        r0[b * 32 + 1:b * 32 + 1 + len(base)] = base
    r1 = np.zeros(K, np.float32)
    r1[0::32] = -63.5
    for b in range(K // 32):
        r1[b * 32 + 1:b * 32 + 1 + len(base)] = base / 2
    return np.stack([r0, r1])


@pytest.mark.parametrize("vdt", [orc.Q8_0, orc.Q8_1, orc.F16])
def test_quantize_rows_bit_exact(ctx, vdt):
    rng = np.random.default_rng(11)
    M, K = 258, 1024
    X = (rng.standard_normal((M, K)) * rng.uniform(1e-3, 30, (M, 1))).astype(np.float32)
    X[:2] = _tie_rows(K)
    X[2] = 0.0  # all-zero row: d = 0, q = 0
    ref = orc.from_float(vdt, X)
    Xd = ctx.to_device(X)
    if vdt == orc.F16:
        qs = ctx.buffer(M * K * 2)
        ctx.quantize_rows(vdt, Xd, M, K, qs, None, None)
        ctx.sync()
        got = qs.download(np.uint16, (M, K))
        assert np.array_equal(got.view(np.uint8).ravel(), ref)
        return
    ns = s3e.act_scale_elems(M, K)
    qs, d, s = ctx.buffer(M * K), ctx.buffer(ns * 2), ctx.buffer(ns * 2)
    ctx.quantize_rows(vdt, Xd, M, K, qs, d, s)
    ctx.sync()
    rq, rd, rs = orc.split_q8(vdt, ref, M, K)
    assert np.array_equal(qs.download(np.int8, (M, K)), rq)
    assert np.array_equal(s3e.unstage_scales(d.download(np.uint16, (ns,)), M, K), rd)
    if vdt == orc.Q8_1:
        assert np.array_equal(s3e.unstage_scales(s.download(np.uint16, (ns,)), M, K), rs)


@pytest.mark.parametrize("wt", [orc.Q4_0, orc.Q4_1, orc.Q8_0, orc.F16],
                         ids=lambda t: {1: "f16", 2: "q4_0", 3: "q4_1", 8: "q8_0"}[t])
@pytest.mark.parametrize("M,N,K", [(200, 256, 160), (130, 384, 1024)])
def test_mul_mat_q_matches_mul_mat(ctx, wt, M, N, K):
    """s3e_mul_mat_q on s3e_quantize_rows output (the documented layout, K not a
    multiple of 128 included) runs the same kernel as s3e_mul_mat: identical."""
    rng = np.random.default_rng(M + N + K + wt)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    wb = orc.to_weight_bytes(wt, W)
    w = ctx.weight(wt, K, N, wb)
    Xd, Y1, Y2 = ctx.to_device(X), ctx.buffer(M * N * 4), ctx.buffer(M * N * 4)
    ctx.mul_mat(w, Xd, M, Y1)
    vdt = orc.VEC_DOT[wt]
    ns = s3e.act_scale_elems(M, K)
    qs, d, s = ctx.buffer(M * K * 2), ctx.buffer(ns * 2), ctx.buffer(ns * 2)
    ctx.quantize_rows(vdt, Xd, M, K, qs, d if wt != orc.F16 else None, s if wt != orc.F16 else None)
    ctx.mul_mat_q(w, qs, d if wt != orc.F16 else None, s if wt == orc.Q4_1 else None, M, Y2)
    ctx.sync()
    a, b = Y1.download(np.float32, (M, N)), Y2.download(np.float32, (M, N))
    assert np.array_equal(a, b)
    ref = orc.mul_mat(wt, wb, N, K, X)
    assert orc.rel_l2(b, ref) <= 1e-5


@pytest.mark.parametrize("rows,n", [(5184, 1024), (77, 96), (33, 4096)])
def test_layer_norm_bit_exact(ctx, rows, n):
    rng = np.random.default_rng(rows + n)
    x = (rng.standard_normal((rows, n)) * rng.uniform(0.01, 20, (rows, 1)) + rng.normal(0, 3, (rows, 1))).astype(np.float32)
    w = (1 + rng.normal(0, 0.1, n)).astype(np.float32)
    b = rng.normal(0, 0.1, n).astype(np.float32)
    ref = orc.layer_norm(x, 1e-5, w, b)
    xd, wd, bd = ctx.to_device(x), ctx.to_device(w), ctx.to_device(b)
    ctx.layer_norm(xd, rows, n, 1e-5, wd, bd, xd)  # in place, as the encoder uses it
    ctx.sync()
    got = xd.download(np.float32, (rows, n))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"{np.sum(got != ref)} values differ"


SHAPES = [(64, 128, 128), (100, 96, 64), (37, 256, 4736), (5184, 4736, 1024), (5184, 1024, 4736),
          (64, 4736, 1024), (64, 1024, 4736)]
WTYPES = [orc.Q4_0, orc.Q4_1, orc.Q8_0, orc.F16, orc.F32]


@pytest.mark.parametrize("wt", WTYPES, ids=lambda t: {0: "f32", 1: "f16", 2: "q4_0", 3: "q4_1", 8: "q8_0"}[t])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_mul_mat(ctx, wt, M, N, K):
    rng = np.random.default_rng(M * 7 + N * 3 + K + wt)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    wb = orc.to_weight_bytes(wt, W)
    ref = orc.mul_mat(wt, wb, N, K, X) + bias
    w = ctx.weight(wt, K, N, wb)
    Xd, bd, Yd = ctx.to_device(X), ctx.to_device(bias), ctx.buffer(M * N * 4)
    ctx.mul_mat(w, Xd, M, Yd, bd)
    ctx.sync()
    Y = Yd.download(np.float32, (M, N))
    err = orc.rel_l2(Y, ref)
    print(f"mul_mat type={wt} M={M} N={N} K={K}: rel_l2={err:.3e} max_abs={orc.max_abs(Y, ref):.3e}")
    assert err <= 1e-5


def _random_shapes(n, seed):
    """Ragged products for every weight type: M from 1 to 900 (the small-M
    kernels up to 64 rows, split-K below a CU's worth of tiles, partial row
    and column tiles), N from 1 to 1500 (not a multiple of 4 or 128), K a
    multiple of 32 (a ggml block) that need not be one of 128 (a stage)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        wt = WTYPES[i % len(WTYPES)]
        M = int(rng.integers(1, 65)) if i % 3 == 0 else int(rng.integers(65, 901))
        out.append((wt, M, int(rng.integers(1, 1501)), 32 * int(rng.integers(1, 81))))
    return out


@pytest.mark.parametrize("wt,M,N,K", _random_shapes(20, 2026),
                         ids=lambda v: str(v) if not isinstance(v, tuple) else None)
def test_mul_mat_ragged_shapes(ctx, wt, M, N, K):
    rng = np.random.default_rng(M * 131 + N * 7 + K + wt)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    wb = orc.to_weight_bytes(wt, W)
    ref = orc.mul_mat(wt, wb, N, K, X) + bias
    w = ctx.weight(wt, K, N, wb)
    Xd, bd, Yd = ctx.to_device(X), ctx.to_device(bias), ctx.buffer(M * N * 4)
    ctx.mul_mat(w, Xd, M, Yd, bd)
    ctx.sync()
    Y = Yd.download(np.float32, (M, N))
    err = orc.rel_l2(Y, ref)
    print(f"ragged mul_mat type={wt} M={M} N={N} K={K}: rel_l2={err:.3e} max_abs={orc.max_abs(Y, ref):.3e}", flush=True)
    assert np.all(np.isfinite(Y))
    assert err <= 1e-5


@pytest.mark.parametrize("M,N,K", [(100, 384, 1024), (777, 1024, 4736), (5184, 4736, 1024), (2000, 4096, 256)])
def test_mul_mat_q_f6(ctx, M, N, K):
    """Q4_0 products on the fp6 kernel (activations as S3E_TYPE_Q8_0_F6X2)
    equal the int8 kernel's bit for bit (the same exact block sums, the same
    scale products and FMA order), and the oracle to fp32 order noise
    (2000 rows end inside a 64-row unit of the fp6 activation layout)."""
    import s3e

    rng = np.random.default_rng(M + N + K)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    wb = orc.to_weight_bytes(orc.Q4_0, W)
    w = ctx.weight(orc.Q4_0, K, N, wb)
    Xd, bd = ctx.to_device(X), ctx.to_device(bias)
    ns = s3e.act_scale_elems(M, K)
    q8, d8 = ctx.buffer(M * K), ctx.buffer(ns * 2)
    f6, d6 = ctx.buffer((M + 63) // 64 * 64 * K * 3 // 2), ctx.buffer(ns * 2)
    ctx.quantize_rows(s3e.TYPE_Q8_0, Xd, M, K, q8, d8, None)
    ctx.quantize_rows(s3e.TYPE_Q8_0_F6X2, Xd, M, K, f6, d6, None)
    Y8, Y6 = ctx.buffer(M * N * 4), ctx.buffer(M * N * 4)
    ctx.mul_mat_q(w, q8, d8, None, M, Y8, bd)
    ctx.mul_mat_q_f6(w, f6, d6, M, Y6, bd)
    ctx.sync()
    y8, y6 = Y8.download(np.float32, (M, N)), Y6.download(np.float32, (M, N))
    ref = orc.mul_mat(orc.Q4_0, wb, N, K, X) + bias
    err = orc.rel_l2(y6, ref)
    print(f"mul_mat_q_f6 M={M} N={N} K={K}: differing from int8 {np.count_nonzero(y6 != y8)}, rel_l2={err:.3e}")
    assert np.array_equal(y6, y8)
    assert err <= 1e-5
    w.free()


def test_mul_mat_q_f6_rejects(ctx):
    import s3e

    rng = np.random.default_rng(9)
    W = rng.normal(0, 0.02, (64, 96)).astype(np.float32)
    w = ctx.weight(orc.Q4_0, 96, 64, orc.to_weight_bytes(orc.Q4_0, W))  # K % 128 != 0: no fp6 copy
    buf = ctx.buffer(1 << 16)
    with pytest.raises(s3e.S3EError):
        ctx.mul_mat_q_f6(w, buf, buf, 8, buf)
    with pytest.raises(s3e.S3EError):
        ctx.quantize_rows(s3e.TYPE_Q8_0_F6X2, buf, 8, 96, buf, buf, None)
    w.free()


SMALL_M = [1, 5, 32, 33, 64]


@pytest.mark.parametrize("wt", [orc.Q4_0, orc.Q4_1, orc.Q8_0, orc.F16],
                         ids=lambda t: {1: "f16", 2: "q4_0", 3: "q4_1", 8: "q8_0"}[t])
@pytest.mark.parametrize("N,K", [(40, 96), (4736, 1024), (1024, 4736), (200, 160)])
def test_mul_mat_small_m(ctx, wt, N, K):
    """The weight-streaming kernel (M ≤ 64) against the oracle at ragged N, K
    not a multiple of 128 and row counts around its 32-row tiles; one weight
    serves every M, so its packed copy is made once and reused."""
    rng = np.random.default_rng(N + K + wt)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    wb = orc.to_weight_bytes(wt, W)
    w = ctx.weight(wt, K, N, wb)
    bd = ctx.to_device(bias)
    for M in SMALL_M:
        X = rng.standard_normal((M, K)).astype(np.float32)
        ref = orc.mul_mat(wt, wb, N, K, X) + bias
        Xd, Yd = ctx.to_device(X), ctx.buffer(M * N * 4)
        ctx.mul_mat(w, Xd, M, Yd, bd)
        ctx.sync()
        Y = Yd.download(np.float32, (M, N))
        err = orc.rel_l2(Y, ref)
        print(f"small-M type={wt} M={M} N={N} K={K}: rel_l2={err:.3e}", flush=True)
        assert err <= 1e-5, M


@pytest.mark.parametrize("wt", [orc.Q4_0, orc.Q8_0], ids=lambda t: {2: "q4_0", 8: "q8_0"}[t])
def test_mul_mat_small_m_split_repeats(ctx, wt):
    """Lone small-M products whose K range is split across work-groups (few
    32-column strips, long K: the fc2 shape has 32 strips over 37 stages of
    128; 96 × 2048 and 96 × 1024 split into 4 and 2 ranges) give the same
    bits on every call, also with products of other widths in between, and
    match the oracle."""
    rng = np.random.default_rng(wt + 11)
    cases = []
    for N, K, M in [(1024, 4736, 64), (4736, 1024, 7), (96, 2048, 33), (1024, 4736, 1), (96, 1024, 33)]:
        W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
        wb = orc.to_weight_bytes(wt, W)
        X = rng.standard_normal((M, K)).astype(np.float32)
        ref = orc.mul_mat(wt, wb, N, K, X)
        cases.append((ctx.weight(wt, K, N, wb), ctx.to_device(X), ctx.buffer(M * N * 4), M, N, K, ref))
    first = {}
    for rep in range(3):
        for i, (w, Xd, Yd, M, N, K, ref) in enumerate(cases):
            ctx.mul_mat(w, Xd, M, Yd)
            ctx.sync()
            Y = Yd.download(np.float32, (M, N))
            if rep == 0:
                err = orc.rel_l2(Y, ref)
                print(f"split small-M type={wt} M={M} N={N} K={K}: rel_l2={err:.3e}", flush=True)
                assert err <= 1e-5, (M, N, K)
                first[i] = Y
            else:
                assert np.array_equal(Y, first[i]), (rep, M, N, K)
    for w, *_ in cases:
        w.free()


@pytest.mark.parametrize("wt", [orc.Q4_0, orc.Q4_1, orc.Q8_0, orc.F16],
                         ids=lambda t: {1: "f16", 2: "q4_0", 3: "q4_1", 8: "q8_0"}[t])
def test_mul_mat_q_batch_matches_single(ctx, wt):
    """Independent products of different shapes in one launch match what
    s3e_mul_mat_q gives for each of them (same block sums, the K range
    accumulated in another order: relative L2 ≤ 1e-6) and the oracle; a
    repeated batch reuses its descriptors and reproduces itself bit for bit,
    and a different batch replaces them."""
    rng = np.random.default_rng(wt + 3)
    M = 48
    shapes = [(3072, 1024), (1024, 1024), (40, 96), (4736, 1024), (1024, 4736)]
    vdt = orc.VEC_DOT[wt]
    ws, xq, ds, ss, ys, bs, ref = [], [], [], [], [], [], []
    for N, K in shapes:
        W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
        ws.append(ctx.weight(wt, K, N, orc.to_weight_bytes(wt, W)))
        X = rng.standard_normal((M, K)).astype(np.float32)
        ns = s3e.act_scale_elems(M, K)
        q, d, s_ = ctx.buffer(M * K * 2), ctx.buffer(ns * 2), ctx.buffer(ns * 2)
        ctx.quantize_rows(vdt, ctx.to_device(X), M, K, q, d if wt != orc.F16 else None,
                          s_ if wt != orc.F16 else None)
        xq.append(q)
        ds.append(d if wt != orc.F16 else None)
        ss.append(s_ if wt == orc.Q4_1 else None)
        bs.append(ctx.to_device(rng.normal(0, 0.1, N).astype(np.float32)))
        ys.append(ctx.buffer(M * N * 4))
        y1 = ctx.buffer(M * N * 4)
        ctx.mul_mat_q(ws[-1], q, ds[-1], ss[-1], M, y1, bs[-1])
        ref.append(y1)
    first = None
    for rep in range(2):
        ctx.mul_mat_q_batch(ws, xq, ds, ss, M, bs, ys)
        ctx.sync()
        outs = [y.download(np.float32, (M, N)) for (N, K), y in zip(shapes, ys)]
        for (N, K), o, r in zip(shapes, outs, ref):
            assert orc.rel_l2(o, r.download(np.float32, (M, N))) <= 1e-6, (rep, N, K)
        if first is None:
            first = outs
        else:
            assert all(np.array_equal(a, b) for a, b in zip(first, outs))
    # a different batch (two of the products, no bias) replaces the descriptors;
    # a product does not depend on its neighbours in the batch
    ctx.mul_mat_q_batch(ws[2:4], xq[2:4], ds[2:4], ss[2:4], M, None, ys[2:4])
    ctx.sync()
    for i in (2, 3):
        N, K = shapes[i]
        bias = bs[i].download(np.float32, (N,))
        got = ys[i].download(np.float32, (M, N))
        assert np.array_equal(got + bias, first[i]) or orc.rel_l2(got + bias, first[i]) <= 1e-6


def test_mul_mat_q_batch_rejects(ctx):
    W = np.zeros((64, 64), np.float32)
    a = ctx.weight(orc.Q8_0, 64, 64, orc.to_weight_bytes(orc.Q8_0, W))
    b = ctx.weight(orc.F16, 64, 64, orc.to_weight_bytes(orc.F16, W))
    q, d, y = ctx.buffer(64 * 64), ctx.buffer(4096), ctx.buffer(64 * 64 * 4)
    with pytest.raises(s3e.S3EError):
        ctx.mul_mat_q_batch([a, b], [q, q], [d, d], None, 8, None, [y, y])  # mixed weight types
    with pytest.raises(s3e.S3EError):
        ctx.mul_mat_q_batch([a], [q], [d], None, 65, None, [y])  # more than 64 rows
    with pytest.raises(s3e.S3EError):
        ctx.mul_mat_q_batch([a], [q], None, None, 8, None, [y])  # quantized without scales


@pytest.mark.parametrize("prec", [0, 1], ids=["fp16", "f32"])
@pytest.mark.parametrize("B,nh,N", [(1, 2, 64), (2, 3, 100), (9, 16, 576), (1, 2, 5184), (1, 16, 5184)])
def test_flash_attn(ctx, B, nh, N, prec):
    rng = np.random.default_rng(B * 100 + nh * 10 + N)
    q = rng.standard_normal((B, nh, N, 64)).astype(np.float32)
    k = rng.standard_normal((B, nh, N, 64)).astype(np.float32)
    # V laid out [B][N][nh][64] and read through strides, like the strided V
    # view of sam3.cpp:3762-3763
    v_tok = rng.standard_normal((B, N, nh, 64)).astype(np.float32)
    v = np.ascontiguousarray(v_tok.transpose(0, 2, 1, 3))
    scale = 1.0 / 8.0
    ref = orc.flash_attn(q, k, v, scale)
    qd, kd, vd = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v_tok)
    od = ctx.buffer(B * N * nh * 64 * 4)
    qk_nb = (1, 64, N * 64, nh * N * 64)
    v_nb = (1, nh * 64, 64, N * nh * 64)
    ctx.flash_attn_ext(qd, qk_nb, kd, qk_nb, vd, v_nb, 64, N, N, nh, B, scale, od, prec=prec)
    ctx.sync()
    out = od.download(np.float32, (B, N, nh, 64))
    err = orc.rel_l2(out, ref)
    print(f"flash_attn prec={prec} B={B} nh={nh} N={N}: rel_l2={err:.3e} max_abs={orc.max_abs(out, ref):.3e}")
    # fp16 operands: the F16 tolerance; split fp16 pairs: f32 attention up to
    # accumulation order and exp2 vs expf rounding
    assert err <= (2e-3 if prec == 0 else 1e-5)


@pytest.mark.parametrize("D,B,nh,Nq,Nkv,prec", [
    (96, 2, 2, 64, 64, 1), (96, 1, 4, 49, 196, 1), (56, 3, 2, 16, 64, 1), (32, 1, 2, 200, 200, 1),
    (72, 1, 3, 100, 130, 0), (128, 1, 2, 300, 300, 1), (64, 1, 1, 256, 4096, 1), (64, 1, 2, 100, 2000, 0),
    (256, 1, 1, 512, 4096, 0), (256, 1, 1, 100, 1100, 0)],
    ids=lambda x: str(x))
def test_flash_attn_head_dims(ctx, D, B, nh, Nq, Nkv, prec):
    """Hiera head dims (96, 56, 72, 32: zero-padded to 64 / 128 internally),
    pooled queries (Nq ≠ Nkv), 128, the memory attention's 256 (fp16
    operands), and single-head shapes long enough in keys to take the
    key-split path; V through strides as in the ViT test."""
    rng = np.random.default_rng(D * 7 + Nq + Nkv)
    q = rng.standard_normal((B, nh, Nq, D)).astype(np.float32)
    k = rng.standard_normal((B, nh, Nkv, D)).astype(np.float32)
    v_tok = rng.standard_normal((B, Nkv, nh, D)).astype(np.float32)
    v = np.ascontiguousarray(v_tok.transpose(0, 2, 1, 3))
    scale = 1.0 / np.sqrt(D)
    ref = orc.flash_attn(q, k, v, scale)
    qd, kd, vd = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v_tok)
    od = ctx.buffer(B * Nq * nh * D * 4)
    print(f"flash_attn D={D} B={B} nh={nh} Nq={Nq} Nkv={Nkv} prec={prec}", flush=True)
    ctx.flash_attn_ext(qd, (1, D, Nq * D, nh * Nq * D), kd, (1, D, Nkv * D, nh * Nkv * D), vd,
                       (1, nh * D, D, Nkv * nh * D), D, Nq, Nkv, nh, B, scale, od, prec=prec)
    ctx.sync()
    out = od.download(np.float32, (B, Nq, nh, D))
    err = orc.rel_l2(out, ref)
    print(f"  rel_l2={err:.3e} max_abs={orc.max_abs(out, ref):.3e}", flush=True)
    assert err <= (2e-3 if prec == 0 else 1e-5)


def _ragged_attn(n, seed):
    """Edge and ragged attention shapes: a single query and key, fewer keys than
    one 32-key tile, then random Nq and Nkv up to 900 with head dims 64 and 128,
    both precisions."""
    out = [(64, 1, 1, 1, 1, 1), (64, 1, 2, 3, 17, 0), (128, 2, 1, 33, 5, 1)]
    rng = np.random.default_rng(seed)
    for i in range(n):
        out.append((64 if i % 2 == 0 else 128, int(rng.integers(1, 3)), int(rng.integers(1, 5)),
                    int(rng.integers(1, 901)), int(rng.integers(1, 901)), i % 3 != 0))
    return [tuple(int(v) for v in c) for c in out]


@pytest.mark.parametrize("D,B,nh,Nq,Nkv,prec", _ragged_attn(7, 2027), ids=lambda x: str(x))
def test_flash_attn_ragged(ctx, D, B, nh, Nq, Nkv, prec):
    rng = np.random.default_rng(D + 3 * Nq + 5 * Nkv + 7 * nh + B)
    q = rng.standard_normal((B, nh, Nq, D)).astype(np.float32)
    k = rng.standard_normal((B, nh, Nkv, D)).astype(np.float32)
    v_tok = rng.standard_normal((B, Nkv, nh, D)).astype(np.float32)
    v = np.ascontiguousarray(v_tok.transpose(0, 2, 1, 3))
    scale = 1.0 / np.sqrt(D)
    ref = orc.flash_attn(q, k, v, scale)
    qd, kd, vd = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v_tok)
    od = ctx.buffer(B * Nq * nh * D * 4)
    print(f"ragged flash_attn D={D} B={B} nh={nh} Nq={Nq} Nkv={Nkv} prec={prec}", flush=True)
    ctx.flash_attn_ext(qd, (1, D, Nq * D, nh * Nq * D), kd, (1, D, Nkv * D, nh * Nkv * D), vd,
                       (1, nh * D, D, Nkv * nh * D), D, Nq, Nkv, nh, B, scale, od, prec=prec)
    ctx.sync()
    out = od.download(np.float32, (B, Nq, nh, D))
    err = orc.rel_l2(out, ref)
    print(f"  rel_l2={err:.3e} max_abs={orc.max_abs(out, ref):.3e}", flush=True)
    assert np.all(np.isfinite(out))
    assert err <= (2e-3 if prec == 0 else 1e-5)


def test_flash_attn_rejects(ctx):
    buf = ctx.buffer(1 << 20)
    nb = (1, 64, 64 * 64, 64 * 64)
    for D, prec in [(130, 1), (6, 1), (256, 1), (192, 0), (0, 1)]:
        with pytest.raises(s3e.S3EError):
            ctx.flash_attn_ext(buf, nb, buf, nb, buf, nb, D, 8, 8, 1, 1, 0.125, buf, prec=prec)
    # past the launch limits (batch × heads on one grid axis, 2^24 tokens);
    # refused on the host before anything is read
    for Nq, Nkv, nh, B in [(8, 8, 65536, 1), (8, 8, 256, 256), ((1 << 24) + 1, 8, 1, 1), (8, (1 << 24) + 1, 1, 1)]:
        with pytest.raises(s3e.S3EError):
            ctx.flash_attn_ext(buf, nb, buf, nb, buf, nb, 64, Nq, Nkv, nh, B, 0.125, buf, prec=1)


@pytest.mark.parametrize("wt", [orc.Q4_0, orc.Q4_1, orc.Q8_0, orc.F16, orc.F32],
                         ids=lambda t: {0: "f32", 1: "f16", 2: "q4_0", 3: "q4_1", 8: "q8_0"}[t])
def test_empty_shapes(ctx, wt):
    """An empty batch: ggml_mul_mat over zero rows of X is a no-op (the call
    succeeds and writes nothing, also through the activation conversion),
    a negative row count is refused, and flash attention refuses an empty
    query, key, head or batch extent."""
    rng = np.random.default_rng(wt + 21)
    N, K = 64, 128
    w = ctx.weight(wt, K, N, orc.to_weight_bytes(wt, rng.normal(0, 0.02, (N, K)).astype(np.float32)))
    X = ctx.to_device(rng.standard_normal((2, K)).astype(np.float32))
    sentinel = np.full((2, N), 7.0, np.float32)
    Yd = ctx.to_device(sentinel)
    ctx.mul_mat(w, X, 0, Yd)
    ctx.sync()
    assert np.array_equal(Yd.download(np.float32, (2, N)), sentinel)
    with pytest.raises(s3e.S3EError):
        ctx.mul_mat(w, X, -1, Yd)
    if wt != orc.F32:
        vdt = orc.VEC_DOT[wt]
        qs = ctx.buffer(4096)
        ctx.quantize_rows(vdt, X, 0, K, qs, qs if vdt != orc.F16 else None, qs if vdt == orc.Q8_1 else None)
        ctx.sync()
    w.free()
    buf = ctx.buffer(1 << 20)
    nb = (1, 64, 64 * 64, 64 * 64)
    for Nq, Nkv, nh, B in [(0, 8, 1, 1), (8, 0, 1, 1), (8, 8, 0, 1), (8, 8, 1, 0)]:
        with pytest.raises(s3e.S3EError):
            ctx.flash_attn_ext(buf, nb, buf, nb, buf, nb, 64, Nq, Nkv, nh, B, 0.125, buf, prec=1)


def _f16_bits(a):
    return np.ascontiguousarray(a.astype(np.float16)).view(np.uint16)


@pytest.mark.parametrize("D,B,nh,Nq,Nkv,layout", [
    (64, 9, 16, 576, 576, "plain"), (64, 1, 16, 5184, 5184, "plain"), (64, 1, 2, 100, 130, "plain"),
    (64, 2, 3, 200, 200, "tokens"), (96, 1, 4, 49, 196, "plain"), (128, 1, 2, 300, 300, "plain"),
    (256, 1, 1, 512, 4096, "plain"), (64, 1, 1, 256, 4096, "tokens")],
    ids=lambda x: str(x))
def test_flash_attn_f16(ctx, D, B, nh, Nq, Nkv, layout):
    """s3e_flash_attn_ext_f16: fp16 Q/K/V bits in ggml's strides.  "plain":
    Q, K, V contiguous [B][nh][N][D] (Q and K read in place at D = 64 / 128);
    "tokens": all three token-major [B][N][nh][D] (copied), like the ViT's
    strided views.  Reference: f32 attention of the same fp16 values; the
    kernel rounds the probabilities to fp16 (the F16 tolerance).  Two calls
    in a row check that the workspace kept from the first (larger or
    smaller) does not leak into the second."""
    rng = np.random.default_rng(D + 3 * Nq + Nkv + (7 if layout == "tokens" else 0))
    qt = rng.standard_normal((B, Nq, nh, D)).astype(np.float16)
    kt = rng.standard_normal((B, Nkv, nh, D)).astype(np.float16)
    vt = rng.standard_normal((B, Nkv, nh, D)).astype(np.float16)
    q, k, v = (np.ascontiguousarray(a.transpose(0, 2, 1, 3)) for a in (qt, kt, vt))
    scale = 1.0 / np.sqrt(D)
    ref = orc.flash_attn(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), scale)
    if layout == "plain":
        src = (q, k, v)
        nbq, nbk = (1, D, Nq * D, nh * Nq * D), (1, D, Nkv * D, nh * Nkv * D)
    else:
        src = (qt, kt, vt)
        nbq, nbk = (1, nh * D, D, Nq * nh * D), (1, nh * D, D, Nkv * nh * D)
    qd, kd, vd = (ctx.to_device(_f16_bits(a)) for a in src)
    od = ctx.buffer(B * Nq * nh * D * 4)
    for call in range(2):
        ctx.flash_attn_ext_f16(qd, nbq, kd, nbk, vd, nbk, D, Nq, Nkv, nh, B, scale, od)
        ctx.sync()
        out = od.download(np.float32, (B, Nq, nh, D))
        err = orc.rel_l2(out, ref)
        print(f"flash_attn_f16 D={D} B={B} nh={nh} Nq={Nq} Nkv={Nkv} {layout} call {call}: rel_l2={err:.3e}")
        assert err <= 2e-3
    for b in (qd, kd, vd, od):
        b.free()


def test_flash_attn_f16_rejects(ctx):
    import s3e

    x = ctx.buffer(64 * 64 * 2)
    o = ctx.buffer(64 * 64 * 4)
    nb = (1, 64, 64 * 64, 64 * 64)
    with pytest.raises(s3e.S3EError):
        ctx.flash_attn_ext_f16(x, nb, x, nb, x, nb, 60 + 2, 64, 64, 1, 1, 0.1, o)  # head dim not a multiple of 4
    with pytest.raises(s3e.S3EError):
        ctx.flash_attn_ext_f16(x, (2, 64, 4096, 4096), x, nb, x, nb, 64, 64, 64, 1, 1, 0.1, o)  # strided d
    # empty extents, and past the launch limits; refused on the host
    for Nq, Nkv, nh, B in [(0, 64, 1, 1), (64, 0, 1, 1), (64, 64, 0, 1), (64, 64, 1, 0), (8, 8, 65536, 1),
                           ((1 << 24) + 1, 8, 1, 1)]:
        with pytest.raises(s3e.S3EError):
            ctx.flash_attn_ext_f16(x, nb, x, nb, x, nb, 64, Nq, Nkv, nh, B, 0.1, o)


def _ggml_q8_0_rows(codes: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """ggml block_q8_0 rows (fp16 d, then 32 int8 codes per block) from codes
    [M][K] and scale bits [M][K/32]."""
    M, K = codes.shape
    out = np.empty((M, K // 32, 34), np.uint8)
    out[:, :, :2] = d_bits.astype(np.uint16).view(np.uint8).reshape(M, K // 32, 2)
    out[:, :, 2:] = codes.reshape(M, K // 32, 32).view(np.uint8)
    return out.reshape(M, -1)


@pytest.mark.parametrize("wt", [orc.Q4_0, orc.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("M,N,K", [(1024, 4096, 1024), (5184, 1024, 4736), (300, 2304, 96)])
def test_mul_mat_q_equals_ggml_i8mm_order(ctx, wt, M, N, K):
    """ggml's ARM vec_dot with two rows per call (vmmlaq_s32, the i8mm path
    of arch/arm/quants.c [ext]) forms every output as one fp32 chain
    acc = fma(S_b, d_w·d_x, acc) over the exact integer block sums S_b, which
    is the engine's order for Q4_0 and Q8_0 products.  On the same
    quantized activations the GPU (int8 kernel; for Q4_0 also the fp6
    kernel) equals the oracle's restatement of that order bit for bit: two
    independent implementations of it agree.  Shapes with enough tiles that
    no K split applies, K a multiple of 128 or not."""
    import s3e

    rng = np.random.default_rng(M + N + K + wt)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    wb = orc.to_weight_bytes(wt, W)
    w = ctx.weight(wt, K, N, wb)
    Xd = ctx.to_device(X)
    ns = s3e.act_scale_elems(M, K)
    q8, d8 = ctx.buffer(M * K), ctx.buffer(ns * 2)
    ctx.quantize_rows(s3e.TYPE_Q8_0, Xd, M, K, q8, d8, None)
    Y = ctx.buffer(M * N * 4)
    ctx.mul_mat_q(w, q8, d8, None, M, Y)
    ctx.sync()
    got = Y.download(np.float32, (M, N))
    codes = q8.download(np.int8, (M, K))
    dbits = s3e.unstage_scales(d8.download(np.uint16, (ns,)), M, K)
    xq = _ggml_q8_0_rows(codes, dbits)
    ref = np.empty((M, N), np.float32)
    orc.LIB.orc_set_variant(4)  # ORC_VARIANT_ARM_I8MM
    try:
        orc.LIB.orc_mul_mat_preq(wt, orc.ptr(wb), N, K, orc.ptr(xq), M, orc.ptr(ref), 0)
    finally:
        orc.LIB.orc_set_variant(0)
    diff = np.count_nonzero(got != ref)
    print(f"i8mm order wt={wt} M={M} N={N} K={K}: {diff} of {got.size} differ, rel_l2={orc.rel_l2(got, ref):.3e}")
    assert diff == 0
    if wt == orc.Q4_0 and K % 128 == 0:
        f6, d6 = ctx.buffer((M + 63) // 64 * 64 * K * 3 // 2), ctx.buffer(ns * 2)
        ctx.quantize_rows(s3e.TYPE_Q8_0_F6X2, Xd, M, K, f6, d6, None)
        Y6 = ctx.buffer(M * N * 4)
        ctx.mul_mat_q_f6(w, f6, d6, M, Y6)
        ctx.sync()
        assert np.array_equal(Y6.download(np.float32, (M, N)), ref)
    w.free()
