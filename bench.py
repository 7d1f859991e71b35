#!/usr/bin/env python3
"""Benchmark: SAM 3 image encoder (ViT backbone + SimpleFPN neck) on one MI355X.

Workload: the SAM 3 visual encoder at 1008×1008 (72×72 tokens, 32 blocks,
width 1024, 16 heads, MLP 4736, 24×24 windows, global blocks 7/15/23/31)
followed by the tracker neck to 256-channel features at 288², 144², 72² and
36² (a visual-only model), random-init weights N(0, 0.02) with the ViT's
linear weights quantized to Q4_0 (default; --ftype selects q8_0, q4_1, f16,
f32), one synthetic uniform-uint8 image preprocessed as sam3.cpp does.  A
step is one full encode of that image with the input already resident in
HBM; value = ms per frame (lower is better).  The neck's share is measured
separately (s3e_run_neck on the same backbone output) and reported as
breakdown.neck_ms.

Also reported, on the same JSON line:
  roofline      — the dominant kernel (the fc1 GEMM, M=5184 N=4736 K=1024,
                  the largest of the four per-block GEMMs, on the kernel the
                  encoder runs for the weight type: the fp6 kernel for Q4_0)
                  timed alone with HIP events on the engine's stream:
                  algorithmic ops 2·M·N·K per launch ÷ average launch time,
                  against the MI355X dense int8 MFMA peak (fp16 for F16
                  weights, fp32 for F32).  `traffic` comes from the committed
                  rocprofv3 FETCH_SIZE / WRITE_SIZE counter summary when
                  present.
  c4_other_weights — the same 1008 px encoder with Q8_0 and F16 linear
                  weights (the other two weight types of the workload), ms
                  per frame.
  attention_fp16 — the ViT attention at F16 precision (fp16 operands, fp32
                  accumulation): 16 heads of 64 over 9 windows of 576 tokens
                  and over the 5184-token global grid, µs per call, TFLOP/s
                  and the fraction of the fp16 dense peak.
  small_m       — weight streaming at M = 64 rows (the C2 small-M shapes):
                  fc1 and fc2 alone, and all four ViT linears of 64 distinct
                  layers in one batched launch, as algorithmic GB/s against
                  the 8 TB/s HBM peak.
  sam2_encoders — the SAM 2.1 Hiera encoders (backbone + FPN to 256-ch
                  levels at 256², 128², 64²) at 1024×1024 on the same kind of
                  input: Hiera-Tiny with F16 weights and Hiera-Base+ with
                  Q8_0 weights, ms per frame.
  preprocess    — sam3_encode_image's preprocessing on the device for a
                  1920×1080 camera frame (resize to 1008² + normalisation):
                  kernel time, the frame's host→device copy, and the whole
                  s3e_encode_image_u8 call against the resident encode.
  cpu_baseline  — the CPU oracle (a C restatement of ggml's CPU path, not
                  the upstream binary) on this host: one whole frame of the
                  same model and image, backbone and neck, on every core the
                  job may use (OMP_NUM_THREADS where the host sets the job's
                  CPU share, else all cores the process can run on; about
                  11 s on 16 threads).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sam3.cpp_amd"))

METRIC = "image-encoder ms/frame (SAM3 ViT 1008², q4_0/q8_0/f16) + % MFMA/HBM peak"
PEAK_TOPS = {"q4_0": 5000.0, "q4_1": 5000.0, "q8_0": 5000.0, "f16": 2500.0, "f32": 157.3}
CFG = dict(img_size=1008, patch=14, embed_dim=1024, depth=32, heads=16, mlp_ratio_x1000=4625, window=24,
           global_idx=(7, 15, 23, 31))
# the measured_peaks entry the fc1 kernel's roofline is also read against
MEASURED_PEAK = {"q4_0": "mfma_i8_32x32x32_TOPS", "q4_1": "mfma_i8_32x32x32_TOPS", "q8_0": "mfma_i8_32x32x32_TOPS",
                 "f16": "mfma_f16_32x32x16_TOPS"}
GEMM_KERNEL = {"q4_0": "k_gemm_f6", "q4_1": "k_gemm", "q8_0": "k_gemm", "f16": "k_gemm", "f32": "k_gemm"}
SAM2_RUNS = [("hiera_t", "f16"), ("hiera_b+", "q8_0")]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def synthetic_image(size: int, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.integers(0, 256, (size, size, 3), dtype=np.uint8)


def preprocess(img: np.ndarray) -> np.ndarray:
    """sam3_preprocess_image for an image already at img_size (sam3.cpp:3486-3514):
    (v/255 − 0.5)/0.5 in float32, HWC → CHW."""
    v = img.astype(np.float32) / np.float32(255.0)
    v = (v - np.float32(0.5)) / np.float32(0.5)
    return np.ascontiguousarray(v.transpose(2, 0, 1))


def read_traffic(path: str):
    """Bytes per launch from a counter summary line 'traffic_bytes_per_launch: N'."""
    try:
        with open(path) as f:
            for line in f:
                m = re.match(r"\s*traffic_bytes_per_launch:\s*([0-9.eE+]+)", line)
                if m:
                    return float(m.group(1))
    except OSError:
        pass
    return None


def gemm_roofline(s3e, ctx, ev, ftype: str, reps: int, shape=(5184, 4736, 1024)):
    """Time one GEMM kernel alone (default: fc1) on pre-converted activations:
    for Q4_0 the fp6 kernel the encoder runs (s3e_mul_mat_q_f6 on
    S3E_TYPE_Q8_0_F6X2), otherwise s3e_mul_mat_q."""
    M, N, K = shape
    rng = np.random.default_rng(1)
    tmap = {"q4_0": s3e.TYPE_Q4_0, "q4_1": s3e.TYPE_Q4_1, "q8_0": s3e.TYPE_Q8_0, "f16": s3e.TYPE_F16,
            "f32": s3e.TYPE_F32}
    wt = tmap[ftype]
    w = ctx.weight(wt, K, N, _random_ggml_bytes(wt, N, K, rng))
    X = rng.standard_normal((M, K)).astype(np.float32)
    Xd = ctx.to_device(X)
    Y = ctx.buffer(M * N * 4)
    run = None
    if wt == s3e.TYPE_Q4_0:
        ns = s3e.act_scale_elems(M, K)
        qs, d = ctx.buffer((M + 63) // 64 * 64 * K * 3 // 2), ctx.buffer(ns * 2)
        ctx.quantize_rows(s3e.TYPE_Q8_0_F6X2, Xd, M, K, qs, d, None)
        run = lambda: ctx.mul_mat_q_f6(w, qs, d, M, Y)
    elif wt in (s3e.TYPE_Q8_0, s3e.TYPE_Q4_1):
        vdt = s3e.TYPE_Q8_1 if wt == s3e.TYPE_Q4_1 else s3e.TYPE_Q8_0
        ns = s3e.act_scale_elems(M, K)
        qs, d, s = ctx.buffer(M * K), ctx.buffer(ns * 2), ctx.buffer(ns * 2)
        ctx.quantize_rows(vdt, Xd, M, K, qs, d, s)
        args = (qs, d, s)
    elif wt == s3e.TYPE_F16:
        qs = ctx.buffer(M * K * 2)
        ctx.quantize_rows(s3e.TYPE_F16, Xd, M, K, qs, None, None)
        args = (qs, None, None)
    else:
        args = (Xd, None, None)
    if run is None:
        run = lambda: ctx.mul_mat_q(w, *args, M, Y)
    for _ in range(3):
        run()
    ctx.sync()
    e0, e1 = ev.create(), ev.create()
    ev.record(e0, ctx.stream)
    for _ in range(reps):
        run()
    ev.record(e1, ctx.stream)
    ms = ev.elapsed_ms(e0, e1) / reps
    ctx.sync()
    ops = 2.0 * M * N * K
    tops = ops / (ms * 1e-3) / 1e12
    return ms, tops, ops


def vendor_gemms(reps: int = 50) -> dict:
    """A yardstick, not the engine: the ViT's GEMM shapes on the vendor
    library through torch (hipBLASLt), fp16 × fp16 (F.linear, weight [N][K])
    and plain int8 × int8 → int32 (torch._int_mm: no per-block scales, so
    less work than a Q4_0 × Q8_0 product), µs per call over `reps` calls."""
    import torch
    import torch.nn.functional as F

    dev = "cuda:0"
    res = {}

    def timeit(f):
        for _ in range(5):
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            f()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3

    g = torch.Generator(device=dev).manual_seed(0)
    for name, M, N, K in (("fc1", 5184, 4736, 1024), ("qkv", 5184, 3072, 1024), ("fc2", 5184, 1024, 4736),
                          ("proj", 5184, 1024, 1024)):
        a = torch.randn(M, K, device=dev, dtype=torch.float16, generator=g)
        w = torch.randn(N, K, device=dev, dtype=torch.float16, generator=g)
        ai = torch.randint(-127, 128, (M, K), device=dev, dtype=torch.int8, generator=g)
        wi = torch.randint(-8, 8, (N, K), device=dev, dtype=torch.int8, generator=g)
        ops = 2.0 * M * N * K
        us16 = timeit(lambda: F.linear(a, w))
        us8 = timeit(lambda: torch._int_mm(ai, wi.t()))
        res[name] = {"M": M, "N": N, "K": K, "fp16_us": round(us16, 1), "fp16_TFLOPs": round(ops / us16 / 1e6, 1),
                     "int8_us": round(us8, 1), "int8_TOPS": round(ops / us8 / 1e6, 1)}
        log(f"vendor {name} M={M} N={N} K={K}: fp16 {us16:.1f} us ({ops / us16 / 1e6:.0f} TFLOP/s), "
            f"int8 {us8:.1f} us ({ops / us8 / 1e6:.0f} TOPS)")
    return res


BPW = {"q4_0": 18 / 32, "q4_1": 20 / 32, "q8_0": 34 / 32, "f16": 2.0}
VIT_LINEARS = [(3072, 1024), (1024, 1024), (4736, 1024), (1024, 4736)]  # qkv, proj, fc1, fc2 (N, K)


def small_m(s3e, ctx, ev, ftype: str, reps: int = 10, hbm_read: float | None = None) -> dict:
    """Weight streaming at M = 64 rows: fc1 and fc2 alone (s3e_mul_mat_q), and
    the four ViT linears of enough distinct layers for ≈ 500 MB of weights in
    one batched launch (s3e_mul_mat_q_batch; 64 layers of Q4_0), twice the
    256 MB Infinity Cache, so every run streams from HBM.  Algorithmic bytes
    per product N·K·bpw + 4·M·K + 4·M·N (ggml bytes per weight, f32 in and
    out)."""
    M = 64
    per_layer = sum(N * K for N, K in VIT_LINEARS) * BPW[ftype]
    layers = max(8, int(round(500e6 / per_layer)))
    tmap = {"q4_0": s3e.TYPE_Q4_0, "q4_1": s3e.TYPE_Q4_1, "q8_0": s3e.TYPE_Q8_0, "f16": s3e.TYPE_F16}
    wt = tmap[ftype]
    vdt = s3e.TYPE_F16 if wt == s3e.TYPE_F16 else (s3e.TYPE_Q8_1 if wt == s3e.TYPE_Q4_1 else s3e.TYPE_Q8_0)
    rng = np.random.default_rng(2)
    acts = {}
    for K in (1024, 4736):
        Xd = ctx.to_device(rng.standard_normal((M, K)).astype(np.float32))
        ns = s3e.act_scale_elems(M, K)
        q, d, sx = ctx.buffer(M * K * 2), ctx.buffer(ns * 2), ctx.buffer(ns * 2)
        ctx.quantize_rows(vdt, Xd, M, K, q, None if wt == s3e.TYPE_F16 else d, None if wt == s3e.TYPE_F16 else sx)
        acts[K] = (q, None if wt == s3e.TYPE_F16 else d, sx if wt == s3e.TYPE_Q4_1 else None)

    def nbytes(N, K):
        return N * K * BPW[ftype] + 4 * M * K + 4 * M * N

    res = {"rows": M, "weights": ftype}
    e0, e1 = ev.create(), ev.create()
    for name, (N, K) in (("fc1", VIT_LINEARS[2]), ("fc2", VIT_LINEARS[3])):
        w = ctx.weight(wt, K, N, _random_ggml_bytes(wt, N, K, rng))
        Y = ctx.buffer(M * N * 4)
        for _ in range(3):
            ctx.mul_mat_q(w, *acts[K], M, Y)
        ctx.sync()
        ev.record(e0, ctx.stream)
        for _ in range(50):
            ctx.mul_mat_q(w, *acts[K], M, Y)
        ev.record(e1, ctx.stream)
        us = ev.elapsed_ms(e0, e1) / 50 * 1e3
        ctx.sync()
        res[f"{name}_us"] = round(us, 2)
        res[f"{name}_GBps"] = round(nbytes(N, K) / (us * 1e-6) / 1e9, 1)
        w.free()
    ws, xs, ds, ss, ys = [], [], [], [], []
    total = 0.0
    for _ in range(layers):
        for N, K in VIT_LINEARS:
            ws.append(ctx.weight(wt, K, N, _random_ggml_bytes(wt, N, K, rng)))
            q, d, sx = acts[K]
            xs.append(q)
            ds.append(d)
            ss.append(sx)
            ys.append(ctx.buffer(M * N * 4))
            total += nbytes(N, K)
    for _ in range(2):
        ctx.mul_mat_q_batch(ws, xs, ds, ss, M, None, ys)
    ctx.sync()
    ev.record(e0, ctx.stream)
    for _ in range(reps):
        ctx.mul_mat_q_batch(ws, xs, ds, ss, M, None, ys)
    ev.record(e1, ctx.stream)
    us = ev.elapsed_ms(e0, e1) / reps * 1e3
    ctx.sync()
    gbps = total / (us * 1e-6) / 1e9
    res["sweep"] = {"products": len(ws), "layers": layers, "bytes": int(total), "us": round(us, 1),
                    "GBps": round(gbps, 1), "frac_hbm": round(gbps / 8000.0, 4)}
    if hbm_read:
        res["sweep"]["frac_measured_read"] = round(gbps / hbm_read, 4)
    for w in ws:
        w.free()
    log(f"small-M {ftype}: fc1 {res['fc1_us']} us ({res['fc1_GBps']} GB/s), fc2 {res['fc2_us']} us "
        f"({res['fc2_GBps']} GB/s); {len(ws)}-product sweep {total / 1e6:.0f} MB in {us:.1f} us = {gbps:.0f} GB/s")
    return res


def axial_rope(dim: int, side: int) -> np.ndarray:
    """Axial RoPE table [side²][dim/2][2] (cos, sin) of sam3_compute_axial_cis
    (sam3.cpp:3555-3586), theta 10000, scale 1: synthetic tracker input."""
    q = dim // 4
    freqs = (1.0 / np.power(np.float32(10000.0), np.arange(q, dtype=np.float32) * 4 / np.float32(dim))).astype(np.float32)
    idx = np.arange(side * side)
    tx = (idx % side).astype(np.float32)[:, None] * freqs[None]
    ty = (idx // side).astype(np.float32)[:, None] * freqs[None]
    ang = np.concatenate([tx, ty], axis=1)
    return np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)


def sam2_encoders(s3e, ctx, ev, steps: int, warmup: int, runs=SAM2_RUNS) -> dict:
    """ms/frame of the SAM 2.1 Hiera encoders at 1024² (input resident in HBM);
    for Hiera-B+ also the C5 tracking frame: the encoder, then the 4-layer
    memory attention of its 64×64 level against 7 memory frames of 4096
    tokens (MD 64, N(0,1)) plus 16 object pointers (64 tokens), timed over
    consecutive frames."""
    res = {}
    tmpdir = os.environ.get("TMPDIR", tempfile.gettempdir())
    for variant, ft in runs:
        path = os.path.join(tmpdir, f"s3e_bench_{variant}_{ft}.ggml")
        c5 = variant == "hiera_b+"
        s3e.synth_write_sam2(path, variant, img_size=1024, ftype=ft, seed=0, std=0.02,
                             mem_attn_layers=4 if c5 else 0)
        model = s3e.Model(ctx, path)
        st = s3e.State(ctx, model)
        img = synthetic_image(1024)
        mean = np.array([0.485, 0.456, 0.406], np.float32)[:, None, None]
        std = np.array([0.229, 0.224, 0.225], np.float32)[:, None, None]
        chw = ((img.astype(np.float32) / np.float32(255)).transpose(2, 0, 1) - mean) / std
        chw_d = ctx.to_device(np.ascontiguousarray(chw, np.float32))
        for _ in range(warmup):
            st.encode_chw(chw_d)
        ctx.sync()
        e0, e1 = ev.create(), ev.create()
        ev.record(e0, ctx.stream)
        for _ in range(steps):
            st.encode_chw(chw_d)
        ev.record(e1, ctx.stream)
        ms = ev.elapsed_ms(e0, e1) / steps
        ctx.sync()
        name = f"{variant.replace('+', 'plus')}_{ft}_1024_ms"
        res[name] = round(ms, 3)
        log(f"{variant} {ft} 1024: {ms:.3f} ms/frame")
        if c5:
            rng = np.random.default_rng(5)
            H, D, MD, frames, ptr = 64, 256, 64, 7, 64
            N, M = H * H, frames * H * H + ptr
            curr = st.device_view("neck_trk_2")
            pos = st.device_view("neck_trk_pe_2")
            prompt = ctx.to_device(rng.standard_normal((M, MD)).astype(np.float32))
            ppos = ctx.to_device((rng.standard_normal((M, MD)) * 0.1).astype(np.float32))
            rq = axial_rope(D, H)
            rope_q, rope_k = ctx.to_device(rq), ctx.to_device(np.concatenate([rq] * frames))
            out = ctx.buffer(N * D * 4)

            def frame(with_encoder=True):
                if with_encoder:
                    st.encode_chw(chw_d)
                st.mem_attn(curr, pos, N, prompt, ppos, M, ptr, rope_q, rope_k, out)

            for _ in range(2):
                frame()
            ctx.sync()
            ev.record(e0, ctx.stream)
            for _ in range(5):
                frame()
            ev.record(e1, ctx.stream)
            fms = ev.elapsed_ms(e0, e1) / 5
            ctx.sync()
            ev.record(e0, ctx.stream)
            for _ in range(5):
                frame(False)
            ev.record(e1, ctx.stream)
            mms = ev.elapsed_ms(e0, e1) / 5
            ctx.sync()
            res["c5_frame_ms"] = round(fms, 3)
            res["c5_mem_attn_ms"] = round(mms, 3)
            log(f"C5 tracking frame (Hiera-B+ {ft} encoder + memory attention 4096 x 28736): {fms:.3f} ms/frame, "
                f"memory attention {mms:.3f} ms")
        st.free()
        model.free()
        try:
            os.remove(path)
        except OSError:
            pass
    return res


def _random_ggml_bytes(wt: int, N: int, K: int, rng) -> np.ndarray:
    """Valid ggml bytes for an N×K weight of type wt with random contents
    (timing only): random quant bytes, fp16 scales 0.002, Q4_1 minima −0.015."""
    if wt == 0:
        return rng.normal(0, 0.02, (N, K)).astype(np.float32).view(np.uint8).ravel()
    if wt == 1:
        return rng.normal(0, 0.02, (N, K)).astype(np.float16).view(np.uint8).ravel()
    bs = {2: 18, 3: 20, 8: 34}[wt]
    out = rng.integers(0, 256, (N, K // 32, bs), dtype=np.uint8)
    out[:, :, 0:2] = np.full((N, K // 32), 0.002, np.float16).view(np.uint8).reshape(N, K // 32, 2)
    if wt == 3:
        out[:, :, 2:4] = np.full((N, K // 32), -0.015, np.float16).view(np.uint8).reshape(N, K // 32, 2)
    return out.ravel()


CAMERA = (1920, 1080)  # a camera frame for the preprocessing leg


def preprocess_leg(s3e, ctx, ev, st, S: int, encode_ms: float, reps: int = 20) -> dict:
    """sam3_encode_image's preprocessing on the device (s3e_preprocess_image:
    uint8 bilinear resize of a 1920×1080 frame to S² + normalisation into
    CHW f32): kernel time with HIP events, algorithmic bytes w·h·3 read +
    12·S² written (the kernel reads each source pixel about once at this
    ratio); the pageable host→device copy of the frame; and the whole
    s3e_encode_image_u8 call (copy + preprocessing + encode + sync) by the
    host clock, against the resident-input encode."""
    w, h = CAMERA
    img = np.random.default_rng(1).integers(0, 256, (h, w, 3), dtype=np.uint8)
    src = ctx.to_device(img)
    chw = ctx.buffer(3 * S * S * 4)
    for _ in range(3):
        ctx.preprocess_image(src, w, h, S, s3e.NORM_SAM3, chw)
    ctx.sync()
    e0, e1 = ev.create(), ev.create()
    ev.record(e0, ctx.stream)
    for _ in range(reps):
        ctx.preprocess_image(src, w, h, S, s3e.NORM_SAM3, chw)
    ev.record(e1, ctx.stream)
    us = ev.elapsed_ms(e0, e1) / reps * 1e3
    ctx.sync()
    nbytes = w * h * 3 + 12 * S * S
    t0 = time.perf_counter()
    for _ in range(reps):
        src.upload(img)
    ctx.sync()
    up_ms = (time.perf_counter() - t0) / reps * 1e3
    st.encode_image_u8(img)
    t0 = time.perf_counter()
    for _ in range(5):
        st.encode_image_u8(img)
    e2e_ms = (time.perf_counter() - t0) / 5 * 1e3
    res = {"input": f"{w}x{h} uint8 RGB -> {S}x{S}", "kernel_us": round(us, 2),
           "kernel_GBps": round(nbytes / (us * 1e-6) / 1e9, 1), "upload_ms": round(up_ms, 3),
           "encode_image_u8_ms": round(e2e_ms, 3), "encode_resident_ms": round(encode_ms, 3)}
    log(f"preprocess {w}x{h} -> {S}: kernel {us:.1f} us ({res['kernel_GBps']} GB/s), upload {up_ms:.2f} ms, "
        f"s3e_encode_image_u8 {e2e_ms:.2f} ms/frame vs {encode_ms:.2f} resident")
    return res


def encode_ms(s3e, ctx, ev, ftype: str, steps: int, warmup: int, neck: int = 1) -> float:
    """ms/frame of the full 1008 px encoder (backbone + tracker neck; with
    neck=2 the full SAM 3 file's backbone + detector and tracker necks) with
    the ViT's linear weights in `ftype`, input resident in HBM."""
    tmpdir = os.environ.get("TMPDIR", tempfile.gettempdir())
    path = os.path.join(tmpdir, f"s3e_bench_sam3_vit_{ftype}_n{neck}.ggml")
    s3e.synth_write(path, ftype=ftype, seed=0, std=0.02, neck=neck, **CFG)
    model = s3e.Model(ctx, path)
    st = s3e.State(ctx, model)
    chw_d = ctx.to_device(preprocess(synthetic_image(CFG["img_size"])))
    for _ in range(warmup):
        st.encode_chw(chw_d)
    ctx.sync()
    e0, e1 = ev.create(), ev.create()
    ev.record(e0, ctx.stream)
    for _ in range(steps):
        st.encode_chw(chw_d)
    ev.record(e1, ctx.stream)
    ms = ev.elapsed_ms(e0, e1) / steps
    ctx.sync()
    st.free()
    model.free()
    try:
        os.remove(path)
    except OSError:
        pass
    log(f"encode {ftype} ({neck} neck{'s' if neck > 1 else ''}): {ms:.3f} ms/frame over {steps} steps")
    return ms


MFMA_FORMS = [("i8_32x32x32", 0, 65536), ("f16_32x32x16", 1, 32768), ("fp6_scaled_32x32x64", 2, 131072),
              ("f16_32x32x8", 3, 16384)]


def measured_peaks(s3e, ctx, ev, reps: int = 5) -> dict:
    """What this GPU reaches (s3e_probe_stream / s3e_probe_mfma): HBM read,
    copy and write rates over buffers far larger than the 256 MB Infinity
    Cache, and each MFMA form's issue rate with eight independent chains per
    wave and no memory traffic."""
    res = {}
    e0, e1 = ev.create(), ev.create()
    nbytes = 4 << 30
    a, b = ctx.buffer(nbytes), ctx.buffer(nbytes // 2)
    for name, mode, nb, moved in (("read", 0, nbytes, nbytes), ("write", 2, nbytes, nbytes),
                                  ("copy", 1, nbytes // 2, nbytes)):
        src, dst = (a, None) if mode == 0 else ((None, a) if mode == 2 else (a, b))
        ctx.probe_stream(mode, dst, src, nb)
        ctx.sync()
        ev.record(e0, ctx.stream)
        for _ in range(reps):
            ctx.probe_stream(mode, dst, src, nb)
        ev.record(e1, ctx.stream)
        ms = ev.elapsed_ms(e0, e1) / reps
        res[f"hbm_{name}_GBps"] = round(moved / ms / 1e6, 1)
        log(f"HBM {name}: {moved / 2**30:.0f} GiB moved in {ms:.3f} ms = {moved / ms / 1e6:.1f} GB/s")
    a.free()
    b.free()
    cus = ctx_cus()
    for name, kind, ops in MFMA_FORMS:
        wps, iters = 2, 4096
        ctx.probe_mfma(kind, 64, wps)
        ctx.sync()
        ev.record(e0, ctx.stream)
        ctx.probe_mfma(kind, iters, wps)
        ev.record(e1, ctx.stream)
        ms = ev.elapsed_ms(e0, e1)
        n = cus * 4 * wps * iters * 8
        tops = n * ops / (ms * 1e-3) / 1e12
        res[f"mfma_{name}_TOPS"] = round(tops, 1)
        log(f"MFMA {name}: {tops:.1f} T(FL)OP/s ({n} instructions in {ms:.3f} ms)")
    ctx.sync()
    return res


def ctx_cus() -> int:
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    v = ctypes.c_int()
    hip.hipDeviceGetAttribute(ctypes.byref(v), 63, 0)  # hipDeviceAttributeMultiprocessorCount
    return v.value


ATTN_SHAPES = [("windowed", 9, 576), ("global", 1, 5184)]  # (name, windows B, tokens N); 16 heads, head dim 64


def attention_fp16(s3e, ctx, ev, reps: int = 20) -> dict:
    """The ViT's attention at F16 precision (ggml_flash_attn_ext with F16
    operands; fp16 probabilities, fp32 accumulation): 16 heads of 64 over 9
    windows of 576 tokens and over the 5184-token global grid, through
    s3e_flash_attn_ext_f16 with fp16 Q, K, V resident in ggml's contiguous
    [B][heads][N][64] layout.  Calls run back to back on the stream; each is
    the attention kernel alone (Q, K and V read where they lie), with no
    allocation or synchronisation.  FLOPs 4·B·heads·N²·64 (QKᵀ and PV), against the
    2.5 PFLOP/s dense fp16 peak."""
    res = {}
    rng = np.random.default_rng(7)
    nh, D = 16, 64
    e0, e1 = ev.create(), ev.create()
    for name, B, N in ATTN_SHAPES:
        h16 = lambda: ctx.to_device(rng.standard_normal((B, nh, N, D)).astype(np.float16).view(np.uint16))
        q, k, v = h16(), h16(), h16()
        o = ctx.buffer(B * N * nh * D * 4)
        nb = (1, D, N * D, nh * N * D)
        run = lambda: ctx.flash_attn_ext_f16(q, nb, k, nb, v, nb, D, N, N, nh, B, 0.125, o)
        for _ in range(3):
            run()
        ctx.sync()
        ev.record(e0, ctx.stream)
        for _ in range(reps):
            run()
        ev.record(e1, ctx.stream)
        us = ev.elapsed_ms(e0, e1) / reps * 1e3
        ctx.sync()
        flops = 4.0 * B * nh * N * N * D
        tf = flops / (us * 1e-6) / 1e12
        res[name] = {"windows": B, "tokens": N, "heads": nh, "us": round(us, 1), "TFLOPs": round(tf, 1),
                     "frac_fp16_peak": round(tf / 2500.0, 4),
                     "scope": "s3e_flash_attn_ext_f16 calls back to back, fp16 operands resident and read in "
                              "place: the attention kernel alone"}
        log(f"attention fp16 {name} {B}x{nh}x{N}: {us:.1f} us, {tf:.1f} TFLOP/s")
        for b in (q, k, v, o):
            b.free()
    return res


def cpu_preprocess_ms(S: int, reps: int = 3) -> float:
    """The oracle's single-threaded sam3_resize_bilinear + sam3_preprocess_image
    (the reference's host loop) on the same 1920×1080 frame."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as orc

    w, h = CAMERA
    img = np.random.default_rng(1).integers(0, 256, (h, w, 3), dtype=np.uint8)
    orc.preprocess_sam3(img, S)
    t0 = time.perf_counter()
    for _ in range(reps):
        orc.preprocess_sam3(img, S)
    return (time.perf_counter() - t0) / reps * 1e3


def cpu_baseline(path: str, img: np.ndarray, threads: int):
    """Oracle on the host: one whole frame (prefix + 32 blocks + tracker neck)
    of the same model and image, after the host preprocessing."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as orc

    om = orc.OracleModel(path)
    chw = orc.preprocess_sam3(img, om.img)
    t0 = time.perf_counter()
    x = om.encode(chw, threads)
    om.neck(x, "trk", threads)
    return (time.perf_counter() - t0) * 1e3


def _short_kernel(name: str) -> str:
    if name.startswith("_Z"):
        # Left mangled by the profiler (it does not demangle _Float16
        # parameters): take the length-prefixed source name k_....
        for m in re.finditer(r"(\d+)(?=k_)", name):
            digits, at = m.group(1), m.end()
            for i in range(len(digits)):
                n = int(digits[i:])
                if name[at + n:at + n + 1] in ("E", "I"):
                    return name[at:at + n]
    m = re.search(r"(k_\w+(<[^>]*>)?)", name)
    return m.group(1) if m else name.split("(")[0][:60]


def summarize_stats(stats_csv: str, frames: int) -> str:
    """Per-kernel table from a rocprofv3 --stats kernel_stats.csv."""
    import csv

    rows = list(csv.DictReader(open(stats_csv)))
    lines = [f"{'kernel':34s} {'calls':>7s} {'avg_us':>9s} {'ms/frame':>9s} {'share':>7s}"]
    for r in rows:
        tot = float(r["TotalDurationNs"]) / 1e6
        lines.append(f"{_short_kernel(r['Name']):34s} {int(r['Calls']):7d} {float(r['AverageNs']) / 1e3:9.1f} "
                     f"{tot / frames:9.3f} {float(r['Percentage']):6.2f}%")
    return "\n".join(lines)


def summarize_trace(trace_csv: str, marker: str, first: int, last: int, frames: int) -> str:
    """Per-kernel table over a window of a rocprofv3 kernel_trace.csv: the
    launches from the `first`-th launch of kernel `marker` (0-based) up to
    before its `last`-th, e.g. the encoder-only frames of a run that also
    times other work."""
    import collections
    import csv

    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    seen, agg = -1, collections.defaultdict(list)
    for r in rows:
        k = _short_kernel(r["Kernel_Name"])
        seen += k == marker
        if first <= seen < last:
            agg[k].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    tot = sum(sum(v) for v in agg.values())
    lines = [f"{'kernel':34s} {'calls':>7s} {'avg_us':>9s} {'ms/frame':>9s} {'share':>7s}"]
    for k, v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"{k:34s} {len(v):7d} {sum(v) / len(v):9.1f} {sum(v) / 1e3 / frames:9.3f} "
                     f"{100 * sum(v) / tot:6.2f}%")
    return "\n".join(lines)


def summarize_grids(trace_csv: str, frames: int) -> str:
    """Per (kernel, grid) table from a rocprofv3 kernel_trace.csv: separates
    launches of one kernel at different shapes (e.g. windowed and global
    attention)."""
    import collections
    import csv

    agg = collections.defaultdict(list)
    for r in csv.DictReader(open(trace_csv)):
        key = (_short_kernel(r["Kernel_Name"]), f"{r['Grid_Size_X']}x{r['Grid_Size_Y']}x{r['Grid_Size_Z']}")
        agg[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    lines = [f"{'kernel':34s} {'grid (threads)':>18s} {'calls':>6s} {'avg_us':>9s} {'ms/frame':>9s}"]
    for (k, g), v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"{k:34s} {g:>18s} {len(v):6d} {sum(v) / len(v):9.1f} {sum(v) / 1e3 / frames:9.3f}")
    return "\n".join(lines)


def summarize_pmc(csvs: list, kernels: list) -> str:
    """Per-kernel averages per dispatch of rocprofv3 --pmc counter CSVs, and
    the derived utilisation: kernel cycles = GRBM_GUI_ACTIVE / 8 (the counter
    sums the 8 XCDs); MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (kernel cycles ×
    1024 SIMDs); VALU issue = SQ_INSTS_VALU × 4 cycles (a wave64 VALU
    instruction occupies a SIMD 4 cycles) / (kernel cycles × 1024)."""
    import collections
    import csv

    agg = collections.defaultdict(lambda: collections.defaultdict(float))
    disp = collections.defaultdict(lambda: collections.defaultdict(set))
    for path in csvs:
        for r in csv.DictReader(open(path)):
            k = _short_kernel(r["Kernel_Name"])
            agg[k][r["Counter_Name"]] += float(r["Counter_Value"])
            disp[k][r["Counter_Name"]].add(r["Dispatch_Id"])
    out = []
    for k in kernels:
        if k not in agg:
            continue
        c = {n: v / len(disp[k][n]) for n, v in agg[k].items()}
        out.append(f"{k}  ({max(len(x) for x in disp[k].values())} dispatches)")
        for n in sorted(c):
            out.append(f"    {n:34s} {c[n]:14.4g}")
        cyc = c.get("GRBM_GUI_ACTIVE", 0) / 8
        if cyc:
            if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
                out.append(f"    {'-> MFMA busy':34s} {c['SQ_VALU_MFMA_BUSY_CYCLES'] / (cyc * 1024):14.3f}")
            if "SQ_INSTS_VALU" in c:
                out.append(f"    {'-> VALU issue':34s} {4 * c['SQ_INSTS_VALU'] / (cyc * 1024):14.3f}")
    return "\n".join(out)


def summarize_counters(fetch_csv: str, write_csv: str, cfetch_csv: str, cwrite_csv: str, copy_bytes: int,
                       kernel: str) -> str:
    """HBM bytes per launch of `kernel` from FETCH_SIZE / WRITE_SIZE (KiB per
    dispatch), each scaled by what the same counter reads for the copy kernel
    of known size."""
    import csv
    import statistics

    def med(path, name):
        vals = [float(r["Counter_Value"]) for r in csv.DictReader(open(path)) if _short_kernel(r["Kernel_Name"]) == name]
        return statistics.median(vals), len(vals)

    f, nf = med(fetch_csv, kernel)
    w, nw = med(write_csv, kernel)
    cf, _ = med(cfetch_csv, "k_copy")
    cw, _ = med(cwrite_csv, "k_copy")
    sf = copy_bytes / (cf * 1024.0)
    sw = copy_bytes / (cw * 1024.0)
    traffic = f * 1024.0 * sf + w * 1024.0 * sw
    return "\n".join([
        f"kernel: {kernel} ({nf} / {nw} dispatches)",
        f"FETCH_SIZE median: {f:.1f} KiB/dispatch  x fetch scale {sf:.3f}  = {f * 1024 * sf / 1e6:.2f} MB",
        f"WRITE_SIZE median: {w:.1f} KiB/dispatch  x write scale {sw:.3f}  = {w * 1024 * sw / 1e6:.2f} MB",
        f"copy calibration: k_copy of {copy_bytes} bytes reads FETCH_SIZE {cf:.1f} KiB, WRITE_SIZE {cw:.1f} KiB",
        f"traffic_bytes_per_launch: {traffic:.0f}",
    ])


def main() -> int:
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-stats":
        print(summarize_stats(sys.argv[2], int(sys.argv[3])))
        return 0
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-trace":
        a = sys.argv[2:]
        print(summarize_trace(a[0], a[1], int(a[2]), int(a[3]), int(a[4])))
        return 0
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-grids":
        print(summarize_grids(sys.argv[2], int(sys.argv[3])))
        return 0
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-pmc":
        # --summarize-pmc a.csv [b.csv ...] -- kernel [kernel ...]
        a = sys.argv[2:]
        i = a.index("--")
        print(summarize_pmc(a[:i], a[i + 1:]))
        return 0
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-counters":
        a = sys.argv[2:]
        print(summarize_counters(a[0], a[1], a[2], a[3], int(a[4]), a[5]))
        return 0
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--ftype", default="q4_0", choices=sorted(PEAK_TOPS))
    ap.add_argument("--gemm-reps", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "gemm_fc1_q4_0_counters.txt"))
    ap.add_argument("--only", choices=["encode", "gemm", "copy", "neck", "preprocess", "sam2", "small_m", "c4",
                                       "attn", "peaks", "vendor"], default=None,
                    help="run one leg only (for profiling runs)")
    ap.add_argument("--sam2-run", default=None, help="with --only sam2: one encoder, e.g. hiera_t:f16")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the encoder shards by "
              f"frame: one process per GPU, whole frames dealt round-robin, no collective)", file=sys.stderr)
        return 2
    import s3e

    ctx = s3e.Context(0)
    ev = s3e.HipEvents()
    out = {}

    if args.only == "copy":
        nbytes = 1 << 30
        a, b = ctx.buffer(nbytes), ctx.buffer(nbytes)
        for _ in range(5):
            ctx.copy(b, a, nbytes)
        ctx.sync()
        e0, e1 = ev.create(), ev.create()
        ev.record(e0, ctx.stream)
        for _ in range(10):
            ctx.copy(b, a, nbytes)
        ev.record(e1, ctx.stream)
        ms = ev.elapsed_ms(e0, e1) / 10
        log(f"copy 1 GiB: {ms:.3f} ms = {2 * nbytes / ms / 1e6:.1f} GB/s (read+write)")
        return 0

    if args.only == "attn":
        attention_fp16(s3e, ctx, ev)
        return 0

    if args.only == "peaks":
        measured_peaks(s3e, ctx, ev)
        return 0

    if args.only == "vendor":
        # the vendor library's fp16 and plain int8 GEMMs, then this engine's fc1
        # for each weight type, on the same box
        vendor_gemms()
        for name, shape in (("fc1", (5184, 4736, 1024)), ("qkv", (5184, 3072, 1024)), ("fc2", (5184, 1024, 4736)),
                            ("proj", (5184, 1024, 1024))):
            for ft in ("q4_0", "q8_0", "f16"):
                ms, tops, _ = gemm_roofline(s3e, ctx, ev, ft, args.gemm_reps, shape)
                log(f"{name} GEMM {ft}: {ms * 1e3:.1f} us/launch, {tops:.1f} TOPS")
        return 0

    if args.only == "c4":
        for ft in ("q8_0", "f16"):
            encode_ms(s3e, ctx, ev, ft, args.steps, args.warmup)
        encode_ms(s3e, ctx, ev, "q4_0", args.steps, args.warmup, neck=2)
        return 0

    if args.only == "small_m":
        for ft in ("q4_0", "q8_0", "q4_1", "f16"):
            small_m(s3e, ctx, ev, ft)
        return 0

    if args.only == "sam2":
        runs = [tuple(args.sam2_run.split(":"))] if args.sam2_run else SAM2_RUNS
        sam2_encoders(s3e, ctx, ev, args.steps, args.warmup, runs)
        return 0

    if args.only is None:
        out["peaks"] = measured_peaks(s3e, ctx, ev)
    if args.only in (None, "gemm"):
        ms, tops, ops = gemm_roofline(s3e, ctx, ev, args.ftype, args.gemm_reps)
        log(f"fc1 GEMM {args.ftype}: {ms * 1e3:.1f} us/launch, {tops:.1f} TOPS")
        out["gemm"] = (ms, tops, ops)
        if args.only == "gemm":
            return 0

    tmpdir = os.environ.get("TMPDIR", tempfile.gettempdir())
    path = os.path.join(tmpdir, f"s3e_bench_sam3_vit_{args.ftype}.ggml")
    t = time.time()
    s3e.synth_write(path, ftype=args.ftype, seed=0, std=0.02, **CFG)
    log(f"synthetic model written in {time.time() - t:.1f}s: {path} ({os.path.getsize(path) / 1e6:.1f} MB)")
    model = s3e.Model(ctx, path)
    st = s3e.State(ctx, model)
    img = synthetic_image(CFG["img_size"])
    chw_d = ctx.to_device(preprocess(img))
    for _ in range(args.warmup):
        st.encode_chw(chw_d)
    ctx.sync()
    e0, e1 = ev.create(), ev.create()
    ctx.sync()
    ev.record(e0, ctx.stream)
    for _ in range(args.steps):
        st.encode_chw(chw_d)
    ev.record(e1, ctx.stream)
    total_ms = ev.elapsed_ms(e0, e1)
    ctx.sync()
    ms_frame = total_ms / args.steps
    log(f"encode: {ms_frame:.3f} ms/frame over {args.steps} steps")
    if args.only == "encode":
        return 0
    # the neck alone on the backbone output just computed
    xd = st.device_view("vit_output")
    for _ in range(2):
        st.run_neck(xd)
    ctx.sync()
    ev.record(e0, ctx.stream)
    for _ in range(args.steps):
        st.run_neck(xd)
    ev.record(e1, ctx.stream)
    neck_ms = ev.elapsed_ms(e0, e1) / args.steps
    ctx.sync()
    log(f"neck: {neck_ms:.3f} ms/frame")
    if args.only == "neck":
        return 0

    pre = preprocess_leg(s3e, ctx, ev, st, CFG["img_size"], ms_frame)
    if args.only == "preprocess":
        return 0
    c4 = {f"{ft}_ms": round(encode_ms(s3e, ctx, ev, ft, max(5, args.steps // 2), 2), 3)
          for ft in ("q4_0", "q8_0", "f16") if ft != args.ftype}
    full_ms = encode_ms(s3e, ctx, ev, args.ftype, max(5, args.steps // 2), 2, neck=2)
    full = {"ms_per_frame": round(full_ms, 3), "GFLOP": 5828.3,
            "TFLOPs": round(5828.3 / full_ms, 1),
            "workload": f"full SAM 3 file ({args.ftype.upper()} linear weights), 1008x1008: ViT backbone + "
                        "detector and tracker SimpleFPN necks (sam3.cpp:6072-6075), image resident"}
    attn = attention_fp16(s3e, ctx, ev)
    sam2 = sam2_encoders(s3e, ctx, ev, max(3, args.steps // 2), 2)
    peaks = out["peaks"]
    sm = small_m(s3e, ctx, ev, args.ftype, hbm_read=peaks["hbm_read_GBps"]) if args.ftype in BPW else None

    gms, gtops, gops = out["gemm"]
    peak = PEAK_TOPS[args.ftype]
    traffic = read_traffic(args.traffic) if args.ftype == "q4_0" else None
    cpu = None
    if not args.no_cpu_baseline:
        # all the cores this job may use: OMP_NUM_THREADS where the job's
        # host sets its CPU share, else every core the process can run on
        host_cores = len(os.sched_getaffinity(0))
        threads = args.cpu_threads or int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or host_cores
        cms = cpu_baseline(path, img, threads)
        log(f"cpu baseline: {cms / 1e3:.1f} s/frame, {threads} threads")
        pms = cpu_preprocess_ms(CFG["img_size"])
        log(f"cpu preprocessing of a {CAMERA[0]}x{CAMERA[1]} frame: {pms:.1f} ms, 1 thread")
        cpu = {"value": round(cms, 1), "unit": "ms/frame", "cores": threads, "host_cores_visible": host_cores,
               "kind": "port",
               "preprocess_ms": round(pms, 2),
               "sample": f"one full frame (prefix + 32 blocks + tracker neck) of the same {args.ftype.upper()} "
                         "model and image on the CPU oracle, a C restatement of ggml's CPU path (AVX2, "
                         "OpenMP), not the upstream binary; preprocess_ms: the oracle's single-threaded resize + "
                         "normalisation of a 1920x1080 frame to 1008x1008, the reference's host loop"}
    try:
        os.remove(path)
    except OSError:
        pass
    line = {
        "metric": METRIC,
        "value": round(ms_frame, 3),
        "unit": "ms/frame",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_frame, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"q4_0": "int8", "q4_1": "int8", "q8_0": "int8", "f16": "f16", "f32": "f32"}[args.ftype],
        "data": "synthetic: random-init weights N(0,0.02), uniform uint8 1008x1008 image, seed 0",
        "config": {"workload": f"SAM 3 visual-only image encoder, 1008x1008 (72x72 tokens): ViT backbone "
                               f"(32 blocks, {args.ftype.upper()} linear weights) + tracker SimpleFPN neck to "
                               f"256-ch features at 288/144/72/36, batch 1",
                   "img_size": 1008, "weights": args.ftype, "blocks": 32, "window": 24,
                   "global_blocks": [7, 15, 23, 31], "neck_levels": [288, 144, 72, 36]},
        "breakdown": {"neck_ms": round(neck_ms, 3), "backbone_ms": round(ms_frame - neck_ms, 3)},
        "c4_other_weights": c4,
        "full_sam3_two_necks": full,
        "attention_fp16": attn,
        "sam2_encoders": sam2,
        "small_m": sm,
        "preprocess": pre,
        "roofline": {"kernel": f"{GEMM_KERNEL[args.ftype]} fc1 M=5184 N=4736 K=1024 ({args.ftype})", "bound": "mfma",
                     "achieved": round(gtops, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(gtops / peak, 4), "traffic": traffic,
                     "us_per_launch": round(gms * 1e3, 2), "ops_per_launch": gops,
                     "peak_measured": peaks.get(MEASURED_PEAK.get(args.ftype, ""), None),
                     "frac_of_measured": (round(gtops / peaks[MEASURED_PEAK[args.ftype]], 4)
                                          if args.ftype in MEASURED_PEAK else None)},
        "measured_peaks": peaks,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
