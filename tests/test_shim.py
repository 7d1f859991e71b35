"""The sam3.h encoder API (include/sam3_encoder.h) on the engine.

CPU part: every declared function is exported by libs3e.so with the C++
signature of sam3.h, and the example program (sam3.cpp_amd/sam3_encode)
fails the way sam3_load_model does (nullptr + a message) for a missing file
and for a file that is not a SAM 3 model — both decided before any GPU call.

GPU part: the example encodes a PPM image through sam3_encode_image and
dumps state tensors in sam3_dump_state_tensor's format; the dumps must match
the oracle's backbone + tracker neck on the same image (end-to-end bound as
in tests/test_gpu_neck.py), and the preprocessed-input path
(sam3_encode_image_from_preprocessed) must give bit-identical dumps.
"""
import os
import re
import subprocess

import numpy as np
import pytest

import oracle_lib as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "sam3.cpp_amd", "sam3_encode")
LIB = os.path.join(ROOT, "sam3.cpp_amd", "libs3e.so")
HEADER = os.path.join(ROOT, "include", "sam3_encoder.h")


def declared():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"\b(sam3_\w+)\s*\(", src)) - {"operator"})


def test_header_functions_are_exported():
    out = subprocess.run(["nm", "-DC", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    names = declared()
    assert len(names) == 16, names
    for n in names:
        assert re.search(rf"\b{n}\(", out), n
    # the C++ signatures of sam3.h (demangled)
    assert "sam3_load_model(sam3_params const&)" in out
    assert "sam3_encode_image(sam3_state&, sam3_model const&, sam3_image const&)" in out
    assert "sam3_dump_state_tensor(sam3_state const&, std::__cxx11::basic_string" in out
    assert "sam3_state_deleter::operator()(sam3_state*) const" in out
    assert ("sam3_test_run_vit_block_stage(sam3_model const&, int, sam3_vit_block_stage, float const*, "
            "long const*, std::vector<float, std::allocator<float> >&, long*, int)") in out
    assert ("sam3_test_run_vit_prefix_stage(sam3_model const&, sam3_vit_prefix_stage, float const*, "
            "long const*, std::vector<float, std::allocator<float> >&, long*, int)") in out


def test_example_fails_like_sam3_load_model(tmp_path):
    r = subprocess.run([EXE, "-m", str(tmp_path / "missing.ggml"), "-i", "x.ppm", "-o", str(tmp_path)],
                       capture_output=True, text=True)
    assert r.returncode == 1 and "failed to open" in r.stderr
    bad = tmp_path / "other.ggml"
    bad.write_bytes(b"ggjt" + b"\0" * 64)
    r = subprocess.run([EXE, "-m", str(bad), "-i", "x.ppm", "-o", str(tmp_path)], capture_output=True, text=True)
    assert r.returncode == 1 and "not a SAM 3 or SAM 2 model file" in r.stderr
    r = subprocess.run([EXE], capture_output=True, text=True)
    assert r.returncode == 1 and "usage" in r.stderr


@pytest.fixture(scope="module")
def s3e_lib():
    import s3e

    return s3e


def _write_ppm(path, img):
    h, w, _ = img.shape
    with open(path, "wb") as f:
        f.write(f"P6\n# synthetic\n{w} {h}\n255\n".encode())
        f.write(np.ascontiguousarray(img, np.uint8).tobytes())


def _read_dump(prefix):
    shape = [int(v) for v in open(prefix + ".shape").read().strip().split(",")]
    data = np.fromfile(prefix + ".bin", dtype=np.float32)
    assert data.size == int(np.prod(shape))
    return shape, data


@pytest.mark.gpu
def test_example_encode_matches_oracle(tmp_path, s3e_lib):
    import ctypes

    path = str(tmp_path / "m.ggml")
    s3e_lib.synth_write(path, img_size=336, patch=14, embed_dim=1024, depth=2, heads=16, window=8,
                        global_idx=(1,), ftype="q8_0", seed=21, std=0.02, random_affine=True, neck=1)
    rng = np.random.default_rng(9)
    img = rng.integers(0, 256, (400, 300, 3), dtype=np.uint8)  # resized to 336² by the engine
    _write_ppm(str(tmp_path / "img.ppm"), img)
    out = str(tmp_path / "a_")
    print("sam3_encode on a 300x400 PPM", flush=True)
    r = subprocess.run([EXE, "-m", path, "-i", str(tmp_path / "img.ppm"), "-o", out, "-r", "2"],
                       capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    assert "visual_only=1" in r.stdout
    om = orc.OracleModel(path)
    chw = orc.preprocess_sam3(img, 336)
    orc.LIB.orc_set_variant.argtypes = [ctypes.c_int]
    refs = []
    for variant in (0, 1):
        orc.LIB.orc_set_variant(variant)
        try:
            v = om.encode(chw)
            refs.append([v] + om.neck(v, "trk"))
        finally:
            orc.LIB.orc_set_variant(0)
    names = ["vit_output"] + [f"neck_trk_{i}" for i in range(4)]
    shapes = [[1024, 24, 24]] + [[256, s, s] for s in (96, 48, 24, 12)]
    for k, (name, shp) in enumerate(zip(names, shapes)):
        shape, got = _read_dump(out + name)
        assert shape == shp, name
        ref = refs[0][k].ravel()
        gap = orc.rel_l2(refs[1][k], refs[0][k])
        gma = orc.max_abs(refs[1][k], refs[0][k])
        rl, ma = orc.rel_l2(got, ref), orc.max_abs(got, ref)
        print(f"{name}: rel_l2={rl:.3e} max_abs={ma:.3e} (ggml order gap {gap:.2e}/{gma:.2e})", flush=True)
        assert rl <= max(1e-3, 2.0 * gap) and ma <= max(5e-3, 2.0 * gma), name

    # preprocessed input of the same image: identical dumps
    chw.astype(np.float32).tofile(str(tmp_path / "img.chw.f32"))
    out2 = str(tmp_path / "b_")
    r = subprocess.run([EXE, "-m", path, "-p", str(tmp_path / "img.chw.f32"), "-s", "336", "-o", out2],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    for name in names:
        assert np.array_equal(_read_dump(out + name)[1], _read_dump(out2 + name)[1]), name
    # img_size mismatch is refused (sam3.cpp:7004-7008)
    r = subprocess.run([EXE, "-m", path, "-p", str(tmp_path / "img.chw.f32"), "-s", "224", "-o", out2],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 1


@pytest.mark.gpu
def test_example_encode_sam2_matches_oracle(tmp_path, s3e_lib):
    """The same program on a SAM 2 file (Hiera-T at 512 px): model type SAM2,
    visual-only, and the default dumps (three FPN levels after scalp, four
    stage outputs) equal to the oracle's to the quantized specification."""
    import ctypes

    path = str(tmp_path / "h.ggml")
    s3e_lib.synth_write_sam2(path, "hiera_t", img_size=512, ftype="q4_0", seed=23, std=0.05, random_affine=True)
    img = np.random.default_rng(10).integers(0, 256, (300, 500, 3), dtype=np.uint8)
    _write_ppm(str(tmp_path / "img.ppm"), img)
    out = str(tmp_path / "h_")
    print("sam3_encode (SAM 2) on a 500x300 PPM", flush=True)
    r = subprocess.run([EXE, "-m", path, "-i", str(tmp_path / "img.ppm"), "-o", out],
                       capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    assert "model: SAM2, visual_only=1" in r.stdout
    om = orc.OracleHiera(path)
    chw = orc.preprocess_sam2(img, 512)
    orc.LIB.orc_set_variant.argtypes = [ctypes.c_int]
    refs = []
    for variant in (0, 1):
        orc.LIB.orc_set_variant(variant)
        try:
            levels, stages = om.encode(chw)
            refs.append(levels + stages)
        finally:
            orc.LIB.orc_set_variant(0)
    names = [f"neck_trk_{i}" for i in range(3)] + [f"hiera_stage_{i}" for i in range(4)]
    shapes = [[256, s, s] for s in (128, 64, 32)] + [[96 << i, 128 >> i, 128 >> i] for i in range(4)]
    for k, (name, shp) in enumerate(zip(names, shapes)):
        shape, got = _read_dump(out + name)
        assert shape == shp, name
        ref = refs[0][k].ravel()
        gap = orc.rel_l2(refs[1][k], refs[0][k])
        gma = orc.max_abs(refs[1][k], refs[0][k])
        rl, ma = orc.rel_l2(got, ref), orc.max_abs(got, ref)
        print(f"{name}: rel_l2={rl:.3e} max_abs={ma:.3e} (ggml order gap {gap:.2e}/{gma:.2e})", flush=True)
        assert rl <= max(1e-3, 2.0 * gap) and ma <= max(5e-3, 2.0 * gma), name


@pytest.mark.gpu
def test_example_stage_hooks_match_oracle(tmp_path, s3e_lib):
    """The test-only entry points of sam3.h through the shim: the prefix, the
    prefix and block sub-stages (each fed the previous stage's output), the
    host references of the F16 linears and the backbone-only encode, each
    compared with the oracle on the same input."""
    path = str(tmp_path / "f.ggml")
    s3e_lib.synth_write(path, img_size=336, patch=14, embed_dim=1024, depth=2, heads=16, window=8,
                        global_idx=(1,), ftype="f16", seed=31, std=0.02, random_affine=True, neck=1)
    chw = orc.preprocess_sam3(np.random.default_rng(12).integers(0, 256, (336, 336, 3), dtype=np.uint8), 336)
    chw.astype(np.float32).tofile(str(tmp_path / "img.chw.f32"))
    om = orc.OracleModel(path)
    for bi in (0, 1):
        out = str(tmp_path / f"s{bi}_")
        print(f"sam3_encode stage hooks, block {bi}", flush=True)
        r = subprocess.run([EXE, "-m", path, "-p", str(tmp_path / "img.chw.f32"), "-s", "336", "-o", out,
                            "-B" if bi == 1 else "-b", str(bi)], capture_output=True, text=True, timeout=120)
        print(r.stdout, r.stderr[-2000:], flush=True)
        assert r.returncode == 0

        def dump(name):
            shape, data = _read_dump(out + name)
            return data, tuple(shape)

        x0, ne0 = dump("block0_input")
        assert ne0 == (1024, 24, 24, 1) and orc.rel_l2(x0, om.prefix(chw).ravel()) <= 1e-5
        img_ne = (336, 336, 3, 1)
        got, ne = dump("stage_PATCH_EMBED")
        ref, one = om.prefix_stage(0, chw, img_ne)
        assert ne == one and orc.rel_l2(got, ref) <= 1e-6
        cols, cne = dump("stage_PATCH_IM2COL")
        assert np.array_equal(cols, om.prefix_stage(1, chw, img_ne)[0])
        got, ne = dump("stage_PATCH_MULMAT")
        ref, one = om.prefix_stage(3, cols, cne)
        assert ne == one and orc.rel_l2(got, ref) <= 1e-6
        # block stages, each on the shim's own previous output
        names = orc.BLOCK_STAGES
        chain = ["NORM1", "WINDOW_PART", "QKV_PROJ", "ATTN_CORE", "ATTN_PROJ", "WINDOW_UNPART"]
        if bi == 1:  # global block: no window stages
            chain = [c for c in chain if not c.startswith("WINDOW")]
        x, xne = x0, ne0
        ins = {}
        for nm in chain:
            got, ne = dump("stage_" + nm)
            ref, one = om.block_stage(bi, names.index(nm), x, xne)
            ins[nm] = (x, xne)
            assert ne == one, nm
            rl = orc.rel_l2(got, ref)
            print(f"shim block {bi} {nm}: rel_l2={rl:.3e}", flush=True)
            assert rl <= (2e-3 if nm == "ATTN_CORE" else 1e-6), nm
            x, xne = got, ne
        x1 = (x0 + x).astype(np.float32)
        n2, _ = dump("stage_NORM2")
        assert np.array_equal(n2, om.block_stage(bi, names.index("NORM2"), x1, ne0)[0])
        x, xne = n2, ne0
        for nm in ("MLP_FC1", "MLP_GELU", "MLP_FC2"):
            got, ne = dump("stage_" + nm)
            ref, one = om.block_stage(bi, names.index(nm), x, xne)
            ins[nm] = (x, xne)
            assert ne == one and orc.rel_l2(got, ref) <= 1e-6, nm
            x, xne = got, ne
        # fc1 → GELU → fp16 rounding of fc2's input: last-bit differences of
        # fc1 flip a few fp16 roundings (ggml's own two evaluation orders are
        # 7.7e-6 apart on such a stage)
        got, _ = dump("stage_MLP")
        assert orc.rel_l2(got, om.block_stage(bi, names.index("MLP"), n2, ne0)[0]) <= 5e-5
        # host references (fp16 operands, one sequential f32 sum per output:
        # its rounding grows with K, 1.2e-6 at K = 4736) = the same linears
        for nm in ("QKV_PROJ", "ATTN_PROJ", "MLP_FC1", "MLP_FC2"):
            got, ne = dump("host_" + nm)
            ref, one = om.block_stage(bi, names.index(nm), *ins[nm])
            assert ne == one and orc.rel_l2(got, ref) <= 1e-5, nm
        got, ne = dump("vit_output")
        assert orc.rel_l2(got, om.encode(chw).ravel()) <= 2e-3


@pytest.mark.gpu
def test_example_encode_img_size(tmp_path, s3e_lib):
    """sam3_params::encode_img_size through the sam3.h API: a SAM 2 file with
    a 512 px native size encoded at 256 px (sam3_create_state, sam3.cpp:
    3392-3402; the Hiera grids halve and the positional embedding is
    re-interpolated) against the oracle at that size; a SAM 3 file refuses a
    non-native size at sam3_create_state."""
    import ctypes

    path = str(tmp_path / "h.ggml")
    s3e_lib.synth_write_sam2(path, "hiera_t", img_size=512, ftype="q8_0", seed=29, std=0.05, random_affine=True)
    img = np.random.default_rng(12).integers(0, 256, (300, 380, 3), dtype=np.uint8)
    _write_ppm(str(tmp_path / "img.ppm"), img)
    out = str(tmp_path / "h_")
    print("sam3_encode (SAM 2, encode_img_size 256)", flush=True)
    r = subprocess.run([EXE, "-m", path, "-i", str(tmp_path / "img.ppm"), "-o", out, "-e", "256"],
                       capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    assert "encode_img_size=256 (model native=512)" in r.stderr
    om = orc.OracleHiera(path)
    om.set_img_size(256)
    chw = orc.preprocess_sam2(img, 256)
    orc.LIB.orc_set_variant.argtypes = [ctypes.c_int]
    refs = []
    for variant in (0, 1):
        orc.LIB.orc_set_variant(variant)
        try:
            levels, stages = om.encode(chw)
            refs.append(levels + stages)
        finally:
            orc.LIB.orc_set_variant(0)
    names = [f"neck_trk_{i}" for i in range(3)] + [f"hiera_stage_{i}" for i in range(4)]
    shapes = [[256, s, s] for s in (64, 32, 16)] + [[96 << i, 64 >> i, 64 >> i] for i in range(4)]
    for k, (name, shp) in enumerate(zip(names, shapes)):
        shape, got = _read_dump(out + name)
        assert shape == shp, name
        ref = refs[0][k].ravel()
        gap, gma = orc.rel_l2(refs[1][k], refs[0][k]), orc.max_abs(refs[1][k], refs[0][k])
        rl, ma = orc.rel_l2(got, ref), orc.max_abs(got, ref)
        print(f"{name} @256: rel_l2={rl:.3e} max_abs={ma:.3e} (ggml order gap {gap:.2e}/{gma:.2e})", flush=True)
        assert rl <= max(1e-3, 2.0 * gap) and ma <= max(5e-3, 2.0 * gma), name
    # a SAM 3 file keeps its native grid
    p3 = str(tmp_path / "v.ggml")
    s3e_lib.synth_write(p3, img_size=336, depth=1, window=8, global_idx=(0,), ftype="q8_0", seed=2)
    r = subprocess.run([EXE, "-m", p3, "-i", str(tmp_path / "img.ppm"), "-o", out, "-e", "224"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "native 336 px" in r.stderr, r.stderr[-1000:]
