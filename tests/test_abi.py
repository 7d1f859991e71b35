"""C-ABI and host-side checks that need no GPU.

- libs3e.so loads and exports every function include/s3e.h declares.
- The synthetic model writer produces sam3.cpp-format files: header,
  hparams, tensor records, 32-byte aligned data, the quantize tool's dtype
  rule (ne0 % 32 == 0 → weight type, else F32; pos_embed/freqs_cis F32).
- The writer's Q4_0/Q4_1/Q8_0 blocks equal the oracle's reference quantizer
  applied to the same weights (two independent restatements of ggml's
  quantize_row_*_ref agree byte for byte).
- Error paths return a status and a message instead of crashing.
"""
import ctypes
import os
import re
import struct
import subprocess
import sys

import numpy as np
import pytest

import oracle_lib as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def s3e():
    import s3e as m

    return m


def declared_functions():
    text = open(os.path.join(ROOT, "include", "s3e.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(s3e_\w+)\s*\(", text)))


def test_exports_every_declared_symbol(s3e):
    names = declared_functions()
    assert len(names) >= 30
    for n in names:
        assert hasattr(s3e.LIB, n), n
    assert sorted(s3e.DECLARED) == names
    assert s3e.LIB.s3e_abi_version() == 6


def read_file(path):
    data = open(path, "rb").read()
    magic, version, ftype, n = struct.unpack_from("<Iiii", data, 0)
    hp = struct.unpack_from("<39i", data, 16)
    off = 16 + 39 * 4
    tensors = {}
    for _ in range(n):
        nd, nl, dt = struct.unpack_from("<iii", data, off)
        off += 12
        ne = struct.unpack_from(f"<{nd}i", data, off)
        off += 4 * nd
        name = data[off:off + nl].decode()
        off += nl
        off += (32 - off % 32) % 32
        nel = int(np.prod(ne))
        nbytes = {0: 4 * nel, 1: 2 * nel, 2: nel // 32 * 18, 3: nel // 32 * 20, 8: nel // 32 * 34}[dt]
        tensors[name] = (dt, ne, off, data[off:off + nbytes])
        off += nbytes
    assert off == len(data)
    return magic, version, ftype, hp, tensors


@pytest.mark.parametrize("ft,code", [("q4_0", 2), ("q4_1", 3), ("q8_0", 8), ("f16", 1), ("f32", 0)])
def test_synth_file_format(s3e, tmp_path, ft, code):
    p = str(tmp_path / f"m_{ft}.ggml")
    s3e.synth_write(p, img_size=168, depth=2, window=4, global_idx=(1,), ftype=ft, seed=2)
    magic, version, ftype, hp, t = read_file(p)
    assert (magic, version, ftype) == (0x73616D33, 3, code)
    assert hp[:8] == (168, 14, 1024, 2, 16, 4625, 4, 4) and hp[8:12] == (1, -1, -1, -1)
    assert hp[-1] == 1  # visual_only
    assert hp[18] == 256  # neck_dim
    assert len(t) == 4 + 13 * 2 + 22  # backbone + tracker neck
    for name, (dt, ne, off, raw) in t.items():
        assert off % 32 == 0, name
        if len(ne) == 1 or "pos_embed" in name or "freqs_cis" in name:
            assert dt == 0, name
        elif code >= 2:
            assert dt == (code if ne[0] % 32 == 0 else 0), name
        elif code == 1:
            # the converters keep "embed" tensors F32 in F16 files (the loader casts them)
            assert dt == (0 if "embed" in name else 1), name
        else:
            assert dt == code, name
    assert t["vit.blocks.1.attn.freqs_cis"][1] == (2, 32, 144)
    assert t["vit.blocks.0.attn.freqs_cis"][1] == (2, 32, 16)
    assert t["vit.patch_embed.proj.weight"][1] == (14, 14, 3, 1024)
    # neck kernels: conv [kW, kH, Cin, Cout], deconvolution [kW, kH, Cout, Cin]
    assert t["neck.trk.0.dconv_2x2_0.weight"][1] == (2, 2, 512, 1024)
    assert t["neck.trk.0.dconv_2x2_1.weight"][1] == (2, 2, 256, 512)
    assert t["neck.trk.1.conv_1x1.weight"][1] == (1, 1, 512, 256)
    assert t["neck.trk.3.conv_1x1.weight"][1] == (1, 1, 1024, 256)
    assert t["neck.trk.2.conv_3x3.weight"][1] == (3, 3, 256, 256)
    assert t["neck.trk.0.conv_3x3.bias"][1] == (256,)
    # the oracle reads the same file
    om = orc.OracleModel(p)
    assert om.hp[:8] == [168, 14, 1024, 2, 16, 4736, 4, 4]
    assert om.hp[13:16] == [256, 1, 1]


@pytest.mark.parametrize("neck,n_extra,visual_only", [(0, 0, 1), (2, 44, 0)])
def test_synth_neck_options(s3e, tmp_path, neck, n_extra, visual_only):
    p = str(tmp_path / f"n{neck}.ggml")
    s3e.synth_write(p, img_size=168, depth=1, window=4, global_idx=(), ftype="q8_0", seed=2, neck=neck,
                    neck_dim=128)
    _, _, _, hp, t = read_file(p)
    assert len(t) == 4 + 13 + n_extra
    assert hp[-1] == visual_only and hp[18] == 128
    if neck == 2:
        assert t["neck.det.2.conv_3x3.weight"][1] == (3, 3, 128, 128)
        assert orc.OracleModel(p).hp[15] == 3


@pytest.mark.parametrize("ft,code", [("q4_0", 2), ("q4_1", 3), ("q8_0", 8)])
def test_writer_quantizer_matches_oracle(s3e, tmp_path, ft, code):
    pf, pq = str(tmp_path / "f32.ggml"), str(tmp_path / f"{ft}.ggml")
    s3e.synth_write(pf, img_size=168, depth=1, window=4, global_idx=(), ftype="f32", seed=9)
    s3e.synth_write(pq, img_size=168, depth=1, window=4, global_idx=(), ftype=ft, seed=9)
    tf, tq = read_file(pf)[4], read_file(pq)[4]
    for name in ("vit.blocks.0.attn.qkv.weight", "vit.blocks.0.mlp.lin2.weight"):
        dtf, ne, _, raw = tf[name]
        w = np.frombuffer(raw, np.float32).reshape(ne[1], ne[0])
        assert tq[name][3] == orc.quantize_ref(code, w).tobytes(), name


def test_synth_rejects_bad_config(s3e, tmp_path):
    with pytest.raises(s3e.S3EError, match="unsupported ftype"):
        s3e.synth_write(str(tmp_path / "x.ggml"), ftype=7, img_size=168, depth=1, window=4, global_idx=())
    with pytest.raises(s3e.S3EError, match="inconsistent"):
        s3e.synth_write(str(tmp_path / "x.ggml"), img_size=170, depth=1, window=4, global_idx=())


def test_null_arguments_report_errors(s3e):
    L = s3e.LIB
    assert L.s3e_ctx_create(0, None) == 1
    assert b"NULL" in L.s3e_last_error()
    assert L.s3e_mul_mat(None, None, None, 0, None, None) == 1
    assert L.s3e_layer_norm(None, None, 0, 0, ctypes.c_float(0), None, None, None) == 1
    assert L.s3e_model_load(None, b"/nonexistent", None) == 1


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
