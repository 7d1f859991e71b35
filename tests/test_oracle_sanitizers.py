"""The CPU oracle under AddressSanitizer and UndefinedBehaviorSanitizer.

`make -C oracle asan` builds the oracle's sources with -fsanitize=address,
undefined together with oracle/asan_check.c, a driver that calls every entry
point once on small odd-sized inputs and then, for each model file named on
its command line, the whole encoder (ViT + both necks, or Hiera + FPN) and
the memory attention.  Any out-of-bounds access, use after free, leak or
undefined operation aborts it with a report; the test asserts a clean exit.
"""
import os
import subprocess

import pytest

import s3e
from model_damage import damaged

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")
BIN = os.path.join(ORACLE, "_asan", "asan_check")


@pytest.fixture(scope="module")
def asan_bin():
    r = subprocess.run(["make", "-C", ORACLE, "asan"], capture_output=True, text=True)
    if r.returncode != 0:
        if "sanitize" in r.stderr and ("cannot find" in r.stderr or "unrecognized" in r.stderr):
            pytest.skip("the C compiler has no sanitizer runtimes")
        raise AssertionError(r.stdout + r.stderr)
    return BIN


def _run(binary, *args):
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=1:halt_on_error=1:abort_on_error=0"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env["OMP_NUM_THREADS"] = "2"
    return subprocess.run([binary, *args], capture_output=True, text=True, env=env, timeout=600)


def test_operators_clean(asan_bin):
    r = _run(asan_bin)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "asan_check: ok (0 model file(s))" in r.stdout


def test_encoders_clean(asan_bin, tmp_path):
    vq = str(tmp_path / "vit_q4_0.ggml")
    vf = str(tmp_path / "vit_f16.ggml")
    hb = str(tmp_path / "hiera_q8_0.ggml")
    # ViT 84 px (6×6 tokens, 3×3 windows, one global block), both necks and a
    # memory-attention layer; an F16 file with the tracker neck; a small
    # four-stage Hiera with its FPN and a memory-attention layer
    s3e.synth_write(vq, img_size=84, patch=14, embed_dim=64, depth=2, heads=2, mlp_ratio_x1000=4000, window=3,
                    global_idx=(1,), ftype="q4_0", seed=3, std=0.05, random_affine=True, neck=2, neck_dim=64,
                    mem_attn_layers=1)
    s3e.synth_write(vf, img_size=84, patch=14, embed_dim=64, depth=2, heads=2, mlp_ratio_x1000=4000, window=3,
                    global_idx=(1,), ftype="f16", seed=4, std=0.05, random_affine=True, neck=1, neck_dim=64)
    s3e.synth_write_sam2(hb, "hiera_t", img_size=64, ftype="q8_0", seed=5, std=0.05, random_affine=True,
                         mem_attn_layers=1, embed_dim=32, stages=(1, 1, 1, 1), global_idx=(),
                         window_spec=(4, 4, 2, 2))
    r = _run(asan_bin, vq, vf, hb)
    assert r.returncode == 0, r.stderr[-4000:]
    out = r.stdout
    assert "asan_check: ok (3 model file(s))" in out
    assert out.count("ViT encoder + trk neck") == 2 and "ViT encoder + det neck" in out
    assert "Hiera encoder + FPN" in out
    assert out.count("memory attention") == 2


def test_damaged_files_load_clean(asan_bin, tmp_path):
    """The oracle's loader on truncated and corrupted copies of a ViT and a
    Hiera file: refusals or models that free cleanly, no memory errors."""
    vq = str(tmp_path / "vit.ggml")
    hb = str(tmp_path / "hiera.ggml")
    s3e.synth_write(vq, img_size=84, patch=14, embed_dim=64, depth=2, heads=2, mlp_ratio_x1000=4000, window=3,
                    global_idx=(1,), ftype="q4_0", seed=3, std=0.05, neck=2, neck_dim=64, mem_attn_layers=1)
    s3e.synth_write_sam2(hb, "hiera_t", img_size=64, ftype="q8_0", seed=5, std=0.05, mem_attn_layers=1,
                         embed_dim=32, stages=(1, 1, 1, 1), global_idx=(), window_spec=(4, 4, 2, 2))
    files = []
    for src in (vq, hb):
        for what, b in damaged(open(src, "rb").read()):
            p = tmp_path / f"{len(files)}_{what}.ggml"
            p.write_bytes(b)
            files.append(str(p))
    r = _run(asan_bin, "--load-only", *files)
    assert r.returncode == 0, r.stderr[-4000:]
    assert f"of {len(files)} refused" in r.stdout
