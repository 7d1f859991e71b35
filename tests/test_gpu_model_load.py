"""s3e_model_load on damaged files: every truncation and every corrupted
header field or tensor record is refused with an error status, never read
past the end of the file or turned into an allocation the file cannot back
(the loader checks each record's size against the bytes left before it
allocates).  The load path only parses, repacks on the host and copies to the
device, so nothing here runs a kernel."""
import pytest

import s3e
from model_damage import damaged

pytestmark = pytest.mark.gpu


def _check(ctx, tmp_path, good):
    m = s3e.Model(ctx, good)  # the undamaged file loads
    m.free()
    data = open(good, "rb").read()
    cases = damaged(data)
    for what, b in cases:
        p = tmp_path / f"{what}.ggml"
        p.write_bytes(b)
        print(f"damaged model file: {what} ({len(b)} bytes)", flush=True)
        with pytest.raises(s3e.S3EError):
            s3e.Model(ctx, str(p))
    return len(cases)


def test_damaged_vit_files_are_refused(ctx, tmp_path):
    path = str(tmp_path / "vit_q4_0.ggml")
    s3e.synth_write(path, img_size=336, patch=14, embed_dim=128, depth=2, heads=2, mlp_ratio_x1000=4000, window=8,
                    global_idx=(1,), ftype="q4_0", seed=2, std=0.05, neck=2, neck_dim=128, mem_attn_layers=1)
    assert _check(ctx, tmp_path, path) > 25


def test_damaged_hiera_files_are_refused(ctx, tmp_path):
    path = str(tmp_path / "hiera_q8_0.ggml")
    s3e.synth_write_sam2(path, "hiera_t", img_size=64, ftype="q8_0", seed=5, std=0.05, mem_attn_layers=1,
                         embed_dim=32, stages=(1, 1, 1, 1), global_idx=(), window_spec=(4, 4, 2, 2))
    assert _check(ctx, tmp_path, path) > 25
