"""GPU parity of the image preprocessing (s3e_preprocess_image:
sam3_resize_bilinear + sam3_preprocess_image, sam3.cpp:3441-3514, and
sam2_preprocess_image, :3518-3544) against the CPU oracle
(orc_preprocess_sam3 / orc_preprocess_sam2, pinned in test_oracle.py and
test_oracle_hiera.py).

The resize is double-precision arithmetic in the reference's order and the
normalisation two correctly rounded f32 operations, so the bar is bit
equality of the CHW f32 output: camera-size down-scales, up-scales,
non-integer ratios, the identity size (no resize), degenerate 1×1 and thin
images, for both normalisations.
"""
import numpy as np
import pytest

import oracle_lib as orc

pytestmark = pytest.mark.gpu

SIZES = [(1920, 1080, 1008), (640, 480, 336), (100, 50, 336), (1008, 1008, 1008), (1007, 1009, 1008),
         (1, 1, 16), (7, 3, 64), (4000, 3000, 1024), (333, 777, 1024), (1024, 1024, 1024), (2, 900, 512)]


def _gpu(ctx, img, S, norm):
    h, w, _ = img.shape
    src = ctx.to_device(np.ascontiguousarray(img))
    out = ctx.buffer(3 * S * S * 4)
    ctx.preprocess_image(src, w, h, S, norm, out)
    ctx.sync()
    return out.download(np.float32, (3, S, S))


@pytest.mark.parametrize("w,h,S", SIZES)
@pytest.mark.parametrize("norm", [0, 1])
def test_preprocess_bit_exact(ctx, w, h, S, norm):
    img = np.random.default_rng(w * 7 + h + norm).integers(0, 256, (h, w, 3), dtype=np.uint8)
    print(f"preprocess {w}x{h} -> {S} norm {norm}", flush=True)
    got = _gpu(ctx, img, S, norm)
    ref = (orc.preprocess_sam3 if norm == 0 else orc.preprocess_sam2)(img, S)
    assert got.shape == ref.shape
    bad = int(np.sum(got != ref))
    assert bad == 0, f"{bad} of {got.size} values differ"


def test_preprocess_rejects(ctx):
    import s3e

    src = ctx.buffer(64)
    out = ctx.buffer(3 * 16 * 16 * 4)
    for args in [(0, 4, 16, 0), (4, 0, 16, 0), (4, 4, 0, 0), (4, 4, 16, 2), (4, 4, 16, -1)]:
        with pytest.raises(s3e.S3EError):
            ctx.preprocess_image(src, *args, out)
