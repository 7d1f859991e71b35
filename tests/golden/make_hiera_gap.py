"""Writes tests/golden/hiera_order_gap.json: how far apart ggml's own CPU
evaluation orders put the SAM 2.1 Hiera-B+ encoder with Q8_0 weights at its
real 1024 px size (the tracking frame's encoder): stage outputs
hiera_stage_0..3 and FPN levels neck_trk_0..2, random-init weights
N(0, 0.05) with random biases and LayerNorm affine (seed 21), uniform random
uint8 image (seed 6) — the model and image of tests/test_gpu_hiera.py's
full-size test.

The orders are the oracle's (orc_set_variant): x86 AVX2, generic C, and
the three ARM NEON forms (the Apple M4 Pro build of the reference's
published timings, vec_dot with one row and with two rows per call).  For
each output the file holds every order's distance from the x86 one and the
largest distance over all pairs ("max_pair"), the yardstick the GPU test
applies to the engine's distance from the x86 order.

Run: python3 tests/golden/make_hiera_gap.py   (about 15 minutes on 8 cores)
"""
import ctypes
import itertools
import json
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "sam3.cpp_amd"))

import oracle_lib as orc  # noqa: E402

orc.LIB.orc_set_variant.argtypes = [ctypes.c_int]
ORDERS = {"x86": 0, "generic": 1, "arm": 2, "arm_dotprod": 3, "arm_i8mm": 4}
CASES = [("hiera_b+", 1024, "q8_0")]


def _dist(a, b):
    return {"rel_l2": orc.rel_l2(b, a), "max_abs": orc.max_abs(b, a)}


def main():
    import s3e

    out = {}
    with tempfile.TemporaryDirectory() as td:
        for variant, img, ft in CASES:
            path = os.path.join(td, f"{variant}_{img}_{ft}.ggml")
            s3e.synth_write_sam2(path, variant, img_size=img, ftype=ft, seed=21, std=0.05, random_affine=True,
                                 neck_dim=256)
            om = orc.OracleHiera(path)
            image = np.random.default_rng(6).integers(0, 256, (img, img, 3), dtype=np.uint8)
            chw = orc.preprocess_sam2(image, om.img)
            outs = {}
            for name, v in ORDERS.items():
                t0 = time.time()
                orc.LIB.orc_set_variant(v)
                levels, stages = om.encode(chw)
                orc.LIB.orc_set_variant(0)
                outs[name] = {**{f"hiera_stage_{i}": s for i, s in enumerate(stages)},
                              **{f"neck_trk_{i}": lv for i, lv in enumerate(levels)}}
                print(f"{variant}@{img} {ft}: {name} in {time.time() - t0:.0f} s", flush=True)
            res = {}
            for key in outs["x86"]:
                per = {o: _dist(outs["x86"][key], outs[o][key]) for o in outs if o != "x86"}
                pairs = [_dist(outs[a][key], outs[b][key]) for a, b in itertools.combinations(outs, 2)]
                per["max_pair"] = {"rel_l2": max(p["rel_l2"] for p in pairs),
                                   "max_abs": max(p["max_abs"] for p in pairs)}
                res[key] = per
                print(variant, key, json.dumps(per["max_pair"]), flush=True)
            out[f"{variant}@{img}:{ft}"] = res
    with open(os.path.join(HERE, "hiera_order_gap.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
