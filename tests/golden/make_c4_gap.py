"""Writes tests/golden/c4_order_gap.json: how far apart ggml's two CPU
evaluation orders (x86 AVX2 and generic C dot products, both restated in the
oracle and selected with orc_set_variant) put the whole SAM 3 ViT encoder and
its tracker neck at the real size: 1008×1008, 32 blocks, window 24, global
blocks 7/15/23/31, random-init Q4_0 weights N(0, 0.02) with random biases and
LayerNorm affine (seed 0), uniform random uint8 image (seed 0) — the model
and image of tests/test_gpu_c4.py.  The generic order is scalar and takes
minutes on the whole encoder, so the distance is measured once here and
committed.  It is the scale against which the GPU's end-to-end distance
from the AVX2 order is judged: both are re-quantization cascades started by
fp32 summation-order differences.

Run: python3 tests/golden/make_c4_gap.py   (about 10 minutes on 8 cores)
"""
import ctypes
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "sam3.cpp_amd"))

import oracle_lib as orc  # noqa: E402
import test_gpu_c4 as c4  # noqa: E402

orc.LIB.orc_set_variant.argtypes = [ctypes.c_int]


def main():
    out = {}
    with tempfile.TemporaryDirectory() as td:
        for ft in ("q4_0",):
            path = os.path.join(td, f"c4_{ft}.ggml")
            c4.c4_model(path, ft)
            om = orc.OracleModel(path)
            chw = orc.preprocess_sam3(c4.c4_image(), c4.IMG)
            res = {}
            for variant in (0, 1):
                orc.LIB.orc_set_variant(variant)
                x = om.encode(chw)
                res[variant] = [x] + om.neck(x, "trk")
                print(f"{ft}: variant {variant} done", flush=True)
            orc.LIB.orc_set_variant(0)
            names = ["vit_output"] + [f"neck_trk_{i}" for i in range(4)]
            out[ft] = {n: {"rel_l2": orc.rel_l2(b, a), "max_abs": orc.max_abs(b, a)}
                       for n, a, b in zip(names, res[0], res[1])}
            print(ft, json.dumps(out[ft]), flush=True)
    with open(os.path.join(HERE, "c4_order_gap.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
