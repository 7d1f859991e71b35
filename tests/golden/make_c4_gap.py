"""Writes tests/golden/c4_order_gap.json: how far apart ggml's own CPU
evaluation orders put the SAM 3 ViT encoder and its tracker neck at the
real size — 1008×1008, 32 blocks, window 24, global blocks 7/15/23/31,
random-init Q4_0 and Q8_0 weights N(0, 0.02) with random biases and
LayerNorm affine (seed 0), uniform random uint8 image (seed 0): the models
and image of tests/test_gpu_c4.py.

The orders (restated in the oracle, selected with orc_set_variant):
  x86      ggml's AVX2 build (the oracle's default);
  generic  ggml's generic scalar dots;
  arm      the Apple M4 Pro build behind the reference's published timings
           (README.md:50-69): llamafile tinyBLAS_Q0_ARM for Q4_0 / Q8_0,
           NEON quantizers (id = 1/d) and f32 dots;
  arm_dotprod, arm_i8mm  ggml's NEON vec_dot with one or two rows per call.

For each weight type the file holds, per output (vit_output, neck_trk_0..3)
and for blocks 0 (windowed) and 7 (global) on the oracle's prefix output
— and under "q4_0_full", for the full SAM 3 file of the same seed (both
necks; its backbone is the visual-only file's), neck_det_0..3 and
neck_trk_0..3 on each build's own backbone output —
the relative L2 / max-abs distance of every order from the x86 one, and the
largest distance over all pairs of orders ("max_pair").  The GPU tests judge
the engine's distance from the x86 order against max_pair: both are
re-quantization cascades started by fp32 summation-order differences, and a
GPU that sat further from the x86 order than ggml's builds sit from each
other would be doing something the reference does not.

Run: python3 tests/golden/make_c4_gap.py   (about an hour on 8 cores)
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
import test_gpu_c4 as c4  # noqa: E402

orc.LIB.orc_set_variant.argtypes = [ctypes.c_int]
ORDERS = {"x86": 0, "generic": 1, "arm": 2, "arm_dotprod": 3, "arm_i8mm": 4}
NAMES = ["vit_output"] + [f"neck_trk_{i}" for i in range(4)]


def _dist(a, b):
    return {"rel_l2": orc.rel_l2(b, a), "max_abs": orc.max_abs(b, a)}


def _summary(outs):
    """outs: order -> array.  Distances from x86, and the largest pair."""
    res = {o: _dist(outs["x86"], outs[o]) for o in outs if o != "x86"}
    pairs = [_dist(outs[a], outs[b]) for a, b in itertools.combinations(outs, 2)]
    res["max_pair"] = {"rel_l2": max(p["rel_l2"] for p in pairs), "max_abs": max(p["max_abs"] for p in pairs)}
    return res


def main():
    out = {}
    with tempfile.TemporaryDirectory() as td:
        for ft in ("q4_0", "q8_0"):
            path = os.path.join(td, f"c4_{ft}.ggml")
            c4.c4_model(path, ft)
            om = orc.OracleModel(path)
            chw = orc.preprocess_sam3(c4.c4_image(), c4.IMG)
            orc.LIB.orc_set_variant(0)
            x0 = om.prefix(chw)
            res = {}
            for bi in (0, 7):
                outs = {}
                for name, v in ORDERS.items():
                    orc.LIB.orc_set_variant(v)
                    outs[name] = om.block(bi, x0)
                orc.LIB.orc_set_variant(0)
                res[f"block_{bi}"] = _summary(outs)
                print(ft, f"block {bi}", json.dumps(res[f"block_{bi}"]["max_pair"]), flush=True)
            full = None
            if ft == "q4_0":
                fpath = os.path.join(td, f"c4_{ft}_full.ggml")
                c4.c4_model(fpath, ft, neck=2)
                full = orc.OracleModel(fpath)
            files = {}
            for name, v in ORDERS.items():
                t0 = time.time()
                orc.LIB.orc_set_variant(v)
                x = om.encode(chw)
                arrs = [x] + om.neck(x, "trk")
                if full is not None:
                    arrs += full.neck(x, "det") + full.neck(x, "trk")
                orc.LIB.orc_set_variant(0)
                files[name] = os.path.join(td, f"{ft}_{name}.npz")
                np.savez(files[name], *arrs)
                del arrs, x
                print(f"{ft}: {name} encoded in {time.time() - t0:.0f} s", flush=True)
            names = NAMES + ([f"full:neck_det_{i}" for i in range(4)] + [f"full:neck_trk_{i}" for i in range(4)]
                             if full is not None else [])
            res_full = {}
            for i, n in enumerate(names):
                outs = {name: np.load(f)[f"arr_{i}"] for name, f in files.items()}
                summ = _summary(outs)
                if n.startswith("full:"):
                    res_full[n[5:]] = summ
                else:
                    res[n] = summ
                print(ft, n, json.dumps(summ["max_pair"]), flush=True)
            out[ft] = res
            if full is not None:
                out[f"{ft}_full"] = res_full
            for f in files.values():
                os.remove(f)
            os.remove(path)
    with open(os.path.join(HERE, "c4_order_gap.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
