"""ctypes access to the CPU oracle (oracle/liboracle.so) for the tests.

The oracle is what the GPU results are compared against: a C restatement of ggml's CPU arithmetic on the
sam3.cpp encoder path.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg load it.
"""
from __future__ import annotations

import ctypes
import os
import struct
import subprocess
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint16, c_void_p

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
LIB_PATH = os.path.join(ORACLE_DIR, "liboracle.so")

F32, F16, Q4_0, Q4_1, Q8_0, Q8_1 = 0, 1, 2, 3, 8, 9
BLOCK_BYTES = {Q4_0: 18, Q4_1: 20, Q8_0: 34, Q8_1: 36}
VEC_DOT = {Q4_0: Q8_0, Q8_0: Q8_0, Q4_1: Q8_1, F16: F16, F32: F32}


def _load():
    if not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-C", ORACLE_DIR], check=True, capture_output=True)
    lib = ctypes.CDLL(LIB_PATH)
    P = c_void_p
    sig = {
        "orc_fp32_to_fp16": (ctypes.c_uint16, [c_float]),
        "orc_fp16_to_fp32": (c_float, [ctypes.c_uint16]),
        "orc_fp16_to_fp32_soft": (c_float, [ctypes.c_uint16]),
        "orc_set_variant": (None, [c_int]),
        "orc_fp32_to_fp16_row": (None, [P, P, c_int64]),
        "orc_fp16_to_fp32_row": (None, [P, P, c_int64]),
        "orc_row_size": (c_size_t, [c_int, c_int64]),
        "orc_vec_dot_type": (c_int, [c_int]),
        "orc_quantize_row_q4_0_ref": (None, [P, P, c_int64]),
        "orc_quantize_row_q4_1_ref": (None, [P, P, c_int64]),
        "orc_quantize_row_q8_0_ref": (None, [P, P, c_int64]),
        "orc_quantize_row_q8_1_ref": (None, [P, P, c_int64]),
        "orc_quantize_row_q8_0": (None, [P, P, c_int64]),
        "orc_quantize_row_q8_1": (None, [P, P, c_int64]),
        "orc_from_float": (None, [c_int, P, P, c_int64]),
        "orc_dequantize_row": (None, [c_int, P, P, c_int64]),
        "orc_vec_dot": (c_float, [c_int, c_int64, P, P]),
        "orc_block_isums": (None, [c_int, c_int64, P, P, P]),
        "orc_mul_mat": (None, [c_int, P, c_int64, c_int64, P, c_int64, P, c_int]),
        "orc_mul_mat_preq": (None, [c_int, P, c_int64, c_int64, P, c_int64, P, c_int]),
        "orc_layer_norm": (None, [P, P, c_int64, c_int64, c_float, P, P, c_int]),
        "orc_gelu_erf": (None, [P, c_int64]),
        "orc_rope": (None, [P, c_int64, c_int64, c_int64, P]),
        "orc_flash_attn_ext": (None, [P, c_int64, c_int64, c_int64, P, c_int64, c_int64, c_int64,
                                      P, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
                                      c_float, P, c_int]),
        "orc_compute_axial_cis": (None, [P, c_int, c_int, c_int, c_float, c_float]),
        "orc_mem_attn_dims": (c_int, [P, POINTER(c_int32)]),
        "orc_mem_attn": (c_int, [P, P, P, c_int64, P, P, c_int64, c_int64, P, P, P, c_int]),
        "orc_preprocess_sam3": (None, [P, c_int, c_int, c_int, P]),
        "orc_model_load": (P, [c_char_p]),
        "orc_model_free": (None, [P]),
        "orc_last_error": (c_char_p, []),
        "orc_model_hparams": (None, [P, POINTER(c_int32)]),
        "orc_vit_prefix": (c_int, [P, P, P, c_int]),
        "orc_vit_block": (c_int, [P, c_int, P, c_int]),
        "orc_vit_encode": (c_int, [P, P, P, c_int]),
        "orc_vit_block_stage": (c_int, [P, c_int, c_int, P, P, P, P, c_int]),
        "orc_vit_prefix_stage": (c_int, [P, c_int, P, P, P, P, c_int]),
        "orc_conv_transpose_2x2": (None, [P, c_int64, c_int64, P, c_int64, c_int64, P, c_int]),
        "orc_conv2d": (None, [c_int, P, c_int64, c_int64, c_int64, c_int64, c_int64, P, c_int64, c_int64, P,
                              c_int]),
        "orc_maxpool2x2": (None, [P, c_int64, c_int64, c_int64, P]),
        "orc_sinusoidal_pe_2d": (None, [c_int, c_int, c_int, P]),
        "orc_neck_dims": (c_int, [P, c_char_p, P, P]),
        "orc_neck": (c_int, [P, c_char_p, P, P, c_int]),
        "orc_resize_bilinear_u8": (None, [P, c_int, c_int, P, c_int, c_int]),
        "orc_preprocess_sam2": (None, [P, c_int, c_int, c_int, P]),
        "orc_gelu_tanh": (None, [P, c_int64]),
        "orc_gelu_tanh_table": (None, [P]),
        "orc_bicubic": (None, [P, c_int, c_int, c_int, P, c_int, c_int]),
        "orc_model_hiera": (P, [P]),
        "orc_hiera_num_blocks": (c_int, [P]),
        "orc_hiera_block_info": (c_int, [P, c_int, P]),
        "orc_hiera_dims": (c_int, [P, P, P]),
        "orc_hiera_pos_embed": (c_int, [P, c_int, c_int, P]),
        "orc_hiera_prefix": (c_int, [P, P, P, c_int]),
        "orc_hiera_block": (c_int, [P, c_int, P, c_int, c_int, P, P, P, c_int]),
        "orc_hiera_fpn": (c_int, [P, P, P, P, c_int]),
        "orc_hiera_encode": (c_int, [P, P, P, P, c_int]),
        "orc_hiera_set_img_size": (c_int, [P, c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


LIB = _load()


def ptr(a: np.ndarray):
    return a.ctypes.data


def row_size(t: int, k: int) -> int:
    return int(LIB.orc_row_size(t, k))


def quantize_ref(t: int, x: np.ndarray) -> np.ndarray:
    """ggml_quantize_chunk reference quantizer (weights): rows of x → bytes."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.reshape(-1, x.shape[-1]).shape
    out = np.zeros(rows * row_size(t, k), dtype=np.uint8)
    fn = {Q4_0: LIB.orc_quantize_row_q4_0_ref, Q4_1: LIB.orc_quantize_row_q4_1_ref,
          Q8_0: LIB.orc_quantize_row_q8_0_ref, Q8_1: LIB.orc_quantize_row_q8_1_ref}[t]
    rs = row_size(t, k)
    for r in range(rows):
        fn(ptr(x) + r * k * 4, ptr(out) + r * rs, k)
    return out


def to_weight_bytes(t: int, w: np.ndarray) -> np.ndarray:
    """N×K float weights → ggml bytes of type t (reference quantizer / fp16 RNE)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    if t == F32:
        return w.view(np.uint8).ravel().copy()
    if t == F16:
        out = np.empty(w.size, dtype=np.uint16)
        LIB.orc_fp32_to_fp16_row(ptr(w), ptr(out), w.size)
        return out.view(np.uint8)
    return quantize_ref(t, w)


def from_float(t: int, x: np.ndarray) -> np.ndarray:
    """ggml from_float of the vec_dot type (activation conversion), row by row."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    rs = row_size(t, k)
    out = np.zeros(rows * rs, dtype=np.uint8)
    for r in range(rows):
        LIB.orc_from_float(t, ptr(x) + r * k * 4, ptr(out) + r * rs, k)
    return out


def dequantize(t: int, data: np.ndarray, rows: int, k: int) -> np.ndarray:
    out = np.empty((rows, k), dtype=np.float32)
    rs = row_size(t, k)
    data = np.ascontiguousarray(data)
    for r in range(rows):
        LIB.orc_dequantize_row(t, ptr(data) + r * rs, ptr(out) + r * k * 4, k)
    return out


def split_q8(t: int, data: np.ndarray, rows: int, k: int):
    """Q8_0/Q8_1 ggml bytes → (qs int8 [rows,k], d uint16 [rows,k/32], s uint16 or None)."""
    bb = BLOCK_BYTES[t]
    blocks = np.ascontiguousarray(data).reshape(rows, k // 32, bb)
    d = blocks[:, :, 0:2].copy().view(np.uint16).reshape(rows, k // 32)
    if t == Q8_1:
        s = blocks[:, :, 2:4].copy().view(np.uint16).reshape(rows, k // 32)
        qs = blocks[:, :, 4:].copy().view(np.int8).reshape(rows, k)
    else:
        s = None
        qs = blocks[:, :, 2:].copy().view(np.int8).reshape(rows, k)
    return qs, d, s


def mul_mat(t: int, wbytes: np.ndarray, N: int, K: int, X: np.ndarray, nthreads: int = 0) -> np.ndarray:
    X = np.ascontiguousarray(X, dtype=np.float32)
    M = X.shape[0]
    Y = np.empty((M, N), dtype=np.float32)
    LIB.orc_mul_mat(t, ptr(wbytes), N, K, ptr(X), M, ptr(Y), nthreads)
    return Y


def layer_norm(x: np.ndarray, eps: float, w=None, b=None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    LIB.orc_layer_norm(ptr(x), ptr(y), x.shape[0], x.shape[1], eps, ptr(w) if w is not None else None,
                       ptr(b) if b is not None else None, 0)
    return y


def flash_attn(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, nthreads: int = 0) -> np.ndarray:
    """q [B, nh, Nq, D], k/v [B, nh, Nkv, D] f32 → O [B, Nq, nh, D] (ggml layout)."""
    q, k, v = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v))
    B, nh, Nq, D = q.shape
    Nkv = k.shape[2]
    o = np.empty((B, Nq, nh, D), dtype=np.float32)
    LIB.orc_flash_attn_ext(ptr(q), D, Nq * D, nh * Nq * D, ptr(k), D, Nkv * D, nh * Nkv * D,
                           ptr(v), D, Nkv * D, nh * Nkv * D, D, Nq, Nkv, nh, B, scale, ptr(o), nthreads)
    return o


class OracleModel:
    def __init__(self, path: str):
        self.h = LIB.orc_model_load(path.encode())
        if not self.h:
            raise RuntimeError("oracle model load failed: " + LIB.orc_last_error().decode())
        hp = (c_int32 * 16)()
        LIB.orc_model_hparams(self.h, hp)
        self.hp = list(hp)
        self.img, self.patch, self.E, self.depth = hp[0], hp[1], hp[2], hp[3]
        self.grid = self.img // self.patch

    def prefix(self, chw: np.ndarray, nthreads: int = 0) -> np.ndarray:
        x = np.empty((self.grid * self.grid, self.E), dtype=np.float32)
        chw = np.ascontiguousarray(chw, dtype=np.float32)
        assert LIB.orc_vit_prefix(self.h, ptr(chw), ptr(x), nthreads) == 0, LIB.orc_last_error()
        return x

    def block(self, i: int, x: np.ndarray, nthreads: int = 0) -> np.ndarray:
        x = np.array(x, dtype=np.float32, copy=True)
        assert LIB.orc_vit_block(self.h, i, ptr(x), nthreads) == 0, LIB.orc_last_error()
        return x

    def encode(self, chw: np.ndarray, nthreads: int = 0) -> np.ndarray:
        x = np.empty((self.grid * self.grid, self.E), dtype=np.float32)
        chw = np.ascontiguousarray(chw, dtype=np.float32)
        assert LIB.orc_vit_encode(self.h, ptr(chw), ptr(x), nthreads) == 0, LIB.orc_last_error()
        return x

    def block_stage(self, i: int, stage: int, x: np.ndarray, ne, nthreads: int = 0) -> tuple:
        """sam3_test_run_vit_block_stage on x (ggml shape ne) → (output, out_ne)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        ine, one = np.array(ne, np.int64), np.zeros(4, np.int64)
        assert LIB.orc_vit_block_stage(self.h, i, stage, ptr(x), ptr(ine), None, ptr(one), nthreads) == 0, \
            LIB.orc_last_error()
        out = np.empty(int(np.prod(one)), np.float32)
        assert LIB.orc_vit_block_stage(self.h, i, stage, ptr(x), ptr(ine), ptr(out), ptr(one), nthreads) == 0, \
            LIB.orc_last_error()
        return out, tuple(int(v) for v in one)

    def prefix_stage(self, stage: int, x: np.ndarray, ne, nthreads: int = 0) -> tuple:
        """sam3_test_run_vit_prefix_stage on x (ggml shape ne) → (output, out_ne)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        ine, one = np.array(ne, np.int64), np.zeros(4, np.int64)
        assert LIB.orc_vit_prefix_stage(self.h, stage, ptr(x), ptr(ine), None, ptr(one), nthreads) == 0, \
            LIB.orc_last_error()
        out = np.empty(int(np.prod(one)), np.float32)
        assert LIB.orc_vit_prefix_stage(self.h, stage, ptr(x), ptr(ine), ptr(out), ptr(one), nthreads) == 0, \
            LIB.orc_last_error()
        return out, tuple(int(v) for v in one)

    def neck_dims(self, which: str = "trk"):
        side = np.zeros(4, np.int64)
        D = np.zeros(1, np.int64)
        assert LIB.orc_neck_dims(self.h, which.encode(), ptr(side), ptr(D)) == 0, LIB.orc_last_error()
        return [int(v) for v in side], int(D[0])

    def neck(self, x: np.ndarray, which: str = "trk", nthreads: int = 0):
        """sam3_build_neck_graph on vit_output x [G², E] → four [side², D] levels."""
        side, D = self.neck_dims(which)
        x = np.ascontiguousarray(x, dtype=np.float32)
        outs = [np.empty((s * s, D), np.float32) for s in side]
        arr = (c_void_p * 4)(*[o.ctypes.data for o in outs])
        rc = LIB.orc_neck(self.h, which.encode(), ptr(x), ctypes.cast(arr, c_void_p), nthreads)
        assert rc == 0, LIB.orc_last_error()
        return outs

    def __del__(self):
        if getattr(self, "h", None) and LIB is not None:
            LIB.orc_model_free(self.h)
            self.h = None


# sam3.h:112-134
BLOCK_STAGES = ["NORM1", "WINDOW_PART", "QKV_PROJ", "ATTN_CORE", "ATTN_PROJ", "WINDOW_UNPART", "NORM2",
                "MLP_FC1", "MLP_GELU", "MLP_FC2", "MLP"]
PREFIX_STAGES = ["PATCH_EMBED", "PATCH_IM2COL", "PATCH_MULMAT_RAW", "PATCH_MULMAT", "POS_ADD", "LN_PRE_NORM",
                 "LN_PRE"]


class HieraHp(ctypes.Structure):
    _fields_ = [
        ("img_size", c_int32), ("embed_dim", c_int32), ("num_heads", c_int32), ("num_stages", c_int32),
        ("stages", c_int32 * 4), ("global_n", c_int32), ("global_idx", c_int32 * 8), ("q_pool", c_int32),
        ("window_spec", c_int32 * 4), ("bkg_h", c_int32), ("bkg_w", c_int32), ("scalp", c_int32),
        ("neck_dim", c_int32), ("fpn_td_n", c_int32), ("fpn_td", c_int32 * 4),
    ]


class OracleHiera:
    """The oracle's SAM 2.x encoder (oracle/orc_hiera.c) on a model file."""

    def __init__(self, path: str):
        self.h = LIB.orc_model_load(path.encode())
        if not self.h:
            raise RuntimeError("oracle model load failed: " + LIB.orc_last_error().decode())
        hp = LIB.orc_model_hiera(self.h)
        assert hp, "not a SAM 2 model"
        self.hp = HieraHp.from_address(hp)
        self.img = self.hp.img_size
        self.nblocks = LIB.orc_hiera_num_blocks(self.h)
        self._dims()

    def _dims(self):
        side, width = np.zeros(4, np.int32), np.zeros(4, np.int32)
        LIB.orc_hiera_dims(self.h, ptr(side), ptr(width))
        self.side, self.width = [int(v) for v in side], [int(v) for v in width]

    def set_img_size(self, img: int):
        """Encode at img pixels per side from now on (sam3_create_state's
        encode_img_size)."""
        assert LIB.orc_hiera_set_img_size(self.h, img) == 0, LIB.orc_last_error()
        self.img = img
        self._dims()

    def block_info(self, i: int):
        out = np.zeros(7, np.int32)
        assert LIB.orc_hiera_block_info(self.h, i, ptr(out)) == 0, LIB.orc_last_error()
        return dict(zip(("dim_in", "dim_out", "heads", "window", "q_stride", "stage", "stage_end"),
                        (int(v) for v in out)))

    def pos_embed(self, H: int, W: int) -> np.ndarray:
        out = np.empty((H, W, self.hp.embed_dim), np.float32)
        assert LIB.orc_hiera_pos_embed(self.h, H, W, ptr(out)) == 0, LIB.orc_last_error()
        return out

    def prefix(self, chw: np.ndarray, nthreads: int = 0) -> np.ndarray:
        G = self.img // 4
        x = np.empty((G * G, self.hp.embed_dim), np.float32)
        chw = np.ascontiguousarray(chw, np.float32)
        assert LIB.orc_hiera_prefix(self.h, ptr(chw), ptr(x), nthreads) == 0, LIB.orc_last_error()
        return x

    def block(self, i: int, x: np.ndarray, H: int, W: int, nthreads: int = 0):
        info = self.block_info(i)
        Ho, Wo = (H // 2, W // 2) if info["q_stride"] else (H, W)
        y = np.empty((Ho * Wo, info["dim_out"]), np.float32)
        ho, wo = np.zeros(1, np.int32), np.zeros(1, np.int32)
        x = np.ascontiguousarray(x, np.float32)
        assert LIB.orc_hiera_block(self.h, i, ptr(x), H, W, ptr(y), ptr(ho), ptr(wo), nthreads) == 0, \
            LIB.orc_last_error()
        assert (int(ho[0]), int(wo[0])) == (Ho, Wo)
        return y, Ho, Wo

    def fpn(self, stages, nthreads: int = 0):
        D = self.hp.neck_dim
        st = [np.ascontiguousarray(s, np.float32) for s in stages]
        outs = [np.empty((s * s, D), np.float32) for s in self.side]
        sarr = (c_void_p * 4)(*[a.ctypes.data for a in st])
        oarr = (c_void_p * 4)(*[a.ctypes.data for a in outs])
        side = np.array(self.side, np.int32)
        assert LIB.orc_hiera_fpn(self.h, ctypes.cast(sarr, c_void_p), ptr(side), ctypes.cast(oarr, c_void_p),
                                 nthreads) == 0, LIB.orc_last_error()
        return outs

    def encode(self, chw: np.ndarray, nthreads: int = 0):
        """FPN levels 0 .. 3 − scalp and the four stage outputs."""
        D = self.hp.neck_dim
        outs = [np.empty((s * s, D), np.float32) for s in self.side]
        stages = [np.empty((s * s, w), np.float32) for s, w in zip(self.side, self.width)]
        oarr = (c_void_p * 4)(*[a.ctypes.data for a in outs])
        sarr = (c_void_p * 4)(*[a.ctypes.data for a in stages])
        chw = np.ascontiguousarray(chw, np.float32)
        assert LIB.orc_hiera_encode(self.h, ptr(chw), ctypes.cast(oarr, c_void_p), ctypes.cast(sarr, c_void_p),
                                    nthreads) == 0, LIB.orc_last_error()
        return outs[:4 - self.hp.scalp], stages

    def __del__(self):
        if getattr(self, "h", None) and LIB is not None:
            LIB.orc_model_free(self.h)
            self.h = None


def preprocess_sam2(img_hwc: np.ndarray, img_size: int) -> np.ndarray:
    img = np.ascontiguousarray(img_hwc, dtype=np.uint8)
    out = np.empty((3, img_size, img_size), dtype=np.float32)
    LIB.orc_preprocess_sam2(ptr(img), img.shape[1], img.shape[0], img_size, ptr(out))
    return out


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    y = np.array(x, np.float32, copy=True)
    LIB.orc_gelu_tanh(ptr(y), y.size)
    return y


def conv_transpose_2x2(w16: np.ndarray, x: np.ndarray, nthreads: int = 0) -> np.ndarray:
    """w16: fp16 bits in ggml order [Cin][Cout][2][2] (ne = [2, 2, Cout, Cin]);
    x: [H, W, Cin] f32 → [2H, 2W, Cout]."""
    Cin, Cout = w16.shape[0], w16.shape[1]
    H, W = x.shape[0], x.shape[1]
    w16 = np.ascontiguousarray(w16, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty((2 * H, 2 * W, Cout), np.float32)
    LIB.orc_conv_transpose_2x2(ptr(w16), Cin, Cout, ptr(x), H, W, ptr(y), nthreads)
    return y


def conv2d(ktype: int, w: np.ndarray, x: np.ndarray, pad: int, nthreads: int = 0) -> np.ndarray:
    """w in ggml order [Cout][Cin][KH][KW] (ne = [KW, KH, Cin, Cout]) as f32 or
    fp16 bits; x: [H, W, Cin] f32 → [OH, OW, Cout]."""
    Cout, Cin, KH, KW = w.shape
    H, W = x.shape[0], x.shape[1]
    w = np.ascontiguousarray(w, dtype=np.uint16 if ktype == F16 else np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    OH, OW = H + 2 * pad - KH + 1, W + 2 * pad - KW + 1
    y = np.empty((OH, OW, Cout), np.float32)
    LIB.orc_conv2d(ktype, ptr(w), KW, KH, Cin, Cout, pad, ptr(x), H, W, ptr(y), nthreads)
    return y


def maxpool2x2(x: np.ndarray) -> np.ndarray:
    H, W, C = x.shape
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(((H - 2) // 2 + 1, (W - 2) // 2 + 1, C), np.float32)
    LIB.orc_maxpool2x2(ptr(x), H, W, C, ptr(y))
    return y


def sinusoidal_pe_2d(H: int, W: int, d: int) -> np.ndarray:
    out = np.empty((H, W, d), np.float32)
    LIB.orc_sinusoidal_pe_2d(H, W, d, ptr(out))
    return out


def axial_cis(dim: int, end_x: int, end_y: int, theta: float = 10000.0, scale: float = 1.0) -> np.ndarray:
    """sam3_compute_axial_cis: [end_x·end_y][dim/2][2] (cos, sin)."""
    out = np.empty((end_x * end_y, dim // 2, 2), np.float32)
    LIB.orc_compute_axial_cis(ptr(out), dim, end_x, end_y, theta, scale)
    return out


def mem_attn_dims(handle) -> tuple:
    """(layers, D, MD, FFN) of a loaded model's memory attention."""
    out = (c_int32 * 4)()
    assert LIB.orc_mem_attn_dims(handle, out) == 0, LIB.orc_last_error()
    return tuple(out)


def mem_attn(handle, curr, src_pos, prompt, prompt_pos, n_ptr: int, rope_q, rope_k, nthreads: int = 0):
    """The oracle's sam3_build_mem_attn_graph on a loaded model (handle)."""
    L, D, MD, FFN = mem_attn_dims(handle)
    curr, src_pos = (np.ascontiguousarray(a, np.float32) for a in (curr, src_pos))
    prompt, prompt_pos = (np.ascontiguousarray(a, np.float32) for a in (prompt, prompt_pos))
    rope_q = np.ascontiguousarray(rope_q, np.float32)
    rope_k = None if rope_k is None else np.ascontiguousarray(rope_k, np.float32)
    N, M = curr.shape[0], prompt.shape[0]
    out = np.empty((N, D), np.float32)
    rc = LIB.orc_mem_attn(handle, ptr(curr), ptr(src_pos), N, ptr(prompt), ptr(prompt_pos), M, n_ptr, ptr(rope_q),
                          None if rope_k is None else ptr(rope_k), ptr(out), nthreads)
    assert rc == 0, LIB.orc_last_error()
    return out


def read_model_file(path: str):
    """Tensor records of a sam3.cpp model file (sam3.cpp:3091-3143):
    name → (dtype, ne, array in file order).  F32/F16 records are returned as
    float32 / float16 arrays of shape ne reversed; others as raw bytes."""
    data = open(path, "rb").read()
    magic, n = struct.unpack_from("<I", data, 0)[0], struct.unpack_from("<i", data, 12)[0]
    off = 16 + (57 if magic == 0x73616D32 else 39) * 4  # SAM 2 files carry 57 hparams
    out = {}
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
        raw = data[off:off + nbytes]
        if dt in (0, 1):
            arr = np.frombuffer(raw, np.float32 if dt == 0 else np.float16).reshape(tuple(reversed(ne)))
        else:
            arr = np.frombuffer(raw, np.uint8)
        out[name] = (dt, tuple(ne), arr)
        off += nbytes
    return out


def preprocess_sam3(img_hwc: np.ndarray, img_size: int) -> np.ndarray:
    img = np.ascontiguousarray(img_hwc, dtype=np.uint8)
    out = np.empty((3, img_size, img_size), dtype=np.float32)
    LIB.orc_preprocess_sam3(ptr(img), img.shape[1], img.shape[0], img_size, ptr(out))
    return out


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def max_abs(a: np.ndarray, b: np.ndarray) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))
