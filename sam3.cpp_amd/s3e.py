"""ctypes binding of the MI355X encoder engine's C ABI (include/s3e.h).

The engine itself is native (sam3.cpp_amd/libs3e.so, built from csrc/); this
module only marshals numpy arrays and device pointers across the C ABI for
the tests and the benchmark.  Importing it fails loudly when the library has
not been built: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint16, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# S3E_LIB_PATH points the binding at another build of the same library.
LIB_PATH = os.environ.get("S3E_LIB_PATH", os.path.join(HERE, "libs3e.so"))

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q4_1, TYPE_Q8_0, TYPE_Q8_1 = 0, 1, 2, 3, 8, 9
TYPE_Q8_0_F6X2 = 64  # the Q8_0 codes split into two fp6 halves (engine layout)
PREC_DEFAULT, PREC_F32 = 0, 1
FTYPE_BY_NAME = {"f32": 0, "f16": 1, "q4_0": 2, "q4_1": 3, "q8_0": 8}


NORM_SAM3 = 0      # (v/255 - 0.5)/0.5
NORM_IMAGENET = 1  # (v/255 - mean)/std, SAM 2


class S3EError(RuntimeError):
    pass


class SynthCfg(ctypes.Structure):
    _fields_ = [
        ("img_size", c_int32), ("patch", c_int32), ("embed_dim", c_int32), ("depth", c_int32),
        ("heads", c_int32), ("mlp_ratio_x1000", c_int32), ("window", c_int32),
        ("n_global", c_int32), ("global_idx", c_int32 * 4),
        ("ftype", c_int32), ("seed", c_uint64), ("std", c_float),
        ("neck", c_int32), ("neck_dim", c_int32), ("mem_attn_layers", c_int32),
    ]


class SynthSam2Cfg(ctypes.Structure):
    _fields_ = [
        ("img_size", c_int32), ("embed_dim", c_int32), ("num_heads", c_int32), ("stages", c_int32 * 4),
        ("global_n", c_int32), ("global_idx", c_int32 * 8), ("q_pool", c_int32), ("window_spec", c_int32 * 4),
        ("bkg_h", c_int32), ("bkg_w", c_int32), ("scalp", c_int32),
        ("neck_dim", c_int32), ("fpn_td_n", c_int32), ("fpn_td", c_int32 * 4),
        ("ftype", c_int32), ("seed", c_uint64), ("std", c_float), ("mem_attn_layers", c_int32),
    ]


# Hiera variants of convert_sam2_to_ggml.py:79-106
HIERA_VARIANTS = {
    "hiera_t": dict(embed_dim=96, num_heads=1, stages=(1, 2, 7, 2), global_idx=(5, 7, 9),
                    window_spec=(8, 4, 14, 7), bkg=(7, 7)),
    "hiera_s": dict(embed_dim=96, num_heads=1, stages=(1, 2, 11, 2), global_idx=(7, 10, 13),
                    window_spec=(8, 4, 14, 7), bkg=(7, 7)),
    "hiera_b+": dict(embed_dim=112, num_heads=2, stages=(2, 3, 16, 3), global_idx=(12, 16, 20),
                     window_spec=(8, 4, 14, 7), bkg=(14, 14)),
    "hiera_l": dict(embed_dim=144, num_heads=2, stages=(2, 6, 36, 4), global_idx=(23, 33, 43),
                    window_spec=(8, 4, 16, 8), bkg=(7, 7)),
}


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
    lib = ctypes.CDLL(LIB_PATH)
    P64 = POINTER(c_int64)
    sig = {
        "s3e_last_error": (c_char_p, []),
        "s3e_abi_version": (c_int, []),
        "s3e_ctx_create": (c_int, [c_int, POINTER(c_void_p)]),
        "s3e_ctx_destroy": (None, [c_void_p]),
        "s3e_ctx_sync": (c_int, [c_void_p]),
        "s3e_ctx_stream": (c_void_p, [c_void_p]),
        "s3e_malloc": (c_int, [c_void_p, c_size_t, POINTER(c_void_p)]),
        "s3e_free": (c_int, [c_void_p, c_void_p]),
        "s3e_memcpy_h2d": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
        "s3e_memcpy_d2h": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
        "s3e_weight_upload": (c_int, [c_void_p, c_int, c_int64, c_int64, c_void_p, c_size_t, POINTER(c_void_p)]),
        "s3e_weight_free": (None, [c_void_p]),
        "s3e_weight_info": (c_int, [c_void_p, P64]),
        "s3e_mul_mat": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
        "s3e_mul_mat_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
        "s3e_quantize_rows": (c_int, [c_void_p, c_int, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p]),
        "s3e_layer_norm": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_float, c_void_p, c_void_p, c_void_p]),
        "s3e_mul_mat_q": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
        "s3e_mul_mat_q_f6": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
        "s3e_mul_mat_q_batch": (c_int, [c_void_p, c_int, POINTER(c_void_p), POINTER(c_void_p), POINTER(c_void_p),
                                        POINTER(c_void_p), c_int64, POINTER(c_void_p), POINTER(c_void_p)]),
        "s3e_copy": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
        "s3e_flash_attn_ext": (c_int, [c_void_p, c_void_p, P64, c_void_p, P64, c_void_p, P64,
                                       c_int64, c_int64, c_int64, c_int64, c_int64, c_float, c_int, c_void_p]),
        "s3e_flash_attn_ext_f16": (c_int, [c_void_p, c_void_p, P64, c_void_p, P64, c_void_p, P64,
                                           c_int64, c_int64, c_int64, c_int64, c_int64, c_float, c_void_p]),
        "s3e_probe_stream": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_size_t]),
        "s3e_probe_mfma": (c_int, [c_void_p, c_int, c_int64, c_int]),
        "s3e_model_load": (c_int, [c_void_p, c_char_p, POINTER(c_void_p)]),
        "s3e_model_free": (None, [c_void_p]),
        "s3e_model_hparams": (c_int, [c_void_p, POINTER(c_int32)]),
        "s3e_state_create": (c_int, [c_void_p, c_void_p, POINTER(c_void_p)]),
        "s3e_state_create_sized": (c_int, [c_void_p, c_void_p, c_int, POINTER(c_void_p)]),
        "s3e_state_free": (None, [c_void_p]),
        "s3e_encode_chw": (c_int, [c_void_p, c_void_p]),
        "s3e_encode_chw_host": (c_int, [c_void_p, c_void_p]),
        "s3e_encode_image_u8": (c_int, [c_void_p, c_void_p, c_int, c_int]),
        "s3e_preprocess_image": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
        "s3e_vit_prefix": (c_int, [c_void_p, c_void_p, c_void_p]),
        "s3e_vit_block": (c_int, [c_void_p, c_int, c_void_p]),
        "s3e_run_neck": (c_int, [c_void_p, c_void_p]),
        "s3e_vit_block_stage": (c_int, [c_void_p, c_int, c_int, c_void_p, P64, c_void_p, P64]),
        "s3e_encode_vit_chw": (c_int, [c_void_p, c_void_p]),
        "s3e_model_tensor_get": (c_int, [c_void_p, c_char_p, POINTER(c_int), P64, c_void_p, c_size_t]),
        "s3e_vit_prefix_stage": (c_int, [c_void_p, c_int, c_void_p, P64, c_void_p, P64]),
        "s3e_hiera_block": (c_int, [c_void_p, c_int, c_void_p, c_int, c_int, c_void_p]),
        "s3e_mem_attn_dims": (c_int, [c_void_p, POINTER(c_int32)]),
        "s3e_mem_attn": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64,
                                 c_void_p, c_void_p, c_void_p]),
        "s3e_model_type": (c_int, [c_void_p]),
        "s3e_state_tensor_info": (c_int, [c_void_p, c_char_p, P64]),
        "s3e_state_tensor_get": (c_int, [c_void_p, c_char_p, c_void_p, c_size_t]),
        "s3e_state_tensor_device": (c_void_p, [c_void_p, c_char_p]),
        "s3e_synth_write": (c_int, [c_char_p, POINTER(SynthCfg)]),
        "s3e_synth_write_sam2": (c_int, [c_char_p, POINTER(SynthSam2Cfg)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


LIB = _load()
DECLARED = [
    "s3e_last_error", "s3e_abi_version", "s3e_ctx_create", "s3e_ctx_destroy", "s3e_ctx_sync", "s3e_ctx_stream",
    "s3e_malloc", "s3e_free", "s3e_memcpy_h2d", "s3e_memcpy_d2h", "s3e_weight_upload", "s3e_weight_free",
    "s3e_weight_info", "s3e_mul_mat", "s3e_mul_mat_noalloc", "s3e_mul_mat_q", "s3e_mul_mat_q_f6", "s3e_mul_mat_q_batch", "s3e_quantize_rows", "s3e_layer_norm", "s3e_copy",
    "s3e_flash_attn_ext", "s3e_flash_attn_ext_f16", "s3e_probe_stream", "s3e_probe_mfma", "s3e_model_load",
    "s3e_model_free", "s3e_model_hparams", "s3e_state_create", "s3e_state_create_sized", "s3e_state_free", "s3e_encode_chw",
    "s3e_encode_chw_host", "s3e_encode_image_u8", "s3e_preprocess_image", "s3e_vit_prefix", "s3e_vit_block", "s3e_vit_block_stage", "s3e_vit_prefix_stage", "s3e_encode_vit_chw", "s3e_model_tensor_get", "s3e_run_neck", "s3e_hiera_block", "s3e_model_type", "s3e_mem_attn_dims", "s3e_mem_attn",
    "s3e_state_tensor_info",
    "s3e_state_tensor_get", "s3e_state_tensor_device", "s3e_synth_write", "s3e_synth_write_sam2",
]


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = LIB.s3e_last_error().decode(errors="replace")
        raise S3EError(f"{what or 's3e'} failed (status {rc}): {msg}")


def synth_write(path: str, *, img_size=1008, patch=14, embed_dim=1024, depth=32, heads=16,
                mlp_ratio_x1000=4625, window=24, global_idx=(7, 15, 23, 31), ftype="q4_0",
                seed=0, std=0.02, random_affine=False, neck=1, neck_dim=256, mem_attn_layers=0) -> None:
    """Write a random-init SAM 3 model file (s3e_synth_write): the ViT
    backbone plus the tracker neck (neck=1, a visual-only file), both necks
    (neck=2) or none (neck=0), and mem_attn_layers memory-attention layers."""
    cfg = SynthCfg()
    cfg.img_size, cfg.patch, cfg.embed_dim, cfg.depth = img_size, patch, embed_dim, depth
    cfg.heads, cfg.mlp_ratio_x1000, cfg.window = heads, mlp_ratio_x1000, window
    g = list(global_idx)[:4]
    cfg.n_global = len(g)
    for i in range(4):
        cfg.global_idx[i] = g[i] if i < len(g) else -1
    cfg.ftype = FTYPE_BY_NAME[ftype] if isinstance(ftype, str) else int(ftype)
    cfg.seed = seed
    cfg.std = -abs(std) if random_affine else abs(std)
    cfg.neck, cfg.neck_dim = int(neck), int(neck_dim)
    cfg.mem_attn_layers = int(mem_attn_layers)
    check(LIB.s3e_synth_write(path.encode(), ctypes.byref(cfg)), "s3e_synth_write")


def synth_write_sam2(path: str, variant: str = "hiera_t", *, img_size=1024, ftype="f16", seed=0, std=0.02,
                     random_affine=False, neck_dim=256, q_pool=3, scalp=1, fpn_td=(2, 3), mem_attn_layers=0,
                     **over) -> None:
    """Write a random-init SAM 2.x encoder file (s3e_synth_write_sam2); keyword
    overrides replace the variant's hparams (embed_dim, num_heads, stages,
    global_idx, window_spec, bkg)."""
    v = dict(HIERA_VARIANTS[variant])
    v.update(over)
    cfg = SynthSam2Cfg()
    cfg.img_size, cfg.embed_dim, cfg.num_heads = img_size, v["embed_dim"], v["num_heads"]
    for i in range(4):
        cfg.stages[i] = v["stages"][i]
        cfg.window_spec[i] = v["window_spec"][i]
    g = list(v["global_idx"])
    cfg.global_n = len(g)
    for i in range(8):
        cfg.global_idx[i] = g[i] if i < len(g) else 0
    cfg.q_pool = q_pool
    cfg.bkg_h, cfg.bkg_w = v["bkg"]
    cfg.scalp, cfg.neck_dim = scalp, neck_dim
    cfg.fpn_td_n = len(fpn_td)
    for i in range(4):
        cfg.fpn_td[i] = fpn_td[i] if i < len(fpn_td) else 0
    cfg.ftype = FTYPE_BY_NAME[ftype] if isinstance(ftype, str) else int(ftype)
    cfg.seed = seed
    cfg.std = -abs(std) if random_affine else abs(std)
    cfg.mem_attn_layers = int(mem_attn_layers)
    check(LIB.s3e_synth_write_sam2(path.encode(), ctypes.byref(cfg)), "s3e_synth_write_sam2")


def act_scale_elems(M: int, K: int) -> int:
    """fp16 elements of one stage-major scale plane written by s3e_quantize_rows
    (row pitch M rounded up to 128, blocks rounded up to a multiple of 4)."""
    return ((K + 127) // 128) * ((M + 127) // 128 * 128) * 4


def unstage_scales(plane: np.ndarray, M: int, K: int) -> np.ndarray:
    """[M][K/32] view of a stage-major scale plane (block b of row r at
    ((b // 4) * Mp + r) * 4 + b % 4)."""
    G, Mp = (K + 127) // 128, (M + 127) // 128 * 128
    return plane.reshape(G, Mp, 4).transpose(1, 0, 2).reshape(Mp, G * 4)[:M, :K // 32]


class DeviceView:
    """A non-owning device pointer (a state tensor)."""

    def __init__(self, ptr: int, nbytes: int):
        self.ptr, self.nbytes = ptr, nbytes


class DeviceBuffer:
    """A device allocation owned by a Context."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = c_void_p()
        check(LIB.s3e_malloc(ctx.handle, max(self.nbytes, 1), ctypes.byref(p)), "s3e_malloc")
        self.ptr = p.value

    def upload(self, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(LIB.s3e_memcpy_h2d(self.ctx.handle, self.ptr, arr.ctypes.data, arr.nbytes), "h2d")
        return self

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(LIB.s3e_memcpy_d2h(self.ctx.handle, out.ctypes.data, self.ptr, out.nbytes), "d2h")
        return out

    def free(self) -> None:
        if self.ptr:
            LIB.s3e_free(self.ctx.handle, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weight:
    def __init__(self, ctx: "Context", ggml_type: int, K: int, N: int, data: np.ndarray):
        self.ctx = ctx
        data = np.ascontiguousarray(data)
        h = c_void_p()
        check(LIB.s3e_weight_upload(ctx.handle, ggml_type, K, N, data.ctypes.data, data.nbytes, ctypes.byref(h)),
              "s3e_weight_upload")
        self.handle = h.value
        self.K, self.N, self.type = K, N, ggml_type

    def info(self):
        out = (c_int64 * 4)()
        check(LIB.s3e_weight_info(self.handle, out), "s3e_weight_info")
        return list(out)

    def free(self):
        if self.handle:
            LIB.s3e_weight_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    def __init__(self, device: int = 0):
        h = c_void_p()
        check(LIB.s3e_ctx_create(device, ctypes.byref(h)), "s3e_ctx_create")
        self.handle = h.value

    def close(self):
        if self.handle:
            LIB.s3e_ctx_destroy(self.handle)
            self.handle = None

    def sync(self):
        check(LIB.s3e_ctx_sync(self.handle), "s3e_ctx_sync")

    @property
    def stream(self) -> int:
        return LIB.s3e_ctx_stream(self.handle)

    def buffer(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, arr: np.ndarray) -> DeviceBuffer:
        arr = np.ascontiguousarray(arr)
        return DeviceBuffer(self, arr.nbytes).upload(arr)

    def preprocess_image(self, hwc: DeviceBuffer, width: int, height: int, img_size: int, norm: int,
                         chw: DeviceBuffer):
        """Resize + normalise a device-resident HWC uint8 image into CHW f32
        (norm: NORM_SAM3 or NORM_IMAGENET)."""
        check(LIB.s3e_preprocess_image(self.handle, hwc.ptr, width, height, img_size, norm, chw.ptr),
              "s3e_preprocess_image")

    def weight(self, ggml_type: int, K: int, N: int, data: np.ndarray) -> Weight:
        return Weight(self, ggml_type, K, N, data)

    def mul_mat_noalloc(self, w: Weight, X: DeviceBuffer, M: int, Y: DeviceBuffer, bias: DeviceBuffer | None = None):
        check(LIB.s3e_mul_mat_noalloc(self.handle, w.handle, X.ptr, M, bias.ptr if bias else None, Y.ptr),
              "s3e_mul_mat_noalloc")

    def mul_mat(self, w: Weight, X: DeviceBuffer, M: int, Y: DeviceBuffer, bias: DeviceBuffer | None = None):
        check(LIB.s3e_mul_mat(self.handle, w.handle, X.ptr, M, bias.ptr if bias else None, Y.ptr), "s3e_mul_mat")

    def quantize_rows(self, vdt: int, X: DeviceBuffer, M: int, K: int, qs: DeviceBuffer,
                      d: DeviceBuffer | None, s: DeviceBuffer | None):
        check(LIB.s3e_quantize_rows(self.handle, vdt, X.ptr, M, K, qs.ptr, d.ptr if d else None,
                                    s.ptr if s else None), "s3e_quantize_rows")

    def mul_mat_q(self, w: Weight, xq: DeviceBuffer, d: DeviceBuffer | None, s: DeviceBuffer | None, M: int,
                  Y: DeviceBuffer, bias: DeviceBuffer | None = None):
        check(LIB.s3e_mul_mat_q(self.handle, w.handle, xq.ptr, d.ptr if d else None, s.ptr if s else None, M,
                                bias.ptr if bias else None, Y.ptr), "s3e_mul_mat_q")

    def mul_mat_q_f6(self, w: Weight, xq: DeviceBuffer, d: DeviceBuffer, M: int, Y: DeviceBuffer,
                     bias: DeviceBuffer | None = None):
        check(LIB.s3e_mul_mat_q_f6(self.handle, w.handle, xq.ptr, d.ptr, M, bias.ptr if bias else None, Y.ptr),
              "s3e_mul_mat_q_f6")

    def mul_mat_q_batch(self, ws, xqs, ds, ss, M: int, biases, Ys):
        """Independent small-M products in one launch (lists of equal length;
        ds / ss / biases may be None or hold None entries)."""
        n = len(ws)
        arr = lambda items: (c_void_p * n)(*[(x.ptr if hasattr(x, "ptr") else x) if x is not None else None
                                             for x in items])
        none = [None] * n
        check(LIB.s3e_mul_mat_q_batch(self.handle, n, (c_void_p * n)(*[w.handle for w in ws]), arr(xqs),
                                      arr(ds or none), arr(ss or none), M, arr(biases or none), arr(Ys)),
              "s3e_mul_mat_q_batch")

    def copy(self, dst: DeviceBuffer, src: DeviceBuffer, nbytes: int):
        check(LIB.s3e_copy(self.handle, dst.ptr, src.ptr, nbytes), "s3e_copy")

    def layer_norm(self, x: DeviceBuffer, rows: int, n: int, eps: float, w: DeviceBuffer | None,
                   b: DeviceBuffer | None, y: DeviceBuffer):
        check(LIB.s3e_layer_norm(self.handle, x.ptr, rows, n, c_float(eps), w.ptr if w else None,
                                 b.ptr if b else None, y.ptr), "s3e_layer_norm")

    def flash_attn_ext(self, q: DeviceBuffer, q_nb, k: DeviceBuffer, k_nb, v: DeviceBuffer, v_nb,
                       D: int, Nq: int, Nkv: int, nh: int, B: int, scale: float, o: DeviceBuffer,
                       prec: int = PREC_F32):
        a = lambda nb: (c_int64 * 4)(*[int(x) for x in nb])
        check(LIB.s3e_flash_attn_ext(self.handle, q.ptr, a(q_nb), k.ptr, a(k_nb), v.ptr, a(v_nb),
                                     D, Nq, Nkv, nh, B, c_float(scale), prec, o.ptr), "s3e_flash_attn_ext")

    def probe_stream(self, mode: int, dst: DeviceBuffer | None, src: DeviceBuffer | None, nbytes: int):
        check(LIB.s3e_probe_stream(self.handle, mode, dst.ptr if dst else None, src.ptr if src else None, nbytes),
              "s3e_probe_stream")

    def probe_mfma(self, kind: int, iters: int, waves_per_simd: int = 2):
        check(LIB.s3e_probe_mfma(self.handle, kind, iters, waves_per_simd), "s3e_probe_mfma")

    def flash_attn_ext_f16(self, q: DeviceBuffer, q_nb, k: DeviceBuffer, k_nb, v: DeviceBuffer, v_nb,
                           D: int, Nq: int, Nkv: int, nh: int, B: int, scale: float, o: DeviceBuffer):
        a = lambda nb: (c_int64 * 4)(*[int(x) for x in nb])
        check(LIB.s3e_flash_attn_ext_f16(self.handle, q.ptr, a(q_nb), k.ptr, a(k_nb), v.ptr, a(v_nb),
                                         D, Nq, Nkv, nh, B, c_float(scale), o.ptr), "s3e_flash_attn_ext_f16")

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    def __init__(self, ctx: Context, path: str):
        self.ctx = ctx
        h = c_void_p()
        check(LIB.s3e_model_load(ctx.handle, path.encode(), ctypes.byref(h)), "s3e_model_load")
        self.handle = h.value
        hp = (c_int32 * 16)()
        check(LIB.s3e_model_hparams(self.handle, hp), "s3e_model_hparams")
        self.hparams = list(hp)
        self.img_size, self.patch, self.E, self.depth = hp[0], hp[1], hp[2], hp[3]
        self.grid = hp[13]
        self.neck_dim, self.necks = hp[14], hp[15]  # necks: bit 0 tracker, bit 1 detector
        self.model_type = LIB.s3e_model_type(self.handle)  # 0 SAM 3, 1 SAM 3 visual-only, 2 SAM 2
        md = (c_int32 * 4)()
        self.mem_attn = tuple(md) if LIB.s3e_mem_attn_dims(self.handle, md) == 0 else None  # (L, D, MD, FFN)
        self.is_sam2 = self.model_type == 2

    def free(self):
        if self.handle:
            LIB.s3e_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class State:
    def __init__(self, ctx: Context, model: Model, img_size: int = 0):
        """img_size: the image size this state encodes (0: the model's own;
        SAM 2 files accept any multiple of 32)."""
        self.ctx, self.model = ctx, model
        h = c_void_p()
        check(LIB.s3e_state_create_sized(ctx.handle, model.handle, int(img_size), ctypes.byref(h)),
              "s3e_state_create_sized")
        self.handle = h.value

    def encode_chw(self, chw: DeviceBuffer):
        check(LIB.s3e_encode_chw(self.handle, chw.ptr), "s3e_encode_chw")

    def encode_chw_host(self, chw: np.ndarray):
        chw = np.ascontiguousarray(chw, dtype=np.float32)
        check(LIB.s3e_encode_chw_host(self.handle, chw.ctypes.data), "s3e_encode_chw_host")
        self.ctx.sync()

    def encode_image_u8(self, hwc: np.ndarray):
        hwc = np.ascontiguousarray(hwc, dtype=np.uint8)
        check(LIB.s3e_encode_image_u8(self.handle, hwc.ctypes.data, hwc.shape[1], hwc.shape[0]),
              "s3e_encode_image_u8")

    def prefix(self, chw: DeviceBuffer, x: DeviceBuffer):
        check(LIB.s3e_vit_prefix(self.handle, chw.ptr, x.ptr), "s3e_vit_prefix")

    def block(self, idx: int, x: DeviceBuffer):
        check(LIB.s3e_vit_block(self.handle, idx, x.ptr), "s3e_vit_block")

    def run_neck(self, x: DeviceBuffer):
        check(LIB.s3e_run_neck(self.handle, x.ptr), "s3e_run_neck")

    def block_stage(self, idx: int, stage: int, x: np.ndarray, ne) -> tuple:
        """Block sub-stage hook on host data x of ggml shape ne → (output, out_ne);
        the input is uploaded and the output downloaded around the device call."""
        return self._stage(lambda *a: LIB.s3e_vit_block_stage(self.handle, idx, stage, *a), x, ne,
                           "s3e_vit_block_stage")

    def prefix_stage(self, stage: int, x: np.ndarray, ne) -> tuple:
        return self._stage(lambda *a: LIB.s3e_vit_prefix_stage(self.handle, stage, *a), x, ne,
                           "s3e_vit_prefix_stage")

    def _stage(self, fn, x, ne, what):
        ine, one = (c_int64 * 4)(*ne), (c_int64 * 4)()
        check(fn(None, ine, None, one), what)
        n = one[0] * one[1] * one[2] * one[3]
        xd = self.ctx.to_device(np.ascontiguousarray(x, dtype=np.float32))
        yd = self.ctx.buffer(4 * n)
        check(fn(xd.ptr, ine, yd.ptr, one), what)
        self.ctx.sync()
        return yd.download(np.float32, (n,)), tuple(int(v) for v in one)

    def mem_attn(self, curr, src_pos, N: int, prompt, prompt_pos, M_total: int, n_ptr: int, rope_q, rope_k, out):
        """Memory attention on device buffers (s3e_mem_attn)."""
        p = lambda b: None if b is None else (b.ptr if hasattr(b, "ptr") else b)
        check(LIB.s3e_mem_attn(self.handle, p(curr), p(src_pos), N, p(prompt), p(prompt_pos), M_total, n_ptr,
                               p(rope_q), p(rope_k), p(out)), "s3e_mem_attn")

    def hiera_block(self, idx: int, x, H: int, W: int, y):
        """Hiera block idx on device rows x ([H·W][dim_in]) into y."""
        xp = x.ptr if hasattr(x, "ptr") else x
        yp = y.ptr if hasattr(y, "ptr") else y
        check(LIB.s3e_hiera_block(self.handle, idx, xp, H, W, yp), "s3e_hiera_block")

    def device_view(self, name: str = "vit_output") -> DeviceView:
        ne = (c_int64 * 4)()
        check(LIB.s3e_state_tensor_info(self.handle, name.encode(), ne), "s3e_state_tensor_info")
        p = LIB.s3e_state_tensor_device(self.handle, name.encode())
        return DeviceView(p, 4 * ne[0] * ne[1] * ne[2] * ne[3])

    def tensor(self, name: str = "vit_output") -> np.ndarray:
        ne = (c_int64 * 4)()
        check(LIB.s3e_state_tensor_info(self.handle, name.encode(), ne), "s3e_state_tensor_info")
        n = ne[0] * ne[1] * ne[2] * ne[3]
        out = np.empty(n, dtype=np.float32)
        check(LIB.s3e_state_tensor_get(self.handle, name.encode(), out.ctypes.data, n), "s3e_state_tensor_get")
        return out.reshape(ne[2] * ne[1], ne[0])

    def free(self):
        if self.handle:
            LIB.s3e_state_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---- HIP events on the engine's stream (timing) -----------------------------
class HipEvents:
    """hipEvent timing on an arbitrary stream, through libamdhip64."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [POINTER(c_void_p)]
        self.hip.hipEventRecord.argtypes = [c_void_p, c_void_p]
        self.hip.hipEventSynchronize.argtypes = [c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [POINTER(c_float), c_void_p, c_void_p]
        self.hip.hipEventDestroy.argtypes = [c_void_p]

    def create(self):
        e = c_void_p()
        if self.hip.hipEventCreate(ctypes.byref(e)) != 0:
            raise S3EError("hipEventCreate failed")
        return e.value

    def record(self, ev, stream):
        if self.hip.hipEventRecord(ev, stream) != 0:
            raise S3EError("hipEventRecord failed")

    def elapsed_ms(self, e0, e1) -> float:
        self.hip.hipEventSynchronize(e1)
        ms = c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), e0, e1) != 0:
            raise S3EError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self, ev):
        self.hip.hipEventDestroy(ev)
