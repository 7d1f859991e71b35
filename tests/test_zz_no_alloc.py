"""s3e_mul_mat_noalloc (the allocation-free s3e_mul_mat, for callers that
cannot allocate) against s3e_mul_mat through the C ABI.

Above 64 rows both run the same conversion and GEMM kernels, so the outputs
must be identical bit for bit; at 64 rows or fewer s3e_mul_mat streams the
weight on the small-M kernel and the two differ only in fp32 summation order
(relative L2 ≤ 1e-6).  Two calls in a row — the C4 fc2 shape, then a
smaller product with another K — check that the scratch array's leftovers
from the first call do not reach the second.  A product too large for the
array is refused.  The call is also captured into a HIP graph on the
context's stream in global capture mode, where a hipMalloc, hipFree or
stream synchronisation inside the call would make the capture fail; the
graph is replayed three times, with eager calls on other inputs between the
replays, and every replay must equal the eager result bit for bit.
"""
import ctypes
from ctypes import POINTER, c_int, c_size_t, c_void_p

import numpy as np
import pytest

import oracle_lib as orc

pytestmark = pytest.mark.gpu

TYPES = [orc.Q4_0, orc.Q4_1, orc.Q8_0, orc.F16, orc.F32]


def _product(ctx, t, M, N, K, seed):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    return ctx.weight(t, K, N, orc.to_weight_bytes(t, W)), ctx.to_device(X), ctx.to_device(b)


@pytest.mark.parametrize("t", TYPES, ids=lambda t: {0: "f32", 1: "f16", 2: "q4_0", 3: "q4_1", 8: "q8_0"}[t])
def test_noalloc_matches_mul_mat(ctx, t):
    for k, (M, N, K) in enumerate([(5184, 1024, 4736), (300, 512, 1024), (40, 256, 1024)]):
        print(f"noalloc type {t}: M={M} N={N} K={K}", flush=True)
        w, Xd, bd = _product(ctx, t, M, N, K, 10 * t + k)
        ref, got = ctx.buffer(M * N * 4), ctx.buffer(M * N * 4)
        ctx.mul_mat(w, Xd, M, ref, bd)
        ctx.mul_mat_noalloc(w, Xd, M, got, bd)
        ctx.sync()
        a, r = got.download(np.float32, (M, N)), ref.download(np.float32, (M, N))
        if M > 64:
            assert np.array_equal(a, r), (M, N, K)
        else:
            assert orc.rel_l2(a, r) <= 1e-6, (M, N, K)
        w.free()


def test_noalloc_refuses_oversize(ctx):
    import s3e

    # F16: 10000 rows of K = 4096 convert to 82 MB, beyond the 64 MiB array
    M, N, K = 10000, 32, 4096
    w, Xd, bd = _product(ctx, orc.F16, M, N, K, 1)
    Y = ctx.buffer(M * N * 4)
    with pytest.raises(s3e.S3EError):
        ctx.mul_mat_noalloc(w, Xd, M, Y, bd)
    # the same weight at a size that fits still works afterwards
    ref = ctx.buffer(100 * N * 4)
    ctx.mul_mat(w, Xd, 100, Y, bd)
    ctx.mul_mat_noalloc(w, Xd, 100, ref, bd)
    ctx.sync()
    assert np.array_equal(ref.download(np.float32, (100, N)), Y.download(np.float32, (100, N)))
    w.free()


class _Graphs:
    """HIP stream capture and graph replay through libamdhip64."""

    def __init__(self):
        h = ctypes.CDLL("libamdhip64.so")
        h.hipStreamBeginCapture.argtypes = [c_void_p, c_int]
        h.hipStreamEndCapture.argtypes = [c_void_p, POINTER(c_void_p)]
        h.hipGraphInstantiate.argtypes = [POINTER(c_void_p), c_void_p, c_void_p, c_void_p, c_size_t]
        h.hipGraphLaunch.argtypes = [c_void_p, c_void_p]
        h.hipGraphExecDestroy.argtypes = [c_void_p]
        h.hipGraphDestroy.argtypes = [c_void_p]
        self.h = h

    def capture(self, stream, fn):
        GLOBAL = 0  # hipStreamCaptureModeGlobal: unsafe calls from any thread fail the capture
        assert self.h.hipStreamBeginCapture(stream, GLOBAL) == 0
        err = None
        try:
            fn()
        except Exception as e:  # noqa: BLE001 - the capture must be ended either way
            err = e
        g = c_void_p()
        rc = self.h.hipStreamEndCapture(stream, ctypes.byref(g))
        if err is not None:
            raise err
        assert rc == 0 and g.value, f"hipStreamEndCapture returned {rc}"
        ex = c_void_p()
        assert self.h.hipGraphInstantiate(ctypes.byref(ex), g, None, None, 0) == 0
        return g, ex


@pytest.mark.parametrize("t", [orc.Q8_0, orc.Q4_0], ids=["q8_0", "q4_0"])
def test_noalloc_under_graph_capture(ctx, t):
    M, N, K = 300, 512, 1024
    print(f"noalloc graph capture type {t}: M={M} N={N} K={K}", flush=True)
    w, Xd, bd = _product(ctx, t, M, N, K, 77 + t)
    _, X2, _ = _product(ctx, t, M, N, K, 78 + t)
    ref, got, other = ctx.buffer(M * N * 4), ctx.buffer(M * N * 4), ctx.buffer(M * N * 4)
    ctx.mul_mat(w, Xd, M, ref, bd)
    ctx.sync()
    want = ref.download(np.float32, (M, N))
    gr = _Graphs()
    g, ex = gr.capture(ctx.stream, lambda: ctx.mul_mat_noalloc(w, Xd, M, got, bd))
    try:
        for rep in range(3):
            got.upload(np.full((M, N), np.nan, np.float32))
            assert gr.h.hipGraphLaunch(ex, ctx.stream) == 0
            ctx.sync()
            assert np.array_equal(got.download(np.float32, (M, N)), want), rep
            # eager work on other inputs between replays: the shared scratch
            # array holds its leftovers when the next replay starts
            ctx.mul_mat_noalloc(w, X2, M, other, bd)
            ctx.sync()
    finally:
        gr.h.hipGraphExecDestroy(ex)
        gr.h.hipGraphDestroy(g)
    w.free()
