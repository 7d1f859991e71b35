"""Pins the oracle's memory attention (oracle/orc_memattn.c) before it is
trusted: sam3_build_mem_attn_graph (sam3.cpp:9224-9337) against a float64
torch restatement built from the weights read back from the model file.

The restatement follows the PyTorch module the reference graph ports (SAM 2's
MemoryAttentionLayer with RoPEAttention, one head): pre-norm self-attention
with RoPE on q and k, pre-norm cross-attention whose keys come from
memory + memory positions and whose values from memory alone, RoPE on the
spatial keys only (object-pointer tokens excluded), a ReLU FFN, residuals
after each, and a final LayerNorm; the input is curr + 0.1·pos.  RoPE here
is torch's complex multiplication (torch.view_as_complex), independent of
the oracle's pairwise formula, with the frequencies of the oracle's
sam3_compute_axial_cis (pinned by the RoPE known answers in test_oracle.py).

With an F32 model file every product in the oracle is an fp32 dot, so the
two agree to fp32 evaluation noise (relative L2 ≤ 1e-5).  A Q8_0 file adds
ggml's activation quantization; the oracle then stays within the Q8 noise
of the float64 result (≤ 2e-2), which checks that the quantized weights
are read and used.
"""
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle_lib as orc

H = 8          # tokens per side (N = 64)
FRAMES = 2     # memory frames (M_spatial = 128)
N_PTR = 8      # object-pointer tokens (two pointers of 4 tokens)


def t64(a):
    return torch.from_numpy(np.asarray(a, np.float64))


def _lin(tensors, name, x):
    w = _w(tensors, name + ".weight")
    return x @ w.T + _w(tensors, name + ".bias")


def _w(tensors, name):
    dt, ne, arr = tensors[name]
    if dt == 0:
        return t64(arr)
    # quantized record: dequantize through the oracle
    n = int(np.prod(ne))
    out = np.empty(n, np.float32)
    orc.LIB.orc_dequantize_row(dt, orc.ptr(np.ascontiguousarray(arr)), orc.ptr(out), n)
    return t64(out.reshape(tuple(reversed(ne))))


def _rope(x, freqs):
    """x [n][D] · (cos + i·sin) per pair, via torch complex numbers."""
    xc = torch.view_as_complex(x.reshape(x.shape[0], -1, 2).contiguous())
    fc = torch.view_as_complex(t64(freqs).reshape(x.shape[0], -1, 2).contiguous())
    return torch.view_as_real(xc * fc).reshape(x.shape)


def _attn(q, k, v):
    s = (q @ k.T) / np.sqrt(q.shape[1])
    return torch.softmax(s, dim=-1) @ v


def torch_mem_attn(tensors, L, curr, src_pos, prompt, prompt_pos, n_ptr, rope_q, rope_k):
    D = curr.shape[1]
    x = t64(curr) + 0.1 * t64(src_pos)
    mem, mpos = t64(prompt), t64(prompt_pos)
    msp = mem.shape[0] - n_ptr
    for l in range(L):
        p = f"mem_attn.layers.{l}."
        ln = lambda z, i: F.layer_norm(z, (D,), _w(tensors, p + f"norm{i}.weight"), _w(tensors, p + f"norm{i}.bias"),
                                       eps=1e-5)
        xn = ln(x, 1)
        q = _rope(_lin(tensors, p + "sa.q_proj", xn), rope_q)
        k = _rope(_lin(tensors, p + "sa.k_proj", xn), rope_q)
        v = _lin(tensors, p + "sa.v_proj", xn)
        x = x + _lin(tensors, p + "sa.out_proj", _attn(q, k, v))
        xn = ln(x, 2)
        q = _rope(_lin(tensors, p + "ca.q_proj", xn), rope_q)
        k = _lin(tensors, p + "ca.k_proj", mem + mpos)
        k = torch.cat([_rope(k[:msp], rope_k), k[msp:]])
        v = _lin(tensors, p + "ca.v_proj", mem)
        x = x + _lin(tensors, p + "ca.out_proj", _attn(q, k, v))
        xn = ln(x, 3)
        x = x + _lin(tensors, p + "linear2", torch.relu(_lin(tensors, p + "linear1", xn)))
    return F.layer_norm(x, (D,), _w(tensors, "mem_attn.norm.weight"), _w(tensors, "mem_attn.norm.bias"),
                        eps=1e-5).numpy()


def make_inputs(D, MD, seed=3, h=H, frames=FRAMES, n_ptr=N_PTR):
    rng = np.random.default_rng(seed)
    N = h * h
    curr = rng.standard_normal((N, D)).astype(np.float32)
    src_pos = orc.sinusoidal_pe_2d(h, h, D).reshape(N, D)
    prompt = rng.standard_normal((frames * N + n_ptr, MD)).astype(np.float32)
    pos64 = orc.sinusoidal_pe_2d(h, h, MD).reshape(N, MD)
    prompt_pos = np.concatenate([pos64] * frames + [rng.standard_normal((n_ptr, MD)).astype(np.float32) * 0.1])
    rope_q = orc.axial_cis(D, h, h)
    rope_k = np.concatenate([rope_q] * frames)
    return curr, src_pos, prompt, prompt_pos.astype(np.float32), rope_q, rope_k


@pytest.fixture(scope="module", params=["f32", "q8_0"])
def model(request, tmp_path_factory):
    import s3e

    p = str(tmp_path_factory.mktemp("ma") / f"ma_{request.param}.ggml")
    # a small Hiera with the memory attention of the SAM 2.1 models (D 256, MD 64, FFN 2048)
    s3e.synth_write_sam2(p, "hiera_t", img_size=64, ftype=request.param, seed=5, std=0.05, random_affine=True,
                         mem_attn_layers=2, embed_dim=32, stages=(1, 1, 1, 1), global_idx=(), window_spec=(4, 4, 2, 2),
                         bkg=(2, 2))
    h = orc.LIB.orc_model_load(p.encode())
    assert h, orc.LIB.orc_last_error()
    yield request.param, h, orc.read_model_file(p)
    orc.LIB.orc_model_free(h)


def test_dims(model):
    ft, h, tensors = model
    assert orc.mem_attn_dims(h) == (2, 256, 64, 2048)


def test_mem_attn_vs_torch(model):
    ft, h, tensors = model
    L, D, MD, FFN = orc.mem_attn_dims(h)
    args = make_inputs(D, MD)
    got = orc.mem_attn(h, *args[:4], N_PTR, *args[4:])
    ref = torch_mem_attn(tensors, L, *args[:4], N_PTR, *args[4:])
    rl = orc.rel_l2(got, ref)
    print(f"{ft}: rel_l2={rl:.3e} max_abs={orc.max_abs(got, ref):.3e}")
    assert rl <= (1e-5 if ft == "f32" else 2e-2)


@pytest.mark.parametrize("model", ["f32"], indirect=True)
def test_pointer_tokens_skip_rope(model):
    """A plant on the CPU: rotating the pointer keys as well must change the
    result (the excluded tail is observable), and leaving every key
    unrotated must too (the spatial keys are rotated).  A structure check,
    on the F32 file only."""
    ft, h, tensors = model
    L, D, MD, FFN = orc.mem_attn_dims(h)
    curr, src_pos, prompt, prompt_pos, rope_q, rope_k = make_inputs(D, MD)
    base = orc.mem_attn(h, curr, src_pos, prompt, prompt_pos, N_PTR, rope_q, rope_k)
    # pointer tokens treated as spatial (n_ptr = 0, rope over every key)
    rope_all = np.concatenate([rope_k, orc.axial_cis(D, 1, N_PTR)])
    alt = orc.mem_attn(h, curr, src_pos, prompt, prompt_pos, 0, rope_q, rope_all)
    assert orc.rel_l2(alt, base) > 1e-4
    ref_alt = torch_mem_attn(tensors, L, curr, src_pos, prompt, prompt_pos, 0, rope_q, rope_all)
    assert orc.rel_l2(alt, ref_alt) <= 1e-5
    # identity RoPE on the keys: differs from the rotated version
    ident = np.zeros_like(rope_k)
    ident[..., 0] = 1.0
    alt2 = orc.mem_attn(h, curr, src_pos, prompt, prompt_pos, N_PTR, rope_q, ident)
    assert orc.rel_l2(alt2, base) > 1e-4


@pytest.mark.parametrize("model", ["f32"], indirect=True)
def test_no_pointer_tokens(model):
    ft, h, tensors = model
    L, D, MD, FFN = orc.mem_attn_dims(h)
    curr, src_pos, prompt, prompt_pos, rope_q, rope_k = make_inputs(D, MD, n_ptr=0)
    got = orc.mem_attn(h, curr, src_pos, prompt, prompt_pos, 0, rope_q, rope_k)
    ref = torch_mem_attn(tensors, L, curr, src_pos, prompt, prompt_pos, 0, rope_q, rope_k)
    assert orc.rel_l2(got, ref) <= 1e-5
