"""Argmax token identity on downstream logits (GPU attention vs the CPU oracle).

Real Whisper weights are not available here, so the logit head is SYNTHETIC and seeded:
logits = (O_merged + residual) @ W_vocab with W_vocab ~ N(0, 1/d) of shape (d, 51864) (the
whisper vocabulary size) and residual ~ N(0, 1). For each position the token argmax of the logits
computed from the GPU attention output must equal the one computed from the oracle's output; the
logits themselves are compared in float64 on the host. This checks that the attention error stays
far below the decision margins a vocabulary projection cares about.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from ffai_amd import flash_attn as fa
from tests.helpers import randn, round_bf16

pytestmark = pytest.mark.gpu

VOCAB = 51864


def _dev(x: np.ndarray, dtype, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def _head(d: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((d, VOCAB)) / np.sqrt(d)).astype(np.float32)


def _argmax_identity(o_gpu: np.ndarray, o_ref: np.ndarray, w: np.ndarray, seed: int):
    """o_*: (positions, d). Returns (#positions, #mismatches, min top-2 margin)."""
    rng = np.random.default_rng(seed)
    resid = rng.standard_normal(o_ref.shape).astype(np.float32)
    lg = (o_gpu.astype(np.float32) + resid) @ w
    lr = (o_ref.astype(np.float32) + resid) @ w
    top = np.argmax(lr, axis=1)
    mism = int(np.sum(np.argmax(lg, axis=1) != top))
    part = np.partition(lr, -2, axis=1)
    margin = float(np.min(part[:, -1] - part[:, -2]))
    return lr.shape[0], mism, margin


def test_argmax_identity_tiny_encoder_f32(gpu):
    """whisper-tiny encoder layer (f32, 6 heads, T=1500, merged output): 1500 positions."""
    rng = np.random.default_rng(101)
    h, t = 6, 1500
    q = randn(rng, (1, h, t, 64)) * np.float32(0.125)
    kt, v = randn(rng, (1, h, 64, t)), randn(rng, (1, h, t, 64))
    out = fa.attend_merged(_dev(q, torch.float32, gpu), _dev(kt, torch.float32, gpu),
                           _dev(v, torch.float32, gpu))
    got = out.cpu().numpy()[0]                        # (T, H*64)
    want = oracle.attend_merged(q, kt, v)[0]
    n, mism, margin = _argmax_identity(got, want, _head(h * 64, 7), 8)
    print(f"tiny encoder argmax: {n} positions, {mism} mismatches, min margin {margin:.3e}")
    assert mism == 0


def test_argmax_identity_beam_decode_bf16(gpu):
    """Beam-5 whisper-medium decode step, 8 layers: cross-attention over 1500 shared frames and
    self-attention over ragged caches, bf16 K/V, f32 outputs; 5 beams x 8 layers x 2 sites."""
    rng = np.random.default_rng(202)
    beams, h, d, t_enc, cap = 5, 16, 64, 1500, 448
    w = _head(h * d, 9)
    gots, wants = [], []
    for layer in range(8):
        q = round_bf16(randn(rng, (beams, h, 1, d)))
        kt = round_bf16(randn(rng, (1, h, d, t_enc)))
        v = round_bf16(randn(rng, (1, h, t_enc, d)))
        o = torch.empty(beams, h, 1, d, dtype=torch.float32, device=gpu)
        fa.attention(_dev(q, torch.bfloat16, gpu).permute(2, 1, 0, 3), _dev(kt, torch.bfloat16, gpu),
                     _dev(v, torch.bfloat16, gpu), k_transposed=True, scale=0.125,
                     out=o.permute(2, 1, 0, 3))
        want = np.swapaxes(oracle.attend_general(np.swapaxes(q, 0, 2), kt, v, k_transposed=True,
                                                 scale=0.125), 0, 2)
        gots.append(o.cpu().numpy().reshape(beams, h * d))
        wants.append(want.reshape(beams, h * d))

        lens = rng.integers(1, cap + 1, size=beams).astype(np.int32)
        qs = round_bf16(randn(rng, (beams, h, 1, d)))
        ks = round_bf16(randn(rng, (beams, h, cap, d)))
        vs = round_bf16(randn(rng, (beams, h, cap, d)))
        os_ = fa.attention(_dev(qs, torch.bfloat16, gpu), _dev(ks, torch.bfloat16, gpu),
                           _dev(vs, torch.bfloat16, gpu), scale=0.125,
                           kv_lens=torch.from_numpy(lens).to(gpu), out_dtype=torch.float32)
        wants.append(oracle.attend_general(qs, ks, vs, k_transposed=False, scale=0.125,
                                           kv_lens=lens).reshape(beams, h * d))
        gots.append(os_.cpu().numpy().reshape(beams, h * d))
    n, mism, margin = _argmax_identity(np.concatenate(gots), np.concatenate(wants), w, 10)
    print(f"beam decode argmax: {n} positions, {mism} mismatches, min margin {margin:.3e}")
    assert mism == 0


def test_argmax_identity_large_v3_rows(gpu):
    """whisper-large-v3 encoder layer shape (B16 H20 T1500 bf16): 96 sampled (batch, row)
    positions of the merged (T, 1280) output against the float64 closed form."""
    from oracle import textbook

    b, h, t, d = 16, 20, 1500, 64
    g = torch.Generator(device="cpu").manual_seed(303)
    q = torch.randn(b, h, t, d, generator=g).to(torch.bfloat16)
    kt = torch.randn(b, h, d, t, generator=g).to(torch.bfloat16)
    v = torch.randn(b, h, t, d, generator=g).to(torch.bfloat16)
    out = fa.attention(q.to(gpu), kt.to(gpu), v.to(gpu), k_transposed=True, scale=0.125,
                       out_dtype=torch.float32).cpu().numpy()
    rng = np.random.default_rng(303)
    rows = np.sort(rng.choice(t, size=32, replace=False))
    bi = [0, 9, 15]
    want = textbook.attention(q[bi].float().numpy(), kt[bi].float().numpy(),
                              v[bi].float().numpy(), k_transposed=True, scale=0.125, rows=rows)
    got = out[bi][:, :, rows]                               # (3, H, 32, D)
    merge = lambda x: np.transpose(x, (0, 2, 1, 3)).reshape(-1, h * d)
    n, mism, margin = _argmax_identity(merge(got), merge(want), _head(h * d, 11), 12)
    print(f"large-v3 argmax: {n} positions, {mism} mismatches, min margin {margin:.3e}")
    assert mism == 0
