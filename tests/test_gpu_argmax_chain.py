"""Argmax token identity on logits the device computes: a whisper-medium beam-5 decode step's
attention half chained on the GPU, against the same chain on the oracle.

GPU chain, per position (5 beams, 16 heads x 64, d 1024, the 51865-token vocabulary):
  self-attention  (decode over each beam's cache)           -> merged (5, 1024)
  h1 = x + F16Gemv(W_o_self)(merged)                          (out-projection, residual)
  q_x = F16Gemv(W_q_cross)(h1) * 1/8                          (the cross query, pre-scaled)
  cross-attention (decode over the window's shared K/V)     -> merged (5, 1024)
  h2 = h1 + F16Gemv(W_o_cross)(merged)
  logits = Int8Vocab(E)(h2); token = argmax                   (decoder.rs:786-812,
                                                               vocab_int8.rs:202-262)
Oracle chain: oracle.attend_general (the reference's tiling, f32), gemv_f16_exact (float64 dots
of the same f16 weights, rounded to f32), vocab_quantize + vocab_logits (the reference's int8
arithmetic, bit for bit). The layer's norms and MLP are left out: they are not on this path.

Two precisions: the reference's own (f32 queries; f32 self-attention caches, f16 cross-attention
cache: text_decoder.rs:771-793, the f32 decode kernel) and this build's device caches (bf16
queries and caches, the 16-bit decode kernel). Weights and inputs are SYNTHETIC and seeded (real
Whisper weights are not available here): W ~ N(0, 1/d) in f16, E ~ N(0, 1/d), x ~ N(0, 1), K/V
~ N(0, 1), cache lengths uniform in [1, 448].

Criterion: with eps the largest difference between the two chains' logits, a token can only
differ where the oracle's top-2 margin is below 2 eps; every token with a larger margin must
match, and eps must stay below a stated bound (1e-3 for the f32 chain, 6e-2 for the bf16 one:
the attention's own bars, 1e-4 and 2e-2, carried through an out-projection of unit gain). The f32
chain must match every token. The test prints the mismatches, eps and the near-ties.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import gemv as og
from oracle import kvcache as okv
from ffai_amd import flash_attn as fa
from ffai_amd.gemv import F16Gemv, Int8Vocab

pytestmark = pytest.mark.gpu

BEAMS, H, HD, D_MODEL, VOCAB, T_ENC, CAP = 5, 16, 64, 1024, 51865, 1500, 448
POSITIONS = 16


@pytest.fixture(scope="module")
def head(gpu):
    rng = np.random.default_rng(90)
    w = [(rng.standard_normal((D_MODEL, D_MODEL)) / np.sqrt(D_MODEL)).astype(np.float16)
         for _ in range(3)]
    emb = (rng.standard_normal((VOCAB, D_MODEL)) / np.sqrt(D_MODEL)).astype(np.float32)
    iv = Int8Vocab(torch.from_numpy(emb).to(gpu))
    q, sc, corr = og.vocab_quantize(emb, 32)
    gemvs = [F16Gemv(torch.from_numpy(x).to(gpu)) for x in w]
    return w, gemvs, iv, (q, sc, corr)


def _heads(x: np.ndarray) -> np.ndarray:  # (beams, d) -> (beams, H, 1, HD)
    return np.ascontiguousarray(x.reshape(BEAMS, H, 1, HD))


@pytest.mark.parametrize("precision", ["reference_f32", "device_bf16"])
def test_decode_step_argmax_on_device_logits(gpu, head, precision):
    w, gemvs, iv, (vq, vsc, vcorr) = head
    ref = precision == "reference_f32"
    store = None if ref else "bf16"
    kv_self_t = torch.float32 if ref else torch.bfloat16
    kv_x_t = torch.float16 if ref else torch.bfloat16
    q_t = torch.float32 if ref else torch.bfloat16
    rnd = (lambda a: a) if ref else (lambda a: okv.round_to(a, "bf16"))
    rnd_x = (lambda a: a.astype(np.float16).astype(np.float32)) if ref else rnd
    dev = lambda a, t: torch.from_numpy(np.ascontiguousarray(a)).to(gpu, t)
    mismatches, margins, n, eps, guarded = 0, [], 0, 0.0, 0
    for pos in range(POSITIONS):
        rng = np.random.default_rng(900 + pos)
        x = rng.standard_normal((BEAMS, D_MODEL)).astype(np.float32)
        lens = rng.integers(1, CAP + 1, BEAMS).astype(np.int32)
        q_s = rnd(rng.standard_normal((BEAMS, H, 1, HD)).astype(np.float32) / 8)
        k_s = rnd(rng.standard_normal((BEAMS, H, CAP, HD)).astype(np.float32))
        v_s = rnd(rng.standard_normal((BEAMS, H, CAP, HD)).astype(np.float32))
        kt_x = rnd_x(rng.standard_normal((1, H, HD, T_ENC)).astype(np.float32))
        v_x = rnd_x(rng.standard_normal((1, H, T_ENC, HD)).astype(np.float32))

        # ---- GPU chain
        o_s = torch.empty(BEAMS, H, 1, HD, device=gpu)
        fa.attention(dev(q_s, q_t), dev(k_s, kv_self_t), dev(v_s, kv_self_t),
                     kv_lens=dev(lens, torch.int32), out=o_s)
        h1 = dev(x, torch.float32) + gemvs[0](o_s.reshape(BEAMS, D_MODEL))
        qx = gemvs[1](h1) * 0.125
        qx_in = qx.to(q_t).reshape(BEAMS, H, 1, HD)
        o_x = torch.empty(BEAMS, H, 1, HD, device=gpu)
        # the beams share the window's K/V (batch stride 0); the f32 path runs one row per head
        kt_d = dev(kt_x, kv_x_t).expand(BEAMS, H, HD, T_ENC)
        v_d = dev(v_x, kv_x_t).expand(BEAMS, H, T_ENC, HD)
        fa.attention(qx_in, kt_d, v_d, k_transposed=True, out=o_x)
        h2 = h1 + gemvs[2](o_x.reshape(BEAMS, D_MODEL))
        logits = iv(h2)
        tok_gpu = logits.argmax(dim=1).cpu().numpy()

        # ---- oracle chain (the same values where the device rounds its inputs to 16 bits)
        f32 = lambda a: np.asarray(a, np.float64).astype(np.float32)
        ro_s = oracle.attend_general(q_s, k_s, v_s, k_transposed=False, kv_lens=lens)
        rh1 = f32(x.astype(np.float64) + og.gemv_f16_exact(w[0], ro_s.reshape(BEAMS, D_MODEL)))
        rqx = f32(og.gemv_f16_exact(w[1], rh1)) * np.float32(0.125)
        rqx = rnd(rqx) if not ref else rqx
        ro_x = oracle.attend_general(_heads(rqx), np.broadcast_to(kt_x, (BEAMS, H, HD, T_ENC)),
                                     np.broadcast_to(v_x, (BEAMS, H, T_ENC, HD)),
                                     k_transposed=True)
        rh2 = f32(rh1.astype(np.float64) + og.gemv_f16_exact(w[2], ro_x.reshape(BEAMS, D_MODEL)))
        rlog = og.vocab_logits(vq, vsc, vcorr, rh2, 32)
        tok_ref = rlog.argmax(axis=1)

        top2 = np.sort(rlog, axis=1)[:, -2:]
        margin = top2[:, 1] - top2[:, 0]
        e = float(np.abs(logits.cpu().numpy().astype(np.float64) - rlog).max())
        eps = max(eps, e)
        clear = margin > 2 * e  # a token that no logit difference of size e can flip
        assert (tok_gpu[clear] == tok_ref[clear]).all(), (pos, margin, e)
        guarded += int(clear.sum())
        mismatches += int((tok_gpu != tok_ref).sum())
        margins.extend(margin.tolist())
        n += BEAMS
        if ref:  # f32 attention: the device's residual stream tracks the oracle's closely
            assert np.abs(h2.cpu().numpy() - rh2).max() < 1e-3
    print(f"argmax chain ({precision}): {n} tokens, {mismatches} mismatches, logit difference "
          f"{eps:.2e}, {n - guarded} tokens within 2x of it (near-ties), smallest top-2 margin "
          f"{min(margins):.4f}")
    assert eps < (1e-3 if ref else 6e-2)
    if ref:
        assert mismatches == 0
