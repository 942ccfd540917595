"""GPU parity of the decoder's multi-token (prompt) steps through the fused kernel, against the
oracle's restatement of the reference's unfused path for them (oracle/kvcache.py):

* self-attention, Attention::forward_self (text_decoder.rs:652-679): the cache grows by the
  step's rows and a multi-token step is masked by causal_mask(q_len, k_len, offset)
  (:902-923), then softmax(q s^2 k^T + mask) v (:863-867);
* cross-attention with 1 < q_len < keys (previous-window conditioning, :799-816), which the
  reference's fused kernel declines and runs as three ops on K/V widened from the f16 cache.

Shapes are whisper-medium's decoder (16 heads, head_dim 64) with the reference's longest
prompt: 223 previous-text tokens + the previous-text marker + 4 start tokens = 228
(decoder.rs:488-498)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kvcache as okv
from ffai_amd import flash_attn as fa
from ffai_amd.kv_cache import KVCache, self_attention_step
from tests.helpers import TOL_BF16, TOL_F32, max_abs, randn

pytestmark = pytest.mark.gpu

HEADS, D, CAP, PROMPT = 16, 64, 448, 228
SCALE = D ** -0.5


def _dev(x, dtype, device):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def _rows(rng, t):
    return okv.round_to(randn(rng, (1, t, HEADS * D)), "bf16")


def _reference_self(ref_k, ref_v, q, offset):
    """forward_self's unfused path on the oracle's raw caches: split, mask if q_len > 1, attend."""
    k, v = okv.split_heads(ref_k, HEADS), okv.split_heads(ref_v, HEADS)
    q_len = q.shape[2]
    mask = okv.causal_mask(q_len, k.shape[2], offset) if q_len > 1 else None
    return okv.three_op_attend(q, k, v, SCALE, mask)


def test_prompt_then_single_tokens(gpu):
    """Step 0: the 228-token prompt at offset 0 (causal); then three one-token steps at offsets
    228, 229, 230 (no mask), each appended in place and attended over the grown cache."""
    rng = np.random.default_rng(40)
    cache = KVCache(1, HEADS, CAP, D, torch.bfloat16, gpu)
    ref_k = ref_v = None
    offset = 0
    for q_len in (PROMPT, 1, 1, 1):
        nk, nv = _rows(rng, q_len), _rows(rng, q_len)
        q = okv.round_to(randn(rng, (1, HEADS, q_len, D)), "bf16")
        out = self_attention_step(cache, _dev(q, torch.bfloat16, gpu), _dev(nk, torch.bfloat16, gpu),
                                  _dev(nv, torch.bfloat16, gpu), offset, SCALE,
                                  out_dtype=torch.float32)
        ref_k, ref_v = okv.self_cache_append(ref_k, nk), okv.self_cache_append(ref_v, nv)
        want = _reference_self(ref_k, ref_v, q, offset)
        err = max_abs(out.cpu().numpy(), want)
        print(f"self step q_len {q_len} offset {offset}: {err:.3e}")
        assert err < TOL_BF16
        offset += q_len
    assert int(cache.lens[0]) == PROMPT + 3


def test_multi_token_step_at_an_offset(gpu):
    """A 3-token step appended after 5 cached positions (offset 5): query i sees keys 0..5+i."""
    rng = np.random.default_rng(41)
    cache = KVCache(1, HEADS, CAP, D, torch.bfloat16, gpu)
    k0, v0 = _rows(rng, 5), _rows(rng, 5)
    cache.append(_dev(k0, torch.bfloat16, gpu), _dev(v0, torch.bfloat16, gpu))
    nk, nv = _rows(rng, 3), _rows(rng, 3)
    q = okv.round_to(randn(rng, (1, HEADS, 3, D)), "bf16")
    out = self_attention_step(cache, _dev(q, torch.bfloat16, gpu), _dev(nk, torch.bfloat16, gpu),
                              _dev(nv, torch.bfloat16, gpu), 5, SCALE, out_dtype=torch.float32)
    want = _reference_self(okv.self_cache_append(k0, nk), okv.self_cache_append(v0, nv), q, 5)
    err = max_abs(out.cpu().numpy(), want)
    print(f"3 tokens at offset 5: {err:.3e}")
    assert err < TOL_BF16


def test_prompt_seeds_every_beam(gpu):
    """decode_beam runs the prompt once and every beam continues from it (decoder.rs:509-512):
    gather the one-slot prompt cache into five beam slots, then a one-token step per beam."""
    rng = np.random.default_rng(42)
    beams = 5
    prompt = KVCache(1, HEADS, CAP, D, torch.bfloat16, gpu)
    pk, pv = _rows(rng, PROMPT), _rows(rng, PROMPT)
    prompt.append(_dev(pk, torch.bfloat16, gpu), _dev(pv, torch.bfloat16, gpu))
    cache = KVCache(beams, HEADS, CAP, D, torch.bfloat16, gpu)
    cache.gather_from(prompt, torch.zeros(beams, dtype=torch.int32, device=gpu))
    assert (cache.lens.cpu().numpy() == PROMPT).all()
    nk = okv.round_to(randn(rng, (beams, 1, HEADS * D)), "bf16")
    nv = okv.round_to(randn(rng, (beams, 1, HEADS * D)), "bf16")
    q = okv.round_to(randn(rng, (beams, HEADS, 1, D)), "bf16")
    out = self_attention_step(cache, _dev(q, torch.bfloat16, gpu), _dev(nk, torch.bfloat16, gpu),
                              _dev(nv, torch.bfloat16, gpu), PROMPT, SCALE,
                              out_dtype=torch.float32).cpu().numpy()
    for b in range(beams):
        want = _reference_self(okv.self_cache_append(pk, nk[b:b + 1]),
                               okv.self_cache_append(pv, nv[b:b + 1]), q[b:b + 1], PROMPT)
        err = max_abs(out[b:b + 1], want)
        assert err < TOL_BF16, (b, err)


@pytest.mark.parametrize("q_dtype", ["f32", "bf16"])
def test_multi_token_cross_attention(gpu, q_dtype):
    """Previous-window conditioning: 228 query tokens over the window's 1500 encoder frames.
    f32 queries read the f16 cross cache (the reference's dtypes, its widened three-op path);
    bf16 queries read a bf16 cache (the all-16-bit device path)."""
    rng = np.random.default_rng(43)
    t_enc = 1500
    kv_dt = "f16" if q_dtype == "f32" else "bf16"
    kt = okv.round_to(randn(rng, (1, HEADS, D, t_enc)), kv_dt)
    v = okv.round_to(randn(rng, (1, HEADS, t_enc, D)), kv_dt)
    q = okv.round_to(randn(rng, (1, HEADS, PROMPT, D)), q_dtype)
    tq = torch.float32 if q_dtype == "f32" else torch.bfloat16
    tkv = torch.float16 if kv_dt == "f16" else torch.bfloat16
    out = fa.attention(_dev(q, tq, gpu), _dev(kt, tkv, gpu), _dev(v, tkv, gpu), k_transposed=True,
                       scale=SCALE, out_dtype=torch.float32)
    want = okv.three_op_attend(q, np.swapaxes(kt, 2, 3), v, SCALE)
    err = max_abs(out.cpu().numpy(), want)
    print(f"cross q_len {PROMPT} q {q_dtype} kv {kv_dt}: {err:.3e}")
    assert err < (TOL_F32 if q_dtype == "f32" else TOL_BF16)
