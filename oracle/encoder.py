"""CPU restatement of the reference's encoder self-attention block. TEST INFRASTRUCTURE ONLY:
used by tests/ and never by the ffai_amd product path.

Follows EncoderAttention (crates/ffai-mercury/src/asr/text_decoder.rs:1009-1139):
  * prescale_key  -- load (:1039-1050): the key weight times head_dim^-0.5
  * encoder_attention -- forward (:1059-1139): q = x Wq^T + bq, k^T = Wk_scaled x^T (no bias),
    v = x Wv^T + bv, heads split, softmax(q k^T) v with no further scale, heads merged,
    out = merged Wo^T + bo; batch items independent (:1069-1076)
Computed in float64. `store` optionally rounds the intermediates the device keeps in a 16-bit
dtype (q, k^T, v and the merged attention output) to that dtype, so that a comparison measures
arithmetic rather than storage rounding.
"""

from __future__ import annotations

import numpy as np

from .kvcache import round_to


def prescale_key(wk: np.ndarray, n_head: int) -> np.ndarray:
    return (wk.astype(np.float64) * (wk.shape[0] // n_head) ** -0.5).astype(np.float32)


def encoder_attention(x, wq, bq, wk_scaled, wv, bv, wo, bo, n_head: int, store: str | None = None):
    """x (b, t, n) -> (b, t, n), float32."""
    rnd = (lambda a: round_to(a, store).astype(np.float64)) if store else (lambda a: a)
    x = x.astype(np.float64)
    b, t, n = x.shape
    hd = n // n_head
    q = rnd(x @ wq.astype(np.float64).T + bq.astype(np.float64))
    kt = rnd(np.einsum("oi,bti->bot", wk_scaled.astype(np.float64), x))   # (b, n, t)
    v = rnd(x @ wv.astype(np.float64).T + bv.astype(np.float64))
    qh = q.reshape(b, t, n_head, hd).transpose(0, 2, 1, 3)                 # (b, h, t, hd)
    kh = kt.reshape(b, n_head, hd, t)                                      # (b, h, hd, t)
    vh = v.reshape(b, t, n_head, hd).transpose(0, 2, 1, 3)
    s = qh @ kh
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    merged = rnd((p @ vh).transpose(0, 2, 1, 3).reshape(b, t, n))
    return (merged @ wo.astype(np.float64).T + bo.astype(np.float64)).astype(np.float32)
