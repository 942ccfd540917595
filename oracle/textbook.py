"""Float64 closed-form attention -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

``softmax(scale * Q K^T + mask) V`` evaluated in float64 with numpy, with no tiling and no
online rescaling: the definition the tiled kernels must agree with. The reference's own kernel
test compares against this closed form through candle's three-op path
(crates/ffai-mercury/src/asr/flash_attn.rs:1005-1021), and its causal mask is
``text_decoder.rs:902-923`` (key j hidden from query i iff j > offset + i).
"""

from __future__ import annotations

import numpy as np


def attention(q, k, v, *, k_transposed: bool = False, scale: float = 1.0, causal: bool = False,
              q_offset: int = 0, kv_lens=None, rows=None) -> np.ndarray:
    """q (B,Hq,Tq,D); k (B,Hkv,D,Tk) if k_transposed else (B,Hkv,Tk,D); v (B,Hkv,Tk,D).
    Hq must be a multiple of Hkv (query head h reads K/V head h // (Hq // Hkv)).
    ``rows`` optionally restricts the computed query rows (an index array into Tq); the result
    then has that many rows. Returns float64 (B,Hq,len(rows) or Tq,D). Fully masked rows are 0."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    if k_transposed:
        k = np.swapaxes(k, 2, 3)
    b, hq, tq, d = q.shape
    hkv, tk = k.shape[1], k.shape[2]
    assert hq % hkv == 0
    group = hq // hkv
    if rows is None:
        rows = np.arange(tq)
    rows = np.asarray(rows)
    out = np.zeros((b, hq, rows.size, d), np.float64)
    for bi in range(b):
        kb = tk if kv_lens is None else int(kv_lens[bi])
        for h in range(hq):
            hk = h // group
            s = (q[bi, h, rows] @ k[bi, hk, :kb].T) * scale
            if causal:
                j = np.arange(kb)[None, :]
                i = rows[:, None]
                s = np.where(j > q_offset + i, -np.inf, s)
            m = np.max(s, axis=1, keepdims=True)
            finite = np.isfinite(m)
            m = np.where(finite, m, 0.0)
            p = np.exp(s - m)
            l = p.sum(axis=1, keepdims=True)
            l = np.where(l > 0, l, 1.0)
            out[bi, h] = (p / l) @ v[bi, hk, :kb]
    return out
