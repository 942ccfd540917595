"""CPU restatement of the reference's decoder attention state. TEST INFRASTRUCTURE ONLY: used by
tests/ and never by the ffai_amd product path.

Follows crates/ffai-mercury/src/asr/text_decoder.rs and decoder.rs:
  * split_heads            -- Attention::split_heads (text_decoder.rs:638-643):
                              (b, L, n_state) -> (b, heads, L, n_state / heads)
  * self_cache_append      -- forward_self (:652-662): the cache of raw projections grows by
                              Tensor::cat along the sequence axis
  * beam_restore           -- TextDecoder::save/restore (:1350-1381) as decode_beam uses them
                              (decoder.rs:559-583): each new beam continues from its parent's state
  * cross_cache_build      -- forward_cross (:706-707, :770-773): K split into heads and
                              transposed to (1, heads, head_dim, T), V split to (1, heads, T,
                              head_dim), both converted to the cache dtype
  * causal_mask            -- causal_mask (:902-923): the mask of a multi-token prompt step
  * three_op_attend        -- the unfused path the reference takes for masked prompt steps and
                              multi-token cross-attention (:832-871, :799-816)
The values are numpy arrays; 16-bit dtypes are represented as float32 values rounded to that
type (round-to-nearest-even), which is what the device caches hold.
"""

from __future__ import annotations

import numpy as np

from . import round_bf16


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Values of x rounded to `dtype` ('f32', 'f16', 'bf16'), returned as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "f32":
        return x.copy()
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return round_bf16(x)
    raise ValueError(dtype)


def split_heads(x: np.ndarray, heads: int) -> np.ndarray:
    b, length, n = x.shape
    return x.reshape(b, length, heads, n // heads).transpose(0, 2, 1, 3)


def self_cache_append(cache: np.ndarray | None, new: np.ndarray) -> np.ndarray:
    """cache (b, L, n) or None, new (b, t, n) -> (b, L + t, n)."""
    return new.copy() if cache is None else np.concatenate([cache, new], axis=1)


def beam_restore(states: list, parents) -> list:
    """The state each new beam continues from: its parent's (shared, not copied: the reference's
    snapshots are refcounted handles that are never written in place)."""
    return [states[int(p)] for p in parents]


def cross_cache_build(k: np.ndarray, v: np.ndarray, heads: int, dtype: str,
                      k_transposed: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """k, v: (T, n_state) projections of one window -> (K^T (heads, head_dim, T) or K rows
    (heads, T, head_dim), V (heads, T, head_dim)), rounded to the cache dtype."""
    ks = split_heads(k[None], heads)[0]
    vs = split_heads(v[None], heads)[0]
    kt = ks.transpose(0, 2, 1) if k_transposed else ks
    return round_to(np.ascontiguousarray(kt), dtype), round_to(np.ascontiguousarray(vs), dtype)


def causal_mask(q_len: int, k_len: int, offset: int) -> np.ndarray:
    """causal_mask (text_decoder.rs:902-923): (q_len, k_len) float32, -inf where key j lies after
    query i's absolute position offset + i, else 0."""
    i = np.arange(q_len)[:, None]
    j = np.arange(k_len)[None, :]
    return np.where(j > offset + i, np.float32(-np.inf), np.float32(0.0)).astype(np.float32)


def three_op_attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
                    mask: np.ndarray | None = None) -> np.ndarray:
    """The reference's unfused attention (Attention::attend + attend_prepared, text_decoder.rs:
    832-871): q (b, h, tq, d) scaled by scale, k (b, h, tk, d) used as K^T, optional additive
    mask (tq, tk) broadcast over b and h, softmax over keys, times v. Computed in float64 (the
    reference's candle ops run in the tensors' dtype, f32 here; the bar is a tolerance)."""
    s = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64) * scale, k.astype(np.float64))
    if mask is not None:
        s = s + mask.astype(np.float64)
    s = s - s.max(axis=-1, keepdims=True)
    w = np.exp(s)
    w /= w.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", w, v.astype(np.float64)).astype(np.float32)
