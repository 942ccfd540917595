"""Device-resident decode-step state on torch device tensors, through include/ffai_kv.h.

The reference keeps each decoder layer's self-attention cache as raw (b, L, n_state)
projections grown by Tensor::cat (crates/ffai-mercury/src/asr/text_decoder.rs:652-662),
re-splits it into heads every step (:840-842), and snapshots/restores it per beam
(:1350-1381; decoder.rs:559-583). Here a KVCache holds the head-major layout the attention
kernels read, appended in place (`append`, or `advance` with the rows written by
gemv.F16Gemv.qkv_into_cache) and reordered by parent beam (`gather_from`);
`cross_kv_build` prepares the cross-attention cache once per window (:706-707, :770-773).
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib as L
from .flash_attn import _DT, _stream_handle


class KVCache:
    """k, v: (slots, heads, capacity, head_dim) of `dtype`; lens: int32[slots] keys per slot.
    Attend over it with flash_attn.attention(q, cache.k, cache.v, kv_lens=cache.lens, ...).

    With `layers`, the cache holds a decoder's whole stack: k, v are (layers, slots, heads,
    capacity, head_dim) and lens (layers, slots); `layer(l)` is layer l's cache (a view), which
    is appended and attended per layer, while `gather_from` reorders every layer in one launch."""

    def __init__(self, slots: int, heads: int, capacity: int, head_dim: int,
                 dtype: torch.dtype = torch.bfloat16, device=None, layers: Optional[int] = None,
                 _views=None):
        if _views is not None:
            self.k, self.v, self.lens = _views
        else:
            device = device or torch.device("cuda")
            lead = (layers,) if layers is not None else ()
            self.k = torch.zeros(*lead, slots, heads, capacity, head_dim, dtype=dtype, device=device)
            self.v = torch.zeros_like(self.k)
            self.lens = torch.zeros(*lead, slots, dtype=torch.int32, device=device)
        self.layers = layers
        self.slots, self.heads, self.capacity, self.head_dim = slots, heads, capacity, head_dim

    def layer(self, l: int) -> "KVCache":
        assert self.layers is not None and 0 <= l < self.layers
        return KVCache(self.slots, self.heads, self.capacity, self.head_dim,
                       _views=(self.k[l], self.v[l], self.lens[l]))

    def view(self) -> L.KVCacheView:
        """The C descriptor of this cache (of layer 0 for a layer stack)."""
        k = self.k[0] if self.layers is not None else self.k
        c = L.KVCacheView()
        c.k, c.v, c.lens = self.k.data_ptr(), self.v.data_ptr(), self.lens.data_ptr()
        c.dtype = _DT[self.k.dtype]
        c.slots, c.heads, c.capacity, c.head_dim = self.slots, self.heads, self.capacity, self.head_dim
        for i in range(3):
            c.strides[i] = k.stride(i)
        return c

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """k_new, v_new: (slots, t, heads * head_dim) projections (f32, f16 or bf16); row t of
        slot s lands at position lens[s] + t (rows past capacity are dropped)."""
        assert self.layers is None, "append to one layer: cache.layer(l).append(...)"
        assert k_new.shape == v_new.shape and k_new.dim() == 3 and k_new.stride(2) == 1
        assert v_new.stride() == k_new.stride() and k_new.dtype == v_new.dtype
        c = self.view()
        L.check(L.load().ffai_kv_append(ctypes.byref(c), k_new.data_ptr(), v_new.data_ptr(),
                                        _DT[k_new.dtype], k_new.shape[1], k_new.stride(0),
                                        k_new.stride(1), _stream_handle(k_new)))

    def advance(self, t_new: int = 1) -> None:
        """lens += t_new (saturating at capacity) in every layer: a decode step's length update
        when F16Gemv.qkv_into_cache writes the step's rows itself."""
        layers, lls = (1, 0) if self.layers is None else (self.layers, self.lens.stride(0))
        c = self.view()
        L.check(L.load().ffai_kv_advance(ctypes.byref(c), t_new, layers, lls,
                                         _stream_handle(self.lens)))

    def gather_from(self, src: "KVCache", parent: torch.Tensor) -> None:
        """Slot i becomes a copy of src's slot parent[i] (a beam step's reorder), in every layer."""
        assert parent.dtype == torch.int32 and parent.is_cuda and parent.numel() == self.slots
        assert self.layers == src.layers
        layers, ls, lls = 1, 0, 0
        if self.layers is not None:
            assert self.k.stride(0) == src.k.stride(0) == self.v.stride(0) == src.v.stride(0)
            assert self.lens.stride(0) == src.lens.stride(0)
            layers, ls, lls = self.layers, self.k.stride(0), self.lens.stride(0)
        d, s = self.view(), src.view()
        L.check(L.load().ffai_kv_gather(ctypes.byref(d), ctypes.byref(s), parent.data_ptr(),
                                        layers, ls, lls, _stream_handle(parent)))


def cross_kv_build(k_proj: torch.Tensor, v_proj: torch.Tensor, heads: int,
                   out_dtype: torch.dtype = torch.bfloat16, k_transposed: bool = True,
                   out: Optional[tuple[torch.Tensor, torch.Tensor]] = None):
    """k_proj, v_proj: (T, heads * head_dim) -> (K, V) with K (heads, head_dim, T) if
    k_transposed else (heads, T, head_dim), V (heads, T, head_dim), in out_dtype."""
    t, n = k_proj.shape
    assert v_proj.shape == k_proj.shape and k_proj.stride(1) == 1 and v_proj.stride() == k_proj.stride()
    d = n // heads
    if out is None:
        k = torch.empty((heads, d, t) if k_transposed else (heads, t, d), dtype=out_dtype,
                        device=k_proj.device)
        v = torch.empty(heads, t, d, dtype=out_dtype, device=k_proj.device)
    else:
        k, v = out
    L.check(L.load().ffai_cross_kv_build(
        k_proj.data_ptr(), v_proj.data_ptr(), _DT[k_proj.dtype], t, heads, d, k_proj.stride(0),
        k.data_ptr(), v.data_ptr(), _DT[out_dtype],
        L.K_TRANSPOSED if k_transposed else L.K_ROWS, _stream_handle(k_proj)))
    return k, v


def self_attention_step(cache: KVCache, q: torch.Tensor, k_new: torch.Tensor,
                        v_new: torch.Tensor, offset: int, scale: float,
                        out: Optional[torch.Tensor] = None,
                        workspace: Optional[torch.Tensor] = None,
                        out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Attention::forward_self (crates/ffai-mercury/src/asr/text_decoder.rs:652-679) on the
    device: append this step's K/V projections to the cache in place (replacing Tensor::cat),
    then attend q over every slot's keys. A multi-token step (a prompt, :663-676) is causal:
    query i sits at absolute position offset + i and sees keys 0..offset + i (causal_mask,
    :902-923); a single-token step needs no mask, as in the reference.

    q: (slots, heads, q_len, head_dim); k_new, v_new: (slots, q_len, heads * head_dim);
    `offset` is the absolute position of the first query token, which the caller knows (the
    cache's lengths before the append), exactly as the reference's caller passes it.
    The weights are softmax(scale * q k^T): scale = head_dim^-0.5 reproduces the reference's
    q * s^2 (:840)."""
    from . import flash_attn as fa

    cache.append(k_new, v_new)
    q_len = q.shape[2]
    return fa.attention(q, cache.k, cache.v, scale=scale, kv_lens=cache.lens,
                        causal=q_len > 1, q_offset=offset if q_len > 1 else 0, out=out,
                        workspace=workspace, out_dtype=out_dtype)
