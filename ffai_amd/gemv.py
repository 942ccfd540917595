"""The decoder's single-row projections on the device, through include/ffai_gemv.h.

F16Gemv mirrors crates/ffai-mercury/src/asr/f16_gemv.rs (f16 weights (out, in), f32
activations and arithmetic); Int8Vocab mirrors vocab_int8.rs (block-scaled int8 vocabulary
weights, 7-bit offset activations). Both take every beam's row in one call.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib as L
from .flash_attn import _DT, _stream_handle


class F16Gemv:
    """F16Gemv::new / forward: `weight` (out, in) is stored as f16 on the device."""

    def __init__(self, weight: torch.Tensor):
        assert weight.dim() == 2 and weight.is_cuda
        self.w = weight.to(torch.float16).contiguous()
        self.out_dim, self.in_dim = self.w.shape

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x: (rows, in) f32, rows <= 16 (one per beam) -> (rows, out) f32."""
        assert x.dtype == torch.float32 and x.dim() == 2 and x.stride(1) == 1
        if out is None:
            out = torch.empty(x.shape[0], self.out_dim, dtype=torch.float32, device=x.device)
        L.check(L.load().ffai_gemv_f16(self.w.data_ptr(), self.out_dim, self.in_dim, x.data_ptr(),
                                       x.shape[0], x.stride(0), out.data_ptr(), out.stride(0),
                                       _stream_handle(x)))
        return out

    __call__ = forward

    def qkv_into_cache(self, x: torch.Tensor, q_out: torch.Tensor, cache,
                       bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The packed (q; k; v) projection of a decode step (weights (3 * heads * head_dim,
        in)): q_out (rows, heads * head_dim) f32 gets the q part, and the k and v rows of beam r
        go into slot r of `cache` (one layer's KVCache) at position lens[r] - 1, the position the
        step's cache.advance() opened. bias: (3 * heads * head_dim,) f32 or None."""
        assert x.dtype == torch.float32 and x.dim() == 2 and x.stride(1) == 1
        n = cache.heads * cache.head_dim
        assert self.out_dim == 3 * n and cache.layers is None
        assert q_out.dtype == torch.float32 and q_out.shape == (x.shape[0], n) and q_out.stride(1) == 1
        if bias is not None:
            assert bias.dtype == torch.float32 and bias.is_contiguous() and bias.numel() == 3 * n
        c = cache.view()
        L.check(L.load().ffai_gemv_f16_qkv_cache(
            self.w.data_ptr(), None if bias is None else bias.data_ptr(), self.in_dim,
            x.data_ptr(), x.shape[0], x.stride(0), q_out.data_ptr(), q_out.stride(0),
            ctypes.byref(c), _stream_handle(x)))
        return q_out


class Int8Vocab:
    """Int8Vocab::new quantizes the (vocab, d) embedding matrix on the device once; forward maps
    (rows, d) f32 activations to (rows, vocab) f32 logits."""

    def __init__(self, embeddings: torch.Tensor, blk: int = 32):
        assert embeddings.dim() == 2 and embeddings.is_cuda and embeddings.is_contiguous()
        self.vocab, self.d = embeddings.shape
        self.blk = blk
        dev = embeddings.device
        self.qw = torch.empty(self.vocab, self.d, dtype=torch.int8, device=dev)
        self.bscale = torch.empty(self.vocab, self.d // blk, dtype=torch.float32, device=dev)
        self.corr = torch.empty(self.vocab, dtype=torch.float32, device=dev)
        L.check(L.load().ffai_vocab_int8_quantize(
            embeddings.data_ptr(), _DT[embeddings.dtype], self.vocab, self.d, blk,
            self.qw.data_ptr(), self.bscale.data_ptr(), self.corr.data_ptr(),
            _stream_handle(embeddings)))
        self._ws: Optional[torch.Tensor] = None

    def workspace_bytes(self, rows: int) -> int:
        n = ctypes.c_size_t(0)
        L.check(L.load().ffai_vocab_int8_workspace_bytes(self.d, rows, ctypes.byref(n)))
        return n.value

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
        assert x.dtype == torch.float32 and x.dim() == 2 and x.stride(1) == 1
        rows = x.shape[0]
        if workspace is None:
            need = self.workspace_bytes(rows)
            if self._ws is None or self._ws.numel() < need:
                self._ws = torch.empty(need, dtype=torch.uint8, device=x.device)
            workspace = self._ws
        if out is None:
            out = torch.empty(rows, self.vocab, dtype=torch.float32, device=x.device)
        L.check(L.load().ffai_vocab_int8_logits(
            self.qw.data_ptr(), self.bscale.data_ptr(), self.corr.data_ptr(), self.vocab, self.d,
            self.blk, x.data_ptr(), rows, x.stride(0), out.data_ptr(), out.stride(0),
            workspace.data_ptr(), workspace.numel(), _stream_handle(x)))
        return out

    __call__ = forward
