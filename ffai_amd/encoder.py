"""The audio encoder's self-attention block on the device, through include/ffai_encoder.h.

Mirrors EncoderAttention (crates/ffai-mercury/src/asr/text_decoder.rs:1009-1139): `load` folds
head_dim^-0.5 into the key weight once (:1039-1050); `forward` runs the q / k^T / v projections,
the fused attention and the out-projection in one stream-ordered library call (hipBLASLt GEMMs
around ffai_attn_fwd), with no head-split copies. Inside the call the windows run in passes of at
most 1500 rows through one workspace, as the reference loops over batch items (:1069-1076).
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib as L
from .flash_attn import _DT, _stream_handle


class EncoderAttention:
    """Weights as the reference holds them: each Linear weight (out, in), each bias (out); the
    key projection has no bias. All tensors are device tensors of one dtype (bf16 or f16).
    `packed` (default) also packs the input projections once, [wq; wk_scaled; wv] and
    [bq; 0; bv], so that a call runs them as one GEMM."""

    def __init__(self, n_state: int, n_head: int, wq, bq, wk_scaled, wv, bv, wo, bo,
                 packed: bool = True):
        self.n_state, self.n_head = n_state, n_head
        self.w = [t.contiguous() for t in (wq, bq, wk_scaled, wv, bv, wo, bo)]
        self.packed = None
        if packed:
            self.packed = (torch.cat([wq, wk_scaled, wv], 0).contiguous(),
                           torch.cat([bq, torch.zeros_like(bq), bv], 0).contiguous())
        self._ws: Optional[torch.Tensor] = None

    @classmethod
    def load(cls, n_state: int, n_head: int, wq, bq, wk, wv, bv, wo, bo,
             packed: bool = True) -> "EncoderAttention":
        """EncoderAttention::load: the key weight pre-scaled by head_dim^-0.5 (computed in f32,
        stored in the weights' dtype)."""
        scale = (n_state // n_head) ** -0.5
        wk_scaled = (wk.float() * scale).to(wk.dtype)
        return cls(n_state, n_head, wq, bq, wk_scaled, wv, bv, wo, bo, packed=packed)

    def _desc(self, x: torch.Tensor) -> L.EncoderAttnDesc:
        d = L.EncoderAttnDesc()
        d.dtype = _DT[x.dtype]
        d.batch, d.seq, d.n_state, d.n_head = x.shape[0], x.shape[1], self.n_state, self.n_head
        return d

    def workspace_bytes(self, x: torch.Tensor) -> int:
        n = ctypes.c_size_t(0)
        L.check(L.load().ffai_encoder_attn_workspace_bytes(ctypes.byref(self._desc(x)),
                                                           ctypes.byref(n)))
        return n.value

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x: (batch, seq, n_state) -> (batch, seq, n_state), in x's dtype."""
        assert x.dim() == 3 and x.shape[2] == self.n_state and x.is_contiguous()
        assert all(t.dtype == x.dtype and t.device == x.device for t in self.w)
        desc = self._desc(x)
        if workspace is None:
            need = self.workspace_bytes(x)
            if self._ws is None or self._ws.numel() < need or self._ws.device != x.device:
                # zeroed once: it holds the attention's split counters (left zero by each call)
                self._ws = torch.zeros(need, dtype=torch.uint8, device=x.device)
            workspace = self._ws
        if out is None:
            out = torch.empty_like(x)
        ptrs = [t.data_ptr() for t in self.w]
        ptrs += [t.data_ptr() for t in self.packed] if self.packed is not None else [None, None]
        w = L.EncoderAttnWeights(*ptrs)
        L.check(L.load().ffai_encoder_attn_fwd(ctypes.byref(desc), x.data_ptr(), ctypes.byref(w),
                                               out.data_ptr(), workspace.data_ptr(),
                                               workspace.numel(), _stream_handle(x)))
        return out

    __call__ = forward
