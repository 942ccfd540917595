"""Host-side mirror of the reference's fused attention API on torch device tensors.

The reference exposes three functions over candle tensors
(crates/ffai-mercury/src/asr/flash_attn.rs):

* ``serves(kt, v) -> bool``                       (:103-129)
* ``attend(q, kt, v, masked) -> Option<Tensor>``   (:212-264, FlashAttnOp :266-413)
* ``attend_merged(q, kt, v) -> Option<Tensor>``    (:131-158, MergedAttnOp :160-210)

This module keeps those names, argument meanings and the decline contract (``None`` where the
reference returns ``Ok(None)``; an exception where it returns ``Err``), and forwards to the C ABI
(``include/ffai_attn.h``) on the caller's current HIP stream. ``attention`` exposes the general
descriptor entry point (batch, bf16/f16, grouped K/V heads, head_dim 128, causal with offset,
ragged key counts, K/V shared across the batch). Torch only provides device memory and streams.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import torch

from . import _lib as L

_DT = {torch.float32: L.F32, torch.float16: L.F16, torch.bfloat16: L.BF16}
_TORCH_DT = {v: k for k, v in _DT.items()}


def _stream_handle(t: Optional[torch.Tensor] = None) -> ctypes.c_void_p:
    """The caller's current HIP stream (None for host tensors, which the library declines
    before touching any stream)."""
    if t is not None and not t.is_cuda:
        return ctypes.c_void_p(None)
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _view(t: torch.Tensor) -> L.TensorView:
    if t.dim() > 4:
        raise ValueError("tensor views are at most 4-D")
    dims = list(t.shape) + [1] * (4 - t.dim())
    strides = list(t.stride()) + [1] * (4 - t.dim())
    v = L.TensorView()
    v.data = t.data_ptr()
    v.dtype = _DT.get(t.dtype, -1)
    v.on_device = 1 if t.is_cuda else 0
    for i in range(4):
        v.dims[i] = dims[i]
        v.strides[i] = strides[i]
    return v


def _workspace(nbytes: int, device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)  # counters start at zero


# -------------------------------------------------------------------------------------------
# Mirrors of the reference functions
# -------------------------------------------------------------------------------------------

def serves(kt: torch.Tensor, v: torch.Tensor) -> bool:
    """flash_attn::serves: whether the decode-shape kernel serves this K/V pair (callers pick the
    cross-attention cache dtype with it)."""
    return L.load().ffai_serves(ctypes.byref(_view(kt)), ctypes.byref(_view(v))) == 1


def attend(q: torch.Tensor, kt: torch.Tensor, v: torch.Tensor,
           masked: bool = False) -> Optional[torch.Tensor]:
    """flash_attn::attend: q (1,H,qlen,64) f32; kt (1,H,64,K) and v (1,H,K,64) f32 (or f16 at
    qlen == 1). Returns (1,H,qlen,64) f32, or None where the reference declines."""
    lib = L.load()
    qv, kv, vv = _view(q), _view(kt), _view(v)
    nbytes = ctypes.c_size_t(0)
    rc = lib.ffai_attend_workspace_bytes(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                         ctypes.byref(nbytes))
    if masked or rc == L.FFAI_DECLINED:
        # let the C mirror apply (and report) the decline, exactly as it would for a caller
        out = torch.empty(0, device=q.device)
        rc = lib.ffai_attend(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), int(masked),
                             ctypes.byref(_view(out)), None, 0, _stream_handle(q))
        return None if L.check(rc) == L.FFAI_DECLINED else out
    L.check(rc)
    out = torch.empty(q.shape[0], q.shape[1], q.shape[2], 64, dtype=torch.float32,
                      device=q.device)
    ws = _workspace(nbytes.value, q.device)
    rc = lib.ffai_attend(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), 0,
                         ctypes.byref(_view(out)),
                         None if ws is None else ws.data_ptr(), nbytes.value, _stream_handle())
    if L.check(rc) == L.FFAI_DECLINED:
        return None
    return out


def attend_merged(q: torch.Tensor, kt: torch.Tensor,
                  v: torch.Tensor) -> Optional[torch.Tensor]:
    """flash_attn::attend_merged: encoder attention writing (1,T,H*64) f32 directly, or None."""
    lib = L.load()
    qv, kv, vv = _view(q), _view(kt), _view(v)
    heads, seq = q.shape[1], q.shape[2]
    out = torch.empty(1, seq, heads * 64, dtype=torch.float32, device=q.device)
    nbytes = ctypes.c_size_t(0)
    rc = lib.ffai_attend_merged_workspace_bytes(ctypes.byref(qv), ctypes.byref(kv),
                                                ctypes.byref(vv), ctypes.byref(nbytes))
    ws = _workspace(nbytes.value, q.device) if rc == L.FFAI_OK else None
    rc = lib.ffai_attend_merged(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                ctypes.byref(_view(out)),
                                None if ws is None else ws.data_ptr(), nbytes.value,
                                _stream_handle(q))
    if L.check(rc) == L.FFAI_DECLINED:
        return None
    return out


def decode_min_keys() -> int:
    return L.load().ffai_get_decode_min_keys()


def set_decode_min_keys(n: int) -> None:
    """knobs::DECODE_MIN_KEYS.set (knobs.rs:163-168)."""
    L.load().ffai_set_decode_min_keys(int(n))


# -------------------------------------------------------------------------------------------
# General descriptor entry point
# -------------------------------------------------------------------------------------------

def make_desc(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor, *,
              k_transposed: bool, scale: float, causal: bool, q_offset: int,
              kv_lens: Optional[torch.Tensor]) -> L.AttnDesc:
    """Descriptor for q (B,Hq,Tq,D), k (B,Hkv,D,Tk) if k_transposed else (B,Hkv,Tk,D),
    v (B,Hkv,Tk,D), out (B,Hq,Tq,D); any strides with a unit innermost stride. A K/V batch
    dimension of size 1 broadcasts (stride 0) across the batch."""
    b, hq, tq, d = q.shape
    hkv = v.shape[1]
    tk = v.shape[2]
    desc = L.AttnDesc()
    desc.q_dtype = _DT[q.dtype]
    desc.kv_dtype = _DT[k.dtype]
    desc.out_dtype = _DT[out.dtype]
    desc.batch, desc.heads_q, desc.heads_kv = b, hq, hkv
    desc.q_len, desc.kv_len, desc.head_dim = tq, tk, d
    desc.k_layout = L.K_TRANSPOSED if k_transposed else L.K_ROWS
    desc.causal = int(causal)
    desc.q_offset = int(q_offset)
    desc.scale = float(scale)

    def strides(t: torch.Tensor, name: str):
        s = list(t.stride())
        if t.shape[0] == 1 and b > 1:
            s[0] = 0
        return s

    for field, t in (("q_strides", q), ("k_strides", k), ("v_strides", v), ("o_strides", out)):
        arr = getattr(desc, field)
        for i, x in enumerate(strides(t, field)):
            arr[i] = x
    desc.kv_lens = None if kv_lens is None else kv_lens.data_ptr()
    return desc


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, k_transposed: bool = False,
              scale: float = 1.0, causal: bool = False, q_offset: int = 0,
              kv_lens: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
              out_dtype: Optional[torch.dtype] = None,
              workspace: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """O = softmax(scale * Q K^T [+ causal mask]) V through ffai_attn_fwd. Returns the output, or
    None when the descriptor is not served. `workspace` (see workspace_bytes) may be reused by
    stream-ordered calls and graph replays."""
    lib = L.load()
    if out is None:
        od = out_dtype or (torch.float32 if q.dtype == torch.float32 else q.dtype)
        out = torch.empty(q.shape[0], q.shape[1], q.shape[2], v.shape[3], dtype=od,
                          device=q.device)
    if kv_lens is not None:
        assert kv_lens.dtype == torch.int32 and kv_lens.is_cuda
    desc = make_desc(q, k, v, out, k_transposed=k_transposed, scale=scale, causal=causal,
                     q_offset=q_offset, kv_lens=kv_lens)
    nbytes = ctypes.c_size_t(0)
    rc = L.check(lib.ffai_attn_workspace_bytes(ctypes.byref(desc), ctypes.byref(nbytes)))
    if rc == L.FFAI_DECLINED:
        return None
    if nbytes.value and (workspace is None or workspace.numel() * workspace.element_size()
                         < nbytes.value):
        workspace = _workspace(nbytes.value, q.device)
    rc = lib.ffai_attn_fwd(ctypes.byref(desc), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                           out.data_ptr(),
                           None if workspace is None else workspace.data_ptr(),
                           0 if workspace is None else workspace.numel() * workspace.element_size(),
                           _stream_handle())
    if L.check(rc) == L.FFAI_DECLINED:
        return None
    return out


def workspace_bytes(q, k, v, out, **kw) -> int:
    desc = make_desc(q, k, v, out, k_transposed=kw.get("k_transposed", False),
                     scale=kw.get("scale", 1.0), causal=kw.get("causal", False),
                     q_offset=kw.get("q_offset", 0), kv_lens=kw.get("kv_lens"))
    n = ctypes.c_size_t(0)
    L.check(L.load().ffai_attn_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)))
    return n.value


def plan(q, k, v, out, **kw) -> dict:
    """The launch plan ffai_attn_fwd uses for these operands (ffai_attn_plan_info), assuming
    the kernels' vector alignment: kernel, workgroup shape, key splits, tiles per split and
    workgroups."""
    desc = make_desc(q, k, v, out, k_transposed=kw.get("k_transposed", False),
                     scale=kw.get("scale", 1.0), causal=kw.get("causal", False),
                     q_offset=kw.get("q_offset", 0), kv_lens=kw.get("kv_lens"))
    return L.plan_info(desc)


def serves_desc(q_dtype: torch.dtype, kv_dtype: torch.dtype, out_dtype: torch.dtype,
                shape: Sequence[int], *, k_transposed: bool = False, causal: bool = False) -> bool:
    """ffai_attn_serves for packed operands: shape = (batch, heads_q, heads_kv, q_len, kv_len,
    head_dim)."""
    b, hq, hkv, tq, tk, d = shape
    desc = L.AttnDesc()
    L.load().ffai_attn_desc_init(ctypes.byref(desc), _DT[q_dtype], _DT[kv_dtype], _DT[out_dtype],
                                 b, hq, hkv, tq, tk, d,
                                 L.K_TRANSPOSED if k_transposed else L.K_ROWS)
    desc.causal = int(causal)
    return L.load().ffai_attn_serves(ctypes.byref(desc)) == 1
