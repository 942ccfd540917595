"""CPU oracle for the fused attention path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker or the timed CPU baseline; the product (``ffai_amd``) never
imports it.

Contents:

* ``liboracle.so`` (built from ``flash_oracle.cpp`` by ``Makefile``): a C++/AVX2 restatement of
  the reference kernel ``crates/ffai-mercury/src/asr/flash_attn.rs`` -- the encoder tiling
  (``flash_head_strided``, :415-487), the decode kernels (``xattn_head`` :602-696,
  ``xattn_head_f16`` :714-789), the exp polynomial (``exp256`` :553-571) -- plus a marked
  extension (batch, GQA, head_dim 128, causal with offset, ragged keys, scale) that the
  reference does not have.
* ``textbook``: float64 numpy closed form ``softmax(scale * Q K^T + mask) V``, independent of
  the tiling; the reference's own unit test checks the kernel against this same closed form
  (flash_attn.rs:1005-1021, via candle's three-op path).

Parity pins for each function live in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from . import textbook  # noqa: F401  (re-export)

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None
_VERSION = 5

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (g++ -O3 -mavx2 -mfma -mf16c)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_version.restype = ctypes.c_int
        if L.oracle_version() != _VERSION:
            raise RuntimeError("stale oracle/liboracle.so: rebuild with `make -C oracle -B`")
        L.oracle_exp_poly.argtypes = [_f32p, _f32p, ctypes.c_long]
        L.oracle_attend_merged.argtypes = [ctypes.c_int, ctypes.c_int, _f32p, _f32p, _f32p,
                                           _f32p, ctypes.c_int]
        L.oracle_attend_f32.argtypes = [ctypes.c_int] * 3 + [_f32p] * 4 + [ctypes.c_int] * 2
        L.oracle_attend_f16kv.argtypes = [ctypes.c_int, ctypes.c_int, _f32p, _u16p, _u16p,
                                          _f32p, ctypes.c_int, ctypes.c_int]
        L.oracle_attend_general.argtypes = (
            [ctypes.c_int] * 6 + [_f32p, _f32p, ctypes.c_int, _f32p, _f32p, ctypes.c_float,
                                  ctypes.c_int, ctypes.c_int, _i32p, ctypes.c_int])
        L.oracle_plant_fault.argtypes = [ctypes.c_int]
        L.oracle_plant_fault.restype = None
        _lib = L
    return _lib


def plant_fault(kind: int) -> None:
    """Tests only: make the oracle commit a known mistake (1 skip rescale, 2 drop the degree-5
    exp term, 3 drop each tile's last key, 4 transposed K index); 0 restores it."""
    lib().oracle_plant_fault(int(kind))


def _f32(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray, typ=_f32p):
    return a.ctypes.data_as(typ)


def default_threads() -> int:
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def exp_poly(x: np.ndarray) -> np.ndarray:
    """The reference's vector exp (flash_attn.rs:553-571)."""
    x = _f32(x).ravel()
    y = np.empty_like(x)
    lib().oracle_exp_poly(_ptr(x), _ptr(y), x.size)
    return y


def attend_merged(q, kt, v, threads: int | None = None) -> np.ndarray:
    """MergedAttnOp (flash_attn.rs:160-210): q (1,H,T,64), kt (1,H,64,T), v (1,H,T,64) f32
    -> (1,T,H*64) f32. The scale is the caller's (already folded into q or kt)."""
    q, kt, v = _f32(q), _f32(kt), _f32(v)
    _, h, t, d = q.shape
    assert d == 64 and kt.shape == (1, h, 64, t) and v.shape == (1, h, t, 64)
    out = np.empty((1, t, h * 64), np.float32)
    rc = lib().oracle_attend_merged(h, t, _ptr(q), _ptr(kt), _ptr(v), _ptr(out),
                                    threads or default_threads())
    assert rc == 0
    return out


def attend_f32(q, kt, v, par_heads: bool = False, threads: int | None = None):
    """FlashAttnOp f32 arms (flash_attn.rs:357-413): encoder (qlen == keys) or decode (qlen == 1).
    Returns (1,H,qlen,64) f32, or None where the reference declines qlen not in {1, keys}."""
    q, kt, v = _f32(q), _f32(kt), _f32(v)
    _, h, ql, d = q.shape
    keys = kt.shape[3]
    assert d == 64 and kt.shape == (1, h, 64, keys) and v.shape == (1, h, keys, 64)
    out = np.empty((1, h, ql, 64), np.float32)
    rc = lib().oracle_attend_f32(h, ql, keys, _ptr(q), _ptr(kt), _ptr(v), _ptr(out),
                                 int(par_heads), threads or default_threads())
    if rc == 1:
        return None
    assert rc == 0
    return out


def attend_f16kv(q, kt16, v16, par_heads: bool = False, threads: int | None = None):
    """FlashAttnOp f16-K/V decode arm (flash_attn.rs:289-356): q (1,H,1,64) f32; kt16, v16 are
    float16 arrays (1,H,64,K) and (1,H,K,64). Returns (1,H,1,64) f32."""
    q = _f32(q)
    kt16 = np.ascontiguousarray(kt16, dtype=np.float16)
    v16 = np.ascontiguousarray(v16, dtype=np.float16)
    _, h, ql, d = q.shape
    keys = kt16.shape[3]
    assert ql == 1 and d == 64 and kt16.shape == (1, h, 64, keys)
    out = np.empty((1, h, 1, 64), np.float32)
    rc = lib().oracle_attend_f16kv(h, keys, _ptr(q), _ptr(kt16.view(np.uint16), _u16p),
                                   _ptr(v16.view(np.uint16), _u16p), _ptr(out), int(par_heads),
                                   threads or default_threads())
    assert rc == 0
    return out


def attend_general(q, k, v, *, k_transposed: bool, scale: float = 1.0, causal: bool = False,
                   q_offset: int = 0, kv_lens=None, threads: int | None = None) -> np.ndarray:
    """Extension, NOT in the reference: q (B,Hq,Tq,D); k (B,Hkv,D,Tk) if k_transposed else
    (B,Hkv,Tk,D); v (B,Hkv,Tk,D); f32 math on the given values. Returns (B,Hq,Tq,D) f32."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    b, hq, tq, d = q.shape
    hkv = v.shape[1]
    tk = v.shape[2]
    out = np.empty((b, hq, tq, d), np.float32)
    lens = None
    if kv_lens is not None:
        lens = np.ascontiguousarray(kv_lens, dtype=np.int32)
        assert lens.shape == (b,)
    rc = lib().oracle_attend_general(b, hq, hkv, tq, tk, d, _ptr(q), _ptr(k), int(k_transposed),
                                     _ptr(v), _ptr(out), float(scale), int(causal),
                                     int(q_offset), None if lens is None else _ptr(lens, _i32p),
                                     threads or default_threads())
    assert rc == 0, rc
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round f32 values to bfloat16 (IEEE round-to-nearest-even), returned as f32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    nan = np.isnan(x)
    out = rounded.astype(np.uint32).view(np.float32).copy()
    out[nan] = np.nan
    return out
