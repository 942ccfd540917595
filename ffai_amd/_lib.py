"""ctypes binding of include/ffai_attn.h (libffai_attn.so, built in-tree by ffai_amd/build.py).

Loading fails loudly when the library has not been built: there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libffai_attn.so")
INCLUDE_DIR = os.path.join(os.path.dirname(HERE), "include")
HEADER_PATH = os.path.join(INCLUDE_DIR, "ffai_attn.h")

FFAI_OK = 0
FFAI_DECLINED = 1
FFAI_ERR_INVALID = -1
FFAI_ERR_HIP = -2
FFAI_ERR_WORKSPACE = -3
FFAI_ERR_DEVICE = -4

F32, F16, BF16 = 0, 1, 2
K_TRANSPOSED, K_ROWS = 0, 1
ABI_VERSION = 1


class AttnDesc(ctypes.Structure):
    _fields_ = [
        ("q_dtype", ctypes.c_int32), ("kv_dtype", ctypes.c_int32), ("out_dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32), ("heads_q", ctypes.c_int32), ("heads_kv", ctypes.c_int32),
        ("q_len", ctypes.c_int32), ("kv_len", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("k_layout", ctypes.c_int32), ("causal", ctypes.c_int32), ("q_offset", ctypes.c_int32),
        ("scale", ctypes.c_float), ("reserved0", ctypes.c_int32),
        ("q_strides", ctypes.c_int64 * 4), ("k_strides", ctypes.c_int64 * 4),
        ("v_strides", ctypes.c_int64 * 4), ("o_strides", ctypes.c_int64 * 4),
        ("kv_lens", ctypes.c_void_p),
    ]


class KVCacheView(ctypes.Structure):
    _fields_ = [
        ("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("lens", ctypes.c_void_p),
        ("dtype", ctypes.c_int32), ("slots", ctypes.c_int32), ("heads", ctypes.c_int32),
        ("capacity", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("reserved0", ctypes.c_int32),
        ("strides", ctypes.c_int64 * 3),
    ]


class EncoderAttnDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("dtype", "batch", "seq", "n_state", "n_head", "reserved0")]


class EncoderAttnWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p)
                for n in ("wq", "bq", "wk_scaled", "wv", "bv", "wo", "bo", "wqkv", "bqkv")]


class TensorView(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("on_device", ctypes.c_int32),
        ("dims", ctypes.c_int64 * 4), ("strides", ctypes.c_int64 * 4),
    ]


_lib = None


class FfaiError(RuntimeError):
    """An error status (< 0) from the C ABI."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"ffai_attn error {code}: {msg}")
        self.code = code


def header_functions() -> list[str]:
    """Names of every function the headers in include/ declare."""
    names = set()
    for fn in sorted(os.listdir(INCLUDE_DIR)):
        if fn.endswith(".h"):
            text = open(os.path.join(INCLUDE_DIR, fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(ffai_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def load():
    """Load libffai_attn.so (raises if it is missing or built for another ABI)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m ffai_amd.build` "
                           "(or __graft_entry__.build()); the attention path has no fallback")
    L = ctypes.CDLL(LIB_PATH)
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    dp = ctypes.POINTER(AttnDesc)
    tp = ctypes.POINTER(TensorView)
    L.ffai_attn_abi_version.restype = ctypes.c_int
    if L.ffai_attn_abi_version() != ABI_VERSION:
        raise RuntimeError("libffai_attn.so ABI mismatch: rebuild it")
    L.ffai_attn_desc_init.argtypes = [dp] + [ctypes.c_int32] * 10
    L.ffai_attn_desc_init.restype = None
    L.ffai_attn_serves.argtypes = [dp]
    L.ffai_attn_workspace_bytes.argtypes = [dp, ctypes.POINTER(sz)]
    L.ffai_attn_fwd.argtypes = [dp, vp, vp, vp, vp, vp, sz, vp]
    L.ffai_attn_plan_info.argtypes = [dp, ctypes.POINTER(ctypes.c_int32)]
    L.ffai_attn_fwd_noalloc.argtypes = [dp, vp, vp, vp, vp, vp]
    L.ffai_attn_noalloc_plan_info.argtypes = [dp, ctypes.POINTER(ctypes.c_int32),
                                              ctypes.POINTER(sz)]
    L.ffai_attn_noalloc_scratch_bytes.restype = sz
    L.ffai_serves.argtypes = [tp, tp]
    L.ffai_attend.argtypes = [tp, tp, tp, ctypes.c_int, tp, vp, sz, vp]
    L.ffai_attend_workspace_bytes.argtypes = [tp, tp, tp, ctypes.POINTER(sz)]
    L.ffai_attend_merged.argtypes = [tp, tp, tp, tp, vp, sz, vp]
    L.ffai_attend_merged_workspace_bytes.argtypes = [tp, tp, tp, ctypes.POINTER(sz)]
    L.ffai_get_decode_min_keys.restype = ctypes.c_int
    L.ffai_set_decode_min_keys.argtypes = [ctypes.c_int]
    L.ffai_set_decode_min_keys.restype = None
    L.ffai_get_decode_tiles_per_wg.restype = ctypes.c_int
    L.ffai_set_decode_tiles_per_wg.argtypes = [ctypes.c_int]
    L.ffai_set_decode_tiles_per_wg.restype = None
    L.ffai_attn_plan_splits.argtypes = [dp, ctypes.POINTER(ctypes.c_int32)]
    L.ffai_set_attn_variant.argtypes = [ctypes.c_int]
    L.ffai_set_attn_variant.restype = None
    L.ffai_get_attn_variant.restype = ctypes.c_int
    L.ffai_set_geometry_override.argtypes = [ctypes.c_int, ctypes.c_int]
    L.ffai_set_geometry_override.restype = None
    L.ffai_set_fwd_split_override.argtypes = [ctypes.c_int, ctypes.c_int]
    L.ffai_set_fwd_split_override.restype = None
    L.ffai_get_fwd_split_override.argtypes = [ctypes.POINTER(ctypes.c_int)] * 2
    L.ffai_get_fwd_split_override.restype = None
    L.ffai_attn_last_error.restype = ctypes.c_char_p
    cp = ctypes.POINTER(KVCacheView)
    i32, i64 = ctypes.c_int32, ctypes.c_int64
    L.ffai_kv_append.argtypes = [cp, vp, vp, i32, i32, i64, i64, vp]
    L.ffai_kv_gather.argtypes = [cp, cp, vp, i32, i64, i64, vp]
    L.ffai_kv_advance.argtypes = [cp, i32, i32, i64, vp]
    L.ffai_cross_kv_build.argtypes = [vp, vp, i32, i32, i32, i32, i64, vp, vp, i32, i32, vp]
    ed, ew = ctypes.POINTER(EncoderAttnDesc), ctypes.POINTER(EncoderAttnWeights)
    L.ffai_encoder_attn_workspace_bytes.argtypes = [ed, ctypes.POINTER(ctypes.c_size_t)]
    L.ffai_encoder_attn_fwd.argtypes = [ed, vp, ew, vp, vp, ctypes.c_size_t, vp]
    L.ffai_gemv_f16.argtypes = [vp, i32, i32, vp, i32, i64, vp, i64, vp]
    L.ffai_gemv_f16_qkv_cache.argtypes = [vp, vp, i32, vp, i32, i64, vp, i64, cp, vp]
    ip = ctypes.POINTER(ctypes.c_int32)
    L.ffai_gemv_f16_plan_info.argtypes = [i32, i32, i32, ip, ip, ip, ip,
                                          ctypes.POINTER(ctypes.c_size_t)]
    L.ffai_vocab_int8_quantize.argtypes = [vp, i32, i32, i32, i32, vp, vp, vp, vp]
    L.ffai_vocab_int8_workspace_bytes.argtypes = [i32, i32, ctypes.POINTER(ctypes.c_size_t)]
    L.ffai_vocab_int8_logits.argtypes = [vp, vp, vp, i32, i32, i32, vp, i32, i64, vp, i64, vp,
                                         ctypes.c_size_t, vp]
    L.ffai_probe_empty.argtypes = [ctypes.c_int, vp]
    L.ffai_probe_read.argtypes = [vp, sz, vp, ctypes.c_int, vp]
    L.ffai_probe_pipes.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
    for name in ("ffai_probe_empty", "ffai_probe_read", "ffai_probe_pipes", "ffai_attn_serves",
                 "ffai_attn_workspace_bytes", "ffai_attn_fwd",
                 "ffai_attn_plan_info", "ffai_attn_plan_splits", "ffai_attn_fwd_noalloc",
                 "ffai_attn_noalloc_plan_info",
                 "ffai_serves",
                 "ffai_attend", "ffai_attend_workspace_bytes", "ffai_attend_merged",
                 "ffai_attend_merged_workspace_bytes", "ffai_kv_append", "ffai_kv_gather",
                 "ffai_kv_advance", "ffai_gemv_f16_qkv_cache",
                 "ffai_cross_kv_build", "ffai_encoder_attn_workspace_bytes",
                 "ffai_encoder_attn_fwd", "ffai_gemv_f16", "ffai_gemv_f16_plan_info",
                 "ffai_vocab_int8_quantize",
                 "ffai_vocab_int8_workspace_bytes", "ffai_vocab_int8_logits"):
        getattr(L, name).restype = ctypes.c_int
    _lib = L
    return L


def gemv_plan_info(out_dim: int, in_dim: int, rows: int) -> dict:
    """The launch shape ffai_gemv_f16 uses for (out_dim, in_dim, rows)."""
    v = [ctypes.c_int32() for _ in range(4)]
    lds = ctypes.c_size_t()
    check(load().ffai_gemv_f16_plan_info(out_dim, in_dim, rows, *[ctypes.byref(a) for a in v],
                                         ctypes.byref(lds)))
    return {"tile_rows": v[0].value, "waves": v[1].value, "blocks_per_wave": v[2].value,
            "passes": v[3].value, "lds_bytes": lds.value}


def plan_info(desc: AttnDesc) -> dict:
    """The launch plan ffai_attn_fwd uses for `desc` with vector-aligned operands."""
    info = (ctypes.c_int32 * 5)()
    check(load().ffai_attn_plan_info(ctypes.byref(desc), info))
    kernel = "decode" if info[0] == 1 else "fwd"
    shape = info[1] if kernel == "decode" else ("wave1", "wave4", "wave4x2", "wave4x2x16")[info[1]]
    out = {"kernel": kernel, "shape": shape, "splits": info[2], "tiles_per_split": info[3],
           "workgroups": info[4]}
    sp = (ctypes.c_int32 * 3)()
    check(load().ffai_attn_plan_splits(ctypes.byref(desc), sp))
    out.update(items=sp[0], split_items=(sp[1], sp[2]))
    return out


def noalloc_plan_info(desc: AttnDesc) -> dict:
    """The launch plan ffai_attn_fwd_noalloc uses for `desc` (vector-aligned operands) and the
    scratch bytes it takes."""
    info = (ctypes.c_int32 * 5)()
    nbytes = ctypes.c_size_t(0)
    check(load().ffai_attn_noalloc_plan_info(ctypes.byref(desc), info, ctypes.byref(nbytes)))
    return {"info": tuple(info), "bytes": nbytes.value}


def set_geometry_override(cus: int, xcds: int) -> None:
    """Plan for a device of `cus` CUs in `xcds` XCDs (0, 0: the current device's geometry)."""
    load().ffai_set_geometry_override(int(cus), int(xcds))


def set_fwd_split_override(items: int, pieces: int) -> None:
    """Force which fused-kernel items run as key-split pieces (0, 0: the planner's choice)."""
    load().ffai_set_fwd_split_override(int(items), int(pieces))


def get_fwd_split_override() -> tuple:
    a, b = ctypes.c_int(), ctypes.c_int()
    load().ffai_get_fwd_split_override(ctypes.byref(a), ctypes.byref(b))
    return a.value, b.value


def last_error() -> str:
    return load().ffai_attn_last_error().decode()


def check(rc: int) -> int:
    """Raise FfaiError for error codes; return FFAI_OK / FFAI_DECLINED unchanged."""
    if rc < 0:
        raise FfaiError(rc, last_error())
    return rc
