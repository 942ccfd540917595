"""The allocation-free entry point ffai_attn_fwd_noalloc against ffai_attn_fwd, through the C ABI.

ffai_attn_fwd_noalloc runs ffai_attn_fwd's plan and kernels with the split-key partials in the
library's per-device scratch instead of a caller workspace. Where ffai_attn_fwd's plan fits the
scratch (every shape below) the plans are the same, so on the same inputs its output must equal
ffai_attn_fwd's bit for bit; a larger plan runs with fewer key pieces (checked on the CPU). Each
GPU case makes two calls in a row, the second on a smaller input, so the second call runs over
the partials the first one left in the scratch.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from ffai_amd import _lib as L
from ffai_amd import flash_attn as fa


def _desc(q, k, v, out, **kw):
    return fa.make_desc(q, k, v, out, k_transposed=kw.get("k_transposed", False),
                        scale=kw.get("scale", 1.0), causal=kw.get("causal", False),
                        q_offset=kw.get("q_offset", 0), kv_lens=kw.get("kv_lens"))


def _both(lib, q, k, v, **kw):
    """Output of ffai_attn_fwd (with a workspace) and of ffai_attn_fwd_noalloc."""
    out_dtype = kw.pop("out_dtype")
    shape = (q.shape[0], q.shape[1], q.shape[2], v.shape[3])
    o_ws = torch.full(shape, float("nan"), dtype=out_dtype, device=q.device)
    o_na = torch.full(shape, float("nan"), dtype=out_dtype, device=q.device)
    d = _desc(q, k, v, o_ws, **kw)
    n = ctypes.c_size_t(0)
    assert lib.ffai_attn_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == L.FFAI_OK
    ws = torch.zeros(max(n.value, 16), dtype=torch.uint8, device=q.device)
    stream = fa._stream_handle()
    rc = lib.ffai_attn_fwd(ctypes.byref(d), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                           o_ws.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    assert rc == L.FFAI_OK, L.last_error()
    d = _desc(q, k, v, o_na, **kw)
    rc = lib.ffai_attn_fwd_noalloc(ctypes.byref(d), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   o_na.data_ptr(), stream)
    assert rc == L.FFAI_OK, L.last_error()
    torch.cuda.synchronize()
    return o_ws, o_na, n.value


def _rand(shape, dtype, dev, gen, mult=1.0):
    return (torch.randn(shape, generator=gen, device=dev) * mult).to(dtype)


def _check(o_ws, o_na, what):
    assert torch.isfinite(o_ws.float()).all(), what
    assert torch.equal(o_ws, o_na), (what, (o_ws.float() - o_na.float()).abs().max().item())


@pytest.mark.gpu
def test_decode_splits_twice(gpu):
    """Beam-5 cross-attention (5 rows over 1500 shared frames, 16 heads: split keys, partials
    in the scratch), then a smaller one (3 rows over 700 frames, 8 heads)."""
    lib = L.load()
    g = torch.Generator(device=gpu).manual_seed(70)
    for heads, rows, frames in ((16, 5, 1500), (8, 3, 700)):
        q = _rand((1, heads, rows, 64), torch.bfloat16, gpu, g)
        kt = _rand((1, heads, 64, frames), torch.bfloat16, gpu, g)
        v = _rand((1, heads, frames, 64), torch.bfloat16, gpu, g)
        o_ws, o_na, nbytes = _both(lib, q, kt, v, k_transposed=True, scale=0.125,
                                   out_dtype=torch.float32)
        assert nbytes > 0  # the plan splits the keys
        _check(o_ws, o_na, f"decode {heads}x{rows}x{frames}")


@pytest.mark.gpu
def test_encoder_splits_twice(gpu):
    """whisper-tiny f32 encoder (6 heads x 1500 rows: four-wave blocks with the keys split, ~7
    MB of partials), then a smaller f32 one (2 heads x 300 rows), then a 16-bit prompt-step
    shape (one-wave blocks, split keys, 228 rows x 16 heads over 1500 frames)."""
    lib = L.load()
    g = torch.Generator(device=gpu).manual_seed(71)
    for heads, t in ((6, 1500), (2, 300)):
        q = _rand((1, heads, t, 64), torch.float32, gpu, g, 0.125)
        kt = _rand((1, heads, 64, t), torch.float32, gpu, g)
        v = _rand((1, heads, t, 64), torch.float32, gpu, g)
        o_ws, o_na, nbytes = _both(lib, q, kt, v, k_transposed=True, out_dtype=torch.float32)
        assert nbytes > 0
        _check(o_ws, o_na, f"encoder f32 {heads}x{t}")
    q = _rand((1, 16, 228, 64), torch.bfloat16, gpu, g)
    kt = _rand((1, 16, 64, 1500), torch.bfloat16, gpu, g)
    v = _rand((1, 16, 1500, 64), torch.bfloat16, gpu, g)
    o_ws, o_na, nbytes = _both(lib, q, kt, v, k_transposed=True, scale=0.125,
                               out_dtype=torch.float32)
    assert nbytes > 0
    _check(o_ws, o_na, "prompt-step cross-attention")


@pytest.mark.gpu
def test_balance_splits_twice(gpu):
    """The splits made for balance only: whisper-small bf16 (B8 H12 T1500, its last 64 items in
    4 key pieces, ~17 MB of partials), then the smaller Qwen2-VL-2B causal prefill (Hq12 Hkv2
    S4096 D128, its 192 longest items in 2 pieces, ~26 MB)."""
    lib = L.load()
    g = torch.Generator(device=gpu).manual_seed(73)
    q = _rand((8, 12, 1500, 64), torch.bfloat16, gpu, g)
    kt = _rand((8, 12, 64, 1500), torch.bfloat16, gpu, g, 2.0)
    v = _rand((8, 12, 1500, 64), torch.bfloat16, gpu, g)
    o_ws, o_na, nbytes = _both(lib, q, kt, v, k_transposed=True, scale=0.125,
                               out_dtype=torch.bfloat16)
    assert nbytes > 0
    _check(o_ws, o_na, "whisper-small tail pieces")
    q = _rand((1, 12, 4096, 128), torch.bfloat16, gpu, g)
    k = _rand((1, 2, 4096, 128), torch.bfloat16, gpu, g)
    v = _rand((1, 2, 4096, 128), torch.bfloat16, gpu, g)
    o_ws, o_na, nbytes = _both(lib, q, k, v, scale=128 ** -0.5, causal=True,
                               out_dtype=torch.bfloat16)
    assert nbytes > 0
    _check(o_ws, o_na, "causal prefill longest pieces")


@pytest.mark.gpu
def test_unsplit_shape_needs_no_scratch(gpu):
    """A shape without partials (4 x 20 heads x 1500 rows, bf16) runs the same through both."""
    lib = L.load()
    g = torch.Generator(device=gpu).manual_seed(72)
    q = _rand((4, 20, 1500, 64), torch.bfloat16, gpu, g)
    kt = _rand((4, 20, 64, 1500), torch.bfloat16, gpu, g)
    v = _rand((4, 20, 1500, 64), torch.bfloat16, gpu, g)
    o_ws, o_na, nbytes = _both(lib, q, kt, v, k_transposed=True, scale=0.125,
                               out_dtype=torch.bfloat16)
    assert nbytes == 0
    _check(o_ws, o_na, "unsplit encoder")


def test_refuses_partials_above_the_scratch():
    """A plan whose partials exceed the scratch is refused before any GPU call: four
    whisper-large-v3 windows (480 items of 256 rows) forced into 8 key pieces each, ~259 MB of
    partials."""
    lib = L.load()
    cap = lib.ffai_attn_noalloc_scratch_bytes()
    assert cap == 48 << 20
    d = L.AttnDesc()
    lib.ffai_attn_desc_init(ctypes.byref(d), L.BF16, L.BF16, L.BF16, 4, 20, 20, 1500, 1500, 64,
                            L.K_TRANSPOSED)
    prev = L.get_fwd_split_override()
    L.set_fwd_split_override(-1, 8)
    try:
        n = ctypes.c_size_t(0)
        assert lib.ffai_attn_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == L.FFAI_OK
        assert n.value > cap
        fake = 0x10000
        rc = lib.ffai_attn_fwd_noalloc(ctypes.byref(d), fake, fake, fake, fake, None)
        assert rc == L.FFAI_ERR_WORKSPACE
        assert "allocation-free" in L.last_error()
        # a descriptor the path declines is declined, as by ffai_attn_fwd
        d.head_dim = 96
        assert lib.ffai_attn_fwd_noalloc(ctypes.byref(d), fake, fake, fake, fake,
                                         None) == L.FFAI_DECLINED
    finally:
        L.set_fwd_split_override(*prev)


@pytest.mark.parametrize("args", [
    # f32, head_dim 64, 42 heads x 3000 rows: ffai_attn_fwd plans ~68 MB of partials
    (L.F32, L.F32, L.F32, 1, 42, 42, 3000, 3000, 64, L.K_TRANSPOSED, 0),
    # bf16 causal, 256 heads x 300 rows: a ~66 MB split for balance
    (L.BF16, L.BF16, L.BF16, 1, 256, 256, 300, 300, 64, L.K_ROWS, 1),
    # the workloads' shapes, whose plans fit
    (L.F32, L.F32, L.F32, 1, 6, 6, 1500, 1500, 64, L.K_TRANSPOSED, 0),
    (L.BF16, L.BF16, L.BF16, 8, 12, 12, 1500, 1500, 64, L.K_TRANSPOSED, 0),
    (L.BF16, L.BF16, L.BF16, 16, 20, 20, 1500, 1500, 64, L.K_TRANSPOSED, 0),
    (L.BF16, L.BF16, L.BF16, 1, 12, 2, 4096, 4096, 128, L.K_ROWS, 1),
    (L.BF16, L.BF16, L.F32, 5, 16, 16, 1, 1500, 64, L.K_ROWS, 0),
    (L.F32, L.F16, L.F32, 1, 16, 16, 1, 1500, 64, L.K_TRANSPOSED, 0),
    # large decode grids: many units, long caches
    (L.BF16, L.BF16, L.F32, 256, 32, 8, 4, 32768, 128, L.K_ROWS, 0),
    (L.F16, L.F16, L.F16, 1024, 16, 16, 1, 8192, 64, L.K_ROWS, 0),
    (L.F32, L.F32, L.F32, 64, 40, 40, 700, 700, 64, L.K_ROWS, 0),
])
def test_noalloc_plan_is_the_fwd_plan_capped_to_the_scratch(args):
    """ffai_attn_fwd_noalloc's plan equals ffai_attn_fwd's whenever that plan's partials fit the
    scratch; otherwise it keeps the kernel and launch shape and takes fewer key pieces, within
    the scratch. No default plan is refused."""
    lib = L.load()
    cap = lib.ffai_attn_noalloc_scratch_bytes()
    *dims, layout, causal = args
    d = L.AttnDesc()
    lib.ffai_attn_desc_init(ctypes.byref(d), *dims, layout)
    d.causal = causal
    n = ctypes.c_size_t(0)
    assert lib.ffai_attn_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == L.FFAI_OK
    fwd = L.plan_info(d)
    fwd_info = (1 if fwd["kernel"] == "decode" else 0,
                fwd["shape"] if fwd["kernel"] == "decode" else
                ("wave1", "wave4", "wave4x2", "wave4x2x16").index(fwd["shape"]),
                fwd["splits"], fwd["tiles_per_split"], fwd["workgroups"])
    na = L.noalloc_plan_info(d)
    assert na["bytes"] <= cap
    if n.value <= cap:
        assert na["info"] == fwd_info
    else:
        assert na["info"][:2] == fwd_info[:2] and na["info"][2] < fwd_info[2]
