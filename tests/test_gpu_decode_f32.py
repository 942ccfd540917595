"""The reference's own decode arms on the f32-query decode kernel (decode_vec_kernel): a query row
in f32 over f16 K/V (flash_attn.rs:289-356, xattn_head_f16 :698-789, the cross-attention cache of
text_decoder.rs:771-793) and over f32 K/V (:370-399, xattn_head :595-696, the self-attention
cache), one row per head, against the oracle's restatements at the f32 bar (1e-4 max-abs).

Beside the reference's surface (attend, batch 1, K^T) the descriptor path runs batched beams with
ragged caches (rows past each length filled with inf and NaN), K as rows, bf16 K/V, a causal
position, key counts that end inside a 4-key chunk, and forced key splits merged in the launch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from ffai_amd import _lib as L
from ffai_amd import flash_attn as fa
from tests.helpers import TOL_F32, max_abs, randn, round_bf16

pytestmark = pytest.mark.gpu


def _dev(x: np.ndarray, dtype, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def _kernel_of(q, k, v, out, **kw) -> str:
    return fa.plan(q, k, v, out, **kw)["kernel"]


@pytest.mark.parametrize("kv", ["f16", "f32"])
@pytest.mark.parametrize("keys", [8, 37, 448, 1500])
def test_reference_arm_h16(gpu, kv, keys):
    """attend() at the whisper-medium decoder's 16 heads: f16 K/V (the cross-attention arm) and f32
    K/V (the self-attention arm), q pre-scaled as the reference's callers pass it."""
    rng = np.random.default_rng(300 + keys)
    q = randn(rng, (1, 16, 1, 64)) * np.float32(0.125)
    kt = randn(rng, (1, 16, 64, keys))
    v = randn(rng, (1, 16, keys, 64))
    tdt = torch.float16 if kv == "f16" else torch.float32
    if kv == "f16":
        kt, v = kt.astype(np.float16), v.astype(np.float16)
    qd, ktd, vd = _dev(q, torch.float32, gpu), _dev(kt, tdt, gpu), _dev(v, tdt, gpu)
    out = torch.empty(1, 16, 1, 64, device=gpu)
    assert _kernel_of(qd, ktd, vd, out, k_transposed=True) == "decode"
    got = fa.attend(qd, ktd, vd)
    assert got is not None
    want = oracle.attend_f16kv(q, kt, v) if kv == "f16" else oracle.attend_f32(q, kt, v)
    err = max_abs(got.cpu().numpy(), want)
    print(f"f32-query decode {kv} K/V, 16 heads x {keys} keys: {err:.3e}")
    assert err < TOL_F32


@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("k_transposed", [True, False])
def test_batched_ragged_beams(gpu, kv_dtype, k_transposed):
    """Five beams' self-attention in one call: per-beam caches of capacity 448 with lengths
    {1, 37, 200, 447, 448}, the rows past each length filled with inf and NaN (never read into
    the result), 16 heads."""
    rng = np.random.default_rng(310)
    b, h, cap = 5, 16, 448
    lens = np.array([1, 37, 200, 447, 448], np.int32)
    q = randn(rng, (b, h, 1, 64)) * np.float32(0.125)
    k = randn(rng, (b, h, cap, 64))
    v = randn(rng, (b, h, cap, 64))
    if kv_dtype == torch.bfloat16:
        k, v = round_bf16(k), round_bf16(v)
    elif kv_dtype == torch.float16:
        k, v = k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)
    want = oracle.attend_general(q, k, v, k_transposed=False, kv_lens=lens)
    kg, vg = k.copy(), v.copy()
    for i, n in enumerate(lens):
        kg[i, :, n:] = np.inf
        vg[i, :, n:] = np.nan
    kd = _dev(np.swapaxes(kg, 2, 3) if k_transposed else kg, kv_dtype, gpu)
    vd = _dev(vg, kv_dtype, gpu)
    qd = _dev(q, torch.float32, gpu)
    out = torch.empty(b, h, 1, 64, device=gpu)
    kl = _dev(lens, torch.int32, gpu)
    assert _kernel_of(qd, kd, vd, out, k_transposed=k_transposed, kv_lens=kl) == "decode"
    fa.attention(qd, kd, vd, k_transposed=k_transposed, kv_lens=kl, out=out)
    err = max_abs(out.cpu().numpy(), want)
    print(f"f32-query decode, 5 ragged beams, {kv_dtype}, kt={k_transposed}: {err:.3e}")
    assert err < TOL_F32


@pytest.mark.parametrize("keys", [1, 3, 5, 63, 65, 1499, 1501])
@pytest.mark.parametrize("k_transposed", [True, False])
def test_key_counts_ending_inside_a_chunk(gpu, keys, k_transposed):
    """Key counts that end inside a 4-key chunk of K^T, or below 4 keys (the chunk clamped
    element by element), and tails of 1 and 63 keys past a whole tile; scale given by the
    descriptor instead of folded into q. K^T is a view of a cache whose rows hold a multiple of 8
    keys (the capacity), as a growing cache would be."""
    rng = np.random.default_rng(320 + keys)
    q = randn(rng, (1, 4, 1, 64))
    k = randn(rng, (1, 4, keys, 64))
    v = randn(rng, (1, 4, keys, 64))
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125)
    if k_transposed:
        cap = -(-keys // 8) * 8
        full = torch.full((1, 4, 64, cap), float("nan"), device=gpu)
        full[..., :keys] = _dev(np.swapaxes(k, 2, 3), torch.float32, gpu)
        kd = full[..., :keys]
    else:
        kd = _dev(k, torch.float32, gpu)
    vd = _dev(v, torch.float32, gpu)
    qd = _dev(q, torch.float32, gpu)
    out = torch.empty(1, 4, 1, 64, device=gpu)
    assert _kernel_of(qd, kd, vd, out, k_transposed=k_transposed, scale=0.125) == "decode"
    fa.attention(qd, kd, vd, k_transposed=k_transposed, scale=0.125, out=out)
    err = max_abs(out.cpu().numpy(), want)
    print(f"f32-query decode K{keys} kt={k_transposed}: {err:.3e}")
    assert err < TOL_F32


@pytest.mark.parametrize("pos", [0, 5, 700, 1499])
def test_causal_position(gpu, pos):
    """One causal query row at position `pos` over a 1500-key cache: keys after it are hidden."""
    rng = np.random.default_rng(330 + pos)
    q = randn(rng, (1, 8, 1, 64)) * np.float32(0.125)
    kt = randn(rng, (1, 8, 64, 1500)).astype(np.float16)
    v = randn(rng, (1, 8, 1500, 64)).astype(np.float16)
    want = oracle.attend_general(q, kt, v, k_transposed=True, causal=True, q_offset=pos)
    out = torch.empty(1, 8, 1, 64, device=gpu)
    fa.attention(_dev(q, torch.float32, gpu), _dev(kt, torch.float16, gpu),
                 _dev(v, torch.float16, gpu), k_transposed=True, causal=True, q_offset=pos,
                 out=out)
    err = max_abs(out.cpu().numpy(), want)
    print(f"f32-query decode causal at {pos}: {err:.3e}")
    assert err < TOL_F32


@pytest.mark.parametrize("tiles_per_wg", [1, 2, 3, 5, 24])
def test_forced_key_splits(gpu, tiles_per_wg):
    """The cross-attention arm's keys split over workgroups (partials merged by each head's last
    workgroup in the launch), 1 to 24 tiles per workgroup, two calls through one workspace."""
    rng = np.random.default_rng(340)
    q = randn(rng, (1, 16, 1, 64)) * np.float32(0.125)
    kt = randn(rng, (1, 16, 64, 1500)).astype(np.float16)
    v = randn(rng, (1, 16, 1500, 64)).astype(np.float16)
    want = oracle.attend_f16kv(q, kt, v)
    prev = L.load().ffai_get_decode_tiles_per_wg()
    L.load().ffai_set_decode_tiles_per_wg(tiles_per_wg)
    try:
        qd, kd, vd = _dev(q, torch.float32, gpu), _dev(kt, torch.float16, gpu), _dev(v, torch.float16, gpu)
        out = torch.empty(1, 16, 1, 64, device=gpu)
        info = fa.plan(qd, kd, vd, out, k_transposed=True)
        assert info["kernel"] == "decode" and info["tiles_per_split"] == tiles_per_wg
        for _ in range(2):
            out.fill_(float("nan"))
            fa.attention(qd, kd, vd, k_transposed=True, out=out)
            err = max_abs(out.cpu().numpy(), want)
            assert err < TOL_F32, err
        print(f"f32-query decode, {info['splits']} splits of {tiles_per_wg} tiles: {err:.3e}")
    finally:
        L.load().ffai_set_decode_tiles_per_wg(prev)


def test_graph_replay_matches_eager(gpu):
    """A captured call replays bit-identically to the eager call, several times with eager work
    between the replays (the split counters reset by the launch itself)."""
    rng = np.random.default_rng(350)
    q = _dev(randn(rng, (1, 16, 1, 64)) * np.float32(0.125), torch.float32, gpu)
    kt = _dev(randn(rng, (1, 16, 64, 1500)), torch.float16, gpu)
    v = _dev(randn(rng, (1, 16, 1500, 64)), torch.float16, gpu)
    eager = torch.empty(1, 16, 1, 64, device=gpu)
    fa.attention(q, kt, v, k_transposed=True, out=eager)
    ws = torch.zeros(max(16, fa.workspace_bytes(q, kt, v, eager, k_transposed=True)),
                     dtype=torch.uint8, device=gpu)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        fa.attention(q, kt, v, k_transposed=True, out=out, workspace=ws)
    for i in range(4):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        fa.attention(q, kt, v, k_transposed=True, out=eager)  # eager work between replays
