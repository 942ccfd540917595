"""GPU parity of the decode launch (at most 32 query rows per K/V head), through the C ABI,
against the CPU oracle. These shapes take decode_kernel (and decode_combine_kernel when the keys
are split): beams stacked as rows over a shared cross-attention cache, grouped query heads, a few
causal tokens, ragged and empty caches, unaligned operands, and workspaces reused across calls
and HIP graph replays."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from ffai_amd import _lib as L
from ffai_amd import flash_attn as fa
from tests.helpers import TOL_BF16, max_abs, randn, round_bf16, round_f16

pytestmark = pytest.mark.gpu


def _dev(x: np.ndarray, dtype, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def _host(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


@pytest.mark.parametrize("tk", [4096, 777])
def test_gqa_decode_d128(gpu, tk):
    """Qwen2-VL-2B-shape decode: 12 query heads over 2 K/V heads, head_dim 128, one new token
    at the end of a cache of tk keys (causal at offset tk - 1 sees every key)."""
    rng = np.random.default_rng(tk)
    hq, hkv, d = 12, 2, 128
    q = round_bf16(randn(rng, (1, hq, 1, d)))
    k = round_bf16(randn(rng, (1, hkv, tk, d)))
    v = round_bf16(randn(rng, (1, hkv, tk, d)))
    scale = d ** -0.5
    out = fa.attention(_dev(q, torch.bfloat16, gpu), _dev(k, torch.bfloat16, gpu),
                       _dev(v, torch.bfloat16, gpu), scale=scale, causal=True, q_offset=tk - 1,
                       out_dtype=torch.float32)
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=scale, causal=True,
                                 q_offset=tk - 1)
    err = max_abs(_host(out), want)
    print(f"gqa decode d128 tk{tk}: {err:.3e}")
    assert err < TOL_BF16


def test_multi_token_causal_f16(gpu):
    """Four new tokens per sequence (group 4 -> 16 rows per K/V head), causal at offset 296 of
    300 keys, f16 in and out, K transposed."""
    rng = np.random.default_rng(11)
    b, hq, hkv, tq, tk, d = 2, 8, 2, 4, 300, 64
    q = round_f16(randn(rng, (b, hq, tq, d)))
    kt = round_f16(randn(rng, (b, hkv, d, tk)))
    v = round_f16(randn(rng, (b, hkv, tk, d)))
    out = fa.attention(_dev(q, torch.float16, gpu), _dev(kt, torch.float16, gpu),
                       _dev(v, torch.float16, gpu), k_transposed=True, scale=0.125, causal=True,
                       q_offset=296)
    assert out.dtype == torch.float16
    want = oracle.attend_general(q, kt, v, k_transposed=True, scale=0.125, causal=True,
                                 q_offset=296)
    err = max_abs(_host(out), want)
    print(f"multi-token causal f16: {err:.3e}")
    assert err < TOL_BF16


def test_thirty_two_rows_bf16_out(gpu):
    """The largest unit: group 8 x 4 tokens = 32 rows over one K/V head, bf16 output."""
    rng = np.random.default_rng(32)
    b, hq, hkv, tq, tk, d = 1, 16, 2, 4, 1000, 64
    q = round_bf16(randn(rng, (b, hq, tq, d)))
    k = round_bf16(randn(rng, (b, hkv, tk, d)))
    v = round_bf16(randn(rng, (b, hkv, tk, d)))
    out = fa.attention(_dev(q, torch.bfloat16, gpu), _dev(k, torch.bfloat16, gpu),
                       _dev(v, torch.bfloat16, gpu), scale=0.125)
    assert out.dtype == torch.bfloat16
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125)
    err = max_abs(_host(out), want)
    print(f"32 rows bf16 out: {err:.3e}")
    assert err < TOL_BF16


def test_ragged_caches_with_empty_one(gpu):
    """Per-beam cache lengths including an empty cache (its rows come out zero, as in the
    oracle) and lengths on and off the 64-key tile edges."""
    rng = np.random.default_rng(7)
    beams, h, cap, d = 6, 4, 448, 64
    lens = np.array([0, 1, 63, 64, 65, 448], np.int32)
    q = round_bf16(randn(rng, (beams, h, 1, d)))
    k = round_bf16(randn(rng, (beams, h, cap, d)))
    v = round_bf16(randn(rng, (beams, h, cap, d)))
    out = fa.attention(_dev(q, torch.bfloat16, gpu), _dev(k, torch.bfloat16, gpu),
                       _dev(v, torch.bfloat16, gpu), scale=0.125,
                       kv_lens=torch.from_numpy(lens).to(gpu), out_dtype=torch.float32)
    got = _host(out)
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125, kv_lens=lens)
    assert np.all(got[0] == 0.0)
    err = max_abs(got, want)
    print(f"ragged with empty cache: {err:.3e}")
    assert err < TOL_BF16


@pytest.mark.parametrize("k_transposed", [False, True])
def test_ragged_caches_with_garbage_past_the_end(gpu, k_transposed):
    """Cache rows past each beam's length hold inf and NaN (stale or never written): a tail tile
    inside the cache's capacity arrives whole by DMA and only the valid keys may count."""
    rng = np.random.default_rng(8)
    beams, h, cap, d = 5, 4, 448, 64
    lens = np.array([1, 63, 100, 383, 447], np.int32)
    q = round_bf16(randn(rng, (beams, h, 1, d)))
    k = round_bf16(randn(rng, (beams, h, cap, d)))
    v = round_bf16(randn(rng, (beams, h, cap, d)))
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125, kv_lens=lens)
    for bi, n in enumerate(lens):
        k[bi, :, n:] = np.nan
        v[bi, :, n:: 2] = np.inf
        v[bi, :, n + 1:: 2] = np.nan
    kd = _dev(np.swapaxes(k, 2, 3) if k_transposed else k, torch.bfloat16, gpu)
    out = fa.attention(_dev(q, torch.bfloat16, gpu), kd, _dev(v, torch.bfloat16, gpu),
                       k_transposed=k_transposed, scale=0.125,
                       kv_lens=torch.from_numpy(lens).to(gpu), out_dtype=torch.float32)
    got = _host(out)
    assert np.isfinite(got).all()
    err = max_abs(got, want)
    print(f"ragged with garbage past the end (k_transposed={k_transposed}): {err:.3e}")
    assert err < TOL_BF16


@pytest.mark.parametrize("d,k_transposed,tk,cut", [(64, True, 1500, 0), (64, True, 1500, 3),
                                                   (64, True, 1484, 0), (64, False, 1503, 2),
                                                   (128, True, 1500, 5), (128, False, 72, 0),
                                                   (64, True, 72, 1)])
def test_last_tile_past_the_operand_end(gpu, d, k_transposed, tk, cut):
    """The operand's last tile holds fewer than 64 keys (1500 frames: 28): it arrives by DMA with
    sources clamped inside the operand, and the valid keys of the K^T chunk that crosses the end
    are patched. `cut` > 0 ends the valid keys (kv_lens) inside that tile, short of the end."""
    rng = np.random.default_rng(tk + d)
    rows, h = 5, 4
    q = round_bf16(randn(rng, (1, h, rows, d)))
    k = round_bf16(randn(rng, (1, h, tk, d)))
    v = round_bf16(randn(rng, (1, h, tk, d)))
    lens = np.array([tk - cut], np.int32)
    kd = _dev(np.swapaxes(k, 2, 3) if k_transposed else k, torch.bfloat16, gpu)
    out = fa.attention(_dev(q, torch.bfloat16, gpu), kd, _dev(v, torch.bfloat16, gpu),
                       k_transposed=k_transposed, scale=d ** -0.5,
                       kv_lens=torch.from_numpy(lens).to(gpu) if cut else None,
                       out_dtype=torch.float32)
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=d ** -0.5,
                                 kv_lens=lens if cut else None)
    err = max_abs(_host(out), want)
    print(f"last tile past the end d{d} kt{int(k_transposed)} tk{tk} cut{cut}: {err:.3e}")
    assert err < TOL_BF16


def test_unaligned_operands(gpu):
    """Operands offset by one element from 16-byte boundaries take the element-wise loads."""
    rng = np.random.default_rng(5)
    b, h, tk, d = 5, 4, 333, 64
    q = round_bf16(randn(rng, (b, h, 1, d)))
    k = round_bf16(randn(rng, (b, h, tk, d)))
    v = round_bf16(randn(rng, (b, h, tk, d)))

    def shifted(x):
        flat = torch.zeros(x.size + 1, dtype=torch.bfloat16, device=gpu)
        flat[1:] = _dev(x.reshape(-1), torch.bfloat16, gpu)
        return flat[1:].view(*x.shape)

    out_flat = torch.zeros(b * h * d + 1, dtype=torch.float32, device=gpu)
    out = out_flat[1:].view(b, h, 1, d)
    res = fa.attention(shifted(q), shifted(k), shifted(v), scale=0.125, out=out)
    assert res is not None
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125)
    err = max_abs(_host(out), want)
    print(f"unaligned decode: {err:.3e}")
    assert err < TOL_BF16


def test_many_units_without_split(gpu):
    """Enough (batch, head) units that each takes its keys in one workgroup (no workspace)."""
    rng = np.random.default_rng(64)
    b, h, tk, d = 64, 16, 200, 64
    q = round_bf16(randn(rng, (b, h, 1, d)))
    k = round_bf16(randn(rng, (b, h, tk, d)))
    v = round_bf16(randn(rng, (b, h, tk, d)))
    qd, kd, vd = (_dev(x, torch.bfloat16, gpu) for x in (q, k, v))
    o = torch.empty(b, h, 1, d, dtype=torch.float32, device=gpu)
    assert fa.workspace_bytes(qd, kd, vd, o, scale=0.125) == 0
    fa.attention(qd, kd, vd, scale=0.125, out=o)
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125)
    err = max_abs(_host(o), want)
    print(f"no-split decode: {err:.3e}")
    assert err < TOL_BF16


def _beam_cross_inputs(rng, gpu, beams=5, h=16, t=1500, d=64):
    q = round_bf16(randn(rng, (beams, h, 1, d)))
    kt = round_bf16(randn(rng, (1, h, d, t)))
    v = round_bf16(randn(rng, (1, h, t, d)))
    return q, kt, v, _dev(q, torch.bfloat16, gpu), _dev(kt, torch.bfloat16, gpu), _dev(v, torch.bfloat16, gpu)


COUNTER_BYTES = 4096  # the split counters at the workspace's start


def test_workspace_reuse_and_graph_replays(gpu):
    """One workspace, zeroed once, serves repeated eager calls and every replay of a captured HIP
    graph (with eager work and synchronisation between replays): each result matches the first
    eager one exactly and the oracle within tolerance, and the split counters are back at zero
    after every call. Past the counters the workspace starts as garbage (0xFF): partials are
    written before they are read."""
    rng = np.random.default_rng(2024)
    q, kt, v, qd, ktd, vd = _beam_cross_inputs(rng, gpu)
    beams, h, _, d = q.shape
    out = torch.empty(beams, h, 1, d, dtype=torch.float32, device=gpu)
    args = dict(k_transposed=True, scale=0.125)
    nbytes = fa.workspace_bytes(qd.permute(2, 1, 0, 3), ktd, vd, out.permute(2, 1, 0, 3), **args)
    assert nbytes > 0
    ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device=gpu)
    ws[:COUNTER_BYTES].zero_()

    def call():
        fa.attention(qd.permute(2, 1, 0, 3), ktd, vd, out=out.permute(2, 1, 0, 3),
                     workspace=ws, **args)

    call()
    torch.cuda.synchronize()
    first = out.clone()
    want = np.swapaxes(oracle.attend_general(np.swapaxes(q, 0, 2), kt, v, **args), 0, 2)
    err = max_abs(_host(first), want)
    print(f"graph test eager: {err:.3e}")
    assert err < TOL_BF16
    for _ in range(3):
        out.zero_()
        call()
        torch.cuda.synchronize()
        assert torch.equal(out, first)
        assert not ws[:COUNTER_BYTES].any()

    graph = torch.cuda.CUDAGraph()
    out.zero_()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        call()
    for i in range(5):
        out.fill_(float(i + 1))     # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first), f"replay {i} differs"
        assert not ws[:COUNTER_BYTES].any(), f"replay {i} left a counter set"


@pytest.fixture
def tiles_knob():
    lib = L.load()
    yield lib.ffai_set_decode_tiles_per_wg
    lib.ffai_set_decode_tiles_per_wg(0)


@pytest.mark.parametrize("tiles_per_wg", [1, 3, 24])
def test_split_merge_never_reads_stale_partials(gpu, tiles_per_wg, tiles_knob):
    """Two beam-5 cross-attention problems alternate 12 times on one workspace. Each call's last
    workgroup merges partials the same call wrote; a stale partial (the other problem's) would
    change the output, so every call must equal its problem's first result bit for bit, for
    splits of 1, 3 and 24 tiles (24, 8 and 1 workgroups per head)."""
    rng = np.random.default_rng(77)
    cases = [_beam_cross_inputs(rng, gpu), _beam_cross_inputs(rng, gpu)]
    beams, h, _, d = cases[0][0].shape
    args = dict(k_transposed=True, scale=0.125)
    outs = [torch.empty(beams, h, 1, d, dtype=torch.float32, device=gpu) for _ in cases]
    nbytes = fa.workspace_bytes(cases[0][3].permute(2, 1, 0, 3), cases[0][4], cases[0][5],
                                outs[0].permute(2, 1, 0, 3), **args)
    tiles_knob(tiles_per_wg)
    nbytes = max(nbytes, fa.workspace_bytes(cases[0][3].permute(2, 1, 0, 3), cases[0][4],
                                            cases[0][5], outs[0].permute(2, 1, 0, 3), **args))
    ws = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=gpu)
    first = [None, None]
    for i in range(24):
        c = i % 2
        _, _, _, qd, ktd, vd = cases[c]
        outs[c].zero_()
        fa.attention(qd.permute(2, 1, 0, 3), ktd, vd, out=outs[c].permute(2, 1, 0, 3),
                     workspace=ws, **args)
        torch.cuda.synchronize()
        if first[c] is None:
            q, kt, v = cases[c][:3]
            want = np.swapaxes(oracle.attend_general(np.swapaxes(q, 0, 2), kt, v, **args), 0, 2)
            assert max_abs(_host(outs[c]), want) < TOL_BF16
            first[c] = outs[c].clone()
        else:
            assert torch.equal(outs[c], first[c]), f"call {i} differs"
    assert not ws[:COUNTER_BYTES].any()


def test_two_calls_share_nothing_but_the_workspace(gpu):
    """Back-to-back calls with different inputs on one workspace (stream-ordered): the second
    sees no state from the first."""
    rng = np.random.default_rng(99)
    q1, kt1, v1, qd1, ktd1, vd1 = _beam_cross_inputs(rng, gpu)
    q2, kt2, v2, qd2, ktd2, vd2 = _beam_cross_inputs(rng, gpu, t=700)
    beams, h, _, d = q1.shape
    args = dict(k_transposed=True, scale=0.125)
    o1 = torch.empty(beams, h, 1, d, dtype=torch.float32, device=gpu)
    o2 = torch.empty_like(o1)
    n = max(fa.workspace_bytes(qd1.permute(2, 1, 0, 3), ktd1, vd1, o1.permute(2, 1, 0, 3), **args),
            fa.workspace_bytes(qd2.permute(2, 1, 0, 3), ktd2, vd2, o2.permute(2, 1, 0, 3), **args))
    ws = torch.zeros(n, dtype=torch.uint8, device=gpu)
    fa.attention(qd1.permute(2, 1, 0, 3), ktd1, vd1, out=o1.permute(2, 1, 0, 3), workspace=ws, **args)
    fa.attention(qd2.permute(2, 1, 0, 3), ktd2, vd2, out=o2.permute(2, 1, 0, 3), workspace=ws, **args)
    w1 = np.swapaxes(oracle.attend_general(np.swapaxes(q1, 0, 2), kt1, v1, **args), 0, 2)
    w2 = np.swapaxes(oracle.attend_general(np.swapaxes(q2, 0, 2), kt2, v2, **args), 0, 2)
    e1, e2 = max_abs(_host(o1), w1), max_abs(_host(o2), w2)
    print(f"shared workspace: {e1:.3e} {e2:.3e}")
    assert e1 < TOL_BF16 and e2 < TOL_BF16
