"""GPU parity of the device-resident decode-step state (include/ffai_kv.h) against the oracle's
restatement of the reference (oracle/kvcache.py): append in place vs Tensor::cat, gather by
parent vs per-beam snapshot/restore, the cross-attention cache build, and a beam decode loop
that attends over the device state, all compared with the reference's own operations."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import kvcache as okv
from ffai_amd import flash_attn as fa
from ffai_amd.kv_cache import KVCache, cross_kv_build
from tests.helpers import TOL_BF16, max_abs, randn

pytestmark = pytest.mark.gpu

TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _dev(x, dtype, device):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


@pytest.mark.parametrize("src,dst", [("f32", "bf16"), ("f32", "f16"), ("bf16", "bf16"), ("f32", "f32")])
def test_append_matches_concatenation(gpu, src, dst):
    """Ragged starting lengths (one at capacity) + two appends of 2 and 1 rows: the valid prefix of
    every slot equals split_heads of the reference's concatenated cache, bit for bit."""
    rng = np.random.default_rng(10)
    slots, heads, d, cap = 5, 4, 64, 80
    start = np.array([0, 3, 40, 78, 80], np.int32)
    cache = KVCache(slots, heads, cap, d, TDT[dst], gpu)
    # initial contents: the oracle's cache for each slot, written through append of `start` rows
    ref_k = [okv.round_to(randn(rng, (1, int(n), heads * d)), src) for n in start]
    ref_v = [okv.round_to(randn(rng, (1, int(n), heads * d)), src) for n in start]
    for s in range(slots):
        if start[s]:
            one = KVCache(1, heads, cap, d, TDT[dst], gpu)
            one.append(_dev(ref_k[s], TDT[src], gpu), _dev(ref_v[s], TDT[src], gpu))
            cache.k[s], cache.v[s] = one.k[0], one.v[0]
    cache.lens.copy_(torch.from_numpy(start))
    for t_new in (2, 1):
        nk = okv.round_to(randn(rng, (slots, t_new, heads * d)), src)
        nv = okv.round_to(randn(rng, (slots, t_new, heads * d)), src)
        cache.append(_dev(nk, TDT[src], gpu), _dev(nv, TDT[src], gpu))
        for s in range(slots):
            ref_k[s] = okv.self_cache_append(ref_k[s], nk[s:s + 1])
            ref_v[s] = okv.self_cache_append(ref_v[s], nv[s:s + 1])
    lens = cache.lens.cpu().numpy()
    np.testing.assert_array_equal(lens, np.minimum(start + 3, cap))
    k, v = cache.k.float().cpu().numpy(), cache.v.float().cpu().numpy()
    for s in range(slots):
        n = int(lens[s])
        want_k = okv.round_to(okv.split_heads(ref_k[s], heads)[0], dst)[:, :n]
        want_v = okv.round_to(okv.split_heads(ref_v[s], heads)[0], dst)[:, :n]
        np.testing.assert_array_equal(k[s, :, :n], want_k)
        np.testing.assert_array_equal(v[s, :, :n], want_v)


@pytest.mark.parametrize("t_new", [1, 20, 200])
def test_append_clamps_lengths_out_of_range(gpu, t_new):
    """A corrupt length (negative, or above capacity) is clamped into [0, capacity] before the
    append, as the gather clamps it: rows of a slot at -1 land from position 0, a slot past
    capacity takes nothing, and no row lands outside the slot's cache. One row (one workgroup
    per slot, length advanced in the same launch), 20 rows (640 units: still one workgroup,
    three units a thread) and 200 rows (one unit a thread over several workgroups per slot,
    separate length update)."""
    rng = np.random.default_rng(17)
    slots, heads, d, cap = 3, 4, 64, 256
    cache = KVCache(slots, heads, cap, d, torch.bfloat16, gpu)
    old_k = okv.round_to(randn(rng, cache.k.shape), "bf16")
    cache.k.copy_(torch.from_numpy(old_k))
    start = np.array([-1, -1000, cap + 7], np.int32)
    cache.lens.copy_(torch.from_numpy(start))
    nk = randn(rng, (slots, t_new, heads * d))
    nv = randn(rng, (slots, t_new, heads * d))
    cache.append(_dev(nk, torch.float32, gpu), _dev(nv, torch.float32, gpu))
    lens = cache.lens.cpu().numpy()
    np.testing.assert_array_equal(lens, [min(t_new, cap), min(t_new, cap), cap])
    k = cache.k.float().cpu().numpy()
    for s in (0, 1):
        want = okv.round_to(okv.split_heads(nk[s:s + 1], heads)[0], "bf16")
        np.testing.assert_array_equal(k[s, :, :t_new], want)
        np.testing.assert_array_equal(k[s, :, t_new:], old_k[s, :, t_new:])
    np.testing.assert_array_equal(k[2], old_k[2])  # a slot past capacity is untouched


def test_long_append_spans_workgroups(gpu):
    """A 200-row append (a prompt's size: 25600 8-element units per slot, several workgroups per
    slot and a separate length update) into ragged slots, one of which runs past capacity."""
    rng = np.random.default_rng(16)
    slots, heads, d, cap, t_new = 3, 16, 64, 448, 200
    start = np.array([0, 10, 300], np.int32)
    cache = KVCache(slots, heads, cap, d, torch.bfloat16, gpu)
    old_k = okv.round_to(randn(rng, cache.k.shape), "bf16")
    cache.k.copy_(torch.from_numpy(old_k))
    cache.lens.copy_(torch.from_numpy(start))
    nk = randn(rng, (slots, t_new, heads * d))
    nv = randn(rng, (slots, t_new, heads * d))
    cache.append(_dev(nk, torch.float32, gpu), _dev(nv, torch.float32, gpu))
    lens = cache.lens.cpu().numpy()
    np.testing.assert_array_equal(lens, np.minimum(start + t_new, cap))
    k, v = cache.k.float().cpu().numpy(), cache.v.float().cpu().numpy()
    for s in range(slots):
        n = int(lens[s] - start[s])
        want_k = okv.round_to(okv.split_heads(nk[s:s + 1, :n], heads)[0], "bf16")
        want_v = okv.round_to(okv.split_heads(nv[s:s + 1, :n], heads)[0], "bf16")
        np.testing.assert_array_equal(k[s, :, start[s]:lens[s]], want_k)
        np.testing.assert_array_equal(v[s, :, start[s]:lens[s]], want_v)
        np.testing.assert_array_equal(k[s, :, :start[s]], old_k[s, :, :start[s]])  # untouched


def test_gather_follows_parents(gpu):
    rng = np.random.default_rng(11)
    slots, heads, d, cap = 5, 16, 64, 448
    src = KVCache(slots, heads, cap, d, torch.bfloat16, gpu)
    dst = KVCache(slots, heads, cap, d, torch.bfloat16, gpu)
    src.k.copy_(torch.from_numpy(randn(rng, src.k.shape)))
    src.v.copy_(torch.from_numpy(randn(rng, src.v.shape)))
    lens = np.array([5, 448, 64, 65, 1], np.int32)
    src.lens.copy_(torch.from_numpy(lens))
    parent = np.array([1, 1, 4, 0, 2], np.int32)
    dst.gather_from(src, torch.from_numpy(parent).to(gpu))
    np.testing.assert_array_equal(dst.lens.cpu().numpy(), lens[parent])
    for i, p in enumerate(parent.tolist()):
        n = int(lens[p])
        assert torch.equal(dst.k[i, :, :n], src.k[p, :, :n])
        assert torch.equal(dst.v[i, :, :n], src.v[p, :, :n])


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("aligned", [True, False])
def test_layered_gather_follows_parents(gpu, dtype, aligned):
    """One launch reorders a 3-layer stack whose layers hold different lengths. The unaligned
    case views caches whose rows start 2 elements into padded rows (row stride head_dim + 4),
    which takes the element-wise copy."""
    rng = np.random.default_rng(15)
    layers, slots, heads, d, cap = 3, 5, 4, 64, 100
    lens = np.array([[5, 100, 64, 65, 1], [0, 7, 99, 3, 50], [100, 100, 100, 100, 100]], np.int32)
    parent = np.array([3, 3, 0, 4, 1], np.int32)
    tdt = TDT[dtype]

    def make():
        if aligned:
            return KVCache(slots, heads, cap, d, tdt, gpu, layers=layers)
        pad_k = torch.zeros(layers, slots, heads, cap, d + 4, dtype=tdt, device=gpu)
        pad_v = torch.zeros_like(pad_k)
        lens_t = torch.zeros(layers, slots, dtype=torch.int32, device=gpu)
        c = KVCache(slots, heads, cap, d, layers=layers,
                    _views=(pad_k[..., 2:2 + d], pad_v[..., 2:2 + d], lens_t))
        c._pads = (pad_k, pad_v)
        return c

    src, dst = make(), make()
    src.k.copy_(torch.from_numpy(randn(rng, src.k.shape)))
    src.v.copy_(torch.from_numpy(randn(rng, src.v.shape)))
    src.lens.copy_(torch.from_numpy(lens))
    dst.gather_from(src, torch.from_numpy(parent).to(gpu))
    np.testing.assert_array_equal(dst.lens.cpu().numpy(), lens[:, parent])
    for l in range(layers):
        for i, p in enumerate(parent.tolist()):
            n = int(lens[l, p])
            assert torch.equal(dst.k[l, i, :, :n], src.k[l, p, :, :n]), (l, i)
            assert torch.equal(dst.v[l, i, :, :n], src.v[l, p, :, :n]), (l, i)
            # positions past the parent's length are left alone
            assert not dst.k[l, i, :, n:].any()
    if not aligned:  # the padding around each row is untouched
        assert not dst._pads[0][..., :2].any() and not dst._pads[0][..., 2 + d:].any()


@pytest.mark.parametrize("k_transposed", [True, False])
@pytest.mark.parametrize("out", ["bf16", "f16"])
def test_cross_cache_build(gpu, k_transposed, out):
    """whisper-medium window: 1500 frames x 16 heads x 64, f32 projections."""
    rng = np.random.default_rng(12)
    t, heads, d = 1500, 16, 64
    kp, vp = randn(rng, (t, heads * d)), randn(rng, (t, heads * d))
    k, v = cross_kv_build(_dev(kp, torch.float32, gpu), _dev(vp, torch.float32, gpu), heads,
                          TDT[out], k_transposed=k_transposed)
    want_k, want_v = okv.cross_cache_build(kp, vp, heads, out, k_transposed=k_transposed)
    np.testing.assert_array_equal(k.float().cpu().numpy(), want_k)
    np.testing.assert_array_equal(v.float().cpu().numpy(), want_v)


def test_beam_decode_over_device_state(gpu):
    """Three beam steps of one decoder layer: each step appends every beam's new K/V, attends
    (self-attention over the beams' caches, cross-attention over a cache built once), then
    reorders the beams by parent. The reference path keeps raw per-beam caches grown by cat and
    restored from the parent's snapshot, and attends with the oracle. Attention outputs agree to
    the bf16 bar and the caches bit for bit at every step."""
    rng = np.random.default_rng(13)
    beams, heads, d, cap, t_enc, prompt = 5, 16, 64, 64, 300, 3
    scale = d ** -0.5
    # cross-attention cache, built once for the window
    kp, vp = randn(rng, (t_enc, heads * d)), randn(rng, (t_enc, heads * d))
    kx, vx = cross_kv_build(_dev(kp, torch.float32, gpu), _dev(vp, torch.float32, gpu), heads,
                            torch.bfloat16)
    want_kx, want_vx = okv.cross_cache_build(kp, vp, heads, "bf16")
    # prompt: one shared prefix, appended to every beam
    cur, nxt = (KVCache(beams, heads, cap, d, torch.bfloat16, gpu) for _ in range(2))
    pk = okv.round_to(randn(rng, (1, prompt, heads * d)), "bf16")
    pv = okv.round_to(randn(rng, (1, prompt, heads * d)), "bf16")
    cur.append(_dev(np.repeat(pk, beams, 0), torch.bfloat16, gpu),
               _dev(np.repeat(pv, beams, 0), torch.bfloat16, gpu))
    ref = [(pk, pv)] * beams  # the reference's per-beam (raw k, raw v) states
    for step in range(3):
        nk = okv.round_to(randn(rng, (beams, 1, heads * d)), "bf16")
        nv = okv.round_to(randn(rng, (beams, 1, heads * d)), "bf16")
        q_self = okv.round_to(randn(rng, (beams, heads, 1, d)), "bf16")
        q_x = okv.round_to(randn(rng, (beams, heads, 1, d)), "bf16")
        cur.append(_dev(nk, torch.bfloat16, gpu), _dev(nv, torch.bfloat16, gpu))
        o_self = fa.attention(_dev(q_self, torch.bfloat16, gpu), cur.k, cur.v, scale=scale,
                              kv_lens=cur.lens, out_dtype=torch.float32)
        o_x = torch.empty(beams, heads, 1, d, dtype=torch.float32, device=gpu)
        fa.attention(_dev(q_x, torch.bfloat16, gpu).permute(2, 1, 0, 3), kx[None], vx[None],
                     k_transposed=True, scale=scale, out=o_x.permute(2, 1, 0, 3))
        # reference: cat, split, attend per beam
        ref = [(okv.self_cache_append(k, nk[b:b + 1]), okv.self_cache_append(v, nv[b:b + 1]))
               for b, (k, v) in enumerate(ref)]
        want_self = np.concatenate([
            oracle.attend_general(q_self[b:b + 1], okv.split_heads(k, heads), okv.split_heads(v, heads),
                                  k_transposed=False, scale=scale) for b, (k, v) in enumerate(ref)])
        want_x = np.swapaxes(oracle.attend_general(np.swapaxes(q_x, 0, 2), want_kx[None], want_vx[None],
                                                   k_transposed=True, scale=scale), 0, 2)
        e_self = max_abs(o_self.cpu().numpy(), want_self)
        e_x = max_abs(o_x.cpu().numpy(), want_x)
        print(f"step {step}: self {e_self:.3e} cross {e_x:.3e}")
        assert e_self < TOL_BF16 and e_x < TOL_BF16
        # beam selection: new beam i continues parent[i]
        parent = rng.integers(0, beams, size=beams).astype(np.int32)
        nxt.gather_from(cur, torch.from_numpy(parent).to(gpu))
        cur, nxt = nxt, cur
        ref = okv.beam_restore(ref, parent)
        n = prompt + step + 1
        assert (cur.lens.cpu().numpy() == n).all()
        k = cur.k.float().cpu().numpy()
        for b in range(beams):
            np.testing.assert_array_equal(k[b, :, :n], okv.split_heads(ref[b][0], heads)[0])


def test_append_and_attend_replay_in_a_graph(gpu):
    """A decode step (append + self-attention) captured once and replayed: every replay appends
    its row at the next position (the lengths live on the device) and attends over the grown
    cache, matching eager execution of the same steps."""
    rng = np.random.default_rng(14)
    beams, heads, d, cap = 5, 4, 64, 32
    scale = d ** -0.5
    g_cache = KVCache(beams, heads, cap, d, torch.bfloat16, gpu)
    e_cache = KVCache(beams, heads, cap, d, torch.bfloat16, gpu)
    nk = torch.empty(beams, 1, heads * d, dtype=torch.bfloat16, device=gpu)
    nv = torch.empty_like(nk)
    q = torch.empty(beams, heads, 1, d, dtype=torch.bfloat16, device=gpu)
    out = torch.empty(beams, heads, 1, d, dtype=torch.float32, device=gpu)
    ws = torch.zeros(max(1, fa.workspace_bytes(q, g_cache.k, g_cache.v, out, scale=scale,
                                               kv_lens=g_cache.lens)), dtype=torch.uint8, device=gpu)

    def step(cache):
        cache.append(nk, nv)
        fa.attention(q, cache.k, cache.v, scale=scale, kv_lens=cache.lens, out=out, workspace=ws)

    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        step(g_cache)
    g_cache.lens.zero_()  # capture does not execute; start from empty caches
    torch.cuda.synchronize()
    for i in range(6):
        nk.copy_(torch.from_numpy(randn(rng, nk.shape)))
        nv.copy_(torch.from_numpy(randn(rng, nv.shape)))
        q.copy_(torch.from_numpy(randn(rng, q.shape)))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        g_out = out.clone()
        step(e_cache)
        torch.cuda.synchronize()
        assert torch.equal(g_out, out), f"replay {i}"
    assert (g_cache.lens.cpu().numpy() == 6).all()
    assert torch.equal(g_cache.k[:, :, :6], e_cache.k[:, :, :6])
