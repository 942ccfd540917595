"""GPU parity of the fused decode-step projection (ffai_gemv_f16_qkv_cache, ffai_gemv.h) and the
all-layer length advance (ffai_kv_advance, ffai_kv.h).

The fused call must equal the unfused sequence it replaces -- the f16 GEMV of the packed q/k/v
weights, the bias added in f32, then ffai_kv_append of the k and v rows -- bit for bit: q, every
cache element and every length. That sequence is itself pinned against the oracle (the GEMV
against the exact float64 dot in test_gpu_gemv.py, the append against the reference's
Tensor::cat in test_gpu_kv.py); here the fused q is also checked against the exact dot plus the
bias, and its cache rows against that value rounded to the cache type."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gemv as og
from oracle import kvcache as okv
from ffai_amd.gemv import F16Gemv
from ffai_amd.kv_cache import KVCache

pytestmark = pytest.mark.gpu

TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _filled_cache(rng, slots, heads, cap, d, dtype, lens, device, layers=None):
    c = KVCache(slots, heads, cap, d, TDT[dtype], device, layers=layers)
    c.k.copy_(torch.from_numpy(rng.standard_normal(tuple(c.k.shape), dtype=np.float32)))
    c.v.copy_(torch.from_numpy(rng.standard_normal(tuple(c.v.shape), dtype=np.float32)))
    c.lens.copy_(torch.from_numpy(np.asarray(lens, np.int32)))
    return c


def _clone(c):
    return KVCache(c.slots, c.heads, c.capacity, c.head_dim, layers=c.layers,
                   _views=(c.k.clone(), c.v.clone(), c.lens.clone()))


def _weights(rng, n, in_dim, device):
    w = torch.from_numpy((rng.standard_normal((3 * n, in_dim)) / np.sqrt(in_dim)).astype(np.float32))
    return F16Gemv(w.to(device))


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("rows,with_bias", [(5, True), (5, False), (1, True)])
@pytest.mark.parametrize("heads,in_dim", [(16, 1024), (20, 1280)])
def test_fused_step_equals_gemv_bias_append(gpu, dtype, rows, with_bias, heads, in_dim):
    """whisper-medium (16 heads x 64, in 1024) and whisper-large (20 x 64, in 1280) widths,
    ragged lengths: q, the K/V caches and the lengths after advance + fused call equal GEMV +
    bias + append bit for bit."""
    rng = np.random.default_rng(90 + rows + heads)
    d, cap = 64, 80
    n = heads * d
    lens = [0, 3, 40, 78, 79][:rows]
    gm = _weights(rng, n, in_dim, gpu)
    x = torch.from_numpy(rng.standard_normal((rows, in_dim), dtype=np.float32)).to(gpu)
    bias = None
    if with_bias:
        b = rng.standard_normal(3 * n).astype(np.float32)
        b[n:2 * n] = 0.0  # k_proj has no bias (text_decoder.rs:609-613)
        bias = torch.from_numpy(b).to(gpu)
    a = _filled_cache(rng, rows, heads, cap, d, dtype, lens, gpu)
    bc = _clone(a)
    # unfused: GEMV, bias, append
    y = gm(x)
    if bias is not None:
        y = y + bias
    a.append(y[:, None, n:2 * n].contiguous(), y[:, None, 2 * n:].contiguous())
    # fused: advance, then the projection writes the rows
    q = torch.empty(rows, n, device=gpu)
    bc.advance(1)
    gm.qkv_into_cache(x, q, bc, bias)
    torch.cuda.synchronize()
    assert torch.equal(q, y[:, :n])
    assert torch.equal(bc.lens, a.lens)
    assert torch.equal(bc.k, a.k) and torch.equal(bc.v, a.v)
    # and against the exact dot products of the same f16 weights
    want = og.gemv_f16_exact(gm.w.cpu().numpy(), x.cpu().numpy())
    if bias is not None:
        want = want + bias.cpu().numpy()
    assert np.max(np.abs(q.cpu().numpy() - want[:, :n])) < 1e-4
    kk, vv = bc.k.float().cpu().numpy(), bc.v.float().cpu().numpy()
    for r in range(rows):
        pos = lens[r]
        for part, arr in ((1, kk), (2, vv)):
            row = want[r, part * n:(part + 1) * n].reshape(heads, d).astype(np.float32)
            tol = 1e-4 if dtype == "f32" else 2.0 ** (-7 if dtype == "bf16" else -10) * 4
            np.testing.assert_allclose(arr[r, :, pos], okv.round_to(row, dtype), rtol=tol,
                                       atol=1e-4)


def test_fewer_rows_than_slots(gpu):
    """Three beams into a five-slot cache: slots 0-2 get their rows, slots 3-4 are untouched."""
    rng = np.random.default_rng(93)
    heads, d, cap, in_dim = 8, 64, 32, 512
    n = heads * d
    gm = _weights(rng, n, in_dim, gpu)
    x = torch.from_numpy(rng.standard_normal((3, in_dim), dtype=np.float32)).to(gpu)
    c = _filled_cache(rng, 5, heads, cap, d, "bf16", [4, 5, 6, 7, 8], gpu)
    before = _clone(c)
    three = KVCache(3, heads, cap, d, _views=(c.k[:3], c.v[:3], c.lens[:3]))
    three.advance(1)
    q = torch.empty(3, n, device=gpu)
    gm.qkv_into_cache(x, q, three)
    ref = KVCache(3, heads, cap, d, _views=(before.k[:3].clone(), before.v[:3].clone(),
                                            before.lens[:3].clone()))
    y = gm(x)
    ref.append(y[:, None, n:2 * n].contiguous(), y[:, None, 2 * n:].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(c.k[:3], ref.k) and torch.equal(c.v[:3], ref.v)
    assert torch.equal(c.lens[:3], ref.lens)
    assert torch.equal(c.k[3:], before.k[3:]) and torch.equal(c.v[3:], before.v[3:])
    assert torch.equal(c.lens[3:], before.lens[3:])


def test_full_and_empty_slots(gpu):
    """A slot already at capacity before the advance keeps its length and has its last row
    replaced (the append would drop the row); a slot of length 0 that was not advanced gets no
    row; lengths out of range are clamped."""
    rng = np.random.default_rng(94)
    heads, d, cap, in_dim = 4, 64, 16, 256
    n = heads * d
    gm = _weights(rng, n, in_dim, gpu)
    x = torch.from_numpy(rng.standard_normal((4, in_dim), dtype=np.float32)).to(gpu)
    c = _filled_cache(rng, 4, heads, cap, d, "f32", [cap, 0, -3, cap + 9], gpu)
    before = _clone(c)
    q = torch.empty(4, n, device=gpu)
    gm.qkv_into_cache(x, q, c)        # no advance: positions lens - 1 (clamped)
    torch.cuda.synchronize()
    y = gm(x).cpu().numpy()
    k, v = c.k.cpu().numpy(), c.v.cpu().numpy()
    k0, v0 = before.k.cpu().numpy(), before.v.cpu().numpy()
    for r, pos in ((0, cap - 1), (3, cap - 1)):
        np.testing.assert_array_equal(k[r, :, pos], y[r, n:2 * n].reshape(heads, d))
        np.testing.assert_array_equal(v[r, :, pos], y[r, 2 * n:].reshape(heads, d))
        np.testing.assert_array_equal(np.delete(k[r], pos, axis=1), np.delete(k0[r], pos, axis=1))
    for r in (1, 2):                  # length 0 and -3: nothing written
        np.testing.assert_array_equal(k[r], k0[r])
        np.testing.assert_array_equal(v[r], v0[r])
    np.testing.assert_array_equal(c.lens.cpu().numpy(), [cap, 0, -3, cap + 9])


@pytest.mark.parametrize("t_new", [1, 3])
def test_advance_every_layer(gpu, t_new):
    """A 24-layer stack of 5 slots: every layer's lengths move by t_new, clamped into
    [0, capacity] first and saturating at capacity, as ffai_kv_append advances them; the K/V
    contents are untouched."""
    rng = np.random.default_rng(95)
    layers, slots, heads, d, cap = 24, 5, 2, 64, 40
    lens = rng.integers(-3, cap + 4, size=(layers, slots)).astype(np.int32)
    lens[0] = [0, 1, cap - 1, cap, cap + 2]
    c = _filled_cache(rng, slots, heads, cap, d, "bf16", lens, gpu, layers=layers)
    k0 = c.k.clone()
    c.advance(t_new)
    torch.cuda.synchronize()
    want = np.minimum(cap, np.clip(lens, 0, cap) + t_new)
    np.testing.assert_array_equal(c.lens.cpu().numpy(), want)
    assert torch.equal(c.k, k0)


def test_decode_steps_fused_equal_unfused(gpu):
    """Three beam-5 decode steps over a 4-layer stack: per step one advance and per layer the
    fused projection, against per layer GEMV + bias + append. The caches and lengths agree bit
    for bit after every step, including the beam reorder between steps."""
    rng = np.random.default_rng(96)
    layers, beams, heads, d, cap, in_dim = 4, 5, 16, 64, 64, 1024
    n = heads * d
    gms = [_weights(rng, n, in_dim, gpu) for _ in range(layers)]
    biases = []
    for _ in range(layers):
        b = rng.standard_normal(3 * n).astype(np.float32)
        b[n:2 * n] = 0.0
        biases.append(torch.from_numpy(b).to(gpu))
    start = np.full((layers, beams), 20, np.int32)
    fused = [_filled_cache(rng, beams, heads, cap, d, "bf16", start, gpu, layers=layers)]
    fused.append(_clone(fused[0]))
    plain = [_clone(fused[0]), _clone(fused[0])]
    q = torch.empty(beams, n, device=gpu)
    for step in range(3):
        x = [torch.from_numpy(rng.standard_normal((beams, in_dim), dtype=np.float32)).to(gpu)
             for _ in range(layers)]
        parent = torch.from_numpy(rng.integers(0, beams, beams).astype(np.int32)).to(gpu)
        cur_f, nxt_f = fused[step % 2], fused[1 - step % 2]
        cur_p, nxt_p = plain[step % 2], plain[1 - step % 2]
        cur_f.advance(1)
        for l in range(layers):
            gms[l].qkv_into_cache(x[l], q, cur_f.layer(l), biases[l])
            y = gms[l](x[l]) + biases[l]
            cur_p.layer(l).append(y[:, None, n:2 * n].contiguous(), y[:, None, 2 * n:].contiguous())
            assert torch.equal(q, y[:, :n])
        nxt_f.gather_from(cur_f, parent)
        nxt_p.gather_from(cur_p, parent)
        torch.cuda.synchronize()
        assert torch.equal(nxt_f.lens, nxt_p.lens)
        assert torch.equal(nxt_f.k, nxt_p.k) and torch.equal(nxt_f.v, nxt_p.v)
