"""GPU parity of fwd16_kernel (attn_kernels16.cuh): the encoder launch shape (16-bit, head_dim 64,
four waves x 64 query rows) rebuilt on 16x16x32 MFMA with one software-pipelined phase per 16-key
unit. The planner never chooses it (it measured 2-4% slower than fwd_kernel's 32x32x16 schedule);
it stays a measured alternative behind ffai_set_attn_variant(3), and these tests force it over the
cases that exercise its paths: DMA and register staging (ragged tails, misaligned operands), K
given transposed and as rows, causal masks, the slow (non-FAST) reference max and its settle
redo, key-split pieces merged in the launch, f32 and 16-bit outputs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from ffai_amd import _lib as L
from ffai_amd import flash_attn as fa
from tests.helpers import TOL_BF16, max_abs, randn, round_bf16, round_f16

pytestmark = pytest.mark.gpu


@pytest.fixture
def x16(gpu):
    lib = L.load()
    prev = lib.ffai_get_attn_variant()
    lib.ffai_set_attn_variant(3)
    yield gpu
    lib.ffai_set_attn_variant(prev)


def _dev(x, dtype, device):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def _case(x16, b, h, t, tk, dtype, k_transposed, out_dtype, *, causal=False, q_offset=0,
          k_mult=1.0, q_mult=1.0, offset=0, lens=None, seed=0):
    rng = np.random.default_rng(seed)
    rnd = round_bf16 if dtype == torch.bfloat16 else round_f16
    q = rnd(randn(rng, (b, h, t, 64)) * np.float32(q_mult))
    k = rnd(randn(rng, (b, h, tk, 64)) * np.float32(k_mult))
    v = rnd(randn(rng, (b, h, tk, 64)))
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125, causal=causal,
                                 q_offset=q_offset, kv_lens=lens)
    kk = np.swapaxes(k, 2, 3) if k_transposed else k

    def put(x):  # a device copy whose data starts `offset` elements into its allocation
        flat = torch.zeros(x.size + offset, dtype=dtype, device=x16)
        flat[offset:] = _dev(x, dtype, x16).reshape(-1)
        return flat[offset:].view(x.shape)

    qd, kd, vd = put(q), put(kk), put(v)
    out = torch.empty(b, h, t, 64, dtype=out_dtype, device=x16)
    kl = None if lens is None else _dev(lens, torch.int32, x16)
    plan = fa.plan(qd, kd, vd, out, k_transposed=k_transposed, scale=0.125, causal=causal,
                   q_offset=q_offset, kv_lens=kl)
    assert plan["kernel"] == "fwd" and plan["shape"] == "wave4x2x16", plan
    fa.attention(qd, kd, vd, k_transposed=k_transposed, scale=0.125, causal=causal,
                 q_offset=q_offset, kv_lens=kl, out=out)
    err = max_abs(out.float().cpu().numpy(), want)
    return err, plan


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k_transposed", [True, False])
def test_encoder_whisper_small_tail_pieces(x16, dtype, k_transposed):
    """B8 H12 T1500 (K x 2): 576 items, the last 64 in 4 key pieces merged in the launch; the
    last tile of every item holds 28 keys (register staging)."""
    err, plan = _case(x16, 8, 12, 1500, 1500, dtype, k_transposed, torch.float32, k_mult=2.0,
                      seed=1)
    assert plan["splits"] == 4
    print(f"x16 whisper-small {dtype} kt={k_transposed}: {err:.3e}")
    assert err < TOL_BF16


def test_large_v3_window_bf16_out(x16):
    err, _ = _case(x16, 1, 20, 1500, 1500, torch.bfloat16, True, torch.bfloat16, seed=2)
    assert err < TOL_BF16


@pytest.mark.parametrize("q_offset", [0, 100])
def test_causal_and_ragged(x16, q_offset):
    """Causal rows at an offset over 700 keys, ragged per-item lengths (one item shorter than a
    tile), K as rows."""
    lens = np.array([700, 37, 420], np.int32)
    err, _ = _case(x16, 3, 4, 600, 700, torch.bfloat16, False, torch.float32, causal=True,
                   q_offset=q_offset, lens=lens, seed=3)
    assert err < TOL_BF16


@pytest.mark.parametrize("k_transposed", [True, False])
def test_score_jumps_slow_reference_and_redo(x16, k_transposed):
    """Scores along one head dimension (so that the scale folded into a 16-bit Q stays exact
    enough): the first unit's rows sit near 87 log2 units, outside the FAST window, so its max is
    the reference; keys 200-259 jump ~58 log2 units above it (weights near 2^58, accepted) and
    keys 640-699 ~173 above (past f32's range: their chunk is redone against its exact max and
    the accumulator rescaled)."""
    rng = np.random.default_rng(78)
    b, h, t, d = 1, 2, 1000, 64
    u = np.zeros(d, np.float32)
    u[3] = 1.0
    q = round_bf16(8.0 * u + 0.05 * randn(rng, (b, h, t, d)))
    amp = np.full(t, 60.0, np.float32)
    amp[200:260] = 100.0
    amp[640:700] = 180.0
    k = round_bf16(amp[None, None, :, None] * u + 0.05 * randn(rng, (b, h, t, d)))
    v = round_bf16(randn(rng, (b, h, t, d)))
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125)
    kk = np.swapaxes(k, 2, 3) if k_transposed else k
    qd, kd, vd = (_dev(x, torch.bfloat16, x16) for x in (q, kk, v))
    out = torch.empty(b, h, t, d, device=x16)
    assert fa.plan(qd, kd, vd, out, k_transposed=k_transposed, scale=0.125)["shape"] == "wave4x2x16"
    fa.attention(qd, kd, vd, k_transposed=k_transposed, scale=0.125, out=out)
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    err = max_abs(got, want)
    print(f"x16 score jumps kt={k_transposed}: {err:.3e}")
    assert err < TOL_BF16


def test_misaligned_operands_take_register_staging(x16):
    """Operands starting 1 element past 16-byte alignment: no DMA, element loads."""
    err, _ = _case(x16, 1, 4, 300, 300, torch.bfloat16, True, torch.float32, offset=1, seed=5)
    assert err < TOL_BF16
