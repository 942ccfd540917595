"""GPU parity of the encoder self-attention block (include/ffai_encoder.h: hipBLASLt projections
around the fused kernel) against the oracle's restatement of EncoderAttention::forward
(oracle/encoder.py). The oracle runs in float64 and rounds the intermediates the device stores
in 16 bits (q, k^T, v, the merged attention output) the same way, so the comparison measures
arithmetic; the bar is the 16-bit one, 2e-2 max-abs, on outputs of order 1."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import encoder as oenc
from oracle import kvcache as okv
from ffai_amd.encoder import EncoderAttention
from tests.helpers import TOL_BF16, max_abs

pytestmark = pytest.mark.gpu

TDT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _case(rng, b, t, n, dt):
    r = lambda a: okv.round_to(a.astype(np.float32), dt)
    x = r(rng.standard_normal((b, t, n)))
    ws = [r(rng.standard_normal((n, n)) / np.sqrt(n)), r(0.1 * rng.standard_normal(n)),
          r(rng.standard_normal((n, n)) / np.sqrt(n)),
          r(rng.standard_normal((n, n)) / np.sqrt(n)), r(0.1 * rng.standard_normal(n)),
          r(rng.standard_normal((n, n)) / np.sqrt(n)), r(0.1 * rng.standard_normal(n))]
    return x, ws


def _run(gpu, x, ws, n_head, dt, packed=True):
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu, TDT[dt])
    wq, bq, wk, wv, bv, wo, bo = ws
    ea = EncoderAttention.load(x.shape[2], n_head, dev(wq), dev(bq), dev(wk), dev(wv), dev(bv),
                               dev(wo), dev(bo), packed=packed)
    got = ea(dev(x)).float().cpu().numpy()
    wk_s = ea.w[2].float().cpu().numpy()  # the device's pre-scaled key weight, as stored
    want = oenc.encoder_attention(x, wq, bq, wk_s, wv, bv, wo, bo, n_head, store=dt)
    return got, want


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("packed", [True, False])
def test_encoder_block_whisper_tiny(gpu, dt, packed):
    """whisper-tiny encoder layer: 6 heads x 64, n_state 384; two windows of 300 frames. Packed:
    one GEMM for q, k and v, K read as rows; unpacked: three GEMMs, K^T as the reference."""
    rng = np.random.default_rng(60)
    x, ws = _case(rng, 2, 300, 384, dt)
    got, want = _run(gpu, x, ws, 6, dt, packed)
    err = max_abs(got, want)
    print(f"encoder block tiny {dt} packed={packed}: {err:.3e} (max |out| {np.abs(want).max():.2f})")
    assert err < TOL_BF16


@pytest.mark.parametrize("packed", [True, False])
def test_encoder_block_large_v3_window(gpu, packed):
    """whisper-large-v3 encoder layer: 20 heads x 64, n_state 1280, one 1500-frame window."""
    rng = np.random.default_rng(61)
    x, ws = _case(rng, 1, 1500, 1280, "bf16")
    got, want = _run(gpu, x, ws, 20, "bf16", packed)
    err = max_abs(got, want)
    print(f"encoder block large-v3 packed={packed}: {err:.3e} (max |out| {np.abs(want).max():.2f})")
    assert err < TOL_BF16


def test_encoder_block_batch_equals_items(gpu):
    """One batched call equals the reference's per-window loop (text_decoder.rs:1069-1076),
    bit for bit: the GEMMs and the attention treat windows independently."""
    rng = np.random.default_rng(62)
    x, ws = _case(rng, 3, 200, 384, "bf16")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu, torch.bfloat16)
    ea = EncoderAttention.load(384, 6, *[dev(w) for w in ws])
    allx = ea(dev(x))
    for i in range(3):
        one = ea(dev(x[i:i + 1]))
        err = (allx[i:i + 1].float() - one.float()).abs().max().item()
        assert err <= 2e-2, (i, err)


def test_encoder_block_windows_run_in_passes(gpu):
    """Eleven 300-frame windows (whisper-tiny width) run as passes of five, five and one window
    (at most 1500 rows per pass) through one workspace sized for a pass; every window matches
    the oracle."""
    rng = np.random.default_rng(63)
    x, ws = _case(rng, 11, 300, 384, "bf16")
    for packed in (True, False):
        got, want = _run(gpu, x, ws, 6, "bf16", packed)
        err = max_abs(got, want)
        print(f"encoder block 11 x 300 packed={packed}: {err:.3e}")
        assert err < TOL_BF16


def test_encoder_block_full_windows_equal_single_calls(gpu):
    """Three 1500-frame windows at whisper-large-v3 width run as three one-window passes: each
    window's output equals a one-window call bit for bit (the same GEMM and attention shapes on
    the same data), and the workspace is one window's."""
    rng = np.random.default_rng(64)
    x, ws = _case(rng, 3, 1500, 1280, "bf16")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu, torch.bfloat16)
    ea = EncoderAttention.load(1280, 20, *[dev(w) for w in ws])
    assert ea.workspace_bytes(dev(x)) == ea.workspace_bytes(dev(x[:1]))
    allx = ea(dev(x))
    for i in range(3):
        one = ea(dev(x[i:i + 1]))
        assert torch.equal(allx[i:i + 1], one), i


@pytest.mark.parametrize("packed", [True, False])
def test_encoder_block_short_last_pass_at_large_v3_width(gpu, packed):
    """Six 300-frame windows at whisper-large-v3 width (20 heads x 64) run as a five-window pass
    and a one-window pass. The shorter pass's smaller grid splits its keys (about 6 MB of
    partials, where the full pass needs none): the call's workspace holds it, and every window
    matches the oracle."""
    rng = np.random.default_rng(65)
    x, ws = _case(rng, 6, 300, 1280, "bf16")
    got, want = _run(gpu, x, ws, 20, "bf16", packed)
    err = max_abs(got, want)
    print(f"encoder block 6 x 300 large-v3 width packed={packed}: {err:.3e}")
    assert err < TOL_BF16
