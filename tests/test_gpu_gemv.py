"""GPU parity of the decoder GEMVs (include/ffai_gemv.h) against the oracle (oracle/gemv.py).

The int8 vocabulary projection reproduces the reference's arithmetic exactly, so quantized
weights, scales, corrections and logits are compared bit for bit (and the selected token is
therefore identical). The f16 GEMV is floating point summed in another order than the
reference's AVX lanes: it is compared with the exact (float64) dot of the same f16 weights,
to f32 summation error, and with the reference test's own bound against f32 weights."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gemv as og
from ffai_amd.gemv import F16Gemv, Int8Vocab

pytestmark = pytest.mark.gpu

WHISPER_VOCAB = 51865


@pytest.mark.parametrize("vocab,d,blk,src", [(4103, 384, 32, "f32"), (1027, 1024, 64, "f32"),
                                             (2053, 1024, 32, "bf16")])
def test_vocab_quantize_bit_exact(gpu, vocab, d, blk, src):
    rng = np.random.default_rng(70)
    emb = rng.standard_normal((vocab, d)).astype(np.float32)
    emb[5, :blk] = 0.0
    t = torch.from_numpy(emb).to(gpu)
    if src == "bf16":
        t = t.to(torch.bfloat16)
        emb = t.float().cpu().numpy()
    iv = Int8Vocab(t, blk)
    q, sc, corr = og.vocab_quantize(emb, blk)
    np.testing.assert_array_equal(iv.qw.cpu().numpy(), q)
    np.testing.assert_array_equal(iv.bscale.cpu().numpy(), sc)
    np.testing.assert_array_equal(iv.corr.cpu().numpy(), corr)


@pytest.mark.parametrize("d,rows,vocab", [(384, 1, WHISPER_VOCAB), (1024, 5, WHISPER_VOCAB),
                                          (1280, 16, 4099)])
def test_vocab_logits_bit_exact(gpu, d, rows, vocab):
    """whisper-tiny (d 384) greedy, whisper-medium (d 1024) beam 5, whisper-large width with 16
    rows: logits equal the oracle's bit for bit, so the argmax tokens are identical."""
    rng = np.random.default_rng(71 + d)
    emb = (rng.standard_normal((vocab, d)) / np.sqrt(d)).astype(np.float32)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    x[0, :7] *= 40.0  # a few large activations set the activation scale
    iv = Int8Vocab(torch.from_numpy(emb).to(gpu))
    got = iv(torch.from_numpy(x).to(gpu)).cpu().numpy()
    q, sc, corr = og.vocab_quantize(emb, 32)
    want = og.vocab_logits(q, sc, corr, x, 32)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(got.argmax(axis=1), want.argmax(axis=1))


@pytest.mark.parametrize("out_dim,in_dim,rows", [(1536, 384, 1), (1024, 1024, 5),
                                                 (4096, 1024, 5), (1024, 4096, 9), (1023, 1280, 16),
                                                 (3840, 1280, 5)])
def test_gemv_f16(gpu, out_dim, in_dim, rows):
    rng = np.random.default_rng(72)
    w = rng.standard_normal((out_dim, in_dim)).astype(np.float32)
    x = rng.standard_normal((rows, in_dim)).astype(np.float32)
    g = F16Gemv(torch.from_numpy(w).to(gpu))
    got = g(torch.from_numpy(x).to(gpu)).cpu().numpy().astype(np.float64)
    w16 = w.astype(np.float16)
    exact = og.gemv_f16_exact(w16, x)
    bound = 1e-5 * (np.abs(x.astype(np.float64)) @ np.abs(w16.astype(np.float64)).T) + 1e-6
    assert (np.abs(got - exact) <= bound).all()
    f32w = x.astype(np.float64) @ w.astype(np.float64).T  # f16_gemv.rs:203-229's bound
    assert np.abs(got - f32w).max() / np.abs(f32w).max() < 5e-3
