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


@pytest.mark.parametrize("d,rows,vocab,blk", [(416, 3, 1000, 32), (384, 7, 2000, 64),
                                              (1024, 12, 3000, 128), (1280, 9, 517, 32),
                                              (96, 1, 33, 32), (4096, 3, 700, 32)])
def test_vocab_logits_blocks_and_ragged_steps(gpu, d, rows, vocab, blk):
    """Block sizes 32/64/128 (the products' 32-element halves stored or added per block), d with
    a trailing half step (416 = 6.5 x 64), 9-12 beams (a second product for beams 8-15), a
    vocabulary that ends inside a workgroup, and 128 blocks per row (scales read from global
    memory instead of LDS): logits equal the oracle's bit for bit."""
    rng = np.random.default_rng(73 + d + blk)
    emb = (rng.standard_normal((vocab, d)) / np.sqrt(d)).astype(np.float32)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    iv = Int8Vocab(torch.from_numpy(emb).to(gpu), blk)
    got = iv(torch.from_numpy(x).to(gpu)).cpu().numpy()
    q, sc, corr = og.vocab_quantize(emb, blk)
    want = og.vocab_logits(q, sc, corr, x, blk)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("offset,pitch", [(1, 1025), (4, 1032), (0, 1028)])
def test_vocab_logits_strided_activations(gpu, offset, pitch):
    """Activation rows read through a row stride wider than d, starting off a 16-byte boundary
    (the element-wise quantization loop) or on one (the register path): logits equal the
    oracle's bit for bit."""
    d, rows, vocab = 1024, 5, 3001
    rng = np.random.default_rng(79 + offset + pitch)
    emb = (rng.standard_normal((vocab, d)) / np.sqrt(d)).astype(np.float32)
    full = rng.standard_normal((rows, pitch)).astype(np.float32)
    x = full[:, offset:offset + d]
    iv = Int8Vocab(torch.from_numpy(emb).to(gpu))
    xg = torch.from_numpy(full).to(gpu)[:, offset:offset + d]
    assert xg.stride(0) == pitch
    got = iv(xg).cpu().numpy()
    q, sc, corr = og.vocab_quantize(emb, 32)
    want = og.vocab_logits(q, sc, corr, np.ascontiguousarray(x), 32)
    np.testing.assert_array_equal(got, want)


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


def _check_f16(got, w16, x):
    exact = og.gemv_f16_exact(w16, x)
    bound = 1e-5 * (np.abs(x.astype(np.float64)) @ np.abs(w16.astype(np.float64)).T)
    assert (np.abs(got.astype(np.float64) - exact) <= bound).all()


@pytest.mark.parametrize("rows", list(range(1, 17)))
def test_gemv_f16_every_beam_count(gpu, rows):
    """Every tile height the launch picks (1..16 rows per tile), ragged dimensions: out_dim not a
    multiple of the tile, in_dim not a multiple of a wave's 32-element blocks."""
    rng = np.random.default_rng(80 + rows)
    for out_dim, in_dim in ((1000, 1032), (77, 40), (300, 8)):
        w16 = rng.standard_normal((out_dim, in_dim)).astype(np.float16)
        x = rng.standard_normal((rows, in_dim)).astype(np.float32)
        got = F16Gemv(torch.from_numpy(w16).to(gpu))(torch.from_numpy(x).to(gpu)).cpu().numpy()
        _check_f16(got, w16, x)


def test_gemv_f16_wide_range_and_subnormal_weights(gpu):
    """x is carried as a power-of-two scale and two f16 halves per (beam, range of elements):
    beams whose magnitudes sit near f32's extremes, a range holding 1e-3 beside 1e4, and f16
    subnormal weights keep the f32 summation bound."""
    rng = np.random.default_rng(90)
    out_dim, in_dim, rows = 1024, 4096, 6
    w = rng.standard_normal((out_dim, in_dim)).astype(np.float32)
    w[:, ::7] *= 1e-6  # f16 subnormals (below 6.1e-5)
    w[:8] *= 1e-6      # rows of subnormals only: a flushed product would zero their sums
    w16 = w.astype(np.float16)
    assert (np.abs(w16[:, ::7]) < 6.1e-5).mean() > 0.9 and (np.abs(w16[:8]) < 6.1e-5).all()
    x = rng.standard_normal((rows, in_dim)).astype(np.float32)
    x[1] *= 1e30
    x[2] *= 1e-30
    x[3, ::64] *= 1e4
    x[4] = 0.0
    x[5, 100:200] *= 1e-3
    got = F16Gemv(torch.from_numpy(w16).to(gpu))(torch.from_numpy(x).to(gpu)).cpu().numpy()
    assert np.isfinite(got).all()
    _check_f16(got, w16, x)
    assert (got[4] == 0).all()


def test_gemv_f16_infinite_input(gpu):
    """An infinite activation gives the infinite sums f32 arithmetic gives (its low half is 0),
    and leaves the other beams untouched."""
    rng = np.random.default_rng(91)
    out_dim, in_dim = 512, 1024
    w16 = rng.standard_normal((out_dim, in_dim)).astype(np.float16)
    w16[w16 == 0] = 1
    x = rng.standard_normal((3, in_dim)).astype(np.float32)
    x[1, 37] = np.inf
    got = F16Gemv(torch.from_numpy(w16).to(gpu))(torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = np.where(w16[:, 37].astype(np.float32) > 0, np.inf, -np.inf)
    np.testing.assert_array_equal(got[1], want)
    _check_f16(got[[0, 2]], w16, x[[0, 2]])


def test_gemv_f16_repeatable(gpu):
    """The waves' partial tiles are summed in a fixed order: two calls give the same bits."""
    rng = np.random.default_rng(92)
    w = torch.from_numpy(rng.standard_normal((4096, 1024)).astype(np.float32)).to(gpu)
    g = F16Gemv(w)
    x = torch.from_numpy(rng.standard_normal((5, 1024)).astype(np.float32)).to(gpu)
    a = g(x)
    b = g(x)
    assert torch.equal(a, b)


# (out_dim, in_dim, rows) selecting each compile-time specialized launch shape of gemv.hip
# (tile rows, waves, blocks per wave, x loads), beside shapes that take the generic kernel
SPECIALIZED = [(1024, 1024, 5), (1024, 1024, 6), (1024, 1024, 7), (1024, 1024, 8),
               (4096, 1024, 1), (3072, 1024, 4), (4096, 1024, 5), (3072, 1024, 8),
               (4096, 1024, 9), (4096, 1024, 16), (1024, 4096, 5), (1024, 4096, 6),
               (1024, 4096, 8), (1024, 1024, 1), (1024, 4096, 1), (1280, 1280, 5),
               (1280, 1280, 6), (3840, 1280, 5), (5120, 1280, 5), (5120, 1280, 6),
               (1280, 5120, 5), (1280, 5120, 4), (1280, 5120, 6), (1280, 6144, 5),
               (1024, 20000, 9)]


@pytest.mark.parametrize("out_dim,in_dim,rows", SPECIALIZED)
def test_gemv_f16_launch_shapes(gpu, out_dim, in_dim, rows):
    rng = np.random.default_rng(out_dim + 3 * in_dim + rows)
    w16 = rng.standard_normal((out_dim, in_dim)).astype(np.float16)
    x = rng.standard_normal((rows, in_dim)).astype(np.float32)
    got = F16Gemv(torch.from_numpy(w16).to(gpu))(torch.from_numpy(x).to(gpu)).cpu().numpy()
    _check_f16(got, w16, x)
