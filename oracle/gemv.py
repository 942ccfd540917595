"""CPU restatement of the reference's decoder GEMVs. TEST INFRASTRUCTURE ONLY: used by tests/
and never by the ffai_amd product path.

Follows crates/ffai-mercury/src/asr/vocab_int8.rs and f16_gemv.rs:
  * rust_round      -- f32::round: half away from zero (used by both quantizers)
  * vocab_quantize  -- Int8Vocab::new (:100-170): per 32-weight block scale = amax / 127,
                       q = round(w / scale) clamped to [-127, 127], corr = 64 * sum over blocks,
                       in order, of scale * blocksum
  * act_quantize    -- Int8VocabOp::cpu_fwd (:233-240): sx = amax / 63, x_u = round(x / sx)
                       clamped to [-64, 63] plus 64
  * vocab_logits    -- Int8VocabOp::cpu_fwd + dot_i8_blocked (:241-262, :282-306): exact integer
                       block dots, acc += (float)blocksum * scale in block order, then
                       (acc - corr) * sx
  * gemv_f16_exact  -- F16Gemv::forward (:117-196): f16 weights widened to f32 times f32
                       activations; computed here exactly (float64), since the reference's
                       own order is a 16-lane AVX tree
The int8 functions use numpy float32 operations, which are IEEE-rounded one at a time (never
fused), so they reproduce the reference's f32 arithmetic bit for bit.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def rust_round(v: np.ndarray) -> np.ndarray:
    """Round half away from zero, exactly: trunc, then step away when the (exact) fractional
    part is >= 0.5."""
    v = np.asarray(v, dtype=F32)
    t = np.trunc(v)
    frac = np.abs(v - t)  # exact for |v| < 2^23
    return (t + np.where(frac >= F32(0.5), np.sign(v), F32(0))).astype(F32)


def vocab_quantize(emb: np.ndarray, blk: int = 32):
    """emb (vocab, d) float32 -> (q int8 (vocab, d), bscale f32 (vocab, nb), corr f32 (vocab,))."""
    emb = np.asarray(emb, dtype=F32)
    vocab, d = emb.shape
    nb = d // blk
    blocks = emb.reshape(vocab, nb, blk)
    amax = np.abs(blocks).max(axis=2)
    sc = np.where(amax > 0, amax / F32(127), F32(1)).astype(F32)
    q = np.clip(rust_round(blocks / sc[:, :, None]), -127, 127).astype(np.int8)
    bsum = q.astype(np.int32).sum(axis=2)
    c = np.zeros(vocab, F32)
    for b in range(nb):
        c = (c + (sc[:, b] * bsum[:, b].astype(F32)).astype(F32)).astype(F32)
    return q.reshape(vocab, d), sc, (F32(64) * c).astype(F32)


def act_quantize(x: np.ndarray):
    """x (rows, d) float32 -> (x_u uint8 (rows, d) in 0..127, sx f32 (rows,))."""
    x = np.asarray(x, dtype=F32)
    amax = np.abs(x).max(axis=1)
    sx = np.where(amax > 0, amax / F32(63), F32(1)).astype(F32)
    xq = np.clip(rust_round(x / sx[:, None]), -64, 63).astype(np.int32)
    return (xq + 64).astype(np.uint8), sx


def vocab_logits(q: np.ndarray, bscale: np.ndarray, corr: np.ndarray, x: np.ndarray, blk: int = 32):
    """(rows, d) activations -> (rows, vocab) float32 logits."""
    xu, sx = act_quantize(x)
    vocab, d = q.shape
    nb = d // blk
    qb = q.reshape(vocab, nb, blk).astype(np.int32)
    out = np.empty((x.shape[0], vocab), F32)
    for r in range(x.shape[0]):
        xb = xu[r].reshape(nb, blk).astype(np.int32)
        s = np.einsum("vbk,bk->vb", qb, xb)  # exact integers
        acc = np.zeros(vocab, F32)
        for b in range(nb):
            acc = (acc + (s[:, b].astype(F32) * bscale[:, b]).astype(F32)).astype(F32)
        out[r] = ((acc - corr).astype(F32) * sx[r]).astype(F32)
    return out


def gemv_f16_exact(w_f16: np.ndarray, x: np.ndarray) -> np.ndarray:
    """w (out, in) float16, x (rows, in) float32 -> (rows, out) float64, exact products."""
    return np.asarray(x, np.float64) @ np.asarray(w_f16, np.float64).T
