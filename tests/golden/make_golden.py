#!/usr/bin/env python3
"""Write the committed golden vectors for the attention path (tests/golden/*.npz).

The reference holds no attention fixtures (its kernel tests draw unseeded candle randn and
compare against the closed form at 1e-4: crates/ffai-mercury/src/asr/flash_attn.rs:1005-1039),
so these vectors are made here: seeded inputs, the oracle's output (the reference algorithm
restated, oracle/flash_oracle.cpp) and the float64 closed form (oracle/textbook.py) for the same
inputs. Every case also records which reference function it exercises.

Run from the repo root:  python tests/golden/make_golden.py [case names to write; default all]
"""

from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from oracle import textbook  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 values already on the bf16 grid -> their 16-bit patterns (lossless)."""
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def main() -> None:
    cases = {}

    # 1. encoder f32, ragged tails (T = 300 = 256 + 44 keys, 4*64 + 44 query rows), merged layout
    rng = np.random.default_rng(1)
    h, t = 2, 300
    q = (rng.standard_normal((1, h, t, 64)) * 0.125).astype(np.float32)
    kt = rng.standard_normal((1, h, 64, t)).astype(np.float32)
    v = rng.standard_normal((1, h, t, 64)).astype(np.float32)
    cases["encoder_f32_h2_t300"] = dict(
        ref="MergedAttnOp / flash_head_strided (flash_attn.rs:160-210, 415-487)",
        q=q, kt=kt, v=v, out=oracle.attend_f32(q, kt, v),
        f64=textbook.attention(q, kt, v, k_transposed=True))

    # 2. decode f32, 37 keys (not a multiple of 8: exercises the scalar tails)
    rng = np.random.default_rng(2)
    q = (rng.standard_normal((1, 6, 1, 64)) * 0.125).astype(np.float32)
    kt = rng.standard_normal((1, 6, 64, 37)).astype(np.float32)
    v = rng.standard_normal((1, 6, 37, 64)).astype(np.float32)
    cases["decode_f32_h6_k37"] = dict(
        ref="FlashAttnOp f32 decode arm, xattn_head (flash_attn.rs:370-399, 602-696)",
        q=q, kt=kt, v=v, out=oracle.attend_f32(q, kt, v),
        f64=textbook.attention(q, kt, v, k_transposed=True))

    # 3. decode with f16 K/V, 300 keys
    rng = np.random.default_rng(3)
    q = (rng.standard_normal((1, 2, 1, 64)) * 0.125).astype(np.float32)
    kt16 = rng.standard_normal((1, 2, 64, 300)).astype(np.float16)
    v16 = rng.standard_normal((1, 2, 300, 64)).astype(np.float16)
    cases["decode_f16kv_h2_k300"] = dict(
        ref="FlashAttnOp f16-K/V decode arm, xattn_head_f16 (flash_attn.rs:289-356, 714-789)",
        q=q, kt16=kt16, v16=v16, out=oracle.attend_f16kv(q, kt16, v16),
        f64=textbook.attention(q, kt16.astype(np.float32), v16.astype(np.float32),
                               k_transposed=True))

    # 4. causal GQA prefill, head_dim 128, bf16-rounded inputs (extension, not reference)
    rng = np.random.default_rng(5)
    hq, hkv, s, d = 4, 2, 130, 128
    q = oracle.round_bf16(rng.standard_normal((1, hq, s, d)).astype(np.float32))
    k = oracle.round_bf16(rng.standard_normal((1, hkv, s, d)).astype(np.float32))
    v = oracle.round_bf16(rng.standard_normal((1, hkv, s, d)).astype(np.float32))
    sc = d ** -0.5
    cases["causal_gqa_bf16_d128_s130"] = dict(
        ref="extension (no reference kernel; mask semantics of text_decoder.rs:902-923)",
        q_bf16=bf16_bits(q), k_bf16=bf16_bits(k), v_bf16=bf16_bits(v), scale=np.float32(sc),
        out=oracle.attend_general(q, k, v, k_transposed=False, scale=sc, causal=True),
        f64=textbook.attention(q, k, v, scale=sc, causal=True))

    # 5. beam self-attention with ragged per-beam key counts (extension)
    rng = np.random.default_rng(6)
    beams, hh, cap = 3, 2, 70
    lens = np.array([1, 33, 70], np.int32)
    q = oracle.round_bf16(rng.standard_normal((beams, hh, 1, 64)).astype(np.float32))
    k = oracle.round_bf16(rng.standard_normal((beams, hh, cap, 64)).astype(np.float32))
    v = oracle.round_bf16(rng.standard_normal((beams, hh, cap, 64)).astype(np.float32))
    cases["ragged_beams_bf16"] = dict(
        ref="extension (per-beam caches, decoder.rs:542-596 / text_decoder.rs:652-679)",
        q_bf16=bf16_bits(q), k_bf16=bf16_bits(k), v_bf16=bf16_bits(v), lens=lens,
        scale=np.float32(0.125),
        out=oracle.attend_general(q, k, v, k_transposed=False, scale=0.125, kv_lens=lens),
        f64=textbook.attention(q, k, v, scale=0.125, kv_lens=lens))

    # 6. encoder f32 at the reference unit test's shape (flash_attn.rs:1005-1021: H = 4,
    #    T = 512, scale on q), merged layout
    rng = np.random.default_rng(7)
    h, t = 4, 512
    q = (rng.standard_normal((1, h, t, 64)) * 0.125).astype(np.float32)
    kt = rng.standard_normal((1, h, 64, t)).astype(np.float32)
    v = rng.standard_normal((1, h, t, 64)).astype(np.float32)
    cases["encoder_f32_h4_t512"] = dict(
        ref="MergedAttnOp at the shape of flash_attn.rs:1005-1021",
        q=q, kt=kt, v=v, out=oracle.attend_f32(q, kt, v),
        f64=textbook.attention(q, kt, v, k_transposed=True))

    # 7. decode with f16 K/V over one 30 s window (1500 frames), 6 heads: the shipped
    #    cross-attention arm at its real key count
    rng = np.random.default_rng(8)
    q = (rng.standard_normal((1, 6, 1, 64)) * 0.125).astype(np.float32)
    kt16 = rng.standard_normal((1, 6, 64, 1500)).astype(np.float16)
    v16 = rng.standard_normal((1, 6, 1500, 64)).astype(np.float16)
    cases["decode_f16kv_h6_k1500"] = dict(
        ref="FlashAttnOp f16-K/V decode arm, xattn_head_f16 (flash_attn.rs:289-356, 714-789)",
        q=q, kt16=kt16, v16=v16, out=oracle.attend_f16kv(q, kt16, v16),
        f64=textbook.attention(q, kt16.astype(np.float32), v16.astype(np.float32),
                               k_transposed=True))

    # 8. bf16-rounded encoder rows at the large-v3 frame count (1500; 2 heads), K transposed as
    #    the reference's encoder produces it; outputs kept for spot rows (first, middle and
    #    last 64) to keep the fixture small
    rng = np.random.default_rng(9)
    h, t = 2, 1500
    q = oracle.round_bf16(rng.standard_normal((1, h, t, 64)).astype(np.float32))
    kt = oracle.round_bf16(rng.standard_normal((1, h, 64, t)).astype(np.float32))
    v = oracle.round_bf16(rng.standard_normal((1, h, t, 64)).astype(np.float32))
    rows = np.r_[0:64, 704:768, 1436:1500].astype(np.int32)
    full = oracle.attend_general(q, kt, v, k_transposed=True, scale=0.125)
    f64 = textbook.attention(q, kt, v, k_transposed=True, scale=0.125)
    cases["encoder_bf16_h2_t1500"] = dict(
        ref="encoder attention on bf16 operands (configs 2/4 at 2 heads; extension of the f32 kernel)",
        q_bf16=bf16_bits(q), kt_bf16=bf16_bits(kt), v_bf16=bf16_bits(v), scale=np.float32(0.125),
        rows=rows, out=full[:, :, rows], f64=f64[:, :, rows])

    only = set(sys.argv[1:])
    for name, arrays in cases.items():
        if only and name not in only:
            continue
        path = os.path.join(OUT, f"{name}.npz")
        ref = arrays.pop("ref")
        # the float64 closed form is stored rounded to f32 (6e-8 relative: far below any bar)
        arrays["f64"] = arrays["f64"].astype(np.float32)
        np.savez_compressed(path, ref=np.array(ref), **arrays)
        print(f"wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB)")


if __name__ == "__main__":
    main()
