/*
 * ffai_gemv.h -- C ABI of the decoder's single-row projections on MI355X (gfx950): the f16
 * weight GEMV and the block-scaled int8 vocabulary projection.
 *
 * Replaces crates/ffai-mercury/src/asr/f16_gemv.rs (F16Gemv: f16 weights, f32 activations,
 * f32 arithmetic) and crates/ffai-mercury/src/asr/vocab_int8.rs (Int8Vocab: one scale per
 * 32-weight block, 7-bit offset activations, a per-row correction folded at load), the two
 * HBM-bound operations of a decode step outside attention (text_decoder.rs:925-1006). Each
 * call takes every beam's row at once, so the weights stream from HBM once per step instead
 * of once per beam.
 *
 * All calls are asynchronous on `stream` (a hipStream_t; NULL = null stream), allocate nothing,
 * take device pointers and return FFAI_OK or a negative ffai_status (ffai_attn.h), with the
 * reason in ffai_attn_last_error().
 */
#ifndef FFAI_GEMV_H
#define FFAI_GEMV_H

#include <stddef.h>
#include <stdint.h>

#include "ffai_attn.h"
#include "ffai_kv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* y[r][o] = sum_i W[o][i] * x[r][i] for r < rows: W (out_dim, in_dim) f16 row-major (the
 * layout QLinear stores, F16Gemv::new, f16_gemv.rs:88-115), x f32 rows (row stride
 * x_row_stride), y f32 rows (row stride y_row_stride). in_dim a multiple of 8 (the reference's
 * decline rule, :101-103), rows <= 16. The reference multiplies and adds in f32
 * (F16Gemv::forward / dot_f16, :117-196). Here the products run on the matrix cores: each x
 * element is scaled by a power of two and carried as the sum of two f16 values (22 significant
 * bits), the f16 x f16 products are exact in f32 and sum in f32, in another order than the
 * reference's 16-lane AVX order; results agree to f32 rounding, not bit for bit. A call gives
 * the same bits every time. An infinite x gives the infinite sums f32 arithmetic gives; an
 * infinite weight can give NaN where f32 arithmetic gives +-inf (it also multiplies x's low
 * half, which may be 0). */
int ffai_gemv_f16(const void* w, int32_t out_dim, int32_t in_dim, const float* x, int32_t rows,
                  int64_t x_row_stride, float* y, int64_t y_row_stride, void* stream);

/* Launch shape ffai_gemv_f16 and ffai_gemv_f16_qkv_cache (with out_dim = 3 * heads * head_dim)
 * choose for (out_dim, in_dim, rows): weight rows per tile (workgroup), waves per workgroup,
 * 32-element blocks per wave and pass, passes over in_dim, and dynamic LDS bytes. A diagnostic
 * query with no counterpart in the reference. */
int ffai_gemv_f16_plan_info(int32_t out_dim, int32_t in_dim, int32_t rows, int32_t* tile_rows,
                            int32_t* waves, int32_t* blocks_per_wave, int32_t* passes,
                            size_t* lds_bytes);

/* The self-attention q/k/v projection of a decode step, with the new K/V rows written straight
 * into the layer's cache: replaces, for single-token steps, the three GEMVs of forward_self
 * (text_decoder.rs:652-655; QLinear::forward, Half arm, :281-293, with its bias added after the
 * product) followed by ffai_kv_append of the k and v rows (the Tensor::cat of :657-662).
 * w: the packed (3 * heads * head_dim, in_dim) f16 weights, rows q, then k, then v; bias: 3 *
 * heads * head_dim f32 (0 for the bias-free k rows) or NULL. Row r of x (beam r, slot r of the
 * cache) gives q row r (row stride q_row_stride, f32) and the k and v rows at position
 * lens[r] - 1 of slot r, converted to the cache dtype by round-to-nearest-even: the step's
 * ffai_kv_advance runs before the layer, so that position is the one it opened. Per output the
 * GEMV sum is that of ffai_gemv_f16 and the bias a separate f32 add, so q and the cache rows
 * equal ffai_gemv_f16 + bias + ffai_kv_append bit for bit, except where the cache was already
 * full before the advance: the append drops the row, this call replaces the last one. A slot
 * whose length is 0 gets no row. rows in [1, 16] and at most c->slots; in_dim a multiple of 8. */
int ffai_gemv_f16_qkv_cache(const void* w, const float* bias, int32_t in_dim, const float* x,
                            int32_t rows, int64_t x_row_stride, float* q, int64_t q_row_stride,
                            const ffai_kv_cache* c, void* stream);

/* Int8Vocab::new (vocab_int8.rs:100-170): quantize the (vocab, d) embedding matrix (f32, f16
 * or bf16, row-major) with one scale per `blk` weights: scale = amax / 127 (1 where the block
 * is all zero), q = round-half-away(w / scale) clamped to [-127, 127]; corr[v] =
 * 64 * sum_b scale_b * sum(q of block b), summed over blocks in order. Writes qw (vocab * d
 * int8), bscale (vocab * d / blk f32) and corr (vocab f32). blk a multiple of 32 dividing d.
 * Bit-identical to the reference's arithmetic (IEEE f32, no fused multiply-add). */
int ffai_vocab_int8_quantize(const void* emb, int32_t emb_dtype, int32_t vocab, int32_t d,
                             int32_t blk, int8_t* qw, float* bscale, float* corr, void* stream);

/* Bytes of device workspace ffai_vocab_int8_logits needs (the quantized activations). */
int ffai_vocab_int8_workspace_bytes(int32_t d, int32_t rows, size_t* bytes);

/* Int8VocabOp::cpu_fwd (vocab_int8.rs:223-262) for `rows` activation rows (one per beam) at
 * once: per row, sx = amax(x) / 63 (1 if x is all zero), x_u = round-half-away(x / sx)
 * clamped to [-64, 63] plus 64; per vocab row v, acc = sum over blocks b, in order, of
 * (dot(x_u, q) over the block as an exact integer) * bscale[v][b]; logit = (acc - corr[v]) * sx.
 * x: rows x d f32 (row stride x_row_stride); logits: rows x vocab f32 (row stride
 * logits_row_stride). Bit-identical to the reference's arithmetic. */
int ffai_vocab_int8_logits(const int8_t* qw, const float* bscale, const float* corr,
                           int32_t vocab, int32_t d, int32_t blk, const float* x, int32_t rows,
                           int64_t x_row_stride, float* logits, int64_t logits_row_stride,
                           void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FFAI_GEMV_H */
