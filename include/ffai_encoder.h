/*
 * ffai_encoder.h -- C ABI of the audio encoder's self-attention block on MI355X (gfx950):
 * projections, fused attention and out-projection in one stream-ordered call.
 *
 * Replaces EncoderAttention::forward (crates/ffai-mercury/src/asr/text_decoder.rs:1059-1139):
 *   q  = x Wq^T + bq                      (self.inner.query, :1088)
 *   kt = Wk_scaled x^T  -> (heads, hd, T)  (key_wt_scaled.matmul(x.t()), :1090-1094; no bias)
 *   v  = x Wv^T + bv                      (self.inner.value, :1097)
 *   merged = attend_merged(q, kt, v)      (:1121-1125; scale already folded into Wk)
 *   out = merged Wo^T + bo                (self.inner.out, :1126)
 * The reference splits q and v into heads with a copy each (:1103-1117) and loops over batch
 * items (:1069-1076). Here the projections land in the layouts the kernel reads by stride (no
 * copies): hipBLASLt GEMMs with bias epilogues (bf16/f16 in and out, f32 accumulation) around
 * ffai_attn_fwd. With packed weights (wqkv, bqkv) the three input projections are one GEMM. The
 * windows run in passes of at most 1500 rows (one 30 s window, or several shorter ones per
 * pass), each pass one launch per GEMM and one attention call, all through the same workspace;
 * a window of more than 1500 frames is refused.
 *
 * All calls are asynchronous on `stream` (a hipStream_t; NULL = null stream), allocate nothing,
 * take device pointers and return FFAI_OK or a negative ffai_status (ffai_attn.h), with the
 * reason in ffai_attn_last_error().
 */
#ifndef FFAI_ENCODER_H
#define FFAI_ENCODER_H

#include <stddef.h>
#include <stdint.h>

#include "ffai_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ffai_encoder_attn_desc {
  int32_t dtype;   /* FFAI_BF16 or FFAI_F16: x, weights, biases and out */
  int32_t batch;   /* windows */
  int32_t seq;     /* frames per window (1500 for 30 s of audio) */
  int32_t n_state; /* model width; head_dim = n_state / n_head must be 64 or 128 */
  int32_t n_head;
  int32_t reserved0;
} ffai_encoder_attn_desc;

/* Weights in the reference's layout: each Linear weight is (out, in) row-major, each bias
 * (out). wk_scaled is the key weight multiplied by head_dim^-0.5 once, at load
 * (EncoderAttention::load, text_decoder.rs:1039-1050); the key projection has no bias.
 * Optionally the three input projections packed once at load: wqkv = [wq; wk_scaled; wv], one
 * (3 n_state, n_state) row-major matrix, and bqkv = [bq; zeros(n_state); bv]. When both are
 * set, one GEMM computes q, k and v side by side (the attention then reads K as rows) and wq,
 * bq, wk_scaled, wv and bv are not read; otherwise those five are required. */
typedef struct ffai_encoder_attn_weights {
  const void* wq;
  const void* bq;
  const void* wk_scaled;
  const void* wv;
  const void* bv;
  const void* wo;
  const void* bo;
  const void* wqkv; /* optional, see above (NULL when not packed) */
  const void* bqkv; /* optional, see above (NULL when not packed) */
} ffai_encoder_attn_weights;

/* Bytes of device workspace ffai_encoder_attn_fwd needs for `d`, packed weights or not: q, k and
 * v and the merged attention output of one pass (at most 1500 rows) in the compute dtype, the
 * attention's own workspace, and GEMM scratch. */
int ffai_encoder_attn_workspace_bytes(const ffai_encoder_attn_desc* d, size_t* bytes);

/* x: (batch, seq, n_state) row-major; out: the same shape. workspace: at least
 * ffai_encoder_attn_workspace_bytes(d), 256-byte aligned, zeroed once before its first use (it
 * holds the attention's split counters, which every call leaves zero). */
int ffai_encoder_attn_fwd(const ffai_encoder_attn_desc* d, const void* x,
                          const ffai_encoder_attn_weights* w, void* out, void* workspace,
                          size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FFAI_ENCODER_H */
