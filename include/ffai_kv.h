/*
 * ffai_kv.h -- C ABI of the device-resident decode-step state that feeds the fused attention
 * path on MI355X (gfx950).
 *
 * The reference keeps the decoder's attention state as candle tensors on the host
 * (crates/ffai-mercury/src/asr/text_decoder.rs):
 *   - the self-attention cache of each layer is the raw (b, L, n_state) projection, grown by
 *     Tensor::cat every step (forward_self, :652-662) and re-split into heads and transposed in
 *     full before every attention call (attend, :840-842);
 *   - beam search snapshots and restores those caches per beam (TextDecoder::save/restore,
 *     :1350-1381; decode_beam, crates/ffai-mercury/src/asr/decoder.rs:559-583);
 *   - the cross-attention cache is split into heads, K transposed, converted to the cache dtype
 *     once per window (forward_cross, :706-707, :770-773).
 * Here the state lives in HBM in the layout the attention kernels read -- head-major rows
 * (slot, head, position, head_dim) -- and three entry points replace those steps:
 *   ffai_kv_append       <- Tensor::cat + split_heads per step (forward_self, :652-662, :840-842)
 *   ffai_kv_advance      <- the length half of that step, for every layer at once, when
 *                           ffai_gemv_f16_qkv_cache (ffai_gemv.h) writes the rows itself
 *   ffai_kv_gather       <- DecoderState save/restore across a beam step (:1350-1381,
 *                           decoder.rs:559-583)
 *   ffai_cross_kv_build  <- the cross-attention cache build (forward_cross, :706-707, :770-773)
 *
 * All calls are asynchronous on `stream` (a hipStream_t; NULL = null stream), allocate nothing,
 * take device pointers, and return FFAI_OK or a negative ffai_status (ffai_attn.h); the reason
 * is then in ffai_attn_last_error(). Strides are in elements.
 */
#ifndef FFAI_KV_H
#define FFAI_KV_H

#include <stddef.h>
#include <stdint.h>

#include "ffai_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* A self-attention K/V cache: k and v are (slots, heads, capacity, head_dim) with head_dim
 * contiguous; lens[s] keys are held by slot s. This is the FFAI_K_ROWS layout ffai_attn_fwd
 * reads with kv_lens = lens (one slot per batch item, e.g. per beam). */
typedef struct ffai_kv_cache {
  void* k;
  void* v;
  int32_t* lens;      /* device int32[slots] */
  int32_t dtype;      /* ffai_dtype of k and v */
  int32_t slots, heads, capacity, head_dim;
  int32_t reserved0;
  int64_t strides[3]; /* slot, head, position strides of k and v (head_dim stride is 1) */
} ffai_kv_cache;

/* Append t_new rows per slot: row t of slot s of the projections (new_k/new_v: element
 * (s, t, h * head_dim + d) at s * src_slot_stride + t * src_row_stride + h * head_dim + d, of
 * src_dtype) goes to position lens[s] + t of head h; then lens[s] += t_new. Rows that would land
 * at or past `capacity` are not written and lens saturates at capacity (the caller sizes the
 * cache for its longest sequence). Values are converted to the cache dtype by round-to-nearest-
 * even. Replaces Tensor::cat of the raw projections (text_decoder.rs:658-662) and the per-step
 * split_heads of the whole cache (:640-643, :840-842). */
int ffai_kv_append(const ffai_kv_cache* c, const void* new_k, const void* new_v, int32_t src_dtype,
                   int32_t t_new, int64_t src_slot_stride, int64_t src_row_stride, void* stream);

/* Advance the lengths of every layer of a layer-stacked cache by t_new, as ffai_kv_append does
 * after writing its rows: lens[l * lens_layer_stride + s] = min(capacity, l0 + t_new) with l0
 * the old length clamped to [0, capacity], for l < layers and s < c->slots (c describes layer
 * 0). With ffai_gemv_f16_qkv_cache (ffai_gemv.h) a decode step calls it once before its layers,
 * in place of one append per layer. layers in [1, 65535]; lens_layer_stride >= slots when
 * layers > 1. */
int ffai_kv_advance(const ffai_kv_cache* c, int32_t t_new, int32_t layers,
                    int64_t lens_layer_stride, void* stream);

/* Beam reorder: slot i of dst becomes a copy of slot parent[i] of src (its first
 * src.lens[parent[i]] positions) and dst.lens[i] = src.lens[parent[i]], in each of `layers`
 * decoder layers at once. dst and src describe layer 0; layer l's k and v start layer_stride
 * elements after layer l-1's (in both caches) and its lens lens_layer_stride ints after
 * (>= slots); with layers == 1 both strides are ignored. parent is a device int32[dst.slots] of
 * values in [0, src.slots), shared by all layers. dst and src must be distinct caches of the
 * same dtype, heads, head_dim and capacity (callers alternate two). One launch per beam step
 * replaces the per-beam DecoderState restore of every layer (decoder.rs:559-583,
 * text_decoder.rs:1350-1381). */
int ffai_kv_gather(const ffai_kv_cache* dst, const ffai_kv_cache* src, const int32_t* parent,
                   int32_t layers, int64_t layer_stride, int64_t lens_layer_stride, void* stream);

/* Cross-attention cache build: k_proj and v_proj are (t, heads * head_dim) row-major (row stride
 * src_row_stride) projections of the encoder output; writes v_out as (heads, t, head_dim) and
 * k_out as (heads, head_dim, t) when k_layout == FFAI_K_TRANSPOSED (the reference's layout) or
 * (heads, t, head_dim) when FFAI_K_ROWS, both packed, in out_dtype (round-to-nearest-even). No
 * scaling: the reference carries the whole scale on q. Replaces forward_cross's
 * split_heads(k).transpose(2,3).contiguous(), split_heads(v).contiguous() and to_dtype
 * (text_decoder.rs:706-707, 770-773). */
int ffai_cross_kv_build(const void* k_proj, const void* v_proj, int32_t src_dtype, int32_t t,
                        int32_t heads, int32_t head_dim, int64_t src_row_stride, void* k_out,
                        void* v_out, int32_t out_dtype, int32_t k_layout, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FFAI_KV_H */
