// Internal interface between the C ABI (attn_api.cpp) and the gfx950 kernels (attn_launch.hip,
// fwd_*.hip, decode.hip). Not installed; callers use include/ffai_attn.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ffai {

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

// Everything a forward launch needs, resolved by the host from an ffai_attn_desc.
struct FwdParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* ws;              // split partials, lane-major: [split items][n_split][waves][column
                          // blocks][D / 32][4][64 lanes] f32x4 O in accumulator order, then
                          // [..][waves][column blocks][32 query columns] (m, l)
  int32_t* counters;      // one per split item (kCounterSlots): zero before the launch and after
  const int32_t* kv_lens; // device int32[B] or nullptr
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;  // k_st: stride between key rows (rows layout) or d rows (K^T)
  int64_t v_sb, v_sh, v_st;
  int64_t o_sb, o_sh, o_st;
  int32_t B, Hq, Hkv, Tq, Tk;
  int32_t causal, q_offset;
  int32_t n_qblk;            // ceil(Tq / block_m)
  // Items are the (batch, head, query block) triples, in rank order: head-major, or for a causal
  // launch longest first (query block descending, then batch and head). Items of rank
  // [split_lo, split_hi) run as n_split pieces (contiguous key ranges of ceil(tiles / n_split)
  // tiles each); the item's last piece to finish merges the others' partials in the same launch.
  int32_t split_lo, split_hi;
  int32_t n_split;           // pieces per split item (1 when no item is split)
  int32_t n_work;            // items + (split_hi - split_lo) * (n_split - 1): works in rank order
  // Dispatch: works [0, sec1_work) take the first sec1_wgs workgroups (a multiple of the XCD
  // count X = 1 << xcd_shift), the rest the remaining ones. With xcd_remap each section deals
  // its works to the X XCDs in contiguous runs (hardware workgroup i goes to XCD i % X), so
  // neighbouring works (one head's query blocks, one item's pieces) share an L2; without it
  // works go in rank order.
  int32_t sec1_work, sec1_wgs;
  int32_t xcd_remap;
  int32_t xcd_shift;         // log2 of the device's XCD count (sections are whole XCD rounds)
  int32_t cus;               // the device's CUs (host side: launch shaping)
  int32_t aligned;           // every operand admits the kernels' vector loads and stores
  int32_t dma;               // 16-bit: whole tiles may go global -> LDS by DMA (aligned, and
                             // each lane's byte offset within a K or V tile fits 32 bits)
  float scale_log2;          // scale * log2(e)
  int32_t o_pair;            // head_dim 64, 16-bit output whose rows admit 16-byte stores: a
                             // lane and its partner (lane ^ 32) exchange halves and store whole
                             // 8-element runs
#ifdef FFAI_STAMPS
  uint64_t* stamps;          // diagnostic builds only: per-wave phase times (attn_common.cuh)
  int32_t stamp_wgs;         // workgroups (by hardware index) that record them
#endif
};

// A decode launch: at most 32 query rows (group x Tq) per (batch, kv-head) unit, operands that
// admit 16-byte Q/K/V row accesses (8-byte K^T rows) and 4-element output stores.
struct DecodeParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* ws;              // split partials: [B*Hkv][n_split][R][D] O, then [..][R][2] (m, l)
  int32_t* counters;      // split counters, one per unit: zero before the launch, zero after
  const int32_t* kv_lens; // device int32[B] or nullptr
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int64_t o_sb, o_sh, o_st;
  int32_t B, Hkv, group, Tq, Tk;  // group = Hq / Hkv; rows per unit R = group * Tq <= 32
  int32_t causal, q_offset;
  int32_t n_split;          // workgroups per unit
  int32_t tiles_per_split;  // 64-key tiles per workgroup
  int32_t n_work;           // B * Hkv * n_split
  float scale_log2;
#ifdef FFAI_STAMPS
  uint64_t* stamps;         // diagnostic builds only: per-workgroup event times
  int32_t stamp_wgs;        // workgroups (by linear hardware index) that record them
#endif
};
// Workspace layout shared by every plan: kCounterBytes of split counters (decode units or split
// fwd items, one int32 each; zero at rest) first, then the partials of whichever kernel the plan
// runs. The counters keep that place whatever plan last used the workspace, so partials never
// overwrite them and a workspace zeroed once stays usable by every plan.
constexpr int kCounterSlots = 1024;
constexpr size_t kCounterBytes = kCounterSlots * sizeof(int32_t);
// Key splits of one decode unit at most (the merge loops over them).
constexpr int kMaxDecodeSplits = 64;
// Pieces of one split fwd item at most (its merge loops over them).
constexpr int kMaxFwdSplits = 64;

// Launchers; return hipSuccess or the launch error.
// mode: kBF16 / kF16 (MFMA bf16/f16 kernel, q and kv the same 16-bit type) or kF32 (f32 MFMA
// kernel; kv may be f32, f16 or bf16, widened to f32 as it is staged).
// out_dtype: kF32, kF16 or kBF16. k_transposed: K^T layout.
// variant: launch shape (see Variant).
enum Variant : int {
  kWave1 = 0,   // 1 wave x 32 query rows per workgroup (decode, short queries)
  kWave4 = 1,   // 4 waves x 32 rows (128 rows; head_dim 128 and the f32 kernel)
  kWave4x2 = 2,  // 4 waves x 64 rows (256 rows; 16-bit head_dim 64: two column blocks per wave)
  kWave4x2x16 = 3  // the same shape on 16x16x32 MFMA (fwd16_kernel, attn_kernels16.cuh)
};
inline int block_m_of(int variant) { return variant == kWave1 ? 32 : variant == kWave4 ? 128 : 256; }

// The grid is sec1_wgs plus the second section's works rounded up to a multiple of 8.
hipError_t launch_fwd(const FwdParams& p, int mode, int kv_dtype, int out_dtype, int head_dim,
                      bool k_transposed, int variant, hipStream_t stream);
// Per-dtype instantiation units (fwd_bf16.hip, fwd_f16.hip, fwd_f32.hip).
hipError_t launch_fwd_bf16(const FwdParams& p, int out_dtype, int d, bool kt, int variant,
                           hipStream_t s);
hipError_t launch_fwd_f16(const FwdParams& p, int out_dtype, int d, bool kt, int variant,
                          hipStream_t s);
hipError_t launch_fwd_f32(const FwdParams& p, int kv_dtype, int d, bool kt, int variant,
                          hipStream_t s);

// The decode kernel with `waves` (1, 2, 4 or 8; 8 only for head_dim 64) waves per workgroup;
// with p.n_split > 1 the unit's last workgroup merges the splits (p.counters zeroed).
hipError_t launch_decode(const DecodeParams& p, int mode, int out_dtype, int head_dim,
                         bool k_transposed, int waves, hipStream_t stream);
// f32 queries, one query row per (batch, kv-head) unit (group x Tq == 1), head_dim 64, K/V of
// type kv_dtype (kF32, kF16 or kBF16), f32 output (decode_vec.hip); `waves` 1, 2, 4 or 8.
hipError_t launch_decode_vec(const DecodeParams& p, int kv_dtype, bool k_transposed, int waves,
                             hipStream_t stream);
// f16 inputs (decode_f16.hip), called by launch_decode.
hipError_t launch_decode_f16(const DecodeParams& p, int out_dtype, int head_dim,
                             bool k_transposed, int waves, hipStream_t stream);

// Error and device helpers of the C ABI (attn_api.cpp), for the other entry-point units.
int api_fail(int code, const char* msg);  // records msg for ffai_attn_last_error, returns code
void api_clear_error();
int api_check_device();                   // FFAI_OK, or an error code on a non-gfx950 device

constexpr int kBlockN = 64;  // keys per tile

}  // namespace ffai
