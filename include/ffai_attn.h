/*
 * ffai_attn.h -- C ABI of the MI355X (gfx950) fused attention path.
 *
 * Replaces the CPU kernel behind the reference's candle CustomOp3 surface
 * (crates/ffai-mercury/src/asr/flash_attn.rs). Two layers:
 *
 *   1. Mirrors of the reference's three public functions, same names, same argument meaning,
 *      same decline contract (return FFAI_DECLINED where the Rust function returns Ok(None)):
 *        ffai_serves        <- flash_attn::serves        (flash_attn.rs:103-129)
 *        ffai_attend        <- flash_attn::attend        (flash_attn.rs:212-264, 266-413)
 *        ffai_attend_merged <- flash_attn::attend_merged (flash_attn.rs:131-158, 160-210)
 *      They take plain tensor views (ffai_tensor) of DEVICE memory and write into a
 *      caller-allocated output: a CustomOp3 shim allocates the output storage and passes it.
 *
 *   2. The general descriptor entry point the mirrors dispatch through, for callers that need
 *      more than the reference served (batch > 1, bf16/f16, grouped K/V heads, head_dim 128,
 *      causal masks with a query offset, ragged per-batch key counts, keys shared across
 *      batch items as in beam-search cross-attention):
 *        ffai_attn_desc_init, ffai_attn_serves, ffai_attn_workspace_bytes, ffai_attn_fwd.
 *
 * Return codes: FFAI_OK (0), FFAI_DECLINED (1, the Ok(None) of the reference: shape, dtype or
 * layout not served -- the caller falls back), negative on error (the Err(candle::Error) of
 * the reference: bad arguments or a HIP failure); ffai_attn_last_error() then describes it.
 *
 * All compute entry points are asynchronous and stream-ordered on `stream` (a hipStream_t;
 * NULL is the device's null stream), allocate no memory, and take device pointers. Distinct
 * streams may be used concurrently from distinct threads. Element strides are in ELEMENTS.
 *
 * Workspace: shapes that split the keys over workgroups need a device workspace of
 * *_workspace_bytes bytes (16-byte aligned) for split counters and partial results. Zero it
 * once, before its first use (hipMemset at allocation, or torch.zeros); every call leaves its
 * counters zero again, so a workspace zeroed once serves any number of calls of any shapes. A
 * workspace belongs to one call at a time: calls that may overlap (different streams) need
 * their own; stream-ordered calls and captured HIP graphs may share one.
 */
#ifndef FFAI_ATTN_H
#define FFAI_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FFAI_ATTN_ABI_VERSION 1

enum ffai_status {
  FFAI_OK = 0,
  FFAI_DECLINED = 1,
  FFAI_ERR_INVALID = -1,   /* malformed descriptor or tensor view                        */
  FFAI_ERR_HIP = -2,       /* a HIP runtime call or kernel launch failed                  */
  FFAI_ERR_WORKSPACE = -3, /* workspace missing or smaller than ffai_attn_workspace_bytes */
  FFAI_ERR_DEVICE = -4     /* current device is not a gfx950 (MI355X-class) GPU           */
};

enum ffai_dtype { FFAI_F32 = 0, FFAI_F16 = 1, FFAI_BF16 = 2 };

enum ffai_k_layout {
  FFAI_K_TRANSPOSED = 0, /* K^T: (batch, heads_kv, head_dim, kv_len), keys contiguous -- the
                            layout the reference's kernel reads (flash_attn.rs:213-217) */
  FFAI_K_ROWS = 1        /* K:   (batch, heads_kv, kv_len, head_dim)                       */
};

/* Strides, in elements, of a 4-D operand: [0] batch, [1] head, [2] row, [3] the second row
 * index. For Q, V, O and rows-layout K: [2] is the stride between sequence rows and [3] must
 * be 1 (head_dim contiguous). For transposed K: [2] is the stride between head_dim rows and [3]
 * must be 1 (keys contiguous). A batch stride of 0 shares one K/V across the batch (the
 * beam-search cross-attention cache). */
typedef struct ffai_attn_desc {
  int32_t q_dtype, kv_dtype, out_dtype; /* ffai_dtype                                    */
  int32_t batch, heads_q, heads_kv;     /* heads_q % heads_kv == 0 (grouped K/V)         */
  int32_t q_len, kv_len, head_dim;      /* head_dim in {64, 128}                         */
  int32_t k_layout;                     /* ffai_k_layout                                 */
  int32_t causal;                       /* key j hidden from query i iff j > q_offset+i  */
  int32_t q_offset;                     /* absolute position of query row 0 (>= 0)       */
  float scale;                          /* scores are multiplied by this before softmax;
                                           1.0 = the reference's pre-scaled convention   */
  int32_t reserved0;
  int64_t q_strides[4], k_strides[4], v_strides[4], o_strides[4];
  const int32_t* kv_lens; /* optional DEVICE int32[batch]: keys valid per batch item (<=
                             kv_len); NULL = kv_len for every item                       */
} ffai_attn_desc;

/* Fill a descriptor for packed operands: q (B,Hq,Tq,D), k per k_layout, v (B,Hkv,Tk,D),
 * out (B,Hq,Tq,D); scale 1, non-causal, no kv_lens. Adjust fields afterwards as needed. */
void ffai_attn_desc_init(ffai_attn_desc* d, int32_t q_dtype, int32_t kv_dtype,
                         int32_t out_dtype, int32_t batch, int32_t heads_q, int32_t heads_kv,
                         int32_t q_len, int32_t kv_len, int32_t head_dim, int32_t k_layout);

/* 1 iff ffai_attn_fwd accepts the descriptor (pointer alignment aside: fwd additionally needs
 * every base pointer aligned to its element size), 0 if it would decline. One predicate for
 * both, so a caller choosing a cache dtype by it never meets a kernel that then declines
 * (the failure flash_attn.rs:113-125 documents). */
int ffai_attn_serves(const ffai_attn_desc* d);

/* Device workspace ffai_attn_fwd needs for this descriptor (split counters and split-key
 * partials; zeroed once before first use, see above); 0 if none. */
int ffai_attn_workspace_bytes(const ffai_attn_desc* d, size_t* bytes);

/* O = softmax(scale * Q K^T [+ causal mask]) V. Returns FFAI_DECLINED for descriptors
 * ffai_attn_serves rejects, FFAI_ERR_WORKSPACE when workspace_bytes is below the required
 * size, FFAI_ERR_HIP when a launch fails. */
int ffai_attn_fwd(const ffai_attn_desc* d, const void* q, const void* k, const void* v,
                  void* out, void* workspace, size_t workspace_bytes, void* stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): ffai_attn_fwd
 * without a workspace argument. The split-key partials go to a scratch array the library owns,
 * one per device (ffai_attn_noalloc_scratch_bytes(): 48 MiB, held from the first call on a
 * device until the process ends); the call allocates nothing. It runs ffai_attn_fwd's kernels
 * on ffai_attn_fwd's plan capped to the scratch: when that plan's partials fit (every shape of
 * the whisper and prefill workloads), the plans are the same and so is the output, bit for bit;
 * otherwise its split items run in fewer key pieces, or whole, and the output equals
 * ffai_attn_fwd's to f32 rounding (ffai_attn_noalloc_plan_info reports the plan). Only a layout
 * forced by ffai_set_fwd_split_override that exceeds the scratch returns FFAI_ERR_WORKSPACE.
 * Every call on one device shares that device's
 * scratch: calls that may overlap on one device (different streams, unordered) race; calls
 * ordered on one stream, and replays of captured graphs, do not. The scratch keeps the last
 * call's partials; nothing in it needs clearing between calls. */
int ffai_attn_fwd_noalloc(const ffai_attn_desc* d, const void* q, const void* k, const void* v,
                          void* out, void* stream);

/* Size in bytes of the per-device scratch behind ffai_attn_fwd_noalloc. */
size_t ffai_attn_noalloc_scratch_bytes(void);

/* Diagnostic, no counterpart in the reference: the launch plan ffai_attn_fwd uses for `d` when
 * every operand admits the kernels' vector accesses (16-byte aligned bases and strides), so a
 * test or benchmark can state which kernel shape it ran. info[0]: kernel (0 the fused
 * encoder/prefill kernel, 1 the decode kernel); info[1]: workgroup shape (fused: 0 one wave x
 * 32 query rows, 1 four waves x 32 rows, 2 four waves x 64 rows, 3 the same on 16x16x32 MFMA;
 * decode: waves per workgroup);
 * info[2]: key splits per work item (1 = no partials); info[3]: 64-key tiles per split;
 * info[4]: workgroups. Returns FFAI_OK, FFAI_DECLINED or FFAI_ERR_INVALID as
 * ffai_attn_workspace_bytes. */
int ffai_attn_plan_info(const ffai_attn_desc* d, int32_t info[5]);

/* Diagnostic, no counterpart in the reference: the plan ffai_attn_fwd_noalloc runs for `d`
 * (info as ffai_attn_plan_info) and the scratch bytes it uses (*bytes, at most
 * ffai_attn_noalloc_scratch_bytes()). Returns as ffai_attn_plan_info. */
int ffai_attn_noalloc_plan_info(const ffai_attn_desc* d, int32_t info[5], size_t* bytes);

/* Diagnostic, no counterpart in the reference: which work items of the fused kernel's plan for
 * `d` run as key-split pieces. Items are the (batch, head, query block) triples in dispatch rank
 * (head-major; for a causal launch longest first); info[0]: items, info[1], info[2]: the split
 * ranks [info[1], info[2]) (empty when nothing is split), each in info[2] of plan_info's pieces.
 * Zeros for a decode plan. Returns as ffai_attn_plan_info. */
int ffai_attn_plan_splits(const ffai_attn_desc* d, int32_t info[3]);

/* ------------------------------------------------------------------------------------------
 * Mirrors of the reference's public functions.
 * ---------------------------------------------------------------------------------------- */

/* A 4-D view of device memory (the reference's tensors are all 4-D at this boundary). */
typedef struct ffai_tensor {
  void* data;         /* device pointer to element (0,0,0,0)          */
  int32_t dtype;      /* ffai_dtype                                   */
  int32_t on_device;  /* 0 = host memory: always declined (the GPU path serves device
                         storage only, as the reference serves Device::Cpu only) */
  int64_t dims[4];
  int64_t strides[4]; /* elements */
} ffai_tensor;

/* flash_attn::serves (flash_attn.rs:103-129): kt (1,h,64,K) and v (1,h,K,64) on the device
 * with K >= max(256, decode_min_keys). Callers use it to choose the cross-attention cache
 * dtype before building the cache. Returns 1 or 0. */
int ffai_serves(const ffai_tensor* kt, const ffai_tensor* v);

/* flash_attn::attend (flash_attn.rs:212-264 + FlashAttnOp, :266-413). q (1,H,qlen,64) f32;
 * kt (1,H,64,K) and v (1,H,K,64) both f32 or both f16 (f16 at qlen == 1 only, as the
 * reference); out (1,H,qlen,64) f32, contiguous. Declines (FFAI_DECLINED) exactly where the
 * reference returns Ok(None): masked, q not f32, batch != 1, head_dim != 64, shape mismatch,
 * K below the floor (decode_min_keys at qlen == 1, 256 otherwise), qlen not in {1, K}.
 * Non-contiguous operands are an error, as the reference's bail! (flash_attn.rs:360-363). */
int ffai_attend(const ffai_tensor* q, const ffai_tensor* kt, const ffai_tensor* v, int masked,
                ffai_tensor* out, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace ffai_attend needs for these operands (0 if none or if it would decline). */
int ffai_attend_workspace_bytes(const ffai_tensor* q, const ffai_tensor* kt,
                                const ffai_tensor* v, size_t* bytes);

/* flash_attn::attend_merged (flash_attn.rs:131-158 + MergedAttnOp, :160-210): encoder
 * attention writing the merged (1,T,H*64) f32 layout. Declines unless batch 1, head_dim 64,
 * all f32, qlen == keys >= 256. The workspace (see ffai_attend_merged_workspace_bytes) holds
 * split-key partials when few heads leave the GPU short of work. */
int ffai_attend_merged(const ffai_tensor* q, const ffai_tensor* kt, const ffai_tensor* v,
                       ffai_tensor* out, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace ffai_attend_merged needs for these operands (0 if none or if it would decline). */
int ffai_attend_merged_workspace_bytes(const ffai_tensor* q, const ffai_tensor* kt,
                                       const ffai_tensor* v, size_t* bytes);

/* Knob mirror of knobs::DECODE_MIN_KEYS (knobs.rs:163-168): key-count floor below which the
 * decode shape declines. Initialised from FFAI_DECODE_MIN_KEYS (default 8) on first use. */
int ffai_get_decode_min_keys(void);
void ffai_set_decode_min_keys(int n);

/* Tuning knob, no counterpart in the reference: 64-key tiles per workgroup of the decode kernel
 * (0 = the planner's choice). Initialised from FFAI_DECODE_TILES_PER_WG on first use. It changes
 * how a decode call splits its keys over workgroups, never its result beyond f32 rounding. */
int ffai_get_decode_tiles_per_wg(void);
void ffai_set_decode_tiles_per_wg(int n);

/* Tuning and test hook, no counterpart in the reference: force which items of the fused
 * kernel run as key-split pieces. items > 0: that many items (the last ones dispatched of a
 * non-causal launch, the longest ones of a causal launch), each in `pieces` pieces (1: no item
 * is split); items < 0: every item; items == 0 or pieces < 1: the planner's choice (the default). The
 * workspace a descriptor needs follows the setting. It changes how a call splits its keys,
 * never its result beyond f32 rounding. */
void ffai_set_fwd_split_override(int items, int pieces);
void ffai_get_fwd_split_override(int* items, int* pieces);

/* Tuning and test hook, no counterpart in the reference: force the fused kernel's launch shape
 * (0 one wave x 32 query rows, 1 four waves x 32, 2 four waves x 64, 3 four waves x 64 on the
 * 16x16x32-MFMA kernel; the last two for 16-bit head_dim 64 only) or -1 for the planner's choice.
 * Initialised from FFAI_ATTN_VARIANT on first use. It changes plans, never results beyond f32
 * rounding. Shape 3 is kept as a measured alternative: it is never chosen by the planner. */
void ffai_set_attn_variant(int variant);
int ffai_get_attn_variant(void);

/* Tuning and test hook, no counterpart in the reference: the device geometry the launch plans
 * balance over. By default the current device's CUs and XCDs (hipDeviceAttributeMultiprocessorCount,
 * hipDeviceAttributeNumberOfXccs: 256 and 8 on an MI355X in single-partition mode, a share of them
 * per partition otherwise; 256 and 8 when no device is visible). cus > 0 and xcds > 0 replace it
 * for every device; 0, 0 restores it. It changes plans, never results beyond f32 rounding. */
void ffai_set_geometry_override(int cus, int xcds);

/* Human-readable description of the last error on the calling thread ("" if none). */
const char* ffai_attn_last_error(void);

/* ABI version of the loaded library (FFAI_ATTN_ABI_VERSION at build time). */
int ffai_attn_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FFAI_ATTN_H */
