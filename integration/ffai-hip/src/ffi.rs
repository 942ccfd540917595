//! Raw declarations of the C ABI in `include/ffai_attn.h`, `ffai_kv.h`, `ffai_encoder.h`,
//! `ffai_gemv.h` and `ffai_probe.h`, field for field and argument for argument.
//! `tests/test_rust_binding_cpu.py` checks that every function the headers declare is declared
//! here with the same number of arguments.

#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

pub const FFAI_ATTN_ABI_VERSION: c_int = 1;

// enum ffai_status
pub const FFAI_OK: c_int = 0;
pub const FFAI_DECLINED: c_int = 1;
pub const FFAI_ERR_INVALID: c_int = -1;
pub const FFAI_ERR_HIP: c_int = -2;
pub const FFAI_ERR_WORKSPACE: c_int = -3;
pub const FFAI_ERR_DEVICE: c_int = -4;

// enum ffai_dtype
pub const FFAI_F32: i32 = 0;
pub const FFAI_F16: i32 = 1;
pub const FFAI_BF16: i32 = 2;

// enum ffai_k_layout
pub const FFAI_K_TRANSPOSED: i32 = 0;
pub const FFAI_K_ROWS: i32 = 1;

/// `ffai_attn_desc`: one attention call (strides in elements; see the header).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct ffai_attn_desc {
    pub q_dtype: i32,
    pub kv_dtype: i32,
    pub out_dtype: i32,
    pub batch: i32,
    pub heads_q: i32,
    pub heads_kv: i32,
    pub q_len: i32,
    pub kv_len: i32,
    pub head_dim: i32,
    pub k_layout: i32,
    pub causal: i32,
    pub q_offset: i32,
    pub scale: f32,
    pub reserved0: i32,
    pub q_strides: [i64; 4],
    pub k_strides: [i64; 4],
    pub v_strides: [i64; 4],
    pub o_strides: [i64; 4],
    pub kv_lens: *const i32,
}

/// `ffai_tensor`: a 4-D view of device memory.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct ffai_tensor {
    pub data: *mut c_void,
    pub dtype: i32,
    pub on_device: i32,
    pub dims: [i64; 4],
    pub strides: [i64; 4],
}

/// `ffai_kv_cache`: a decoder self-attention cache (include/ffai_kv.h).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct ffai_kv_cache {
    pub k: *mut c_void,
    pub v: *mut c_void,
    pub lens: *mut i32,
    pub dtype: i32,
    pub slots: i32,
    pub heads: i32,
    pub capacity: i32,
    pub head_dim: i32,
    pub reserved0: i32,
    pub strides: [i64; 3],
}

/// `ffai_encoder_attn_desc` (include/ffai_encoder.h).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct ffai_encoder_attn_desc {
    pub dtype: i32,
    pub batch: i32,
    pub seq: i32,
    pub n_state: i32,
    pub n_head: i32,
    pub reserved0: i32,
}

/// `ffai_encoder_attn_weights` (include/ffai_encoder.h); `wqkv`/`bqkv` null when not packed.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct ffai_encoder_attn_weights {
    pub wq: *const c_void,
    pub bq: *const c_void,
    pub wk_scaled: *const c_void,
    pub wv: *const c_void,
    pub bv: *const c_void,
    pub wo: *const c_void,
    pub bo: *const c_void,
    pub wqkv: *const c_void,
    pub bqkv: *const c_void,
}

extern "C" {
    // ---- include/ffai_attn.h: descriptor path
    pub fn ffai_attn_desc_init(d: *mut ffai_attn_desc, q_dtype: i32, kv_dtype: i32,
                               out_dtype: i32, batch: i32, heads_q: i32, heads_kv: i32,
                               q_len: i32, kv_len: i32, head_dim: i32, k_layout: i32);
    pub fn ffai_attn_serves(d: *const ffai_attn_desc) -> c_int;
    pub fn ffai_attn_workspace_bytes(d: *const ffai_attn_desc, bytes: *mut usize) -> c_int;
    pub fn ffai_attn_fwd(d: *const ffai_attn_desc, q: *const c_void, k: *const c_void,
                         v: *const c_void, out: *mut c_void, workspace: *mut c_void,
                         workspace_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn ffai_attn_fwd_noalloc(d: *const ffai_attn_desc, q: *const c_void, k: *const c_void,
                                 v: *const c_void, out: *mut c_void, stream: *mut c_void)
                                 -> c_int;
    pub fn ffai_attn_noalloc_scratch_bytes() -> usize;
    pub fn ffai_attn_plan_info(d: *const ffai_attn_desc, info: *mut i32) -> c_int;
    pub fn ffai_attn_plan_splits(d: *const ffai_attn_desc, info: *mut i32) -> c_int;
    pub fn ffai_attn_noalloc_plan_info(d: *const ffai_attn_desc, info: *mut i32,
                                       bytes: *mut usize) -> c_int;

    // ---- include/ffai_attn.h: mirrors of flash_attn.rs
    pub fn ffai_serves(kt: *const ffai_tensor, v: *const ffai_tensor) -> c_int;
    pub fn ffai_attend(q: *const ffai_tensor, kt: *const ffai_tensor, v: *const ffai_tensor,
                       masked: c_int, out: *mut ffai_tensor, workspace: *mut c_void,
                       workspace_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn ffai_attend_workspace_bytes(q: *const ffai_tensor, kt: *const ffai_tensor,
                                       v: *const ffai_tensor, bytes: *mut usize) -> c_int;
    pub fn ffai_attend_merged(q: *const ffai_tensor, kt: *const ffai_tensor,
                              v: *const ffai_tensor, out: *mut ffai_tensor,
                              workspace: *mut c_void, workspace_bytes: usize,
                              stream: *mut c_void) -> c_int;
    pub fn ffai_attend_merged_workspace_bytes(q: *const ffai_tensor, kt: *const ffai_tensor,
                                              v: *const ffai_tensor, bytes: *mut usize)
                                              -> c_int;

    // ---- include/ffai_attn.h: knobs and errors
    pub fn ffai_get_decode_min_keys() -> c_int;
    pub fn ffai_set_decode_min_keys(n: c_int);
    pub fn ffai_get_decode_tiles_per_wg() -> c_int;
    pub fn ffai_set_decode_tiles_per_wg(n: c_int);
    pub fn ffai_set_attn_variant(variant: c_int);
    pub fn ffai_get_attn_variant() -> c_int;
    pub fn ffai_set_geometry_override(cus: c_int, xcds: c_int);
    pub fn ffai_set_fwd_split_override(items: c_int, pieces: c_int);
    pub fn ffai_get_fwd_split_override(items: *mut c_int, pieces: *mut c_int);
    pub fn ffai_attn_last_error() -> *const c_char;
    pub fn ffai_attn_abi_version() -> c_int;

    // ---- include/ffai_kv.h
    pub fn ffai_kv_append(c: *const ffai_kv_cache, new_k: *const c_void, new_v: *const c_void,
                          src_dtype: i32, t_new: i32, src_slot_stride: i64,
                          src_row_stride: i64, stream: *mut c_void) -> c_int;
    pub fn ffai_kv_gather(dst: *const ffai_kv_cache, src: *const ffai_kv_cache,
                          parent: *const i32, layers: i32, layer_stride: i64,
                          lens_layer_stride: i64, stream: *mut c_void) -> c_int;
    pub fn ffai_kv_advance(c: *const ffai_kv_cache, t_new: i32, layers: i32,
                           lens_layer_stride: i64, stream: *mut c_void) -> c_int;
    pub fn ffai_cross_kv_build(k_proj: *const c_void, v_proj: *const c_void, src_dtype: i32,
                               t: i32, heads: i32, head_dim: i32, src_row_stride: i64,
                               k_out: *mut c_void, v_out: *mut c_void, out_dtype: i32,
                               k_layout: i32, stream: *mut c_void) -> c_int;

    // ---- include/ffai_encoder.h
    pub fn ffai_encoder_attn_workspace_bytes(d: *const ffai_encoder_attn_desc,
                                             bytes: *mut usize) -> c_int;
    pub fn ffai_encoder_attn_fwd(d: *const ffai_encoder_attn_desc, x: *const c_void,
                                 w: *const ffai_encoder_attn_weights, out: *mut c_void,
                                 workspace: *mut c_void, workspace_bytes: usize,
                                 stream: *mut c_void) -> c_int;

    // ---- include/ffai_gemv.h
    pub fn ffai_gemv_f16(w: *const c_void, out_dim: i32, in_dim: i32, x: *const f32, rows: i32,
                         x_row_stride: i64, y: *mut f32, y_row_stride: i64,
                         stream: *mut c_void) -> c_int;
    pub fn ffai_gemv_f16_plan_info(out_dim: i32, in_dim: i32, rows: i32, tile_rows: *mut i32,
                                   waves: *mut i32, blocks_per_wave: *mut i32, passes: *mut i32,
                                   lds_bytes: *mut usize) -> c_int;
    pub fn ffai_gemv_f16_qkv_cache(w: *const c_void, bias: *const f32, in_dim: i32,
                                   x: *const f32, rows: i32, x_row_stride: i64, q: *mut f32,
                                   q_row_stride: i64, c: *const ffai_kv_cache,
                                   stream: *mut c_void) -> c_int;
    pub fn ffai_vocab_int8_quantize(emb: *const c_void, emb_dtype: i32, vocab: i32, d: i32,
                                    blk: i32, qw: *mut i8, bscale: *mut f32, corr: *mut f32,
                                    stream: *mut c_void) -> c_int;
    pub fn ffai_vocab_int8_workspace_bytes(d: i32, rows: i32, bytes: *mut usize) -> c_int;
    pub fn ffai_vocab_int8_logits(qw: *const i8, bscale: *const f32, corr: *const f32,
                                  vocab: i32, d: i32, blk: i32, x: *const f32, rows: i32,
                                  x_row_stride: i64, logits: *mut f32, logits_row_stride: i64,
                                  workspace: *mut c_void, workspace_bytes: usize,
                                  stream: *mut c_void) -> c_int;

    // ---- include/ffai_probe.h (diagnostics)
    pub fn ffai_probe_empty(workgroups: c_int, stream: *mut c_void) -> c_int;
    pub fn ffai_probe_read(src: *const c_void, bytes: usize, out: *mut f32, workgroups: c_int,
                           stream: *mut c_void) -> c_int;
    pub fn ffai_probe_pipes(kind: c_int, workgroups: c_int, iters: c_int, out: *mut f32,
                            stream: *mut c_void) -> c_int;
}
