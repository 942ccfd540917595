//! ffai-hip: the MI355X (gfx950) fused attention of FFai's Whisper path as a Rust crate.
//!
//! `build.rs` compiles `libffai_attn.so` from this repository's HIP sources (or links a
//! prebuilt one) and `ffi` declares its C ABI (`include/*.h`). `flash_attn` offers the
//! reference's `serves` / `attend` / `attend_merged` over device views, for a candle HIP backend
//! to call from its `CustomOp3` device path in place of `cpu_fwd`
//! (crates/ffai-mercury/src/asr/flash_attn.rs:165-178, 272-285), plus the general descriptor
//! call. ffai-mercury would take it behind a `hip` feature, as ffai-core forwards its `cuda` and
//! `metal` features to candle (crates/ffai-core/Cargo.toml:27-28).

pub mod ffi;
pub mod flash_attn;

pub use flash_attn::{attend, attend_merged, serves, Attention, DType, DeviceView, FfaiError,
                     Workspace};

/// The ABI version of the linked library matches the one these declarations were written for.
pub fn abi_matches() -> bool {
    // SAFETY: a plain getter of the library.
    unsafe { ffi::ffai_attn_abi_version() == ffi::FFAI_ATTN_ABI_VERSION }
}
