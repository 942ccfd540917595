// Types and device helpers shared by the gfx950 attention kernels (fwd_kernel, decode_kernel).
#pragma once

#include "attn_kernels.h"

#include <type_traits>

namespace ffai {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int BN = kBlockN;
constexpr float kNegInf = -__builtin_huge_valf();
// The running max is only raised when a tile's max exceeds it by more than this (log2 units).
constexpr float kRescaleSlack = 8.0f;
// 16-bit encoder kernel: a lane's sum of 16 weights above this (2^64) sends the subtile to the
// exact-max path, so no weight exceeds it.
constexpr float kWeightSumBound = 18446744073709551616.0f;
// 16-bit encoder kernel: when every row max of a wave's first 32 keys lies in this window
// (scaled log2 units), the wave takes 0 as every row's reference max, so a weight is exp2 of the
// score itself: the largest weight of a row is then at least 2^-64, and a subtile's lane sum
// starts far below kWeightSumBound.
constexpr float kFastMaxLo = -64.0f;
constexpr float kFastMaxHi = 32.0f;
// The same window for f16 weights, which are subnormal below 2^-14, flush to zero below 2^-24 and
// overflow above 65504: a row max below -4 would leave every weight of the row subnormal or zero
// (a row of scores near -40 would sum to 0), so f16 takes the fast path only when the largest
// weight of the first subtile lies in [2^-4, 2^15]. Keys 10 log2 units below that max are then
// still normal, and the keys that underflow weigh at most 2^-20 of the max each.
constexpr float kFastMaxLoF16 = -4.0f;
constexpr float kFastMaxHiF16 = 15.0f;

template <int DT>
using store_t = std::conditional_t<DT == kF32, float, uint16_t>;

// Cache-policy operand of the buffer load/store builtins: SC1 set, i.e. device scope (the access
// is coherent at the device level: stores reach the coherence point before they are
// acknowledged, loads do not hit a stale copy in a non-coherent cache).
constexpr int kDeviceScope = 16;
// Fourth dword of a raw (unformatted, stride 0) buffer resource on this GPU.
constexpr int kBufferWord3 = 0x00020000;

// ---------------------------------------------------------------------------------------------
// Conversions.
// ---------------------------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ float to_f32(uint32_t bits16) {
  if constexpr (DT == kBF16) {
    return __uint_as_float(bits16 << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
  }
}

// Two floats to a packed pair (round to nearest even; one v_cvt_pk_* instruction).
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const f32x2 x = {lo, hi};
  if constexpr (DT == kBF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, f16x2));
  }
}

template <int DT>
__device__ __forceinline__ uint16_t from_f32(float x) {
  return (uint16_t)(pack2<DT>(x, 0.f) & 0xffffu);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The same value from lane l and lane l^32 (v_permlane32_swap): returns {own, partner} in some
// order, which is all a max or a sum needs.
__device__ __forceinline__ float partner_max(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float partner_sum(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Element k (0..7) of eight 16-bit values held in a u32x4, paired with the same element of a
// second row: low half from `r0`, high half from `r1` (one v_perm_b32).
__device__ __forceinline__ uint32_t pair_elem(u32x4 r0, u32x4 r1, int k) {
  const uint32_t a = r0[k >> 1], b = r1[k >> 1];
  return (k & 1) ? __builtin_amdgcn_perm(b, a, 0x07060302u)
                 : __builtin_amdgcn_perm(b, a, 0x05040100u);
}
// Same for four 16-bit values held in a u32x2.
__device__ __forceinline__ uint32_t pair_elem4(u32x2 r0, u32x2 r1, int k) {
  const uint32_t a = r0[k >> 1], b = r1[k >> 1];
  return (k & 1) ? __builtin_amdgcn_perm(b, a, 0x07060302u)
                 : __builtin_amdgcn_perm(b, a, 0x05040100u);
}

// Transposing LDS read (ds_read_b64_tr_b16): see the geometry note at its use.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_tr(const uint16_t* p) {
  typedef __attribute__((address_space(3))) s16x4* lds_ptr;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr)(p)));
}

// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4): lane l's
// bytes land at LDS byte address `lds_block` + 16 l. Issued as inline assembly so that the
// compiler does not wait for it before unrelated LDS reads (it cannot tell which buffer a DMA
// fills); the caller waits (vm_wait_all) before the barrier that publishes the data. M0 is set
// here and used by nothing else in these kernels. An LDS DMA that reads M0 right after a scalar
// instruction wrote it needs one wait state on this GPU generation (the compiler inserts the
// same s_nop before its own LDS DMA); inside inline assembly the compiler cannot, so the nop is
// written here.
__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds_block) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds_block), "v"(src)
               : "memory", "m0");
}
// The same with a wave-uniform 64-bit base (SGPRs) plus a per-lane 32-bit byte offset, so that
// per tile only the scalar base moves. NT marks the load non-temporal (streamed data that should
// not displace cached lines).
template <bool NT = false>
__device__ __forceinline__ void lds_dma16_sbase(const void* base, uint32_t offset,
                                                uint32_t lds_block) {
  // the compiler cannot always prove the base uniform; the asm needs it in SGPRs
  const uint64_t b = (uint64_t)(uintptr_t)base;
  // (readfirstlane returns a signed int: each half goes through uint32_t, not sign-extended)
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const uint64_t sb = (uint64_t)lo | ((uint64_t)hi << 32);
  base = (const void*)(uintptr_t)sb;
  lds_block = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_block);
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt"
                 :
                 : "s"(lds_block), "v"(offset), "s"(base)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(lds_block), "v"(offset), "s"(base)
                 : "memory", "m0");
}
// A wave-uniform pointer taken into scalar registers (readfirstlane of each half).
__device__ __forceinline__ const char* uniform_ptr(const char* ptr) {
  const uint64_t b = (uint64_t)(uintptr_t)ptr;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  return (const char*)(uintptr_t)((uint64_t)lo | ((uint64_t)hi << 32));
}
// s_waitcnt vmcnt(0) lgkmcnt(0): every outstanding global load (DMA included) and LDS access done.
__device__ __forceinline__ void vm_wait_all() { __builtin_amdgcn_s_waitcnt(0x0070); }
// LDS byte address of a shared-memory pointer.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// Workgroup and work-item indices read straight from the registers the hardware loads at
// launch. (blockIdx / threadIdx go through device-library functions that this toolchain leaves
// out of line: every kernel would start with calls into code far from its own, each a cold
// instruction fetch before the first load is issued.) Work-items: one-dimensional workgroups.
__device__ __forceinline__ int wg_id_x() { return (int)__builtin_amdgcn_workgroup_id_x(); }
__device__ __forceinline__ int wg_id_y() { return (int)__builtin_amdgcn_workgroup_id_y(); }
__device__ __forceinline__ int wg_id_z() { return (int)__builtin_amdgcn_workgroup_id_z(); }
__device__ __forceinline__ int item_id() { return (int)__builtin_amdgcn_workitem_id_x(); }

#ifdef FFAI_STAMPS
// ---------------------------------------------------------------------------------------------
// Phase timestamps, compiled only into the diagnostic library (FFAI_STAMPS,
// libffai_attn_stamps.so; the product library's code has none of this). Times come from the
// shader clock counter (s_memtime) and, for calibration, the 100 MHz real-time counter
// (s_memrealtime); both are scalar reads. Results are written from one lane with vector buffer
// stores.
// Layout of the fused kernel's record (16-bit path), per recording workgroup and wave, 32 u64:
//   [0..5] phase sums over the wave's tiles, in s_memtime ticks: B, settle 0, C, settle 1,
//          barrier (the wait for the tile's DMA and the workgroup), D (staging and the last
//          products); [6] tiles; [7] s_memtime and [8] s_memrealtime at the loop's start, [9]
//          and [10] at its end; [11] s_memrealtime at kernel entry, [12] after the wave's last
//          store was issued and [13] once its stores were acknowledged (zero for a split piece
//          that leaves the merge to another); [14] where the wave ran:
//          HW_ID (wave slot, SIMD, CU, shader array, engine) in the low 32 bits, the XCC in the
//          high; [15] s_memrealtime once the prologue's Q loads and first tile copies were
//          issued, [16] once they landed and [17] after the workgroup barrier that follows;
//          [18] before the Q loads are issued; [19..31] zero.
// The decode kernel's record, per recording workgroup (wave 0), 8 u64 of s_memtime: [0] entry,
// [1] first K/V load issued, [2] first tile landed, [3] tile loop done, [4] waves' partials
// merged in LDS, [5] end; [6] 1 if this workgroup wrote the output (unsplit, or the unit's last
// split), [7] s_memrealtime at entry.
__device__ __forceinline__ uint64_t stamp_clock() { return __builtin_amdgcn_s_memtime(); }
__device__ __forceinline__ uint64_t stamp_realtime() { return __builtin_amdgcn_s_memrealtime(); }
// HW_ID (hardware register 4) and XCC_ID (register 20), read whole: s_getreg's operand is
// register | offset << 6 | (bits - 1) << 11.
__device__ __forceinline__ uint64_t stamp_where() {
  const uint32_t hw = __builtin_amdgcn_s_getreg(4 | (31 << 11));
  const uint32_t xcc = __builtin_amdgcn_s_getreg(20 | (15 << 11));
  return ((uint64_t)xcc << 32) | hw;
}
__device__ __forceinline__ void stamp_put(uint64_t* base, int64_t index, uint64_t value) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(base, (short)0, 0x7fffffff, kBufferWord3);
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, value), r, (int)(index * 8), 0,
                                        0);
}
#endif

template <int DT>
__device__ __forceinline__ f32x16 mfma16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == kBF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// 16x16x32: A lane l holds row l%16, contraction elements 8(l/16) .. +7; B the same elements of
// column l%16; D lane l holds rows 4(l/16) .. +3 of column l%16.
template <int DT>
__device__ __forceinline__ f32x4 mfma16x16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == kBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}
// The same value from the four lanes l, l^16, l^32, l^48 (v_permlane16_swap, v_permlane32_swap):
// the max or the sum over all four.
__device__ __forceinline__ float quad_max(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return partner_max(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}
__device__ __forceinline__ float quad_sum(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return partner_sum(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}

// Max and sum over all 64 lanes, the result in every lane: within each row of 16 lanes by DPP
// (quad permutes, then rotations by 4 and 8 lanes), then over the four rows (quad_max / quad_sum).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xf, 0xf, false));
}
__device__ __forceinline__ float wave_max_all(float v) {
  v = fmaxf(v, dpp_mov<0xb1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_mov<0x4e>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_mov<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp_mov<0x128>(v));  // row_ror:8
  return quad_max(v);
}
__device__ __forceinline__ float wave_sum_all(float v) {
  v += dpp_mov<0xb1>(v);
  v += dpp_mov<0x4e>(v);
  v += dpp_mov<0x124>(v);
  v += dpp_mov<0x128>(v);
  return quad_sum(v);
}

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------------
// Loads. "vec" loads assume the launch's alignment check passed; "elem" loads take any address.
// Every helper reads only addresses of valid elements: callers clamp indices into range and
// zero what is out of range, so no branch (and no wait) splits a tile's loads.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x2 ld8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }

// 8 consecutive 16-bit elements, element-wise (any alignment).
__device__ __forceinline__ u32x4 ld8h_elem(const uint16_t* p) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 16);
  return u32x4{w[0], w[1], w[2], w[3]};
}

// Four elements widened to f32 from f32, f16 or bf16 storage.
template <int DT, bool VEC>
__device__ __forceinline__ f32x4 ld4f(const store_t<DT>* p) {
  if constexpr (DT == kF32) {
    if constexpr (VEC) return *reinterpret_cast<const f32x4*>(p);
    return f32x4{p[0], p[1], p[2], p[3]};
  } else {
    uint32_t w0, w1;
    if constexpr (VEC) {
      const u32x2 a = ld8(p);
      w0 = a.x;
      w1 = a.y;
    } else {
      w0 = (uint32_t)p[0] | ((uint32_t)p[1] << 16);
      w1 = (uint32_t)p[2] | ((uint32_t)p[3] << 16);
    }
    return f32x4{to_f32<DT>(w0 & 0xffffu), to_f32<DT>(w0 >> 16), to_f32<DT>(w1 & 0xffffu),
                 to_f32<DT>(w1 >> 16)};
  }
}

// Store four consecutive outputs.
template <int DT, bool VEC>
__device__ __forceinline__ void st4(store_t<DT>* p, f32x4 x) {
  if constexpr (DT == kF32) {
    if constexpr (VEC) {
      *reinterpret_cast<f32x4*>(p) = x;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) p[e] = x[e];
    }
  } else {
    const uint32_t a = pack2<DT>(x[0], x[1]), b = pack2<DT>(x[2], x[3]);
    if constexpr (VEC) {
      *reinterpret_cast<u32x2*>(p) = u32x2{a, b};
    } else {
      p[0] = (uint16_t)(a & 0xffffu);
      p[1] = (uint16_t)(a >> 16);
      p[2] = (uint16_t)(b & 0xffffu);
      p[3] = (uint16_t)(b >> 16);
    }
  }
}

}  // namespace
}  // namespace ffai
