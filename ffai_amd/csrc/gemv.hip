// The decoder's single-row projections (include/ffai_gemv.h): the f16-weight GEMV and the
// block-scaled int8 vocabulary projection, every beam's row in one pass over the weights.
//
// The int8 path reproduces the reference's arithmetic exactly: its integer dot products are
// exact (7-bit offset activations times 8-bit weights never saturate in the reference's i16
// pair sums, and v_dot4 accumulates in i32), and its float steps -- divisions, rounding half
// away from zero, the in-order sum over blocks of (block sum * scale), the correction and the
// final scale -- are done with explicitly rounded f32 operations, never fused.
#include "../../include/ffai_gemv.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "attn_common.cuh"

namespace ffai {
namespace {

// Sum over the wave's 64 lanes in VALU cross-lane moves (DPP), no LDS permutes: within each
// 16-lane row by quad permutes and row rotations, then rows 0-3 folded into lane 63 by the row
// broadcasts of lanes 15 and 31 (lanes without a source add 0); the total is read from lane 63.
__device__ __forceinline__ float dpp_add(float v, int x) { return v + __builtin_bit_cast(float, x); }
__device__ __forceinline__ float wave_sum(float v) {
  auto mv = [](float a, auto ctrl) {
    return __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a), decltype(ctrl)::value, 0xf,
                                       0xf, false);
  };
  v = dpp_add(v, mv(v, std::integral_constant<int, 0xb1>{}));   // quad_perm [1,0,3,2]
  v = dpp_add(v, mv(v, std::integral_constant<int, 0x4e>{}));   // quad_perm [2,3,0,1]
  v = dpp_add(v, mv(v, std::integral_constant<int, 0x124>{}));  // row_ror:4
  v = dpp_add(v, mv(v, std::integral_constant<int, 0x128>{}));  // row_ror:8
  v = dpp_add(v, mv(v, std::integral_constant<int, 0x142>{}));  // row_bcast:15
  v = dpp_add(v, mv(v, std::integral_constant<int, 0x143>{}));  // row_bcast:31
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// ---- f16 GEMV ---------------------------------------------------------------------------------
// A workgroup of 4 waves, one output row per wave: lane l takes the row's 16-byte weight chunks
// l, l + 64, ... (coalesced along the row, four in flight per lane), widens them to f32 and
// multiplies them with every beam's x, read straight from global memory (the few KB of x stay
// in L2; staging them in LDS behind a barrier put a second dependent round trip in front of the
// weight loads), then the wave reduces each beam's sum.
// Lane partial sums of output row `wr` with every beam's x (the wave sums them afterwards).
template <int R>
__device__ __forceinline__ void gemv_row(const uint16_t* __restrict__ wr, int in_dim,
                                         const float* __restrict__ x, int rows, int64_t xs,
                                         int lane, float (&acc)[R]) {
  const int chunks = in_dim / 8;
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  constexpr int kBatch = 4;  // weight chunks in flight per lane
  for (int c0 = lane; c0 < chunks; c0 += 64 * kBatch) {
    u32x4 wv[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int c = min(c0 + 64 * j, chunks - 1);
      wv[j] = ld16(wr + 8 * c);
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int c = c0 + 64 * j;
      if (c >= chunks) break;
      float wf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        wf[2 * e] = to_f32<kF16>(wv[j][e] & 0xffffu);
        wf[2 * e + 1] = to_f32<kF16>(wv[j][e] >> 16);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        // beams past `rows` repeat the last one's x (R is the compiled width); never stored
        const float* xr = x + min(r, rows - 1) * xs + 8 * c;
        const f32x4 a = *reinterpret_cast<const f32x4*>(xr);
        const f32x4 b = *reinterpret_cast<const f32x4*>(xr + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[r] = __builtin_fmaf(wf[e], a[e], acc[r]);
          acc[r] = __builtin_fmaf(wf[4 + e], b[e], acc[r]);
        }
      }
    }
  }
}

template <int R>
__global__ __launch_bounds__(256) void gemv_f16_kernel(const uint16_t* __restrict__ w,
                                                       int out_dim, int in_dim,
                                                       const float* __restrict__ x, int rows,
                                                       int64_t xs, float* __restrict__ y,
                                                       int64_t ys) {
  const int tid = item_id(), lane = tid & 63, wave = tid >> 6;
  const int o = wg_id_x() * 4 + wave;
  if (o >= out_dim) return;
  float acc[R];
  gemv_row<R>(w + (int64_t)o * in_dim, in_dim, x, rows, xs, lane, acc);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_sum(acc[r]);
    if (lane == r && r < rows) y[r * ys + o] = v;
  }
}

// The self-attention q/k/v projection of a decode step with the new K/V rows written straight
// into the layer's cache: weights packed (q; k; v), n = heads * head_dim outputs each. Output o
// of beam r is the GEMV sum plus bias[o] (a separate f32 add, as the reference adds the bias
// after the product); q goes to row r of `q`, k and v to position lens[r] - 1 of slot r, head
// o / head_dim, converted to the cache type by round-to-nearest-even. The step's length advance
// (ffai_kv_advance) runs before the layer, so lens[r] - 1 is the position it opened.
struct QkvCacheParams {
  const float* bias;  // 3n, or null
  float* q;
  int64_t qs;         // q row stride
  void* ck;
  void* cv;
  const int32_t* lens;
  int64_t cs, ch, cp;  // cache slot, head, position strides (elements)
  int32_t n, head_dim, capacity;
};

template <int R, int CDT>
__global__ __launch_bounds__(256) void gemv_f16_qkv_kernel(const uint16_t* __restrict__ w,
                                                           int in_dim,
                                                           const float* __restrict__ x, int rows,
                                                           int64_t xs, QkvCacheParams p) {
  const int tid = item_id(), lane = tid & 63, wave = tid >> 6;
  const int o = wg_id_x() * 4 + wave;
  if (o >= 3 * p.n) return;
  float acc[R];
  gemv_row<R>(w + (int64_t)o * in_dim, in_dim, x, rows, xs, lane, acc);
  const int part = o / p.n;  // 0: q, 1: k, 2: v
  const int oo = o - part * p.n;
  const int h = oo / p.head_dim, d = oo - h * p.head_dim;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float v = wave_sum(acc[r]);
    if (p.bias) v = v + p.bias[o];
    if (lane == r && r < rows) {
      if (part == 0) {
        p.q[r * p.qs + oo] = v;
      } else {
        // a length outside [1, capacity] is clamped; 0 (no advance) writes nothing
        const int pos = min(max(p.lens[r], 0), p.capacity) - 1;
        if (pos >= 0) {
          store_t<CDT>* c = reinterpret_cast<store_t<CDT>*>(part == 1 ? p.ck : p.cv) +
                            (int64_t)r * p.cs + (int64_t)h * p.ch + (int64_t)pos * p.cp + d;
          if constexpr (CDT == kF32) *c = v;
          else *c = from_f32<CDT>(v);
        }
      }
    }
  }
}

template <int R>
hipError_t launch_gemv_any(const uint16_t* w, int out_dim, int in_dim, const float* x, int rows,
                           int64_t xs, float* y, int64_t ys, hipStream_t st) {
  const unsigned grid = (unsigned)((out_dim + 3) / 4);
  hipLaunchKernelGGL((gemv_f16_kernel<R>), dim3(grid), dim3(256), 0, st, w, out_dim,
                     in_dim, x, rows, xs, y, ys);
  return hipGetLastError();
}

template <int R>
hipError_t launch_qkv_cache(const uint16_t* w, int in_dim, const float* x, int rows, int64_t xs,
                            const QkvCacheParams& p, int cdt, hipStream_t st) {
  const unsigned grid = (unsigned)((3 * p.n + 3) / 4);
  if (cdt == kF32)
    hipLaunchKernelGGL((gemv_f16_qkv_kernel<R, kF32>), dim3(grid), dim3(256), 0, st, w, in_dim, x,
                       rows, xs, p);
  else if (cdt == kF16)
    hipLaunchKernelGGL((gemv_f16_qkv_kernel<R, kF16>), dim3(grid), dim3(256), 0, st, w, in_dim, x,
                       rows, xs, p);
  else
    hipLaunchKernelGGL((gemv_f16_qkv_kernel<R, kBF16>), dim3(grid), dim3(256), 0, st, w, in_dim,
                       x, rows, xs, p);
  return hipGetLastError();
}

// ---- int8 vocabulary projection -------------------------------------------------------------
// round(), as Rust's f32::round: half away from zero (HIP's roundf)
__device__ __forceinline__ float round_away(float v) { return roundf(v); }

template <int DT>
__global__ __launch_bounds__(256) void vocab_quantize_kernel(const store_t<DT>* __restrict__ emb,
                                                             int vocab, int d, int blk,
                                                             int8_t* __restrict__ qw,
                                                             float* __restrict__ bscale,
                                                             float* __restrict__ corr) {
  // one thread per vocabulary row, blocks in order (the correction sums over them in order).
  // Every multiply and add rounds on its own, as in the reference: HIP contracts a * b + c into
  // one fused operation by default, so contraction is off here, and the operations are written
  // as operators in this scope (the contract setting follows the source location of each
  // operation; header helpers such as __fmul_rn keep the default).
#pragma clang fp contract(off)
  const int v = wg_id_x() * 256 + item_id();
  if (v >= vocab) return;
  const int nb = d / blk;
  const store_t<DT>* row = emb + (int64_t)v * d;
  float c = 0.f;
  for (int b = 0; b < nb; ++b) {
    float amax = 0.f;
    for (int k = 0; k < blk; ++k) {
      float wv;
      if constexpr (DT == kF32) wv = row[b * blk + k];
      else wv = to_f32<DT>(row[b * blk + k]);
      amax = fmaxf(amax, fabsf(wv));
    }
    const float sc = amax > 0.f ? __fdiv_rn(amax, 127.f) : 1.f;
    bscale[(int64_t)v * nb + b] = sc;
    int bsum = 0;
    for (int k = 0; k < blk; ++k) {
      float wv;
      if constexpr (DT == kF32) wv = row[b * blk + k];
      else wv = to_f32<DT>(row[b * blk + k]);
      const float qf = fminf(fmaxf(round_away(__fdiv_rn(wv, sc)), -127.f), 127.f);
      const int q = (int)qf;
      qw[(int64_t)v * d + b * blk + k] = (int8_t)q;
      bsum += q;
    }
    c = c + sc * (float)bsum;
  }
  corr[v] = 64.f * c;
}

// Per activation row: sx = amax / 63; x_u = round(x / sx) clamped to [-64, 63], plus 64 (0..127,
// held as int8 for v_dot4). Workspace: rows * d bytes of x_u (16-byte aligned rows), then sx.
__global__ __launch_bounds__(256) void vocab_act_quant_kernel(const float* __restrict__ x,
                                                              int64_t xs, int d, int d_pad,
                                                              int8_t* __restrict__ xu,
                                                              float* __restrict__ sx_out) {
#pragma clang fp contract(off)
  const int r = wg_id_x();
  const float* xr = x + r * xs;
  __shared__ float red[256];
  float m = 0.f;
  for (int k = item_id(); k < d; k += 256) m = fmaxf(m, fabsf(xr[k]));
  red[item_id()] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (item_id() < s) red[item_id()] = fmaxf(red[item_id()], red[item_id() + s]);
    __syncthreads();
  }
  const float amax = red[0];
  const float sx = amax > 0.f ? __fdiv_rn(amax, 63.f) : 1.f;
  for (int k = item_id(); k < d; k += 256) {
    const float qf = fminf(fmaxf(round_away(__fdiv_rn(xr[k], sx)), -64.f), 63.f);
    xu[(int64_t)r * d_pad + k] = (int8_t)((int)qf + 64);
  }
  if (item_id() == 0) sx_out[r] = sx;
}

// Workgroup: kVocabRowsPerWg vocabulary rows (4 per wave). Phase 1: lane l takes 16-byte chunks
// l, l + 64, ... of a row, four v_dot4 per chunk and beam, and adds the exact partial into its
// block's sum in LDS. Phase 2: one thread per (beam, row) runs the in-order float sum over blocks.
constexpr int kVocabRowsPerWg = 16;

__global__ __launch_bounds__(256) void vocab_logits_kernel(
    const int8_t* __restrict__ qw, const float* __restrict__ bscale,
    const float* __restrict__ corr, int vocab, int d, int blk, int rows,
    const int8_t* __restrict__ xu, int d_pad, const float* __restrict__ sx,
    float* __restrict__ logits, int64_t ls) {
#pragma clang fp contract(off)  // separately rounded multiply and add, as in the reference
  extern __shared__ int bs_lds[];  // [rows][kVocabRowsPerWg][nb]
  const int nb = d / blk;
  const int v0 = wg_id_x() * kVocabRowsPerWg;
  const int n_bs = rows * kVocabRowsPerWg * nb;
  for (int i = item_id(); i < n_bs; i += 256) bs_lds[i] = 0;
  __syncthreads();
  const int wave = item_id() >> 6, lane = item_id() & 63;
  const int chunks = d / 16;
  for (int j = 0; j < kVocabRowsPerWg / 4; ++j) {
    const int rl = wave * (kVocabRowsPerWg / 4) + j;  // row within the workgroup
    const int v = v0 + rl;
    if (v >= vocab) break;
    for (int c = lane; c < chunks; c += 64) {
      const u32x4 wv = *reinterpret_cast<const u32x4*>(qw + (int64_t)v * d + 16 * c);
      const int b = (16 * c) / blk;
      for (int r = 0; r < rows; ++r) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(xu + (int64_t)r * d_pad + 16 * c);
        int s = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) s = __builtin_amdgcn_sdot4((int)xv[e], (int)wv[e], s, false);
        atomicAdd(&bs_lds[(r * kVocabRowsPerWg + rl) * nb + b], s);
      }
    }
  }
  __syncthreads();
  for (int t = item_id(); t < rows * kVocabRowsPerWg; t += 256) {
    const int r = t / kVocabRowsPerWg, rl = t % kVocabRowsPerWg;
    const int v = v0 + rl;
    if (v >= vocab) continue;
    const int* bsr = bs_lds + (r * kVocabRowsPerWg + rl) * nb;
    const float* scr = bscale + (int64_t)v * nb;
    float acc = 0.f;
    for (int b = 0; b < nb; ++b) acc = acc + (float)bsr[b] * scr[b];
    logits[r * ls + v] = (acc - corr[v]) * sx[r];
  }
}

}  // namespace
}  // namespace ffai

using namespace ffai;

namespace {
constexpr int kMaxGemvRows = 16;
size_t pad16(size_t n) { return (n + 15) & ~size_t(15); }
size_t vocab_lds_bytes(int d, int blk, int rows) {
  return (size_t)rows * kVocabRowsPerWg * (d / blk) * sizeof(int);
}
constexpr size_t kVocabLdsMax = 48 * 1024;
}  // namespace

extern "C" {

int ffai_gemv_f16(const void* w, int32_t out_dim, int32_t in_dim, const float* x, int32_t rows,
                  int64_t x_row_stride, float* y, int64_t y_row_stride, void* stream) {
  api_clear_error();
  if (!w || !x || !y) return api_fail(FFAI_ERR_INVALID, "null pointer");
  if (out_dim < 1 || in_dim < 8 || in_dim % 8) return api_fail(FFAI_ERR_INVALID, "out_dim >= 1 and in_dim a multiple of 8");
  if (rows < 1 || rows > kMaxGemvRows) return api_fail(FFAI_ERR_INVALID, "rows must be in [1, 16]");
  if ((rows > 1 && (x_row_stride < in_dim || y_row_stride < out_dim)) || x_row_stride % 4)
    return api_fail(FFAI_ERR_INVALID, "bad row strides (x rows need 16-byte alignment)");
  if ((uintptr_t)w % 16 || (uintptr_t)x % 16 || (uintptr_t)y % 4)
    return api_fail(FFAI_ERR_INVALID, "w and x must be 16-byte aligned");
  if ((int64_t)out_dim * in_dim >= (int64_t(1) << 40)) return api_fail(FFAI_ERR_INVALID, "weights too large");
  const int rc = api_check_device();
  if (rc != FFAI_OK) return rc;
  const auto* wp = static_cast<const uint16_t*>(w);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (rows) {
    case 1: e = launch_gemv_any<1>(wp, out_dim, in_dim, x, rows, x_row_stride, y, y_row_stride, st); break;
    case 2: e = launch_gemv_any<2>(wp, out_dim, in_dim, x, rows, x_row_stride, y, y_row_stride, st); break;
    case 3: e = launch_gemv_any<3>(wp, out_dim, in_dim, x, rows, x_row_stride, y, y_row_stride, st); break;
    case 4: e = launch_gemv_any<4>(wp, out_dim, in_dim, x, rows, x_row_stride, y, y_row_stride, st); break;
    case 5: e = launch_gemv_any<5>(wp, out_dim, in_dim, x, rows, x_row_stride, y, y_row_stride, st); break;
    case 6: e = launch_gemv_any<6>(wp, out_dim, in_dim, x, rows, x_row_stride, y, y_row_stride, st); break;
    case 7: e = launch_gemv_any<7>(wp, out_dim, in_dim, x, rows, x_row_stride, y, y_row_stride, st); break;
    case 8: e = launch_gemv_any<8>(wp, out_dim, in_dim, x, rows, x_row_stride, y, y_row_stride, st); break;
    default: e = launch_gemv_any<16>(wp, out_dim, in_dim, x, rows, x_row_stride, y, y_row_stride, st); break;
  }
  if (e != hipSuccess) return api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
  return FFAI_OK;
}

int ffai_gemv_f16_qkv_cache(const void* w, const float* bias, int32_t in_dim, const float* x,
                            int32_t rows, int64_t x_row_stride, float* q, int64_t q_row_stride,
                            const ffai_kv_cache* c, void* stream) {
  api_clear_error();
  if (!w || !x || !q || !c || !c->k || !c->v || !c->lens) return api_fail(FFAI_ERR_INVALID, "null pointer");
  if (c->dtype != FFAI_F32 && c->dtype != FFAI_F16 && c->dtype != FFAI_BF16)
    return api_fail(FFAI_ERR_INVALID, "unknown cache dtype");
  if (c->slots < 1 || c->heads < 1 || c->capacity < 1 || c->head_dim < 8 || c->head_dim % 8)
    return api_fail(FFAI_ERR_INVALID, "slots, heads, capacity >= 1 and head_dim a multiple of 8");
  if (c->strides[0] < 0 || c->strides[1] < 0 || c->strides[2] < c->head_dim)
    return api_fail(FFAI_ERR_INVALID, "bad cache strides");
  if (in_dim < 8 || in_dim % 8) return api_fail(FFAI_ERR_INVALID, "in_dim must be a multiple of 8");
  if (rows < 1 || rows > kMaxGemvRows || rows > c->slots)
    return api_fail(FFAI_ERR_INVALID, "rows must be in [1, 16] and at most the cache's slots");
  const int64_t n = (int64_t)c->heads * c->head_dim;
  if (3 * n >= (int64_t(1) << 31) || 3 * n * in_dim >= (int64_t(1) << 40))
    return api_fail(FFAI_ERR_INVALID, "weights too large");
  if ((rows > 1 && (x_row_stride < in_dim || q_row_stride < n)) || x_row_stride % 4)
    return api_fail(FFAI_ERR_INVALID, "bad row strides (x rows need 16-byte alignment)");
  const size_t es = c->dtype == FFAI_F32 ? 4 : 2;
  if ((uintptr_t)w % 16 || (uintptr_t)x % 16 || (uintptr_t)q % 4 || (uintptr_t)bias % 4 ||
      (uintptr_t)c->k % es || (uintptr_t)c->v % es)
    return api_fail(FFAI_ERR_INVALID, "w and x must be 16-byte aligned, q, bias and the cache "
                                      "aligned to their elements");
  const int rc = api_check_device();
  if (rc != FFAI_OK) return rc;
  QkvCacheParams p{};
  p.bias = bias; p.q = q; p.qs = q_row_stride;
  p.ck = c->k; p.cv = c->v; p.lens = c->lens;
  p.cs = c->strides[0]; p.ch = c->strides[1]; p.cp = c->strides[2];
  p.n = (int32_t)n; p.head_dim = c->head_dim; p.capacity = c->capacity;
  const auto* wp = static_cast<const uint16_t*>(w);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int cdt = c->dtype;  // FFAI_F32 / F16 / BF16 are kF32 / kF16 / kBF16
  hipError_t e;
  switch (rows) {
    case 1: e = launch_qkv_cache<1>(wp, in_dim, x, rows, x_row_stride, p, cdt, st); break;
    case 2: e = launch_qkv_cache<2>(wp, in_dim, x, rows, x_row_stride, p, cdt, st); break;
    case 3: e = launch_qkv_cache<3>(wp, in_dim, x, rows, x_row_stride, p, cdt, st); break;
    case 4: e = launch_qkv_cache<4>(wp, in_dim, x, rows, x_row_stride, p, cdt, st); break;
    case 5: e = launch_qkv_cache<5>(wp, in_dim, x, rows, x_row_stride, p, cdt, st); break;
    case 6: e = launch_qkv_cache<6>(wp, in_dim, x, rows, x_row_stride, p, cdt, st); break;
    case 7: e = launch_qkv_cache<7>(wp, in_dim, x, rows, x_row_stride, p, cdt, st); break;
    case 8: e = launch_qkv_cache<8>(wp, in_dim, x, rows, x_row_stride, p, cdt, st); break;
    default: e = launch_qkv_cache<16>(wp, in_dim, x, rows, x_row_stride, p, cdt, st); break;
  }
  if (e != hipSuccess) return api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
  return FFAI_OK;
}

int ffai_vocab_int8_quantize(const void* emb, int32_t emb_dtype, int32_t vocab, int32_t d,
                             int32_t blk, int8_t* qw, float* bscale, float* corr, void* stream) {
  api_clear_error();
  if (!emb || !qw || !bscale || !corr) return api_fail(FFAI_ERR_INVALID, "null pointer");
  if (vocab < 1 || d < 32 || blk < 32 || blk % 32 || d % blk)
    return api_fail(FFAI_ERR_INVALID, "vocab >= 1, blk a multiple of 32 dividing d");
  const int dt = emb_dtype == FFAI_F32 ? kF32 : emb_dtype == FFAI_F16 ? kF16 : emb_dtype == FFAI_BF16 ? kBF16 : -1;
  if (dt < 0) return api_fail(FFAI_ERR_INVALID, "unknown dtype");
  const int rc = api_check_device();
  if (rc != FFAI_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((vocab + 255) / 256));
  if (dt == kF32)
    hipLaunchKernelGGL((vocab_quantize_kernel<kF32>), grid, dim3(256), 0, st,
                       static_cast<const float*>(emb), vocab, d, blk, qw, bscale, corr);
  else if (dt == kF16)
    hipLaunchKernelGGL((vocab_quantize_kernel<kF16>), grid, dim3(256), 0, st,
                       static_cast<const uint16_t*>(emb), vocab, d, blk, qw, bscale, corr);
  else
    hipLaunchKernelGGL((vocab_quantize_kernel<kBF16>), grid, dim3(256), 0, st,
                       static_cast<const uint16_t*>(emb), vocab, d, blk, qw, bscale, corr);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
  return FFAI_OK;
}

int ffai_vocab_int8_workspace_bytes(int32_t d, int32_t rows, size_t* bytes) {
  api_clear_error();
  if (!bytes) return api_fail(FFAI_ERR_INVALID, "null bytes pointer");
  if (d < 1 || rows < 1) return api_fail(FFAI_ERR_INVALID, "d and rows must be positive");
  *bytes = (size_t)rows * pad16(d) + pad16((size_t)rows * sizeof(float));
  return FFAI_OK;
}

int ffai_vocab_int8_logits(const int8_t* qw, const float* bscale, const float* corr,
                           int32_t vocab, int32_t d, int32_t blk, const float* x, int32_t rows,
                           int64_t x_row_stride, float* logits, int64_t logits_row_stride,
                           void* workspace, size_t workspace_bytes, void* stream) {
  api_clear_error();
  if (!qw || !bscale || !corr || !x || !logits || !workspace)
    return api_fail(FFAI_ERR_INVALID, "null pointer");
  if (vocab < 1 || d < 32 || blk < 32 || blk % 32 || d % blk)
    return api_fail(FFAI_ERR_INVALID, "vocab >= 1, blk a multiple of 32 dividing d");
  if (rows < 1 || rows > kMaxGemvRows) return api_fail(FFAI_ERR_INVALID, "rows must be in [1, 16]");
  if ((rows > 1 && (x_row_stride < d || logits_row_stride < vocab)))
    return api_fail(FFAI_ERR_INVALID, "bad row strides");
  if ((uintptr_t)qw % 16 || (uintptr_t)workspace % 16)
    return api_fail(FFAI_ERR_INVALID, "qw and workspace must be 16-byte aligned");
  if (vocab_lds_bytes(d, blk, rows) > kVocabLdsMax)
    return api_fail(FFAI_ERR_INVALID, "rows * (d / blk) too large for one workgroup's block sums");
  size_t need = 0;
  ffai_vocab_int8_workspace_bytes(d, rows, &need);
  if (workspace_bytes < need) return api_fail(FFAI_ERR_WORKSPACE, "workspace smaller than ffai_vocab_int8_workspace_bytes");
  const int rc = api_check_device();
  if (rc != FFAI_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int d_pad = (int)pad16(d);
  int8_t* xu = static_cast<int8_t*>(workspace);
  float* sx = reinterpret_cast<float*>(static_cast<char*>(workspace) + (size_t)rows * d_pad);
  hipLaunchKernelGGL(vocab_act_quant_kernel, dim3(rows), dim3(256), 0, st, x, x_row_stride, d, d_pad,
                     xu, sx);
  const dim3 grid((unsigned)((vocab + kVocabRowsPerWg - 1) / kVocabRowsPerWg));
  hipLaunchKernelGGL(vocab_logits_kernel, grid, dim3(256), vocab_lds_bytes(d, blk, rows), st, qw,
                     bscale, corr, vocab, d, blk, rows, xu, d_pad, sx, logits, logits_row_stride);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
  return FFAI_OK;
}

}  // extern "C"
