// Device-resident decode-step state (include/ffai_kv.h): appending a step's K/V projections to
// head-major caches in place, gathering caches by parent beam, and building the
// cross-attention cache. All three are HBM-bound copies with a layout change and a dtype
// conversion; each thread moves 8 elements (16 bytes at 16-bit) per access.
#include "../../include/ffai_kv.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <initializer_list>
#include <type_traits>

#include "attn_common.cuh"

namespace ffai {
namespace {

// ---- 8-element loads and stores with conversion through f32 --------------------------------
template <int DT>
__device__ __forceinline__ void load8(const store_t<DT>* p, bool vec, float (&x)[8]) {
  if constexpr (DT == kF32) {
    if (vec) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = a[i], x[4 + i] = b[i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = p[i];
    }
  } else {
    uint32_t w[4];
    if (vec) {
      const u32x4 a = ld16(p);
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = a[i];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 16);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = to_f32<DT>(w[i] & 0xffffu);
      x[2 * i + 1] = to_f32<DT>(w[i] >> 16);
    }
  }
}

template <int DT>
__device__ __forceinline__ void store8(store_t<DT>* p, bool vec, const float (&x)[8]) {
  if constexpr (DT == kF32) {
    if (vec) {
      *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
      *reinterpret_cast<f32x4*>(p + 4) = f32x4{x[4], x[5], x[6], x[7]};
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) p[i] = x[i];
    }
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack2<DT>(x[2 * i], x[2 * i + 1]);
    if (vec) {
      *reinterpret_cast<u32x4*>(p) = u32x4{w[0], w[1], w[2], w[3]};
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[2 * i] = (uint16_t)(w[i] & 0xffffu);
        p[2 * i + 1] = (uint16_t)(w[i] >> 16);
      }
    }
  }
}

struct AppendParams {
  const void* src_k;
  const void* src_v;
  void* k;
  void* v;
  int32_t* lens;
  int64_t src_ss, src_rs;      // source slot and row strides
  int64_t ks, kh, kp;          // cache slot, head, position strides
  int32_t heads, head_dim, capacity, t_new;
  int32_t src_vec, dst_vec;    // 8-element vector accesses are aligned
  int32_t units_per_block;     // 8-element units of one slot's rows per workgroup
  int32_t advance;             // this launch also advances lens (one workgroup per slot)
};

// Workgroup (slot, blockIdx.y) moves units [y * units_per_block, ...) of the slot's t_new rows
// to positions lens[slot] + t. With one workgroup per slot (`advance`) every thread reads
// lens[slot] before the barrier and thread 0 advances it after, so the position each row lands
// on is fixed for the whole call; with several, kv_advance_kernel advances lens afterwards (the
// workgroups of one slot cannot order their reads of lens before its update).
template <int SRC, int DST>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendParams p) {
  const int s = wg_id_x();
  // a length outside [0, capacity] (corrupt or uninitialised) is clamped, as the gather does, so
  // no row lands before the slot's cache or past it
  const int len0 = min(max(p.lens[s], 0), p.capacity);
  const int row_units = p.heads * p.head_dim / 8;
  const int units = p.t_new * row_units;
  const int u_begin = wg_id_y() * p.units_per_block;
  const int u_end = min(units, u_begin + p.units_per_block);
  const auto* sk = reinterpret_cast<const store_t<SRC>*>(p.src_k) + (int64_t)s * p.src_ss;
  const auto* sv = reinterpret_cast<const store_t<SRC>*>(p.src_v) + (int64_t)s * p.src_ss;
  auto* dk = reinterpret_cast<store_t<DST>*>(p.k) + (int64_t)s * p.ks;
  auto* dv = reinterpret_cast<store_t<DST>*>(p.v) + (int64_t)s * p.ks;
  for (int u = u_begin + item_id(); u < u_end; u += 256) {
    const int t = u / row_units;
    const int col = (u - t * row_units) * 8;  // h * head_dim + d
    const int h = col / p.head_dim, d = col - h * p.head_dim;
    const int pos = len0 + t;
    if (pos >= p.capacity) continue;
    const int64_t so = (int64_t)t * p.src_rs + col;
    const int64_t doff = (int64_t)h * p.kh + (int64_t)pos * p.kp + d;
    float x[8];
    load8<SRC>(sk + so, p.src_vec, x);
    store8<DST>(dk + doff, p.dst_vec, x);
    load8<SRC>(sv + so, p.src_vec, x);
    store8<DST>(dv + doff, p.dst_vec, x);
  }
  if (p.advance) {
    __syncthreads();
    if (item_id() == 0) p.lens[s] = min(p.capacity, len0 + p.t_new);
  }
}

__global__ __launch_bounds__(256) void kv_advance_kernel(int32_t* lens, int slots, int capacity,
                                                         int t_new) {
  const int s = wg_id_x() * 256 + item_id();
  if (s < slots) lens[s] = min(capacity, min(max(lens[s], 0), capacity) + t_new);
}

// The same for every layer of a layer-stacked cache (blockIdx.y: the layer).
__global__ __launch_bounds__(256) void kv_advance_layers_kernel(int32_t* lens, int slots,
                                                                int64_t layer_stride,
                                                                int capacity, int t_new) {
  const int s = wg_id_x() * 256 + item_id();
  int32_t* l = lens + (int64_t)wg_id_y() * layer_stride;
  if (s < slots) l[s] = min(capacity, min(max(l[s], 0), capacity) + t_new);
}

struct GatherParams {
  char* dk;
  char* dv;
  int32_t* dlens;
  const char* sk;
  const char* sv;
  const int32_t* slens;
  const int32_t* parent;
  int64_t ds, dh, dp;  // destination slot, head, position strides (bytes)
  int64_t ss, sh, sp;  // source strides (bytes)
  int64_t layer_stride, lens_layer_stride;  // bytes between layers' k/v; ints between lens
  int32_t src_slots, heads, capacity, n_blk;
  int32_t row_units;   // units per key row (16 bytes each when vec, else one element)
  int32_t vec;
};

// Workgroup (layer blockIdx.y; slot i, head h, 64-position block): copies the block if it holds
// any of the parent's keys. The caches have one dtype, so rows move as raw bytes: 16-byte units
// when every row start is 16-byte aligned, else one element (ES bytes) at a time. Each thread
// issues all its loads before its stores. Parent indices and lengths are clamped into range, so
// no access leaves either cache.
template <int ES>
__global__ __launch_bounds__(256) void kv_gather_kernel(GatherParams p) {
  using elem_t = std::conditional_t<ES == 4, uint32_t, uint16_t>;
  constexpr int kPer = 4;  // units per thread per pass, for K and for V
  const int blk = wg_id_x() % p.n_blk;
  const int h = (wg_id_x() / p.n_blk) % p.heads;
  const int i = wg_id_x() / (p.n_blk * p.heads);
  const int64_t lo = (int64_t)wg_id_y() * p.layer_stride;
  const int32_t* slens = p.slens + (int64_t)wg_id_y() * p.lens_layer_stride;
  const int par = min(max(p.parent[i], 0), p.src_slots - 1);
  const int len = min(max(slens[par], 0), p.capacity);
  if (blk == 0 && h == 0 && item_id() == 0)
    p.dlens[(int64_t)wg_id_y() * p.lens_layer_stride + i] = len;
  const int pos0 = blk * 64;
  if (pos0 >= len) return;
  const int n = min(64, len - pos0) * p.row_units;
  const char* sk = p.sk + lo + (int64_t)par * p.ss + (int64_t)h * p.sh + (int64_t)pos0 * p.sp;
  const char* sv = p.sv + lo + (int64_t)par * p.ss + (int64_t)h * p.sh + (int64_t)pos0 * p.sp;
  char* dk = p.dk + lo + (int64_t)i * p.ds + (int64_t)h * p.dh + (int64_t)pos0 * p.dp;
  char* dv = p.dv + lo + (int64_t)i * p.ds + (int64_t)h * p.dh + (int64_t)pos0 * p.dp;
  const int ub = p.vec ? 16 : ES;  // bytes per unit
  for (int base = item_id(); base < n; base += 256 * kPer) {
    if (p.vec) {
      u32x4 a[kPer], b[kPer];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int u = base + j * 256;
        if (u < n) {
          const int r = u / p.row_units, c = (u - r * p.row_units) * ub;
          a[j] = *reinterpret_cast<const u32x4*>(sk + r * p.sp + c);
          b[j] = *reinterpret_cast<const u32x4*>(sv + r * p.sp + c);
        }
      }
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int u = base + j * 256;
        if (u < n) {
          const int r = u / p.row_units, c = (u - r * p.row_units) * ub;
          *reinterpret_cast<u32x4*>(dk + r * p.dp + c) = a[j];
          *reinterpret_cast<u32x4*>(dv + r * p.dp + c) = b[j];
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int u = base + j * 256;
        if (u < n) {
          const int r = u / p.row_units, c = (u - r * p.row_units) * ub;
          *reinterpret_cast<elem_t*>(dk + r * p.dp + c) = *reinterpret_cast<const elem_t*>(sk + r * p.sp + c);
          *reinterpret_cast<elem_t*>(dv + r * p.dp + c) = *reinterpret_cast<const elem_t*>(sv + r * p.sp + c);
        }
      }
    }
  }
}

struct CrossParams {
  const void* sk;
  const void* sv;
  void* k;
  void* v;
  int64_t src_rs;
  int32_t t, heads, head_dim, n_tblk;
  int32_t src_vec;
};

// V (and K in rows layout): output row (h, t) = input row t, columns h*D .. h*D + D - 1.
template <int SRC, int DST>
__global__ __launch_bounds__(256) void cross_rows_kernel(const void* src, void* dst, CrossParams p) {
  const int row_units = p.heads * p.head_dim / 8;
  const int64_t units = (int64_t)p.t * row_units;
  const auto* s = reinterpret_cast<const store_t<SRC>*>(src);
  auto* o = reinterpret_cast<store_t<DST>*>(dst);
  for (int64_t u = (int64_t)wg_id_x() * 256 + item_id(); u < units; u += (int64_t)gridDim.x * 256) {
    const int t = (int)(u / row_units);
    const int col = (int)(u - (int64_t)t * row_units) * 8;
    const int h = col / p.head_dim, d = col - h * p.head_dim;
    float x[8];
    load8<SRC>(s + (int64_t)t * p.src_rs + col, p.src_vec, x);
    store8<DST>(o + ((int64_t)h * p.t + t) * p.head_dim + d, true, x);
  }
}

// K^T: output (h, d, t). Workgroup (head h, 64-frame block): the block's 64 x head_dim values go
// through LDS so that both the reads (along d) and the writes (along t) are contiguous.
template <int SRC, int DST>
__global__ __launch_bounds__(256) void cross_kt_kernel(CrossParams p) {
  __shared__ float tile[64][128 + 1];
  const int tb = wg_id_x() % p.n_tblk, h = wg_id_x() / p.n_tblk;
  const int t0 = tb * 64;
  const int rows = min(64, p.t - t0);
  const int du = p.head_dim / 8;
  const auto* s = reinterpret_cast<const store_t<SRC>*>(p.sk);
  for (int u = item_id(); u < rows * du; u += 256) {
    const int r = u / du, d = (u - r * du) * 8;
    float x[8];
    load8<SRC>(s + (int64_t)(t0 + r) * p.src_rs + h * p.head_dim + d, p.src_vec, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[r][d + e] = x[e];
  }
  __syncthreads();
  auto* o = reinterpret_cast<store_t<DST>*>(p.k) + (int64_t)h * p.head_dim * p.t;
  // one output element per thread and step: row d, frame t0 + c
  for (int u = item_id(); u < p.head_dim * 64; u += 256) {
    const int d = u / 64, c = u % 64;
    if (c >= rows) continue;
    const float x = tile[c][d];
    if constexpr (DST == kF32) o[(int64_t)d * p.t + t0 + c] = x;
    else o[(int64_t)d * p.t + t0 + c] = from_f32<DST>(x);
  }
}

int dt_of(int32_t d) {
  return d == FFAI_F32 ? kF32 : d == FFAI_F16 ? kF16 : d == FFAI_BF16 ? kBF16 : -1;
}
size_t esize(int dt) { return dt == kF32 ? 4 : 2; }

// Dispatch a kernel template over (SRC, DST) dtypes.
template <template <int, int> class K, class... A>
hipError_t dispatch2(int src, int dst, A&&... a) {
#define FFAI_D2(S, D) \
  if (src == S && dst == D) return K<S, D>::run(a...);
  FFAI_D2(kF32, kF32) FFAI_D2(kF32, kF16) FFAI_D2(kF32, kBF16)
  FFAI_D2(kF16, kF32) FFAI_D2(kF16, kF16) FFAI_D2(kF16, kBF16)
  FFAI_D2(kBF16, kF32) FFAI_D2(kBF16, kF16) FFAI_D2(kBF16, kBF16)
#undef FFAI_D2
  return hipErrorInvalidValue;
}

template <int S, int D>
struct AppendLaunch {
  // Up to kOneBlockUnits 8-element units a slot (a decode step's row, a few rows) go to one
  // workgroup, which advances lens in the same launch. More (a prompt's hundreds of rows) go one
  // unit per thread, 256 a workgroup, so that the copy is spread over the CUs; a second,
  // one-thread-per-slot launch then advances lens. A 228-row whisper-medium prompt (29184 units)
  // took 9.7 us a layer in 8 workgroups of 4096 units: each CU moved ~390 KB.
  static constexpr int kOneBlockUnits = 1024;
  static hipError_t run(AppendParams p, int slots, hipStream_t st) {
    const int64_t units = (int64_t)p.t_new * p.heads * p.head_dim / 8;
    const int64_t nblk =
        units <= kOneBlockUnits ? 1 : std::min<int64_t>((units + 255) / 256, 65535);
    p.units_per_block = (int)((units + nblk - 1) / nblk);
    p.advance = nblk == 1;
    hipLaunchKernelGGL((kv_append_kernel<S, D>), dim3(slots, (unsigned)nblk), dim3(256), 0, st, p);
    if (nblk > 1)
      hipLaunchKernelGGL(kv_advance_kernel, dim3((slots + 255) / 256), dim3(256), 0, st, p.lens,
                         slots, p.capacity, p.t_new);
    return hipGetLastError();
  }
};
template <int S, int D>
struct CrossLaunch {
  static hipError_t run(const CrossParams& p, bool kt, hipStream_t st) {
    const int64_t units = (int64_t)p.t * p.heads * p.head_dim / 8;
    const unsigned grid = (unsigned)std::min<int64_t>((units + 255) / 256, 4096);
    hipLaunchKernelGGL((cross_rows_kernel<S, D>), dim3(grid), dim3(256), 0, st, p.sv, p.v, p);
    if (kt) {
      hipLaunchKernelGGL((cross_kt_kernel<S, D>), dim3((unsigned)(p.heads * p.n_tblk)), dim3(256), 0,
                         st, p);
    } else {
      hipLaunchKernelGGL((cross_rows_kernel<S, D>), dim3(grid), dim3(256), 0, st, p.sk, p.k, p);
    }
    return hipGetLastError();
  }
};

bool aligned8(const void* base, size_t es, std::initializer_list<int64_t> strides) {
  if ((uintptr_t)base % (8 * es)) return false;
  for (int64_t s : strides)
    if (s % 8) return false;
  return true;
}

int check_cache(const ffai_kv_cache* c) {
  if (!c || !c->k || !c->v || !c->lens) return api_fail(FFAI_ERR_INVALID, "null cache pointer");
  if (dt_of(c->dtype) < 0) return api_fail(FFAI_ERR_INVALID, "unknown cache dtype");
  if (c->slots < 1 || c->heads < 1 || c->capacity < 1 || c->head_dim < 8 || c->head_dim % 8)
    return api_fail(FFAI_ERR_INVALID, "slots, heads, capacity >= 1 and head_dim a multiple of 8");
  if (c->strides[0] < 0 || c->strides[1] < 0 || c->strides[2] < c->head_dim)
    return api_fail(FFAI_ERR_INVALID, "bad cache strides");
  const size_t es = esize(dt_of(c->dtype));
  if ((uintptr_t)c->k % es || (uintptr_t)c->v % es)
    return api_fail(FFAI_ERR_INVALID, "cache pointer not aligned to its element size");
  return FFAI_OK;
}

}  // namespace
}  // namespace ffai

using namespace ffai;

extern "C" {

int ffai_kv_append(const ffai_kv_cache* c, const void* new_k, const void* new_v, int32_t src_dtype,
                   int32_t t_new, int64_t src_slot_stride, int64_t src_row_stride, void* stream) {
  api_clear_error();
  int rc = check_cache(c);
  if (rc != FFAI_OK) return rc;
  const int sdt = dt_of(src_dtype);
  if (sdt < 0) return api_fail(FFAI_ERR_INVALID, "unknown source dtype");
  if (!new_k || !new_v) return api_fail(FFAI_ERR_INVALID, "null source pointer");
  if (t_new < 0) return api_fail(FFAI_ERR_INVALID, "t_new must be >= 0");
  if ((int64_t)t_new * c->heads * c->head_dim / 8 >= (int64_t(1) << 31))
    return api_fail(FFAI_ERR_INVALID, "t_new * heads * head_dim too large");
  if (src_row_stride < (int64_t)c->heads * c->head_dim || src_slot_stride < 0)
    return api_fail(FFAI_ERR_INVALID, "bad source strides");
  if ((uintptr_t)new_k % esize(sdt) || (uintptr_t)new_v % esize(sdt))
    return api_fail(FFAI_ERR_INVALID, "source pointer not aligned to its element size");
  if (t_new == 0) return FFAI_OK;
  rc = api_check_device();
  if (rc != FFAI_OK) return rc;
  AppendParams p{};
  p.src_k = new_k; p.src_v = new_v; p.k = c->k; p.v = c->v; p.lens = c->lens;
  p.src_ss = src_slot_stride; p.src_rs = src_row_stride;
  p.ks = c->strides[0]; p.kh = c->strides[1]; p.kp = c->strides[2];
  p.heads = c->heads; p.head_dim = c->head_dim; p.capacity = c->capacity; p.t_new = t_new;
  p.src_vec = aligned8(new_k, esize(sdt), {src_slot_stride, src_row_stride}) &&
              aligned8(new_v, esize(sdt), {0});
  p.dst_vec = aligned8(c->k, esize(dt_of(c->dtype)), {c->strides[0], c->strides[1], c->strides[2]}) &&
              aligned8(c->v, esize(dt_of(c->dtype)), {0});
  const hipError_t e = dispatch2<AppendLaunch>(sdt, dt_of(c->dtype), p, c->slots,
                                               static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
  return FFAI_OK;
}

int ffai_kv_advance(const ffai_kv_cache* c, int32_t t_new, int32_t layers,
                    int64_t lens_layer_stride, void* stream) {
  api_clear_error();
  int rc = check_cache(c);
  if (rc != FFAI_OK) return rc;
  if (t_new < 0) return api_fail(FFAI_ERR_INVALID, "t_new must be >= 0");
  if (layers < 1 || layers > 65535) return api_fail(FFAI_ERR_INVALID, "layers must be in [1, 65535]");
  if (layers > 1 && lens_layer_stride < c->slots)
    return api_fail(FFAI_ERR_INVALID, "lens_layer_stride must separate the layers");
  if (layers == 1) lens_layer_stride = 0;
  if (t_new == 0) return FFAI_OK;
  rc = api_check_device();
  if (rc != FFAI_OK) return rc;
  hipLaunchKernelGGL(kv_advance_layers_kernel, dim3((unsigned)((c->slots + 255) / 256), (unsigned)layers),
                     dim3(256), 0, static_cast<hipStream_t>(stream), c->lens, c->slots,
                     lens_layer_stride, c->capacity, t_new);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
  return FFAI_OK;
}

int ffai_kv_gather(const ffai_kv_cache* dst, const ffai_kv_cache* src, const int32_t* parent,
                   int32_t layers, int64_t layer_stride, int64_t lens_layer_stride, void* stream) {
  api_clear_error();
  int rc = check_cache(dst);
  if (rc != FFAI_OK) return rc;
  rc = check_cache(src);
  if (rc != FFAI_OK) return rc;
  if (!parent) return api_fail(FFAI_ERR_INVALID, "null parent pointer");
  if (dst->dtype != src->dtype || dst->heads != src->heads || dst->head_dim != src->head_dim ||
      dst->capacity != src->capacity)
    return api_fail(FFAI_ERR_INVALID, "dst and src differ in dtype, heads, head_dim or capacity");
  if (dst->k == src->k || dst->v == src->v || dst->lens == src->lens)
    return api_fail(FFAI_ERR_INVALID, "dst and src must be distinct caches");
  if (layers < 1 || layers > 65535) return api_fail(FFAI_ERR_INVALID, "layers must be in [1, 65535]");
  if (layers > 1 && (layer_stride <= 0 || lens_layer_stride < dst->slots || lens_layer_stride < src->slots))
    return api_fail(FFAI_ERR_INVALID, "layer strides must separate the layers");
  if (layers == 1) layer_stride = lens_layer_stride = 0;
  rc = api_check_device();
  if (rc != FFAI_OK) return rc;
  const int64_t es = (int64_t)esize(dt_of(dst->dtype));
  GatherParams p{};
  p.dk = static_cast<char*>(dst->k); p.dv = static_cast<char*>(dst->v); p.dlens = dst->lens;
  p.sk = static_cast<const char*>(src->k); p.sv = static_cast<const char*>(src->v);
  p.slens = src->lens; p.parent = parent;
  p.ds = dst->strides[0] * es; p.dh = dst->strides[1] * es; p.dp = dst->strides[2] * es;
  p.ss = src->strides[0] * es; p.sh = src->strides[1] * es; p.sp = src->strides[2] * es;
  p.layer_stride = layer_stride * es; p.lens_layer_stride = lens_layer_stride;
  p.src_slots = src->slots; p.heads = dst->heads;
  p.capacity = dst->capacity; p.n_blk = (dst->capacity + 63) / 64;
  p.vec = aligned8(dst->k, es, {dst->strides[0], dst->strides[1], dst->strides[2], layer_stride}) &&
          aligned8(dst->v, es, {0}) && aligned8(src->k, es, {src->strides[0], src->strides[1], src->strides[2]}) &&
          aligned8(src->v, es, {0}) && (dst->head_dim * es) % 16 == 0;
  p.row_units = p.vec ? (int32_t)(dst->head_dim * es / 16) : dst->head_dim;
  const dim3 grid((unsigned)((int64_t)dst->slots * dst->heads * p.n_blk), (unsigned)layers);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (es == 4) hipLaunchKernelGGL((kv_gather_kernel<4>), grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL((kv_gather_kernel<2>), grid, dim3(256), 0, st, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
  return FFAI_OK;
}

int ffai_cross_kv_build(const void* k_proj, const void* v_proj, int32_t src_dtype, int32_t t,
                        int32_t heads, int32_t head_dim, int64_t src_row_stride, void* k_out,
                        void* v_out, int32_t out_dtype, int32_t k_layout, void* stream) {
  api_clear_error();
  const int sdt = dt_of(src_dtype), odt = dt_of(out_dtype);
  if (sdt < 0 || odt < 0) return api_fail(FFAI_ERR_INVALID, "unknown dtype");
  if (!k_proj || !v_proj || !k_out || !v_out) return api_fail(FFAI_ERR_INVALID, "null pointer");
  if (t < 1 || heads < 1 || head_dim < 8 || head_dim % 8 || head_dim > 128)
    return api_fail(FFAI_ERR_INVALID, "t, heads >= 1 and head_dim a multiple of 8 up to 128");
  if (src_row_stride < (int64_t)heads * head_dim)
    return api_fail(FFAI_ERR_INVALID, "source row stride shorter than heads * head_dim");
  if (k_layout != FFAI_K_TRANSPOSED && k_layout != FFAI_K_ROWS)
    return api_fail(FFAI_ERR_INVALID, "unknown k_layout");
  if ((uintptr_t)k_proj % esize(sdt) || (uintptr_t)v_proj % esize(sdt) ||
      (uintptr_t)k_out % (8 * esize(odt)) || (uintptr_t)v_out % (8 * esize(odt)))
    return api_fail(FFAI_ERR_INVALID, "sources aligned to their element size, outputs to 8 elements");
  const int rc = api_check_device();
  if (rc != FFAI_OK) return rc;
  CrossParams p{};
  p.sk = k_proj; p.sv = v_proj; p.k = k_out; p.v = v_out;
  p.src_rs = src_row_stride; p.t = t; p.heads = heads; p.head_dim = head_dim;
  p.n_tblk = (t + 63) / 64;
  p.src_vec = aligned8(k_proj, esize(sdt), {src_row_stride}) && aligned8(v_proj, esize(sdt), {0});
  const hipError_t e = dispatch2<CrossLaunch>(sdt, odt, p, k_layout == FFAI_K_TRANSPOSED,
                                              static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
  return FFAI_OK;
}

}  // extern "C"
