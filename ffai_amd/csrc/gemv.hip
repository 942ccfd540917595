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

// ---- f16 GEMV on the matrix cores ------------------------------------------------------------
// y = W x for up to 16 beams as v_mfma_f32_16x16x32_f16 tiles: the weights are the A operand,
// loaded from HBM straight into the operand layout (lane l: row l % 16, eight consecutive
// elements at 8 (l / 16) of each 32-element block), and the beams are the B operand's columns.
// A one-row-per-wave VALU design reads every beam's x chunk again beside each 16-byte weight
// chunk (ten x loads per weight load at five beams), and those loads, not the weights, set its
// time; here x is read once per wave and shared by all the tile's rows.
//
// Tiles of TR weight rows, TR a power of two >= rows: MFMA row m = q TR + r holds weight row r
// over K part q, column n = q TR + b holds beam b over the same part (QN = 16 / TR parts), and
// the diagonal blocks C[q TR + r][q TR + b] are the parts' sums (the other blocks are computed
// and discarded: the matrix core has time to spare, HBM does not). Smaller tiles give short
// outputs more workgroups. A workgroup of NW waves owns one tile over the whole K: wave w takes
// 32 NJ elements of every part per pass; the waves' partial tiles meet in LDS and are summed in
// a fixed order, so every call gives the same bits.
//
// x to f16 without losing precision: per (column, wave, pass), x is scaled by a power of two s
// that brings max |x| into [2^14, 2^15), and split into hi = f16(x s) and lo = f16(x s - hi)
// (x s - hi is exact in f32). hi + lo carries x s to 22 significant bits; the f16 x f16
// products are exact in f32 and sum in f32; the tile is then multiplied by 1/s (exact). Elements
// more than 2^28 below their column's maximum fall into f16's subnormal range (absolute error
// below 2^-39 of the maximum). A column range holding an infinite element keeps its hi halves
// only (lo = 0, where inf - inf would give NaN), so an infinite x gives the infinite products
// f32 arithmetic gives.
//
// Loads: x first (dense: consecutive lanes take consecutive 16-byte pieces of each column's
// range, so every lane of the load is used), then the weights; loads complete in issue order,
// so the split of x runs while the weights are in flight. The split values reach the B layout
// through the wave's own LDS region (no workgroup barrier). Every load reads a clamped, valid
// address unconditionally and out-of-range elements are zeroed by a select afterwards (a load
// on one side of a branch makes the compiler wait for all loads at the join).
struct GemvParams {
  const uint16_t* w;
  const float* x;
  int64_t xs;
  float* y;
  int64_t ys;
  int32_t out_dim, in_dim, rows;
  int32_t tr_log2;  // tile rows TR = 1 << tr_log2
  int32_t nw;       // waves per workgroup
  int32_t passes;   // K passes of QN * nw * 32 NJ elements
};

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

// Max over groups of G consecutive lanes (G = 8, 16, 32 or 64; every lane gets its group's max).
template <int G>
__device__ __forceinline__ float group_max(float v) {
  v = fmaxf(v, dpp_mov<0xb1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_mov<0x4e>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror: the other quad of the 8
  if constexpr (G >= 16) v = fmaxf(v, dpp_mov<0x140>(v));  // row_mirror: the other 8 of the 16
  if constexpr (G >= 32) {
    const uint32_t u = __float_as_uint(v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);  // lanes l and l ^ 16
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  if constexpr (G >= 64) v = partner_max(v);  // lanes l and l ^ 32
  return v;
}

// EPI 0: y[b][o] = sum. EPI 1: the q/k/v epilogue, cache elements of type CDT.
// TL >= 0: a specialized launch shape known at compile time (tile rows 1 << TL, NW waves, one
// pass, the first NXL dense x loads hold every beam; ROWS > 0: exactly ROWS beams); the
// compiler then folds the index arithmetic and unrolls the waves' reduction (~0.3-0.8 us per
// call at the decoder's shapes).
// TL < 0: the shape comes from the parameters.
template <int NJ, int EPI, int CDT, int TL = -1, int NW = 0, int NXL = 0, int ROWS = 0>
__global__ __launch_bounds__(1024) void gemv_f16_kernel(GemvParams p, QkvCacheParams qp) {
  constexpr bool SPEC = TL >= 0;
  const int rows = ROWS > 0 ? ROWS : p.rows;  // beams (x rows)
  constexpr int KW = 32 * NJ;  // elements of one part per wave and pass
  constexpr int RS = KW + 8;   // LDS row of a column (halves; 16 bytes of it hold the scale)
  constexpr int LPC = KW / 4;  // lanes per column in the dense x load
  constexpr int NI = LPC / 4;  // dense x loads for all 16 columns
  extern __shared__ __attribute__((aligned(16))) uint16_t gemv_lds[];
  const int tid = item_id(), lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tl = SPEC ? TL : p.tr_log2, tr = 1 << tl, qn = 16 >> tl;
  const int nw = SPEC ? NW : p.nw;
  const int kp = nw * KW;  // one part's elements per pass
  const int m = lane & 15, g = lane >> 4;
  const int q = m >> tl, r = m & (tr - 1);  // A row m: weight row r of part q
  const int tile = wg_id_x();
  const uint16_t* wr = p.w + (int64_t)min(tile * tr + r, p.out_dim - 1) * p.in_dim;
  // this wave's LDS region: the hi rows of the columns that hold a beam (QN * rows of them,
  // column (part, beam) at row part * rows + beam), then their lo rows; at least the 304 floats
  // of the partial tile
  const int ncol = qn * rows;
  const int reg = max(2 * ncol * RS, 608);
  uint16_t* xw = gemv_lds + wave * reg;
  const bool nv = (m & (tr - 1)) < rows;  // B column m holds a beam
  const int ncm = (m >> tl) * rows + (m & (tr - 1));  // and its LDS row when it does
  const int ni = (ncol * LPC + 63) / 64;  // dense x loads that hold a beam
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int ps = 0; ps < (SPEC ? 1 : p.passes); ++ps) {
    const int kb = ps * qn * kp + wave * KW;
    // Dense x: load slot v = 0..15 is beam v / QN over part v % QN (MFMA column part TR + beam),
    // LPC lanes per slot, 4 elements each. Slots of beams >= rows load a valid beam's elements
    // and fill LDS rows that are never read; no branch, no division.
    // (A generic instance with more than 8 loads issues 4 before the weights and each later one
    // 4 slots ahead of its use, so that 4 stay in flight without holding all 16 in registers.)
    constexpr int NX1 = (SPEC || NI <= 8) ? NI : 4;
    f32x4 xv[NI];
    auto load_x = [&](int i) __attribute__((always_inline)) {
      const int f = 64 * i + lane, v = f / LPC;
      const int b = min(v >> (4 - tl), rows - 1), part = v & (qn - 1);
      const int k = min(kb + part * kp + 4 * (f % LPC), p.in_dim - 4);
      xv[i] = *reinterpret_cast<const f32x4*>(p.x + b * p.xs + k);
    };
#pragma unroll
    for (int i = 0; i < NX1; ++i) {
      if (SPEC && i >= NXL) break;
      load_x(i);
    }
    __builtin_amdgcn_sched_barrier(0);
    u32x4 a[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      a[j] = ld16(wr + min(kb + q * kp + 32 * j + 8 * g, p.in_dim - 8));
    // split the loaded slots that hold a beam (the first QN * rows; the rest are never read)
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      // every address is clamped inside x: the prefetch needs no test of ni (a load under a
      // branch would make the compiler wait for every load at the join)
      if constexpr (NX1 < NI) {
        if (i + NX1 < NI) load_x(i + NX1);
      }
      if (SPEC ? i >= NXL : i >= ni) {  // wave-uniform
        if constexpr (NX1 < NI) continue;  // (a loop of 16 with a load would not unroll on break)
        else break;
      }
      const int f = 64 * i + lane, v = f / LPC, c4 = f % LPC;
      const int b = v >> (4 - tl), part = v & (qn - 1);
      const bool ok = kb + part * kp + 4 * c4 < p.in_dim;
      float mx = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xv[i][e] = ok ? xv[i][e] : 0.f;
        mx = fmaxf(mx, fabsf(xv[i][e]));
      }
      mx = group_max<LPC>(mx);
      // s = 2^(14 - e) for max in [2^e, 2^(e+1)): biased exponent 141 - e = 268 - (max >> 23),
      // kept in [1, 253] so that s and 1/s are normal
      const int sb = min(max(268 - (int)(__float_as_uint(mx) >> 23), 1), 253);
      const float sc = __uint_as_float((uint32_t)sb << 23);
      const bool fin = mx < __builtin_inff();  // an infinite element: its column keeps hi only
      uint32_t hp[2], lp[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float v0 = xv[i][2 * e] * sc, v1 = xv[i][2 * e + 1] * sc;
        const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
        const _Float16 l0 = (_Float16)(v0 - (float)h0), l1 = (_Float16)(v1 - (float)h1);
        hp[e] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        lp[e] = fin ? (uint32_t)__builtin_bit_cast(uint16_t, l0) |
                          ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16)
                    : 0u;
      }
      if (b < rows) {  // the last load's slots past the beams hold nothing to keep
        const int n = part * rows + b;
        *reinterpret_cast<u32x2*>(xw + n * RS + 4 * c4) = u32x2{hp[0], hp[1]};
        *reinterpret_cast<u32x2*>(xw + (ncol + n) * RS + 4 * c4) = u32x2{lp[0], lp[1]};
        if (c4 == 0) xw[n * RS + KW] = (uint16_t)sb;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      u32x4 bh = {0u, 0u, 0u, 0u}, bl = bh;
      if (nv) {
        bh = ld16(xw + ncm * RS + 32 * j + 8 * g);
        bl = ld16(xw + (ncol + ncm) * RS + 32 * j + 8 * g);
      }
      const bool kin = kb + q * kp + 32 * j + 8 * g < p.in_dim;
      u32x4 aj;
#pragma unroll
      for (int e = 0; e < 4; ++e) aj[e] = kin ? a[j][e] : 0u;
      c = mfma16x16<kF16>(aj, bh, c);
      c = mfma16x16<kF16>(aj, bl, c);
    }
    // D lane l holds rows 4 (l / 16) .. +3 of column l % 16 = m: the column's 1/s
    const int sb = nv ? (int)xw[ncm * RS + KW] : 127;
    const float inv = __uint_as_float((uint32_t)(254 - sb) << 23);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(c[e], inv, acc[e]);
    // the next pass rewrites this region: its reads are done (one wave's LDS accesses complete
    // in order)
  }
  // the waves' partial tiles, each in its own region: sum over parts and waves in a fixed order.
  // Lane l's 4 floats at word 4 l + 16 (l / 16): the readers below take one value each, threads
  // of a beam walking the tile rows, and unpadded those of a beam fell on the same 4 banks
  reinterpret_cast<f32x4*>(xw + 2 * 16 * (lane >> 4))[lane] = acc;
  __syncthreads();
  for (int t = tid; t < (rows << tl); t += nw * 64) {
    const int b = t >> tl, rr = t & (tr - 1);  // beam b, tile row rr
    const int o = tile * tr + rr;
    if (o >= p.out_dim) continue;
    float v = 0.f;
    for (int qq = 0; qq < qn; ++qq) {
      const int mm = (qq << tl) + rr, nn = (qq << tl) + b;
      const int l = nn + 16 * (mm >> 2), e = mm & 3;
      // all the waves' values first (independent LDS reads), then the sum in wave order
      float pv[16];
#pragma unroll
      for (int ww = 0; ww < 16; ++ww)
        pv[ww] = ww < nw ? reinterpret_cast<const float*>(
                               gemv_lds + ww * reg)[4 * l + e + 16 * (l >> 4)]
                         : 0.f;
#pragma unroll
      for (int ww = 0; ww < 16; ++ww) v += pv[ww];
    }
    if constexpr (EPI == 0) {
      p.y[b * p.ys + o] = v;
    } else {
      if (qp.bias) v = v + qp.bias[o];
      const int part = o / qp.n;  // 0: q, 1: k, 2: v
      const int oo = o - part * qp.n;
      if (part == 0) {
        qp.q[b * qp.qs + oo] = v;
      } else {
        // a length outside [1, capacity] is clamped; 0 (no advance) writes nothing
        const int pos = min(max(qp.lens[b], 0), qp.capacity) - 1;
        if (pos >= 0) {
          const int h = oo / qp.head_dim, d = oo - h * qp.head_dim;
          store_t<CDT>* cptr = reinterpret_cast<store_t<CDT>*>(part == 1 ? qp.ck : qp.cv) +
                               (int64_t)b * qp.cs + (int64_t)h * qp.ch + (int64_t)pos * qp.cp + d;
          if constexpr (CDT == kF32) *cptr = v;
          else *cptr = from_f32<CDT>(v);
        }
      }
    }
  }
}

// Launch shape for (out_dim, in_dim, rows): the largest tile (<= 16 rows, >= rows) that still
// gives ~192 workgroups, then per part the fewest passes with at most 16 waves, 32 NJ elements
// each (NJ 2, 4 or 8; 1 for a single block), NJ halved while the waves' LDS regions would exceed
// the CU's 160 KB.
struct GemvShape {
  int tr_log2, nw, nj, passes;
  size_t lds;
};
GemvShape gemv_shape(int out_dim, int in_dim, int rows) {
  int min_tl = 0;
  while ((1 << min_tl) < rows) ++min_tl;
  int tl = 4;
  while (tl > min_tl && (out_dim + (1 << tl) - 1) / (1 << tl) < 192) --tl;
  const int qn = 16 >> tl;
  const int bpp = (in_dim / 8 + 4 * qn - 1) / (4 * qn);  // 32-element blocks per part
  GemvShape s{};
  s.tr_log2 = tl;
  s.nj = bpp == 1 ? 1 : (bpp + 1) / 2 <= 16 ? 2 : (bpp + 3) / 4 <= 16 ? 4 : 8;
  for (;;) {
    s.nw = std::min(16, (bpp + s.nj - 1) / s.nj);
    s.passes = (bpp + s.nw * s.nj - 1) / (s.nw * s.nj);
    // per wave: hi and lo rows (32 NJ + 8 halves) of the QN * rows columns holding a beam, at
    // least the 304 floats of the partial tile
    const size_t reg = std::max<size_t>((size_t)2 * qn * rows * (32 * s.nj + 8), 608);
    s.lds = (size_t)s.nw * reg * 2;
    if (s.lds <= 160 * 1024 || s.nj == 1) break;
    s.nj /= 2;
  }
  return s;
}

// One kernel instance on its launch shape. Dynamic LDS above 64 KB is allowed once per instance
// (up to the CU's 160 KB): the static lives in the instance's own function.
template <int NJ, int EPI, int CDT, int TL = -1, int NW = 0, int NXL = 0, int ROWS = 0>
hipError_t launch_one(size_t lds, dim3 grid, dim3 block, hipStream_t st, const GemvParams& p,
                      const QkvCacheParams& qp) {
  auto kern = gemv_f16_kernel<NJ, EPI, CDT, TL, NW, NXL, ROWS>;
  if (lds > 65536) {
    static const hipError_t allowed = hipFuncSetAttribute(
        reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
        160 * 1024);
    if (allowed != hipSuccess) return allowed;
  }
  hipLaunchKernelGGL(kern, grid, block, lds, st, p, qp);
  return hipGetLastError();
}

// The specialized shape (TL, NW, NJ, NXL) if the call's shape is it and its beams fit NXL loads
// (and number ROWS, if ROWS > 0).
template <int EPI, int CDT, int TL, int NW, int NJ, int NXL, int ROWS = 0>
bool try_spec(const GemvShape& s, int nxl, dim3 grid, hipStream_t st, const GemvParams& p,
              const QkvCacheParams& qp, hipError_t& e) {
  if (s.tr_log2 != TL || s.nw != NW || s.nj != NJ || s.passes != 1 || nxl > NXL) return false;
  if (ROWS > 0 && p.rows != ROWS) return false;
  e = launch_one<NJ, EPI, CDT, TL, NW, NXL, ROWS>(s.lds, grid, dim3(64 * NW), st, p, qp);
  return true;
}

template <int EPI, int CDT>
hipError_t launch_gemv(GemvParams p, const QkvCacheParams& qp, int out_rows, hipStream_t st) {
  const GemvShape s = gemv_shape(out_rows, p.in_dim, p.rows);
  p.tr_log2 = s.tr_log2;
  p.nw = s.nw;
  p.passes = s.passes;
  const dim3 grid((unsigned)((out_rows + (1 << s.tr_log2) - 1) >> s.tr_log2));
  // dense x loads that hold a beam: (16 >> tl) parts x rows columns, 8 NJ lanes each
  const int nxl = ((16 >> s.tr_log2) * p.rows * 8 * s.nj + 63) / 64;
  hipError_t e = hipSuccess;
  // the whisper decoders' projections, beam 5 and greedy: medium (d 1024: n x n, 3n x n, 4n x n,
  // n x 4n) and large (d 1280, beam 5: n x n, 3n x n and 4n x n, n x 4n)
  if constexpr (EPI == 0) {
    if (try_spec<EPI, CDT, 3, 8, 2, 3, 5>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 3, 8, 2, 4>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 4, 16, 2, 1>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 4, 16, 2, 2, 5>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 4, 16, 2, 2>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 4, 16, 2, 4>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 3, 16, 4, 5, 5>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 3, 16, 4, 8>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 2, 4, 2, 1, 1>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 2, 16, 2, 1, 1>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 3, 10, 2, 3, 5>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 4, 10, 4, 3, 5>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 3, 10, 8, 10, 5>(s, nxl, grid, st, p, qp, e))
      return e;
  } else {
    if (try_spec<EPI, CDT, 4, 16, 2, 1>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 4, 16, 2, 2, 5>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 4, 16, 2, 2>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 4, 16, 2, 4>(s, nxl, grid, st, p, qp, e) ||
        try_spec<EPI, CDT, 4, 10, 4, 3, 5>(s, nxl, grid, st, p, qp, e))
      return e;
  }
  const dim3 block(64 * s.nw);
  if (s.nj == 1) return launch_one<1, EPI, CDT>(s.lds, grid, block, st, p, qp);
  if (s.nj == 2) return launch_one<2, EPI, CDT>(s.lds, grid, block, st, p, qp);
  if (s.nj == 4) return launch_one<4, EPI, CDT>(s.lds, grid, block, st, p, qp);
  return launch_one<8, EPI, CDT>(s.lds, grid, block, st, p, qp);
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
// held as int8 for the integer products). Workspace: rows * d bytes of x_u (16-byte aligned
// rows), then sx. One wave per row: the row max by DPP and lane swaps (a max is the same in any
// order), no barrier.
// One wave per beam row. NC > 0 (d <= 256 NC, x rows 16-byte aligned): lane l holds elements
// 4 l + 256 i .. +3 (i < NC) in registers, the row's loads issued together and read once. NC = 0:
// a strided loop over the row.
template <int NC>
__global__ __launch_bounds__(64) void vocab_act_quant_kernel(const float* __restrict__ x,
                                                             int64_t xs, int d, int d_pad,
                                                             int8_t* __restrict__ xu,
                                                             float* __restrict__ sx_out) {
#pragma clang fp contract(off)
  const int r = wg_id_x(), lane = item_id();
  const float* xr = x + r * xs;
  int8_t* xq = xu + (int64_t)r * d_pad;
  // q = round(x / sx) clamped to [-64, 63], stored offset by 64
  auto quant = [](float v, float sx) __attribute__((always_inline)) {
    return (int)fminf(fmaxf(round_away(__fdiv_rn(v, sx)), -64.f), 63.f) + 64;
  };
  float sx;
  if constexpr (NC > 0) {
    f32x4 v[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i)
      v[i] = *reinterpret_cast<const f32x4*>(xr + min(4 * lane + 256 * i, d - 4));
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i)
      if (4 * lane + 256 * i < d)
#pragma unroll
        for (int e = 0; e < 4; ++e) m = fmaxf(m, fabsf(v[i][e]));
    const float amax = wave_max_all(m);
    sx = amax > 0.f ? __fdiv_rn(amax, 63.f) : 1.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int k = 4 * lane + 256 * i;
      if (k < d) {
        uint32_t packed = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) packed |= (uint32_t)quant(v[i][e], sx) << (8 * e);
        *reinterpret_cast<uint32_t*>(xq + k) = packed;  // d_pad and the workspace: 16-byte aligned
      }
    }
  } else {
    float m = 0.f;
    for (int k = lane; k < d; k += 64) m = fmaxf(m, fabsf(xr[k]));
    const float amax = wave_max_all(m);
    sx = amax > 0.f ? __fdiv_rn(amax, 63.f) : 1.f;
    for (int k = lane; k < d; k += 64) xq[k] = (int8_t)quant(xr[k], sx);
  }
  if (lane == 0) sx_out[r] = sx;
}

// Workgroup: kVocabRowsPerWg = 16 vocabulary rows. Phase 1 on the matrix cores
// (v_mfma_i32_16x16x64_i8, exact integer products and sums): the 16 rows are the A operand, lane
// l holding bytes 16 (l / 16) .. +15 of row l % 16 in each 64-element step. The B columns are
// (beam b, half h) = b % 8 + 8 h: beam b's activations over the step's half h (32 elements, which
// lie inside one block since blocks are multiples of 32) and zero over the other half, so
// C[row][b % 8 + 8 h] is that half's exact dot, added into its block's sum in LDS (stored
// directly when blocks are 32 elements, each sum then having one contribution). Beams 8-15 take a
// second product (a second instance, NG = 2, so that up to 8 beams keep the registers of one).
// Each wave takes four consecutive steps per round trip, the activations loaded before the
// weights: beside a one-row-per-wave dot loop this reads each activation once per 16 rows
// instead of once per row, and needs no LDS atomics. Phase 2: one thread per (beam, row) runs
// the in-order float sum over blocks (LDS rows of nb + 1 words: at nb words the 64 lanes of
// each of its reads fell in two banks, and that phase cost as much as streaming the weights),
// then the workgroup ends.
constexpr int kVocabRowsPerWg = 16;
constexpr int kVocabSteps = 4;  // 64-element steps per wave and round trip
constexpr int kVocabScPerLane = 4;  // block scales per lane: 16 rows x up to 64 blocks

typedef int i32x4 __attribute__((ext_vector_type(4)));

template <int NG>  // products per step: groups of 8 beams (1 for rows <= 8, else 2)
__global__ __launch_bounds__(256) void vocab_logits_kernel(
    const int8_t* __restrict__ qw, const float* __restrict__ bscale,
    const float* __restrict__ corr, int vocab, int d, int blk, int rows,
    const int8_t* __restrict__ xu, int d_pad, const float* __restrict__ sx,
    float* __restrict__ logits, int64_t ls) {
#pragma clang fp contract(off)  // separately rounded multiply and add, as in the reference
  // [rows][kVocabRowsPerWg][nb] block sums, then the rows' scales, rows of nb + 1 words: phase 2
  // walks a row per thread, and an even stride put all 64 lanes of a read in two banks
  extern __shared__ int bs_lds[];
  const int nb = d / blk, nbs = nb + 1;
  const int v0 = wg_id_x() * kVocabRowsPerWg;
  float* sc_lds = reinterpret_cast<float*>(bs_lds + rows * kVocabRowsPerWg * nbs);
  const bool single = blk == 32;  // one contribution per block sum: stores, no zeroing
  // the workgroup's block scales (kVocabRowsPerWg * nb contiguous floats), loaded before the
  // operands so that they land with them; to LDS after the products
  const int n_sc = min(kVocabRowsPerWg, vocab - v0) * nb;
  const bool sc_staged = kVocabRowsPerWg * nb <= 256 * kVocabScPerLane;  // else read in phase 2
  float scv[kVocabScPerLane];
#pragma unroll
  for (int i = 0; i < kVocabScPerLane; ++i)
    scv[i] = bscale[(int64_t)v0 * nb + min(item_id() + 256 * i, n_sc - 1)];
  if (!single) {
    const int n_bs = rows * kVocabRowsPerWg * nbs;
    for (int i = item_id(); i < n_bs; i += 256) bs_lds[i] = 0;
    __syncthreads();
  }
  {
    const int wave = item_id() >> 6, lane = item_id() & 63;
    const int m = lane & 15, g = lane >> 4;
    const int steps = (d + 63) / 64;
    const int8_t* arow = qw + (int64_t)min(v0 + m, vocab - 1) * d;
    for (int s0 = wave * kVocabSteps; s0 < steps; s0 += 4 * kVocabSteps) {
      // activations first, then the weights; every address clamped to valid data, inactive
      // operands zeroed afterwards (a load on one side of a branch would make the compiler wait
      // for all loads at the join)
      u32x4 bx[NG][kVocabSteps], av[kVocabSteps];
#pragma unroll
      for (int gr = 0; gr < NG; ++gr)
#pragma unroll
        for (int j = 0; j < kVocabSteps; ++j) {
          const int bb = min((m & 7) + 8 * gr, rows - 1);
          const int k = min(64 * (s0 + j) + 16 * g, d - 16);
          bx[gr][j] = *reinterpret_cast<const u32x4*>(xu + (int64_t)bb * d_pad + k);
        }
#pragma unroll
      for (int j = 0; j < kVocabSteps; ++j)
        av[j] = *reinterpret_cast<const u32x4*>(arow + min(64 * (s0 + j) + 16 * g, d - 16));
#pragma unroll
      for (int j = 0; j < kVocabSteps; ++j) {
        const int st = s0 + j;
        if (st >= steps) break;  // wave-uniform
#pragma unroll
        for (int gr = 0; gr < NG; ++gr) {
          const int b = (m & 7) + 8 * gr, h = m >> 3;
          const bool on = b < rows && (g >> 1) == h && 64 * st + 16 * g < d;
          u32x4 bv;
#pragma unroll
          for (int e = 0; e < 4; ++e) bv[e] = on ? bx[gr][j][e] : 0u;
          const i32x4 c = __builtin_amdgcn_mfma_i32_16x16x64_i8(
              __builtin_bit_cast(i32x4, av[j]), __builtin_bit_cast(i32x4, bv),
              i32x4{0, 0, 0, 0}, 0, 0, 0);
          // D lane l holds rows 4 (l / 16) .. +3 of column l % 16 = m: beam b, half h
          const int k0 = 64 * st + 32 * h;
          if (b < rows && k0 < d) {
            const int blkx = k0 / blk;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              int* dst = &bs_lds[(b * kVocabRowsPerWg + 4 * g + i) * nbs + blkx];
              if (single) *dst = c[i];
              else atomicAdd(dst, c[i]);
            }
          }
        }
      }
    }
  }

  if (sc_staged) {
#pragma unroll
    for (int i = 0; i < kVocabScPerLane; ++i) {
      const int idx = item_id() + 256 * i;  // scale idx of the workgroup's rows: row idx / nb
      if (idx < n_sc) sc_lds[idx + idx / nb] = scv[i];
    }
  }
  __syncthreads();
  for (int t = item_id(); t < rows * kVocabRowsPerWg; t += 256) {
    const int r = t / kVocabRowsPerWg, rl = t % kVocabRowsPerWg;
    const int v = v0 + rl;
    if (v >= vocab) continue;
    const int* bsr = bs_lds + (r * kVocabRowsPerWg + rl) * nbs;
    const float* scr = sc_staged ? sc_lds + rl * nbs : bscale + (int64_t)v * nb;
    float acc = 0.f;
#pragma unroll 8
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
  // block sums of every (beam, row, block), then the rows' block scales when they are staged
  const int nb = d / blk;
  const int staged = kVocabRowsPerWg * nb <= 256 * kVocabScPerLane ? 1 : 0;
  return (size_t)(rows + staged) * kVocabRowsPerWg * (nb + 1) * sizeof(int);
}
constexpr size_t kVocabLdsMax = 64 * 1024;
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
  GemvParams p{};
  p.w = static_cast<const uint16_t*>(w);
  p.x = x; p.xs = x_row_stride; p.y = y; p.ys = y_row_stride;
  p.out_dim = out_dim; p.in_dim = in_dim; p.rows = rows;
  const hipError_t e = launch_gemv<0, kF32>(p, QkvCacheParams{}, out_dim,
                                            static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
  return FFAI_OK;
}

int ffai_gemv_f16_plan_info(int32_t out_dim, int32_t in_dim, int32_t rows, int32_t* tile_rows,
                            int32_t* waves, int32_t* blocks_per_wave, int32_t* passes,
                            size_t* lds_bytes) {
  api_clear_error();
  if (!tile_rows || !waves || !blocks_per_wave || !passes || !lds_bytes)
    return api_fail(FFAI_ERR_INVALID, "null pointer");
  if (out_dim < 1 || in_dim < 8 || in_dim % 8) return api_fail(FFAI_ERR_INVALID, "out_dim >= 1 and in_dim a multiple of 8");
  if (rows < 1 || rows > kMaxGemvRows) return api_fail(FFAI_ERR_INVALID, "rows must be in [1, 16]");
  const GemvShape s = gemv_shape(out_dim, in_dim, rows);
  *tile_rows = 1 << s.tr_log2;
  *waves = s.nw;
  *blocks_per_wave = s.nj;
  *passes = s.passes;
  *lds_bytes = s.lds;
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
  GemvParams gp{};
  gp.w = static_cast<const uint16_t*>(w);
  gp.x = x; gp.xs = x_row_stride;
  gp.out_dim = (int32_t)(3 * n); gp.in_dim = in_dim; gp.rows = rows;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int cdt = c->dtype;  // FFAI_F32 / F16 / BF16 are kF32 / kF16 / kBF16
  const hipError_t e = cdt == kF32   ? launch_gemv<1, kF32>(gp, p, (int)(3 * n), st)
                       : cdt == kF16 ? launch_gemv<1, kF16>(gp, p, (int)(3 * n), st)
                                     : launch_gemv<1, kBF16>(gp, p, (int)(3 * n), st);
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
  // d is a multiple of 32: whole 16-byte chunks when the rows are 16-byte aligned
  const bool xa = (uintptr_t)x % 16 == 0 && (rows == 1 || x_row_stride % 4 == 0);
  const int nc = xa ? (d + 255) / 256 : 0;
  auto quant = nc == 0 ? vocab_act_quant_kernel<0>
               : nc <= 2 ? vocab_act_quant_kernel<2>
               : nc <= 4 ? vocab_act_quant_kernel<4>
               : nc <= 8 ? vocab_act_quant_kernel<8> : vocab_act_quant_kernel<0>;
  hipLaunchKernelGGL(quant, dim3(rows), dim3(64), 0, st, x, x_row_stride, d, d_pad, xu, sx);
  const dim3 grid((unsigned)((vocab + kVocabRowsPerWg - 1) / kVocabRowsPerWg));
  if (rows <= 8)
    hipLaunchKernelGGL(vocab_logits_kernel<1>, grid, dim3(256), vocab_lds_bytes(d, blk, rows), st,
                       qw, bscale, corr, vocab, d, blk, rows, xu, d_pad, sx, logits,
                       logits_row_stride);
  else
    hipLaunchKernelGGL(vocab_logits_kernel<2>, grid, dim3(256), vocab_lds_bytes(d, blk, rows), st,
                       qw, bscale, corr, vocab, d, blk, rows, xu, d_pad, sx, logits,
                       logits_row_stride);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
  return FFAI_OK;
}

}  // extern "C"
