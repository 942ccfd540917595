// gfx950 (MI355X) fused attention kernels: O = softmax(scale * Q K^T [+ mask]) V in one pass.
//
// Design (one workgroup = NW waves = 32*NW query rows of one (batch, q-head); keys in tiles
// of 64):
//   * Both contractions run on MFMA with the score tile computed TRANSPOSED, S^T = K Q^T
//     (32 keys x 32 queries per v_mfma_f32_32x32x16_{bf16,f16} / 32x32x2_f32). In the 32x32
//     accumulator layout lane l owns query column l%32 and 16 of the 32 keys, lane l^32 the
//     other 16, so every softmax statistic (row max, row sum, rescale factor) is a per-lane
//     scalar: the only cross-lane traffic is one exchange with lane l^32 per tile for the max.
//   * The probabilities stay in registers: the accumulator of S^T is already the B operand
//     of O^T = V^T P^T once the key order inside each 16-key MFMA step is permuted the same
//     way on both operands (the contraction is a sum, so any shared order is exact).
//   * K and V tiles are staged through LDS once per workgroup: K as rows [key][d] (A operand
//     of the first product), V transposed [d][key] (A operand of the second). The reference's
//     K^T layout and V's row layout are transposed on the way in with register permutes.
//     The next tile's global loads are issued before the current tile's MFMAs.
//   * Online softmax in base 2: p = exp2(s*scale*log2e - m*scale*log2e) with v_exp_f32; the
//     accumulator is rescaled by exp2(m_old - m_new) per tile.
//   * Workgroup ids are remapped so that all query blocks of one (batch, kv-head) run on the
//     same XCD (the hardware deals workgroup i to XCD i % 8) and share that XCD's L2.
//   * Few-query shapes (decode) split the keys over workgroups; partial (O, m, l) go to the
//     workspace and combine_kernel merges them by log-sum-exp.

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
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int BN = kBlockN;
constexpr float kNegInf = -__builtin_huge_valf();

template <int DT>
using store_t = std::conditional_t<DT == kF32, float, uint16_t>;

// ---------------------------------------------------------------------------------------------
// Scalar conversions.
// ---------------------------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ float to_f32(uint32_t bits16) {
  if constexpr (DT == kBF16) {
    return __uint_as_float(bits16 << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
  }
}

template <int DT>
__device__ __forceinline__ uint32_t from_f32(float x) {  // round to nearest even
  if constexpr (DT == kBF16) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  } else {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
}

template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return from_f32<DT>(lo) | (from_f32<DT>(hi) << 16);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------------------------
// Global loads of short contiguous runs. `n` elements are valid (the rest read as zero and are
// never touched); `vec` is the widest access, in elements, that every address of this operand is
// aligned to (uniform over the launch).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ u32x4 load8_h(const uint16_t* p, int n, int vec) {
  if (n >= 8) {
    if (vec >= 8) return *reinterpret_cast<const u32x4*>(p);
    if (vec >= 4) {
      const u32x2 a = reinterpret_cast<const u32x2*>(p)[0];
      const u32x2 b = reinterpret_cast<const u32x2*>(p)[1];
      return u32x4{a.x, a.y, b.x, b.y};
    }
    if (vec >= 2) {
      const uint32_t* w = reinterpret_cast<const uint32_t*>(p);
      return u32x4{w[0], w[1], w[2], w[3]};
    }
  }
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (e < n) w[e >> 1] |= (uint32_t)p[e] << (16 * (e & 1));
  return u32x4{w[0], w[1], w[2], w[3]};
}

// Four elements widened to f32 (source f32, f16 or bf16).
template <int DT>
__device__ __forceinline__ f32x4 load4_f(const store_t<DT>* p, int n, int vec) {
  if constexpr (DT == kF32) {
    if (n >= 4) {
      if (vec >= 4) return *reinterpret_cast<const f32x4*>(p);
      if (vec >= 2) {
        const f32x2 a = reinterpret_cast<const f32x2*>(p)[0];
        const f32x2 b = reinterpret_cast<const f32x2*>(p)[1];
        return f32x4{a.x, a.y, b.x, b.y};
      }
    }
    f32x4 r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (e < n) r[e] = p[e];
    return r;
  } else {
    uint32_t w0 = 0u, w1 = 0u;
    if (n >= 4 && vec >= 4) {
      const u32x2 a = *reinterpret_cast<const u32x2*>(p);
      w0 = a.x;
      w1 = a.y;
    } else if (n >= 4 && vec >= 2) {
      w0 = reinterpret_cast<const uint32_t*>(p)[0];
      w1 = reinterpret_cast<const uint32_t*>(p)[1];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < n) {
          const uint32_t x = (uint32_t)p[e] << (16 * (e & 1));
          if (e < 2) w0 |= x; else w1 |= x;
        }
    }
    return f32x4{to_f32<DT>(w0 & 0xffffu), to_f32<DT>(w0 >> 16), to_f32<DT>(w1 & 0xffffu),
                 to_f32<DT>(w1 >> 16)};
  }
}

// Store four consecutive outputs.
template <int DT>
__device__ __forceinline__ void store4(store_t<DT>* p, f32x4 x, int vec) {
  if constexpr (DT == kF32) {
    if (vec >= 4) {
      *reinterpret_cast<f32x4*>(p) = x;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) p[e] = x[e];
    }
  } else {
    if (vec >= 4) {
      *reinterpret_cast<u32x2*>(p) = u32x2{pack2<DT>(x[0], x[1]), pack2<DT>(x[2], x[3])};
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) p[e] = (uint16_t)from_f32<DT>(x[e]);
    }
  }
}

// Element k (0..7) of eight 16-bit values held in a u32x4, paired with the same element of a
// second row: low half from `r0`, high half from `r1` (one v_perm_b32).
__device__ __forceinline__ uint32_t pair_elem(u32x4 r0, u32x4 r1, int k) {
  const uint32_t a = r0[k >> 1], b = r1[k >> 1];
  return (k & 1) ? __builtin_amdgcn_perm(b, a, 0x07060302u) : __builtin_amdgcn_perm(b, a, 0x05040100u);
}

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

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------------
// The forward kernel.
//   MODE  kBF16 / kF16: Q, K, V are that 16-bit type; both products on 32x32x16 MFMA.
//         kF32: Q f32, K/V of type KVT widened to f32 in LDS; both products on 32x32x2 f32 MFMA.
//   OUTT  output type. D head_dim. KT: K given transposed (d-major). NW waves per workgroup.
// ---------------------------------------------------------------------------------------------
template <int MODE, int KVT, int OUTT, int D, bool KT, int NW>
__global__ __launch_bounds__(NW * 64) void fwd_kernel(FwdParams p) {
  constexpr int NT = NW * 64;
  constexpr bool F32 = (MODE == kF32);
  using LT = std::conditional_t<F32, float, uint16_t>;  // LDS / compute storage type
  using KVS = store_t<KVT>;                            // K/V global storage type
  using QS = store_t<MODE>;                            // Q global storage type
  static_assert(F32 || KVT == MODE, "16-bit kernels read Q, K and V of one type");
  // LDS rows padded so that the MFMA operand reads below are bank-conflict free.
  constexpr int KROW = F32 ? D + 4 : D + 8;   // K rows [key][d]
  constexpr int VROW = BN + 4;                // V^T rows [d][key]
  __shared__ __attribute__((aligned(16))) LT k_lds[BN * KROW];
  __shared__ __attribute__((aligned(16))) LT v_lds[D * VROW];

  // ---- which (batch, head, query block, key split) this workgroup computes
  const int hw = blockIdx.x;
  const int work = (hw & 7) * (int)(gridDim.x >> 3) + (hw >> 3);
  if (work >= p.n_work) return;
  int rest = work;
  const int split = rest % p.n_split;
  rest /= p.n_split;
  int qb = rest % p.n_qblk;
  rest /= p.n_qblk;
  const int h = rest % p.Hq;
  const int b = rest / p.Hq;
  if (p.causal) qb = p.n_qblk - 1 - qb;  // longest rows first
  const int hk = h / (p.Hq / p.Hkv);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;    // lane group: which half of each MFMA contraction step
  const int n32 = lane & 31;  // query column of the accumulators
  constexpr int BM = NW * 32;
  const int q0 = qb * BM + wave * 32;  // this wave's first query row
  const int qrow = q0 + n32;

  int kv_end = p.Tk;
  if (p.kv_lens) kv_end = min(kv_end, max(0, p.kv_lens[b]));
  int kv_blk = kv_end;  // keys any row of this workgroup may see
  if (p.causal) kv_blk = min(kv_end, max(0, p.q_offset + min(qb * BM + BM, p.Tq)));
  const int n_tiles = (kv_blk + BN - 1) / BN;
  const int t_begin = split * p.tiles_per_split;
  const int t_end = min(n_tiles, t_begin + p.tiles_per_split);

  const QS* qp = reinterpret_cast<const QS*>(p.q) + b * p.q_sb + h * p.q_sh;
  const KVS* kp = reinterpret_cast<const KVS*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const KVS* vp = reinterpret_cast<const KVS*>(p.v) + b * p.v_sb + hk * p.v_sh;

  // ---- Q fragments (B operand of S^T = K Q^T), resident for the whole key loop
  constexpr int QF = F32 ? D / 2 : D / 16;
  std::conditional_t<F32, float, u32x4> qf[QF];
  {
    const bool ok = qrow < p.Tq;
    const QS* qr = qp + (int64_t)qrow * p.q_st;
    if constexpr (F32) {
      // step (j, e): lane group g supplies d = 8j + 4g + e
#pragma unroll
      for (int j = 0; j < D / 8; ++j) {
        const f32x4 x = load4_f<kF32>(qr + 8 * j + 4 * g, ok ? 4 : 0, p.q_vec);
#pragma unroll
        for (int e = 0; e < 4; ++e) qf[4 * j + e] = x[e];
      }
    } else {
      // step s: lane group g supplies d = 16s + 8g .. +7
#pragma unroll
      for (int s = 0; s < D / 16; ++s) qf[s] = load8_h(qr + 16 * s + 8 * g, ok ? 8 : 0, p.q_vec);
    }
  }

  // ---- staging registers for one K/V tile
  // 16-bit: K rows -> units of 8 elements; K^T -> units of (2 d-rows x 8 keys); V -> units of
  //         (2 keys x 8 d). f32: K rows -> 4 elements; K^T -> (4 d-rows x 4 keys); V -> (4 x 4).
  constexpr int K_UNITS = F32 ? (KT ? (D / 4) * (BN / 4) : BN * (D / 4))
                              : (KT ? (D / 2) * (BN / 8) : BN * (D / 8));
  constexpr int V_UNITS = F32 ? (BN / 4) * (D / 4) : (BN / 2) * (D / 8);
  constexpr int K_PER = (K_UNITS + NT - 1) / NT;
  constexpr int V_PER = (V_UNITS + NT - 1) / NT;
  constexpr int K_REGS = F32 ? (KT ? 4 : 1) : (KT ? 2 : 1);  // loads per unit
  constexpr int V_REGS = F32 ? 4 : 2;
  using SR = std::conditional_t<F32, f32x4, u32x4>;
  SR kreg[K_PER * K_REGS];
  SR vreg[V_PER * V_REGS];

  auto load_tile = [&](int it) {
    const int kb = it * BN;
#pragma unroll
    for (int i = 0; i < K_PER; ++i) {
      const int u = tid + i * NT;
      if (K_UNITS % NT != 0 && u >= K_UNITS) continue;
      if constexpr (F32) {
        if constexpr (KT) {
          const int d4 = u / (BN / 4), k4 = u % (BN / 4);
          const int key0 = kb + 4 * k4;
          const int n = min(max(kv_end - key0, 0), 4);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            kreg[4 * i + r] = load4_f<KVT>(kp + (int64_t)(4 * d4 + r) * p.k_st + key0, n, p.k_vec);
        } else {
          const int key = u / (D / 4), c = u % (D / 4);
          const int ok = (kb + key < kv_end) ? 4 : 0;
          kreg[i] = load4_f<KVT>(kp + (int64_t)(kb + key) * p.k_st + 4 * c, ok, p.k_vec);
        }
      } else {
        if constexpr (KT) {
          const int dp = u / (BN / 8), kc = u % (BN / 8);
          const int key0 = kb + 8 * kc;
          const int n = min(max(kv_end - key0, 0), 8);
          const KVS* r0 = kp + (int64_t)(2 * dp) * p.k_st + key0;
          kreg[2 * i] = load8_h(r0, n, p.k_vec);
          kreg[2 * i + 1] = load8_h(r0 + p.k_st, n, p.k_vec);
        } else {
          const int key = u / (D / 8), c = u % (D / 8);
          const int ok = (kb + key < kv_end) ? 8 : 0;
          kreg[i] = load8_h(kp + (int64_t)(kb + key) * p.k_st + 8 * c, ok, p.k_vec);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < V_PER; ++i) {
      const int u = tid + i * NT;
      if (V_UNITS % NT != 0 && u >= V_UNITS) continue;
      if constexpr (F32) {
        const int k4 = u / (D / 4), d4 = u % (D / 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kb + 4 * k4 + r;
          vreg[4 * i + r] =
              load4_f<KVT>(vp + (int64_t)key * p.v_st + 4 * d4, key < kv_end ? 4 : 0, p.v_vec);
        }
      } else {
        const int kp2 = u / (D / 8), c = u % (D / 8);
        const int key = kb + 2 * kp2;
        vreg[2 * i] = load8_h(vp + (int64_t)key * p.v_st + 8 * c, key < kv_end ? 8 : 0, p.v_vec);
        vreg[2 * i + 1] =
            load8_h(vp + (int64_t)(key + 1) * p.v_st + 8 * c, key + 1 < kv_end ? 8 : 0, p.v_vec);
      }
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < K_PER; ++i) {
      const int u = tid + i * NT;
      if (K_UNITS % NT != 0 && u >= K_UNITS) continue;
      if constexpr (F32) {
        if constexpr (KT) {
          const int d4 = u / (BN / 4), k4 = u % (BN / 4);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const f32x4 col = {kreg[4 * i][c], kreg[4 * i + 1][c], kreg[4 * i + 2][c],
                               kreg[4 * i + 3][c]};
            *reinterpret_cast<f32x4*>(&k_lds[(4 * k4 + c) * KROW + 4 * d4]) = col;
          }
        } else {
          const int key = u / (D / 4), c = u % (D / 4);
          *reinterpret_cast<f32x4*>(&k_lds[key * KROW + 4 * c]) = kreg[i];
        }
      } else {
        if constexpr (KT) {
          const int dp = u / (BN / 8), kc = u % (BN / 8);
          uint32_t* kw = reinterpret_cast<uint32_t*>(k_lds);
#pragma unroll
          for (int kk = 0; kk < 8; ++kk)
            kw[(8 * kc + kk) * (KROW / 2) + dp] = pair_elem(kreg[2 * i], kreg[2 * i + 1], kk);
        } else {
          const int key = u / (D / 8), c = u % (D / 8);
          *reinterpret_cast<u32x4*>(&k_lds[key * KROW + 8 * c]) = kreg[i];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < V_PER; ++i) {
      const int u = tid + i * NT;
      if (V_UNITS % NT != 0 && u >= V_UNITS) continue;
      if constexpr (F32) {
        const int k4 = u / (D / 4), d4 = u % (D / 4);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x4 col = {vreg[4 * i][c], vreg[4 * i + 1][c], vreg[4 * i + 2][c],
                             vreg[4 * i + 3][c]};
          *reinterpret_cast<f32x4*>(&v_lds[(4 * d4 + c) * VROW + 4 * k4]) = col;
        }
      } else {
        const int kp2 = u / (D / 8), c = u % (D / 8);
        uint32_t* vw = reinterpret_cast<uint32_t*>(v_lds);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          vw[(8 * c + e) * (VROW / 2) + kp2] = pair_elem(vreg[2 * i], vreg[2 * i + 1], e);
      }
    }
  };

  // ---- online-softmax state: this lane's query row, its half of the keys
  f32x16 oacc[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
  float m_run = kNegInf;  // running max of raw scores (row-wide after the exchange)
  float l_run = 0.f;      // running sum of this lane's weights
  const float sl2 = p.scale_log2;

  if (t_begin < t_end) load_tile(t_begin);
  for (int it = t_begin; it < t_end; ++it) {
    __syncthreads();  // every wave is done reading the previous tile
    store_tile();
    __syncthreads();
    if (it + 1 < t_end) load_tile(it + 1);  // in flight during this tile's MFMAs

    // ---- S^T = K Q^T for 2 x 32 keys: sacc[st][i] <-> key 32st + 8(i/4) + 4g + i%4
    f32x16 sacc[2];
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[st][r] = 0.f;
    if constexpr (F32) {
#pragma unroll
      for (int j = 0; j < D / 8; ++j)
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const f32x4 a =
              *reinterpret_cast<const f32x4*>(&k_lds[(32 * st + n32) * KROW + 8 * j + 4 * g]);
#pragma unroll
          for (int e = 0; e < 4; ++e) sacc[st] = mfma_f32(a[e], qf[4 * j + e], sacc[st]);
        }
    } else {
#pragma unroll
      for (int s = 0; s < D / 16; ++s)
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const u32x4 a =
              *reinterpret_cast<const u32x4*>(&k_lds[(32 * st + n32) * KROW + 16 * s + 8 * g]);
          sacc[st] = mfma16<MODE>(a, qf[s], sacc[st]);
        }
    }

    // ---- mask keys past this row's end (ragged tail, causal diagonal)
    const int kb = it * BN;
    const bool tail = kb + BN > kv_end;
    const bool diag = p.causal && (kb + BN - 1 > p.q_offset + q0);
    if (tail || diag) {
      const int lim = p.causal ? min(kv_end - 1, p.q_offset + qrow) : kv_end - 1;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb + 32 * st + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key > lim) sacc[st][r] = kNegInf;
        }
    }

    // ---- online softmax (base 2)
    float mx = kNegInf;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[st][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;  // row fully masked so far
    const float corr = fast_exp2((m_run - m_use) * sl2);
    const float mc = m_use * sl2;
    float rs = 0.f;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = fast_exp2(__builtin_fmaf(sacc[st][r], sl2, -mc));
        sacc[st][r] = e;
        rs += e;
      }
    l_run = __builtin_fmaf(l_run, corr, rs);
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) oacc[dt] *= corr;

    // ---- O^T += V^T P^T
    if constexpr (F32) {
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(
                &v_lds[(32 * dt + n32) * VROW + 32 * st + 8 * j + 4 * g]);
#pragma unroll
            for (int e = 0; e < 4; ++e) oacc[dt] = mfma_f32(a[e], sacc[st][4 * j + e], oacc[dt]);
          }
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const f32x16& sv = sacc[t >> 1];
        const int o = 8 * (t & 1);
        const u32x4 pf = {pack2<MODE>(sv[o + 0], sv[o + 1]), pack2<MODE>(sv[o + 2], sv[o + 3]),
                          pack2<MODE>(sv[o + 4], sv[o + 5]), pack2<MODE>(sv[o + 6], sv[o + 7])};
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          const LT* vr = &v_lds[(32 * dt + n32) * VROW + 16 * t + 4 * g];
          const u32x2 a0 = *reinterpret_cast<const u32x2*>(vr);
          const u32x2 a1 = *reinterpret_cast<const u32x2*>(vr + 8);
          oacc[dt] = mfma16<MODE>(u32x4{a0.x, a0.y, a1.x, a1.y}, pf, oacc[dt]);
        }
      }
    }
  }

  // ---- epilogue: oacc[dt][4r + e] <-> d = 32dt + 8r + 4g + e of query qrow
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (qrow >= p.Tq) return;
  if (p.n_split == 1) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    store_t<OUTT>* op = reinterpret_cast<store_t<OUTT>*>(p.o) + b * p.o_sb + h * p.o_sh +
                        (int64_t)qrow * p.o_st;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const f32x4 x = {oacc[dt][4 * r] * inv, oacc[dt][4 * r + 1] * inv,
                         oacc[dt][4 * r + 2] * inv, oacc[dt][4 * r + 3] * inv};
        store4<OUTT>(op + 32 * dt + 8 * r + 4 * g, x, p.o_vec);
      }
  } else {
    const int64_t prow = ((int64_t)(b * p.Hq + h) * p.n_split + split) * p.Tq + qrow;
    float* wo = p.ws + prow * D;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const f32x4 x = {oacc[dt][4 * r], oacc[dt][4 * r + 1], oacc[dt][4 * r + 2],
                         oacc[dt][4 * r + 3]};
        *reinterpret_cast<f32x4*>(wo + 32 * dt + 8 * r + 4 * g) = x;
      }
    if (g == 0) {
      float* ml = p.ws + (int64_t)p.B * p.Hq * p.n_split * p.Tq * D + prow * 2;
      *reinterpret_cast<f32x2*>(ml) = f32x2{m_run, l_tot};
    }
  }
}

// Merge split-key partials by log-sum-exp: one 64-lane workgroup per (batch, head, query row).
template <int OUTT, int D>
__global__ __launch_bounds__(64) void combine_kernel(CombineParams p) {
  const int row = blockIdx.x;
  const int t = row % p.Tq;
  const int bh = row / p.Tq;
  const int h = bh % p.Hq, b = bh / p.Hq;
  const int64_t base = (int64_t)bh * p.n_split * p.Tq + t;  // partial row of split 0
  const float* wo = p.ws + base * D;
  const float* ml = p.ws + (int64_t)p.B * p.Hq * p.n_split * p.Tq * D + base * 2;
  const int64_t so = (int64_t)p.Tq * D, sml = (int64_t)p.Tq * 2;
  float m = kNegInf;
  for (int s = 0; s < p.n_split; ++s) m = fmaxf(m, ml[s * sml]);
  const float mu = (m == kNegInf) ? 0.f : m;
  constexpr int PER = D / 64;
  float acc[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) acc[i] = 0.f;
  float l = 0.f;
  for (int s = 0; s < p.n_split; ++s) {
    const float w = fast_exp2((ml[s * sml] - mu) * p.scale_log2);
    l = __builtin_fmaf(w, ml[s * sml + 1], l);
#pragma unroll
    for (int i = 0; i < PER; ++i) acc[i] = __builtin_fmaf(w, wo[s * so + threadIdx.x + 64 * i], acc[i]);
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  store_t<OUTT>* op =
      reinterpret_cast<store_t<OUTT>*>(p.o) + b * p.o_sb + h * p.o_sh + (int64_t)t * p.o_st;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const float x = acc[i] * inv;
    if constexpr (OUTT == kF32) op[threadIdx.x + 64 * i] = x;
    else op[threadIdx.x + 64 * i] = (uint16_t)from_f32<OUTT>(x);
  }
}

}  // namespace
}  // namespace ffai
