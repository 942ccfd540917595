// gfx950 (MI355X) fused attention kernels: O = softmax(scale * Q K^T [+ mask]) V in one pass.
//
// Design (one workgroup = NW waves; each wave owns QW x 32 query rows of one (batch, q-head);
// keys stream in tiles of 64):
//   * Both contractions run on MFMA with the score tile computed TRANSPOSED, S^T = K Q^T
//     (32 keys x 32 queries per v_mfma_f32_32x32x16_{bf16,f16} / 32x32x2_f32). In the 32x32
//     accumulator layout lane l owns query column l%32 and 16 of the 32 keys, lane l^32 the
//     other 16, so every softmax statistic (row max, row sum, rescale factor) is a per-lane
//     scalar; the only cross-lane step is a v_permlane32_swap when a row max is taken.
//   * The probabilities stay in registers: the accumulator of S^T is already the B operand
//     of O^T = V^T P^T once the key order inside each 16-key MFMA step is permuted the same
//     way on both operands (the contraction is a sum, so any shared order is exact).
//   * With QW = 2 a wave computes two 32-query column blocks against each K/V fragment it
//     reads from LDS, halving LDS operand traffic per FLOP (at 32 queries per wave the LDS
//     read bandwidth alone would cap the MFMA pipes near 80 %).
//   * K and V tiles are staged through LDS once per workgroup. f32: double-buffered, K as rows
//     and V transposed, permuted in registers on the way in. 16-bit: three buffers filled by
//     global->LDS DMA in the layout they have in HBM (K^T or K rows, V rows), read back with
//     transposing LDS reads where an operand needs the other orientation. One barrier per tile.
//   * Online softmax in base 2 with v_exp_f32. f32 kernel: the running max only moves when a
//     tile's max exceeds it by more than 2^8 in probability. 16-bit kernels: no max is taken on
//     the common path at all. Q carries scale*log2(e), so scores come out of the first product
//     in the exponent's units. When every row max of a wave's first 32 keys is moderate, the
//     reference max is 0 and a weight is exp2 of the accumulator itself; otherwise it is that
//     first max. A subtile whose weights would exceed 2^64 (or overflow) is redone against its
//     exact max, with the accumulator rescaled; that is rare for real scores, and it keeps every
//     weight and sum finite in f32.
//   * Workgroup ids are remapped so that all query blocks of one (batch, kv-head) run on the
//     same XCD (the hardware deals workgroup i to XCD i % XCDs) and share that XCD's L2.
//   * Items (batch, head, query block) may run as several pieces, each a contiguous key range:
//     every item of a short grid, the last round's items of a long one, the longest items of a
//     causal one. Pieces write partial (O, m, l) to the workspace and the item's last piece to
//     finish merges them by log-sum-exp in the same launch.
#pragma once

#include "attn_common.cuh"

namespace ffai {
namespace {

// ---------------------------------------------------------------------------------------------
// The forward kernel.
//   MODE  kBF16 / kF16: Q, K, V are that 16-bit type; both products on 32x32x16 MFMA.
//         kF32: Q f32, K/V of type KVT widened to f32 in LDS; both products on 32x32x2 f32 MFMA.
//   OUTT  output type. D head_dim. KT: K given transposed (d-major). NW waves per workgroup.
//   QW    32-query column blocks per wave.
// ---------------------------------------------------------------------------------------------
// Four-wave launches are built for two workgroups per CU (<= 256 VGPRs): the second wave on each
// SIMD is what hides the first one's exp and dependency latencies.
template <int MODE, int KVT, int OUTT, int D, bool KT, int NW, int QW>
__global__ __launch_bounds__(NW * 64, (NW == 4 && (D == 64 || MODE != kF32)) ? 2 : 1) void fwd_kernel(FwdParams p) {
  constexpr int NT = NW * 64;
  constexpr bool F32 = (MODE == kF32);
  using LT = std::conditional_t<F32, float, uint16_t>;  // LDS / compute storage type
  using KVS = store_t<KVT>;                            // K/V global storage type
  using QS = store_t<MODE>;                            // Q global storage type
  static_assert(F32 || KVT == MODE, "16-bit kernels read Q, K and V of one type");
  static_assert(!F32 || QW == 1, "the f32 kernel uses one column block per wave");
  // LDS tiles.
  //   f32:    K [key][d] (KROW = D + 4), V^T [d][key] (VROW = BN + 4) - transposed on the way in;
  //           rows padded so that the 128-bit stores and the operand reads are conflict-free.
  //   16-bit: K [key][d] when K comes as rows, K^T [d][key] when it comes transposed, V [key][d]:
  //           all stored as they lie in HBM (so whole tiles go global -> LDS by DMA), the operands
  //           that need the other orientation read with ds_read_b64_tr_b16. Rows are unpadded;
  //           instead each row's 16-byte chunks are XOR-permuted (swz_*) so that the fragment
  //           reads of a wave spread over all banks.
  constexpr int KROW = F32 ? D + 4 : D;
  constexpr int KTROW = BN;
  constexpr int VROW = F32 ? BN + 4 : D;
  constexpr int KBUF = (!F32 && KT) ? D * KTROW : BN * KROW;
  constexpr int VBUF = F32 ? D * VROW : BN * VROW;
  // f32: double-buffered, one barrier per tile at the tile's end. 16-bit: the next tile is
  // staged and published (barrier) before the current tile's last product, so that product
  // overlaps the next tile's first one. Tile i's K is last read before the barrier of tile i,
  // its V after it (the last product): when that barrier stages tile i + 2, K(i + 2) can take
  // K(i)'s buffer but V(i + 2) needs a third. Head_dim 128 keeps two K buffers (80 KB of LDS:
  // two workgroups per CU); head_dim 64 keeps three of each (48 KB, as measured).
  constexpr int NBUF = F32 ? 2 : 3;                    // V buffers
  constexpr int NBK = F32 ? 2 : (D == 128 ? 2 : 3);  // K buffers
  __shared__ __attribute__((aligned(16))) LT k_lds[NBK * KBUF];
  __shared__ __attribute__((aligned(16))) LT v_lds[NBUF * VBUF];

  // ---- which work (an item, or one piece of a split item) this workgroup computes
  const int hw = wg_id_x();
#ifdef FFAI_STAMPS
  const uint64_t st_e0 = stamp_realtime();
  // prologue times go to the record as they are taken (nothing stays live across the loop)
#define FFAI_STAMP_PRO(k) \
  __builtin_amdgcn_sched_barrier(0); \
  stamp_now(k, stamp_realtime()); \
  __builtin_amdgcn_sched_barrier(0)
#else
#define FFAI_STAMP_PRO(k)
#endif
  int work;
  const int xs = p.xcd_shift, xm = (1 << xs) - 1;  // XCDs: 1 << xs
  if (hw < p.sec1_wgs) {
    work = p.xcd_remap ? (hw & xm) * (p.sec1_wgs >> xs) + (hw >> xs) : hw;
    if (work >= p.sec1_work) return;
  } else {
    // n: a multiple of 1 << xs. (gridDim is an out-of-line call, run only by this section's
    // workgroups; computing n from the parameters instead, with no call left in the kernel,
    // changes the register allocation of the 16-bit head_dim-64 instantiations to one that
    // spills.)
    const int x = hw - p.sec1_wgs, n = (int)gridDim.x - p.sec1_wgs;
    work = p.sec1_work + (p.xcd_remap ? (x & xm) * (n >> xs) + (x >> xs) : x);
    if (work >= p.n_work) return;
  }
  const int n_pieces = (p.split_hi - p.split_lo) * p.n_split;
  int rank, split = -1;  // split: the piece of a split item, -1 for a whole item
  if (work < p.split_lo) {
    rank = work;
  } else if (work < p.split_lo + n_pieces) {
    rank = p.split_lo + (work - p.split_lo) / p.n_split;
    split = (work - p.split_lo) % p.n_split;
  } else {
    rank = work - n_pieces + (p.split_hi - p.split_lo);
  }
  int qb, bh;
  if (p.causal) {  // longest rows first: query block descending, then (batch, head)
    const int nbh = p.B * p.Hq;
    qb = p.n_qblk - 1 - rank / nbh;
    bh = rank % nbh;
  } else {
    qb = rank % p.n_qblk;
    bh = rank / p.n_qblk;
  }
  const int h = bh % p.Hq;
  const int b = bh / p.Hq;
  const int hk = h / (p.Hq / p.Hkv);

  const int tid = item_id();
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps q0 scalar
  const int g = lane >> 5;    // lane group: which half of each MFMA contraction step
  const int n32 = lane & 31;  // query column of the accumulators
  constexpr int BM = NW * 32 * QW;
  const int q0 = qb * BM + wave * 32 * QW;  // this wave's first query row
#ifdef FFAI_STAMPS
  const int64_t st_rec = (p.stamps && hw < p.stamp_wgs) ? ((int64_t)hw * NW + wave) * 32 : -1;
  auto stamp_now = [&](int k, uint64_t v) {
    if (st_rec >= 0 && lane == 0) stamp_put(p.stamps, st_rec + k, v);
  };
  stamp_now(11, st_e0);
  stamp_now(14, stamp_where());
#endif

  int kv_end = p.Tk;
  if (p.kv_lens) kv_end = min(kv_end, max(0, p.kv_lens[b]));
  kv_end = __builtin_amdgcn_readfirstlane(kv_end);  // uniform (one batch item per workgroup)
  int kv_blk = kv_end;  // keys any row of this workgroup may see
  if (p.causal) kv_blk = min(kv_end, max(0, p.q_offset + min(qb * BM + BM, p.Tq)));
  const int n_tiles = (kv_blk + BN - 1) / BN;
  const int tps = split < 0 ? n_tiles : (n_tiles + p.n_split - 1) / p.n_split;
  const int t_begin = split < 0 ? 0 : split * tps;
  const int t_end = min(n_tiles, t_begin + tps);
  const bool aligned = p.aligned != 0;

  const QS* qp = reinterpret_cast<const QS*>(p.q) + b * p.q_sb + h * p.q_sh;
  const KVS* kp = reinterpret_cast<const KVS*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const KVS* vp = reinterpret_cast<const KVS*>(p.v) + b * p.v_sb + hk * p.v_sh;
  const char* kp_dma = uniform_ptr(reinterpret_cast<const char*>(kp));
  const char* vp_dma = uniform_ptr(reinterpret_cast<const char*>(vp));

  FFAI_STAMP_PRO(18);
  // ---- Q fragments (B operand of S^T = K Q^T), resident for the whole key loop
  constexpr int QF = F32 ? D / 2 : D / 16;
  std::conditional_t<F32, float, u32x4> qf[QW][QF];
#pragma unroll
  for (int c = 0; c < QW; ++c) {
    const int row = q0 + 32 * c + n32;
    const bool ok = row < p.Tq;
    const QS* qr = qp + (int64_t)min(row, p.Tq - 1) * p.q_st;
    if constexpr (F32) {
      // step (j, e): lane group g supplies d = 8j + 4g + e
#pragma unroll
      for (int j = 0; j < D / 8; ++j) {
        const f32x4 x = aligned ? ld4f<kF32, true>(qr + 8 * j + 4 * g)
                                : ld4f<kF32, false>(qr + 8 * j + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) qf[c][4 * j + e] = ok ? x[e] : 0.f;
      }
    } else {
      // step s: lane group g supplies d = 16s + 8g .. +7
#pragma unroll
      for (int s = 0; s < D / 16; ++s) {
        const u32x4 x = aligned ? ld16(qr + 16 * s + 8 * g) : ld8h_elem(qr + 16 * s + 8 * g);
        qf[c][s] = ok ? x : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

  // ---- staging: global -> registers (two tiles ahead) -> LDS
  // f32:    K rows -> units of 4 elements; K^T -> 4 d-rows x 4 keys (transposed in registers);
  //         V -> 4 keys x 4 d (transposed in registers).
  // 16-bit: K rows, K^T rows and V rows -> units of 8 elements (one 128-bit LDS store each);
  //         K^T rows are only 8-byte aligned in general (row stride = key count), so they are
  //         read from global memory as two 8-byte halves.
  constexpr int K_UNITS = F32 ? (KT ? (D / 4) * (BN / 4) : BN * (D / 4))
                              : (KT ? D * (BN / 8) : BN * (D / 8));
  constexpr int V_UNITS = F32 ? (BN / 4) * (D / 4) : BN * (D / 8);
  static_assert(K_UNITS % NT == 0 && V_UNITS % NT == 0, "staging units must tile the workgroup");
  constexpr int K_PER = K_UNITS / NT;
  constexpr int V_PER = V_UNITS / NT;
  using SR = std::conditional_t<F32, f32x4, u32x4>;
  constexpr int K_REGS = F32 ? (KT ? 4 : 1) : 1;  // registers per unit
  constexpr int V_REGS = F32 ? 4 : 1;
  SR kreg[K_PER * K_REGS];
  SR vreg[V_PER * V_REGS];

  // 16-bit LDS chunk permutations (chunk = 8 elements = 16 bytes; an XOR, so its own inverse):
  //   K^T rows (64 keys, 128 B) and 128-byte V rows: the transposing reads of a half-wave touch
  //   4 consecutive rows x 64 B, rows 2 and 3 land on rows 0 and 1's banks unless their chunks
  //   are flipped into the other half of the row;
  //   256-byte V rows (head_dim 128): all rows start on bank 0, so rows r..r+3 take 4 distinct
  //   64-byte quarters;
  //   K rows (16-byte reads, one chunk per lane from 32 consecutive rows): even rows 0..14 (and
  //   odd rows) must hit 8 (16) distinct chunks.
  auto swz_kt = [](int r, int c) { return c ^ (4 * ((r >> 1) & 1)); };
  auto swz_v = [](int r, int c) { return D == 64 ? c ^ (4 * ((r >> 1) & 1)) : c ^ (4 * (r & 3)); };
  auto swz_kr = [](int r, int c) { return D == 64 ? c ^ ((r >> 1) & 7) : c ^ (r & 15); };
  (void)swz_kt;
  (void)swz_v;
  (void)swz_kr;

  // Load tile `it` into kreg/vreg. Interior tiles of an aligned launch take unconditional
  // vector loads (the uniform `full` branch); tail tiles clamp every index to the last valid key,
  // so they too read only valid addresses without divergent branches. Rows past the last key are
  // zeroed by store_tile (K^T tails, loaded element-wise, are zeroed here): no value loaded here
  // is used before the tile is stored.
  auto load_tile = [&](int it) {
    const int kb = it * BN;
    const int klast = kv_end - 1;
    const bool full = aligned && (kb + BN <= kv_end);
#pragma unroll
    for (int i = 0; i < K_PER; ++i) {
      const int u = tid + i * NT;
      if constexpr (F32) {
        if constexpr (KT) {
          const int d4 = u / (BN / 4), k4 = u % (BN / 4);
          const int key0 = kb + 4 * k4;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const KVS* row = kp + (int64_t)(4 * d4 + r) * p.k_st;
            f32x4 x;
            if (full) {
              x = ld4f<KVT, true>(row + key0);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const KVS y = row[min(key0 + e, klast)];
                float f;
                if constexpr (KVT == kF32) f = y;
                else f = to_f32<KVT>(y);
                x[e] = (key0 + e <= klast) ? f : 0.f;
              }
            }
            kreg[4 * i + r] = x;
          }
        } else {
          const int key = kb + u / (D / 4), c = u % (D / 4);
          const KVS* src = kp + (int64_t)min(key, klast) * p.k_st + 4 * c;
          kreg[i] = aligned ? ld4f<KVT, true>(src) : ld4f<KVT, false>(src);
        }
      } else {
        if constexpr (KT) {
          const int d = u / (BN / 8), kc = u % (BN / 8);
          const int key0 = kb + 8 * kc;
          const uint16_t* row = kp + (int64_t)d * p.k_st;
          u32x4 x;
          if (full) {
            const u32x2 lo = ld8(row + key0), hi = ld8(row + key0 + 4);
            x = u32x4{lo.x, lo.y, hi.x, hi.y};
          } else {
            uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const uint32_t y = row[min(key0 + e, klast)];
              w[e >> 1] |= (key0 + e <= klast ? y : 0u) << (16 * (e & 1));
            }
            x = u32x4{w[0], w[1], w[2], w[3]};
          }
          kreg[i] = x;
        } else {
          const int key = kb + u / (D / 8), c = u % (D / 8);
          const uint16_t* src = kp + (int64_t)min(key, klast) * p.k_st + 8 * c;
          kreg[i] = aligned ? ld16(src) : ld8h_elem(src);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < V_PER; ++i) {
      const int u = tid + i * NT;
      if constexpr (F32) {
        const int k4 = u / (D / 4), d4 = u % (D / 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kb + 4 * k4 + r;
          const KVS* src = vp + (int64_t)min(key, klast) * p.v_st + 4 * d4;
          vreg[4 * i + r] = aligned ? ld4f<KVT, true>(src) : ld4f<KVT, false>(src);
        }
      } else {
        const int key = kb + u / (D / 8), c = u % (D / 8);
        const uint16_t* src = vp + (int64_t)min(key, klast) * p.v_st + 8 * c;
        vreg[i] = aligned ? ld16(src) : ld8h_elem(src);
      }
    }
  };

  // Write the tile `it` held in kreg/vreg to LDS buffer `buf`. Rows past the last valid key
  // (they were loaded from the clamped address) are zeroed here rather than at load time, so
  // that nothing waits for the loads until the tile is stored, one iteration later.
  auto store_tile = [&](int kbuf, int vbuf, int it) {
    LT* kl = k_lds + kbuf * KBUF;
    LT* vl = v_lds + vbuf * VBUF;
    const int kb = it * BN;
    const int klast = kv_end - 1;
    const bool full = kb + BN <= kv_end;
#pragma unroll
    for (int i = 0; i < K_PER; ++i) {
      const int u = tid + i * NT;
      if constexpr (F32) {
        if constexpr (KT) {
          const int d4 = u / (BN / 4), k4 = u % (BN / 4);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const f32x4 col = {kreg[4 * i][c], kreg[4 * i + 1][c], kreg[4 * i + 2][c],
                               kreg[4 * i + 3][c]};
            *reinterpret_cast<f32x4*>(&kl[(4 * k4 + c) * KROW + 4 * d4]) = col;
          }
        } else {
          const int key = u / (D / 4), c = u % (D / 4);
          *reinterpret_cast<f32x4*>(&kl[key * KROW + 4 * c]) =
              (full || kb + key <= klast) ? kreg[i] : f32x4{0.f, 0.f, 0.f, 0.f};
        }
      } else {
        if constexpr (KT) {
          const int d = u / (BN / 8), kc = u % (BN / 8);
          *reinterpret_cast<u32x4*>(&kl[d * KTROW + 8 * swz_kt(d, kc)]) = kreg[i];
        } else {
          const int key = u / (D / 8), c = u % (D / 8);
          *reinterpret_cast<u32x4*>(&kl[key * KROW + 8 * swz_kr(key, c)]) =
              (full || kb + key <= klast) ? kreg[i] : u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
#pragma unroll
    for (int i = 0; i < V_PER; ++i) {
      const int u = tid + i * NT;
      if constexpr (F32) {
        const int k4 = u / (D / 4), d4 = u % (D / 4);
        f32x4 rw[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          rw[r] = (full || kb + 4 * k4 + r <= klast) ? vreg[4 * i + r] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x4 col = {rw[0][c], rw[1][c], rw[2][c], rw[3][c]};
          *reinterpret_cast<f32x4*>(&vl[(4 * d4 + c) * VROW + 4 * k4]) = col;
        }
      } else {
        const int key = u / (D / 8), c = u % (D / 8);
        *reinterpret_cast<u32x4*>(&vl[key * VROW + 8 * swz_v(key, c)]) =
            (full || kb + key <= klast) ? vreg[i] : u32x4{0u, 0u, 0u, 0u};
      }
    }
  };

  // 16-bit, full tile of an aligned launch: global -> LDS directly (lds_dma16), one 1024-byte
  // LDS block (64 chunks) per wave instruction. Lane l of a block fills LDS chunk l, i.e.
  // physical chunk pc of row r, with the row's logical chunk swz(r, pc). Completion is awaited
  // (vm_wait_all) before the next workgroup barrier.
  // DMA geometry: each thread moves KB/NW 16-byte chunks of the K tile and VB/NW of the V tile
  // per tile; its byte offsets from the tile's first key (the XOR chunk permutation included)
  // are the same for every tile, so they are computed once and each tile only moves the
  // wave-uniform base.
  constexpr int KB_ = (!F32) ? KBUF / 512 : NW, VB_ = (!F32) ? VBUF / 512 : NW;  // 1 KB blocks
  uint32_t dma_koff[KB_ / NW], dma_voff[VB_ / NW];
  if constexpr (!F32) {
    static_assert(KB_ % NW == 0 && VB_ % NW == 0, "DMA blocks must tile the workgroup");
#pragma unroll
    for (int j = 0; j < KB_ / NW; ++j) {
      const int L = (j * NW + wave) * 64 + lane;
      if constexpr (KT) {
        const int r = L / (BN / 8), pc = L % (BN / 8);
        dma_koff[j] = (uint32_t)(2 * ((int64_t)r * p.k_st + 8 * swz_kt(r, pc)));
      } else {
        const int r = L / (D / 8), pc = L % (D / 8);
        dma_koff[j] = (uint32_t)(2 * ((int64_t)r * p.k_st + 8 * swz_kr(r, pc)));
      }
    }
#pragma unroll
    for (int j = 0; j < VB_ / NW; ++j) {
      const int L = (j * NW + wave) * 64 + lane;
      const int r = L / (D / 8), pc = L % (D / 8);
      dma_voff[j] = (uint32_t)(2 * ((int64_t)r * p.v_st + 8 * swz_v(r, pc)));
    }
  }
  auto dma_tile = [&](int kbuf, int vbuf, int it) {
    if constexpr (!F32) {
      const uint32_t kl = lds_addr(k_lds + kbuf * KBUF);
      const uint32_t vl = lds_addr(v_lds + vbuf * VBUF);
      // the tile index and the head's bases are wave-uniform: taken into scalar registers, the
      // 64-bit address arithmetic runs on the scalar unit instead of the VALU
      const int64_t kb = (int64_t)__builtin_amdgcn_readfirstlane(it) * BN;
      const char* kbase = uniform_ptr(kp_dma) + 2 * (KT ? kb : kb * p.k_st);
      const char* vbase = uniform_ptr(vp_dma) + 2 * kb * p.v_st;
#pragma unroll
      for (int j = 0; j < KB_ / NW; ++j)
        lds_dma16_sbase(kbase, dma_koff[j], kl + (j * NW + wave) * 1024);
#pragma unroll
      for (int j = 0; j < VB_ / NW; ++j)
        lds_dma16_sbase(vbase, dma_voff[j], vl + (j * NW + wave) * 1024);
    }
  };
  // Stage tile `it` into K buffer `kbuf` and V buffer `vbuf`: by DMA when whole and aligned,
  // else through registers (clamped, zero-filled tail; element-wise loads when misaligned),
  // synchronously.
  auto stage_tile = [&](int kbuf, int vbuf, int it) {
    if (p.dma && it * BN + BN <= kv_end) {
      dma_tile(kbuf, vbuf, it);
    } else {
      load_tile(it);
      store_tile(kbuf, vbuf, it);
    }
  };

  // ---- online-softmax state, per column block: this lane's query row, its half of the keys
  f32x16 oacc[QW][D / 32];
#pragma unroll
  for (int c = 0; c < QW; ++c)
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[c][dt][r] = 0.f;
  float m_s[QW];  // running max, already multiplied by scale*log2(e) (row-wide)
  float l_run[QW];  // running sum of this lane's weights
#pragma unroll
  for (int c = 0; c < QW; ++c) {
    m_s[c] = kNegInf;
    l_run[c] = 0.f;
  }
  const float sl2 = p.scale_log2;

  if (t_begin < t_end) {
    if constexpr (F32) {
      load_tile(t_begin);
      store_tile(0, 0, t_begin);
      if (t_begin + 1 < t_end) load_tile(t_begin + 1);
    } else {
      stage_tile(0, 0, t_begin);
      if (t_begin + 1 < t_end) stage_tile(1, 1, t_begin + 1);
      FFAI_STAMP_PRO(15);
      vm_wait_all();
      FFAI_STAMP_PRO(16);
    }
  }
  __syncthreads();
  FFAI_STAMP_PRO(17);
#undef FFAI_STAMP_PRO

  // Mask the keys of 32-key subtile `st` past each row's end (ragged tail, causal diagonal).
  // sacc[c][st][i] <-> key kb + 32st + 8(i/4) + 4g + i%4 of query q0 + 32c + n32.
  auto mask_subtile = [&](f32x16 (&sacc)[QW][2], int kb, int st) {
#pragma unroll
    for (int c = 0; c < QW; ++c) {
      const int qrow = q0 + 32 * c + n32;
      const int lim = p.causal ? min(kv_end - 1, p.q_offset + qrow) : kv_end - 1;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + 32 * st + 8 * (r >> 2) + 4 * g + (r & 3);
        if (key > lim) sacc[c][st][r] = kNegInf;
      }
    }
  };

  if constexpr (F32) {
    // ---------------------------------------------------------------------------------------
    // f32: both products on 32x32x2 f32 MFMA (MFMA-bound by a wide margin; no interleaving).
    // ---------------------------------------------------------------------------------------
    for (int it = t_begin; it < t_end; ++it) {
      const int buf = (it - t_begin) & 1;
      const LT* kl = k_lds + buf * KBUF;
      const LT* vl = v_lds + buf * VBUF;
      f32x16 sacc[QW][2];
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[0][st][r] = 0.f;
#pragma unroll
      for (int j = 0; j < D / 8; ++j)
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const f32x4 a =
              *reinterpret_cast<const f32x4*>(&kl[(32 * st + n32) * KROW + 8 * j + 4 * g]);
#pragma unroll
          for (int e = 0; e < 4; ++e) sacc[0][st] = mfma_f32(a[e], qf[0][4 * j + e], sacc[0][st]);
        }
      const int kb = it * BN;
      if (kb + BN > kv_end || (p.causal && kb + BN - 1 > p.q_offset + q0)) {
        mask_subtile(sacc, kb, 0);
        mask_subtile(sacc, kb, 1);
      }
      float mx = kNegInf;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; r += 2) mx = fmaxf(mx, fmaxf(sacc[0][st][r], sacc[0][st][r + 1]));
      const float mx_s = partner_max(mx) * sl2;
      if (__builtin_amdgcn_ballot_w64(mx_s > m_s[0] + kRescaleSlack) != 0) {
        const float m_new = fmaxf(m_s[0], mx_s);
        const float corr = fast_exp2(m_s[0] - ((m_new == kNegInf) ? 0.f : m_new));
        m_s[0] = m_new;
        l_run[0] *= corr;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) oacc[0][dt] *= corr;
      }
      const float mc = (m_s[0] == kNegInf) ? 0.f : m_s[0];
      float rs = 0.f;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = fast_exp2(__builtin_fmaf(sacc[0][st][r], sl2, -mc));
          sacc[0][st][r] = e;
          rs += e;
        }
      l_run[0] += rs;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(
                &vl[(32 * dt + n32) * VROW + 32 * st + 8 * j + 4 * g]);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              oacc[0][dt] = mfma_f32(a[e], sacc[0][st][4 * j + e], oacc[0][dt]);
          }
      if (it + 1 < t_end) {
        store_tile(buf ^ 1, buf ^ 1, it + 1);
        if (it + 2 < t_end) load_tile(it + 2);
      }
      __syncthreads();
    }
  } else {
    // ---------------------------------------------------------------------------------------
    // 16-bit: each 64-key tile runs as MFMA groups, each interleaved with VALU work that does
    // not depend on it, so the matrix pipe and the exp/FMA pipe run side by side:
    //   B  S^T(subtile 1)    || exp/pack/sum(0)   then the rare redo and rescale
    //   C  O^T += V^T P^T(0) || exp/pack/sum(1)   then the rare redo and rescale
    //      stage the next tile into LDS, barrier
    //   D  O^T += V^T P^T(1) and S^T(subtile 0) of the NEXT tile
    // so a tile never starts with its operand reads exposed.
    // Probabilities are packed to 16 bits as they are produced; row sums use v_dot2 on the
    // packed pairs, i.e. they sum exactly the weights the second product consumes.
    // ---------------------------------------------------------------------------------------
    // head_dim 64: fold scale*log2(e) into Q once (an f32 product rounded to the 16-bit type,
    // the same rounding the inputs already carry), so that scores leave the first product in
    // scaled log2 units. If a scaled element would not be finite in the 16-bit type, the wave
    // keeps Q as given and every score is multiplied instead (qmul).
    float qmul = 1.f;
    if constexpr (D != 64) {
      qmul = sl2;  // head_dim 128 keeps Q as given (the fold measured slower there)
    } else {
      constexpr uint32_t kInfBits = MODE == kBF16 ? 0x7f80u : 0x7c00u;
      u32x4 qs[QW][D / 16];
#pragma unroll
      for (int c = 0; c < QW; ++c)
#pragma unroll
        for (int s = 0; s < D / 16; ++s) {
          uint32_t w4[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t w = qf[c][s][k];
            w4[k] = pack2<MODE>(to_f32<MODE>(w & 0xffffu) * sl2, to_f32<MODE>(w >> 16) * sl2);
          }
          qs[c][s] = u32x4{w4[0], w4[1], w4[2], w4[3]};
        }
      // Only a factor above 1 can carry a finite element past the type's largest (below it the
      // product rounds to at most the input's magnitude; an inf or NaN input stays one either
      // way). Then bit 15 (31) of ovf ends up set when the low (high) half of some scaled pair
      // has an all-ones exponent: that half's exponent bits plus the increment that carries an
      // all-ones exponent into bit 15, OR-ed over the pairs (vector operations only).
      uint32_t ovf = 0u;
      if (sl2 > 1.f) {
        constexpr uint32_t kExp2 = kInfBits * 0x10001u;
        constexpr uint32_t kCarry2 = (0x8000u - kInfBits) * 0x10001u;
#pragma unroll
        for (int c = 0; c < QW; ++c)
#pragma unroll
          for (int s = 0; s < D / 16; ++s)
#pragma unroll
            for (int k = 0; k < 4; ++k) ovf |= (qs[c][s][k] & kExp2) + kCarry2;
      }
      if (__builtin_amdgcn_ballot_w64((ovf & 0x80008000u) != 0u) == 0) {
#pragma unroll
        for (int c = 0; c < QW; ++c)
#pragma unroll
          for (int s = 0; s < D / 16; ++s) qf[c][s] = qs[c][s];
      } else {
        qmul = sl2;
      }
    }
    bool fast = false;  // m_s is 0 for every row of the wave and qmul is 1
    constexpr std::integral_constant<bool, true> kFastTag{};
    constexpr std::integral_constant<bool, false> kSlowTag{};
    constexpr int NQK = (D / 16) * QW;        // MFMAs per subtile in S^T
    constexpr int NPV = 2 * (D / 32) * QW;    // MFMAs per subtile in O^T
    u32x4 pf[QW][4];   // packed P: pf[c][t] = keys 16t..16t+15 of the tile, B-operand order
    f32x16 sacc[QW][2];  // S^T of the tile's two 32-key subtiles, per column block

    // Transposing-read geometry: in each 16-lane group, lane j reads 4 elements of row
    // (r0 + j/4) at column (c0 + 4*(j%4)); lane j then holds column c0 + j of rows r0..r0+3.
    const int jt = lane & 15;
    const int tr_row = jt >> 2, tr_col = 4 * (jt & 3);
    const int half16 = 16 * ((lane >> 4) & 1);  // which 16 of the 32 M-rows this group covers
    // A operand of S^T for subtile st, contraction step s: K(key = 32st + n32, d = 16s + 8g + e).
    auto kfrag = [&](const LT* kl, int st, int s) -> u32x4 {
      if constexpr (KT) {
        // rows r and r + 4 share the chunk permutation (it depends on bit 1 of the row)
        const int r = 16 * s + 8 * g + tr_row;
        const int col = 32 * st + half16 + tr_col;
        const LT* base = &kl[r * KTROW + 8 * swz_kt(r, col >> 3) + (col & 7)];
        const u32x2 lo = lds_tr(base), hi = lds_tr(base + 4 * KTROW);
        return u32x4{lo.x, lo.y, hi.x, hi.y};
      } else {
        const int r = 32 * st + n32;
        return *reinterpret_cast<const u32x4*>(&kl[r * KROW + 8 * swz_kr(r, 2 * s + g)]);
      }
    };
    auto qk = [&](f32x16 (&sacc)[QW][2], const LT* kl, int st) {
#pragma unroll
      for (int s = 0; s < D / 16; ++s) {
        const u32x4 a = kfrag(kl, st, s);
#pragma unroll
        for (int c = 0; c < QW; ++c) sacc[c][st] = mfma16<MODE>(a, qf[c][s], sacc[c][st]);
      }
    };
    float rs_s[QW];    // this lane's sum of the weights of the subtile just exponentiated
    float corr_s[QW];  // accumulator rescale owed by the last redo of column block c
    // Weights of column block c, subtile st, from its 16 scores `sv` against the reference max
    // mc (scaled log2 units), packed to 16 bits into pf; returns this lane's sum of the packed
    // weights (v_dot2 on the packed pairs: exactly the weights the second product consumes).
    auto exps_c = [&](const f32x16& sv, int c, int st, float mc) -> float {
      float rs = 0.f;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        // Each packed pair is kept in a scalar and the operand tuple is assembled once: reads of
        // a vector lane through a reference were mis-lowered (every read saw lane 0).
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float e0 = fast_exp2(__builtin_fmaf(sv[8 * h2 + 2 * k], qmul, -mc));
          const float e1 = fast_exp2(__builtin_fmaf(sv[8 * h2 + 2 * k + 1], qmul, -mc));
          const uint32_t pk = pack2<MODE>(e0, e1);
          w[k] = pk;
          if constexpr (MODE == kBF16) {
            rs = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk),
                                                 bf16x2{(__bf16)1.f, (__bf16)1.f}, rs, false);
          } else {
            rs = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pk),
                                        f16x2{(_Float16)1.f, (_Float16)1.f}, rs, false);
          }
        }
        pf[c][2 * st + h2] = u32x4{w[0], w[1], w[2], w[3]};
      }
      return rs;
    };
    // Common path, inside the phase: weights against the current reference max m_s, with no max
    // taken. m_s starts either at 0 (FAST: every row max of the wave's first subtile lies in
    // [kFastMaxLo, kFastMaxHi] ([kFastMaxLoF16, kFastMaxHiF16] for f16 weights) and Q carries
    // the scale, so a weight is exp2 of the accumulator itself) or at the row max of the first
    // subtile; it is raised only in `settle`, when a subtile's weights leave the range below,
    // and the wave then leaves FAST for good. Either way the largest weight of a row is at least
    // 2^kFastMaxLo (bf16; 2^kFastMaxLoF16, a normal number, for f16), so nothing that matters
    // underflows. Work unit: pair k (scores 2k, 2k+1) of column block c of subtile st.
    constexpr int NPAIR = QW * 8;  // pairs per subtile
    uint32_t pw[QW][8];            // packed pairs of the subtile being exponentiated
    auto exp_pair = [&](int st, int pidx, auto fast_tag) {
      constexpr bool FAST = decltype(fast_tag)::value;
      const int c = pidx >> 3, k = pidx & 7;
      float x0 = sacc[c][st][2 * k], x1 = sacc[c][st][2 * k + 1];
      if constexpr (!FAST) {
        x0 = __builtin_fmaf(x0, qmul, -m_s[c]);
        x1 = __builtin_fmaf(x1, qmul, -m_s[c]);
      }
      const float e0 = fast_exp2(x0);
      const float e1 = fast_exp2(x1);
      const uint32_t pk = pack2<MODE>(e0, e1);
      pw[c][k] = pk;
      if constexpr (MODE == kBF16) {
        rs_s[c] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk),
                                                  bf16x2{(__bf16)1.f, (__bf16)1.f}, rs_s[c], false);
      } else {
        rs_s[c] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pk),
                                         f16x2{(_Float16)1.f, (_Float16)1.f}, rs_s[c], false);
      }
    };
    auto publish_pairs = [&](int st) {
#pragma unroll
      for (int c = 0; c < QW; ++c) {
        pf[c][2 * st] = u32x4{pw[c][0], pw[c][1], pw[c][2], pw[c][3]};
        pf[c][2 * st + 1] = u32x4{pw[c][4], pw[c][5], pw[c][6], pw[c][7]};
      }
    };
    // After the phase: a lane sum above kWeightSumBound (so some weight may be), or inf/NaN (a
    // score far above m_s, or m_s still -inf because every key so far was masked), makes the
    // whole wave redo that subtile against the subtile's exact row max (rare: with N(0,1)-like
    // scores only the first tile of a row can take it). Every weight therefore stays at most
    // 2^64, and the row sums and accumulators stay finite in f32 for any realistic key count.
    // The test compares bit patterns: the build assumes no NaNs, so a float compare could be
    // folded.
    // `redone`: the last settle redid a subtile, so the accumulator owes corr_s (wave-uniform).
    bool redone = false;
    auto settle = [&](int st) {
      // as unsigned bit patterns the lane sums (>= +0 when finite) compare above the bound
      // exactly when too large, inf or NaN (of either sign)
      uint32_t hi = 0u;
#pragma unroll
      for (int c = 0; c < QW; ++c) {
        corr_s[c] = 1.f;
        hi = max(hi, __float_as_uint(rs_s[c]));
      }
      redone = __builtin_amdgcn_ballot_w64(hi > __float_as_uint(kWeightSumBound)) != 0;
      if (redone) {
#pragma unroll
        for (int c = 0; c < QW; ++c) {
          const f32x16& sv = sacc[c][st];
          float mx = kNegInf;
#pragma unroll
          for (int r = 0; r < 16; r += 2) mx = fmaxf(mx, fmaxf(sv[r], sv[r + 1]));
          const float mx_s = partner_max(mx) * qmul;
          const float m_old = m_s[c];
          const float m_new = fmaxf(m_old, mx_s);
          corr_s[c] = (m_new == m_old) ? 1.f : fast_exp2(m_old - m_new);
          m_s[c] = m_new;
          rs_s[c] = exps_c(sv, c, st, (m_new == kNegInf) ? 0.f : m_new);
        }
        bool moved = false;
#pragma unroll
        for (int c = 0; c < QW; ++c) moved = moved || m_s[c] != 0.f;
        fast = fast && __builtin_amdgcn_ballot_w64(moved) == 0;
      }
#pragma unroll
      for (int c = 0; c < QW; ++c) l_run[c] = __builtin_fmaf(l_run[c], corr_s[c], rs_s[c]);
    };
    // Apply the rescale a redo left owing to the accumulator (whole wave, rare). Kept apart from
    // `settle`: inside its branch the accumulator would need copies on the common path.
    auto rescale = [&]() {
      if (redone) {
#pragma unroll
        for (int c = 0; c < QW; ++c)
#pragma unroll
          for (int dt = 0; dt < D / 32; ++dt) oacc[c][dt] *= corr_s[c];
      }
    };
    auto pv = [&](const LT* vl, int st) {
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int t = 2 * st + h2;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          // V tile [key][d]: A(d = 32dt + n32, keys 16t + 4g + e (e < 4), 16t + 8 + 4g + e - 4);
          // rows r and r + 8 share the chunk permutation
          const int r = 16 * t + 4 * g + tr_row;
          const int col = 32 * dt + half16 + tr_col;
          const LT* base = &vl[r * VROW + 8 * swz_v(r, col >> 3) + (col & 7)];
          const u32x2 a0 = lds_tr(base), a1 = lds_tr(base + 8 * VROW);
          const u32x4 a = {a0.x, a0.y, a1.x, a1.y};
#pragma unroll
          for (int c = 0; c < QW; ++c) oacc[c][dt] = mfma16<MODE>(a, pf[c][t], oacc[c][dt]);
        }
      }
    };

    // The two phases that hide the exp work. Each issues its fragment reads first, then its
    // MFMAs one at a time, each followed by an equal share of the exp/pack/sum pairs of the
    // other subtile, fenced so that the compiler keeps that order: one wave then keeps the
    // matrix pipe and the VALU busy together instead of issuing its MFMAs back to back.
    //   B: S^T(subtile 1) || exps(subtile 0);   C: O^T += V^T P^T(subtile 0) || exps(subtile 1)
    auto phase_b = [&](const LT* kl, auto fast_tag) {
      u32x4 a[D / 16];
#pragma unroll
      for (int s = 0; s < D / 16; ++s) a[s] = kfrag(kl, 1, s);
#pragma unroll
      for (int c = 0; c < QW; ++c) rs_s[c] = 0.f;
#pragma unroll
      for (int i = 0; i < NQK; ++i) {
        const int s = i / QW, c = i % QW;
#pragma unroll
        for (int j = i * NPAIR / NQK; j < (i + 1) * NPAIR / NQK; ++j) exp_pair(0, j, fast_tag);
        sacc[c][1] = mfma16<MODE>(a[s], qf[c][s], sacc[c][1]);
        __builtin_amdgcn_sched_barrier(0);
      }
      publish_pairs(0);
    };
    auto vfrag = [&](const LT* vl, int t, int dt) -> u32x4 {
      // V tile [key][d]: A(d = 32dt + n32, keys 16t + 4g + e (e < 4), 16t + 8 + 4g + e - 4);
      // rows r and r + 8 share the chunk permutation
      const int r = 16 * t + 4 * g + tr_row;
      const int col = 32 * dt + half16 + tr_col;
      const LT* base = &vl[r * VROW + 8 * swz_v(r, col >> 3) + (col & 7)];
      const u32x2 a0 = lds_tr(base), a1 = lds_tr(base + 8 * VROW);
      return u32x4{a0.x, a0.y, a1.x, a1.y};
    };
    auto phase_c = [&](const LT* vl, auto fast_tag) {
      u32x4 a[2][D / 32];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) a[h2][dt] = vfrag(vl, h2, dt);
#pragma unroll
      for (int c = 0; c < QW; ++c) rs_s[c] = 0.f;
#pragma unroll
      for (int i = 0; i < NPV; ++i) {
        const int h2 = i / (QW * (D / 32)), dt = (i / QW) % (D / 32), c = i % QW;
#pragma unroll
        for (int j = i * NPAIR / NPV; j < (i + 1) * NPAIR / NPV; ++j) exp_pair(1, j, fast_tag);
        oacc[c][dt] = mfma16<MODE>(a[h2][dt], pf[c][h2], oacc[c][dt]);
        __builtin_amdgcn_sched_barrier(0);
      }
      publish_pairs(1);
    };

    // wave-uniform, and made visibly so, so that masking is a scalar branch rather than
    // predicated selects on every tile
    const int q0_s = __builtin_amdgcn_readfirstlane(q0);
    auto need_mask_of = [&](int it) {
      // the tile index is taken into a scalar register first: the test is then scalar code
      const int kb = __builtin_amdgcn_readfirstlane(it) * BN;
      return kb + BN > kv_end || (p.causal && kb + BN - 1 > p.q_offset + q0_s);
    };
    auto zero_sub = [&](int st) {
#pragma unroll
      for (int c = 0; c < QW; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[c][st][r] = 0.f;
    };
    // S^T of the first tile's subtile 0 (later tiles get theirs in the previous iteration's D)
    if (t_begin < t_end) {
      zero_sub(0);
      qk(sacc, k_lds, 0);
      if (need_mask_of(t_begin)) mask_subtile(sacc, t_begin * BN, 0);
      // the reference max: this subtile's row max (-inf if all of it is masked), or 0 for the
      // whole wave when every such max is in the FAST window
      bool wide = false;
      constexpr float fast_lo = MODE == kF16 ? kFastMaxLoF16 : kFastMaxLo;
      constexpr float fast_hi = MODE == kF16 ? kFastMaxHiF16 : kFastMaxHi;
#pragma unroll
      for (int c = 0; c < QW; ++c) {
        float mx = kNegInf;
#pragma unroll
        for (int r = 0; r < 16; r += 2) mx = fmaxf(mx, fmaxf(sacc[c][0][r], sacc[c][0][r + 1]));
        m_s[c] = partner_max(mx) * qmul;
        wide = wide || !(m_s[c] >= fast_lo && m_s[c] <= fast_hi);
      }
      fast = D == 64 && qmul == 1.f && __builtin_amdgcn_ballot_w64(wide) == 0;
      if (fast) {
#pragma unroll
        for (int c = 0; c < QW; ++c) m_s[c] = 0.f;
      }
    }
#ifdef FFAI_STAMPS
    // phase times of this wave (diagnostic builds only; see attn_common.cuh)
    // (32-bit sums of the low halves of the counter: differences modulo 2^32 are exact for any
    // phase shorter than 2^32 ticks; fewer scalar registers than 64-bit ones)
    uint32_t st_acc[6] = {0, 0, 0, 0, 0, 0};
    uint32_t st_tiles = 0;
    stamp_now(7, stamp_clock());
    stamp_now(8, stamp_realtime());
#define FFAI_STAMP_AT(var) \
  __builtin_amdgcn_sched_barrier(0); \
  const uint32_t var = (uint32_t)stamp_clock(); \
  __builtin_amdgcn_sched_barrier(0)
#else
#define FFAI_STAMP_AT(var)
#endif
    for (int it = t_begin; it < t_end; ++it) {
      const LT* kl = k_lds + ((it - t_begin) % NBK) * KBUF;
      const LT* vl = v_lds + ((it - t_begin) % NBUF) * VBUF;
      const int kb = it * BN;
      const bool need_mask = need_mask_of(it);
      FFAI_STAMP_AT(st_t0);
      zero_sub(1);
      // B
      __builtin_amdgcn_sched_barrier(0);
      if (D == 64 && fast) phase_b(kl, kFastTag);
      else phase_b(kl, kSlowTag);
      __builtin_amdgcn_sched_barrier(0);
      FFAI_STAMP_AT(st_t1);
      settle(0);
      rescale();
      if (need_mask) mask_subtile(sacc, kb, 1);
      FFAI_STAMP_AT(st_t2);
      // C
      __builtin_amdgcn_sched_barrier(0);
      if (D == 64 && fast) phase_c(vl, kFastTag);
      else phase_c(vl, kSlowTag);
      __builtin_amdgcn_sched_barrier(0);
      FFAI_STAMP_AT(st_t3);
      settle(1);
      rescale();
      FFAI_STAMP_AT(st_t4);
      // Publish tile it + 1 (staged one iteration ago; the barrier also awaits its DMA), then
      // stage tile it + 2 into the buffer of tile it - 1, which every wave has finished with
      // once it passes this barrier.
      const bool more = it + 1 < t_end;
      const int nkbuf = (it + 1 - t_begin) % NBK;
      vm_wait_all();
      __syncthreads();
      FFAI_STAMP_AT(st_t5);
      if (it + 2 < t_end) stage_tile((it + 2 - t_begin) % NBK, (it + 2 - t_begin) % NBUF, it + 2);
      // D: O^T += V^T P^T for subtile 1, and S^T of the next tile's subtile 0
      pv(vl, 1);
      if (more) {
        zero_sub(0);
        qk(sacc, k_lds + nkbuf * KBUF, 0);
        if (need_mask_of(it + 1)) mask_subtile(sacc, (it + 1) * BN, 0);
      }
#ifdef FFAI_STAMPS
      FFAI_STAMP_AT(st_t6);
      st_acc[0] += st_t1 - st_t0;
      st_acc[1] += st_t2 - st_t1;
      st_acc[2] += st_t3 - st_t2;
      st_acc[3] += st_t4 - st_t3;
      st_acc[4] += st_t5 - st_t4;
      st_acc[5] += st_t6 - st_t5;
      ++st_tiles;
#endif
    }
#ifdef FFAI_STAMPS
#undef FFAI_STAMP_AT
    if (st_rec >= 0 && lane == 0) {
      const uint64_t st_c1 = stamp_clock(), st_r1 = stamp_realtime();
      const int64_t rec = st_rec;
#pragma unroll
      for (int k = 0; k < 6; ++k) stamp_put(p.stamps, rec + k, st_acc[k]);
      stamp_put(p.stamps, rec + 6, st_tiles);
      stamp_put(p.stamps, rec + 9, st_c1);
      stamp_put(p.stamps, rec + 10, st_r1);
    }
#endif
  }

#ifdef FFAI_STAMPS
  // exit times (recording workgroups, lane 0)
  auto stamp_exit = [&]() {
    if (st_rec >= 0 && lane == 0) {
      const uint64_t e1 = stamp_realtime();
      vm_wait_all();
      const uint64_t e2 = stamp_realtime();
      stamp_put(p.stamps, st_rec + 12, e1);
      stamp_put(p.stamps, st_rec + 13, e2);
    }
  };
#endif
  // ---- epilogue: oacc[c][dt][4r + e] <-> d = 32dt + 8r + 4g + e of query q0 + 32c + n32
  float l_tot[QW];
#pragma unroll
  for (int c = 0; c < QW; ++c) l_tot[c] = partner_sum(l_run[c]);
  if (split >= 0) {
    // A piece of a split item: publish this piece's partial (unnormalised O rows, and per row the
    // reference max m in scaled log2 units and the weight sum l), count the piece, and let the
    // item's last piece merge every piece's partial, in piece order, by log-sum-exp.
    const int S = p.n_split;
    const int j = rank - p.split_lo;  // the item's counter and partial slot
    const int64_t rows_all = (int64_t)(p.split_hi - p.split_lo) * S * BM;
    const int64_t o_floats = rows_all * D;
    // a buffer resource over exactly the partials (an access past them reads 0 / is dropped)
    const __amdgpu_buffer_rsrc_t ws_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        p.ws, (short)0, (int)((o_floats + rows_all * 2) * 4), kBufferWord3);
    // Partials are laid out lane-major, in the accumulators' register order: for piece
    // (item j, piece s), wave w and column block c, register group (dt, r) of all 64 lanes is
    // 1 KB of consecutive f32x4, so that every store and load instruction moves whole cache
    // lines; (m, l) follows per (piece, wave, c) as 32 f32x2 by query column. Only the kernel
    // itself reads them, and the last piece's thread (w, lane) merges exactly what thread
    // (w, lane) of every piece wrote.
    auto cw_of = [&](int s, int c) {  // (piece, wave, column block) index
      return ((int64_t)(j * S + s) * NW + wave) * QW + c;
    };
    // Device-scope (sc1) stores: each reaches the device's coherence point before it is
    // acknowledged, so the last piece reads it on whichever XCD that piece runs.
#pragma unroll
    for (int c = 0; c < QW; ++c) {
      if (q0 + 32 * c + n32 >= p.Tq) continue;
      const int64_t cw = cw_of(split, c);
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const f32x4 x = {oacc[c][dt][4 * r], oacc[c][dt][4 * r + 1], oacc[c][dt][4 * r + 2],
                           oacc[c][dt][4 * r + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(
              x, ws_rsrc, (int)((((cw * (D / 32) + dt) * 4 + r) * 64 + lane) * 16), 0,
              kDeviceScope);
        }
      if (g == 0)
        __builtin_amdgcn_raw_buffer_store_b64(f32x2{m_s[c], l_tot[c]}, ws_rsrc,
                                              (int)(o_floats * 4 + (cw * 32 + n32) * 8), 0,
                                              kDeviceScope);
    }
    // Ordering: every thread waits until its stores are acknowledged (vmcnt(0); a device-scope
    // store is acknowledged once visible at device scope), the barrier makes that true of the
    // whole workgroup, and only then does one thread add 1 to the item's counter (device-scope
    // atomic). The piece that reads S - 1 back is the item's last: every other piece's partial
    // was visible before its increment, which precedes this one in the counter's order, and this
    // workgroup's device-scope loads are issued after that increment returned. The last piece
    // sets the counter back to 0 for the next launch (no piece ever waits for another).
    // The flag lives in the tile buffers, which every wave has finished with at the barrier (a
    // __shared__ int of its own would push head_dim 128's 80 KB past two workgroups per CU).
    int* s_last = reinterpret_cast<int*>(k_lds);
    vm_wait_all();
    __syncthreads();
    if (tid == 0) {
      const int done =
          __hip_atomic_fetch_add(p.counters + j, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *s_last = (done == S - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!*s_last) return;  // (its exit is not stamped: doing so here spills registers)
    // Merge all S pieces (this one's too, as stored) in piece order, so that the result does not
    // depend on which piece finished last: KP pieces' loads in flight per round trip.
    constexpr int KP = 2;
#pragma unroll
    for (int c = 0; c < QW; ++c) {
      m_s[c] = kNegInf;
      l_tot[c] = 0.f;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[c][dt][r] = 0.f;
    }
#pragma unroll 1
    for (int s0 = 0; s0 < S; s0 += KP) {
      f32x2 ml[KP][QW];
      f32x4 xs[KP][QW][D / 32][4];
#pragma unroll
      for (int u = 0; u < KP; ++u) {
        const int s = min(s0 + u, S - 1);  // clamped; a slot past the last piece counts as empty
#pragma unroll
        for (int c = 0; c < QW; ++c) {
          const int64_t cw = cw_of(s, c);
          ml[u][c] = __builtin_amdgcn_raw_buffer_load_b64(
              ws_rsrc, (int)(o_floats * 4 + (cw * 32 + n32) * 8), 0, kDeviceScope);
#pragma unroll
          for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              xs[u][c][dt][r] = __builtin_amdgcn_raw_buffer_load_b128(
                  ws_rsrc, (int)((((cw * (D / 32) + dt) * 4 + r) * 64 + lane) * 16), 0,
                  kDeviceScope);
        }
      }
#pragma unroll
      for (int u = 0; u < KP; ++u) {
        const bool real = s0 + u < S;  // wave-uniform
#pragma unroll
        for (int c = 0; c < QW; ++c) {
          const float m = real ? ml[u][c][0] : kNegInf;
          const float m_new = fmaxf(m_s[c], m);
          const float mc = (m_new == kNegInf) ? 0.f : m_new;  // both empty: weights 0, not NaN
          const float c_old = fast_exp2(m_s[c] - mc);          // 0 while m_s is -inf
          const float c_new = fast_exp2(m - mc);               // 0 for an empty piece
          l_tot[c] = l_tot[c] * c_old + (real ? ml[u][c][1] : 0.f) * c_new;
#pragma unroll
          for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
              for (int e = 0; e < 4; ++e)
                oacc[c][dt][4 * r + e] =
                    oacc[c][dt][4 * r + e] * c_old + (real ? xs[u][c][dt][r][e] : 0.f) * c_new;
          m_s[c] = m_new;
        }
      }
    }
    if (tid == 0) __hip_atomic_store(p.counters + j, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if constexpr (OUTT != kF32 && D == 64) {
    if (p.o_pair) {
      // Lane (n32, g) holds d = 32dt + 8r + 4g .. +3 of its row; its partner (lane ^ 32, the same
      // row) the other half of each 8-element run. One v_permlane32_swap per packed word hands
      // the low lanes whole runs r = 0, 2 and the high lanes runs 1, 3: half the store
      // instructions, each 16 bytes per lane. (Both lanes of a pair take the row test's branch
      // alike, so every swap pairs two active lanes.)
#pragma unroll
      for (int c = 0; c < QW; ++c) {
        const int qrow = q0 + 32 * c + n32;
        if (qrow >= p.Tq) continue;
        const float inv = l_tot[c] > 0.f ? 1.f / l_tot[c] : 0.f;
        store_t<OUTT>* op = reinterpret_cast<store_t<OUTT>*>(p.o) + b * p.o_sb + h * p.o_sh +
                            (int64_t)qrow * p.o_st;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
          for (int rp = 0; rp < 4; rp += 2) {
            const f32x16& a = oacc[c][dt];
            const uint32_t x0 = pack2<OUTT>(a[4 * rp] * inv, a[4 * rp + 1] * inv);
            const uint32_t x1 = pack2<OUTT>(a[4 * rp + 2] * inv, a[4 * rp + 3] * inv);
            const uint32_t y0 = pack2<OUTT>(a[4 * rp + 4] * inv, a[4 * rp + 5] * inv);
            const uint32_t y1 = pack2<OUTT>(a[4 * rp + 6] * inv, a[4 * rp + 7] * inv);
            // low lanes: {own x, partner's x} = run rp; high lanes: {partner's y, own y} = run
            // rp + 1
            const auto s0 = __builtin_amdgcn_permlane32_swap(x0, y0, false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(x1, y1, false, false);
            *reinterpret_cast<u32x4*>(op + 32 * dt + 8 * (rp + g)) =
                u32x4{s0[0], s1[0], s0[1], s1[1]};
          }
      }
#ifdef FFAI_STAMPS
      stamp_exit();
#endif
      return;
    }
  }
#pragma unroll
  for (int c = 0; c < QW; ++c) {
    const int qrow = q0 + 32 * c + n32;
    if (qrow >= p.Tq) continue;
    const float inv = l_tot[c] > 0.f ? 1.f / l_tot[c] : 0.f;
    store_t<OUTT>* op = reinterpret_cast<store_t<OUTT>*>(p.o) + b * p.o_sb + h * p.o_sh +
                        (int64_t)qrow * p.o_st;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const f32x4 x = {oacc[c][dt][4 * r] * inv, oacc[c][dt][4 * r + 1] * inv,
                         oacc[c][dt][4 * r + 2] * inv, oacc[c][dt][4 * r + 3] * inv};
        if (aligned) st4<OUTT, true>(op + 32 * dt + 8 * r + 4 * g, x);
        else st4<OUTT, false>(op + 32 * dt + 8 * r + 4 * g, x);
      }
  }
#ifdef FFAI_STAMPS
  stamp_exit();
#endif
}

}  // namespace
}  // namespace ffai
