// gfx950 fused attention, the encoder launch shape on 16x16x32 MFMA: 16-bit Q/K/V, head_dim 64,
// four waves x 64 query rows per workgroup, two workgroups per CU. Same contract as fwd_kernel
// (attn_kernels.cuh) for this shape: work mapping and dispatch sections, key-split pieces merged
// in the launch, K given transposed or as rows, ragged and causal masks, f32 or 16-bit output.
//
// Design:
//   * Keys stream in 64-key tiles through a three-buffer LDS ring (whole tiles by DMA, tails and
//     misaligned launches through registers), one workgroup barrier per tile.
//   * S^T = K Q^T per 16-key UNIT on v_mfma_f32_16x16x32: 4 column blocks of 16 queries x 2
//     head-dim steps of 32 = 8 MFMAs; lane l holds query column l % 16 of each block and keys
//     4 (l / 16) .. +3 of the unit (16 f32 per lane per unit).
//   * O^T += V^T P^T per 32-key CHUNK (two units): 4 head-dim blocks of 16 x 4 column blocks =
//     16 MFMAs. The B operand is the two units' packed weights exactly as they lie in the lanes
//     (keys 4g .. 4g + 3 of each unit for lane group g), and V is read in that key order by two
//     transposing LDS reads, so P never goes through LDS.
//   * Software pipeline, one phase per unit: phase i runs S^T of unit i + 1 and half of the PV of
//     the chunk finished two units before (8 + 8 MFMAs), interleaved with unit i's exps, packs
//     and row sums. Every phase keeps both the matrix pipe and the VALU busy.
//   * Softmax as in fwd_kernel's 16-bit path: base 2 with v_exp_f32, scale folded into Q, a fixed
//     reference max per row (0 in the FAST window), row sums by v_dot2 on the packed weights, and
//     a settle check per chunk that redoes the chunk against its exact max when a weight could
//     exceed 2^64 (or overflowed).
#pragma once

#include "attn_common.cuh"

namespace ffai {
namespace {

template <int MODE, int OUTT, bool KT>
__global__ __launch_bounds__(256, 2) void fwd16_kernel(FwdParams p) {
  static_assert(MODE == kBF16 || MODE == kF16, "16-bit inputs");
  constexpr int D = 64;
  constexpr int NW = 4;
  constexpr int NT = NW * 64;
  constexpr int BM = NW * 64;  // query rows per workgroup
  constexpr int NC = 4;        // 16-query column blocks per wave
  constexpr int NBUF = 3;
  constexpr int TILE = BN * D;  // 16-bit elements per K or V tile
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[NBUF * TILE];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[NBUF * TILE];

  // ---- which work (an item, or one piece of a split item) this workgroup computes
  const int hw = wg_id_x();
  int work;
  const int xs = p.xcd_shift, xm = (1 << xs) - 1;
  if (hw < p.sec1_wgs) {
    work = p.xcd_remap ? (hw & xm) * (p.sec1_wgs >> xs) + (hw >> xs) : hw;
    if (work >= p.sec1_work) return;
  } else {
    const int x = hw - p.sec1_wgs, n = ((p.n_work - p.sec1_work + xm) >> xs) << xs;
    work = p.sec1_work + (p.xcd_remap ? (x & xm) * (n >> xs) + (x >> xs) : x);
    if (work >= p.n_work) return;
  }
  const int n_pieces = (p.split_hi - p.split_lo) * p.n_split;
  int rank, split = -1;
  if (work < p.split_lo) {
    rank = work;
  } else if (work < p.split_lo + n_pieces) {
    rank = p.split_lo + (work - p.split_lo) / p.n_split;
    split = (work - p.split_lo) % p.n_split;
  } else {
    rank = work - n_pieces + (p.split_hi - p.split_lo);
  }
  int qb, bh;
  if (p.causal) {
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
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15;  // query column within a 16-block; key / d row of an A fragment
  const int g = lane >> 4;    // lane group: contraction elements 8g .., accumulator rows 4g ..
  const int q0 = qb * BM + wave * 64;

  int kv_end = p.Tk;
  if (p.kv_lens) kv_end = min(kv_end, max(0, p.kv_lens[b]));
  kv_end = __builtin_amdgcn_readfirstlane(kv_end);
  int kv_blk = kv_end;
  if (p.causal) kv_blk = min(kv_end, max(0, p.q_offset + min(qb * BM + BM, p.Tq)));
  const int n_tiles = (kv_blk + BN - 1) / BN;
  const int tps = split < 0 ? n_tiles : (n_tiles + p.n_split - 1) / p.n_split;
  const int t_begin = split < 0 ? 0 : split * tps;
  const int t_end = min(n_tiles, t_begin + tps);
  const bool aligned = p.aligned != 0;

  const uint16_t* qp = reinterpret_cast<const uint16_t*>(p.q) + b * p.q_sb + h * p.q_sh;
  const uint16_t* kp = reinterpret_cast<const uint16_t*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const uint16_t* vp = reinterpret_cast<const uint16_t*>(p.v) + b * p.v_sb + hk * p.v_sh;
  const char* kp_dma = uniform_ptr(reinterpret_cast<const char*>(kp));
  const char* vp_dma = uniform_ptr(reinterpret_cast<const char*>(vp));

  // ---- Q fragments (B operand of S^T): block c, step s: row q0 + 16c + n16, d = 32s + 8g .. +7
  u32x4 qf[NC][2];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int row = q0 + 16 * c + n16;
    const bool ok = row < p.Tq;
    const uint16_t* qr = qp + (int64_t)min(row, p.Tq - 1) * p.q_st;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 x = aligned ? ld16(qr + 32 * s + 8 * g) : ld8h_elem(qr + 32 * s + 8 * g);
      qf[c][s] = ok ? x : u32x4{0u, 0u, 0u, 0u};
    }
  }

  // ---- LDS layouts, 16-byte chunks XOR-permuted per row (an XOR: its own inverse). A
  // transposing read covers, per 16 lanes, 4 rows x 32 bytes; the permutations put the rows
  // that one 32-lane pass reads on distinct banks.
  //   K^T [d][key] (128-byte rows): 32-byte segments swapped by bits 1 and 3 of the row (rows r
  //   and r + 4 share it);  V [key][d]: by bits 1-2 (rows r and r + 16 share it);
  //   K [key][d]: 16-byte chunks by bits 1-3 (the 16-byte fragment reads of 16 rows).
  auto swz_kt = [](int r, int c) { return c ^ (2 * (((r >> 1) & 1) | ((r >> 2) & 2))); };
  auto swz_v = [](int r, int c) { return c ^ (2 * ((r >> 1) & 3)); };
  auto swz_kr = [](int r, int c) { return c ^ ((r >> 1) & 7); };

  // ---- staging through registers (tail tiles, misaligned launches): keys clamped to the last
  // valid one, rows past it zeroed when stored
  constexpr int UNITS = TILE / 8;      // 16-byte units per tile
  constexpr int PER = UNITS / NT;      // per thread: 2
  u32x4 kreg[PER], vreg[PER];
  auto load_tile = [&](int it) {
    const int kb = it * BN;
    const int klast = kv_end - 1;
    const bool full = aligned && (kb + BN <= kv_end);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      if constexpr (KT) {
        const int d = u / (BN / 8), kc = u % (BN / 8);
        const int key0 = kb + 8 * kc;
        const uint16_t* row = kp + (int64_t)d * p.k_st;
        if (full) {
          const u32x2 lo = ld8(row + key0), hi = ld8(row + key0 + 4);
          kreg[i] = u32x4{lo.x, lo.y, hi.x, hi.y};
        } else {
          uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t y = row[min(key0 + e, klast)];
            w[e >> 1] |= (key0 + e <= klast ? y : 0u) << (16 * (e & 1));
          }
          kreg[i] = u32x4{w[0], w[1], w[2], w[3]};
        }
      } else {
        const int key = kb + u / (D / 8), c = u % (D / 8);
        const uint16_t* src = kp + (int64_t)min(key, klast) * p.k_st + 8 * c;
        kreg[i] = aligned ? ld16(src) : ld8h_elem(src);
      }
      const int key = kb + u / (D / 8), c = u % (D / 8);
      const uint16_t* src = vp + (int64_t)min(key, klast) * p.v_st + 8 * c;
      vreg[i] = aligned ? ld16(src) : ld8h_elem(src);
    }
  };
  auto store_tile = [&](int buf, int it) {
    uint16_t* kl = k_lds + buf * TILE;
    uint16_t* vl = v_lds + buf * TILE;
    const int kb = it * BN;
    const int klast = kv_end - 1;
    const bool full = kb + BN <= kv_end;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      if constexpr (KT) {
        const int d = u / (BN / 8), kc = u % (BN / 8);
        *reinterpret_cast<u32x4*>(&kl[d * BN + 8 * swz_kt(d, kc)]) = kreg[i];
      } else {
        const int key = u / (D / 8), c = u % (D / 8);
        *reinterpret_cast<u32x4*>(&kl[key * D + 8 * swz_kr(key, c)]) =
            (full || kb + key <= klast) ? kreg[i] : u32x4{0u, 0u, 0u, 0u};
      }
      const int key = u / (D / 8), c = u % (D / 8);
      *reinterpret_cast<u32x4*>(&vl[key * D + 8 * swz_v(key, c)]) =
          (full || kb + key <= klast) ? vreg[i] : u32x4{0u, 0u, 0u, 0u};
    }
  };
  // whole tiles of an aligned launch: global -> LDS by DMA, 1 KB blocks, lane offsets computed
  // once (the swizzle included), the wave-uniform tile base in scalar registers
  constexpr int BLK = TILE / 512;  // 1 KB blocks per tile: 8, two per wave
  uint32_t dma_koff[BLK / NW], dma_voff[BLK / NW];
#pragma unroll
  for (int j = 0; j < BLK / NW; ++j) {
    const int L = (j * NW + wave) * 64 + lane;
    const int r = L / 8, pc = L % 8;
    dma_koff[j] = (uint32_t)(2 * ((int64_t)r * p.k_st + 8 * (KT ? swz_kt(r, pc) : swz_kr(r, pc))));
    dma_voff[j] = (uint32_t)(2 * ((int64_t)r * p.v_st + 8 * swz_v(r, pc)));
  }
  auto dma_tile = [&](int buf, int it) {
    const uint32_t kl = lds_addr(k_lds + buf * TILE);
    const uint32_t vl = lds_addr(v_lds + buf * TILE);
    const int64_t kb = (int64_t)__builtin_amdgcn_readfirstlane(it) * BN;
    const char* kbase = uniform_ptr(kp_dma) + 2 * (KT ? kb : kb * p.k_st);
    const char* vbase = uniform_ptr(vp_dma) + 2 * kb * p.v_st;
#pragma unroll
    for (int j = 0; j < BLK / NW; ++j)
      lds_dma16_sbase(kbase, dma_koff[j], kl + (j * NW + wave) * 1024);
#pragma unroll
    for (int j = 0; j < BLK / NW; ++j)
      lds_dma16_sbase(vbase, dma_voff[j], vl + (j * NW + wave) * 1024);
  };
  auto stage_tile = [&](int buf, int it) {
    if (p.dma && it * BN + BN <= kv_end) {
      dma_tile(buf, it);
    } else {
      load_tile(it);
      store_tile(buf, it);
    }
  };

  // ---- state
  f32x4 oacc[NC][4];  // O^T block (c, db): query column 16c + n16, d = 16db + 4g .. +3
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int db = 0; db < 4; ++db) oacc[c][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_s[NC], l_run[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    m_s[c] = kNegInf;
    l_run[c] = 0.f;
  }
  const float sl2 = p.scale_log2;

  if (t_begin < t_end) {
    stage_tile(0, t_begin);
    if (t_begin + 1 < t_end) stage_tile(1, t_begin + 1);
    vm_wait_all();
  }
  __syncthreads();

  // scale * log2(e) folded into Q (f32 product rounded to the 16-bit type), unless a folded
  // element would not be finite: then Q stays as given and every score is multiplied (qmul)
  float qmul = 1.f;
  {
    constexpr uint32_t kInfBits = MODE == kBF16 ? 0x7f80u : 0x7c00u;
    u32x4 qs[NC][2];
    // Bit 15 (31) of ovf ends up set when the low (high) half of some scaled pair has an all-ones
    // exponent (inf or NaN): that half's exponent bits plus the increment that carries an
    // all-ones exponent into bit 15, OR-ed over the pairs; vector operations only, no chain of
    // compares into scalar registers.
    constexpr uint32_t kExp2 = kInfBits * 0x10001u;
    constexpr uint32_t kCarry2 = (0x8000u - kInfBits) * 0x10001u;
    uint32_t ovf = 0u;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        uint32_t w4[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t w = qf[c][s][k];
          const uint32_t y =
              pack2<MODE>(to_f32<MODE>(w & 0xffffu) * sl2, to_f32<MODE>(w >> 16) * sl2);
          ovf |= (y & kExp2) + kCarry2;
          w4[k] = y;
        }
        qs[c][s] = u32x4{w4[0], w4[1], w4[2], w4[3]};
      }
    if (__builtin_amdgcn_ballot_w64((ovf & 0x80008000u) != 0u) == 0) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int s = 0; s < 2; ++s) qf[c][s] = qs[c][s];
    } else {
      qmul = sl2;
    }
  }

  // ---- fragments. Transposing-read geometry: in each 16-lane group, lane j reads 4 elements
  // of row r0 + j / 4 at column c0 + 4 (j % 4) and then holds column c0 + j of rows r0 .. r0 + 3.
  const int tr_row = n16 >> 2, tr_col = 4 * (n16 & 3);
  // A operand of S^T for unit u, step s: key 16u + n16, d = 32s + 8g .. +7
  auto kfrag = [&](const uint16_t* kl, int u, int s) -> u32x4 {
    if constexpr (KT) {
      const int r = 32 * s + 8 * g + tr_row;  // rows r and r + 4 share the permutation
      const int col = 16 * u + tr_col;
      const uint16_t* base = &kl[r * BN + 8 * swz_kt(r, col >> 3) + (col & 7)];
      const u32x2 lo = lds_tr(base), hi = lds_tr(base + 4 * BN);
      return u32x4{lo.x, lo.y, hi.x, hi.y};
    } else {
      const int r = 16 * u + n16;
      return *reinterpret_cast<const u32x4*>(&kl[r * D + 8 * swz_kr(r, 4 * s + g)]);
    }
  };
  // A operand of O^T for chunk ch (units 2ch, 2ch + 1), head-dim block db: d = 16db + n16,
  // keys 32ch + 4g + e (e < 4) and 32ch + 16 + 4g + e - 4 (e >= 4)
  auto vfrag = [&](const uint16_t* vl, int ch, int db) -> u32x4 {
    const int r = 32 * ch + 4 * g + tr_row;  // rows r and r + 16 share the permutation
    const int col = 16 * db + tr_col;
    const uint16_t* base = &vl[r * D + 8 * swz_v(r, col >> 3) + (col & 7)];
    const u32x2 a0 = lds_tr(base), a1 = lds_tr(base + 16 * D);
    return u32x4{a0.x, a0.y, a1.x, a1.y};
  };

  // scores of the units in flight: sacc[u % 4][c] <-> keys kb + 16u + 4g + r of column 16c + n16
  f32x4 sacc[4][NC];
  // packed weights per chunk parity: pf[ch % 2][c] = {unit 2ch keys (0,1), (2,3), unit 2ch + 1
  // keys (0,1), (2,3)}, the B operand of the chunk's PV
  u32x4 pf[2][NC];
  float rs[2][NC];  // this lane's sum of the packed weights of the chunk's two units
  bool fast = false;

  const int q0_s = __builtin_amdgcn_readfirstlane(q0);
  auto need_mask_of = [&](int unit_key0) {  // unit_key0: the unit's first key (wave-uniform)
    const int k0 = __builtin_amdgcn_readfirstlane(unit_key0);
    return k0 + 16 > kv_end || (p.causal && k0 + 15 > p.q_offset + q0_s);
  };
  auto mask_unit = [&](f32x4 (&sv)[NC], int unit_key0) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int qrow = q0 + 16 * c + n16;
      const int lim = p.causal ? min(kv_end - 1, p.q_offset + qrow) : kv_end - 1;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (unit_key0 + 4 * g + r > lim) sv[c][r] = kNegInf;
    }
  };
  auto zero_unit = [&](f32x4 (&sv)[NC]) {
#pragma unroll
    for (int c = 0; c < NC; ++c) sv[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  // one exp pair: scores r = 2k, 2k + 1 of column block c -> a packed pair, summed into rs
  auto exp_pair = [&](const f32x4 (&sv)[NC], int c, int k, float mc, bool slow) -> uint32_t {
    float x0 = sv[c][2 * k], x1 = sv[c][2 * k + 1];
    if (slow) {
      x0 = __builtin_fmaf(x0, qmul, -mc);
      x1 = __builtin_fmaf(x1, qmul, -mc);
    }
    return pack2<MODE>(fast_exp2(x0), fast_exp2(x1));
  };
  auto dot_ones = [&](uint32_t pk, float acc) -> float {
    if constexpr (MODE == kBF16) {
      return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk),
                                             bf16x2{(__bf16)1.f, (__bf16)1.f}, acc, false);
    } else {
      return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pk),
                                    f16x2{(_Float16)1.f, (_Float16)1.f}, acc, false);
    }
  };

  // The first tile's phases 0 and 1 run the PV of a "previous chunk" that does not exist: its
  // weights are zero and its V buffer (the ring's third, staged only at the first barrier) is
  // zeroed here, so they add exact zeros (0 x NaN from stale LDS would not be).
#pragma unroll
  for (int c = 0; c < NC; ++c) pf[1][c] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < TILE / 8 / NT; ++i)
    *reinterpret_cast<u32x4*>(&v_lds[2 * TILE + 8 * (tid + i * NT)]) = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();

  // S^T of the first tile's unit 0, its mask, and the reference max
  if (t_begin < t_end) {
    zero_unit(sacc[0]);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 a = kfrag(k_lds, 0, s);
#pragma unroll
      for (int c = 0; c < NC; ++c) sacc[0][c] = mfma16x16<MODE>(a, qf[c][s], sacc[0][c]);
    }
    if (need_mask_of(t_begin * BN)) mask_unit(sacc[0], t_begin * BN);
    bool wide = false;
    constexpr float fast_lo = MODE == kF16 ? kFastMaxLoF16 : kFastMaxLo;
    constexpr float fast_hi = MODE == kF16 ? kFastMaxHiF16 : kFastMaxHi;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float mx = fmaxf(fmaxf(sacc[0][c][0], sacc[0][c][1]), fmaxf(sacc[0][c][2], sacc[0][c][3]));
      m_s[c] = quad_max(mx) * qmul;
      wide = wide || !(m_s[c] >= fast_lo && m_s[c] <= fast_hi);
    }
    fast = qmul == 1.f && __builtin_amdgcn_ballot_w64(wide) == 0;
    if (fast) {
#pragma unroll
      for (int c = 0; c < NC; ++c) m_s[c] = 0.f;
    }
  }

  // The settle check of a chunk, at the end of its second unit's phase: a lane sum above 2^64
  // (or inf / NaN: a score far above the reference max, or a reference max still -inf) redoes
  // both units against the chunk's exact max, rescales the accumulator owed and leaves the
  // wave's FAST window for good if a max moved; then the row sums are added. The two units'
  // scores are recomputed from K (still in LDS) and Q rather than kept: the redo is rare, and
  // the registers are better spent on the common path.
  auto settle = [&](int par, const uint16_t* kl, int key0, int su0) {
    uint32_t hi = 0u;
#pragma unroll
    for (int c = 0; c < NC; ++c) hi = max(hi, __float_as_uint(rs[par][c]));
    if (__builtin_amdgcn_ballot_w64(hi > __float_as_uint(kWeightSumBound)) != 0) {
      f32x4 sv[2][NC];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        zero_unit(sv[h2]);
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const u32x4 a = kfrag(kl, su0 + h2, st);
#pragma unroll
          for (int c = 0; c < NC; ++c) sv[h2][c] = mfma16x16<MODE>(a, qf[c][st], sv[h2][c]);
        }
        if (need_mask_of(key0 + 16 * h2)) mask_unit(sv[h2], key0 + 16 * h2);
      }
      bool moved = false;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float mx = kNegInf;
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, fmaxf(sv[0][c][r], sv[1][c][r]));
        const float mx_s = quad_max(mx) * qmul;
        const float m_old = m_s[c];
        const float m_new = fmaxf(m_old, mx_s);
        const float corr = (m_new == m_old) ? 1.f : fast_exp2(m_old - m_new);
        m_s[c] = m_new;
        moved = moved || m_new != 0.f;
        const float mc = (m_new == kNegInf) ? 0.f : m_new;
        float sum = 0.f;
        uint32_t w4[4];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          w4[k] = exp_pair(sv[0], c, k, mc, true);
          w4[2 + k] = exp_pair(sv[1], c, k, mc, true);
          sum = dot_ones(w4[k], dot_ones(w4[2 + k], sum));
        }
        pf[par][c] = u32x4{w4[0], w4[1], w4[2], w4[3]};
        rs[par][c] = sum;
        l_run[c] *= corr;
#pragma unroll
        for (int db = 0; db < 4; ++db) oacc[c][db] *= corr;
      }
      fast = fast && __builtin_amdgcn_ballot_w64(moved) == 0;
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) l_run[c] += rs[par][c];
  };

  // The tile loop, one phase per unit U of the tile: unit U's exps (chunk U / 2 of the tile,
  // packed-weight parity U / 2), interleaved with S^T of the next unit (U + 1, or the next tile's
  // unit 0: on the last tile it is computed and never used) and half U % 2 of the PV of the
  // chunk before (U = 2, 3: the tile's chunk 0; U = 0, 1: the previous tile's chunk 1, zeros on
  // the first tile). The chunk's settle check ends its second phase; the tile's barrier follows
  // phase 1.
  for (int it = t_begin; it < t_end; ++it) {
    const int j = it - t_begin;
    const uint16_t* kl = k_lds + (j % NBUF) * TILE;
    const uint16_t* vl = v_lds + (j % NBUF) * TILE;
    const uint16_t* vl_prev = v_lds + ((j + NBUF - 1) % NBUF) * TILE;  // tile it - 1's V
    const uint16_t* kl_next = k_lds + ((j + 1) % NBUF) * TILE;         // tile it + 1's K
    const int kb = it * BN;
#pragma unroll
    for (int U = 0; U < 4; ++U) {
      const int par = U >> 1;            // this unit's chunk parity
      const bool second = (U & 1) != 0;  // the chunk's second unit
      const int pv_par = par ^ 1;
      const uint16_t* pv_vl = U >= 2 ? vl : vl_prev;
      const int pv_ch = U >= 2 ? 0 : 1;
      const int H = U & 1;               // PV head-dim blocks 2H, 2H + 1
      const uint16_t* s_kl = U < 3 ? kl : kl_next;
      const int s_u = (U + 1) & 3;
      if (need_mask_of(kb + 16 * U)) mask_unit(sacc[U], kb + 16 * U);
      if (!fast) {
        // outside the FAST window the exponent is s * qmul - m (one FMA per score, before the
        // phase, so that the phase itself is one code path)
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int r = 0; r < 4; ++r) sacc[U][c][r] = __builtin_fmaf(sacc[U][c][r], qmul, -m_s[c]);
      }
      u32x4 ka[2], va[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) ka[s] = kfrag(s_kl, s_u, s);
#pragma unroll
      for (int d2 = 0; d2 < 2; ++d2) va[d2] = vfrag(pv_vl, pv_ch, 2 * H + d2);
      zero_unit(sacc[s_u]);
      if (!second) {
#pragma unroll
        for (int c = 0; c < NC; ++c) rs[par][c] = 0.f;
      }
      uint32_t w[NC][2];
      // 16 MFMA slots: 0..7 PV (block 2H + slot / 4, column slot % 4), 8..15 S^T (step
      // (slot - 8) / 4, column slot % 4); exp pair k of column c before slot 2 (2c + k)
      {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int slot = 0; slot < 16; ++slot) {
          if ((slot & 1) == 0) {
            const int c = slot >> 2, k = (slot >> 1) & 1;
            w[c][k] = exp_pair(sacc[U], c, k, 0.f, false);
            rs[par][c] = dot_ones(w[c][k], rs[par][c]);
          }
          if (slot < 8) {
            const int d2 = slot >> 2, c = slot & 3;
            oacc[c][2 * H + d2] = mfma16x16<MODE>(va[d2], pf[pv_par][c], oacc[c][2 * H + d2]);
          } else {
            const int st = (slot - 8) >> 2, c = slot & 3;
            sacc[s_u][c] = mfma16x16<MODE>(ka[st], qf[c][st], sacc[s_u][c]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // the unit's packed weights into its chunk's B operand
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (!second) {
          pf[par][c][0] = w[c][0];
          pf[par][c][1] = w[c][1];
        } else {
          pf[par][c][2] = w[c][0];
          pf[par][c][3] = w[c][1];
        }
      }
      if (second) settle(par, kl, kb + 16 * (U - 1), U - 1);
      if (U == 1) {
        // publish tile it + 1 (staged one tile ago), then stage tile it + 2 into the buffer of
        // tile it - 1, which every wave finished with (its V's last PV ran in phase 1)
        vm_wait_all();
        __syncthreads();
        if (it + 2 < t_end) stage_tile((j + 2) % NBUF, it + 2);
      }
    }
  }
  // the last chunk's PV (both halves), after the loop
  if (t_begin < t_end) {
    const uint16_t* vl = v_lds + ((t_end - 1 - t_begin) % NBUF) * TILE;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const u32x4 a = vfrag(vl, 1, db);
#pragma unroll
      for (int c = 0; c < NC; ++c) oacc[c][db] = mfma16x16<MODE>(a, pf[1][c], oacc[c][db]);
    }
  }

  // ---- epilogue: oacc[c][db][r] <-> d = 16db + 4g + r of query q0 + 16c + n16
  float l_tot[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) l_tot[c] = quad_sum(l_run[c]);
  if (split >= 0) {
    // a piece of a split item: publish the partial (lane-major, in the accumulators' register
    // order: per (piece, wave, column block, head-dim block) 64 lanes x f32x4 = 1 KB; then per
    // (piece, wave, column block) 16 (m, l) pairs), count the piece, the item's last piece merges
    const int S = p.n_split;
    const int jj = rank - p.split_lo;
    const int64_t rows_all = (int64_t)(p.split_hi - p.split_lo) * S * BM;
    const int64_t o_floats = rows_all * D;
    const __amdgpu_buffer_rsrc_t ws_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        p.ws, (short)0, (int)((o_floats + rows_all * 2) * 4), kBufferWord3);
    auto cw_of = [&](int s, int c) { return ((int64_t)(jj * S + s) * NW + wave) * NC + c; };
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (q0 + 16 * c + n16 >= p.Tq) continue;
      const int64_t cw = cw_of(split, c);
#pragma unroll
      for (int db = 0; db < 4; ++db)
        __builtin_amdgcn_raw_buffer_store_b128(oacc[c][db], ws_rsrc,
                                               (int)(((cw * 4 + db) * 64 + lane) * 16), 0,
                                               kDeviceScope);
      if (g == 0)
        __builtin_amdgcn_raw_buffer_store_b64(f32x2{m_s[c], l_tot[c]}, ws_rsrc,
                                              (int)(o_floats * 4 + (cw * 16 + n16) * 8), 0,
                                              kDeviceScope);
    }
    int* s_last = reinterpret_cast<int*>(k_lds);
    vm_wait_all();
    __syncthreads();
    if (tid == 0) {
      const int done =
          __hip_atomic_fetch_add(p.counters + jj, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *s_last = (done == S - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!*s_last) return;
    constexpr int KP = 2;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      m_s[c] = kNegInf;
      l_tot[c] = 0.f;
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[c][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll 1
    for (int s0 = 0; s0 < S; s0 += KP) {
      f32x2 ml[KP][NC];
      f32x4 xs4[KP][NC][4];
#pragma unroll
      for (int u = 0; u < KP; ++u) {
        const int s = min(s0 + u, S - 1);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int64_t cw = cw_of(s, c);
          ml[u][c] = __builtin_amdgcn_raw_buffer_load_b64(
              ws_rsrc, (int)(o_floats * 4 + (cw * 16 + n16) * 8), 0, kDeviceScope);
#pragma unroll
          for (int db = 0; db < 4; ++db)
            xs4[u][c][db] = __builtin_amdgcn_raw_buffer_load_b128(
                ws_rsrc, (int)(((cw * 4 + db) * 64 + lane) * 16), 0, kDeviceScope);
        }
      }
#pragma unroll
      for (int u = 0; u < KP; ++u) {
        const bool real = s0 + u < S;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const float m = real ? ml[u][c][0] : kNegInf;
          const float m_new = fmaxf(m_s[c], m);
          const float mc = (m_new == kNegInf) ? 0.f : m_new;
          const float c_old = fast_exp2(m_s[c] - mc);
          const float c_new = fast_exp2(m - mc);
          l_tot[c] = l_tot[c] * c_old + (real ? ml[u][c][1] : 0.f) * c_new;
#pragma unroll
          for (int db = 0; db < 4; ++db)
            oacc[c][db] = oacc[c][db] * c_old + (real ? xs4[u][c][db] : f32x4{0.f, 0.f, 0.f, 0.f}) * c_new;
          m_s[c] = m_new;
        }
      }
    }
    if (tid == 0) __hip_atomic_store(p.counters + jj, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int qrow = q0 + 16 * c + n16;
    if (qrow >= p.Tq) continue;
    const float inv = l_tot[c] > 0.f ? 1.f / l_tot[c] : 0.f;
    store_t<OUTT>* op = reinterpret_cast<store_t<OUTT>*>(p.o) + b * p.o_sb + h * p.o_sh +
                        (int64_t)qrow * p.o_st;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const f32x4 x = oacc[c][db] * inv;
      if (aligned) st4<OUTT, true>(op + 16 * db + 4 * g, x);
      else st4<OUTT, false>(op + 16 * db + 4 * g, x);
    }
  }
}

}  // namespace
}  // namespace ffai
