// gfx950 decode-shaped attention: at most 32 query rows read each K/V head (single-token decode,
// beams stacked as rows over a shared cross-attention cache, grouped query heads, a few
// speculative tokens). Memory- and latency-bound, so the design minimises the dependent steps
// between launch and the last store:
//   * one workgroup = NWD waves over one (batch, kv-head) and one key range; each wave takes its
//     own 64-key tiles, so all the tiles' K/V loads are in flight at once and the waves'
//     softmax/MFMA chains run side by side on the CU's SIMDs;
//   * the rows of a (batch, kv-head) unit -- every query head of the group and every query
//     position -- are the 32 columns of one S^T = K Q^T MFMA block, so K and V are read once
//     per kv-head however many heads or beams share them;
//   * the waves' partial (O, max, sum) merge through LDS. When one workgroup covers a unit's
//     keys it writes the output directly; otherwise each writes its merged partial with
//     device-scope stores and counts itself on the unit's counter, and the unit's last
//     workgroup merges every split's partial and writes the output, in the same launch. (A
//     device-scope release fence per workgroup would write back the whole L2 here; stores that
//     are themselves device-scope need no fence, only their acknowledgement.)
//   * each wave's tile region is its own: whole tiles arrive by DMA (global -> LDS, no staging
//     registers) into unpadded, XOR-swizzled rows, and a wave waits only for its own loads;
//   * the tile loop is not unrolled: a cold workgroup fetches little code.
// MFMA operands and fragment layouts are those of fwd_kernel's 16-bit path (attn_kernels.cuh).
#pragma once

#include "attn_common.cuh"

namespace ffai {
namespace {

// Output row n (of the unit's R rows), chunk c4 of 4 elements, normalised by l.
template <int OUTT, int D>
__device__ __forceinline__ void store_row_chunk(const DecodeParams& p, int b, int hk, int n, int c4,
                                                f32x4 acc, float l) {
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int h = hk * p.group + n / p.Tq, t = n % p.Tq;
  store_t<OUTT>* op = reinterpret_cast<store_t<OUTT>*>(p.o) + b * p.o_sb + h * p.o_sh +
                      (int64_t)t * p.o_st + 4 * c4;
  st4<OUTT, true>(op, acc * inv);
}

// The end of a decode unit's workgroup, shared by the decode kernels: merge the NWD waves'
// partials from LDS and write the unit's rows, or, when the unit's keys are split over
// workgroups, this split's merged partial, and let the unit's last split merge them all.
// LDS layout of wave w's partial (floats from mbase + w * WST): its R <= MR rows of O at
// n * OROW, then the rows' maxima (scaled log2 units) at MR * OROW + n and weight sums at
// MR * OROW + MR + n. Every thread of the workgroup calls it, after a barrier that publishes the
// partials.
// Returns true when this workgroup wrote the unit's rows (unsplit, or the unit's last split).
template <int OUTT, int D, int NWD, int OROW, int MR, int WST>
__device__ __forceinline__ bool finish_unit(const DecodeParams& p, const float* mbase, int b,
                                            int hk, int unit, int split, int R, int tid) {
  constexpr int C4 = D / 4;  // 4-float chunks per row
  const int items = R * C4;
  const int64_t prow0 = ((int64_t)unit * p.n_split + split) * R;  // this split's first partial row
  // the partials: O rows [units][n_split][R][D], then (m, l) pairs [units][n_split][R][2], as a
  // buffer resource over exactly those bytes (an access past them would read 0 / be dropped)
  const int64_t o_floats = (int64_t)p.B * p.Hkv * p.n_split * R * D;
  const int64_t ws_bytes = (o_floats + (int64_t)p.B * p.Hkv * p.n_split * R * 2) * 4;
  const __amdgpu_buffer_rsrc_t ws_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      p.ws, (short)0, (int)(p.n_split > 1 ? ws_bytes : 0), kBufferWord3);

#pragma unroll 1
  for (int it = tid; it < items; it += NWD * 64) {
    const int n = it / C4, c4 = it % C4;
    float mw[NWD];
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < NWD; ++w) {
      mw[w] = mbase[w * WST + MR * OROW + n];
      M = fmaxf(M, mw[w]);
    }
    const float Mc = (M == kNegInf) ? 0.f : M;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < NWD; ++w) {
      const float* mb = mbase + w * WST;
      const float wt = fast_exp2(mw[w] - Mc);  // 0 for an empty wave (m = -inf)
      acc += wt * *reinterpret_cast<const f32x4*>(&mb[n * OROW + 4 * c4]);
      L = __builtin_fmaf(wt, mb[MR * OROW + MR + n], L);
    }
    if (p.n_split == 1) {
      store_row_chunk<OUTT, D>(p, b, hk, n, c4, acc, L);
    } else {
      // This split's partial, written with device-scope (sc1) buffer stores: each one reaches
      // the device's coherence point before it is acknowledged, so the unit's last workgroup
      // reads it wherever (on whichever XCD) it runs, without a write-back of this L2's dirty
      // lines.
      __builtin_amdgcn_raw_buffer_store_b128(acc, ws_rsrc, (int)(((prow0 + n) * D + 4 * c4) * 4),
                                             0, kDeviceScope);
      if (c4 == 0)
        __builtin_amdgcn_raw_buffer_store_b64(f32x2{M, L}, ws_rsrc,
                                              (int)((o_floats + (prow0 + n) * 2) * 4), 0,
                                              kDeviceScope);
    }
  }
  if (p.n_split == 1) return true;

  // ---- count this split; the unit's last one merges them all.
  // Ordering: every thread waits for its partial stores to be acknowledged (vmcnt(0): device-
  // scope stores are acknowledged once they are visible at device scope), the barrier makes that
  // true of the whole workgroup, and only then does one thread add 1 to the unit's counter (a
  // device-scope atomic). The workgroup that reads n_split - 1 back is the unit's last: every
  // other split's partial was visible before its increment, which precedes this one in the
  // counter's order, and this workgroup's device-scope loads are issued after that increment
  // returns. The last workgroup sets the counter back to 0 for the next call (no wait anywhere:
  // a workgroup that is not last simply ends).
  __shared__ int s_last;
  vm_wait_all();
  __syncthreads();
  if (tid == 0) {
    const int done = __hip_atomic_fetch_add(p.counters + unit, 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    s_last = (done == p.n_split - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return false;
  const int S = p.n_split;
  const int64_t uo = (int64_t)unit * S * R * D;               // the unit's first O row (floats)
  const int64_t uml = o_floats + (int64_t)unit * S * R * 2;   // and its first (m, l) pair
  // Online log-sum-exp merge over the splits, eight at a time: the eight splits' device-scope
  // loads are issued together (clamped to the last split; those past it count as empty), then
  // merged in split order, so one round trip covers eight partials. (Sixteen at a time measured
  // slower at 8 and 12 splits: the unrolled merge doubles the code a cold workgroup fetches.)
  constexpr int KS = 8;
#pragma unroll 1
  for (int it = tid; it < items; it += NWD * 64) {
    const int n = it / C4, c4 = it % C4;
    float M = kNegInf, L = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int s0 = 0; s0 < S; s0 += KS) {
      f32x2 mlj[KS];
      f32x4 xj[KS];
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        const int row = min(s0 + j, S - 1) * R + n;
        mlj[j] = __builtin_amdgcn_raw_buffer_load_b64(ws_rsrc, (int)((uml + row * 2) * 4), 0,
                                                      kDeviceScope);
        xj[j] = __builtin_amdgcn_raw_buffer_load_b128(ws_rsrc, (int)((uo + row * D + 4 * c4) * 4),
                                                      0, kDeviceScope);
      }
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        const float m = (s0 + j < S) ? mlj[j][0] : kNegInf;
        const float m_new = fmaxf(M, m);
        if (m_new == kNegInf) continue;  // nothing seen yet (every key so far masked)
        const float c_old = fast_exp2(M - m_new);  // 0 while M is -inf
        const float c_new = fast_exp2(m - m_new);  // 0 for an empty split
        acc = acc * c_old + xj[j] * c_new;
        L = L * c_old + mlj[j][1] * c_new;
        M = m_new;
      }
    }
    store_row_chunk<OUTT, D>(p, b, hk, n, c4, acc, L);
  }
  if (tid == 0) __hip_atomic_store(p.counters + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// NC: 16-column blocks of query rows (1 for units of at most 16 rows, 2 for up to 32).
template <int MODE, int OUTT, int D, bool KT, int NWD, int NC>
__global__ __launch_bounds__(NWD * 64) void decode_kernel(DecodeParams p) {
  static_assert(MODE == kBF16 || MODE == kF16, "decode kernel reads 16-bit Q, K and V");
  // Per-wave LDS: one K tile ([key][d] or [d][key]) and one V tile ([key][d]), 16-bit, rows
  // unpadded with each row's 16-byte chunks XOR-permuted (swz_*, as in fwd_kernel) so that whole
  // tiles arrive by DMA and the fragment reads still spread over the banks.
  constexpr int KROW = D;
  constexpr int KTROW = BN;
  constexpr int VROW = D;
  constexpr int KBUF = KT ? D * KTROW : BN * KROW;
  constexpr int VBUF = BN * VROW;
  constexpr int WBUF = KBUF + VBUF;  // 16-bit elements per wave
  // After the tiles: per-wave merge area of 32 rows x OROW floats, then 32 maxima, 32 sums.
  constexpr int OROW = D + 4;
  constexpr int MBUF = 32 * OROW + 64;
  static_assert(MBUF * 4 <= WBUF * 2, "the merge area fits in the wave's tile area");
  static_assert((WBUF * 2) % 16 == 0 && (KBUF * 2) % 16 == 0, "16-byte aligned regions");
  __shared__ __attribute__((aligned(16))) uint16_t lds[NWD * WBUF];

  // ---- which (batch, kv-head, key split): the grid is (splits, kv-heads, batch), so the
  //      indices are the workgroup's own and its operand addresses are scalar arithmetic (a
  //      division of a flat index cost ~0.3 us of dependent vector instructions before the first
  //      K/V load could be issued)
  const int split = wg_id_x();
  const int hk = wg_id_y();
  const int b = wg_id_z();
  const int unit = b * p.Hkv + hk;

  const int tid = item_id();
  const int lane = tid & 63;
  // wave-uniform, and made visibly so: the tile choices below are then scalar branches, and the
  // compiler does not wait on one branch's loads before another's (it did: the register-staging
  // loads of the tail path made it await the Q loads before issuing any K/V DMA)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4;   // lane group: contraction elements 8 q4 .., accumulator rows 4 q4 ..
  const int n16 = lane & 15;  // this lane's column in each 16-column block
  const int R = p.group * p.Tq;
  // the unit's query row of column c (block c / 16): n = 16 c + n16; columns past R repeat row
  // R - 1 (each column's scores, weights and sums stay in that column, and only the first R
  // are read back)
  int t_row[NC], h_row[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int rn = min(16 * c + n16, R - 1);
    t_row[c] = rn % p.Tq;
    h_row[c] = hk * p.group + rn / p.Tq;
  }

  int kv_end = p.Tk;
  if (p.kv_lens) kv_end = min(kv_end, max(0, p.kv_lens[b]));
  kv_end = __builtin_amdgcn_readfirstlane(kv_end);  // uniform (one batch item per workgroup)
  int kv_blk = kv_end;  // keys any row of the unit may see
  if (p.causal) kv_blk = min(kv_end, max(0, p.q_offset + p.Tq));
  const int n_tiles = (kv_blk + BN - 1) / BN;
  const int t_begin = split * p.tiles_per_split;
  const int t_end = min(n_tiles, t_begin + p.tiles_per_split);
  const int iters = t_end > t_begin ? (t_end - t_begin + NWD - 1) / NWD : 0;
  const float sl2 = p.scale_log2;
  int lim[NC];  // the last key column block c's row may see
#pragma unroll
  for (int c = 0; c < NC; ++c) lim[c] = p.causal ? min(kv_end - 1, p.q_offset + t_row[c]) : kv_end - 1;

  const uint16_t* kp = reinterpret_cast<const uint16_t*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const uint16_t* vp = reinterpret_cast<const uint16_t*>(p.v) + b * p.v_sb + hk * p.v_sh;

  // O^T per column block, 16 d per accumulator: oacc[c][db][r] <-> d = 16 db + 4 q4 + r of
  // column 16 c + n16
  f32x4 oacc[NC][D / 16];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int db = 0; db < D / 16; ++db) oacc[c][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_s[NC], l_run[NC];  // running max (scaled log2 units, the same in all four lane
                             // groups) and this lane group's part of the running sum
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    m_s[c] = kNegInf;
    l_run[c] = 0.f;
  }

  uint16_t* kl = lds + wave * WBUF;
  uint16_t* vl = kl + KBUF;
  // 16-byte chunk permutations of the tiles' rows (the same as fwd_kernel's)
  auto swz_kt = [](int r, int c) { return c ^ (4 * ((r >> 1) & 1)); };
  auto swz_v = [](int r, int c) { return D == 64 ? c ^ (4 * ((r >> 1) & 1)) : c ^ (4 * (r & 3)); };
  auto swz_kr = [](int r, int c) { return D == 64 ? c ^ ((r >> 1) & 7) : c ^ (r & 15); };
  // transposing LDS reads: in each 16-lane group, lane j reads 4 elements of row r0 + j / 4 at
  // column c0 + 4 (j % 4), and then holds column c0 + j of rows r0 .. r0 + 3
  const int tr_row = n16 >> 2, tr_col = 4 * (n16 & 3);

  // ---- staging (the host launches this kernel only for operands that admit its vector
  //      accesses). Rows of K and V: 16-byte units, the key index clamped to the last valid key
  //      and zeroed past it. K^T rows: 4-key (8-byte) chunks, each loaded when all four keys are
  //      valid and zeroed otherwise; the one chunk per row that straddles the last valid key is
  //      then patched element by element in LDS. Every address stays inside the operand.
  // The wave's own tile, whole and aligned: global -> LDS by DMA (16-byte chunks, lane L of
  // block j fills slot L of the block; the chunk placed there is the one the swizzle assigns).
  // A 1 KB block holds 64 / (chunks per row) whole rows. Each lane's byte offset from the tile's
  // first row (its row, the chunk permutation) is 32-bit lane arithmetic, the same for every
  // tile (the host keeps a tile's rows within 2^31 bytes of its first); only the wave-uniform
  // tile base moves, in scalar registers. (Block bases of their own, one 64-bit scalar pair per
  // block and operand, made the compiler park them in vector-register lanes.)
  constexpr int KCH = KT ? BN / 8 : D / 8, KRB = 64 / KCH;  // K: chunks per row, rows per block
  constexpr int VCH = D / 8, VRB = 64 / VCH;
  const int kr = lane / KCH, kpc = lane % KCH, vr = lane / VCH, vpc = lane % VCH;
  // `valid`: the tile's keys before the end of the cache (wave-uniform). Blocks of K or V rows
  // that hold none of them are not read: their LDS rows keep stale values, whose keys are masked
  // and whose V rows are cleared once the DMA has landed (ragged tails of per-beam caches).
  auto dma_tile = [&](int it, int valid) {
    const int64_t kb = (int64_t)it * BN;
    const uint32_t kla = lds_addr(kl), vla = lds_addr(vl);
    const char* kbase = reinterpret_cast<const char*>(kp + (KT ? kb : kb * p.k_st));
    const char* vbase = reinterpret_cast<const char*>(vp + kb * p.v_st);
#pragma unroll
    for (int j = 0; j < KBUF / 512; ++j) {
      const int r = j * KRB + kr;
      const uint32_t off =
          (uint32_t)(2 * (r * p.k_st + 8 * (KT ? swz_kt(r, kpc) : swz_kr(r, kpc))));
      if (KT || j * KRB < valid) lds_dma16_sbase<true>(kbase, off, kla + j * 1024);
    }
#pragma unroll
    for (int j = 0; j < VBUF / 512; ++j) {
      const int r = j * VRB + vr;
      const uint32_t off = (uint32_t)(2 * (r * p.v_st + 8 * swz_v(r, vpc)));
      if (j * VRB < valid) lds_dma16_sbase<true>(vbase, off, vla + j * 1024);
    }
  };
  // The operand's last tile, when it has at least 8 keys but fewer than 64 (cross-attention over
  // 1500 frames): DMA as well, each lane's source clamped inside the operand. K/V rows past the
  // last valid key read that key's row instead; K^T 8-key chunks that would cross the
  // operand's end read the tile's first chunk. The slots of masked keys then hold finite
  // stand-ins; the valid keys of the one K^T chunk that crosses the end are patched afterwards.
  auto dma_tile_clamped = [&](int it) {
    const int kb = it * BN;
    const int klast = kv_end - 1;
    const uint32_t kla = lds_addr(kl), vla = lds_addr(vl);
    const char* kbase = reinterpret_cast<const char*>(kp + (KT ? kb : (int64_t)kb * p.k_st));
    const char* vbase = reinterpret_cast<const char*>(vp + (int64_t)kb * p.v_st);
#pragma unroll
    for (int j = 0; j < KBUF / 512; ++j) {
      const int r = j * KRB + kr;
      if constexpr (KT) {
        const int c0 = kb + 8 * swz_kt(r, kpc);
        const int src = c0 + 8 <= p.Tk ? c0 : kb;
        const uint32_t off = (uint32_t)(2 * (r * p.k_st + (src - kb)));
        lds_dma16_sbase<true>(kbase, off, kla + j * 1024);
      } else {
        const int key = min(kb + r, klast);
        const uint32_t off = (uint32_t)(2 * ((key - kb) * p.k_st + 8 * swz_kr(r, kpc)));
        lds_dma16_sbase<true>(kbase, off, kla + j * 1024);
      }
    }
#pragma unroll
    for (int j = 0; j < VBUF / 512; ++j) {
      const int r = j * VRB + vr;
      const int key = min(kb + r, klast);
      const uint32_t off = (uint32_t)(2 * ((key - kb) * p.v_st + 8 * swz_v(r, vpc)));
      lds_dma16_sbase<true>(vbase, off, vla + j * 1024);
    }
  };
  // The valid keys of the 8-key K^T chunk that crosses the operand's end, element by element:
  // loaded together with the clamped DMA (so both share one memory round trip) and written
  // over the DMA's stand-in once it has landed. Each lane holds its d-rows' (at most 7) keys.
  constexpr int PROWS = D / 64;
  uint16_t patch[PROWS][7];
  auto patch_kt_load = [&]() {
    const int klast = kv_end - 1;
    const int s0 = klast & ~7;
#pragma unroll
    for (int i = 0; i < PROWS; ++i) {
      const uint16_t* row = kp + (int64_t)(lane + 64 * i) * p.k_st;
#pragma unroll
      for (int x = 0; x < 7; ++x) patch[i][x] = row[min(s0 + x, klast)];
    }
  };
  auto patch_kt_store = [&](int it) {
    const int kb = it * BN;
    const int klast = kv_end - 1;
    const int s0 = klast & ~7;
#pragma unroll
    for (int i = 0; i < PROWS; ++i) {
      const int d = lane + 64 * i;
#pragma unroll
      for (int x = 0; x < 7; ++x) {
        const int col = s0 + x - kb;
        if (s0 + x <= klast) kl[d * KTROW + 8 * swz_kt(d, col >> 3) + (col & 7)] = patch[i][x];
      }
    }
  };
  // Tail tiles (past the last valid key) and misaligned K^T rows: through registers. Rows of K
  // and V: 16-byte units, the key index clamped to the last valid key and zeroed past it. K^T
  // rows: 4-key (8-byte) chunks, each loaded when all four keys are valid and zeroed otherwise;
  // the one chunk per row that straddles the last valid key is then patched element by element
  // in LDS. Every address stays inside the operand; stores go to the swizzled slots.
  auto stage_tile = [&](int it) {
    const int kb = it * BN;
    const int klast = kv_end - 1;
    u32x4 kreg[D / 8], vreg[D / 8];
#pragma unroll
    for (int j = 0; j < D / 8; ++j) {
      const int u = lane + 64 * j;
      if constexpr (KT) {
        const int d = u / (BN / 8), kc = u % (BN / 8);
        const int k4 = kb + 8 * kc;
        const uint16_t* row = kp + (int64_t)d * p.k_st;
        const bool v0 = k4 + 3 <= klast, v1 = k4 + 7 <= klast;
        const u32x2 lo = ld8(row + (v0 ? k4 : 0)), hi = ld8(row + (v1 ? k4 + 4 : 0));
        kreg[j] = u32x4{v0 ? lo.x : 0u, v0 ? lo.y : 0u, v1 ? hi.x : 0u, v1 ? hi.y : 0u};
      } else {
        const int key = kb + u / (D / 8), c = u % (D / 8);
        const u32x4 x = ld16(kp + (int64_t)min(key, klast) * p.k_st + 8 * c);
        kreg[j] = key <= klast ? x : u32x4{0u, 0u, 0u, 0u};
      }
      const int key = kb + u / (D / 8), c = u % (D / 8);
      const u32x4 x = ld16(vp + (int64_t)min(key, klast) * p.v_st + 8 * c);
      vreg[j] = key <= klast ? x : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < D / 8; ++j) {
      const int u = lane + 64 * j;
      if constexpr (KT) {
        const int d = u / (BN / 8), kc = u % (BN / 8);
        *reinterpret_cast<u32x4*>(&kl[d * KTROW + 8 * swz_kt(d, kc)]) = kreg[j];
      } else {
        const int key = u / (D / 8), c = u % (D / 8);
        *reinterpret_cast<u32x4*>(&kl[key * KROW + 8 * swz_kr(key, c)]) = kreg[j];
      }
      const int key = u / (D / 8), c = u % (D / 8);
      *reinterpret_cast<u32x4*>(&vl[key * VROW + 8 * swz_v(key, c)]) = vreg[j];
    }
    if constexpr (KT) {
      const int k4s = klast & ~3;  // the straddling chunk, when the valid keys end inside one
      if (klast < kb + BN - 1 && (klast & 3) != 3) {
        for (int d = lane; d < D; d += 64) {
          const uint16_t* row = kp + (int64_t)d * p.k_st;
          uint16_t e[3];
#pragma unroll
          for (int x = 0; x < 3; ++x) e[x] = row[min(k4s + x, klast)];
#pragma unroll
          for (int x = 0; x < 3; ++x) {
            const int col = k4s - kb + x;
            if (k4s + x <= klast) kl[d * KTROW + 8 * swz_kt(d, col >> 3) + (col & 7)] = e[x];
          }
        }
      }
    }
  };

  // A ragged tail that still lies inside the operand's rows (a per-beam cache shorter than its
  // capacity) comes by DMA too. Its keys past the end are masked below, but their V rows may hold
  // anything (inf, NaN) and a masked weight of 0 times NaN is NaN: they are cleared in LDS once
  // the DMA has landed. (K^T only) the chunk that crosses the operand's end is not read whole by
  // the DMA and is patched.
  auto tail_dma_of = [&](int kb) { return kb + BN > kv_end && kb + BN <= p.Tk; };
  auto end_dma_of = [&](int kb) { return kb + BN > p.Tk && kb + 8 <= p.Tk; };
  auto patch_end_of = [&](int kb) {
    return KT && end_dma_of(kb) && ((kv_end - 1) & ~7) + 8 > p.Tk;
  };
  // Issue tile `it`'s loads (by DMA, or through registers for a short end).
  auto issue_tile = [&](int it) {
    const int kb = it * BN;
    if (kb + BN <= kv_end || tail_dma_of(kb)) dma_tile(it, min(BN, kv_end - kb));
    else if (end_dma_of(kb)) dma_tile_clamped(it);
    else stage_tile(it);
    if (patch_end_of(kb)) patch_kt_load();
  };
#ifdef FFAI_STAMPS
  // event times of the workgroup, recorded by wave 0 (diagnostic builds only; attn_common.cuh),
  // for head_dim 64 (the head_dim-128 instantiations keep their register budget without them)
  constexpr bool ST = D == 64;
  const int st_wg = split + p.n_split * (hk + p.Hkv * b);  // the linear workgroup index
  const bool st_rec = ST && p.stamps && st_wg < p.stamp_wgs && tid == 0;
  uint64_t st_e[6] = {0, 0, 0, 0, 0, 0};
  const uint64_t st_r0 = ST ? stamp_realtime() : 0;
  if constexpr (ST) st_e[0] = stamp_clock();
#endif
  // The wave's first tile goes out before the Q loads: the DMA is a compiler barrier for memory
  // accesses, so nothing is outstanding when it is issued. (Issued after them, the compiler made
  // the DMA wait for the Q loads: registers it reuses were load targets on the register-staging
  // path, and one in-order counter covers both.)
  if (iters > 0 && t_begin + wave < t_end) issue_tile(t_begin + wave);
#ifdef FFAI_STAMPS
  if constexpr (ST) st_e[1] = stamp_clock();
#endif
  // ---- Q fragments (issued after the wave's first K/V loads): B operand of S^T, block c,
  //      contraction chunk h: d = 32 h + 8 q4 .. +7 of column 16 c + n16's row
  u32x4 qf[NC][D / 32];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint16_t* qr = reinterpret_cast<const uint16_t*>(p.q) + b * p.q_sb +
                         h_row[c] * p.q_sh + (int64_t)t_row[c] * p.q_st;
#pragma unroll
    for (int h = 0; h < D / 32; ++h) qf[c][h] = ld16(qr + 32 * h + 8 * q4);
  }

#pragma unroll 1
  for (int i = 0; i < iters; ++i) {
    const int it = t_begin + wave + NWD * i;
    const bool has = it < t_end;  // wave-uniform
    const int kb = it * BN;
    if (!has) continue;
    if (i > 0) {
      // the tile region is this wave's own: reuse needs only its own earlier LDS reads done
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      issue_tile(it);
    }
    const bool tail_dma = tail_dma_of(kb), end_dma = end_dma_of(kb);
    const bool patch_end = patch_end_of(kb);
    vm_wait_all();
#ifdef FFAI_STAMPS
    if (ST && i == 0) st_e[2] = stamp_clock();
#endif
    if (patch_end) patch_kt_store(it);
    if (tail_dma || end_dma) {
      constexpr int RU = D / 8;  // 16-byte units per V row; the swizzle stays within a row
      for (int u = max(0, kv_end - kb) * RU + lane; u < BN * RU; u += 64)
        *reinterpret_cast<u32x4*>(&vl[8 * u]) = u32x4{0u, 0u, 0u, 0u};
    }

    // ---- S^T per 16-key block kb4 of the tile, on 16x16x32 MFMA:
    //      sacc[c][kb4][r] <-> key kb + 16 kb4 + 4 q4 + r of column 16 c + n16
    f32x4 sacc[NC][4];
#pragma unroll
    for (int kb4 = 0; kb4 < 4; ++kb4) {
#pragma unroll
      for (int c = 0; c < NC; ++c) sacc[c][kb4] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int h = 0; h < D / 32; ++h) {
        // A: key 16 kb4 + n16, d = 32 h + 8 q4 .. +7
        u32x4 a;
        if constexpr (KT) {
          // K^T [d][key]: rows r and r + 4 share the chunk permutation (bit 1 of the row)
          const int r = 32 * h + 8 * q4 + tr_row, col = 16 * kb4 + tr_col;
          const uint16_t* base = &kl[r * KTROW + 8 * swz_kt(r, col >> 3) + (col & 7)];
          const u32x2 lo = lds_tr(base), hi = lds_tr(base + 4 * KTROW);
          a = u32x4{lo.x, lo.y, hi.x, hi.y};
        } else {
          const int r = 16 * kb4 + n16;
          a = *reinterpret_cast<const u32x4*>(&kl[r * KROW + 8 * swz_kr(r, 4 * h + q4)]);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) sacc[c][kb4] = mfma16x16<MODE>(a, qf[c][h], sacc[c][kb4]);
      }
    }
    // ---- mask (only tiles that reach past a row's last visible key: the ragged end, or the
    //      causal diagonal of the unit's first row), max, rescale, weights
    if (kb + BN > kv_end || (p.causal && kb + BN - 1 > p.q_offset)) {  // wave-uniform
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int kb4 = 0; kb4 < 4; ++kb4)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (kb + 16 * kb4 + 4 * q4 + r > lim[c]) sacc[c][kb4][r] = kNegInf;
    }
    // P per column block and 32-key chunk ch, the B operand of O^T += V^T P^T: lane group q4's
    // contraction slots e hold keys 32 ch + 4 q4 + e (e < 4) and 32 ch + 16 + 4 q4 + e - 4
    // (blocks 2 ch and 2 ch + 1 of S^T as they lie in the lane); V is read in the same order
    u32x4 pf[NC][2];
    float corr[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float mx = kNegInf;
#pragma unroll
      for (int kb4 = 0; kb4 < 4; ++kb4)
        mx = fmaxf(mx, fmaxf(fmaxf(sacc[c][kb4][0], sacc[c][kb4][1]),
                             fmaxf(sacc[c][kb4][2], sacc[c][kb4][3])));
      const float m_new = fmaxf(m_s[c], quad_max(mx) * sl2);
      corr[c] = (m_new == kNegInf) ? 1.f : fast_exp2(m_s[c] - m_new);
      m_s[c] = m_new;
      const float mc = (m_new == kNegInf) ? 0.f : m_new;
      float rs = 0.f;
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const f32x4& sv = sacc[c][2 * ch + (k >> 1)];
          const float e0 = fast_exp2(__builtin_fmaf(sv[2 * (k & 1)], sl2, -mc));
          const float e1 = fast_exp2(__builtin_fmaf(sv[2 * (k & 1) + 1], sl2, -mc));
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
        pf[c][ch] = u32x4{w[0], w[1], w[2], w[3]};
      }
      l_run[c] = __builtin_fmaf(l_run[c], corr[c], rs);
    }
    if (i > 0) {  // the first tile finds the accumulators still zero (wave-uniform)
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int db = 0; db < D / 16; ++db) oacc[c][db] *= corr[c];
    }
    // ---- O^T += V^T P^T: A(d = 16 db + n16, slot e) = V(key of slot e, d), read transposed from
    //      the [key][d] tile: rows r and r + 16 share the chunk permutation
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        const int r = 32 * ch + 4 * q4 + tr_row, col = 16 * db + tr_col;
        const uint16_t* base = &vl[r * VROW + 8 * swz_v(r, col >> 3) + (col & 7)];
        const u32x2 a0 = lds_tr(base), a1 = lds_tr(base + 16 * VROW);
        const u32x4 a = {a0.x, a0.y, a1.x, a1.y};
#pragma unroll
        for (int c = 0; c < NC; ++c) oacc[c][db] = mfma16x16<MODE>(a, pf[c][ch], oacc[c][db]);
      }
  }

  // ---- merge the waves' partials through LDS (the tile area is free once all waves pass here)
#ifdef FFAI_STAMPS
  if (ST && iters == 0) st_e[2] = stamp_clock();
  if constexpr (ST) st_e[3] = stamp_clock();
#endif
  __syncthreads();
  float* mbase = reinterpret_cast<float*>(lds);
  {
    float* mb = mbase + wave * (WBUF / 2);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float l_tot = quad_sum(l_run[c]);  // the whole wave takes part (lane swaps)
      const int n = 16 * c + n16;
      // only the unit's R rows are read back: the other columns' lanes write nothing
      if (n < R) {
#pragma unroll
        for (int db = 0; db < D / 16; ++db)
          *reinterpret_cast<f32x4*>(&mb[n * OROW + 16 * db + 4 * q4]) = oacc[c][db];
        if (q4 == 0) {
          mb[32 * OROW + n] = m_s[c];
          mb[32 * OROW + 32 + n] = l_tot;
        }
      }
    }
  }
  __syncthreads();
#ifdef FFAI_STAMPS
  if constexpr (ST) st_e[4] = stamp_clock();
  const bool st_wrote =
#endif
  finish_unit<OUTT, D, NWD, OROW, 32, WBUF / 2>(p, mbase, b, hk, unit, split, R, tid);
#ifdef FFAI_STAMPS
  if constexpr (ST) st_e[5] = stamp_clock();
  if (st_rec) {
#pragma unroll
    for (int k = 0; k < 6; ++k) stamp_put(p.stamps, (int64_t)st_wg * 8 + k, st_e[k]);
    stamp_put(p.stamps, (int64_t)st_wg * 8 + 6, st_wrote ? 1u : 0u);
    stamp_put(p.stamps, (int64_t)st_wg * 8 + 7, st_r0);
  }
#endif
}


// ---------------------------------------------------------------------------------------------
// f32 queries, one query row per (batch, kv-head) unit, head_dim 64: the reference's own decode
// arms, a query row in f32 over f16 K/V (flash_attn.rs:289-356, xattn_head_f16 :698-789: the
// cross-attention cache) or f32 K/V (:370-399, xattn_head :595-696: the self-attention cache),
// and bf16 K/V alike. With one row the two products are matrix-vector products: an MFMA would
// compute 16 columns to keep one, so this kernel runs them on the VALU in f32, reading K and V
// straight into registers with 16-byte (8-byte for 16-bit K^T) vector loads, every load of a
// wave's 64-key tile in flight at once (24 or 32 loads per lane, under the 63 a wave can have
// outstanding):
//   * scores: lane (kq, dg) = (lane % 16, lane / 16) takes keys 4 kq .. 4 kq + 3 over head dims
//     16 dg .. 16 dg + 15: K^T (the reference's layout) as 4-key chunks of 16 d-rows, K as rows
//     as 16-d slices of 4 rows. The four d-groups' partial dot products are summed across the
//     lane groups (v_permlane16/32_swap), so every lane holds its 4 keys' full scores;
//   * softmax: online over the wave's tiles, in base 2 with v_exp_f32; the tile max over the 16
//     lanes of a row by DPP;
//   * PV: the weights go through a 256-byte LDS slot of the wave; lane (c, g) takes a 16-byte
//     chunk c of the V rows (4 f32 or 8 16-bit elements of d) for the rows of group g, and the
//     groups' partial outputs are summed at the end.
// Waves take their own 64-key tiles and merge through LDS; split units merge as in
// decode_kernel (finish_unit). The host launches it for f32 queries, group x q_len == 1,
// head_dim 64, 4-element-aligned operands, and heads whose K and V lie within 2^31 bytes.
template <int KVT, bool KT, int NWD>
__global__ __launch_bounds__(NWD * 64) void decode_vec_kernel(DecodeParams p) {
  constexpr int D = 64;
  constexpr int OROW = D + 4;     // merge area of a wave: its O row,
  constexpr int WST = OROW + 4;   // then its max and weight sum (16-byte aligned stride)
  using KVS = store_t<KVT>;
  constexpr int ES = (int)sizeof(KVS);
  constexpr int VE = 16 / ES;        // V elements per 16-byte chunk: 4 (f32) or 8 (16-bit)
  constexpr int VC = D / VE;         // chunks per V row: lanes per row group
  constexpr int VG = 64 / VC;        // row groups: 4 (f32) or 8 (16-bit)
  constexpr int VR = BN / VG;        // rows per group: 16 or 8
  using KR = std::conditional_t<KVT == kF32, f32x4, u32x2>;  // 4 K elements as loaded
  __shared__ __attribute__((aligned(16))) float mlds[NWD * WST];
  __shared__ __attribute__((aligned(16))) float wlds[NWD * BN];  // each wave's tile weights

  const int split = wg_id_x();
  const int hk = wg_id_y();
  const int b = wg_id_z();
  const int unit = b * p.Hkv + hk;
  const int tid = item_id();
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kq = lane & 15, dg = lane >> 4;  // scores: keys 4 kq + e, d in [16 dg, 16 dg + 16)
  const int vc = lane % VC, vg = lane / VC;  // PV: chunk vc of d, rows VR vg .. VR vg + VR - 1

  int kv_end = p.Tk;
  if (p.kv_lens) kv_end = min(kv_end, max(0, p.kv_lens[b]));
  kv_end = __builtin_amdgcn_readfirstlane(kv_end);  // uniform (one batch item per workgroup)
  // the row's last visible key (q_len 1: the row's position is q_offset)
  const int lim = p.causal ? min(kv_end - 1, p.q_offset) : kv_end - 1;
  const int n_tiles = (max(0, lim + 1) + BN - 1) / BN;
  const int t_begin = split * p.tiles_per_split;
  const int t_end = min(n_tiles, t_begin + p.tiles_per_split);
  const float sl2 = p.scale_log2;

  const KVS* kp = reinterpret_cast<const KVS*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const KVS* vp = reinterpret_cast<const KVS*>(p.v) + b * p.v_sb + hk * p.v_sh;
  // this lane's 16 query elements, d = 16 dg .. 16 dg + 15 (head hk * group, position 0)
  const float* qr =
      reinterpret_cast<const float*>(p.q) + b * p.q_sb + (int64_t)hk * p.group * p.q_sh + 16 * dg;
  float q[16];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(qr + 4 * c);
#pragma unroll
    for (int e = 0; e < 4; ++e) q[4 * c + e] = x[e];
  }
  // K and V are read at 32-bit byte offsets from the head's base, stepped in vector registers
  // (an empty asm after each step keeps the compiler from hoisting 16 row offsets per operand
  // into scalar registers)
  const char* kb8 = reinterpret_cast<const char*>(kp);
  const char* vb8 = reinterpret_cast<const char*>(vp);
  const uint32_t kstep = (uint32_t)p.k_st * (uint32_t)ES;
  const uint32_t vstep = (uint32_t)p.v_st * (uint32_t)ES;
  float* wl = wlds + wave * BN;

  f32x4 o4[VE / 4];      // this lane's partial O over its row group, d = VE vc ..
#pragma unroll
  for (int i = 0; i < VE / 4; ++i) o4[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_s = kNegInf;   // running max, scaled log2 units (wave-uniform)
  float l_run = 0.f;     // running weight sum of this lane's 4 keys
#pragma unroll 1
  for (int it = t_begin + wave; it < t_end; it += NWD) {
    const int kb = it * BN;
    const int k0 = kb + 4 * kq;  // this lane's first key
    // ---- loads, as raw bits (widened after every load is issued): K (4 keys x 16 d) and V
    //      (VR rows x one 16-byte chunk)
    KR kraw[16];  // K^T layout: element e of kraw[i] = K(key k0 + e, d = 16 dg + i);
                  // rows: element e of kraw[4 r + c] = K(key k0 + r, d = 16 dg + 4 c + e)
    if constexpr (KT) {
      // a chunk wholly past the operand's end reads the row's first chunk instead (its keys
      // are masked); only a chunk that straddles the end goes element by element
      const int kc0 = k0 < p.Tk ? k0 : 0;
      uint32_t off = ((uint32_t)(16 * dg) * (uint32_t)p.k_st + (uint32_t)kc0) * ES;
      if (kc0 + 4 <= p.Tk) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          kraw[i] = *reinterpret_cast<const KR*>(kb8 + off);
          off += kstep;
          asm volatile("" : "+v"(off));
        }
      } else {
        // the chunk holding the operand's last key (or an operand of fewer than 4 keys):
        // elements clamped to the last key
        const int cl = max(0, min(3, p.Tk - 1 - kc0));
        uint32_t off0 = off;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const KVS* r = reinterpret_cast<const KVS*>(kb8 + off0);
          if constexpr (KVT == kF32) {
            kraw[i] = f32x4{r[0], r[min(1, cl)], r[min(2, cl)], r[min(3, cl)]};
          } else {
            kraw[i] = u32x2{(uint32_t)r[0] | ((uint32_t)r[min(1, cl)] << 16),
                            (uint32_t)r[min(2, cl)] | ((uint32_t)r[min(3, cl)] << 16)};
          }
          off0 += kstep;
          asm volatile("" : "+v"(off0));
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const KVS* kr = kp + (int64_t)min(k0 + r, kv_end - 1) * p.k_st + 16 * dg;
#pragma unroll
        for (int c = 0; c < 4; ++c) kraw[4 * r + c] = *reinterpret_cast<const KR*>(kr + 4 * c);
      }
    }
    u32x4 vx[VR];  // row VR vg + i, elements VE vc .. VE vc + VE - 1 (raw bits)
    {
      const int r0 = kb + VR * vg;
      uint32_t off = ((uint32_t)r0 * (uint32_t)p.v_st + (uint32_t)(VE * vc)) * ES;
      if (kb + BN <= kv_end) {
#pragma unroll
        for (int i = 0; i < VR; ++i) {
          vx[i] = ld16(vb8 + off);
          off += vstep;
          asm volatile("" : "+v"(off));
        }
      } else {
        // the last tile: rows past the last valid one read that row (their weights are 0)
#pragma unroll
        for (int i = 0; i < VR; ++i) {
          const uint32_t row = (uint32_t)min(r0 + i, kv_end - 1);
          vx[i] = ld16(vb8 + (row * (uint32_t)p.v_st + (uint32_t)(VE * vc)) * ES);
        }
      }
    }
    // every load of the tile is issued before the first product waits for one
    __builtin_amdgcn_sched_barrier(0);

    f32x4 kx[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if constexpr (KVT == kF32) {
        kx[i] = kraw[i];
      } else {
        kx[i] = f32x4{to_f32<KVT>(kraw[i].x & 0xffffu), to_f32<KVT>(kraw[i].x >> 16),
                      to_f32<KVT>(kraw[i].y & 0xffffu), to_f32<KVT>(kraw[i].y >> 16)};
      }
    }
    // ---- scores of keys k0 .. k0 + 3: this lane's 16 d, then summed over the 4 d-groups
    float sc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float kv = KT ? kx[i][e] : kx[4 * e + i / 4][i % 4];
        a = __builtin_fmaf(q[i], kv, a);
      }
      sc[e] = quad_sum(a);
    }
    float tmax = kNegInf;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sc[e] = (k0 + e <= lim) ? sc[e] * sl2 : kNegInf;
      tmax = fmaxf(tmax, sc[e]);
    }
    tmax = fmaxf(tmax, dpp_mov<0xb1>(tmax));   // max over the row's 16 lanes
    tmax = fmaxf(tmax, dpp_mov<0x4e>(tmax));
    tmax = fmaxf(tmax, dpp_mov<0x124>(tmax));
    tmax = fmaxf(tmax, dpp_mov<0x128>(tmax));
    // the tile's first key is visible, so the max is finite from the first tile on
    const float m_new = fmaxf(m_s, tmax);
    const float corr = (m_new == m_s) ? 1.f : fast_exp2(m_s - m_new);
    m_s = m_new;
    f32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = fast_exp2(sc[e] - m_new);  // 0 for a masked key
    l_run = __builtin_fmaf(l_run, corr, (w[0] + w[1]) + (w[2] + w[3]));
    // ---- weights through LDS (the wave's own slot: ordering within the wave only)
    if (dg == 0) *reinterpret_cast<f32x4*>(&wl[4 * kq]) = w;
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the slot is written
    f32x4 wr[VR / 4];
#pragma unroll
    for (int i = 0; i < VR / 4; ++i) wr[i] = *reinterpret_cast<const f32x4*>(&wl[VR * vg + 4 * i]);
    // ---- O += w V over this lane's rows
#pragma unroll
    for (int c = 0; c < VE / 4; ++c) o4[c] *= corr;
#pragma unroll
    for (int i = 0; i < VR; ++i) {
      const float wi = wr[i / 4][i % 4];
      if constexpr (KVT == kF32) {
        o4[0] += wi * __builtin_bit_cast(f32x4, vx[i]);
      } else {
#pragma unroll
        for (int c = 0; c < VE / 4; ++c) {
          const f32x4 v = {to_f32<KVT>(vx[i][2 * c] & 0xffffu), to_f32<KVT>(vx[i][2 * c] >> 16),
                           to_f32<KVT>(vx[i][2 * c + 1] & 0xffffu),
                           to_f32<KVT>(vx[i][2 * c + 1] >> 16)};
          o4[c] += wi * v;
        }
      }
    }
    // the slot is rewritten by the next tile: its reads must be done (LDS returns in order)
    __builtin_amdgcn_s_waitcnt(0xc07f);
  }

  // ---- this wave's partial to LDS (a wave without tiles leaves m = -inf, l = 0, O = 0): O
  // summed over the row groups (lanes vc + VC g), l over the 16 lanes of a row
  float l_tot = l_run;
  l_tot += dpp_mov<0xb1>(l_tot);
  l_tot += dpp_mov<0x4e>(l_tot);
  l_tot += dpp_mov<0x124>(l_tot);
  l_tot += dpp_mov<0x128>(l_tot);
#pragma unroll
  for (int c = 0; c < VE / 4; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = o4[c][e];
      if constexpr (VG == 8) x += dpp_mov<0x128>(x);  // lanes l and l ^ 8 (row_ror:8)
      o4[c][e] = quad_sum(x);
    }
  float* mb = mlds + wave * WST;
  if (vg == 0) {
#pragma unroll
    for (int c = 0; c < VE / 4; ++c) *reinterpret_cast<f32x4*>(&mb[VE * vc + 4 * c]) = o4[c];
  }
  if (lane == 0) {
    mb[OROW] = m_s;
    mb[OROW + 1] = l_tot;
  }
  __syncthreads();
  finish_unit<kF32, D, NWD, OROW, 1, WST>(p, mlds, b, hk, unit, split, 1, tid);
}

}  // namespace
}  // namespace ffai
