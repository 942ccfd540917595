// C ABI of the gfx950 fused attention path (include/ffai_attn.h): descriptor validation, the
// serves predicate, launch planning, and the mirrors of the reference's public functions
// (crates/ffai-mercury/src/asr/flash_attn.rs: serves :103-129, attend :212-264 with
// FlashAttnOp::cpu_fwd :266-413, attend_merged :131-158 with MergedAttnOp::cpu_fwd :160-210).

#include "../../include/ffai_attn.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "attn_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

// ---- device check: the kernels are compiled for gfx950 only --------------------------------
constexpr int kMaxDevices = 64;
std::atomic<int> g_dev_state[kMaxDevices];  // 0 unknown, 1 gfx950, 2 other

int check_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(FFAI_ERR_HIP, "hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return fail(FFAI_ERR_DEVICE, "device index out of range");
  int st = g_dev_state[dev].load(std::memory_order_acquire);
  if (st == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess)
      return fail(FFAI_ERR_HIP, "hipGetDeviceProperties failed");
    st = (std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) ? 1 : 2;
    g_dev_state[dev].store(st, std::memory_order_release);
  }
  if (st != 1) return fail(FFAI_ERR_DEVICE, "current device is not gfx950");
  return FFAI_OK;
}

// ---- device geometry: CUs and XCDs of the current device, which the launch plans balance over.
// An MI355X in its default (single-partition) mode has 256 CUs in 8 XCDs; a partitioned one
// shows each partition as a device with its share. Without a device (planning on a host with no
// GPU) the plans assume the full chip. ffai_set_geometry_override replaces it (tests, sweeps).
struct Geometry {
  int cus = 256;
  int xcds = 8;
};
std::atomic<int> g_geo_cus[kMaxDevices], g_geo_xcds[kMaxDevices];  // 0: not yet read
std::atomic<int> g_geo_override_cus{0}, g_geo_override_xcds{0};

Geometry device_geometry() {
  Geometry g;
  const int oc = g_geo_override_cus.load(std::memory_order_relaxed);
  const int ox = g_geo_override_xcds.load(std::memory_order_relaxed);
  if (oc > 0 && ox > 0) {
    g.cus = oc;
    g.xcds = ox;
    return g;
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return g;
  int cus = g_geo_cus[dev].load(std::memory_order_acquire);
  int xcds = g_geo_xcds[dev].load(std::memory_order_acquire);
  if (cus == 0 || xcds == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus < 1)
      cus = g.cus;
    if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess ||
        xcds < 1)
      xcds = g.xcds;
    g_geo_xcds[dev].store(xcds, std::memory_order_release);
    g_geo_cus[dev].store(cus, std::memory_order_release);
  }
  g.cus = cus;
  g.xcds = xcds;
  return g;
}

// log2 of the XCD count when it is a power of two (the remap deals workgroups by mask and
// shift), else -1 (no remap).
int xcd_shift_of(int xcds) {
  int s = 0;
  while ((1 << s) < xcds) ++s;
  return (1 << s) == xcds ? s : -1;
}

// ---- knobs (mirror of knobs::DECODE_MIN_KEYS, knobs.rs:163-168) ------------------------------
std::atomic<int> g_decode_min_keys{-1};

int decode_min_keys() {
  int v = g_decode_min_keys.load(std::memory_order_relaxed);
  if (v < 0) {
    int init = 8;
    if (const char* e = std::getenv("FFAI_DECODE_MIN_KEYS")) {
      char* end = nullptr;
      const long n = std::strtol(e, &end, 10);
      if (end != e && *end == '\0' && n >= 0 && n < (1L << 30)) init = (int)n;
    }
    int expected = -1;
    g_decode_min_keys.compare_exchange_strong(expected, init, std::memory_order_relaxed);
    v = g_decode_min_keys.load(std::memory_order_relaxed);
  }
  return v;
}

// Tuning and test hook, no counterpart in the reference: force which fwd items run as pieces.
// items > 0: that many items (the last ones of a non-causal grid, the longest ones of a causal
// grid) in `pieces` pieces each (1: no item split); items < 0: every item; items == 0 or
// pieces < 1: the planner's choice.
std::atomic<int> g_split_items{0};
std::atomic<int> g_split_pieces{0};

// Tuning knob, no counterpart in the reference: 64-key tiles per decode workgroup (0 = the
// planner's choice). Initialised from FFAI_DECODE_TILES_PER_WG on first use.
std::atomic<int> g_decode_tps{-1};

int decode_tiles_per_wg() {
  int v = g_decode_tps.load(std::memory_order_relaxed);
  if (v < 0) {
    int init = 0;
    if (const char* e = std::getenv("FFAI_DECODE_TILES_PER_WG")) {
      char* end = nullptr;
      const long n = std::strtol(e, &end, 10);
      if (end != e && *end == '\0' && n > 0 && n < (1L << 20)) init = (int)n;
    }
    int expected = -1;
    g_decode_tps.compare_exchange_strong(expected, init, std::memory_order_relaxed);
    v = g_decode_tps.load(std::memory_order_relaxed);
  }
  return v;
}

// Tuning knob, no counterpart in the reference: a forced launch shape of the fused kernel (-1:
// the planner's choice). Initialised from FFAI_ATTN_VARIANT on first use.
std::atomic<int> g_attn_variant{-2};

int attn_variant() {
  int v = g_attn_variant.load(std::memory_order_relaxed);
  if (v == -2) {
    int init = -1;
    if (const char* e = std::getenv("FFAI_ATTN_VARIANT"))
      if (e[0] >= '0' && e[0] <= '3' && e[1] == '\0') init = e[0] - '0';
    int expected = -2;
    g_attn_variant.compare_exchange_strong(expected, init, std::memory_order_relaxed);
    v = g_attn_variant.load(std::memory_order_relaxed);
  }
  return v;
}

constexpr int kMinSeq = 256;  // flash_attn.rs:55 (MIN_SEQ)
constexpr int kHD = 64;       // flash_attn.rs:50

size_t elem_size(int dt) { return dt == FFAI_F32 ? 4 : 2; }
bool valid_dtype(int dt) { return dt == FFAI_F32 || dt == FFAI_F16 || dt == FFAI_BF16; }

// ---- descriptor validation ----------------------------------------------------------------
// Returns FFAI_OK when served, FFAI_DECLINED when well formed but not served,
// FFAI_ERR_INVALID when malformed. `why` receives the reason.
int check_desc(const ffai_attn_desc* d, std::string* why) {
  if (!d) { *why = "null descriptor"; return FFAI_ERR_INVALID; }
  if (!valid_dtype(d->q_dtype) || !valid_dtype(d->kv_dtype) || !valid_dtype(d->out_dtype)) {
    *why = "unknown dtype"; return FFAI_ERR_INVALID;
  }
  if (d->batch < 1 || d->heads_q < 1 || d->heads_kv < 1 || d->q_len < 1 || d->kv_len < 1) {
    *why = "sizes must be positive"; return FFAI_ERR_INVALID;
  }
  if (d->heads_q % d->heads_kv != 0) { *why = "heads_q must be a multiple of heads_kv"; return FFAI_ERR_INVALID; }
  if (d->k_layout != FFAI_K_TRANSPOSED && d->k_layout != FFAI_K_ROWS) { *why = "unknown k_layout"; return FFAI_ERR_INVALID; }
  if (d->causal != 0 && d->causal != 1) { *why = "causal must be 0 or 1"; return FFAI_ERR_INVALID; }
  if (d->q_offset < 0) { *why = "q_offset must be >= 0"; return FFAI_ERR_INVALID; }
  if (!(d->scale > 0.f) || !std::isfinite(d->scale)) { *why = "scale must be finite and > 0"; return FFAI_ERR_INVALID; }
  const int64_t* all[4] = {d->q_strides, d->k_strides, d->v_strides, d->o_strides};
  for (const int64_t* s : all) {
    if (s[3] != 1) { *why = "innermost stride must be 1"; return FFAI_ERR_INVALID; }
    if (s[0] < 0 || s[1] < 0 || s[2] < 1) { *why = "strides must be non-negative (row stride >= 1)"; return FFAI_ERR_INVALID; }
  }
  // every index the kernels form must fit in int32 where they use int
  const int64_t big = (int64_t)1 << 30;
  if ((int64_t)d->batch * d->heads_q * ((d->q_len + 31) / 32) * ((d->kv_len + 63) / 64) > big) {
    *why = "problem too large"; return FFAI_ERR_INVALID;
  }
  // ---- served combinations
  if (d->head_dim != 64 && d->head_dim != 128) { *why = "head_dim must be 64 or 128"; return FFAI_DECLINED; }
  if (d->q_dtype == FFAI_F32) {
    if (d->out_dtype != FFAI_F32) { *why = "f32 queries produce f32 output"; return FFAI_DECLINED; }
    if (d->head_dim != 64) { *why = "f32 path serves head_dim 64"; return FFAI_DECLINED; }
  } else {
    if (d->kv_dtype != d->q_dtype) { *why = "16-bit queries need K/V of the same type"; return FFAI_DECLINED; }
    if (d->out_dtype != FFAI_F32 && d->out_dtype != d->q_dtype) {
      *why = "output must be f32 or the input type"; return FFAI_DECLINED;
    }
  }
  return FFAI_OK;
}

// Widest aligned access (elements, power of two <= max_vec) valid for every address formed
// from `base` plus multiples of the three outer strides plus multiples of max_vec.
int vec_of(const void* base, size_t esize, const int64_t* strides, int max_vec) {
  int v = max_vec;
  while (v > 1) {
    const uintptr_t bytes = (uintptr_t)v * esize;
    bool ok = ((uintptr_t)base % bytes) == 0;
    for (int i = 0; i < 3 && ok; ++i) ok = (strides[i] % v) == 0;
    if (ok) break;
    v >>= 1;
  }
  return v;
}

struct Plan {
  bool decode;  // decode_kernel (few rows per kv-head) instead of fwd_kernel
  int waves;    // decode: waves per workgroup
  int variant;
  int n_qblk;
  int n_split;          // pieces per split unit (decode) or split item (fwd)
  int tiles_per_split;  // 64-key tiles per piece (fwd: of the longest item)
  int n_work;
  // fwd: items [split_lo, split_hi) of n_items run as n_split pieces; dispatch sections
  int n_items, split_lo, split_hi, sec1_work;
  bool xcd_remap;
  bool x16;       // the four-wave x 64-row shape runs on fwd16_kernel (16x16x32 MFMA)
  int xcd_shift;  // log2 of the XCDs the sections are rounded to (0: one)
  int cus;
  size_t ws_bytes;
};

// Decode launch: 16-bit inputs and at most 32 query rows per (batch, kv-head), so one MFMA
// column block holds every row that reads a K/V head. Each wave of a workgroup takes one 64-key
// tile. A unit with more tiles than its workgroup's waves is split over workgroups, whose
// partials the unit's last workgroup merges in the same launch (counters at the workspace's
// start). When the units alone leave the GPU short of workgroups, a workgroup takes fewer tiles
// so that more of them stream keys at once.
// `max_ws`: the workspace available; a split that would need more is coarsened (more tiles per
// workgroup) until it fits, down to no split.
// f32 queries take the f32 decode kernel (decode_vec_kernel: the reference's decode arms, one
// query row per unit, head_dim 64); 16-bit ones the MFMA decode kernel (up to 32 rows).
bool plan_decode(const ffai_attn_desc* d, bool allow_split, size_t max_ws, const Geometry& geo,
                 Plan* p) {
  const int group = d->heads_q / d->heads_kv;
  const int64_t rows = (int64_t)group * d->q_len;
  const bool vec = d->q_dtype == FFAI_F32;
  if (!allow_split) return false;
  if (vec ? (rows != 1 || d->head_dim != 64) : rows > 32) return false;
  if (!vec && d->k_layout == FFAI_K_TRANSPOSED && d->kv_len < 4) return false;  // 4-key chunks
  // the DMA addresses a tile's rows (head_dim rows of K^T, 64 key rows of K and V) by 32-bit
  // byte offsets from the tile's first row
  // (f32 decode kernel: a head's K^T columns and V rows, (head_dim x k_st) and (kv_len x v_st)
  // elements, by 32-bit byte offsets from the head's base)
  const int64_t lim = int64_t(1) << 31;
  const int64_t es = vec ? (d->kv_dtype == FFAI_F32 ? 4 : 2) : 2;
  if (int64_t(std::max(d->head_dim, ffai::kBlockN)) * d->k_strides[2] * es >= lim ||
      int64_t(ffai::kBlockN) * d->v_strides[2] * es >= lim)
    return false;
  if (vec && ((int64_t)d->kv_len * d->v_strides[2] + d->head_dim) * es >= lim) return false;
  if (vec && d->k_layout == FFAI_K_TRANSPOSED &&
      ((int64_t)d->head_dim * d->k_strides[2] + d->kv_len) * es >= lim)
    return false;
  const int64_t units = (int64_t)d->batch * d->heads_kv;
  int64_t kv_blk = d->kv_len;
  if (d->causal) kv_blk = std::min<int64_t>(kv_blk, (int64_t)d->q_offset + d->q_len);
  const int64_t n_tiles = std::max<int64_t>(1, (kv_blk + ffai::kBlockN - 1) / ffai::kBlockN);
  // 16-bit kernel: LDS, 16 KB (32 KB at head_dim 128) a wave; f32 kernel: registers
  const int max_waves = (vec || d->head_dim == 64) ? 8 : 4;
  // A grid of at least kMinWorkgroups stays at max_waves tiles per workgroup; a smaller one is
  // split towards kSplitWorkgroups. A split costs the unit's last workgroup ~3.5 us of device-
  // scope round trips (its partial acknowledged, the counter, the other partials), about what a
  // second launch cost. Measured, beam-5 whisper-medium step (24 layers, graphs), tiles per
  // workgroup for the cross-attention (16 heads x 24 tiles): 1: 397 us, 2: 249, 3: 224, 4: 225,
  // 6: 241, 8: 253, 24 (unsplit): 375; the self-attention's 80 units split at all: 191-212
  // against 165 unsplit. (Measured on 256 CUs: the bounds scale with the device's CUs.)
  const int64_t kMinWorkgroups = std::max(1, geo.cus / 4), kSplitWorkgroups = std::max(1, geo.cus / 2);
  int64_t tps = max_waves;
  // The f32 decode kernel issues all of a wave's loads for its tile at once: a unit that its
  // workgroup's waves cover in one round of tiles stays whole (a split would add the merge's
  // round trips to one round of loads).
  if (units * ((n_tiles + tps - 1) / tps) < kMinWorkgroups && !(vec && n_tiles <= max_waves))
    tps = std::max<int64_t>(1, n_tiles * units / kSplitWorkgroups);
  // a tuning knob (ffai_set_decode_tiles_per_wg / FFAI_DECODE_TILES_PER_WG) may force it
  const int forced_tps = decode_tiles_per_wg();
  if (forced_tps > 0) tps = forced_tps;
  tps = std::min(tps, n_tiles);
  // splits need a counter slot per unit and stay within the merge's bound
  if (units > ffai::kCounterSlots) tps = n_tiles;
  if ((n_tiles + tps - 1) / tps > ffai::kMaxDecodeSplits)
    tps = (n_tiles + ffai::kMaxDecodeSplits - 1) / ffai::kMaxDecodeSplits;
  // every split is there for speed only: under a workspace cap, fewer and longer splits
  auto split_bytes = [&](int64_t t) {
    const int64_t n = (n_tiles + t - 1) / t;
    return n > 1 ? ffai::kCounterBytes + (size_t)(units * n * rows * (d->head_dim + 2) * 4) : 0;
  };
  while (tps < n_tiles && split_bytes(tps) > max_ws) ++tps;
  p->decode = true;
  // as many waves as tiles per workgroup (1, 2, 4 or max_waves); a workgroup's waves loop when
  // it holds more tiles than that
  int waves = 1;
  while (waves < tps && waves < max_waves) waves *= 2;
  p->waves = waves;
  p->variant = 0;
  p->n_qblk = 1;
  p->tiles_per_split = (int)tps;
  p->n_split = (int)((n_tiles + tps - 1) / tps);
  p->n_work = (int)(units * p->n_split);
  p->ws_bytes = split_bytes(tps);
  return true;
}

// `vector_ok`: the operands admit the decode kernel's vector accesses (it has no element-wise
// path; misaligned decode shapes take fwd_kernel).
// `max_ws`: the workspace available. Every split serves speed only, so a plan whose partials
// would exceed it runs its split items in fewer pieces, or whole, instead.
Plan make_plan(const ffai_attn_desc* d, bool allow_split, bool vector_ok,
               size_t max_ws = SIZE_MAX) {
  Plan p{};
  const Geometry geo = device_geometry();
  const int64_t cus = geo.cus;
  p.cus = geo.cus;
  p.xcd_shift = std::max(0, xcd_shift_of(geo.xcds));
  if (vector_ok && plan_decode(d, allow_split, max_ws, geo, &p)) return p;
  const int64_t bh = (int64_t)d->batch * d->heads_q;
  const bool f32 = d->q_dtype == FFAI_F32;
  const int n_tiles = (d->kv_len + ffai::kBlockN - 1) / ffai::kBlockN;
  auto work_of = [&](int v) {
    const int bm = ffai::block_m_of(v);
    return bh * ((d->q_len + bm - 1) / bm);
  };
  p.variant = ffai::kWave1;
  if (d->q_len > 32) p.variant = ffai::kWave4;
  if (!f32 && d->head_dim == 64 && d->q_len >= 256) p.variant = ffai::kWave4x2;
  if (p.variant == ffai::kWave4x2 && work_of(p.variant) < cus) p.variant = ffai::kWave4;
  // A one-wave workgroup holds a whole tile ring (48 KB of LDS in 16-bit, 68 KB in f32) for
  // one wave, so at most three (two) of them run per CU. Short grids of 16-bit rows fewer than
  // the encoder's (a prompt step: 228 rows) still run best on it; long runs and f32 keep four
  // waves and split the keys instead (measured: whisper-large-v3 window, 20 heads x 1500 rows,
  // bf16: 42.5 against 69.7 us; whisper-tiny f32: 66 against 154 us).
  if (p.variant == ffai::kWave4 && work_of(p.variant) < cus && !f32 && d->q_len < 256)
    p.variant = ffai::kWave1;
  // A forced launch shape (ffai_set_attn_variant, initialised from FFAI_ATTN_VARIANT: 0, 1, 2
  // or 3) where it is instantiated: a tuning knob. 3 is the four-wave x 64-row shape on
  // fwd16_kernel (16x16x32 MFMA), which measured 2-4% slower than fwd_kernel's and is not
  // chosen otherwise.
  const int forced = attn_variant();
  p.x16 = false;
  if (forced == ffai::kWave1 || forced == ffai::kWave4 ||
      ((forced == ffai::kWave4x2 || forced == ffai::kWave4x2x16) && !f32 && d->head_dim == 64)) {
    p.variant = forced == ffai::kWave4x2x16 ? ffai::kWave4x2 : forced;
    p.x16 = forced == ffai::kWave4x2x16;
  }
  const int64_t items = work_of(p.variant);
  const int bm = ffai::block_m_of(p.variant);
  p.n_qblk = (d->q_len + bm - 1) / bm;
  p.n_items = (int)items;
  p.n_split = 1;
  p.tiles_per_split = n_tiles;
  p.split_lo = p.split_hi = 0;
  // Short grids run every item in pieces (merged in the launch). 16-bit four-wave grids of fewer
  // items than CUs take up to three, so that about every CU holds a piece: whisper-tiny (6
  // heads, 72 items) bf16 17.1 us in 3 pieces against 26.3 whole (6: 17.0); a whisper-large-v3
  // window (20 heads, 240 items) runs whole: 27.4 us against 26.6 in 2 and 27.4 in 3. f32
  // four-wave grids (two workgroups per CU) of fewer items than CUs fill the 512 slots:
  // whisper-tiny f32 50.5 us in 6 pieces against 56.4 in 3, 66.2 in 4 (288 works: a second
  // round) and 77.9 in 2; up to 1024 items they aim at ~4096 waves (300 items: 183 us in 4
  // pieces against 236 whole, 197 in 2, 211 in 8). One-wave 16-bit grids (prompt steps,
  // misaligned decode) fill at most the 768 slots of three workgroups per CU (48 KB of LDS
  // each): the cross-attention of 228 tokens, 128 items, 14.6 us in 6 pieces against 15.4 in 5,
  // 15.7 in 4 and 19.2 in 7 (896 workgroups: a second round). One-wave f32 grids (two per CU)
  // keep about 512 workgroups: f32 decode over 1500 keys, 6 heads: 25.9 us in 24 pieces, 32.7
  // in 8, 193 whole; 80 items: 55.8 in 7, 73.9 in 4, 86.8 in 24.
  // (Measured on 256 CUs; the slot counts below scale with the device's CUs.)
  int64_t want = 1;
  if (p.variant == ffai::kWave1) {
    if (f32 && items < 2 * cus) want = std::min<int64_t>(24, (2 * cus + items - 1) / items);
    else if (!f32 && items < 3 * cus) want = std::min<int64_t>(ffai::kMaxFwdSplits, 3 * cus / items);
  } else if (items < cus) {
    want = f32 ? 2 * cus / items : std::max<int64_t>(1, std::min<int64_t>(3, cus / items));
  } else if (f32 && items < 4 * cus) {
    want = (16 * cus + 4 * items - 1) / (4 * items);
  }
  // FFAI_ATTN_SPLITS (> 0) forces the pieces of every item: a tuning knob.
  static const int forced_splits = [] {
    const char* e = std::getenv("FFAI_ATTN_SPLITS");
    return e ? std::atoi(e) : 0;
  }();
  if (forced_splits > 0) want = forced_splits;
  int64_t lo = 0, hi = want > 1 ? items : 0;
  if (want == 1 && !f32) {
    // Long grids split only the items that would leave the GPU partly idle at the end.
    // Resident workgroups: four-wave x 64 rows and head_dim 128 two per CU (VGPRs, LDS), four
    // waves x 32 rows at head_dim 64 and one-wave shapes three.
    const int64_t slots = cus * ((p.variant == ffai::kWave4x2 || d->head_dim == 128) ? 2 : 3);
    if (d->causal) {
      // Causal, rank order longest first: when the longest item is well above a resident slot's
      // share of the work, it bounds the launch; the items longer than half the longest go in 2
      // pieces. Qwen2-VL-2B prefill (Hq 12, S 4096, D 128: 384 items of 2..64 tiles, the 192
      // longest split): 72.5 us against 89.3 unsplit (same run; 108 before rank-order dispatch;
      // 144 / 288 items 81.8 / 76.3, 3 pieces 96.0).
      const int64_t nbh = (int64_t)d->batch * d->heads_q;
      auto tiles_of = [&](int64_t qb) {  // keys any row of query block qb sees, in tiles
        const int64_t kv = std::min<int64_t>(d->kv_len, std::max<int64_t>(0, d->q_offset + std::min<int64_t>((qb + 1) * bm, d->q_len)));
        return (kv + ffai::kBlockN - 1) / ffai::kBlockN;
      };
      int64_t total = 0;
      for (int64_t qb = 0; qb < p.n_qblk; ++qb) total += tiles_of(qb) * nbh;
      const int64_t longest = tiles_of(p.n_qblk - 1);
      if (longest >= 4 && longest * 5 > 6 * (total / slots)) {
        int64_t n = 0;  // rank order: query blocks descending, all (batch, head) of each
        for (int64_t qb = p.n_qblk - 1; qb >= 0 && 2 * tiles_of(qb) > longest; --qb) n += nbh;
        if (n > 0) { want = 2; lo = 0; hi = n; }
      }
    } else if (items > slots && n_tiles >= 8) {
      // Non-causal: a last round of at most a quarter of the slots runs its items in 4 pieces.
      // whisper-small (B8 H12 T1500: 576 items, 512 resident): 75.2 us with the last 64 items
      // in 4 pieces against 88.0 unsplit (2: 78.1, 6: 87.5).
      const int64_t tail = items % slots;
      if (tail > 0 && 4 * tail <= slots) {
        want = 4; lo = items - tail; hi = items;
      } else if (tail > 0 && 3 * tail >= slots && p.variant == ffai::kWave4x2) {
        // A last round of at least a third of the slots: the last k items go in n pieces so
        // that the last round holds exactly one work per slot, tail - k whole items and k * n
        // pieces. A CU then pairs a whole item with a piece, and the whole item runs alone once
        // the piece is done. whisper-large-v3 (1920 items, a last round of 384: its last 128 in
        // 2 pieces, 2048 works): 211.3 us against 215.7 unsplit (5 interleaved rounds; the last
        // 64 in 3 pieces, also 2048 works, 213.2; 2048 +- 64 or 128 works 215-221).
        const int64_t n = 2 * tail >= slots ? 2 : 3;
        const int64_t k = (slots - tail) / (n - 1);
        if (k >= 1 && k <= tail) { want = n; lo = items - k; hi = items; }
      }
    }
  }
  // ffai_set_fwd_split_override forces the split items and their pieces.
  const int o_items = g_split_items.load(std::memory_order_relaxed);
  const int o_pieces = g_split_pieces.load(std::memory_order_relaxed);
  const bool overridden = o_items != 0 && o_pieces >= 1;
  if (overridden) {  // pieces 1: nothing split
    want = o_pieces;
    const int64_t n = o_items < 0 ? items : std::min<int64_t>(o_items, items);
    // non-causal: the items dispatched last; causal: the longest, dispatched first
    lo = d->causal ? 0 : items - n;
    hi = d->causal ? n : items;
  }
  // a counter slot per split item; the partials addressed by 32-bit byte offsets
  want = std::min<int64_t>({want, n_tiles, ffai::kMaxFwdSplits});
  // no piece without tiles: as many pieces as ceil(tiles / n)-tile ranges cover the keys (a
  // forced layout is kept as given)
  if (want > 1 && !overridden) want = (n_tiles + (n_tiles + want - 1) / want - 1) / ((n_tiles + want - 1) / want);
  auto bytes_of = [&](int64_t n) { return (hi - lo) * n * bm * (d->head_dim + 2) * 4; };
  // under a workspace cap, fewer pieces (a forced layout is kept as given: it is refused later
  // if it does not fit)
  while (!overridden && want > 1 && ffai::kCounterBytes + (size_t)bytes_of(want) > max_ws) --want;
  if (allow_split && want > 1 && hi > lo && hi - lo <= ffai::kCounterSlots &&
      bytes_of(want) < (int64_t(1) << 31)) {
    p.n_split = (int)want;
    p.tiles_per_split = (n_tiles + p.n_split - 1) / p.n_split;
    p.split_lo = (int)lo;
    p.split_hi = (int)hi;
  }
  const int64_t pieces = (int64_t)(p.split_hi - p.split_lo) * p.n_split;
  p.n_work = (int)(items + pieces - (p.split_hi - p.split_lo));
  // Dispatch. Causal: rank order (longest first) across all XCDs. Otherwise each section's works
  // go to the XCDs in contiguous runs (one head's query blocks, one item's pieces share an L2);
  // split items at the end of the grid form the second section, so that they are dealt to every
  // XCD and dispatched after the whole items.
  p.xcd_remap = !d->causal && xcd_shift_of(geo.xcds) > 0;
  p.sec1_work = (p.split_hi > p.split_lo && p.split_lo > 0) ? p.split_lo : p.n_work;
  const size_t part_bytes = (size_t)pieces * bm * (d->head_dim + 2) * 4;
  p.ws_bytes = pieces > 0 ? ffai::kCounterBytes + part_bytes : 0;
  return p;
}

// Workspace for a descriptor whatever the operands' alignment turns out to be.
size_t plan_ws_bytes(const ffai_attn_desc* d) {
  return std::max(make_plan(d, true, true).ws_bytes, make_plan(d, true, false).ws_bytes);
}

// ---- allocation-free entry point: a library-owned split-key scratch per device ----------------
// ffai_attn_fwd_noalloc keeps the split counters and split-key partials in this array instead
// of a caller workspace (the counters start at zero, as a static array does, and every call
// leaves them zero). Its plans are ffai_attn_fwd's with the workspace capped at kScratchBytes:
// a plan whose partials would not fit runs its split items in fewer pieces, or whole (splits
// serve speed only), so only a layout forced by ffai_set_fwd_split_override can be refused.
// In host code `scratch` names a host-side stand-in, not device memory: the device address is
// taken once per device with hipGetSymbolAddress (that device current) and kept in
// g_scratch_ptr; only that address is handed to kernels. The array lives until the process
// ends, and every call on one device shares it.
constexpr size_t kScratchBytes = size_t(48) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch (hipGetSymbolAddress on first use per device).
int scratch_for_current(void** ptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(FFAI_ERR_HIP, "hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return fail(FFAI_ERR_DEVICE, "device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(FFAI_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return FFAI_OK;
}

#ifdef FFAI_STAMPS
// Diagnostic library only (libffai_attn_stamps.so, built with FFAI_STAMPS): the device buffer
// the kernels write their phase times into (see attn_common.cuh), set by ffai_stamps_set.
std::atomic<uint64_t*> g_stamp_buf{nullptr};
std::atomic<size_t> g_stamp_bytes{0};
#endif

// `use_scratch`: the partials go to the library's scratch (ws and ws_bytes are ignored).
int run_fwd(const ffai_attn_desc* d, const void* q, const void* k, const void* v, void* out,
            void* ws, size_t ws_bytes, void* stream, bool allow_split, bool use_scratch = false) {
  g_last_error.clear();
  std::string why;
  const int rc = check_desc(d, &why);
  if (rc == FFAI_DECLINED) return fail(FFAI_DECLINED, "declined: " + why);
  if (rc != FFAI_OK) return fail(rc, why);
  if (!q || !k || !v || !out) return fail(FFAI_ERR_INVALID, "null operand pointer");
  const size_t qs = elem_size(d->q_dtype), ks = elem_size(d->kv_dtype), os = elem_size(d->out_dtype);
  if ((uintptr_t)q % qs || (uintptr_t)k % ks || (uintptr_t)v % ks || (uintptr_t)out % os)
    return fail(FFAI_ERR_INVALID, "operand pointer not aligned to its element size");

  const bool f32 = d->q_dtype == FFAI_F32;
  const bool kt = d->k_layout == FFAI_K_TRANSPOSED;
  // The kernels' vector accesses: Q rows 16 B (4 f32 or 8 16-bit elements); K rows and V rows
  // 16 B in the 16-bit kernels, 4 elements in the f32 kernel; K^T rows 4 keys; O 4 elements.
  const int need_q = f32 ? 4 : 8, need_kv = f32 ? 4 : 8, need_k = kt ? 4 : need_kv;
  const bool aligned = vec_of(q, qs, d->q_strides, need_q) == need_q &&
                       vec_of(k, ks, d->k_strides, need_k) == need_k &&
                       vec_of(v, ks, d->v_strides, need_kv) == need_kv &&
                       vec_of(out, os, d->o_strides, 4) == 4;

  const Plan pl = make_plan(d, allow_split, aligned, use_scratch ? kScratchBytes : SIZE_MAX);
  if (use_scratch && pl.ws_bytes > kScratchBytes)
    return fail(FFAI_ERR_WORKSPACE,
                "this shape needs " + std::to_string(pl.ws_bytes) +
                    " bytes of split-key partials; the allocation-free entry point holds at most " +
                    std::to_string(kScratchBytes) + " (use ffai_attn_fwd with a workspace)");
  const int dev = check_device();
  if (dev != FFAI_OK) return dev;
  if (use_scratch && pl.ws_bytes > 0) {
    const int src = scratch_for_current(&ws);
    if (src != FFAI_OK) return src;
    ws_bytes = kScratchBytes;
  }
  if (pl.ws_bytes > 0) {
    if (!ws || ws_bytes < pl.ws_bytes)
      return fail(FFAI_ERR_WORKSPACE, "workspace smaller than ffai_attn_workspace_bytes");
    if ((uintptr_t)ws % 16) return fail(FFAI_ERR_INVALID, "workspace must be 16-byte aligned");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int mode = f32 ? ffai::kF32 : (d->q_dtype == FFAI_BF16 ? ffai::kBF16 : ffai::kF16);
  const int kvt = d->kv_dtype == FFAI_F32 ? ffai::kF32 : (d->kv_dtype == FFAI_BF16 ? ffai::kBF16 : ffai::kF16);
  const int ot = d->out_dtype == FFAI_F32 ? ffai::kF32 : (d->out_dtype == FFAI_BF16 ? ffai::kBF16 : ffai::kF16);

  // workspace: split counters first (decode plans), then the partials
  float* partials = pl.ws_bytes > 0
                        ? reinterpret_cast<float*>(static_cast<char*>(ws) + ffai::kCounterBytes)
                        : nullptr;
  if (pl.decode) {
    ffai::DecodeParams p{};
    p.q = q; p.k = k; p.v = v; p.o = out;
    p.ws = partials;
    p.counters = static_cast<int32_t*>(ws);
    p.kv_lens = d->kv_lens;
    p.q_sb = d->q_strides[0]; p.q_sh = d->q_strides[1]; p.q_st = d->q_strides[2];
    p.k_sb = d->k_strides[0]; p.k_sh = d->k_strides[1]; p.k_st = d->k_strides[2];
    p.v_sb = d->v_strides[0]; p.v_sh = d->v_strides[1]; p.v_st = d->v_strides[2];
    p.o_sb = d->o_strides[0]; p.o_sh = d->o_strides[1]; p.o_st = d->o_strides[2];
    p.B = d->batch; p.Hkv = d->heads_kv; p.group = d->heads_q / d->heads_kv;
    p.Tq = d->q_len; p.Tk = d->kv_len;
    p.causal = d->causal; p.q_offset = d->q_offset;
    p.n_split = pl.n_split; p.tiles_per_split = pl.tiles_per_split; p.n_work = pl.n_work;
    p.scale_log2 = d->scale * 1.4426950408889634f;
#ifdef FFAI_STAMPS
    p.stamps = g_stamp_buf.load();
    p.stamp_wgs = (int)std::min<size_t>(g_stamp_bytes.load() / 64, INT32_MAX);
#endif
    const hipError_t e = f32 ? ffai::launch_decode_vec(p, kvt, kt, pl.waves, s)
                             : ffai::launch_decode(p, mode, ot, d->head_dim, kt, pl.waves, s);
    if (e != hipSuccess) return fail(FFAI_ERR_HIP, std::string("decode launch: ") + hipGetErrorString(e));
    return FFAI_OK;
  }

  ffai::FwdParams p{};
  p.q = q; p.k = k; p.v = v; p.o = out;
  p.ws = partials;
  p.kv_lens = d->kv_lens;
  p.q_sb = d->q_strides[0]; p.q_sh = d->q_strides[1]; p.q_st = d->q_strides[2];
  p.k_sb = d->k_strides[0]; p.k_sh = d->k_strides[1]; p.k_st = d->k_strides[2];
  p.v_sb = d->v_strides[0]; p.v_sh = d->v_strides[1]; p.v_st = d->v_strides[2];
  p.o_sb = d->o_strides[0]; p.o_sh = d->o_strides[1]; p.o_st = d->o_strides[2];
  p.B = d->batch; p.Hq = d->heads_q; p.Hkv = d->heads_kv; p.Tq = d->q_len; p.Tk = d->kv_len;
  p.causal = d->causal; p.q_offset = d->q_offset;
  p.n_qblk = pl.n_qblk;
  p.split_lo = pl.split_lo; p.split_hi = pl.split_hi; p.n_split = pl.n_split;
  p.n_work = pl.n_work;
  p.sec1_work = pl.sec1_work;
  p.xcd_shift = pl.xcd_shift;
  p.cus = pl.cus;
  {
    const int xr = 1 << pl.xcd_shift;
    p.sec1_wgs = (pl.sec1_work + xr - 1) / xr * xr;
  }
  p.xcd_remap = pl.xcd_remap ? 1 : 0;
  p.counters = static_cast<int32_t*>(ws);
  p.aligned = aligned;
  {
    // the DMA path addresses a tile's rows by 32-bit byte offsets from the tile's first key
    const int64_t k_rows = kt ? d->head_dim : ffai::kBlockN;
    const int64_t lim = int64_t(1) << 31;
    p.dma = aligned && !f32 && k_rows * d->k_strides[2] * 2 < lim &&
            int64_t(ffai::kBlockN) * d->v_strides[2] * 2 < lim;
  }
  p.scale_log2 = d->scale * 1.4426950408889634f;
  {
    static const bool pair_off = [] {
      const char* e = std::getenv("FFAI_FWD_PAIR_STORE");
      return e && e[0] == '0';
    }();
    p.o_pair = !pair_off && !f32 && d->out_dtype != FFAI_F32 && d->head_dim == 64 &&
               vec_of(out, os, d->o_strides, 8) == 8;
  }
#ifdef FFAI_STAMPS
  p.stamps = g_stamp_buf.load();
  p.stamp_wgs = (int)std::min<size_t>(g_stamp_bytes.load() / 1024, INT32_MAX);
#endif
  const hipError_t e = ffai::launch_fwd(p, mode, kvt, ot, d->head_dim, kt,
                                        pl.x16 ? ffai::kWave4x2x16 : pl.variant, s);
  if (e != hipSuccess) return fail(FFAI_ERR_HIP, std::string("fwd launch: ") + hipGetErrorString(e));
  return FFAI_OK;
}

// ---- tensor-view helpers for the mirrors -----------------------------------------------------
bool contiguous(const ffai_tensor* t) {
  int64_t expect = 1;
  for (int i = 3; i >= 0; --i) {
    if (t->dims[i] != 1 && t->strides[i] != expect) return false;
    expect *= t->dims[i];
  }
  return true;
}

bool dims_are(const ffai_tensor* t, int64_t a, int64_t b, int64_t c, int64_t d) {
  return t->dims[0] == a && t->dims[1] == b && t->dims[2] == c && t->dims[3] == d;
}

void packed_strides(int64_t* s, int64_t d1, int64_t d2, int64_t d3) {
  s[3] = 1; s[2] = d3; s[1] = d2 * d3; s[0] = d1 * d2 * d3;
}

// The shape part of attend's accept set (flash_attn.rs:218-262), shared by ffai_attend and
// ffai_attend_workspace_bytes. Returns FFAI_OK or FFAI_DECLINED.
int attend_accepts(const ffai_tensor* q, const ffai_tensor* kt, const ffai_tensor* v, int masked,
                   std::string* why) {
  if (masked) { *why = "masked attention is served by the caller's fallback"; return FFAI_DECLINED; }
  if (!q->on_device || !kt->on_device || !v->on_device) { *why = "host tensors"; return FFAI_DECLINED; }
  if (q->dtype != FFAI_F32) { *why = "q must be f32"; return FFAI_DECLINED; }
  const bool kv_half = kt->dtype == FFAI_F16;
  if (kv_half && v->dtype != FFAI_F16) { *why = "K f16 needs V f16"; return FFAI_DECLINED; }
  if (!kv_half && (kt->dtype != FFAI_F32 || v->dtype != FFAI_F32)) { *why = "K/V must be f32 or f16"; return FFAI_DECLINED; }
  const int64_t b = q->dims[0], heads = q->dims[1], qlen = q->dims[2], hd = q->dims[3];
  if (b != 1 || hd != kHD) { *why = "batch 1, head_dim 64 only"; return FFAI_DECLINED; }
  if (kt->dims[0] != 1 || kt->dims[1] != heads || kt->dims[2] != kHD) { *why = "kt shape"; return FFAI_DECLINED; }
  const int64_t keys = kt->dims[3];
  if (!dims_are(v, 1, heads, keys, kHD)) { *why = "v shape"; return FFAI_DECLINED; }
  const int64_t floor = qlen == 1 ? decode_min_keys() : kMinSeq;
  if (keys < floor) { *why = "fewer keys than the floor"; return FFAI_DECLINED; }
  if (qlen != 1 && qlen != keys) { *why = "qlen must be 1 or keys"; return FFAI_DECLINED; }
  return FFAI_OK;
}

void attend_desc(const ffai_tensor* q, const ffai_tensor* kt, const ffai_tensor* v,
                 ffai_attn_desc* d) {
  const int heads = (int)q->dims[1], qlen = (int)q->dims[2], keys = (int)kt->dims[3];
  ffai_attn_desc_init(d, FFAI_F32, kt->dtype, FFAI_F32, 1, heads, heads, qlen, keys, kHD,
                      FFAI_K_TRANSPOSED);
  (void)v;
}

// attend_merged's accept set (flash_attn.rs:135-153).
int merged_accepts(const ffai_tensor* q, const ffai_tensor* kt, const ffai_tensor* v,
                   std::string* why) {
  const int64_t b = q->dims[0], heads = q->dims[1], qlen = q->dims[2], hd = q->dims[3];
  if (b != 1 || hd != kHD || !q->on_device || !kt->on_device || !v->on_device) {
    *why = "batch 1, head_dim 64, device tensors only"; return FFAI_DECLINED;
  }
  if (q->dtype != FFAI_F32 || kt->dtype != FFAI_F32 || v->dtype != FFAI_F32) {
    *why = "f32 only"; return FFAI_DECLINED;
  }
  if (kt->dims[0] != 1 || kt->dims[1] != heads || kt->dims[2] != kHD) { *why = "kt shape"; return FFAI_DECLINED; }
  const int64_t keys = kt->dims[3];
  if (!dims_are(v, 1, heads, keys, kHD) || qlen != keys || keys < kMinSeq) {
    *why = "v shape, qlen != keys or keys < 256"; return FFAI_DECLINED;
  }
  return FFAI_OK;
}

// Merged layout: query row i of head h lands at i*H*64 + h*64 (flash_attn.rs:188-207).
void merged_desc(const ffai_tensor* q, const ffai_tensor* kt, const ffai_tensor* v,
                 ffai_attn_desc* d) {
  attend_desc(q, kt, v, d);
  const int64_t heads = q->dims[1], keys = kt->dims[3];
  d->o_strides[0] = keys * heads * kHD;
  d->o_strides[1] = kHD;
  d->o_strides[2] = heads * kHD;
  d->o_strides[3] = 1;
}

}  // namespace

// Shared with the other C-ABI translation units (kv_cache.hip) through attn_kernels.h.
namespace ffai {
int api_fail(int code, const char* msg) { return fail(code, msg); }
void api_clear_error() { g_last_error.clear(); }
int api_check_device() { return check_device(); }
}  // namespace ffai

extern "C" {

void ffai_attn_desc_init(ffai_attn_desc* d, int32_t q_dtype, int32_t kv_dtype, int32_t out_dtype,
                         int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t q_len,
                         int32_t kv_len, int32_t head_dim, int32_t k_layout) {
  if (!d) return;
  std::memset(d, 0, sizeof(*d));
  d->q_dtype = q_dtype; d->kv_dtype = kv_dtype; d->out_dtype = out_dtype;
  d->batch = batch; d->heads_q = heads_q; d->heads_kv = heads_kv;
  d->q_len = q_len; d->kv_len = kv_len; d->head_dim = head_dim;
  d->k_layout = k_layout;
  d->scale = 1.0f;
  packed_strides(d->q_strides, heads_q, q_len, head_dim);
  if (k_layout == FFAI_K_TRANSPOSED) packed_strides(d->k_strides, heads_kv, head_dim, kv_len);
  else packed_strides(d->k_strides, heads_kv, kv_len, head_dim);
  packed_strides(d->v_strides, heads_kv, kv_len, head_dim);
  packed_strides(d->o_strides, heads_q, q_len, head_dim);
}

int ffai_attn_serves(const ffai_attn_desc* d) {
  std::string why;
  return check_desc(d, &why) == FFAI_OK ? 1 : 0;
}

int ffai_attn_workspace_bytes(const ffai_attn_desc* d, size_t* bytes) {
  if (!bytes) return fail(FFAI_ERR_INVALID, "null bytes pointer");
  *bytes = 0;
  std::string why;
  const int rc = check_desc(d, &why);
  if (rc == FFAI_DECLINED) return fail(FFAI_DECLINED, "declined: " + why);
  if (rc != FFAI_OK) return fail(rc, why);
  *bytes = plan_ws_bytes(d);
  return FFAI_OK;
}

int ffai_attn_fwd(const ffai_attn_desc* d, const void* q, const void* k, const void* v,
                  void* out, void* workspace, size_t workspace_bytes, void* stream) {
  return run_fwd(d, q, k, v, out, workspace, workspace_bytes, stream, true);
}

int ffai_attn_fwd_noalloc(const ffai_attn_desc* d, const void* q, const void* k, const void* v,
                          void* out, void* stream) {
  return run_fwd(d, q, k, v, out, nullptr, 0, stream, true, true);
}

size_t ffai_attn_noalloc_scratch_bytes(void) { return kScratchBytes; }

int ffai_attn_plan_info(const ffai_attn_desc* d, int32_t info[5]) {
  if (!info) return fail(FFAI_ERR_INVALID, "null info pointer");
  std::string why;
  const int rc = check_desc(d, &why);
  if (rc == FFAI_DECLINED) return fail(FFAI_DECLINED, "declined: " + why);
  if (rc != FFAI_OK) return fail(rc, why);
  const Plan p = make_plan(d, true, true);
  info[0] = p.decode ? 1 : 0;
  info[1] = p.decode ? p.waves : (p.x16 ? ffai::kWave4x2x16 : p.variant);
  info[2] = p.n_split;
  info[3] = p.tiles_per_split;
  info[4] = p.n_work;
  return FFAI_OK;
}

int ffai_attn_noalloc_plan_info(const ffai_attn_desc* d, int32_t info[5], size_t* bytes) {
  if (!info || !bytes) return fail(FFAI_ERR_INVALID, "null info or bytes pointer");
  *bytes = 0;
  std::string why;
  const int rc = check_desc(d, &why);
  if (rc == FFAI_DECLINED) return fail(FFAI_DECLINED, "declined: " + why);
  if (rc != FFAI_OK) return fail(rc, why);
  const Plan p = make_plan(d, true, true, kScratchBytes);
  info[0] = p.decode ? 1 : 0;
  info[1] = p.decode ? p.waves : (p.x16 ? ffai::kWave4x2x16 : p.variant);
  info[2] = p.n_split;
  info[3] = p.tiles_per_split;
  info[4] = p.n_work;
  *bytes = p.ws_bytes;
  return FFAI_OK;
}

int ffai_attn_plan_splits(const ffai_attn_desc* d, int32_t info[3]) {
  if (!info) return fail(FFAI_ERR_INVALID, "null info pointer");
  std::string why;
  const int rc = check_desc(d, &why);
  if (rc == FFAI_DECLINED) return fail(FFAI_DECLINED, "declined: " + why);
  if (rc != FFAI_OK) return fail(rc, why);
  const Plan p = make_plan(d, true, true);
  info[0] = p.decode ? 0 : p.n_items;
  info[1] = p.decode ? 0 : p.split_lo;
  info[2] = p.decode ? 0 : p.split_hi;
  return FFAI_OK;
}

int ffai_serves(const ffai_tensor* kt, const ffai_tensor* v) {
  if (!kt || !v || !kt->on_device || !v->on_device) return 0;
  if (kt->dims[0] != 1 || kt->dims[2] != kHD || v->dims[0] != 1 || v->dims[3] != kHD) return 0;
  const int64_t keys = kt->dims[3];
  return (kt->dims[1] == v->dims[1] && v->dims[2] == keys &&
          keys >= std::max<int64_t>(kMinSeq, decode_min_keys()))
             ? 1
             : 0;
}

int ffai_attend_workspace_bytes(const ffai_tensor* q, const ffai_tensor* kt, const ffai_tensor* v,
                                size_t* bytes) {
  if (!bytes) return fail(FFAI_ERR_INVALID, "null bytes pointer");
  *bytes = 0;
  if (!q || !kt || !v) return fail(FFAI_ERR_INVALID, "null tensor");
  std::string why;
  if (attend_accepts(q, kt, v, 0, &why) != FFAI_OK) return fail(FFAI_DECLINED, "declined: " + why);
  ffai_attn_desc d;
  attend_desc(q, kt, v, &d);
  *bytes = plan_ws_bytes(&d);
  return FFAI_OK;
}

int ffai_attend(const ffai_tensor* q, const ffai_tensor* kt, const ffai_tensor* v, int masked,
                ffai_tensor* out, void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (!q || !kt || !v || !out) return fail(FFAI_ERR_INVALID, "null tensor");
  std::string why;
  if (attend_accepts(q, kt, v, masked, &why) != FFAI_OK) return fail(FFAI_DECLINED, "declined: " + why);
  const int64_t heads = q->dims[1], qlen = q->dims[2];
  // cpu_fwd's own checks (flash_attn.rs:289-296, 357-363): the f16 arm is the decode shape only;
  // anything else that is not all-f32 and contiguous is an error, not a decline.
  if (kt->dtype == FFAI_F16 && qlen != 1) return fail(FFAI_ERR_INVALID, "flash-attn: f32 only");
  if (!contiguous(q) || !contiguous(kt) || !contiguous(v))
    return fail(FFAI_ERR_INVALID, "flash-attn: contiguous operands only");
  if (out->dtype != FFAI_F32 || !out->on_device || !dims_are(out, 1, heads, qlen, kHD) || !contiguous(out))
    return fail(FFAI_ERR_INVALID, "out must be a contiguous f32 (1,H,qlen,64) device tensor");
  ffai_attn_desc d;
  attend_desc(q, kt, v, &d);
  return run_fwd(&d, q->data, kt->data, v->data, out->data, workspace, workspace_bytes, stream, true);
}

int ffai_attend_merged(const ffai_tensor* q, const ffai_tensor* kt, const ffai_tensor* v,
                       ffai_tensor* out, void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (!q || !kt || !v || !out) return fail(FFAI_ERR_INVALID, "null tensor");
  std::string why;
  if (merged_accepts(q, kt, v, &why) != FFAI_OK) return fail(FFAI_DECLINED, "declined: " + why);
  const int64_t heads = q->dims[1], keys = kt->dims[3];
  if (!contiguous(q) || !contiguous(kt) || !contiguous(v))
    return fail(FFAI_ERR_INVALID, "flash-attn-merged: contiguous only");
  if (out->dtype != FFAI_F32 || !out->on_device || !dims_are(out, 1, keys, heads * kHD, 1) ||
      out->strides[0] != keys * heads * kHD || out->strides[1] != heads * kHD || out->strides[2] != 1)
    return fail(FFAI_ERR_INVALID, "out must be a contiguous f32 (1,T,H*64) device tensor");
  ffai_attn_desc d;
  merged_desc(q, kt, v, &d);
  return run_fwd(&d, q->data, kt->data, v->data, out->data, workspace, workspace_bytes, stream,
                 true);
}

int ffai_attend_merged_workspace_bytes(const ffai_tensor* q, const ffai_tensor* kt,
                                       const ffai_tensor* v, size_t* bytes) {
  if (!bytes) return fail(FFAI_ERR_INVALID, "null bytes pointer");
  *bytes = 0;
  if (!q || !kt || !v) return fail(FFAI_ERR_INVALID, "null tensor");
  std::string why;
  if (merged_accepts(q, kt, v, &why) != FFAI_OK) return fail(FFAI_DECLINED, "declined: " + why);
  ffai_attn_desc d;
  merged_desc(q, kt, v, &d);
  *bytes = plan_ws_bytes(&d);
  return FFAI_OK;
}

int ffai_get_decode_min_keys(void) { return decode_min_keys(); }

int ffai_get_decode_tiles_per_wg(void) { return decode_tiles_per_wg(); }

void ffai_set_decode_tiles_per_wg(int n) {
  if (n >= 0) g_decode_tps.store(n, std::memory_order_relaxed);
}

void ffai_set_attn_variant(int variant) {
  g_attn_variant.store(variant >= 0 && variant <= 3 ? variant : -1, std::memory_order_relaxed);
}

int ffai_get_attn_variant(void) { return attn_variant(); }

void ffai_set_geometry_override(int cus, int xcds) {
  const bool on = cus > 0 && xcds > 0;
  g_geo_override_xcds.store(on ? xcds : 0, std::memory_order_relaxed);
  g_geo_override_cus.store(on ? cus : 0, std::memory_order_relaxed);
}

void ffai_set_fwd_split_override(int items, int pieces) {
  g_split_items.store(items, std::memory_order_relaxed);
  g_split_pieces.store(pieces, std::memory_order_relaxed);
}

void ffai_get_fwd_split_override(int* items, int* pieces) {
  if (items) *items = g_split_items.load(std::memory_order_relaxed);
  if (pieces) *pieces = g_split_pieces.load(std::memory_order_relaxed);
}

void ffai_set_decode_min_keys(int n) {
  if (n >= 0) g_decode_min_keys.store(n, std::memory_order_relaxed);
}

const char* ffai_attn_last_error(void) { return g_last_error.c_str(); }

#ifdef FFAI_STAMPS
// Diagnostic library only: record phase times of the fused kernel's 16-bit path (1024 bytes per
// workgroup: 4 waves x 32 u64) and the 16-bit decode kernel (64 bytes per workgroup) into
// `buf` (device memory, `bytes` long; workgroups past it record nothing). NULL stops recording.
int ffai_stamps_set(void* buf, size_t bytes) {
  g_stamp_bytes.store(buf ? bytes : 0);
  g_stamp_buf.store(static_cast<uint64_t*>(buf));
  return FFAI_OK;
}
#endif

int ffai_attn_abi_version(void) { return FFAI_ATTN_ABI_VERSION; }

}  // extern "C"
