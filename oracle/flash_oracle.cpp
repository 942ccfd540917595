// CPU oracle for the fused attention path. TEST INFRASTRUCTURE ONLY.
//
// This file restates, in C++ with AVX2/FMA/F16C, the algorithm of the reference's fused
// attention kernel (crates/ffai-mercury/src/asr/flash_attn.rs). It exists to check the HIP
// kernels and to time the reference's CPU algorithm on the same host. Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the product path
// (ffai_amd/) never does.
//
// Two groups of entry points:
//   * reference restatement - follows flash_attn.rs step by step (tile sizes BQ=64/BK=256,
//     4x16 register blocks, the reference's exp polynomial, online rescale with the
//     `run_max.is_finite()` guard and the `correction != 1` skip, the two-pass decode
//     kernels for f32 and f16 K/V);
//   * extension (NOT in the reference) - the same online-softmax tiling generalised to what
//     the GPU path also serves: batch, grouped K/V heads, head_dim 128, query length !=
//     key length, a causal mask with a query offset, ragged per-batch key counts, K given
//     either transposed (d-major) or as rows, and an explicit score scale.
//
// Parity status of each function is recorded where it is checked (tests/test_oracle.py).

#include <immintrin.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <limits>
#include <atomic>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include <sched.h>

namespace {

constexpr int kBQ = 64;   // query rows per tile        (flash_attn.rs:48)
constexpr int kBK = 256;  // keys per tile              (flash_attn.rs:49)
constexpr int kHD = 64;   // head_dim of the reference  (flash_attn.rs:50)

constexpr float kNegInf = -std::numeric_limits<float>::infinity();

// Planted mistakes, for the tests that prove the oracle's checks can fail (never set otherwise):
// 1 = skip the accumulator rescale, 2 = drop the degree-5 term of the exp polynomial,
// 3 = lose the last key of every tile, 4 = use K^T's row instead of its column (transposed index).
int g_fault = 0;

// ---------------------------------------------------------------------------------------------
// Vector primitives: flash_attn.rs:545-593.
// exp(x) = 2^(x*log2 e): the rounded integer part goes straight into the exponent field, the
// fractional part in [-0.5, 0.5] through the reference's degree-5 polynomial, input clamped at -87.
// ---------------------------------------------------------------------------------------------
__attribute__((target("avx2,fma"))) inline __m256 vexp(__m256 x) {
  const __m256 xc = _mm256_max_ps(x, _mm256_set1_ps(-87.0f));
  const __m256 t = _mm256_mul_ps(xc, _mm256_set1_ps(1.44269504088896340736f));
  const __m256 n = _mm256_round_ps(t, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  const __m256 f = _mm256_sub_ps(t, n);
  // Horner over the polynomial coefficients of flash_attn.rs:559-564, highest degree first.
  static const float kC[6] = {0.0013333558f, 0.009618129f, 0.05550411f,
                              0.2402265f,    0.6931472f,   1.0f};
  __m256 poly = _mm256_set1_ps(g_fault == 2 ? 0.0f : kC[0]);
  for (int i = 1; i < 6; ++i) poly = _mm256_fmadd_ps(poly, f, _mm256_set1_ps(kC[i]));
  const __m256i bits =
      _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(n), _mm256_set1_epi32(127)), 23);
  return _mm256_mul_ps(poly, _mm256_castsi256_ps(bits));
}

__attribute__((target("avx2,fma"))) inline float vmax_all(__m256 v) {
  __m128 m = _mm_max_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  m = _mm_max_ps(m, _mm_movehl_ps(m, m));
  m = _mm_max_ss(m, _mm_shuffle_ps(m, m, 1));
  return _mm_cvtss_f32(m);
}

__attribute__((target("avx2,fma"))) inline float vsum_all(__m256 v) {
  __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
  return _mm_cvtss_f32(s);
}

inline float f16_bits_to_f32(uint16_t h) {
  // IEEE binary16 -> binary32, exact (what F16C's vcvtph2ps computes).
  return _cvtsh_ss(h);
}

// ---------------------------------------------------------------------------------------------
// Scores tile: flash_attn.rs:791-873. S[i, j] = sum_t Q[i, t] * K^T[t, k0 + j] for rows < `rows`
// and cols < `cols`, written with row stride kBK. 4 query rows x 16 key columns stay in registers
// across the contraction; scalar loops cover row and column tails.
// `kt_at(t, j)` is element (t, j) of the transposed key block; `kt_row` is the stride between
// consecutive t (the reference uses seq) and keys are contiguous within a row.
// ---------------------------------------------------------------------------------------------
template <int D>
__attribute__((target("avx2,fma"))) void scores_block(const float* q, int q_row, const float* kt,
                                                      long kt_row, int k0, int rows, int cols,
                                                      float* s) {
  int i0 = 0;
  for (; i0 + 4 <= rows; i0 += 4) {
    int j0 = 0;
    for (; j0 + 16 <= cols; j0 += 16) {
      __m256 acc[4][2];
      for (int m = 0; m < 4; ++m) acc[m][0] = acc[m][1] = _mm256_setzero_ps();
      for (int t = 0; t < D; ++t) {
        const float* kp = kt + t * kt_row + k0 + j0;
        const __m256 k_lo = _mm256_loadu_ps(kp);
        const __m256 k_hi = _mm256_loadu_ps(kp + 8);
        for (int m = 0; m < 4; ++m) {
          const __m256 qb = _mm256_set1_ps(q[(i0 + m) * q_row + t]);
          acc[m][0] = _mm256_fmadd_ps(qb, k_lo, acc[m][0]);
          acc[m][1] = _mm256_fmadd_ps(qb, k_hi, acc[m][1]);
        }
      }
      for (int m = 0; m < 4; ++m) {
        _mm256_storeu_ps(s + (i0 + m) * kBK + j0, acc[m][0]);
        _mm256_storeu_ps(s + (i0 + m) * kBK + j0 + 8, acc[m][1]);
      }
    }
    for (int j = j0; j < cols; ++j) {
      for (int m = 0; m < 4; ++m) {
        float a = 0.0f;
        for (int t = 0; t < D; ++t) a += q[(i0 + m) * q_row + t] * kt[t * kt_row + k0 + j];
        s[(i0 + m) * kBK + j] = a;
      }
    }
  }
  for (int i = i0; i < rows; ++i) {
    for (int j = 0; j < cols; ++j) {
      float a = 0.0f;
      for (int t = 0; t < D; ++t) a += q[i * q_row + t] * kt[t * kt_row + k0 + j];
      s[i * kBK + j] = a;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// P.V accumulation: flash_attn.rs:875-948. acc[i, d] += sum_j P[i, j] * V[k0 + j, d], 4 rows x 16
// head dims in registers; V rows have stride `v_row`.
// ---------------------------------------------------------------------------------------------
template <int D>
__attribute__((target("avx2,fma"))) void pv_block(const float* p, const float* v, long v_row,
                                                  float* acc, int rows, int k0, int cols) {
  int i0 = 0;
  for (; i0 + 4 <= rows; i0 += 4) {
    for (int d0 = 0; d0 < D; d0 += 16) {
      __m256 a[4][2];
      for (int m = 0; m < 4; ++m) {
        a[m][0] = _mm256_loadu_ps(acc + (i0 + m) * D + d0);
        a[m][1] = _mm256_loadu_ps(acc + (i0 + m) * D + d0 + 8);
      }
      for (int j = 0; j < cols; ++j) {
        const float* vp = v + (long)(k0 + j) * v_row + d0;
        const __m256 v_lo = _mm256_loadu_ps(vp);
        const __m256 v_hi = _mm256_loadu_ps(vp + 8);
        for (int m = 0; m < 4; ++m) {
          const __m256 pb = _mm256_set1_ps(p[(i0 + m) * kBK + j]);
          a[m][0] = _mm256_fmadd_ps(pb, v_lo, a[m][0]);
          a[m][1] = _mm256_fmadd_ps(pb, v_hi, a[m][1]);
        }
      }
      for (int m = 0; m < 4; ++m) {
        _mm256_storeu_ps(acc + (i0 + m) * D + d0, a[m][0]);
        _mm256_storeu_ps(acc + (i0 + m) * D + d0 + 8, a[m][1]);
      }
    }
  }
  for (int i = i0; i < rows; ++i) {
    for (int j = 0; j < cols; ++j) {
      const float pj = p[i * kBK + j];
      for (int d = 0; d < D; ++d) acc[i * D + d] += pj * v[(long)(k0 + j) * v_row + d];
    }
  }
}

struct RowStep {
  float new_max, correction, block_sum;
};

// ---------------------------------------------------------------------------------------------
// Online softmax over one score row: flash_attn.rs:950-998. Returns the new running max, the
// rescale factor for what was accumulated so far (0 when nothing was: the running max was not
// finite) and the sum of this block's weights; the weights overwrite the scores in place.
// ---------------------------------------------------------------------------------------------
__attribute__((target("avx2,fma"))) RowStep softmax_step(float* row, int cols, float run_max) {
  __m256 vm = _mm256_set1_ps(kNegInf);
  int j = 0;
  for (; j + 8 <= cols; j += 8) vm = _mm256_max_ps(vm, _mm256_loadu_ps(row + j));
  float block_max = cols >= 8 ? vmax_all(vm) : kNegInf;
  for (int r = j; r < cols; ++r) block_max = std::max(block_max, row[r]);

  const float new_max = std::max(run_max, block_max);
  const float correction = std::isfinite(run_max) ? std::exp(run_max - new_max) : 0.0f;

  const __m256 vnm = _mm256_set1_ps(new_max);
  __m256 vs = _mm256_setzero_ps();
  j = 0;
  for (; j + 8 <= cols; j += 8) {
    const __m256 w = vexp(_mm256_sub_ps(_mm256_loadu_ps(row + j), vnm));
    _mm256_storeu_ps(row + j, w);
    vs = _mm256_add_ps(vs, w);
  }
  float block_sum = cols >= 8 ? vsum_all(vs) : 0.0f;
  for (int r = j; r < cols; ++r) {
    row[r] = std::exp(row[r] - new_max);
    block_sum += row[r];
  }
  return {new_max, correction, block_sum};
}

// ---------------------------------------------------------------------------------------------
// One encoder head: flash_attn.rs:415-487 (`flash_head_strided`). q (seq, 64), kt (64, seq),
// v (seq, 64); output rows `out_stride` apart (64 for (H, T, 64), H*64 for the merged layout).
// ---------------------------------------------------------------------------------------------
__attribute__((target("avx2,fma"))) void encoder_head(const float* q, const float* kt,
                                                      const float* v, float* out, int seq,
                                                      long out_stride) {
  std::vector<float> scores(kBQ * kBK), acc(kBQ * kHD), run_max(kBQ), run_sum(kBQ);
  for (int q0 = 0; q0 < seq; q0 += kBQ) {
    const int rows = std::min(kBQ, seq - q0);
    std::fill(acc.begin(), acc.begin() + rows * kHD, 0.0f);
    std::fill(run_max.begin(), run_max.begin() + rows, kNegInf);
    std::fill(run_sum.begin(), run_sum.begin() + rows, 0.0f);
    const float* qb = q + (long)q0 * kHD;
    for (int k0 = 0; k0 < seq; k0 += kBK) {
      const int cols = std::min(kBK, seq - k0) - (g_fault == 3 ? 1 : 0);
      scores_block<kHD>(qb, kHD, kt, seq, k0, rows, cols, scores.data());
      if (g_fault == 4)  // read K^T[j, t] instead of K^T[t, j] (square tiles only)
        for (int i = 0; i < rows; ++i)
          for (int j = 0; j < cols; ++j) {
            float a = 0.0f;
            for (int t = 0; t < kHD; ++t) a += qb[i * kHD + t] * kt[(long)(k0 + j) * seq + t];
            scores[i * kBK + j] = a;
          }
      for (int i = 0; i < rows; ++i) {
        const RowStep st = softmax_step(&scores[i * kBK], cols, run_max[i]);
        run_sum[i] = std::fma(run_sum[i], st.correction, st.block_sum);
        run_max[i] = st.new_max;
        if (st.correction != 1.0f && g_fault != 1)
          for (int d = 0; d < kHD; ++d) acc[i * kHD + d] *= st.correction;
      }
      pv_block<kHD>(scores.data(), v, kHD, acc.data(), rows, k0, cols);
    }
    for (int i = 0; i < rows; ++i) {
      const float inv = 1.0f / run_sum[i];
      float* o = out + (long)(q0 + i) * out_stride;
      for (int d = 0; d < kHD; ++d) o[d] = acc[i * kHD + d] * inv;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Decode heads: flash_attn.rs:595-696 (`xattn_head`, f32 K/V) and :698-789 (`xattn_head_f16`).
// Two passes over the keys with a K-sized scratch row: scores by a contraction-outermost AXPY,
// a full-row softmax, then the weighted sum of V rows in eight 8-wide accumulators.
// `Load` widens one 8-wide group of K/V elements to f32.
// ---------------------------------------------------------------------------------------------
struct LoadF32 {
  using T = float;
  __attribute__((target("avx2,fma"))) static __m256 load8(const float* p) {
    return _mm256_loadu_ps(p);
  }
  static float load1(const float* p) { return *p; }
};
struct LoadF16 {
  using T = uint16_t;
  __attribute__((target("avx2,fma,f16c"))) static __m256 load8(const uint16_t* p) {
    return _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(p)));
  }
  static float load1(const uint16_t* p) { return f16_bits_to_f32(*p); }
};

template <class L>
__attribute__((target("avx2,fma,f16c"))) void decode_head(const float* q,
                                                          const typename L::T* kt,
                                                          const typename L::T* v, float* out,
                                                          int keys, float* s) {
  std::fill(s, s + keys, 0.0f);
  for (int t = 0; t < kHD; ++t) {
    const __m256 qv = _mm256_set1_ps(q[t]);
    const typename L::T* kr = kt + (long)t * keys;
    int j = 0;
    for (; j + 8 <= keys; j += 8)
      _mm256_storeu_ps(s + j, _mm256_fmadd_ps(qv, L::load8(kr + j), _mm256_loadu_ps(s + j)));
    for (; j < keys; ++j) s[j] += q[t] * L::load1(kr + j);
  }

  __m256 vm = _mm256_set1_ps(kNegInf);
  int j = 0;
  for (; j + 8 <= keys; j += 8) vm = _mm256_max_ps(vm, _mm256_loadu_ps(s + j));
  float mx = keys >= 8 ? vmax_all(vm) : kNegInf;
  for (int r = j; r < keys; ++r) mx = std::max(mx, s[r]);

  const __m256 vmx = _mm256_set1_ps(mx);
  __m256 vs = _mm256_setzero_ps();
  j = 0;
  for (; j + 8 <= keys; j += 8) {
    const __m256 w = vexp(_mm256_sub_ps(_mm256_loadu_ps(s + j), vmx));
    _mm256_storeu_ps(s + j, w);
    vs = _mm256_add_ps(vs, w);
  }
  float sum = keys >= 8 ? vsum_all(vs) : 0.0f;
  for (int r = j; r < keys; ++r) {
    s[r] = std::exp(s[r] - mx);
    sum += s[r];
  }
  const float inv = 1.0f / sum;

  __m256 a[8];
  for (int c = 0; c < 8; ++c) a[c] = _mm256_setzero_ps();
  for (int r = 0; r < keys; ++r) {
    const __m256 w = _mm256_set1_ps(s[r] * inv);
    const typename L::T* vp = v + (long)r * kHD;
    for (int c = 0; c < 8; ++c) a[c] = _mm256_fmadd_ps(w, L::load8(vp + 8 * c), a[c]);
  }
  for (int c = 0; c < 8; ++c) _mm256_storeu_ps(out + 8 * c, a[c]);
}

// A persistent pool of worker threads, as rayon's global pool (the reference's `par_iter`s,
// flash_attn.rs:199,402): created on first use with as many workers as the process may run on,
// then reused by every call, so a call pays a wake-up and no thread creation. parallel_for(n,
// threads, f) runs f(0..n-1) on up to `threads` threads (the caller is one of them); jobs are
// handed out in index order through an atomic counter. Calls are serialised (one at a time).
class Pool {
 public:
  static Pool& get() {
    static Pool* p = new Pool();  // never destroyed: the workers live as long as the process
    return *p;
  }
  template <class F>
  void run(int n, int threads, F&& f) {
    std::lock_guard<std::mutex> call(call_mu_);
    threads = std::max(1, std::min({threads, n, (int)workers_.size() + 1}));
    if (threads == 1) {
      for (int i = 0; i < n; ++i) f(i);
      return;
    }
    std::function<void(int)> job = [&f](int i) { f(i); };
    {
      std::lock_guard<std::mutex> lk(mu_);
      job_ = &job;
      n_ = n;
      next_.store(0);
      helpers_ = threads - 1;
      running_ = threads - 1;
      ++generation_;
    }
    cv_.notify_all();
    drain();
    std::unique_lock<std::mutex> lk(mu_);
    done_cv_.wait(lk, [&] { return running_ == 0; });
    job_ = nullptr;
  }

 private:
  Pool() {
    int nw = 1;
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof(set), &set) == 0) nw = std::max(1, CPU_COUNT(&set));
    for (int w = 0; w < nw - 1; ++w) workers_.emplace_back([this, w] { loop(w); });
    for (auto& t : workers_) t.detach();
  }
  void drain() {
    for (int i = next_.fetch_add(1); i < n_; i = next_.fetch_add(1)) (*job_)(i);
  }
  void loop(int w) {
    long seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return generation_ != seen; });
        seen = generation_;
        if (w >= helpers_) continue;  // this call wants fewer threads
      }
      drain();
      std::lock_guard<std::mutex> lk(mu_);
      if (--running_ == 0) done_cv_.notify_one();
    }
  }
  std::vector<std::thread> workers_;
  std::mutex call_mu_, mu_;
  std::condition_variable cv_, done_cv_;
  std::function<void(int)>* job_ = nullptr;
  std::atomic<int> next_{0};
  int n_ = 0, helpers_ = 0, running_ = 0;
  long generation_ = 0;
};

template <class F>
void parallel_for(int n, int threads, F&& f) {
  Pool::get().run(n, threads, f);
}

// ---------------------------------------------------------------------------------------------
// Extension (not in the reference): the encoder tiling generalised. One (batch, q-head) pair.
// Scores are multiplied by `scale` before the softmax (scale 1 reproduces the reference's
// pre-scaled convention). Masked keys (causal, or beyond this batch item's key count) get weight
// exactly 0. The first key is always visible to every query when q_offset >= 0, so each row has
// a finite running max after its first block.
// ---------------------------------------------------------------------------------------------
template <int D>
__attribute__((target("avx2,fma"))) void general_head(const float* q, long q_row,
                                                      const float* kt_packed, long kt_row,
                                                      const float* v, long v_row, float* out,
                                                      long out_row, int qlen, int keys,
                                                      float scale, int causal, int q_offset) {
  std::vector<float> scores(kBQ * kBK), acc(kBQ * D), run_max(kBQ), run_sum(kBQ);
  std::vector<float> qs(kBQ * D);
  for (int q0 = 0; q0 < qlen; q0 += kBQ) {
    const int rows = std::min(kBQ, qlen - q0);
    std::fill(acc.begin(), acc.begin() + rows * D, 0.0f);
    std::fill(run_max.begin(), run_max.begin() + rows, kNegInf);
    std::fill(run_sum.begin(), run_sum.begin() + rows, 0.0f);
    for (int i = 0; i < rows; ++i)
      for (int t = 0; t < D; ++t) qs[i * D + t] = q[(long)(q0 + i) * q_row + t];
    int kend = keys;
    if (causal) kend = std::min(keys, std::max(0, q_offset + q0 + rows));
    for (int k0 = 0; k0 < kend; k0 += kBK) {
      const int cols = std::min(kBK, kend - k0);
      scores_block<D>(qs.data(), D, kt_packed, kt_row, k0, rows, cols, scores.data());
      for (int i = 0; i < rows; ++i) {
        float* row = &scores[i * kBK];
        const int lim = causal ? q_offset + q0 + i : std::numeric_limits<int>::max();
        for (int j = 0; j < cols; ++j) row[j] = (k0 + j > lim) ? kNegInf : row[j] * scale;
        RowStep st = softmax_step(row, cols, run_max[i]);
        if (!std::isfinite(st.new_max)) {  // every key so far masked: nothing accumulated
          for (int j = 0; j < cols; ++j) row[j] = 0.0f;
          st.block_sum = 0.0f;
          st.correction = 0.0f;
        } else {
          for (int j = 0; j < cols; ++j)
            if (k0 + j > lim) row[j] = 0.0f;  // masked weight is exactly zero
          if (causal) {
            float bs = 0.0f;
            for (int j = 0; j < cols; ++j) bs += row[j];
            st.block_sum = bs;
          }
        }
        run_sum[i] = std::fma(run_sum[i], st.correction, st.block_sum);
        run_max[i] = st.new_max;
        if (st.correction != 1.0f)
          for (int d = 0; d < D; ++d) acc[i * D + d] *= st.correction;
      }
      pv_block<D>(scores.data(), v, v_row, acc.data(), rows, k0, cols);
    }
    for (int i = 0; i < rows; ++i) {
      const float inv = run_sum[i] > 0.0f ? 1.0f / run_sum[i] : 0.0f;
      float* o = out + (long)(q0 + i) * out_row;
      for (int d = 0; d < D; ++d) o[d] = acc[i * D + d] * inv;
    }
  }
}

}  // namespace

extern "C" {

// Version tag so a stale build is detectable from Python.
int oracle_version() { return 5; }

// Test hook: plant one of the mistakes listed at g_fault (0 restores the faithful oracle).
void oracle_plant_fault(int kind) { g_fault = kind; }

// exp polynomial of flash_attn.rs:553-571 on n floats (tails padded internally).
__attribute__((target("avx2,fma"))) void oracle_exp_poly(const float* x, float* y, long n) {
  long i = 0;
  for (; i + 8 <= n; i += 8) _mm256_storeu_ps(y + i, vexp(_mm256_loadu_ps(x + i)));
  if (i < n) {
    float buf[8] = {0}, res[8];
    for (long r = i; r < n; ++r) buf[r - i] = x[r];
    _mm256_storeu_ps(res, vexp(_mm256_loadu_ps(buf)));
    for (long r = i; r < n; ++r) y[r] = res[r - i];
  }
}

// MergedAttnOp::cpu_fwd (flash_attn.rs:160-210): q (1,H,T,64), kt (1,H,64,T), v (1,H,T,64)
// -> out (1,T,H*64). Heads in parallel over `threads` threads.
int oracle_attend_merged(int heads, int seq, const float* q, const float* kt, const float* v,
                         float* out, int threads) {
  if (heads <= 0 || seq <= 0) return -1;
  const long per = (long)seq * kHD;
  parallel_for(heads, threads, [&](int h) {
    encoder_head(q + h * per, kt + h * per, v + h * per, out + (long)h * kHD, seq,
                 (long)heads * kHD);
  });
  return 0;
}

// FlashAttnOp::cpu_fwd f32 arms (flash_attn.rs:357-413): qlen == keys -> encoder kernel per head
// (parallel), qlen == 1 -> xattn_head per head, serial unless `par_heads`.
// out (1,H,qlen,64).
int oracle_attend_f32(int heads, int qlen, int keys, const float* q, const float* kt,
                      const float* v, float* out, int par_heads, int threads) {
  if (heads <= 0 || keys <= 0) return -1;
  if (qlen == 1) {
    const int nt = par_heads ? threads : 1;
    std::vector<float> scratch((size_t)heads * keys);
    parallel_for(heads, nt, [&](int h) {
      decode_head<LoadF32>(q + h * kHD, kt + (long)h * kHD * keys, v + (long)h * keys * kHD,
                           out + h * kHD, keys, scratch.data() + (long)h * keys);
    });
    return 0;
  }
  if (qlen != keys) return 1;  // declined (flash_attn.rs:254-258)
  const long per = (long)keys * kHD;
  parallel_for(heads, threads, [&](int h) {
    encoder_head(q + h * per, kt + h * per, v + h * per, out + h * per, keys, kHD);
  });
  return 0;
}

// FlashAttnOp::cpu_fwd f16-K/V decode arm (flash_attn.rs:289-356): q (1,H,1,64) f32, kt
// (1,H,64,K) and v (1,H,K,64) as IEEE binary16 bit patterns -> out (1,H,1,64) f32.
int oracle_attend_f16kv(int heads, int keys, const float* q, const uint16_t* kt,
                        const uint16_t* v, float* out, int par_heads, int threads) {
  if (heads <= 0 || keys <= 0) return -1;
  const int nt = par_heads ? threads : 1;
  std::vector<float> scratch((size_t)heads * keys);
  parallel_for(heads, nt, [&](int h) {
    decode_head<LoadF16>(q + h * kHD, kt + (long)h * kHD * keys, v + (long)h * keys * kHD,
                         out + h * kHD, keys, scratch.data() + (long)h * keys);
  });
  return 0;
}

// Extension (not reference). q (B,Hq,Tq,D), k either transposed (B,Hkv,D,Tk) when
// k_transposed != 0 or rows (B,Hkv,Tk,D), v (B,Hkv,Tk,D), all f32 and packed; out (B,Hq,Tq,D).
// kv_lens (optional, host) limits the keys of each batch item. Pairs (b, h) run in parallel.
int oracle_attend_general(int batch, int heads_q, int heads_kv, int qlen, int keys, int head_dim,
                          const float* q, const float* k, int k_transposed, const float* v,
                          float* out, float scale, int causal, int q_offset,
                          const int* kv_lens, int threads) {
  if (batch <= 0 || heads_q <= 0 || heads_kv <= 0 || heads_q % heads_kv) return -1;
  if (head_dim != 64 && head_dim != 128) return -1;
  const int group = heads_q / heads_kv;
  const long D = head_dim;
  parallel_for(batch * heads_q, threads, [&](int bh) {
    const int b = bh / heads_q, h = bh % heads_q, hk = h / group;
    const int kb = kv_lens ? std::min(keys, std::max(0, kv_lens[b])) : keys;
    const float* qp = q + ((long)b * heads_q + h) * qlen * D;
    const float* kp = k + ((long)b * heads_kv + hk) * keys * D;
    const float* vp = v + ((long)b * heads_kv + hk) * keys * D;
    float* op = out + ((long)b * heads_q + h) * qlen * D;
    // The tiles want K^T (d-major, keys contiguous); pack rows-layout K once per head.
    std::vector<float> kt_buf;
    const float* ktp = kp;
    long kt_row = keys;
    if (!k_transposed) {
      kt_buf.resize((size_t)D * std::max(kb, 1));
      for (int j = 0; j < kb; ++j)
        for (int t = 0; t < D; ++t) kt_buf[(size_t)t * kb + j] = kp[(long)j * D + t];
      ktp = kt_buf.data();
      kt_row = std::max(kb, 1);
    }
    if (kb == 0) {
      for (long i = 0; i < (long)qlen * D; ++i) op[i] = 0.0f;
      return;
    }
    if (head_dim == 64)
      general_head<64>(qp, D, ktp, kt_row, vp, D, op, D, qlen, kb, scale, causal, q_offset);
    else
      general_head<128>(qp, D, ktp, kt_row, vp, D, op, D, qlen, kb, scale, causal, q_offset);
  });
  return 0;
}

}  // extern "C"
