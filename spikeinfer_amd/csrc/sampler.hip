// Batched token sampler: one workgroup per row of logits, no host round trip.
//
// Reference semantics: spikeinfer/engine/sampler.py:48-177 -- penalties
// (repetition, then presence + frequency; :98-119), temperature (:69-75),
// min_p (:137-141), top_k (:143-153), top_p (:155-159), then a draw from the
// softmax of what survived (:162-168); greedy rows (temperature < 1e-5,
// sampling_params.py:74) take the argmax of the penalised logits (:64-67).
//
// MI355X design.  No sort of the 151,936-entry row.  Every filter keeps a
// prefix of the row in one total order -- value descending, index ascending
// (the reference leaves the order of equal logits to torch.topk; this kernel
// fixes it) -- so the result is one cut (key K, first t elements of key K):
//   * min_p keeps exp(x - max) >= min_p (a value threshold);
//   * top_k: a 3-pass radix select (11/11/10 bits of the order-preserving
//     key) on element counts finds the k-th element;
//   * top_p: the same radix select on probability mass finds the last element
//     whose preceding mass is below top_p of the surviving mass.  Mass is
//     fixed point (weight * 2^40 in uint64), so sums are exact and the cut is
//     deterministic whatever the atomic order;
//   * ties at the cut are ranked in index order with one block scan.
// The draw is an inverse CDF in index order over the kept weights with a
// caller-supplied uniform u in [0, 1): the first token whose inclusive
// cumulative weight exceeds u * total.
// Histograms, the seen-token bitmap and the count hash live in LDS; the row
// itself is re-read from L2 on each pass.
#include "common.hpp"
#include "lif_math.hpp"

namespace spk {
namespace smp {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kBins = 2048;            // 11-bit digits
constexpr int kMaxVocab = 262144;      // bitmap capacity (32 KB)
constexpr int kMaxHist = 2048;         // history tokens per row
constexpr int kHashSlots = 2 * kMaxHist;
constexpr float kGreedyTemp = 1e-5f;
constexpr double kMassScale = 1099511627776.0;  // 2^40

constexpr int kCand = 8192;  // LDS candidate capacity (the fast path)

struct Params {
  float temp, min_p, top_p, rep, presence, frequency;
  int top_k;
  bool use_hash;
};

struct Shared {
  uint32_t seen[kMaxVocab / 32];      // generated-token bitmap
  int32_t hkey[kHashSlots];           // token + 1 -> count (frequency penalty)
  int32_t hcnt[kHashSlots];
  unsigned long long hist[kBins];     // radix histograms (counts or fixed-point mass)
  float cx[kCand];                    // candidates, in index order: value x ...
  int32_t ci[kCand];                  // ... and vocabulary index
  unsigned long long wsum[kWaves];
  unsigned long long bcast[4];
  float fbcast[kWaves];
};

// Order-preserving unsigned key of a float (larger float -> larger key).
__device__ __forceinline__ uint32_t fkey(float x) {
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float unkey(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ int hash_slot(int tok) {
  return static_cast<int>((static_cast<uint32_t>(tok) * 2654435761u) % kHashSlots);
}

// Penalised logit (sampler.py:98-119): repetition first, then presence and
// frequency, for tokens generated so far.
__device__ __forceinline__ float penalise(const Params &P, const Shared &sh, int i, float v) {
  if (!((sh.seen[i >> 5] >> (i & 31)) & 1u)) return v;
  if (P.rep != 1.f) v = v > 0.f ? v / P.rep : v * P.rep;
  if (P.presence != 0.f || P.frequency != 0.f) {
    float cnt = 1.f;
    if (P.use_hash) {
      int s = hash_slot(i);
      while (sh.hkey[s] != i + 1) s = (s + 1) % kHashSlots;
      cnt = static_cast<float>(sh.hcnt[s]);
    }
    v = v - (P.presence + P.frequency * cnt);
  }
  return v;
}

__device__ __forceinline__ unsigned long long shfl_up_u64(unsigned long long v, int d) {
  const uint32_t lo = __shfl_up(static_cast<uint32_t>(v), d);
  const uint32_t hi = __shfl_up(static_cast<uint32_t>(v >> 32), d);
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

// Exclusive prefix sum over the workgroup in thread order; *total gets the sum.
__device__ __forceinline__ unsigned long long block_exclusive_scan(unsigned long long v, Shared &sh,
                                                   unsigned long long *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned long long inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const unsigned long long o = shfl_up_u64(inc, d);
    if (lane >= d) inc += o;
  }
  __syncthreads();
  if (lane == 63) sh.wsum[wave] = inc;
  __syncthreads();
  unsigned long long before = 0, all = 0;
  for (int w = 0; w < kWaves; ++w) {
    const unsigned long long s = sh.wsum[w];
    if (w < wave) before += s;
    all += s;
  }
  *total = all;
  return before + inc - v;
}

__device__ __forceinline__ float block_max(float v, Shared &sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) v = fmaxf(v, __shfl_xor(v, d));
  __syncthreads();
  if (lane == 0) sh.fbcast[wave] = v;
  __syncthreads();
  float m = sh.fbcast[0];
  for (int w = 1; w < kWaves; ++w) m = fmaxf(m, sh.fbcast[w]);
  return m;
}

__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long v, Shared &sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), d);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), d);
    const unsigned long long o = (static_cast<unsigned long long>(hi) << 32) | lo;
    v = o > v ? o : v;
  }
  __syncthreads();
  if (lane == 0) sh.wsum[wave] = v;
  __syncthreads();
  unsigned long long m = sh.wsum[0];
  for (int w = 1; w < kWaves; ++w) m = sh.wsum[w] > m ? sh.wsum[w] : m;
  return m;
}

// Given the 2048-bin histogram in sh.hist, finds the bin b (scanning from the
// top) with above < target <= above + hist[b], where above = base + the bins
// over b.  Writes b and its `above` to sh.bcast[0..1]; bcast[2] = 1 if found.
constexpr int kBinsPerThread = kBins / kThreads;
__device__ __forceinline__ void select_bin(Shared &sh, unsigned long long base, double target) {
  const int top = kBins - 1 - kBinsPerThread * static_cast<int>(threadIdx.x);  // this thread's highest bin
  unsigned long long h[kBinsPerThread], sum = 0;
#pragma unroll
  for (int r = 0; r < kBinsPerThread; ++r) sum += (h[r] = sh.hist[top - r]);
  unsigned long long total;
  unsigned long long before = base + block_exclusive_scan(sum, sh, &total);
  if (threadIdx.x == 0) sh.bcast[2] = 0;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kBinsPerThread; ++r) {
    if ((double)before < target && target <= (double)(before + h[r])) {
      sh.bcast[0] = top - r;
      sh.bcast[1] = before;
      sh.bcast[2] = 1;
    }
    before += h[r];
  }
  __syncthreads();
}

__device__ __forceinline__ unsigned long long mass_of(float x, float m) {
  return static_cast<unsigned long long>(static_cast<double>(expf(x - m)) * kMassScale);
}

__device__ __forceinline__ void zero_hist(Shared &sh) {
  __syncthreads();
  for (int b = threadIdx.x; b < kBins; b += kThreads) sh.hist[b] = 0;
  __syncthreads();
}

// ---- element sources ----------------------------------------------------------------
// each(f): every element once, f(index, x), any order; chunk(f): this thread's
// contiguous range, in index order (ranges ascend with the thread id).

// The logits row in global memory; x = penalise(raw) / temperature.
template <int DT, bool VEC>
struct GlobalSrc {
  typedef typename Elem<DT>::T E;
  static constexpr int W = VEC ? Elem<DT>::kVec : 1;  // 16 bytes per load
  typedef E Vec __attribute__((ext_vector_type(W)));
  const E *p;
  int V;
  Params P;
  const Shared *sh;

  __device__ __forceinline__ float x(int i, E raw) const {
    return penalise(P, *sh, i, elem_to_f32<DT>(raw)) / P.temp;
  }
  template <class F> __device__ __forceinline__ void each_raw(F f) const {
    const int nv = V / W;
    const Vec *pv = reinterpret_cast<const Vec *>(p);
    int v = threadIdx.x;
    for (; v + 3 * kThreads < nv; v += 4 * kThreads) {
      const Vec a0 = pv[v], a1 = pv[v + kThreads], a2 = pv[v + 2 * kThreads],
                a3 = pv[v + 3 * kThreads];
#pragma unroll
      for (int j = 0; j < W; ++j) f(v * W + j, a0[j]);
#pragma unroll
      for (int j = 0; j < W; ++j) f((v + kThreads) * W + j, a1[j]);
#pragma unroll
      for (int j = 0; j < W; ++j) f((v + 2 * kThreads) * W + j, a2[j]);
#pragma unroll
      for (int j = 0; j < W; ++j) f((v + 3 * kThreads) * W + j, a3[j]);
    }
    for (; v < nv; v += kThreads) {
      const Vec a = pv[v];
#pragma unroll
      for (int j = 0; j < W; ++j) f(v * W + j, a[j]);
    }
    for (int i = nv * W + threadIdx.x; i < V; i += kThreads) f(i, p[i]);
  }
  template <class F> __device__ __forceinline__ void each(F f) const {
    each_raw([&](int i, E raw) { f(i, x(i, raw)); });
  }
  template <class F> __device__ __forceinline__ void chunk(F f) const {
    const int per = ((V + kThreads - 1) / kThreads + W - 1) / W * W;
    const int lo = min(V, static_cast<int>(threadIdx.x) * per), hi = min(V, lo + per);
    int i = lo;
    // Four 16-byte loads in flight per iteration.
    for (; i + 4 * W <= hi; i += 4 * W) {
      const Vec *q = reinterpret_cast<const Vec *>(p + i);
      const Vec a0 = q[0], a1 = q[1], a2 = q[2], a3 = q[3];
#pragma unroll
      for (int j = 0; j < W; ++j) f(i + j, x(i + j, a0[j]));
#pragma unroll
      for (int j = 0; j < W; ++j) f(i + W + j, x(i + W + j, a1[j]));
#pragma unroll
      for (int j = 0; j < W; ++j) f(i + 2 * W + j, x(i + 2 * W + j, a2[j]));
#pragma unroll
      for (int j = 0; j < W; ++j) f(i + 3 * W + j, x(i + 3 * W + j, a3[j]));
    }
    for (; i + W <= hi; i += W) {
      const Vec a = *reinterpret_cast<const Vec *>(p + i);
#pragma unroll
      for (int j = 0; j < W; ++j) f(i + j, x(i + j, a[j]));
    }
    for (; i < hi; ++i) f(i, x(i, p[i]));
  }
};

// The candidates gathered into LDS (index order).
struct CandSrc {
  const Shared *sh;
  int n;
  template <class F> __device__ __forceinline__ void each(F f) const {
    for (int j = threadIdx.x; j < n; j += kThreads) f(sh->ci[j], sh->cx[j]);
  }
  template <class F> __device__ __forceinline__ void chunk(F f) const {
    const int per = (n + kThreads - 1) / kThreads;
    const int lo = min(n, static_cast<int>(threadIdx.x) * per), hi = min(n, lo + per);
    for (int j = lo; j < hi; ++j) f(sh->ci[j], sh->cx[j]);
  }
};

// min_p -> top_k -> top_p -> draw over a source; returns the token.  `Z_all`
// (when have_Z) is the alive mass of the whole row, needed when the source is
// a candidate subset and no top-k cut bounds the survivors inside it.
template <class Src>
__device__ __forceinline__ int64_t filter_and_draw(const Src src, Shared &sh, const Params P, float m,
                                   long long k_req, bool have_Z, unsigned long long Z_all,
                                   float u) {
  auto alive = [&](float x) { return P.min_p <= 0.f || expf(x - m) >= P.min_p; };

  // top-k: cut (Kk, tk) on element counts.
  uint32_t Kk = 0;                // elements with key > Kk are kept
  unsigned long long tk = ~0ull;  // ties at Kk kept, in index order (~0: all)
  if (k_req > 0) {
    unsigned long long c = 0;
    src.each([&](int, float x) { c += alive(x) ? 1 : 0; });
    unsigned long long alive_cnt;
    block_exclusive_scan(c, sh, &alive_cnt);
    if (static_cast<unsigned long long>(k_req) < alive_cnt) {
      uint32_t prefix = 0;
      unsigned long long above = 0;
      for (int pass = 0; pass < 3; ++pass) {
        const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
        const uint32_t dmask = pass == 2 ? 0x3ffu : 0x7ffu;
        const int hi_shift = shift + (pass == 2 ? 10 : 11);
        zero_hist(sh);
        src.each([&](int, float x) {
          if (!alive(x)) return;
          const uint32_t k = fkey(x);
          if (pass > 0 && (k >> hi_shift) != (prefix >> hi_shift)) return;
          atomicAdd(&sh.hist[(k >> shift) & dmask], 1ull);
        });
        __syncthreads();
        select_bin(sh, above, static_cast<double>(k_req));
        prefix |= static_cast<uint32_t>(sh.bcast[0]) << shift;
        above = sh.bcast[1];
      }
      Kk = prefix;
      tk = static_cast<unsigned long long>(k_req) - above;
    }
  }
  const bool k_partial = tk != ~0ull;
  auto in_s_nontie = [&](float x, uint32_t k) {
    return alive(x) && (k > Kk || (k == Kk && !k_partial));
  };
  const unsigned long long wK = k_partial ? mass_of(unkey(Kk), m) : 0;

  // top-p: cut (Kf, tf) on the survivors' probability mass.
  uint32_t Kf = Kk;
  unsigned long long tf = tk;
  if (P.top_p < 1.f) {
    unsigned long long Z;
    if (have_Z && !k_partial) {
      Z = Z_all;
    } else {
      unsigned long long z = 0;
      src.each([&](int, float x) {
        if (in_s_nontie(x, fkey(x))) z += mass_of(x, m);
      });
      block_exclusive_scan(z, sh, &Z);
      if (k_partial) Z += tk * wK;
    }
    const double target = static_cast<double>(P.top_p) * static_cast<double>(Z);
    uint32_t prefix = 0;
    unsigned long long above = 0;
    bool found = true;
    for (int pass = 0; pass < 3 && found; ++pass) {
      const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
      const uint32_t dmask = pass == 2 ? 0x3ffu : 0x7ffu;
      const int hi_shift = shift + (pass == 2 ? 10 : 11);
      zero_hist(sh);
      src.each([&](int, float x) {
        const uint32_t k = fkey(x);
        if (!in_s_nontie(x, k)) return;
        if (pass > 0 && (k >> hi_shift) != (prefix >> hi_shift)) return;
        atomicAdd(&sh.hist[(k >> shift) & dmask], mass_of(x, m));
      });
      __syncthreads();
      // The kept ties of the top-k cut all weigh wK: add them analytically.
      if (threadIdx.x == 0 && k_partial && (pass == 0 || (Kk >> hi_shift) == (prefix >> hi_shift)))
        sh.hist[(Kk >> shift) & dmask] += tk * wK;
      __syncthreads();
      select_bin(sh, above, target);
      found = sh.bcast[2] != 0;
      prefix |= static_cast<uint32_t>(sh.bcast[0]) << shift;
      above = sh.bcast[1];
    }
    if (found) {
      Kf = prefix;
      const unsigned long long w = mass_of(unkey(Kf), m);
      // Ties at Kf kept: the first j with above + (j - 1) * w < target.
      unsigned long long j =
          w ? static_cast<unsigned long long>(ceil((target - static_cast<double>(above)) / static_cast<double>(w)))
            : 1;
      if (j < 1) j = 1;
      if (Kf == Kk && k_partial && j > tk) j = tk;
      tf = j;
    }
  }

  // Draw: inverse CDF in index order over the kept weights.  Ties at Kf are
  // ranked by a scan of per-thread tie counts.
  const bool f_partial = tf != ~0ull;
  unsigned long long wsum = 0, ties = 0;
  src.chunk([&](int, float x) {
    const uint32_t k = fkey(x);
    if (!alive(x) || k < Kf) return;
    if (k == Kf && f_partial) {
      ++ties;
      return;
    }
    wsum += mass_of(x, m);
  });
  unsigned long long tot_ties;
  const unsigned long long rank0 = block_exclusive_scan(ties, sh, &tot_ties);
  unsigned long long kept_ties = 0;
  if (f_partial) kept_ties = rank0 >= tf ? 0 : (tf - rank0 < ties ? tf - rank0 : ties);
  const unsigned long long wf = f_partial ? mass_of(unkey(Kf), m) : 0;
  const unsigned long long mine = wsum + kept_ties * wf;
  unsigned long long Wtot;
  const unsigned long long before = block_exclusive_scan(mine, sh, &Wtot);
  unsigned long long target =
      static_cast<unsigned long long>(static_cast<double>(u) * static_cast<double>(Wtot));
  if (target >= Wtot) target = Wtot ? Wtot - 1 : 0;
  if (threadIdx.x == 0) sh.bcast[3] = 0;  // unreachable fallback: the top element always weighs 2^40
  __syncthreads();
  if (mine > 0 && before <= target && target < before + mine) {
    unsigned long long acc = before, seen_ties = 0;
    bool done = false;
    src.chunk([&](int i, float x) {
      if (done) return;
      const uint32_t k = fkey(x);
      if (!alive(x) || k < Kf) return;
      unsigned long long w;
      if (k == Kf && f_partial) {
        if (seen_ties++ >= kept_ties) return;
        w = wf;
      } else {
        w = mass_of(x, m);
      }
      acc += w;
      if (acc > target) {
        sh.bcast[3] = static_cast<unsigned long long>(i);
        done = true;
      }
    });
  }
  __syncthreads();
  return static_cast<int64_t>(sh.bcast[3]);
}

template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void sample_kernel(
    const void *logits, int64_t row_stride, int V, const float *temperature,
    const int32_t *top_k, const float *top_p, const float *min_p, const float *rep,
    const float *presence, const float *frequency, const int64_t *history, int64_t hist_stride,
    const int32_t *hist_len, int64_t hist_len_stride, const float *uniforms, int64_t *out) {
  typedef typename Elem<DT>::T E;
  extern __shared__ __align__(16) char smem_raw[];
  Shared &sh = *reinterpret_cast<Shared *>(smem_raw);
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  Params P;
  P.temp = temperature[row];
  P.top_k = top_k ? top_k[row] : -1;
  P.top_p = top_p ? top_p[row] : 1.f;
  P.min_p = min_p ? min_p[row] : 0.f;
  P.rep = rep ? rep[row] : 1.f;
  P.presence = presence ? presence[row] : 0.f;
  P.frequency = frequency ? frequency[row] : 0.f;
  P.use_hash = P.frequency != 0.f;

  // ---- history -> seen bitmap (+ counts) ------------------------------------
  const int nwords = (V + 31) >> 5;
  for (int w = tid; w < nwords; w += kThreads) sh.seen[w] = 0u;
  if (P.use_hash)
    for (int s = tid; s < kHashSlots; s += kThreads) sh.hkey[s] = 0, sh.hcnt[s] = 0;
  __syncthreads();
  if (history && hist_len) {
    int nh = hist_len[row * hist_len_stride];
    // At most one row of history (the row stride) and kMaxHist tokens.
    const int64_t cap = hist_stride < kMaxHist ? hist_stride : kMaxHist;
    nh = nh < 0 ? 0 : (nh > cap ? static_cast<int>(cap) : nh);
    for (int j = tid; j < nh; j += kThreads) {
      const int64_t tok = history[row * hist_stride + j];
      if (tok < 0 || tok >= V) continue;
      const int t32 = static_cast<int>(tok);
      atomicOr(&sh.seen[t32 >> 5], 1u << (t32 & 31));
      if (P.use_hash) {
        int s = hash_slot(t32);
        while (true) {
          const int prev = atomicCAS(&sh.hkey[s], 0, t32 + 1);
          if (prev == 0 || prev == t32 + 1) break;
          s = (s + 1) % kHashSlots;
        }
        atomicAdd(&sh.hcnt[s], 1);
      }
    }
  }
  __syncthreads();

  GlobalSrc<DT, VEC> g;
  g.p = reinterpret_cast<const E *>(logits) + row * row_stride;
  g.V = V;
  g.P = P;
  g.sh = &sh;

  // ---- greedy: argmax of the penalised logits, first index on ties ------------
  if (P.temp < kGreedyTemp) {
    unsigned long long best = 0;
    g.each_raw([&](int i, E raw) {
      const unsigned long long k =
          (static_cast<unsigned long long>(fkey(penalise(P, sh, i, elem_to_f32<DT>(raw)))) << 32) |
          (0xffffffffu - static_cast<uint32_t>(i));
      best = k > best ? k : best;
    });
    best = block_max_u64(best, sh);
    if (tid == 0) out[row] = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(best));
    return;
  }

  const long long k_req = (P.top_k < 0 || P.top_k >= V) ? -1 : P.top_k;
  const float u = uniforms ? uniforms[row] : 0.f;

  // ---- pass A: max, and the top-digit count histogram for a top-k cut ----------
  zero_hist(sh);
  float m = -INFINITY;
  g.each([&](int, float x) {
    m = fmaxf(m, x);
    if (k_req > 0) atomicAdd(&sh.hist[fkey(x) >> 21], 1ull);
  });
  m = block_max(m, sh);
  auto alive = [&](float x) { return P.min_p <= 0.f || expf(x - m) >= P.min_p; };

  // ---- candidate bound: every kept element has key >= L --------------------------
  // With top-k: the first-digit bin of the k-th largest element (alive or not:
  // the k largest alive are the k largest when k are alive, and otherwise all
  // alive elements are above that bin anyway).  With top-p only: the
  // first-digit bin where the alive mass, from the top, reaches top_p of the
  // whole.
  bool fast = false, have_Z = false;
  uint32_t L = 0;
  unsigned long long Z_all = 0;
  if (k_req > 0) {
    select_bin(sh, 0, static_cast<double>(k_req));
    L = static_cast<uint32_t>(sh.bcast[0]) << 21;
    fast = sh.bcast[1] + sh.hist[sh.bcast[0]] <= static_cast<unsigned long long>(kCand);
  } else if (P.top_p < 1.f) {
    zero_hist(sh);
    g.each([&](int, float x) {
      if (alive(x)) atomicAdd(&sh.hist[fkey(x) >> 21], mass_of(x, m));
    });
    __syncthreads();
    unsigned long long mine = 0;
    for (int b = tid; b < kBins; b += kThreads) mine += sh.hist[b];
    block_exclusive_scan(mine, sh, &Z_all);
    select_bin(sh, 0, static_cast<double>(P.top_p) * static_cast<double>(Z_all));
    L = static_cast<uint32_t>(sh.bcast[0]) << 21;
    have_Z = fast = sh.bcast[2] != 0;
  }
  int64_t tok;
  if (fast) {
    // Ordered compaction of the elements with key >= L into LDS.
    unsigned long long c = 0;
    g.chunk([&](int, float x) { c += fkey(x) >= L ? 1 : 0; });
    unsigned long long n_c;
    const unsigned long long off = block_exclusive_scan(c, sh, &n_c);
    fast = n_c <= static_cast<unsigned long long>(kCand);
    if (fast) {
      int o = static_cast<int>(off);
      g.chunk([&](int i, float x) {
        if (fkey(x) >= L) {
          sh.cx[o] = x;
          sh.ci[o] = i;
          ++o;
        }
      });
      __syncthreads();
      CandSrc cs;
      cs.sh = &sh;
      cs.n = static_cast<int>(n_c);
      tok = filter_and_draw(cs, sh, P, m, k_req, have_Z, Z_all, u);
    }
  }
  if (!fast) tok = filter_and_draw(g, sh, P, m, k_req, false, 0, u);
  if (tid == 0) out[row] = tok;
}

struct Args {
  const void *logits;
  int64_t row_stride;
  int V;
  const float *temperature;
  const int32_t *top_k;
  const float *top_p, *min_p, *rep, *presence, *frequency;
  const int64_t *history;
  int64_t hist_stride;
  const int32_t *hist_len;
  int64_t hist_len_stride;
  const float *uniforms;
  int64_t *out;
};

template <int DT, bool VEC>
int launch(const Args &a, int rows, hipStream_t stream) {
  static bool attr_set = false;  // per instantiation
  const size_t shm = sizeof(Shared);
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&sample_kernel<DT, VEC>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(shm));
    if (e != hipSuccess) return fail(SPK_EHIP, "sample: %s", hipGetErrorString(e));
    attr_set = true;
  }
  sample_kernel<DT, VEC><<<rows, kThreads, shm, stream>>>(
      a.logits, a.row_stride, a.V, a.temperature, a.top_k, a.top_p, a.min_p, a.rep, a.presence,
      a.frequency, a.history, a.hist_stride, a.hist_len, a.hist_len_stride, a.uniforms, a.out);
  return check_launch("sample");
}

}  // namespace smp
}  // namespace spk

using namespace spk;

extern "C" size_t spk_sample_shared_bytes(void) { return sizeof(smp::Shared); }

extern "C" int spk_sample(const void *logits, int logits_dtype, int64_t row_stride, int rows,
                          int vocab, const float *temperature, const int32_t *top_k,
                          const float *top_p, const float *min_p, const float *repetition_penalty,
                          const float *presence_penalty, const float *frequency_penalty,
                          const int64_t *history, int64_t history_stride, const int32_t *history_len,
                          int64_t history_len_stride, const float *uniforms, int64_t *out_tokens,
                          void *stream) {
  if (!valid_float_dtype(logits_dtype))
    return fail(SPK_EINVAL, "sample: logits dtype %d is not a float type", logits_dtype);
  if (!logits || !temperature || !out_tokens) return fail(SPK_EINVAL, "sample: null pointer");
  if (rows < 0 || vocab < 1 || vocab > smp::kMaxVocab || row_stride < vocab)
    return fail(SPK_EINVAL, "sample: vocab=%d must be in [1, %d] and row_stride >= vocab", vocab,
                smp::kMaxVocab);
  if (history && (!history_len || history_stride < 1))
    return fail(SPK_EINVAL, "sample: history needs history_len and a row stride >= 1");
  if (rows == 0) return SPK_OK;
  smp::Args a{logits, row_stride, vocab, temperature, top_k, top_p, min_p, repetition_penalty,
              presence_penalty, frequency_penalty, history, history_stride, history_len,
              history_len_stride, uniforms, out_tokens};
  const size_t esz = logits_dtype == SPK_F32 ? 4 : 2;
  const bool vec = (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && (row_stride * esz) % 16 == 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (logits_dtype) {
    case SPK_F32: return vec ? smp::launch<SPK_F32, true>(a, rows, s) : smp::launch<SPK_F32, false>(a, rows, s);
    case SPK_F16: return vec ? smp::launch<SPK_F16, true>(a, rows, s) : smp::launch<SPK_F16, false>(a, rows, s);
    default: return vec ? smp::launch<SPK_BF16, true>(a, rows, s) : smp::launch<SPK_BF16, false>(a, rows, s);
  }
}
