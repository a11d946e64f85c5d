#pragma once
// Batched token sampler (kernel templates; instantiated per logits dtype in
// sampler_f32.hip, sampler_f16.hip and sampler_bf16.hip): one workgroup per row of logits, no host round trip.
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
// fixes it) -- so each cut is a key K plus, among the elements of key K, the
// ones up to some index:
//   * min_p keeps exp(x - max) >= min_p (a value threshold);
//   * top_k: radix select (11/11/10-bit digits of the order-preserving key)
//     on element counts finds the k-th element, and a radix select on the
//     indices of its ties finds how far into them the cut goes;
//   * top_p: the same on probability mass finds the last element whose
//     preceding mass is below top_p of the surviving mass.  Mass is fixed
//     point (weight * 2^40 in uint64), so sums are exact and the cut is
//     deterministic whatever the atomic order.
// The draw takes the element whose interval of the kept mass, accumulated in
// the same total order, holds u * total, for a caller-supplied uniform u in
// [0, 1): one more mass select and one index select.
// Nothing depends on the order elements are visited in, so every pass over
// the row is a coalesced sweep.  With a top-k cut, one sweep gathers the
// elements at or above a sample-estimated threshold into LDS (a few hundred at
// top-k 50) and every later pass runs over those; histograms, the seen-token
// bitmap and the count hash live in LDS too.
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
constexpr int kNoCutCand = 4096;  // without a top-k cut: about 1.5x this many candidates (the margin below)

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
// Penalty of a token known to be in the history.
template <class SH>
__device__ __forceinline__ float penalise_seen(const Params &P, const SH &sh, int i, float v) {
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

__device__ __forceinline__ float penalise(const Params &P, const Shared &sh, int i, float v) {
  if (!((sh.seen[i >> 5] >> (i & 31)) & 1u)) return v;
  return penalise_seen(P, sh, i, v);
}

__device__ __forceinline__ unsigned long long shfl_up_u64(unsigned long long v, int d) {
  const uint32_t lo = __shfl_up(static_cast<uint32_t>(v), d);
  const uint32_t hi = __shfl_up(static_cast<uint32_t>(v >> 32), d);
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

// Exclusive prefix sum over the workgroup in thread order; *total gets the sum.
template <class SH>
__device__ __forceinline__ unsigned long long block_exclusive_scan(unsigned long long v, SH &sh,
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

// Fixed-point mass of a weight e = exp(x - m): e * 2^40, truncated.
__device__ __forceinline__ unsigned long long mass_of_e(float e) {
  return static_cast<unsigned long long>(static_cast<double>(e) * kMassScale);
}
__device__ __forceinline__ unsigned long long mass_of(float x, float m) { return mass_of_e(expf(x - m)); }

__device__ __forceinline__ void zero_hist(Shared &sh) {
  __syncthreads();
  for (int b = threadIdx.x; b < kBins; b += kThreads) sh.hist[b] = 0;
  __syncthreads();
}

// ---- element sources ----------------------------------------------------------------
// each(f) visits every element once, f(index, x), in no particular order.

// The logits row in global memory; x = penalise(raw) / temperature.  Coalesced
// 16-byte loads, eight in flight per thread.
template <int DT, bool VEC>
struct GlobalSrc {
  typedef typename Elem<DT>::T E;
  static constexpr int W = VEC ? Elem<DT>::kVec : 1;
  static constexpr int kInFlight = 8;
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
    for (; v + (kInFlight - 1) * kThreads < nv; v += kInFlight * kThreads) {
      Vec a[kInFlight];
#pragma unroll
      for (int u = 0; u < kInFlight; ++u) a[u] = pv[v + u * kThreads];
#pragma unroll
      for (int u = 0; u < kInFlight; ++u)
#pragma unroll
        for (int j = 0; j < W; ++j) f((v + u * kThreads) * W + j, a[u][j]);
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
  // f(i, v) with v the penalised logit, not divided by the temperature (an
  // order-preserving map of x): one bitmap word per vector, none without
  // history.
  template <class F> __device__ __forceinline__ void each_pen(F f, bool has_hist) const {
    const int nv = V / W;
    const Vec *pv = reinterpret_cast<const Vec *>(p);
    auto one = [&](int b, const Vec &a) {
      const uint32_t bits = has_hist ? (sh->seen[b >> 5] >> (b & 31)) : 0u;
#pragma unroll
      for (int j = 0; j < W; ++j) {
        float v = elem_to_f32<DT>(a[j]);
        if ((bits >> j) & 1u) v = penalise_seen(P, *sh, b + j, v);
        f(b + j, v);
      }
    };
    int v = threadIdx.x;
    for (; v + (kInFlight - 1) * kThreads < nv; v += kInFlight * kThreads) {
      Vec a[kInFlight];
#pragma unroll
      for (int u = 0; u < kInFlight; ++u) a[u] = pv[v + u * kThreads];
#pragma unroll
      for (int u = 0; u < kInFlight; ++u) one((v + u * kThreads) * W, a[u]);
    }
    for (; v < nv; v += kThreads) one(v * W, pv[v]);
    for (int i = nv * W + threadIdx.x; i < V; i += kThreads) {
      const float raw = elem_to_f32<DT>(p[i]);
      f(i, has_hist ? penalise(P, *sh, i, raw) : raw);
    }
  }
};

// Candidates gathered into LDS (any order).
struct CandSrc {
  const Shared *sh;
  int n;
  template <class F> __device__ __forceinline__ void each(F f) const {
    for (int j = threadIdx.x; j < n; j += kThreads) f(sh->ci[j], sh->cx[j]);
  }
};

// Every kSampleStride-th element of the row, gathered into the candidate value
// array before the candidates themselves are.
constexpr int kSampleStride = 32;
struct SampleSrc {
  const Shared *sh;
  int n;
  template <class F> __device__ __forceinline__ void each(F f) const {
    for (int j = threadIdx.x; j < n; j += kThreads) f(j, sh->cx[j]);
  }
};

// ---- order statistics over a source ---------------------------------------------------
// All cuts below are prefixes of one total order: key descending, then index
// ascending.  They are found with radix selects (11/11/10-bit digits of the
// key, 10/10-bit digits of the index), so no pass depends on visiting order.

// Key of the k-th largest element (k >= 1) among those where pred(i, x) holds;
// `above` gets how many have a larger key.
template <class Src, class Pred>
__device__ __forceinline__ uint32_t radix_rank(const Src &src, Shared &sh, unsigned long long k,
                                               Pred pred, unsigned long long &above) {
  uint32_t prefix = 0;
  above = 0;
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const uint32_t dmask = pass == 2 ? 0x3ffu : 0x7ffu;
    const int hi_shift = shift + (pass == 2 ? 10 : 11);
    zero_hist(sh);
    src.each([&](int i, float x) {
      if (!pred(i, x)) return;
      const uint32_t key = fkey(x);
      if (pass > 0 && (key >> hi_shift) != (prefix >> hi_shift)) return;
      atomicAdd(&sh.hist[(key >> shift) & dmask], 1ull);
    });
    __syncthreads();
    select_bin(sh, above, static_cast<double>(k));
    prefix |= static_cast<uint32_t>(sh.bcast[0]) << shift;
    above = sh.bcast[1];
  }
  return prefix;
}

// Key K where the fixed-point mass of the pred elements, accumulated from the
// largest key down, reaches `target`: mass(keys > K) < target <=
// mass(keys >= K).  `extra` is mass to count at key Kx besides the visited
// elements (ties whose membership is decided by index).  Returns false if
// the total is below target.
template <class Src, class Pred>
__device__ __forceinline__ bool mass_select(const Src &src, Shared &sh, Pred pred, float m,
                                            double target, uint32_t Kx, unsigned long long extra,
                                            uint32_t &K, unsigned long long &above) {
  uint32_t prefix = 0;
  above = 0;
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const uint32_t dmask = pass == 2 ? 0x3ffu : 0x7ffu;
    const int hi_shift = shift + (pass == 2 ? 10 : 11);
    zero_hist(sh);
    src.each([&](int i, float x) {
      if (!pred(i, x)) return;
      const uint32_t key = fkey(x);
      if (pass > 0 && (key >> hi_shift) != (prefix >> hi_shift)) return;
      atomicAdd(&sh.hist[(key >> shift) & dmask], mass_of(x, m));
    });
    __syncthreads();
    if (threadIdx.x == 0 && extra && (pass == 0 || (Kx >> hi_shift) == (prefix >> hi_shift)))
      sh.hist[(Kx >> shift) & dmask] += extra;
    __syncthreads();
    select_bin(sh, above, target);
    if (!sh.bcast[2]) return false;
    prefix |= static_cast<uint32_t>(sh.bcast[0]) << shift;
    above = sh.bcast[1];
  }
  K = prefix;
  return true;
}

// Index of the j-th smallest index (j >= 1) among the pred elements (indices
// below 2^20; the vocabulary limit is 2^18).
template <class Src, class Pred>
__device__ __forceinline__ int index_rank(const Src &src, Shared &sh, unsigned long long j,
                                          Pred pred) {
  // Ascending index = descending (2^20 - 1 - index).
  uint32_t prefix = 0;
  unsigned long long above = 0;
  for (int pass = 0; pass < 2; ++pass) {
    const int shift = pass == 0 ? 10 : 0;
    zero_hist(sh);
    src.each([&](int i, float x) {
      if (!pred(i, x)) return;
      const uint32_t r = 0xfffffu - static_cast<uint32_t>(i);
      if (pass > 0 && (r >> 10) != (prefix >> 10)) return;
      atomicAdd(&sh.hist[(r >> shift) & 0x3ffu], 1ull);
    });
    __syncthreads();
    select_bin(sh, above, static_cast<double>(j));
    prefix |= static_cast<uint32_t>(sh.bcast[0]) << shift;
    above = sh.bcast[1];
  }
  return static_cast<int>(0xfffffu - prefix);
}

template <class Src, class Pred>
__device__ __forceinline__ unsigned long long count_if(const Src &src, Shared &sh, Pred pred) {
  unsigned long long c = 0, total;
  src.each([&](int i, float x) { c += pred(i, x) ? 1 : 0; });
  block_exclusive_scan(c, sh, &total);
  return total;
}

template <class Src, class Pred>
__device__ __forceinline__ unsigned long long mass_if(const Src &src, Shared &sh, float m, Pred pred) {
  unsigned long long z = 0, total;
  src.each([&](int i, float x) {
    if (pred(i, x)) z += mass_of(x, m);
  });
  block_exclusive_scan(z, sh, &total);
  return total;
}

// min_p -> top_k -> top_p -> draw over a source; returns the token.  `Z_all`
// (when have_Z) is the alive mass of the whole row, used when the source is a
// candidate subset and no top-k cut bounds the survivors inside it.
// `partial`: src holds only a prefix of the order (the candidates), no top-k
// was requested, and Z_all is the mass of every element min_p keeps in the
// whole row.  A top-p cut or a draw that falls beyond the prefix then returns
// -1 (the caller takes the whole row) instead of being decided on the prefix.
template <class Src>
__device__ __forceinline__ int64_t filter_and_draw(const Src src, Shared &sh, const Params P,
                                                   float m, long long k_req, bool have_Z,
                                                   unsigned long long Z_all, float u,
                                                   bool partial = false) {
  auto alive = [&](float x) { return P.min_p <= 0.f || expf(x - m) >= P.min_p; };
  constexpr int kAll = 0x7fffffff;

  // top-k: kept = key > Kk, or key == Kk and index <= Ik.
  uint32_t Kk = 0;
  int Ik = kAll;
  bool k_cut = false;
  if (k_req > 0) {
    const unsigned long long alive_cnt = count_if(src, sh, [&](int, float x) { return alive(x); });
    if (static_cast<unsigned long long>(k_req) < alive_cnt) {
      unsigned long long above;
      Kk = radix_rank(src, sh, static_cast<unsigned long long>(k_req),
                      [&](int, float x) { return alive(x); }, above);
      Ik = index_rank(src, sh, static_cast<unsigned long long>(k_req) - above,
                      [&](int, float x) { return alive(x) && fkey(x) == Kk; });
      k_cut = true;
    }
  }
  auto in_s = [&](int i, float x) {
    const uint32_t k = fkey(x);
    return alive(x) && (k > Kk || (k == Kk && i <= Ik));
  };

  // top-p over the survivors: kept = in_s and (key > Kf, or key == Kf and
  // index <= If), the shortest prefix whose mass reaches top_p of theirs.
  uint32_t Kf = Kk;
  int If = Ik;
  if (P.top_p < 1.f) {
    const unsigned long long Z = (have_Z && !k_cut) ? Z_all : mass_if(src, sh, m, in_s);
    const double target = static_cast<double>(P.top_p) * static_cast<double>(Z);
    uint32_t K;
    unsigned long long above;
    if (mass_select(src, sh, in_s, m, target, 0u, 0ull, K, above)) {
      const unsigned long long w = mass_of(unkey(K), m);
      // Ties at K kept: the first j (by index) with above + (j - 1) * w < target.
      unsigned long long j =
          w ? static_cast<unsigned long long>(ceil((target - static_cast<double>(above)) / static_cast<double>(w)))
            : 1;
      if (j < 1) j = 1;
      auto tie = [&](int i, float x) { return in_s(i, x) && fkey(x) == K; };
      const unsigned long long c = count_if(src, sh, tie);
      Kf = K;
      If = j >= c ? kAll : index_rank(src, sh, j, tie);
    } else if (partial) {
      return -1;  // the cut lies past the prefix
    }
  }
  auto kept = [&](int i, float x) {
    const uint32_t k = fkey(x);
    return in_s(i, x) && (k > Kf || (k == Kf && i <= If));
  };

  // Draw: the element whose interval of the kept mass, accumulated in the same
  // order (key descending, index ascending), holds u * total.
  // Kept mass: over src, except for a prefix with nothing cut (then the whole
  // row's min_p survivors).
  const bool whole = partial && !(P.top_p < 1.f);
  const unsigned long long Wtot = whole ? Z_all : mass_if(src, sh, m, kept);
  unsigned long long T = static_cast<unsigned long long>(static_cast<double>(u) * static_cast<double>(Wtot));
  if (T >= Wtot) T = Wtot ? Wtot - 1 : 0;
  uint32_t K;
  unsigned long long above;
  if (!mass_select(src, sh, kept, m, static_cast<double>(T) + 1.0, 0u, 0ull, K, above)) {
    if (whole) return -1;  // the draw lies past the prefix
    // Unreachable otherwise: the largest kept element always weighs 2^40.
    return static_cast<int64_t>(index_rank(src, sh, 1, kept));
  }
  const unsigned long long w = mass_of(unkey(K), m);
  const unsigned long long jt = w ? (T - above) / w : 0;
  return static_cast<int64_t>(
      index_rank(src, sh, jt + 1, [&](int i, float x) { return kept(i, x) && fkey(x) == K; }));
}


// ---- sliced candidate stage (rows with a top-k cut) ------------------------------
// The two sweeps over a row are most of the one-workgroup path's time.  For
// rows with 0 < top_k <= kFastMaxK a first launch splits each row into
// kSlices slices, one workgroup each (sample_slices_kernel):
//   * the slice goes into registers once, with the penalties, as keys of the
//     penalised values v; every kSampleStride-th one is a sample;
//   * the r-th largest sample (r = k / kSampleStride + 3, doubled while the
//     candidates fall short) fixes a bound x_B on x = v / temperature, turned
//     once into the smallest v key whose x reaches x_B (a bisection over keys,
//     x monotone in v), so the passes compare keys and divide only the
//     candidates {x >= x_B}, a prefix of the slice in the total order (x
//     descending, index ascending);
//   * with at least k of them (or the whole slice) they hold the slice's k
//     largest: each candidate's rank among them is counted, and the first
//     min(k, n) go to the workspace in order.
// The row kernel then merges a row's lists (ranks by binary search), which
// gives the row's top-k in order, and finishes with prefix sums over it:
// min_p, top_p and the draw are the same cuts as filter_and_draw's, computed
// from the same fixed-point masses with the same comparisons.  A slice that
// cannot certify its list (more than kSliceCand candidates) marks itself -1,
// and sample_kernel takes its row on the one-workgroup path.
constexpr int kSlices = 8;
constexpr int kSliceThreads = 512;
constexpr int kSliceCand = 1024;
constexpr int kFastMaxK = 256;
static_assert(kFastMaxK < kThreads, "the finish takes one thread per kept position");
constexpr int kSliceMaxLen = ((kMaxVocab + kSlices - 1) / kSlices + 255) & ~255;
constexpr int kSliceSamples = kSliceMaxLen / kSampleStride;
constexpr int kSampleRegs = kSliceSamples / 64;  // samples a lane of wave 0 reads

__host__ __device__ inline int slice_len(int V) { return ((V + kSlices - 1) / kSlices + 255) & ~255; }

// k of a row's top-k cut, or -1 (no cut).
__device__ __forceinline__ long long k_request(int top_k, int V) {
  return (top_k < 0 || top_k >= V) ? -1 : top_k;
}
__device__ __forceinline__ bool sliced_row(float temp, long long k_req) {
  return !(temp < kGreedyTemp) && k_req > 0 && k_req <= kFastMaxK;
}

// The total order as one integer: larger = earlier (x descending, index ascending).
__device__ __forceinline__ unsigned long long order_key(float x, int i) {
  return (static_cast<unsigned long long>(fkey(x)) << 32) | (0xffffffffu - static_cast<uint32_t>(i));
}

// Workspace: x [rows][kSlices][kFastMaxK] float, index the same in int32,
// then count [rows][kSlices] int32, maximum v [rows][kSlices] float and the
// open rows' alive mass [rows][kSlices] uint64.
struct SliceWs {
  float *x;
  int32_t *idx;
  int32_t *count;
  float *vmax;
  unsigned long long *zpart;
};
__host__ __device__ inline size_t slice_ws_bytes(int rows) {
  return static_cast<size_t>(rows) * kSlices * (2 * kFastMaxK * 4 + 16);
}
__host__ __device__ inline SliceWs slice_ws(void *base, int rows) {
  char *b = static_cast<char *>(base);
  const size_t n = static_cast<size_t>(rows) * kSlices;
  SliceWs w;
  w.x = reinterpret_cast<float *>(b);
  w.idx = reinterpret_cast<int32_t *>(b + n * kFastMaxK * 4);
  w.count = reinterpret_cast<int32_t *>(b + 2 * n * kFastMaxK * 4);
  w.vmax = reinterpret_cast<float *>(b + 2 * n * kFastMaxK * 4 + n * 4);
  w.zpart = reinterpret_cast<unsigned long long *>(b + 2 * n * kFastMaxK * 4 + n * 8);
  return w;
}

// Stages a call may run (the caller's `stages` bits): the top-k stage for rows
// with 0 < top_k <= kFastMaxK, the open stage for rows with no top-k cut and
// a top-p or min-p cut (open_row).
constexpr int kStageTopK = 1;
constexpr int kStageOpen = 2;
// Launch modes of sample_slices_kernel.
constexpr int kModeTopK = 0;     // top-k rows: list of the slice's k largest
constexpr int kModeOpenMax = 1;  // open rows: the slice's largest penalised logit only
constexpr int kModeOpen = 2;     // open rows: list of the slice's kOpenK largest + alive mass
// An open row's slices list their kOpenK largest: the merged lists then
// certify about the row's first 400 (the largest of the slices' 64th keys).
constexpr int kOpenK = 64;
// Open rows the stage takes: sampled, no top-k cut, and a top-p or min-p cut
// (a draw over the whole mass lands past the certified prefix too often, and
// one such row sends the batch's slowest workgroup down the whole row).
__device__ __forceinline__ bool open_row(float temp, long long k_req, float top_p, float min_p) {
  return !(temp < kGreedyTemp) && k_req <= 0 && (top_p < 1.f || min_p > 0.f);
}

// Maximum over the wave (DPP within rows of 16, then the four rows).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  auto dpp = [](uint32_t x, int ctrl) -> uint32_t {
    switch (ctrl) {
      case 0xB1: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0xB1, 0xF, 0xF, false));
      case 0x4E: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x4E, 0xF, 0xF, false));
      case 0x141: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x141, 0xF, 0xF, false));
      default: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x140, 0xF, 0xF, false));
    }
  };
  v = max(v, dpp(v, 0xB1));   // quad_perm [1,0,3,2]
  v = max(v, dpp(v, 0x4E));   // quad_perm [2,3,0,1]
  v = max(v, dpp(v, 0x141));  // row_half_mirror
  v = max(v, dpp(v, 0x140));  // row_mirror
  const uint32_t r0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 0));
  const uint32_t r1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 16));
  const uint32_t r2 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 32));
  const uint32_t r3 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 48));
  return max(max(r0, r1), max(r2, r3));
}

struct SliceShared {
  uint32_t seen[kSliceMaxLen / 32];  // the slice's generated-token bits
  int32_t hkey[kHashSlots];          // token + 1 -> count, tokens of the slice
  int32_t hcnt[kHashSlots];
  uint32_t samp[kSliceSamples];      // sample keys (of v)
  unsigned long long cand[kSliceCand + 16];  // candidates' order keys (+ a zero batch)
  float fmax[kSliceThreads / 64];
  uint32_t wcount[kSliceThreads / 64];
  unsigned long long zw[kSliceThreads / 64];
  uint32_t bound;
};

// A thread's share of a slice: vectors v = threadIdx.x + q * kSliceThreads
// of the slice's whole vectors (elements v * W ..), every load issued at once
// (vectors past them re-read the first and are dropped), plus one of the < W
// trailing elements.  After pass A it holds the keys of the penalised
// logits, so later passes only compare keys.  No load leaves the slice.
// Needs 16-byte aligned rows (the host checks).
template <int DT>
struct SliceRegs {
  typedef typename Elem<DT>::T E;
  static constexpr int W = Elem<DT>::kVec;
  static constexpr int kVecs = kSliceMaxLen / (W * kSliceThreads);
  typedef E Vec __attribute__((ext_vector_type(W)));
  Vec a[kVecs];
  E tail;
  uint32_t key[kVecs * W + 1];  // slot q * W + j; the last one the trailing element
  int nv;                       // whole vectors of the slice
  bool tail_valid;

  __device__ __forceinline__ void load(const E *row, int c0, int n) {
    const Vec *pv = reinterpret_cast<const Vec *>(row + c0);
    nv = n / W;
    if (nv > 0) {  // (a slice of fewer than W elements has no whole vector to re-read)
#pragma unroll
      for (int q = 0; q < kVecs; ++q) {
        const int v = threadIdx.x + q * kSliceThreads;
        a[q] = pv[v < nv ? v : 0];
      }
    }
    const int t = nv * W + static_cast<int>(threadIdx.x);
    tail_valid = t < n;
    tail = row[c0 + (tail_valid ? t : 0)];
  }
  __device__ __forceinline__ bool valid(int slot) const {
    return slot == kVecs * W ? tail_valid : static_cast<int>(threadIdx.x) + (slot / W) * kSliceThreads < nv;
  }
  __device__ __forceinline__ int elem(int slot) const {  // offset in the slice
    return slot == kVecs * W ? nv * W + static_cast<int>(threadIdx.x)
                             : (static_cast<int>(threadIdx.x) + (slot / W) * kSliceThreads) * W + slot % W;
  }
  // Pass A: key of every penalised logit; f(b, v) for each valid element.
  template <class F>
  __device__ __forceinline__ void penalise_all(int c0, const Params &P, const SliceShared &sh, bool has_hist, F f) {
#pragma unroll
    for (int q = 0; q < kVecs; ++q) {
      const int v = threadIdx.x + q * kSliceThreads;
      const int b = v * W;
      const bool ok = v < nv;
      const uint32_t bits = has_hist && ok ? ((sh.seen[b >> 5] >> (b & 31)) & ((1u << W) - 1u)) : 0u;
#pragma unroll
      for (int j = 0; j < W; ++j) {
        float x = elem_to_f32<DT>(a[q][j]);
        if ((bits >> j) & 1u) x = penalise_seen(P, sh, c0 + b + j, x);
        key[q * W + j] = fkey(x);
        if (ok) f(b + j, x);
      }
    }
    const int b = nv * W + static_cast<int>(threadIdx.x);
    float x = elem_to_f32<DT>(tail);
    if (tail_valid && has_hist && ((sh.seen[b >> 5] >> (b & 31)) & 1u)) x = penalise_seen(P, sh, c0 + b, x);
    key[kVecs * W] = fkey(x);
    if (tail_valid) f(b, x);
  }
};

template <int DT, int MODE>
__global__ __launch_bounds__(kSliceThreads) void sample_slices_kernel(
    const void *logits, int64_t row_stride, int V, const float *temperature, const int32_t *top_k,
    const float *top_p, const float *min_p, const float *rep, const float *presence,
    const float *frequency, const int64_t *history, int64_t hist_stride, const int32_t *hist_len,
    int64_t hist_len_stride, SliceWs ws) {
  typedef typename Elem<DT>::T E;
  __shared__ SliceShared sh;
  const int row = blockIdx.x / kSlices, sl = blockIdx.x % kSlices;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  Params P;
  P.temp = temperature[row];
  P.top_k = top_k ? top_k[row] : -1;
  P.rep = rep ? rep[row] : 1.f;
  P.presence = presence ? presence[row] : 0.f;
  P.frequency = frequency ? frequency[row] : 0.f;
  P.use_hash = P.frequency != 0.f;
  P.top_p = MODE != kModeTopK && top_p ? top_p[row] : 1.f;
  P.min_p = MODE != kModeTopK && min_p ? min_p[row] : 0.f;
  const long long k_row = k_request(P.top_k, V);
  if (MODE == kModeTopK ? !sliced_row(P.temp, k_row) : !open_row(P.temp, k_row, P.top_p, P.min_p))
    return;  // the row workgroup does not read this slice
  const long long k_req = MODE == kModeTopK ? k_row : static_cast<long long>(kOpenK);
  const int64_t ws_i = static_cast<int64_t>(row) * kSlices + sl;
  const int L = slice_len(V), c0 = sl * L, c1 = min(V, c0 + L);
  if (c0 >= c1) {
    if (tid == 0) {
      if (MODE != kModeOpenMax) ws.count[ws_i] = 0;
      if (MODE != kModeOpen) ws.vmax[ws_i] = -INFINITY;
      if (MODE == kModeOpen) ws.zpart[ws_i] = 0ull;
    }
    return;
  }
  // Open rows: the row's largest penalised logit, from the max-only launch
  // before this one (vector loads, not the scalar cache).
  float m_row = -INFINITY;
  if (MODE == kModeOpen) {
#pragma unroll
    for (int s2 = 0; s2 < kSlices; ++s2)
      m_row = fmaxf(m_row, __hip_atomic_load(ws.vmax + static_cast<int64_t>(row) * kSlices + s2,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  }
  SliceRegs<DT> rg;  // the slice's logits, loaded while the history is read
  rg.load(reinterpret_cast<const E *>(logits) + row * row_stride, c0, c1 - c0);
  // ---- history -> the slice's bits (+ counts) ----
  for (int w = tid; w < (c1 - c0 + 31) / 32; w += kSliceThreads) sh.seen[w] = 0u;
  if (P.use_hash)
    for (int s2 = tid; s2 < kHashSlots; s2 += kSliceThreads) sh.hkey[s2] = 0, sh.hcnt[s2] = 0;
  __syncthreads();
  int nh = 0;
  if (history && hist_len) {
    nh = hist_len[row * hist_len_stride];
    const int64_t cap = hist_stride < kMaxHist ? hist_stride : kMaxHist;
    nh = nh < 0 ? 0 : (nh > cap ? static_cast<int>(cap) : nh);
    for (int j = tid; j < nh; j += kSliceThreads) {
      const int64_t tok = history[row * hist_stride + j];
      if (tok < c0 || tok >= c1) continue;
      const int t32 = static_cast<int>(tok);
      atomicOr(&sh.seen[(t32 - c0) >> 5], 1u << ((t32 - c0) & 31));
      if (P.use_hash) {
        int h = hash_slot(t32);
        while (true) {
          const int prev = atomicCAS(&sh.hkey[h], 0, t32 + 1);
          if (prev == 0 || prev == t32 + 1) break;
          h = (h + 1) % kHashSlots;
        }
        atomicAdd(&sh.hcnt[h], 1);
      }
    }
  }
  __syncthreads();
  const bool has_hist = nh > 0;

  // ---- maximum and samples (keys of v) ----
  float mv = -INFINITY;
  rg.penalise_all(c0, P, sh, has_hist, [&](int b, float v) {
    mv = fmaxf(mv, v);
    if (MODE != kModeOpenMax && (b % kSampleStride) == 0) sh.samp[b / kSampleStride] = fkey(v);
  });
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) mv = fmaxf(mv, __shfl_xor(mv, d));
  if (lane == 0) sh.fmax[wave] = mv;
  __syncthreads();
  if constexpr (MODE == kModeOpenMax) {
    if (tid == 0) {
      float m = sh.fmax[0];
      for (int w = 1; w < kSliceThreads / 64; ++w) m = fmaxf(m, sh.fmax[w]);
      ws.vmax[ws_i] = m;
    }
    return;
  }

  // ---- bound and candidates.  Wave 0 takes the r-th largest sample, then
  // the smallest v key whose x reaches that sample's x; every thread counts
  // its elements at or above it.  Too few candidates (fewer than k, the
  // slice not exhausted): r doubles and the registers are counted again. ----
  const int n_s = (c1 - c0 + kSampleStride - 1) / kSampleStride;
  const long long kk = (k_req + kSampleStride - 1) / kSampleStride;
  int r = static_cast<int>(min<long long>(n_s, kk + 3));
  uint32_t n = 0, mine = 0, incl = 0, bound = 0;
  while (true) {
    if (wave == 0) {
      uint32_t key[kSampleRegs];  // sample keys; 0 (a NaN's key) past the samples
#pragma unroll
      for (int q = 0; q < kSampleRegs; ++q) {
        const int j = q * 64 + lane;
        key[q] = j < n_s ? sh.samp[j] : 0u;
      }
      uint32_t best = 0;
      for (int it = 0; it < min(r, n_s); ++it) {  // remove the largest r - 1 times, one copy each
        uint32_t m = 0;
#pragma unroll
        for (int q = 0; q < kSampleRegs; ++q) m = key[q] > m ? key[q] : m;
        best = wave_max_u32(m);
        const unsigned long long holders = __ballot(m == best);
        if (lane == static_cast<int>(__builtin_ctzll(holders))) {
          bool done = false;
#pragma unroll
          for (int q = 0; q < kSampleRegs; ++q)
            if (!done && key[q] == best) {
              key[q] = 0u;
              done = true;
            }
        }
      }
      // The smallest key k in (0, best] with unkey(k) / temp >= unkey(best) /
      // temp (key 0 is a NaN's: never): 64 keys tested a round, one a lane.
      const float xb = unkey(best) / P.temp;
      uint32_t lo = 0, hi = best;
      while (hi - lo > 1) {
        const uint32_t step = (hi - lo + 63) / 64;
        const uint32_t k = min(hi, lo + step * static_cast<uint32_t>(lane + 1));
        const unsigned long long t = __ballot(unkey(k) / P.temp >= xb);  // lane 63 tests hi
        if (t == 0) break;  // only with a NaN bound: keep hi
        const int first = static_cast<int>(__builtin_ctzll(t));
        hi = min(hi, lo + step * static_cast<uint32_t>(first + 1));
        lo = first == 0 ? lo : lo + step * static_cast<uint32_t>(first);
      }
      if (lane == 0) sh.bound = r > n_s ? 0u : hi;  // r past the samples: every element
    }
    __syncthreads();
    bound = sh.bound;
    mine = 0;
#pragma unroll
    for (int q = 0; q <= SliceRegs<DT>::kVecs * SliceRegs<DT>::W; ++q)
      mine += rg.valid(q) && rg.key[q] >= bound ? 1u : 0u;
    incl = mine;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t o = __shfl_up(incl, d);
      if (lane >= d) incl += o;
    }
    if (lane == 63) sh.wcount[wave] = incl;
    __syncthreads();
    n = 0;
#pragma unroll
    for (int w = 0; w < kSliceThreads / 64; ++w) n += sh.wcount[w];
    __syncthreads();  // wcount and bound are rewritten by a retry
    if (static_cast<long long>(n) >= k_req || static_cast<int>(n) == c1 - c0 || r > n_s) break;
    r = r == n_s ? n_s + 1 : min(n_s, 2 * r);
  }
  uint32_t off = incl - mine;
#pragma unroll
  for (int w = 0; w < kSliceThreads / 64; ++w) off += w < wave ? sh.wcount[w] : 0u;
  if (mine) {
#pragma unroll
    for (int q = 0; q <= SliceRegs<DT>::kVecs * SliceRegs<DT>::W; ++q) {
      if (!(rg.valid(q) && rg.key[q] >= bound)) continue;
      if (off < static_cast<uint32_t>(kSliceCand)) sh.cand[off] = order_key(unkey(rg.key[q]) / P.temp, c0 + rg.elem(q));
      ++off;
    }
  }
  if (n <= static_cast<uint32_t>(kSliceCand) && tid < 16) sh.cand[n + tid] = 0ull;
  __syncthreads();
  const bool ok = n <= static_cast<uint32_t>(kSliceCand) &&
                  (static_cast<long long>(n) >= k_req || static_cast<int>(n) == c1 - c0);
  const int nk = static_cast<int>(min<long long>(n, k_req));
  if (ok) {
    // The first nk candidates in order, each placed by its rank among them.
    float *xo = ws.x + ws_i * kFastMaxK;
    int32_t *io = ws.idx + ws_i * kFastMaxK;
    for (int c = tid; c < static_cast<int>(n); c += kSliceThreads) {
      const unsigned long long kc = sh.cand[c];
      int rank = 0;
      // 16 keys a batch, loads first (keys past n are zero: never greater).
      for (int d0 = 0; d0 < static_cast<int>(n); d0 += 16) {
        unsigned long long kd[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) kd[q] = sh.cand[d0 + q];
#pragma unroll
        for (int q = 0; q < 16; ++q) rank += kd[q] > kc ? 1 : 0;
      }
      if (rank < nk) {
        xo[rank] = unkey(static_cast<uint32_t>(kc >> 32));
        io[rank] = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(kc));
      }
    }
  }
  if constexpr (MODE == kModeOpen) {
    // The slice's share of the row's alive mass, element for element the sum
    // the one-workgroup path forms (x = v / temperature, the same min_p test
    // and fixed-point mass against the row's largest x); integer sums, so the
    // row's total is exact whatever the order.
    const float m = m_row / P.temp;
    unsigned long long z = 0;
#pragma unroll
    for (int q = 0; q <= SliceRegs<DT>::kVecs * SliceRegs<DT>::W; ++q) {
      if (!rg.valid(q)) continue;
      const float x = unkey(rg.key[q]) / P.temp;
      const float e = expf(x - m);
      if (P.min_p <= 0.f || e >= P.min_p) z += mass_of_e(e);
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
      const uint32_t lo = __shfl_xor(static_cast<uint32_t>(z), d);
      const uint32_t hi = __shfl_xor(static_cast<uint32_t>(z >> 32), d);
      z += (static_cast<unsigned long long>(hi) << 32) | lo;
    }
    if (lane == 0) sh.zw[wave] = z;
    __syncthreads();
    if (tid == 0) {
      unsigned long long zs = 0;
      for (int w = 0; w < kSliceThreads / 64; ++w) zs += sh.zw[w];
      ws.zpart[ws_i] = zs;
      ws.count[ws_i] = ok ? nk : -1;
    }
  } else {
    if (tid == 0) {
      ws.count[ws_i] = ok ? nk : -1;
      float m = sh.fmax[0];
      for (int w = 1; w < kSliceThreads / 64; ++w) m = fmaxf(m, sh.fmax[w]);
      ws.vmax[ws_i] = m;
    }
  }
}

// Merged positions the finish holds (one a thread).
constexpr int kOpenPrefix = kThreads;
static_assert(kSlices * kOpenK <= kOpenPrefix, "an open row's merged lists fit the finish");

struct FinishShared {
  unsigned long long lists[kSlices * kFastMaxK];  // the slices' lists as order keys
  float cx[kOpenPrefix];                          // the merged prefix, in order
  int32_t ci[kOpenPrefix];
  unsigned long long cums[kOpenPrefix + 1];       // kept mass before each position
  unsigned long long wsum[kWaves];
  unsigned long long bcast[4];
};

// Whether the slices certified row `row`'s lists (every count >= 0); n gets
// the counts and *vmax the row's largest penalised logit.
__device__ __forceinline__ bool sliced_lists(const SliceWs &ws, int row, int (&n)[kSlices], float *vmax) {
  bool ok = true;
  float mv = -INFINITY;
#pragma unroll
  for (int sl = 0; sl < kSlices; ++sl) {
    // Vector loads (not the scalar cache): the slices kernel wrote these.
    n[sl] = __hip_atomic_load(ws.count + static_cast<int64_t>(row) * kSlices + sl, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
    ok = ok && n[sl] >= 0;
    mv = fmaxf(mv, __hip_atomic_load(ws.vmax + static_cast<int64_t>(row) * kSlices + sl, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT));
  }
  *vmax = mv;
  return ok;
}

// The row's sliced finish (see above): the merged top-k in sh.cx / sh.ci, in
// order, then min_p, top_p and the draw as filter_and_draw makes them.
//
// Open rows (no top-k cut; `open`): every slice listed its kOpenK largest,
// so the merged lists are the row's order up to the first element any slice
// left out.  The certified prefix is every element whose key is above the
// last listed key of each slice that listed fewer than all its elements
// (whole key groups only, since ties are ordered by index).  min_p keeps a prefix of it; the top-p target is
// top_p of the whole row's alive mass (the slices' exact partial sums), and
// the draw is over the top-p prefix or, without a top-p cut, over that whole
// mass.  A cut or a draw past the certified prefix returns -1: the caller
// then takes the row through the one-workgroup path.  Every kept decision is
// the one the whole-row computation makes.
__device__ __forceinline__ int64_t sliced_finish(FinishShared &sh, const SliceWs &ws, int row, const Params &P,
                                                 long long k_req, float u, const int (&n)[kSlices], float m,
                                                 bool open, int V) {
  const int tid = threadIdx.x;
  // Merge: element j of slice s goes to position j + (number of elements of
  // the other slices earlier in the order), found by binary search in each
  // (sorted) list, staged in LDS as order keys.  Positions >= k are dropped.
  const int64_t base = static_cast<int64_t>(row) * kSlices * kFastMaxK;
  unsigned long long *lists = sh.lists;
  int total = 0;
#pragma unroll
  for (int s = 0; s < kSlices; ++s) {
    for (int j = tid; j < n[s]; j += kThreads)
      lists[s * kFastMaxK + j] = order_key(ws.x[base + s * kFastMaxK + j], ws.idx[base + s * kFastMaxK + j]);
    total += n[s];
  }
  __syncthreads();
  const int kept_k = open ? total : static_cast<int>(min<long long>(k_req, total));
  for (int e = tid; e < total; e += kThreads) {  // element e of the lists, concatenated
    int s = 0, j = e, before = 0;  // (list, position) of e; n[] indexed by constants only
#pragma unroll
    for (int t = 0; t < kSlices; ++t) {
      if (e >= before && e < before + n[t]) {
        s = t;
        j = e - before;
      }
      before += n[t];
    }
    const unsigned long long kj = lists[s * kFastMaxK + j];
    int pos = j;
#pragma unroll
    for (int t = 0; t < kSlices; ++t) {
      if (t == s) continue;
      int lo = 0, hi = n[t];  // count of list t's elements earlier than kj
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (lists[t * kFastMaxK + mid] > kj) lo = mid + 1;
        else hi = mid;
      }
      pos += lo;
    }
    if (pos < kept_k) {
      sh.cx[pos] = unkey(static_cast<uint32_t>(kj >> 32));
      sh.ci[pos] = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(kj));
    }
  }
  __syncthreads();
  // Open rows: keys above `cut` (when has_cut) are certified.
  bool has_cut = false;
  uint32_t cut = 0;
  unsigned long long Z_all = 0;
  if (open) {
    const int L = slice_len(V);
#pragma unroll
    for (int t = 0; t < kSlices; ++t) {
      const int len_t = max(0, min(V, (t + 1) * L) - t * L);
      if (n[t] < len_t) {  // (an empty list of a non-empty slice certifies nothing)
        const uint32_t kt = n[t] > 0 ? static_cast<uint32_t>(lists[t * kFastMaxK + n[t] - 1] >> 32) : 0xffffffffu;
        cut = has_cut ? max(cut, kt) : kt;
        has_cut = true;
      }
      Z_all += __hip_atomic_load(ws.zpart + static_cast<int64_t>(row) * kSlices + t, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // Per position j < kept_k (one thread each; kept_k <= kOpenPrefix = kThreads).
  const int j = tid;
  const float x0 = j < kept_k ? sh.cx[j] : 0.f;
  const bool live = j < kept_k && !(has_cut && fkey(x0) <= cut);
  const float x = live ? x0 : 0.f;
  const uint32_t key = fkey(x);
  const bool alive = live && (P.min_p <= 0.f || expf(x - m) >= P.min_p);
  // The alive elements are a prefix; the top-k cut keeps the first min(k, alive).
  const int n1 = __syncthreads_count(alive);
  const bool in1 = j < n1;
  const unsigned long long w = in1 ? mass_of(x, m) : 0ull;
  unsigned long long Z;
  const unsigned long long cum = block_exclusive_scan(w, sh, &Z);  // mass before position j
  // Group start of j (first position with j's key) = j - (earlier equal keys).
  int gs = j;
  if (in1)
    while (gs > 0 && fkey(sh.cx[gs - 1]) == key) --gs;
  // cum of each position, for the group lookups
  unsigned long long *cums = sh.cums;
  if (in1) cums[j] = cum;
  if (tid == 0) cums[n1] = Z;
  __syncthreads();
  // top_p: the group K with mass(keys > K) < target <= mass(keys >= K) (the
  // first element of each group tests its group), then j ties of it.
  int n2 = n1;
  if (P.top_p < 1.f) {
    const double target = static_cast<double>(P.top_p) * static_cast<double>(open ? Z_all : Z);
    if (tid == 0) sh.bcast[2] = 0;
    __syncthreads();
    if (in1 && gs == j) {
      int ge = j + 1;
      while (ge < n1 && fkey(sh.cx[ge]) == key) ++ge;
      const unsigned long long before = cum, after = cums[ge];
      if (static_cast<double>(before) < target && target <= static_cast<double>(after)) {
        unsigned long long jt = w ? static_cast<unsigned long long>(ceil((target - static_cast<double>(before)) /
                                                                         static_cast<double>(w)))
                                  : 1;
        if (jt < 1) jt = 1;
        const unsigned long long c = static_cast<unsigned long long>(ge - j);
        sh.bcast[0] = static_cast<unsigned long long>(j) + (jt >= c ? c : jt);
        sh.bcast[2] = 1;
      }
    }
    __syncthreads();
    const bool found = sh.bcast[2] != 0;
    if (found) n2 = static_cast<int>(sh.bcast[0]);
    __syncthreads();
    if (open && !found) return -1;  // the cut lies past the certified prefix
  }
  // Draw: the element whose interval of the kept mass holds u * total (an
  // open row without a top-p cut: the whole row's alive mass).
  const unsigned long long Wtot = open && !(P.top_p < 1.f) ? Z_all : cums[n2];
  unsigned long long T = static_cast<unsigned long long>(static_cast<double>(u) * static_cast<double>(Wtot));
  if (T >= Wtot) T = Wtot ? Wtot - 1 : 0;
  const double target = static_cast<double>(T) + 1.0;
  if (tid == 0) sh.bcast[2] = 0;
  __syncthreads();
  if (j < n2 && gs == j) {
    int ge = j + 1;
    while (ge < n2 && fkey(sh.cx[ge]) == key) ++ge;
    const unsigned long long before = cum, after = cums[ge];
    if (static_cast<double>(before) < target && target <= static_cast<double>(after)) {
      const unsigned long long jt = w ? (T - before) / w : 0;
      sh.bcast[0] = static_cast<unsigned long long>(sh.ci[j + static_cast<int>(jt)]);
      sh.bcast[2] = 1;
    }
  }
  __syncthreads();
  if (sh.bcast[2]) return static_cast<int64_t>(sh.bcast[0]);
  if (open && !(P.top_p < 1.f)) return -1;  // the draw lies past the certified prefix
  // No interval holds it (not reached: the first kept element weighs 2^40):
  // the smallest kept index.
  int best = 0x7fffffff;
  for (int q = 0; q < n2; ++q) best = min(best, static_cast<int>(sh.ci[q]));
  return best;
}

template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void sample_kernel(
    const void *logits, int64_t row_stride, int V, const float *temperature,
    const int32_t *top_k, const float *top_p, const float *min_p, const float *rep,
    const float *presence, const float *frequency, const int64_t *history, int64_t hist_stride,
    const int32_t *hist_len, int64_t hist_len_stride, const float *uniforms, int64_t *out, SliceWs ws,
    int stages) {
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

  // ---- sliced rows whose slices certified their lists: merge and finish ------
  // (an open row's finish may leave the row undecided: then the row takes the
  // one-workgroup path below)
  const bool topk_s = (stages & kStageTopK) && sliced_row(P.temp, k_request(P.top_k, V));
  const bool open_s = (stages & kStageOpen) && open_row(P.temp, k_request(P.top_k, V), P.top_p, P.min_p);
  if (ws.count && (topk_s || open_s)) {
    int n[kSlices];
    float mv;
    if (sliced_lists(ws, row, n, &mv)) {
      static_assert(sizeof(FinishShared) <= sizeof(Shared), "the finish reuses the row kernel's LDS");
      const int64_t tok = sliced_finish(*reinterpret_cast<FinishShared *>(smem_raw), ws, row, P,
                                        k_request(P.top_k, V), uniforms ? uniforms[row] : 0.f, n, mv / P.temp,
                                        open_s, V);
      if (tok >= 0) {
        if (tid == 0) out[row] = tok;
        return;
      }
      __syncthreads();  // the one-workgroup path reuses the LDS
    }
  }

  // ---- history -> seen bitmap (+ counts) ------------------------------------
  const int nwords = (V + 31) >> 5;
  for (int w = tid; w < nwords; w += kThreads) sh.seen[w] = 0u;
  if (P.use_hash)
    for (int s = tid; s < kHashSlots; s += kThreads) sh.hkey[s] = 0, sh.hcnt[s] = 0;
  __syncthreads();
  int nh = 0;
  if (history && hist_len) {
    nh = hist_len[row * hist_len_stride];
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

  const long long k_req = k_request(P.top_k, V);
  const float u = uniforms ? uniforms[row] : 0.f;

  // ---- pass A (on the penalised logits v; x = v / temperature preserves
  // their order): max, and every 32nd value as a sample ----
  const bool has_hist = nh > 0;
  float mv = -INFINITY;
  const bool sample = true;  // the candidate bound comes from these samples
  g.each_pen([&](int i, float v) {
    mv = fmaxf(mv, v);
    if (sample && (i % kSampleStride) == 0) sh.cx[i / kSampleStride] = v;
  }, has_hist);
  mv = block_max(mv, sh);
  const float m = mv / P.temp;  // the largest x

  // ---- candidates: the elements at or above a bound L, a prefix of the
  // order, gathered into LDS.  L is taken from the samples: with a top-k cut,
  // the r-th largest sample, r a margin above k / kSampleStride, so that when
  // the candidates number at least k and fit in LDS the k largest (alive or
  // not) are among them, and so is everything any later cut keeps.  Without a
  // top-k cut, about kNoCutCand candidates; the same sweep then sums the mass
  // of every min_p survivor of the row, and the candidates decide the row
  // whenever the top-p cut and the draw fall inside them.  Otherwise the row
  // itself is the source.  The bound is taken 64 key steps low: an element
  // just under it in v may round to the same x as one above it.
  int64_t tok = -1;
  unsigned long long Z_alive = 0;
  {
    SampleSrc smp_src;
    smp_src.sh = &sh;
    smp_src.n = (V + kSampleStride - 1) / kSampleStride;
    const long long kk = k_req > 0 ? (k_req + kSampleStride - 1) / kSampleStride
                                   : kNoCutCand / kSampleStride;
    const long long r = min<long long>(smp_src.n, kk + (kk + 1) / 2 + 8);
    unsigned long long above;
    const uint32_t Ls =
        radix_rank(smp_src, sh, static_cast<unsigned long long>(r), [](int, float) { return true; }, above);
    const uint32_t L = Ls > 64u ? Ls - 64u : 0u;
    // Unordered append; the counter keeps counting past the capacity.
    __syncthreads();
    if (tid == 0) sh.bcast[3] = 0;
    __syncthreads();
    const bool sum_alive = k_req <= 0;
    unsigned long long z = 0;
    g.each_pen([&](int i, float v) {
      if (sum_alive) {
        const float e = expf(v / P.temp - m);
        if (P.min_p <= 0.f || e >= P.min_p) z += mass_of_e(e);
      }
      if (fkey(v) < L) return;
      const unsigned long long o = atomicAdd(&sh.bcast[3], 1ull);
      if (o < static_cast<unsigned long long>(kCand)) {
        sh.cx[o] = v / P.temp;
        sh.ci[o] = i;
      }
    }, has_hist);
    __syncthreads();
    const unsigned long long n_c = sh.bcast[3];
    if (sum_alive) block_exclusive_scan(z, sh, &Z_alive);
    if (n_c <= static_cast<unsigned long long>(kCand) &&
        n_c >= static_cast<unsigned long long>(k_req > 0 ? k_req : 1)) {
      CandSrc cs;
      cs.sh = &sh;
      cs.n = static_cast<int>(n_c);
      tok = k_req > 0 ? filter_and_draw(cs, sh, P, m, k_req, false, 0, u)
                      : filter_and_draw(cs, sh, P, m, k_req, true, Z_alive, u, true);
    }
  }
  if (tok < 0) tok = filter_and_draw(g, sh, P, m, k_req, k_req <= 0, Z_alive, u);
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
  void *workspace;  // slice_ws_bytes(rows), or null: one workgroup per row throughout
  int stages;       // kStageTopK | kStageOpen: the sliced stages to run (with a workspace)
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
  SliceWs ws{nullptr, nullptr, nullptr, nullptr, nullptr};
  int stages = 0;
  if constexpr (VEC) {  // the sliced stages read whole 16-byte vectors: aligned rows only
    if (a.workspace && a.stages) {
      ws = slice_ws(a.workspace, rows);
      stages = a.stages;
      if (stages & kStageOpen) {  // the row maxima, then the lists and masses
        sample_slices_kernel<DT, kModeOpenMax><<<rows * kSlices, kSliceThreads, 0, stream>>>(
            a.logits, a.row_stride, a.V, a.temperature, a.top_k, a.top_p, a.min_p, a.rep, a.presence, a.frequency,
            a.history, a.hist_stride, a.hist_len, a.hist_len_stride, ws);
        sample_slices_kernel<DT, kModeOpen><<<rows * kSlices, kSliceThreads, 0, stream>>>(
            a.logits, a.row_stride, a.V, a.temperature, a.top_k, a.top_p, a.min_p, a.rep, a.presence, a.frequency,
            a.history, a.hist_stride, a.hist_len, a.hist_len_stride, ws);
      }
      if (stages & kStageTopK)
        sample_slices_kernel<DT, kModeTopK><<<rows * kSlices, kSliceThreads, 0, stream>>>(
            a.logits, a.row_stride, a.V, a.temperature, a.top_k, a.top_p, a.min_p, a.rep, a.presence, a.frequency,
            a.history, a.hist_stride, a.hist_len, a.hist_len_stride, ws);
    }
  }
  sample_kernel<DT, VEC><<<rows, kThreads, shm, stream>>>(
      a.logits, a.row_stride, a.V, a.temperature, a.top_k, a.top_p, a.min_p, a.rep, a.presence,
      a.frequency, a.history, a.hist_stride, a.hist_len, a.hist_len_stride, a.uniforms, a.out, ws, stages);
  return check_launch("sample");
}


#define SPK_SAMPLER_INSTANTIATE(DT)                                      \
  template int launch<DT, true>(const Args &, int, hipStream_t);         \
  template int launch<DT, false>(const Args &, int, hipStream_t);

}  // namespace smp
}  // namespace spk
