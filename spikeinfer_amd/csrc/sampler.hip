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

namespace spk {
namespace smp {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kBins = 2048;            // 11-bit digits
constexpr int kMaxVocab = 262144;      // bitmap capacity (32 KB)
constexpr int kMaxHist = 2048;         // history tokens per row
constexpr int kHashSlots = 2 * kMaxHist;
constexpr float kGreedyTemp = 1e-5f;
constexpr double kMassScale = 1099511627776.0;  // 2^40

struct Row {
  const void *logits;
  int dtype;
  int V;
  float temp, min_p, top_p, rep, presence, frequency;
  int top_k;
};

struct Shared {
  uint32_t seen[kMaxVocab / 32];
  int32_t hkey[kHashSlots];
  int32_t hcnt[kHashSlots];
  unsigned long long hist[kBins];
  unsigned long long wsum[kWaves];
  unsigned long long bcast[4];
  float fbcast[kWaves];
};

__device__ __forceinline__ float logit_at(const Row &r, int i) {
  switch (r.dtype) {
    case SPK_F32: return static_cast<const float *>(r.logits)[i];
    case SPK_F16: return static_cast<float>(static_cast<const _Float16 *>(r.logits)[i]);
    default: return bf16_bits_to_f32(static_cast<const uint16_t *>(r.logits)[i]);
  }
}

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
__device__ __forceinline__ float penalised(const Row &r, const Shared &sh, int i, bool use_hash) {
  float v = logit_at(r, i);
  if (!((sh.seen[i >> 5] >> (i & 31)) & 1u)) return v;
  if (r.rep != 1.f) v = v > 0.f ? v / r.rep : v * r.rep;
  if (r.presence != 0.f || r.frequency != 0.f) {
    float cnt = 1.f;
    if (use_hash) {
      int s = hash_slot(i);
      while (sh.hkey[s] != i + 1) s = (s + 1) % kHashSlots;
      cnt = static_cast<float>(sh.hcnt[s]);
    }
    v = v - (r.presence + r.frequency * cnt);
  }
  return v;
}

__device__ __forceinline__ unsigned long long shfl_up_u64(unsigned long long v, int d) {
  const uint32_t lo = __shfl_up(static_cast<uint32_t>(v), d);
  const uint32_t hi = __shfl_up(static_cast<uint32_t>(v >> 32), d);
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

// Exclusive prefix sum over the workgroup in thread order; *total gets the sum.
__device__ unsigned long long block_exclusive_scan(unsigned long long v, Shared &sh,
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

__device__ float block_max(float v, Shared &sh) {
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

__device__ unsigned long long block_max_u64(unsigned long long v, Shared &sh) {
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
__device__ void select_bin(Shared &sh, unsigned long long base, double target) {
  const int j = threadIdx.x;
  const int b1 = kBins - 1 - 2 * j, b2 = b1 - 1;
  const unsigned long long h1 = sh.hist[b1], h2 = sh.hist[b2];
  unsigned long long total;
  const unsigned long long before = base + block_exclusive_scan(h1 + h2, sh, &total);
  if (j == 0) sh.bcast[2] = 0;
  __syncthreads();
  if ((double)before < target && target <= (double)(before + h1)) {
    sh.bcast[0] = b1;
    sh.bcast[1] = before;
    sh.bcast[2] = 1;
  } else if ((double)(before + h1) < target && target <= (double)(before + h1 + h2)) {
    sh.bcast[0] = b2;
    sh.bcast[1] = before + h1;
    sh.bcast[2] = 1;
  }
  __syncthreads();
}

__device__ __forceinline__ unsigned long long mass_of(float x, float m) {
  return static_cast<unsigned long long>(static_cast<double>(expf(x - m)) * kMassScale);
}

__global__ __launch_bounds__(kThreads) void sample_kernel(
    const void *logits, int dtype, int64_t row_stride, int V, const float *temperature,
    const int32_t *top_k, const float *top_p, const float *min_p, const float *rep,
    const float *presence, const float *frequency, const int64_t *history, int64_t hist_stride,
    const int32_t *hist_len, int64_t hist_len_stride, const float *uniforms, int64_t *out) {
  extern __shared__ __align__(16) char smem_raw[];
  Shared &sh = *reinterpret_cast<Shared *>(smem_raw);
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  Row r;
  r.logits = static_cast<const char *>(logits) +
             row * row_stride * (dtype == SPK_F32 ? 4 : 2);
  r.dtype = dtype;
  r.V = V;
  r.temp = temperature[row];
  r.top_k = top_k ? top_k[row] : -1;
  r.top_p = top_p ? top_p[row] : 1.f;
  r.min_p = min_p ? min_p[row] : 0.f;
  r.rep = rep ? rep[row] : 1.f;
  r.presence = presence ? presence[row] : 0.f;
  r.frequency = frequency ? frequency[row] : 0.f;

  // ---- history -> seen bitmap (+ counts) ------------------------------------
  const int nwords = (V + 31) >> 5;
  for (int w = tid; w < nwords; w += kThreads) sh.seen[w] = 0u;
  const bool use_hash = r.frequency != 0.f;
  if (use_hash)
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
      if (use_hash) {
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

  // ---- greedy: argmax of the penalised logits, first index on ties ------------
  if (r.temp < kGreedyTemp) {
    unsigned long long best = 0;
    for (int i = tid; i < V; i += kThreads) {
      const unsigned long long k = (static_cast<unsigned long long>(fkey(penalised(r, sh, i, use_hash))) << 32) |
                                   (0xffffffffu - static_cast<uint32_t>(i));
      best = k > best ? k : best;
    }
    best = block_max_u64(best, sh);
    if (tid == 0) out[row] = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(best));
    return;
  }

  // ---- max of x = penalised / temperature --------------------------------------
  float m = -INFINITY;
  for (int i = tid; i < V; i += kThreads) m = fmaxf(m, penalised(r, sh, i, use_hash) / r.temp);
  m = block_max(m, sh);
  const float min_p_v = r.min_p;
  auto alive = [&](float x) { return min_p_v <= 0.f || expf(x - m) >= min_p_v; };

  // ---- top-k: cut (Kk, tk) on element counts ----------------------------------------
  uint32_t Kk = 0;                // cut key; elements with key > Kk all kept
  unsigned long long tk = ~0ull;  // ties at Kk kept (in index order); ~0 = all
  unsigned long long alive_cnt = 0;
  {
    unsigned long long c = 0;
    for (int i = tid; i < V; i += kThreads) c += alive(penalised(r, sh, i, use_hash) / r.temp) ? 1 : 0;
    unsigned long long tot;
    block_exclusive_scan(c, sh, &tot);
    alive_cnt = tot;
  }
  const long long k_req = (r.top_k < 0 || r.top_k >= V) ? -1 : r.top_k;
  if (k_req > 0 && static_cast<unsigned long long>(k_req) < alive_cnt) {
    uint32_t prefix = 0;
    unsigned long long above = 0;
    for (int pass = 0; pass < 3; ++pass) {
      const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
      const uint32_t dmask = pass == 2 ? 0x3ffu : 0x7ffu;
      const int hi_shift = shift + (pass == 2 ? 10 : 11);
      for (int b = tid; b < kBins; b += kThreads) sh.hist[b] = 0;
      __syncthreads();
      for (int i = tid; i < V; i += kThreads) {
        const float x = penalised(r, sh, i, use_hash) / r.temp;
        if (!alive(x)) continue;
        const uint32_t k = fkey(x);
        if (pass > 0 && (k >> hi_shift) != (prefix >> hi_shift)) continue;
        atomicAdd(&sh.hist[(k >> shift) & dmask], 1ull);
      }
      __syncthreads();
      select_bin(sh, above, static_cast<double>(k_req));
      prefix |= static_cast<uint32_t>(sh.bcast[0]) << shift;
      above = sh.bcast[1];
      __syncthreads();
    }
    Kk = prefix;
    tk = static_cast<unsigned long long>(k_req) - above;
  }

  // Membership in the survivors of min_p and top_k, ties at Kk aside.
  const bool k_partial = tk != ~0ull;
  auto in_s_nontie = [&](float x, uint32_t k) {
    return alive(x) && (k > Kk || (k == Kk && !k_partial));
  };
  const float xK = unkey(Kk);
  const unsigned long long wK = k_partial ? mass_of(xK, m) : 0;

  // ---- top-p: cut (Kf, tf) on probability mass of the survivors ----------------------
  uint32_t Kf = Kk;
  unsigned long long tf = tk;
  if (r.top_p < 1.f) {
    unsigned long long z = 0;
    for (int i = tid; i < V; i += kThreads) {
      const float x = penalised(r, sh, i, use_hash) / r.temp;
      if (in_s_nontie(x, fkey(x))) z += mass_of(x, m);
    }
    unsigned long long Z;
    block_exclusive_scan(z, sh, &Z);
    if (k_partial) Z += tk * wK;
    const double target = static_cast<double>(r.top_p) * static_cast<double>(Z);
    uint32_t prefix = 0;
    unsigned long long above = 0;
    bool found = true;
    for (int pass = 0; pass < 3; ++pass) {
      const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
      const uint32_t dmask = pass == 2 ? 0x3ffu : 0x7ffu;
      const int hi_shift = shift + (pass == 2 ? 10 : 11);
      for (int b = tid; b < kBins; b += kThreads) sh.hist[b] = 0;
      __syncthreads();
      for (int i = tid; i < V; i += kThreads) {
        const float x = penalised(r, sh, i, use_hash) / r.temp;
        const uint32_t k = fkey(x);
        if (!in_s_nontie(x, k)) continue;
        if (pass > 0 && (k >> hi_shift) != (prefix >> hi_shift)) continue;
        atomicAdd(&sh.hist[(k >> shift) & dmask], mass_of(x, m));
      }
      __syncthreads();
      // The kept ties of the top-k cut all weigh wK: add them analytically.
      if (tid == 0 && k_partial && (pass == 0 || (Kk >> hi_shift) == (prefix >> hi_shift)))
        sh.hist[(Kk >> shift) & dmask] += tk * wK;
      __syncthreads();
      select_bin(sh, above, target);
      if (!sh.bcast[2]) found = false;
      prefix |= static_cast<uint32_t>(sh.bcast[0]) << shift;
      above = sh.bcast[1];
      __syncthreads();
      if (!found) break;
    }
    if (found) {
      Kf = prefix;
      const unsigned long long w = mass_of(unkey(Kf), m);
      // Ties at Kf kept: the first j with above + (j - 1) * w < target.
      unsigned long long j = w ? static_cast<unsigned long long>(ceil((target - static_cast<double>(above)) / static_cast<double>(w))) : 1;
      if (j < 1) j = 1;
      if (Kf == Kk && k_partial && j > tk) j = tk;
      tf = j;
    }
  }

  // ---- draw: inverse CDF in index order over the kept weights --------------------------
  // Thread tid owns the contiguous chunk [lo, hi); ties at Kf are ranked by a
  // scan of per-chunk tie counts.
  const int chunk = (V + kThreads - 1) / kThreads;
  const int lo = min(V, tid * chunk), hi = min(V, lo + chunk);
  const bool f_partial = tf != ~0ull;
  unsigned long long wsum = 0, ties = 0;
  for (int i = lo; i < hi; ++i) {
    const float x = penalised(r, sh, i, use_hash) / r.temp;
    const uint32_t k = fkey(x);
    if (!alive(x) || k < Kf) continue;
    if (k == Kf && f_partial) {
      ++ties;
      continue;
    }
    wsum += mass_of(x, m);
  }
  unsigned long long tot_ties;
  const unsigned long long rank0 = block_exclusive_scan(ties, sh, &tot_ties);
  unsigned long long kept_ties = 0;
  if (f_partial) {
    kept_ties = rank0 >= tf ? 0 : (tf - rank0 < ties ? tf - rank0 : ties);
  }
  const unsigned long long wf = f_partial ? mass_of(unkey(Kf), m) : 0;
  const unsigned long long mine = wsum + kept_ties * wf;
  unsigned long long Wtot;
  const unsigned long long before = block_exclusive_scan(mine, sh, &Wtot);
  const float u = uniforms ? uniforms[row] : 0.f;
  unsigned long long target = static_cast<unsigned long long>(static_cast<double>(u) * static_cast<double>(Wtot));
  if (target >= Wtot) target = Wtot ? Wtot - 1 : 0;
  if (tid == 0) sh.bcast[3] = ~0ull;
  __syncthreads();
  if (mine > 0 && before <= target && target < before + mine) {
    unsigned long long acc = before, seen_ties = 0;
    for (int i = lo; i < hi; ++i) {
      const float x = penalised(r, sh, i, use_hash) / r.temp;
      const uint32_t k = fkey(x);
      if (!alive(x) || k < Kf) continue;
      unsigned long long w;
      if (k == Kf && f_partial) {
        if (seen_ties++ >= kept_ties) continue;
        w = wf;
      } else {
        w = mass_of(x, m);
      }
      acc += w;
      if (acc > target) {
        sh.bcast[3] = static_cast<unsigned long long>(i);
        break;
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    unsigned long long pick = sh.bcast[3];
    if (pick == ~0ull) {
      // Every kept weight rounded to zero: fall back to the top element.
      pick = 0;
    }
    out[row] = static_cast<int64_t>(pick);
  }
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
  static bool attr_set = false;
  const size_t shm = sizeof(smp::Shared);
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&smp::sample_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(shm));
    if (e != hipSuccess) return fail(SPK_EHIP, "sample: %s", hipGetErrorString(e));
    attr_set = true;
  }
  smp::sample_kernel<<<rows, smp::kThreads, shm, static_cast<hipStream_t>(stream)>>>(
      logits, logits_dtype, row_stride, vocab, temperature, top_k, top_p, min_p,
      repetition_penalty, presence_penalty, frequency_penalty, history, history_stride,
      history_len, history_len_stride, uniforms, out_tokens);
  return check_launch("sample");
}
