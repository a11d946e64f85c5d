// Per-layer operators of the spiking decoder around the two GEMMs: the fused
// q/k/v RoPE -> LIF -> pack -> cache write, the fused MLP gate LIF * up,
// residual-add + RMSNorm, the final RMSNorm + rate-coded mean over T, and the
// device-side step advance that lets a captured decode step replay without
// the host.
//
// Reference semantics (the composition each kernel replaces):
//   * spikeinfer/modeling_fast.py:89-99 (_apply_rope_t), :121-135 (spike_qkv),
//     :186-190 (MLP), :206-211 (decoder layer), :319 (norm + mean over T);
//   * transformers Qwen2RMSNorm (fp32 variance, rsqrt, cast, weight multiply);
//   * spikeinfer/attention.py:138-149 (k/v cache scatter, q packing);
//   * spikeinfer/engine/model_runner.py:89-100 (position, slot and seq_len of
//     the next decode token).
// Every elementwise result is rounded to the tensor dtype where the torch
// composition rounds it, so the spike bits equal those of the composition on
// the same projection output.  Compiled with -ffp-contract=off.
#include "common.hpp"
#include "lif_math.hpp"
#include "norm_rows.hpp"

namespace spk {

constexpr int kTBatchQkv = 4;  // timesteps whose loads are issued together
// q/k/v launches with at least this many 8-channel lanes (prefill) take the
// vector kernel; smaller ones (decode) the channel-pair kernel.
constexpr int64_t kQkvWideThreads = 256 * 256;
constexpr int kMaxMeanT = 8;   // timesteps rmsnorm_mean_t keeps in registers
constexpr int kNormRegVecs = 4;  // 16-byte vectors per lane add_rmsnorm keeps in registers

// ---- residual add + RMSNorm ---------------------------------------------------
// One wave per row.  h <- round(h + delta) (when delta is given), then
// out = round(weight * round(x * rsqrt(mean(x^2) + eps))) with x = float(h).
template <int DT>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(typename Elem<DT>::T *h,
                                                          const typename Elem<DT>::T *delta,
                                                          const typename Elem<DT>::T *weight,
                                                          typename Elem<DT>::T *out, int64_t rows,
                                                          int hidden, float eps) {
  typedef typename Elem<DT>::T E;
  constexpr int V = Elem<DT>::kVec;
  typedef E Vec __attribute__((ext_vector_type(V)));
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x * (int64_t)(blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  Vec *hr = reinterpret_cast<Vec *>(h + row * hidden);
  const Vec *dr = delta ? reinterpret_cast<const Vec *>(delta + row * hidden) : nullptr;
  const Vec *wr = reinterpret_cast<const Vec *>(weight);
  Vec *orow = reinterpret_cast<Vec *>(out + row * hidden);
  const int nv = hidden / V;
  auto add = [&](Vec x, int v) {
    if (dr) {
      const Vec d = dr[v];
#pragma unroll
      for (int i = 0; i < V; ++i) x[i] = f32_to_elem<DT>(elem_to_f32<DT>(x[i]) + elem_to_f32<DT>(d[i]));
      hr[v] = x;
    }
    return x;
  };
  auto sumsq = [&](const Vec &x) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float f = elem_to_f32<DT>(x[i]);
      ss += f * f;
    }
    return ss;
  };
  auto norm = [&](const Vec &x, const Vec &w, int v, float r) {
    Vec y;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float n = round_to<DT>(elem_to_f32<DT>(x[i]) * r);
      y[i] = f32_to_elem<DT>(elem_to_f32<DT>(w[i]) * n);
    }
    orow[v] = y;
  };
  float ss = 0.f;
  if (nv <= 64 * kNormRegVecs) {
    // The row stays in registers between the two halves; the weights are
    // loaded with it, ahead of the reduction.
    Vec xs[kNormRegVecs], ws[kNormRegVecs];
#pragma unroll
    for (int k = 0; k < kNormRegVecs; ++k) {
      const int v = lane + 64 * k;
      if (v < nv) ws[k] = wr[v];
    }
#pragma unroll
    for (int k = 0; k < kNormRegVecs; ++k) {
      const int v = lane + 64 * k;
      if (v < nv) {
        xs[k] = add(hr[v], v);
        ss += sumsq(xs[k]);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float r = rsqrtf(ss * (1.f / static_cast<float>(hidden)) + eps);
#pragma unroll
    for (int k = 0; k < kNormRegVecs; ++k) {
      const int v = lane + 64 * k;
      if (v < nv) norm(xs[k], ws[k], v, r);
    }
    return;
  }
  for (int v = lane; v < nv; v += 64) ss += sumsq(add(hr[v], v));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  const float r = rsqrtf(ss * (1.f / static_cast<float>(hidden)) + eps);
  for (int v = lane; v < nv; v += 64) norm(hr[v], wr[v], v, r);
}


// add_rmsnorm for rows of at most 64 * kNormRegVecs vectors (hidden 896 at
// bf16 is 112): every load of the row -- weights, h, delta -- is issued at once
// (lanes past the row re-read its last vector and drop it), so a wave waits
// for one memory round trip; with a branch per load the compiler waited for
// each in turn.
template <int DT, bool ADD>
__global__ __launch_bounds__(64) void add_rmsnorm_reg_kernel(typename Elem<DT>::T *h,
                                                             const typename Elem<DT>::T *delta,
                                                             const typename Elem<DT>::T *weight,
                                                             typename Elem<DT>::T *out, int hidden,
                                                             float eps) {
  typedef typename Elem<DT>::T E;
  constexpr int V = Elem<DT>::kVec;
  typedef E Vec __attribute__((ext_vector_type(V)));
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  Vec *hr = reinterpret_cast<Vec *>(h + row * hidden);
  const Vec *dr = reinterpret_cast<const Vec *>(delta + (ADD ? row * hidden : 0));
  const Vec *wr = reinterpret_cast<const Vec *>(weight);
  Vec *orow = reinterpret_cast<Vec *>(out + row * hidden);
  const int nv = hidden / V;
  Vec xs[kNormRegVecs], ds[kNormRegVecs], ws[kNormRegVecs];
#pragma unroll
  for (int k = 0; k < kNormRegVecs; ++k) {
    const int v = min(lane + 64 * k, nv - 1);
    ws[k] = wr[v];
    xs[k] = hr[v];
    if (ADD) ds[k] = dr[v];
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNormRegVecs; ++k) {
    const int v = lane + 64 * k;
    const bool mine = v < nv;
    if (ADD) {
#pragma unroll
      for (int i = 0; i < V; ++i) xs[k][i] = f32_to_elem<DT>(elem_to_f32<DT>(xs[k][i]) + elem_to_f32<DT>(ds[k][i]));
      if (mine) hr[v] = xs[k];
    }
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float f = elem_to_f32<DT>(xs[k][i]);
      part += f * f;
    }
    ss += mine ? part : 0.f;
  }
  const float r = rsqrtf(wave_sum(ss) * (1.f / static_cast<float>(hidden)) + eps);
#pragma unroll
  for (int k = 0; k < kNormRegVecs; ++k) {
    const int v = lane + 64 * k;
    if (v >= nv) continue;
    Vec y;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float n = round_to<DT>(elem_to_f32<DT>(xs[k][i]) * r);
      y[i] = f32_to_elem<DT>(elem_to_f32<DT>(ws[k][i]) * n);
    }
    orow[v] = y;
  }
}

// ---- embedding + first RMSNorm ------------------------------------------------
// One wave per token: e = embed[clamp(ids[i], 0, vocab - 1)], then for every
// timestep t: h[t, i] = e and out[t, i] = round(weight * round(e * r)) with
// r = rsqrt(mean(e^2) + eps) (the input is the same at every timestep, so the
// norm is computed once).
template <int DT>
__global__ __launch_bounds__(256) void embed_rmsnorm_kernel(const int64_t *ids,
                                                            const typename Elem<DT>::T *embed,
                                                            int64_t vocab,
                                                            const typename Elem<DT>::T *weight,
                                                            typename Elem<DT>::T *h,
                                                            typename Elem<DT>::T *out, int T,
                                                            int64_t n, int hidden, float eps) {
  typedef typename Elem<DT>::T E;
  constexpr int V = Elem<DT>::kVec;
  typedef E Vec __attribute__((ext_vector_type(V)));
  const int lane = threadIdx.x & 63;
  const int64_t tok = blockIdx.x * (int64_t)(blockDim.x >> 6) + (threadIdx.x >> 6);
  if (tok >= n) return;
  int64_t id = ids[tok];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  const Vec *er = reinterpret_cast<const Vec *>(embed + id * hidden);
  const Vec *wr = reinterpret_cast<const Vec *>(weight);
  const int nv = hidden / V;
  const int64_t tstep = n * hidden / V;  // Vecs per timestep
  Vec *hr = reinterpret_cast<Vec *>(h + tok * hidden);
  Vec *orow = reinterpret_cast<Vec *>(out + tok * hidden);
  auto emit = [&](const Vec &e, const Vec &w, int v, float r) {
    Vec y;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float nrm = round_to<DT>(elem_to_f32<DT>(e[i]) * r);
      y[i] = f32_to_elem<DT>(elem_to_f32<DT>(w[i]) * nrm);
    }
    for (int t = 0; t < T; ++t) {
      hr[t * tstep + v] = e;
      orow[t * tstep + v] = y;
    }
  };
  auto sumsq = [&](const Vec &x) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float f = elem_to_f32<DT>(x[i]);
      ss += f * f;
    }
    return ss;
  };
  float ss = 0.f;
  if (nv <= 64 * kNormRegVecs) {
    Vec es[kNormRegVecs], ws[kNormRegVecs];
#pragma unroll
    for (int k = 0; k < kNormRegVecs; ++k) {
      const int v = lane + 64 * k;
      if (v < nv) {
        es[k] = er[v];
        ws[k] = wr[v];
        ss += sumsq(es[k]);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float r = rsqrtf(ss * (1.f / static_cast<float>(hidden)) + eps);
#pragma unroll
    for (int k = 0; k < kNormRegVecs; ++k) {
      const int v = lane + 64 * k;
      if (v < nv) emit(es[k], ws[k], v, r);
    }
    return;
  }
  for (int v = lane; v < nv; v += 64) ss += sumsq(er[v]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  const float r = rsqrtf(ss * (1.f / static_cast<float>(hidden)) + eps);
  for (int v = lane; v < nv; v += 64) emit(er[v], wr[v], v, r);
}

// ---- final RMSNorm + mean over the T timesteps --------------------------------
// h [T, rows, hidden] (+ delta, rounded, when given; h is not written) ->
// out [rows, hidden] = round(sum_t norm_t * (1/T)).
template <int DT>
__global__ __launch_bounds__(256) void rmsnorm_mean_t_kernel(const typename Elem<DT>::T *h,
                                                             const typename Elem<DT>::T *delta,
                                                             const typename Elem<DT>::T *weight,
                                                             typename Elem<DT>::T *out, int T,
                                                             int64_t rows, int hidden, float eps) {
  typedef typename Elem<DT>::T E;
  constexpr int V = Elem<DT>::kVec;
  typedef E Vec __attribute__((ext_vector_type(V)));
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x * (int64_t)(blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nv = hidden / V;
  const Vec *wr = reinterpret_cast<const Vec *>(weight);
  Vec *orow = reinterpret_cast<Vec *>(out + row * hidden);
  auto load = [&](int t, int v) {
    Vec x = reinterpret_cast<const Vec *>(h + (t * rows + row) * hidden)[v];
    if (delta) {
      const Vec d = reinterpret_cast<const Vec *>(delta + (t * rows + row) * hidden)[v];
#pragma unroll
      for (int i = 0; i < V; ++i) x[i] = f32_to_elem<DT>(elem_to_f32<DT>(x[i]) + elem_to_f32<DT>(d[i]));
    }
    return x;
  };
  // Pass 1: the T inverse RMS values.
  float rs[kMaxMeanT];
#pragma unroll
  for (int t = 0; t < kMaxMeanT; ++t) {
    if (t >= T) break;
    float ss = 0.f;
    for (int v = lane; v < nv; v += 64) {
      const Vec x = load(t, v);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float f = elem_to_f32<DT>(x[i]);
        ss += f * f;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    rs[t] = rsqrtf(ss * (1.f / static_cast<float>(hidden)) + eps);
  }
  // Pass 2: normalise each timestep and average in fp32, t in order.
  for (int v = lane; v < nv; v += 64) {
    const Vec w = wr[v];
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
#pragma unroll
    for (int t = 0; t < kMaxMeanT; ++t) {
      if (t >= T) break;
      const Vec x = load(t, v);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float n = round_to<DT>(elem_to_f32<DT>(x[i]) * rs[t]);
        acc[i] += round_to<DT>(elem_to_f32<DT>(w[i]) * n);
      }
    }
    Vec y;
#pragma unroll
    for (int i = 0; i < V; ++i) y[i] = f32_to_elem<DT>(acc[i] * (1.f / static_cast<float>(T)));
    orow[v] = y;
  }
}

// The same for rows of at most 2 * 64 vectors and T <= 4 (hidden 896 at bf16):
// one wave per row with every load of the row -- all timesteps of h and delta,
// the weights -- issued at once (lanes past the row re-read its last vector),
// DPP sums; the same roundings and t order as rmsnorm_mean_t_kernel.
constexpr int kMeanRegVecs = 2;
constexpr int kMeanRegT = 4;
template <int DT, bool ADD>
__global__ __launch_bounds__(64) void rmsnorm_mean_t_reg_kernel(const typename Elem<DT>::T *h,
                                                                const typename Elem<DT>::T *delta,
                                                                const typename Elem<DT>::T *weight,
                                                                typename Elem<DT>::T *out, int T,
                                                                int64_t rows, int hidden, float eps) {
  typedef typename Elem<DT>::T E;
  constexpr int V = Elem<DT>::kVec;
  typedef E Vec __attribute__((ext_vector_type(V)));
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int nv = hidden / V;
  Vec x[kMeanRegT][kMeanRegVecs], d[kMeanRegT][kMeanRegVecs], w[kMeanRegVecs];
#pragma unroll
  for (int k = 0; k < kMeanRegVecs; ++k) {
    const int v = min(lane + 64 * k, nv - 1);
    w[k] = reinterpret_cast<const Vec *>(weight)[v];
#pragma unroll
    for (int t = 0; t < kMeanRegT; ++t) {
      const int64_t off = (min(t, T - 1) * rows + row) * hidden;
      x[t][k] = reinterpret_cast<const Vec *>(h + off)[v];
      if (ADD) d[t][k] = reinterpret_cast<const Vec *>(delta + off)[v];
    }
  }
  float rs[kMeanRegT];
#pragma unroll
  for (int t = 0; t < kMeanRegT; ++t) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kMeanRegVecs; ++k) {
      if (ADD) {
#pragma unroll
        for (int i = 0; i < V; ++i)
          x[t][k][i] = f32_to_elem<DT>(elem_to_f32<DT>(x[t][k][i]) + elem_to_f32<DT>(d[t][k][i]));
      }
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float f = elem_to_f32<DT>(x[t][k][i]);
        part += f * f;
      }
      ss += lane + 64 * k < nv ? part : 0.f;
    }
    rs[t] = rsqrtf(wave_sum(ss) * (1.f / static_cast<float>(hidden)) + eps);
  }
  Vec *orow = reinterpret_cast<Vec *>(out + row * hidden);
#pragma unroll
  for (int k = 0; k < kMeanRegVecs; ++k) {
    const int v = lane + 64 * k;
    if (v >= nv) continue;
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
#pragma unroll
    for (int t = 0; t < kMeanRegT; ++t) {
      if (t >= T) break;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float n = round_to<DT>(elem_to_f32<DT>(x[t][k][i]) * rs[t]);
        acc[i] += round_to<DT>(elem_to_f32<DT>(w[k][i]) * n);
      }
    }
    Vec y;
#pragma unroll
    for (int i = 0; i < V; ++i) y[i] = f32_to_elem<DT>(acc[i] * (1.f / static_cast<float>(T)));
    orow[v] = y;
  }
}

// ---- fused q/k/v: RoPE -> LIF -> pack -> packed q / cache slots -------------------
struct QkvParams {
  const void *x;           // [T, n_tok, (Hq + 2 Hkv) * D], channel stride 1
  int64_t xs0, xs1;
  const void *cos, *sin;   // [n_tok, D], or [table_rows, D] indexed by pos[token]
  const int64_t *pos;      // nullptr: row = token
  int64_t table_rows;
  const void *beta, *th;   // [3, D] contiguous: q, k, v sites
  int param_dtype;
  uint64_t *q_packed;      // [T, n_q, Hq, W] (strides in int32 words)
  int64_t qs0, qs1, qs2, n_q;
  uint64_t *k_cache, *v_cache;  // [T, Hkv, slots, W] (strides in int32 words)
  int64_t cs0, cs1, cs2;
  const int64_t *slots;
  int64_t num_slots;
  void *dense[3];          // optional [T, H, n_tok, D] spikes per site
  int T;
  int64_t n_tok;
  int Hq, Hkv, D;
};

// Wide launches (prefill): D/8 lanes per (token, head) row, 8 channels (16
// bytes) per lane, fewer and wider memory accesses than the pair layout.  The
// rotate-half partner of channel c < D/2 is c + D/2, held by lane sub ^ (D/16)
// of the same row; rows never straddle a wave (64 % (D/8) == 0).
template <int DT>
__global__ __launch_bounds__(256) void qkv_rope_lif_pack_vec_kernel(QkvParams p) {
  typedef typename Elem<DT>::T E;
  typedef E Vec __attribute__((ext_vector_type(8)));
  const int L = p.D >> 3;
  const int Htot = p.Hq + 2 * p.Hkv;
  const int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t row = g / L;
  const int sub = static_cast<int>(g - row * L);
  const bool active = row < p.n_tok * Htot;
  const int64_t tok = active ? row / Htot : 0;
  const int hh = active ? static_cast<int>(row - tok * Htot) : 0;
  const int site = hh < p.Hq ? 0 : (hh < p.Hq + p.Hkv ? 1 : 2);
  const int h = site == 0 ? hh : (site == 1 ? hh - p.Hq : hh - p.Hq - p.Hkv);
  const int cl = sub * 8;                      // channel within the head
  const int half = L >> 1;
  const bool low = sub < half;                 // channels below D/2
  const bool rope = site != 2;

  float beta[8], th[8], u[8], cs[8], sn[8];
  int64_t crow = tok;
  if (p.pos && active) {  // positions outside the table read its nearest row
    const int64_t q = p.pos[tok];
    crow = q < 0 ? 0 : (q >= p.table_rows ? p.table_rows - 1 : q);
  }
  const Vec cv = active ? reinterpret_cast<const Vec *>(static_cast<const E *>(p.cos) + crow * p.D)[sub] : Vec{};
  const Vec sv = active ? reinterpret_cast<const Vec *>(static_cast<const E *>(p.sin) + crow * p.D)[sub] : Vec{};
  load_params(p.beta, p.param_dtype, site * p.D + cl, beta);
  load_params(p.th, p.param_dtype, site * p.D + cl, th);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    beta[i] = clamp01(beta[i]);
    u[i] = 0.f;
    cs[i] = elem_to_f32<DT>(cv[i]);
    sn[i] = elem_to_f32<DT>(sv[i]);
  }

  // Destination of this row's packed words.
  uint64_t *dst = nullptr;
  int64_t dstep = 0;  // per timestep, in uint64 words
  if (active) {
    if (site == 0) {
      if (tok < p.n_q) {
        dst = p.q_packed + (tok * p.qs1 + h * p.qs2) / 2;
        dstep = p.qs0 / 2;
      }
    } else {
      const int64_t slot = p.slots[tok];
      if (slot >= 0 && slot < p.num_slots) {
        dst = (site == 1 ? p.k_cache : p.v_cache) + (h * p.cs1 + slot * p.cs2) / 2;
        dstep = p.cs0 / 2;
      }
    }
  }
  E *dense = active ? static_cast<E *>(p.dense[site]) : nullptr;
  const int Hs = site == 0 ? p.Hq : p.Hkv;
  const int64_t dense_row = (static_cast<int64_t>(h) * p.n_tok + tok) * p.D + cl;
  const int64_t dense_tstep = static_cast<int64_t>(Hs) * p.n_tok * p.D;

  const E *xrow = static_cast<const E *>(p.x) + tok * p.xs1 + hh * p.D + cl;
  for (int t0 = 0; t0 < p.T; t0 += kTBatchQkv) {
    Vec xv[kTBatchQkv];
#pragma unroll
    for (int k = 0; k < kTBatchQkv; ++k)
      xv[k] = (active && t0 + k < p.T)
                  ? __builtin_nontemporal_load(reinterpret_cast<const Vec *>(xrow + (t0 + k) * p.xs0))
                  : Vec{};
#pragma unroll
    for (int k = 0; k < kTBatchQkv; ++k) {
      if (t0 + k >= p.T) break;
      const int t = t0 + k;
      const Vec x = xv[k];
      // Partner half of the head (all lanes take part in the exchange).
      Vec xp;
      {
        typedef uint32_t U4 __attribute__((ext_vector_type(4)));
        U4 w = __builtin_bit_cast(U4, x);
        U4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = __shfl_xor(w[j], half);
        xp = __builtin_bit_cast(Vec, r);
      }
      uint32_t byte = 0;
      Vec spk;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float cur = elem_to_f32<DT>(x[i]);
        if (rope) {
          const float xr = low ? -elem_to_f32<DT>(xp[i]) : elem_to_f32<DT>(xp[i]);
          cur = round_to<DT>(round_to<DT>(cur * cs[i]) + round_to<DT>(xr * sn[i]));
        }
        const bool s = lif_step(u[i], cur, beta[i], th[i]);
        byte |= s ? (1u << i) : 0u;
        spk[i] = spike_elem<DT>(s);
      }
      // OR the 8 spike bytes of each aligned 8-lane group into a 64-bit word.
      const int s8 = sub & 7;
      uint32_t lo = s8 < 4 ? byte << (8 * s8) : 0u;
      uint32_t hi = s8 < 4 ? 0u : byte << (8 * (s8 - 4));
#pragma unroll
      for (int off = 1; off < 8; off <<= 1) {
        lo |= __shfl_xor(lo, off);
        hi |= __shfl_xor(hi, off);
      }
      if (dst && s8 == 0) dst[t * dstep + (sub >> 3)] = (static_cast<uint64_t>(hi) << 32) | lo;
      if (dense) *reinterpret_cast<Vec *>(dense + t * dense_tstep + dense_row) = spk;
    }
  }
}

// R = min(D/2, 64) lanes per (token, head) row; lane `sub` owns the channel
// pairs (c, c + D/2) for c = sub + R*j, j < D/(2R), so the rotate-half
// partner of each channel is in the same lane.  Rows never straddle a wave
// (64 % R == 0), and the packed words come from wave ballots: bit `lane` of
// ballot(spike of c) is channel c of the lane's row.
template <int DT>
__global__ __launch_bounds__(256) void qkv_rope_lif_pack_kernel(QkvParams p) {
  typedef typename Elem<DT>::T E;
  constexpr int kMaxPairs = 4;                 // D <= 512
  const int half = p.D >> 1;
  const int R = half < 64 ? half : 64;
  const int P = half / R;
  const int Htot = p.Hq + 2 * p.Hkv;
  const int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t row = g / R;
  const int sub = static_cast<int>(g - row * R);
  const int lane = threadIdx.x & 63;
  const bool active = row < p.n_tok * Htot;
  const int64_t tok = active ? row / Htot : 0;
  const int hh = active ? static_cast<int>(row - tok * Htot) : 0;
  const int site = hh < p.Hq ? 0 : (hh < p.Hq + p.Hkv ? 1 : 2);
  const int h = site == 0 ? hh : (site == 1 ? hh - p.Hq : hh - p.Hq - p.Hkv);
  const bool rope = site != 2;

  float blo[kMaxPairs], bhi[kMaxPairs], tlo[kMaxPairs], thi[kMaxPairs];
  float clo[kMaxPairs], chi[kMaxPairs], slo[kMaxPairs], shi[kMaxPairs];
  float ulo[kMaxPairs], uhi[kMaxPairs];
  int64_t crow = tok;
  if (p.pos && active) {  // positions outside the table read its nearest row
    const int64_t q = p.pos[tok];
    crow = q < 0 ? 0 : (q >= p.table_rows ? p.table_rows - 1 : q);
  }
  const E *cosr = static_cast<const E *>(p.cos) + crow * p.D;
  const E *sinr = static_cast<const E *>(p.sin) + crow * p.D;
#pragma unroll
  for (int j = 0; j < kMaxPairs; ++j) {
    if (j >= P) break;
    const int c = sub + R * j;
    float b1[1], t1[1];
    load_params(p.beta, p.param_dtype, site * p.D + c, b1);
    blo[j] = clamp01(b1[0]);
    load_params(p.th, p.param_dtype, site * p.D + c, t1);
    tlo[j] = t1[0];
    load_params(p.beta, p.param_dtype, site * p.D + c + half, b1);
    bhi[j] = clamp01(b1[0]);
    load_params(p.th, p.param_dtype, site * p.D + c + half, t1);
    thi[j] = t1[0];
    clo[j] = active ? elem_to_f32<DT>(cosr[c]) : 0.f;
    chi[j] = active ? elem_to_f32<DT>(cosr[c + half]) : 0.f;
    slo[j] = active ? elem_to_f32<DT>(sinr[c]) : 0.f;
    shi[j] = active ? elem_to_f32<DT>(sinr[c + half]) : 0.f;
    ulo[j] = uhi[j] = 0.f;
  }

  // Destination of this row's packed words (D/64 per timestep).
  uint64_t *dst = nullptr;
  int64_t dstep = 0;  // per timestep, in uint64 words
  if (active) {
    if (site == 0) {
      if (tok < p.n_q) {
        dst = p.q_packed + (tok * p.qs1 + h * p.qs2) / 2;
        dstep = p.qs0 / 2;
      }
    } else {
      const int64_t slot = p.slots[tok];
      if (slot >= 0 && slot < p.num_slots) {
        dst = (site == 1 ? p.k_cache : p.v_cache) + (h * p.cs1 + slot * p.cs2) / 2;
        dstep = p.cs0 / 2;
      }
    }
  }
  E *dense = active ? static_cast<E *>(p.dense[site]) : nullptr;
  const int Hs = site == 0 ? p.Hq : p.Hkv;
  const int64_t dense_row = (static_cast<int64_t>(h) * p.n_tok + tok) * p.D;
  const int64_t dense_tstep = static_cast<int64_t>(Hs) * p.n_tok * p.D;
  const int rshift = R == 32 ? 32 * ((lane >> 5) & 1) : 0;  // this row's bits of a ballot

  const E *xrow = static_cast<const E *>(p.x) + tok * p.xs1 + hh * p.D;
  for (int t0 = 0; t0 < p.T; t0 += kTBatchQkv) {
    E xl[kTBatchQkv][kMaxPairs], xh[kTBatchQkv][kMaxPairs];
#pragma unroll
    for (int k = 0; k < kTBatchQkv; ++k)
#pragma unroll
      for (int j = 0; j < kMaxPairs; ++j) {
        const bool ld = active && t0 + k < p.T && j < P;
        xl[k][j] = ld ? xrow[(t0 + k) * p.xs0 + sub + R * j] : E{};
        xh[k][j] = ld ? xrow[(t0 + k) * p.xs0 + sub + R * j + half] : E{};
      }
#pragma unroll
    for (int k = 0; k < kTBatchQkv; ++k) {
      if (t0 + k >= p.T) break;
      const int t = t0 + k;
#pragma unroll
      for (int j = 0; j < kMaxPairs; ++j) {
        if (j >= P) break;
        float lo = elem_to_f32<DT>(xl[k][j]), hi = elem_to_f32<DT>(xh[k][j]);
        if (rope) {
          const float rl = round_to<DT>(round_to<DT>(lo * clo[j]) + round_to<DT>(-hi * slo[j]));
          const float rh = round_to<DT>(round_to<DT>(hi * chi[j]) + round_to<DT>(lo * shi[j]));
          lo = rl;
          hi = rh;
        }
        const bool sl = lif_step(ulo[j], lo, blo[j], tlo[j]);
        const bool sh = lif_step(uhi[j], hi, bhi[j], thi[j]);
        const uint64_t ml = __ballot(sl), mh = __ballot(sh);
        if (dst && sub == 0) {
          if (R == 32) {
            dst[t * dstep] = ((ml >> rshift) & 0xffffffffull) | (((mh >> rshift) & 0xffffffffull) << 32);
          } else {
            dst[t * dstep + j] = ml;
            dst[t * dstep + P + j] = mh;
          }
        }
        if (dense) {
          dense[t * dense_tstep + dense_row + sub + R * j] = spike_elem<DT>(sl);
          dense[t * dense_tstep + dense_row + sub + R * j + half] = spike_elem<DT>(sh);
        }
      }
    }
  }
}

// ---- MLP gate: LIF(gate) * up ----------------------------------------------------
// x [T, rows, 2I] (gate in columns [0, I), up in [I, 2I)), out [T, rows, I]
// contiguous = round(spike * up), the product the reference forms in the
// model dtype.
template <int DT>
__global__ __launch_bounds__(256) void lif_gate_mul_kernel(const typename Elem<DT>::T *x, int64_t xs0,
                                                           int64_t xs1, const void *beta_p,
                                                           const void *th_p, int param_dtype,
                                                           typename Elem<DT>::T *out, int T,
                                                           int64_t rows, int I) {
  typedef typename Elem<DT>::T E;
  constexpr int V = Elem<DT>::kVec;
  typedef E Vec __attribute__((ext_vector_type(V)));
  const int64_t groups = rows * (I / V);
  const int64_t gi = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (gi >= groups) return;
  const int64_t row = gi / (I / V);
  const int c0 = static_cast<int>(gi - row * (I / V)) * V;
  float beta[V], th[V], zth[V], u[V];
  bool r[V];
  load_params(beta_p, param_dtype, c0, beta);
  load_params(th_p, param_dtype, c0, th);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    beta[i] = clamp01(beta[i]);
    u[i] = 0.f;
    zth[i] = 0.f * th[i];
    r[i] = 0.f - th[i] > 0.f;
  }
  const E *grow = x + row * xs1 + c0;
  E *orow = out + row * I + c0;
  for (int t0 = 0; t0 < T; t0 += kTBatchQkv) {
    Vec gv[kTBatchQkv], uv[kTBatchQkv];
#pragma unroll
    for (int k = 0; k < kTBatchQkv; ++k) {
      if (t0 + k < T) {
        gv[k] = __builtin_nontemporal_load(reinterpret_cast<const Vec *>(grow + (t0 + k) * xs0));
        uv[k] = __builtin_nontemporal_load(reinterpret_cast<const Vec *>(grow + (t0 + k) * xs0 + I));
      }
    }
#pragma unroll
    for (int k = 0; k < kTBatchQkv; ++k) {
      if (t0 + k >= T) break;
      Vec y;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const bool s = lif_step_r(u[i], r[i], elem_to_f32<DT>(gv[k][i]), beta[i], th[i], zth[i]);
        y[i] = f32_to_elem<DT>((s ? 1.f : 0.f) * elem_to_f32<DT>(uv[k][i]));
      }
      __builtin_nontemporal_store(y, reinterpret_cast<Vec *>(orow + (t0 + k) * rows * I));
    }
  }
}

// ---- device-side decode advance ----------------------------------------------------
// Row i < n_live takes its sampled token as the next input at position p + 1
// (slot from its block table, seq_len p + 2).  A row whose next position falls
// outside its table stays where it is.  n_live is min(n_rows, *live) when
// `live` is given (a device count a captured graph can change).  One workgroup.
// Uniform in [0, 1) for (seed, step): SplitMix64's output function (Steele,
// Lea, Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014)
// on seed + (step + 1) * golden gamma, top 24 bits.
__device__ __forceinline__ float step_uniform(uint64_t seed, uint32_t step) {
  uint64_t z = seed + (static_cast<uint64_t>(step) + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return static_cast<float>(z >> 40) * (1.f / 16777216.f);
}

__global__ __launch_bounds__(1024) void decode_advance_kernel(
    const int64_t *next, int64_t *input_ids, int64_t *positions, int32_t *seq_lens,
    int64_t *slot_mapping, const int32_t *tables, int64_t ts0, int64_t ts1, int max_blocks,
    int block_size, int n_rows, const int32_t *live, int64_t *history, int32_t *step,
    int hist_cap, const int64_t *rng_seeds, float *uniforms) {
  const int s = step ? *step : 0;
  // the next step's draws (every row: a parked row's value is never used)
  if (uniforms)
    for (int i = threadIdx.x; i < n_rows; i += blockDim.x)
      uniforms[i] = step_uniform(static_cast<uint64_t>(rng_seeds[i]), static_cast<uint32_t>(s + 1));
  const int n_live = live ? min(n_rows, max(0, *live)) : n_rows;
  for (int i = threadIdx.x; i < n_live; i += blockDim.x) {
    const int64_t tok = next[i];
    if (history && s < hist_cap) history[static_cast<int64_t>(i) * hist_cap + s] = tok;
    const int64_t pos = positions[i] + 1;
    const int64_t blk = pos / block_size;
    if (blk >= max_blocks) continue;
    input_ids[i] = tok;
    positions[i] = pos;
    seq_lens[i] = static_cast<int32_t>(pos + 1);
    slot_mapping[i] = static_cast<int64_t>(tables[i * ts0 + blk * ts1]) * block_size + pos % block_size;
  }
  __syncthreads();
  if (step && threadIdx.x == 0) *step = s + 1;
}

}  // namespace spk

using namespace spk;

namespace {
inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
inline bool vec_dtype(int d) { return d == SPK_F32 || d == SPK_F16 || d == SPK_BF16; }
inline int vec_of(int d) { return d == SPK_F32 ? 4 : 8; }
}  // namespace

extern "C" int spk_add_rmsnorm(void *h, const void *delta, const void *weight, void *out,
                               int dtype, int64_t rows, int hidden, float eps, void *stream) {
  if (!vec_dtype(dtype)) return fail(SPK_EINVAL, "add_rmsnorm: dtype %d is not a float type", dtype);
  if (!h || !weight || !out) return fail(SPK_EINVAL, "add_rmsnorm: null pointer");
  if (rows < 0 || hidden <= 0 || hidden % vec_of(dtype))
    return fail(SPK_EINVAL, "add_rmsnorm: hidden=%d must be a positive multiple of %d", hidden,
                vec_of(dtype));
  if (!aligned16(h) || !aligned16(weight) || !aligned16(out) || (delta && !aligned16(delta)))
    return fail(SPK_EINVAL, "add_rmsnorm: buffers must be 16-byte aligned");
  if (rows == 0) return SPK_OK;
  // One wave (one row) per workgroup: the rows spread over 4x the CUs of
  // 4-wave workgroups, and the decode step runs ~20 us faster (47 calls).
  const dim3 grid(static_cast<unsigned>(rows));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool reg = hidden / vec_of(dtype) <= 64 * kNormRegVecs;
  switch (dtype) {
#define SPK_CASE(DT)                                                                          \
  case DT:                                                                                    \
    if (reg && delta)                                                                         \
      add_rmsnorm_reg_kernel<DT, true><<<grid, 64, 0, s>>>(                                   \
          static_cast<Elem<DT>::T *>(h), static_cast<const Elem<DT>::T *>(delta),            \
          static_cast<const Elem<DT>::T *>(weight), static_cast<Elem<DT>::T *>(out), hidden,  \
          eps);                                                                               \
    else if (reg)                                                                             \
      add_rmsnorm_reg_kernel<DT, false><<<grid, 64, 0, s>>>(                                  \
          static_cast<Elem<DT>::T *>(h), nullptr, static_cast<const Elem<DT>::T *>(weight),  \
          static_cast<Elem<DT>::T *>(out), hidden, eps);                                      \
    else                                                                                      \
      add_rmsnorm_kernel<DT><<<grid, 64, 0, s>>>(                                            \
          static_cast<Elem<DT>::T *>(h), static_cast<const Elem<DT>::T *>(delta),            \
          static_cast<const Elem<DT>::T *>(weight), static_cast<Elem<DT>::T *>(out), rows,    \
          hidden, eps);                                                                       \
    break;
    SPK_CASE(SPK_F32) SPK_CASE(SPK_F16) SPK_CASE(SPK_BF16)
#undef SPK_CASE
  }
  return check_launch("add_rmsnorm");
}

extern "C" int spk_embed_rmsnorm(const int64_t *ids, const void *embed, int64_t vocab,
                                 const void *weight, void *h, void *out, int dtype, int T,
                                 int64_t n, int hidden, float eps, void *stream) {
  if (!valid_float_dtype(dtype)) return fail(SPK_EINVAL, "embed_rmsnorm: dtype %d", dtype);
  if (T < 1 || n < 0 || vocab < 1 || hidden <= 0 || hidden % vec_of(dtype))
    return fail(SPK_EINVAL, "embed_rmsnorm: bad shape T=%d n=%lld vocab=%lld hidden=%d", T,
                (long long)n, (long long)vocab, hidden);
  if (n > 0 && (!ids || !embed || !weight || !h || !out))
    return fail(SPK_EINVAL, "embed_rmsnorm: null pointer");
  if (!aligned16(embed) || !aligned16(weight) || !aligned16(h) || !aligned16(out))
    return fail(SPK_EINVAL, "embed_rmsnorm: buffers must be 16-byte aligned");
  if (n == 0) return SPK_OK;
  const dim3 grid(static_cast<unsigned>((n + 3) / 4));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
#define SPK_CASE(DT)                                                                          \
  case DT:                                                                                    \
    embed_rmsnorm_kernel<DT><<<grid, 256, 0, s>>>(                                            \
        ids, static_cast<const Elem<DT>::T *>(embed), vocab,                                  \
        static_cast<const Elem<DT>::T *>(weight), static_cast<Elem<DT>::T *>(h),              \
        static_cast<Elem<DT>::T *>(out), T, n, hidden, eps);                                  \
    break;
    SPK_CASE(SPK_F32) SPK_CASE(SPK_F16) SPK_CASE(SPK_BF16)
#undef SPK_CASE
  }
  return check_launch("embed_rmsnorm");
}

extern "C" int spk_rmsnorm_mean_t(const void *h, const void *delta, const void *weight, void *out,
                                  int dtype, int T, int64_t rows, int hidden, float eps,
                                  void *stream) {
  if (!vec_dtype(dtype)) return fail(SPK_EINVAL, "rmsnorm_mean_t: dtype %d is not a float type", dtype);
  if (!h || !weight || !out) return fail(SPK_EINVAL, "rmsnorm_mean_t: null pointer");
  if (T < 1 || T > kMaxMeanT) return fail(SPK_EUNSUPPORTED, "rmsnorm_mean_t: T=%d outside [1, %d]", T, kMaxMeanT);
  if (rows < 0 || hidden <= 0 || hidden % vec_of(dtype))
    return fail(SPK_EINVAL, "rmsnorm_mean_t: hidden=%d must be a positive multiple of %d", hidden,
                vec_of(dtype));
  if (!aligned16(h) || !aligned16(weight) || !aligned16(out) || (delta && !aligned16(delta)))
    return fail(SPK_EINVAL, "rmsnorm_mean_t: buffers must be 16-byte aligned");
  if (rows == 0) return SPK_OK;
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (hidden / vec_of(dtype) <= 64 * kMeanRegVecs && T <= kMeanRegT) {
    const dim3 g1(static_cast<unsigned>(rows));
    switch (dtype) {
#define SPK_CASE(DT)                                                                          \
  case DT:                                                                                    \
    if (delta)                                                                                \
      rmsnorm_mean_t_reg_kernel<DT, true><<<g1, 64, 0, s>>>(                                  \
          static_cast<const Elem<DT>::T *>(h), static_cast<const Elem<DT>::T *>(delta),       \
          static_cast<const Elem<DT>::T *>(weight), static_cast<Elem<DT>::T *>(out), T, rows, \
          hidden, eps);                                                                       \
    else                                                                                      \
      rmsnorm_mean_t_reg_kernel<DT, false><<<g1, 64, 0, s>>>(                                 \
          static_cast<const Elem<DT>::T *>(h), nullptr,                                       \
          static_cast<const Elem<DT>::T *>(weight), static_cast<Elem<DT>::T *>(out), T, rows, \
          hidden, eps);                                                                       \
    break;
      SPK_CASE(SPK_F32) SPK_CASE(SPK_F16) SPK_CASE(SPK_BF16)
#undef SPK_CASE
    }
    return check_launch("rmsnorm_mean_t");
  }
  switch (dtype) {
#define SPK_CASE(DT)                                                                          \
  case DT:                                                                                    \
    rmsnorm_mean_t_kernel<DT><<<grid, 256, 0, s>>>(                                           \
        static_cast<const Elem<DT>::T *>(h), static_cast<const Elem<DT>::T *>(delta),         \
        static_cast<const Elem<DT>::T *>(weight), static_cast<Elem<DT>::T *>(out), T, rows,   \
        hidden, eps);                                                                         \
    break;
    SPK_CASE(SPK_F32) SPK_CASE(SPK_F16) SPK_CASE(SPK_BF16)
#undef SPK_CASE
  }
  return check_launch("rmsnorm_mean_t");
}

extern "C" int spk_qkv_rope_lif_pack(
    const void *x, int x_dtype, const int64_t x_strides[2], const void *cos, const void *sin,
    const int64_t *positions, int64_t table_rows,
    const void *beta, const void *threshold, int param_dtype, int32_t *q_packed,
    const int64_t q_strides[3], int64_t n_q, int32_t *k_cache, int32_t *v_cache,
    const int64_t cache_strides[3], const int64_t *slot_mapping, int64_t num_slots,
    void *dense_q, void *dense_k, void *dense_v, int T, int64_t n_tok, int Hq, int Hkv, int D,
    void *stream) {
  if (x_dtype != SPK_BF16 && x_dtype != SPK_F16)
    return fail(SPK_EUNSUPPORTED, "qkv_rope_lif_pack: input dtype %d (bf16 or f16 only)", x_dtype);
  if (!valid_float_dtype(param_dtype))
    return fail(SPK_EINVAL, "qkv_rope_lif_pack: parameter dtype %d is not a float type", param_dtype);
  if (D < 64 || D > 512 || (D & (D - 1)))
    return fail(SPK_EUNSUPPORTED, "qkv_rope_lif_pack: head_dim=%d (power of two in [64, 512])", D);
  if (T < 1 || n_tok < 0 || Hq < 1 || Hkv < 1 || n_q < 0 || n_q > n_tok)
    return fail(SPK_EINVAL, "qkv_rope_lif_pack: bad shape T=%d n_tok=%lld Hq=%d Hkv=%d n_q=%lld", T,
                (long long)n_tok, Hq, Hkv, (long long)n_q);
  if (!x || !cos || !sin || !beta || !threshold || !k_cache || !v_cache || !slot_mapping ||
      (n_q > 0 && !q_packed))
    return fail(SPK_EINVAL, "qkv_rope_lif_pack: null pointer");
  if (!aligned16(x) || !aligned16(cos) || !aligned16(sin) || (x_strides[0] % 8) ||
      (x_strides[1] % 8))
    return fail(SPK_EINVAL, "qkv_rope_lif_pack: x/cos/sin must be 16-byte aligned with strides %% 8");
  if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 7 ||
      (cache_strides[0] | cache_strides[1] | cache_strides[2]) & 1)
    return fail(SPK_EINVAL, "qkv_rope_lif_pack: caches must be 8-byte aligned with even strides");
  if (n_q > 0 && ((reinterpret_cast<uintptr_t>(q_packed) & 7) ||
                  ((q_strides[0] | q_strides[1] | q_strides[2]) & 1)))
    return fail(SPK_EINVAL, "qkv_rope_lif_pack: q buffer must be 8-byte aligned with even strides");
  void *dense[3] = {dense_q, dense_k, dense_v};
  for (void *d : dense)
    if (d && !aligned16(d)) return fail(SPK_EINVAL, "qkv_rope_lif_pack: dense outputs must be 16-byte aligned");
  if (positions && table_rows < 1)
    return fail(SPK_EINVAL, "qkv_rope_lif_pack: positions need a table of at least one row");
  if (n_tok == 0) return SPK_OK;
  QkvParams p;
  p.x = x;
  p.xs0 = x_strides[0];
  p.xs1 = x_strides[1];
  p.cos = cos;
  p.sin = sin;
  p.pos = positions;
  p.table_rows = table_rows;
  p.beta = beta;
  p.th = threshold;
  p.param_dtype = param_dtype;
  p.q_packed = reinterpret_cast<uint64_t *>(q_packed);
  p.qs0 = q_strides ? q_strides[0] : 0;
  p.qs1 = q_strides ? q_strides[1] : 0;
  p.qs2 = q_strides ? q_strides[2] : 0;
  p.n_q = n_q;
  p.k_cache = reinterpret_cast<uint64_t *>(k_cache);
  p.v_cache = reinterpret_cast<uint64_t *>(v_cache);
  p.cs0 = cache_strides[0];
  p.cs1 = cache_strides[1];
  p.cs2 = cache_strides[2];
  p.slots = slot_mapping;
  p.num_slots = num_slots;
  for (int i = 0; i < 3; ++i) p.dense[i] = dense[i];
  p.T = T;
  p.n_tok = n_tok;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.D = D;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t rows = n_tok * (Hq + 2 * Hkv);
  if (rows * (D / 8) >= kQkvWideThreads) {  // enough work for 8 channels per lane
    const dim3 grid(static_cast<unsigned>((rows * (D / 8) + 255) / 256));
    if (x_dtype == SPK_BF16)
      qkv_rope_lif_pack_vec_kernel<SPK_BF16><<<grid, 256, 0, s>>>(p);
    else
      qkv_rope_lif_pack_vec_kernel<SPK_F16><<<grid, 256, 0, s>>>(p);
  } else {
    const int64_t threads = rows * (D / 2 < 64 ? D / 2 : 64);
    const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
    if (x_dtype == SPK_BF16)
      qkv_rope_lif_pack_kernel<SPK_BF16><<<grid, 256, 0, s>>>(p);
    else
      qkv_rope_lif_pack_kernel<SPK_F16><<<grid, 256, 0, s>>>(p);
  }
  return check_launch("qkv_rope_lif_pack");
}

extern "C" int spk_lif_gate_mul(const void *x, int dtype, const int64_t x_strides[2],
                                const void *beta, const void *threshold, int param_dtype,
                                void *out, int T, int64_t rows, int I, void *stream) {
  if (!vec_dtype(dtype)) return fail(SPK_EINVAL, "lif_gate_mul: dtype %d is not a float type", dtype);
  if (!valid_float_dtype(param_dtype))
    return fail(SPK_EINVAL, "lif_gate_mul: parameter dtype %d is not a float type", param_dtype);
  if (!x || !beta || !threshold || !out) return fail(SPK_EINVAL, "lif_gate_mul: null pointer");
  const int V = vec_of(dtype);
  if (T < 1 || rows < 0 || I <= 0 || I % V)
    return fail(SPK_EINVAL, "lif_gate_mul: intermediate=%d must be a positive multiple of %d", I, V);
  if (!aligned16(x) || !aligned16(out) || x_strides[0] % V || x_strides[1] % V)
    return fail(SPK_EINVAL, "lif_gate_mul: buffers must be 16-byte aligned, strides %% %d", V);
  if (rows == 0) return SPK_OK;
  const int64_t groups = rows * (I / V);
  const dim3 grid(static_cast<unsigned>((groups + 255) / 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
#define SPK_CASE(DT)                                                                          \
  case DT:                                                                                    \
    lif_gate_mul_kernel<DT><<<grid, 256, 0, s>>>(static_cast<const Elem<DT>::T *>(x),         \
                                                 x_strides[0], x_strides[1], beta, threshold, \
                                                 param_dtype, static_cast<Elem<DT>::T *>(out), \
                                                 T, rows, I);                                 \
    break;
    SPK_CASE(SPK_F32) SPK_CASE(SPK_F16) SPK_CASE(SPK_BF16)
#undef SPK_CASE
  }
  return check_launch("lif_gate_mul");
}

extern "C" int spk_decode_advance(const int64_t *next_tokens, int64_t *input_ids,
                                  int64_t *positions, int32_t *seq_lens, int64_t *slot_mapping,
                                  const int32_t *block_tables, int64_t bt_stride0,
                                  int64_t bt_stride1, int max_blocks, int block_size, int n_rows,
                                  const int32_t *live, int64_t *history, int32_t *step,
                                  int hist_cap, const int64_t *rng_seeds, float *uniforms,
                                  void *stream) {
  if (!next_tokens || !input_ids || !positions || !seq_lens || !slot_mapping || !block_tables)
    return fail(SPK_EINVAL, "decode_advance: null pointer");
  if (uniforms && (!rng_seeds || !step))
    return fail(SPK_EINVAL, "decode_advance: uniforms need rng_seeds and a step counter");
  if (n_rows < 0 || max_blocks < 1 || !is_pow2(block_size))
    return fail(SPK_EINVAL, "decode_advance: bad shape n_rows=%d max_blocks=%d block_size=%d",
                n_rows, max_blocks, block_size);
  if (history && (!step || hist_cap < 1))
    return fail(SPK_EINVAL, "decode_advance: history needs a step counter and hist_cap >= 1");
  if (n_rows == 0) return SPK_OK;
  decode_advance_kernel<<<1, 1024, 0, static_cast<hipStream_t>(stream)>>>(
      next_tokens, input_ids, positions, seq_lens, slot_mapping, block_tables, bt_stride0,
      bt_stride1, max_blocks, block_size, n_rows, live, history, step, hist_cap, rng_seeds,
      uniforms);
  return check_launch("decode_advance");
}
