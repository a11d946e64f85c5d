// LIF neuron, bit-packing and the fused LIF -> pack -> paged-cache scatter.
//
// Reference semantics: spikeinfer/kernels/lif_triton.py:13-28, 96-105 (the
// recurrence, evaluated in fp32 with separate multiply and add roundings:
// `enable_fp_fusion=False` at :222-227) and spikeinfer/kernels/packing.py:16-23
// (bit i of int32 word w is channel 32*w + i).
//
// This file is compiled with -ffp-contract=off: `beta*u + x` must round twice,
// exactly as PyTorch eager does, or a membrane that lands within an ulp of the
// threshold flips its spike.
#include "common.hpp"
#include "lif_math.hpp"

namespace spk {

struct LifParams {
  const void *x;
  int x_dtype;
  const void *beta;
  const void *th;
  int param_dtype;
  int T;
};


// ---- dense LIF: [T, M, N] -> spikes [T, M, N] -----------------------------
__global__ __launch_bounds__(256) void lif_dense_kernel(LifParams p, int64_t xs0, int64_t xs1,
                                                        int64_t xs2, const float *mem0,
                                                        void *spikes, int spike_dtype,
                                                        float *u_out, int64_t M, int N) {
  const int64_t total = M * N;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = e / N;
    const int c = static_cast<int>(e - m * N);
    const float beta = clamp01(load_as_f32(p.beta, c, p.param_dtype));
    const float th = load_as_f32(p.th, c, p.param_dtype);
    float u = mem0 ? mem0[e] : 0.f;
    const int64_t xoff = m * xs1 + c * xs2;
    for (int t = 0; t < p.T; ++t) {
      const bool s = lif_step(u, load_as_f32(p.x, t * xs0 + xoff, p.x_dtype), beta, th);
      store_spike(spikes, t * total + e, spike_dtype, s);
    }
    if (u_out) u_out[e] = u;
  }
}

// ---- fused LIF + pack + scatter --------------------------------------------
// One wave per (token, head) row; lane = channel (CPL chunks of 64 channels).
// Per timestep the wave's 64 spikes become one 64-bit word by __ballot, and
// lanes 0..W-1 store the int32 words straight to the packed buffer or to the
// cache slot the token maps to.
template <int CPL>
__global__ __launch_bounds__(256) void lif_pack_kernel(LifParams p, int64_t xs0, int64_t xs1,
                                                       int64_t xs2, int64_t xs3, uint32_t *packed,
                                                       int64_t ps0, int64_t ps1, int64_t ps2,
                                                       const int64_t *slots, int64_t num_slots,
                                                       void *spikes, int spike_dtype,
                                                       int64_t n_tok, int H, int D) {
  const int lane = threadIdx.x & 63;
  const int W = (D + 31) >> 5;
  const int64_t rows = n_tok * H;
  const int64_t waves_total = (int64_t)gridDim.x * (blockDim.x >> 6);
  float beta[CPL], th[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + 64 * c;
    beta[c] = ch < D ? clamp01(load_as_f32(p.beta, ch, p.param_dtype)) : 0.f;
    th[c] = ch < D ? load_as_f32(p.th, ch, p.param_dtype) : 1.f;
  }
  for (int64_t row = blockIdx.x * (int64_t)(blockDim.x >> 6) + (threadIdx.x >> 6); row < rows;
       row += waves_total) {
    const int64_t tok = row / H;
    const int h = static_cast<int>(row - tok * H);
    int64_t dst = 0;
    bool write = true;
    if (slots) {
      const int64_t slot = slots[tok];
      write = slot >= 0 && slot < num_slots;
      dst = h * ps1 + slot * ps2;
    } else {
      dst = tok * ps1 + h * ps2;
    }
    float u[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) u[c] = 0.f;
    for (int t = 0; t < p.T; ++t) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ch = lane + 64 * c;
        bool s = false;
        if (ch < D) {
          const float cur = load_as_f32(p.x, t * xs0 + tok * xs1 + h * xs2 + ch * xs3, p.x_dtype);
          s = lif_step(u[c], cur, beta[c], th[c]);
          if (spikes)
            store_spike(spikes, ((t * n_tok + tok) * H + h) * (int64_t)D + ch, spike_dtype, s);
        }
        const uint64_t mask = __ballot(s);
        // Lanes 0 and 1 store the two int32 words of this 64-channel chunk.
        const int w = 2 * c + lane;
        if (write && lane < 2 && w < W)
          packed[t * ps0 + dst + w] = static_cast<uint32_t>(mask >> (32 * lane));
      }
    }
  }
}


// ---- vectorised paths: 16 bytes per lane ---------------------------------
constexpr int kTBatch = 4;  // timesteps whose loads are issued together
// Dense LIF over rows of N contiguous channels (N % kVec == 0, 16-byte aligned
// rows): each thread owns kVec consecutive channels of one row, loads and
// stores 16 bytes per timestep.  Spikes are written in the input's dtype.
template <int DT>
__global__ __launch_bounds__(256) void lif_dense_vec_kernel(LifParams p, int64_t xs0, int64_t xs1,
                                                            const float *mem0, void *spikes,
                                                            float *u_out, int64_t M, int N) {
  typedef typename Elem<DT>::T E;
  constexpr int V = Elem<DT>::kVec;
  typedef E Vec __attribute__((ext_vector_type(V)));
  const int64_t groups = M * (N / V);
  const int64_t total = M * N;
  for (int64_t gi = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; gi < groups;
       gi += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = gi / (N / V);
    const int c0 = static_cast<int>(gi - m * (N / V)) * V;
    float beta[V], th[V], zth[V], u[V];
    bool r[V];
    load_params(p.beta, p.param_dtype, c0, beta);
    load_params(p.th, p.param_dtype, c0, th);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      beta[i] = clamp01(beta[i]);
      u[i] = mem0 ? mem0[m * N + c0 + i] : 0.f;
      zth[i] = 0.f * th[i];
      r[i] = u[i] - th[i] > 0.f;
    }
    const E *xrow = static_cast<const E *>(p.x) + m * xs1 + c0;
    E *srow = static_cast<E *>(spikes) + m * N + c0;
    for (int t0 = 0; t0 < p.T; t0 += kTBatch) {
      // All loads of up to kTBatch timesteps in flight before the recurrence.
      Vec xv[kTBatch];
#pragma unroll
      for (int k = 0; k < kTBatch; ++k)
        if (t0 + k < p.T)
          xv[k] = __builtin_nontemporal_load(reinterpret_cast<const Vec *>(xrow + (t0 + k) * xs0));
#pragma unroll
      for (int k = 0; k < kTBatch; ++k) {
        if (t0 + k >= p.T) break;
        Vec sv;
#pragma unroll
        for (int i = 0; i < V; ++i)
          sv[i] = spike_elem<DT>(lif_step_r(u[i], r[i], elem_to_f32<DT>(xv[k][i]), beta[i], th[i], zth[i]));
        __builtin_nontemporal_store(sv, reinterpret_cast<Vec *>(srow + (t0 + k) * total));
      }
    }
    if (u_out) {
#pragma unroll
      for (int i = 0; i < V; ++i) u_out[m * N + c0 + i] = u[i];
    }
  }
}

// ---- pack / unpack ---------------------------------------------------------
// One wave per row; each 64-channel chunk is one __ballot.
__global__ __launch_bounds__(256) void pack_kernel(const void *x, int x_dtype, int64_t row_stride,
                                                   uint32_t *out, int64_t rows, int C) {
  const int lane = threadIdx.x & 63;
  const int W = (C + 31) >> 5;
  const int64_t waves_total = (int64_t)gridDim.x * (blockDim.x >> 6);
  for (int64_t row = blockIdx.x * (int64_t)(blockDim.x >> 6) + (threadIdx.x >> 6); row < rows;
       row += waves_total) {
    for (int c0 = 0; c0 < C; c0 += 64) {
      const int ch = c0 + lane;
      const bool s = ch < C && load_nonzero(x, row * row_stride + ch, x_dtype);
      const uint64_t mask = __ballot(s);
      const int w = (c0 >> 5) + lane;
      if (lane < 2 && w < W) out[row * W + w] = static_cast<uint32_t>(mask >> (32 * lane));
    }
  }
}

__global__ __launch_bounds__(256) void unpack_kernel(const uint32_t *words, int64_t rows, int C,
                                                     void *out, int out_dtype) {
  const int W = (C + 31) >> 5;
  const int64_t total = rows * C;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / C;
    const int c = static_cast<int>(e - r * C);
    const bool s = (words[r * W + (c >> 5)] >> (c & 31)) & 1u;
    store_spike(out, e, out_dtype, s);
  }
}

// Vector forms for rows of whole 64-channel chunks (C % 64 == 0) with
// 16-byte aligned rows: each lane moves 16 bytes (PER = 16 / element size
// elements), G = 64 / PER lanes cover one chunk, i.e. one uint64 of packed
// words (int32 words 2c, 2c+1 of the row, little-endian).  Same bit tests as
// load_nonzero / the same values as store_spike.
template <int DT>
struct PackVec {
  static constexpr int kEsz = DT == SPK_U8 ? 1 : (DT == SPK_F16 || DT == SPK_BF16) ? 2 : 4;
  static constexpr int kPer = 16 / kEsz;  // elements per lane
  static constexpr int kG = 64 / kPer;    // lanes per 64-channel chunk
  // Bit i set where element i of the lane's 16 bytes is nonzero.
  __device__ static uint32_t bits(const uint4 &v) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t b = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (kEsz == 4) {
        const uint32_t m = DT == SPK_F32 ? 0x7fffffffu : 0xffffffffu;
        b |= ((w[j] & m) != 0u ? 1u : 0u) << j;
      } else if constexpr (kEsz == 2) {
        b |= ((w[j] & 0x7fffu) != 0u ? 1u : 0u) << (2 * j);
        b |= ((w[j] & 0x7fff0000u) != 0u ? 1u : 0u) << (2 * j + 1);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) b |= ((w[j] >> (8 * k)) & 0xffu ? 1u : 0u) << (4 * j + k);
      }
    }
    return b;
  }
  // 16 bytes of 0/1 elements from kPer bits.
  __device__ static uint4 spikes(uint32_t b) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (kEsz == 4) {
        w[j] = (b >> j) & 1u ? (DT == SPK_F32 ? 0x3f800000u : 1u) : 0u;
      } else if constexpr (kEsz == 2) {
        constexpr uint32_t one = DT == SPK_F16 ? 0x3c00u : 0x3f80u;
        w[j] = ((b >> (2 * j)) & 1u ? one : 0u) | ((b >> (2 * j + 1)) & 1u ? one << 16 : 0u);
      } else {
        uint32_t x = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) x |= ((b >> (4 * j + k)) & 1u) << (8 * k);
        w[j] = x;
      }
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};

// The loop runs per wave (every lane takes part in the shuffles); lanes past
// the last chunk load nothing and store nothing.
template <int DT>
__global__ __launch_bounds__(256) void pack_vec_kernel(const char *x, int64_t row_stride_bytes,
                                                       uint64_t *out, int64_t rows, int C) {
  using P = PackVec<DT>;
  const int lane = threadIdx.x & 63, sub = lane % P::kG;
  const int64_t cpr = C >> 6, total = rows * cpr;
  constexpr int kPerWave = 64 / P::kG;
  const int64_t step = (int64_t)gridDim.x * (blockDim.x >> 6) * kPerWave;
  for (int64_t base = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * kPerWave;
       base < total; base += step) {
    const int64_t ci = base + lane / P::kG;
    const bool valid = ci < total;
    const int64_t row = valid ? ci / cpr : 0;
    const int64_t ch = valid ? ci - row * cpr : 0;
    uint32_t b = 0;
    if (valid) {
      typedef unsigned int v4u __attribute__((ext_vector_type(4)));
      const v4u v = __builtin_nontemporal_load(
          reinterpret_cast<const v4u *>(x + row * row_stride_bytes + (ch * 64 + sub * P::kPer) * P::kEsz));
      b = P::bits(make_uint4(v.x, v.y, v.z, v.w));
    }
    // Bit offset of this lane in the chunk's word; kPer divides 32, so a
    // lane's bits never straddle the two halves.
    const int sh = sub * P::kPer;
    uint32_t lo = sh < 32 ? b << sh : 0u;
    uint32_t hi = sh < 32 ? 0u : b << (sh - 32);
#pragma unroll
    for (int off = 1; off < P::kG; off <<= 1) {
      lo |= __shfl_xor(lo, off);
      hi |= __shfl_xor(hi, off);
    }
    if (valid && sub == 0) out[ci] = (static_cast<uint64_t>(hi) << 32) | lo;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void unpack_vec_kernel(const uint64_t *words, int64_t rows, int C,
                                                         char *out) {
  using P = PackVec<DT>;
  const int64_t total_lanes = rows * (C >> 6) * P::kG;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total_lanes;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t ci = i / P::kG;  // chunk (row-major over rows x C/64)
    const int sub = static_cast<int>(i - ci * P::kG);
    const uint64_t w = words[ci];
    const uint32_t b = static_cast<uint32_t>(w >> (sub * P::kPer)) & ((1u << P::kPer) - 1u);
    reinterpret_cast<uint4 *>(out)[i] = P::spikes(b);
  }
}

inline unsigned grid_for(int64_t items, int per_block) {
  int64_t g = (items + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;  // grid-stride loops cover the rest
  return static_cast<unsigned>(g);
}

// ---- several LIF-pack sites in one launch -----------------------------------
// The 64-channel groups of all sites are numbered one after the other, each
// site starting at a multiple of 8 groups (one wave's worth), so the site is
// uniform over a wave and its fields stay in scalar registers.  An 8-lane group
// then packs its 64 channels for every timestep (8 per lane).
constexpr int kMaxSites = 4;
static_assert(sizeof(SpkLifSite) == 120, "SpkLifSite layout (the Python binding packs it field by field)");
constexpr int kGroupsPerWave = 8;
struct MultiSites {
  SpkLifSite s[kMaxSites];
  int64_t gstart[kMaxSites + 1];  // first group of each site (multiples of 8), then the end
  int64_t gcount[kMaxSites];      // groups of each site
  int nsites;
  int T;
  const int64_t *slots;
};

// OR of v over the 8 lanes of each aligned lane octet (DPP: swap neighbours,
// swap pairs, then mirror within the half row -- each step pairs lanes of the
// octet that hold disjoint partial results).
__device__ __forceinline__ uint32_t or_octet(uint32_t v) {
  v |= static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xB1, 0xF, 0xF, false));
  v |= static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4E, 0xF, 0xF, false));
  v |= static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x141, 0xF, 0xF, false));
  return v;
}

// The x loads of a group are issued before its parameter and slot loads (they
// do not depend on them), so a wave waits for one memory round trip, not two.
template <int DT>
__global__ __launch_bounds__(256) void lif_pack_sites_kernel(MultiSites m) {
  typedef typename Elem<DT>::T E;
  typedef E Vec __attribute__((ext_vector_type(8)));
  const int lane = threadIdx.x & 63;
  const int sub = lane & 7;
  const int64_t groups = m.gstart[m.nsites];
  const int64_t gstride = (int64_t)gridDim.x * (blockDim.x >> 3);  // a multiple of 8
  for (int64_t gw = blockIdx.x * (int64_t)(blockDim.x >> 3) + (threadIdx.x >> 6) * kGroupsPerWave;
       gw < groups; gw += gstride) {
    int si = 0;
#pragma unroll
    for (int k = 1; k < kMaxSites; ++k) si += (k < m.nsites && gw >= m.gstart[k]) ? 1 : 0;
    si = __builtin_amdgcn_readfirstlane(si);  // wave-uniform: the wave's groups share a site
    const SpkLifSite &st = m.s[si];
    const int64_t li = gw - m.gstart[si] + (lane >> 3);
    if (li >= m.gcount[si]) continue;  // the padding after a site (whole octets)
    const int gpr = st.D >> 6;
    const int64_t row = li / gpr;
    const int grp = static_cast<int>(li - row * gpr);
    const int64_t tok = row / st.H;
    const int h = static_cast<int>(row - tok * st.H);
    const int c0 = grp * 64 + sub * 8;
    const E *xrow = static_cast<const E *>(st.x) + tok * st.x_strides[1] + h * st.x_strides[2] + c0;
    const int64_t xs0 = st.x_strides[0];
    // Unconditional loads (timesteps past T re-read the last one): a branch
    // per load would make the compiler wait for each before the next.
    Vec xv[kTBatch];
#pragma unroll
    for (int k = 0; k < kTBatch; ++k)
      xv[k] = __builtin_nontemporal_load(reinterpret_cast<const Vec *>(xrow + min(k, m.T - 1) * xs0));
    float beta[8], th[8], zth[8], u[8];
    bool r[8];
    load_params(st.beta, st.param_dtype, c0, beta);
    load_params(st.threshold, st.param_dtype, c0, th);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      beta[i] = clamp01(beta[i]);
      u[i] = 0.f;
      zth[i] = 0.f * th[i];
      r[i] = 0.f - th[i] > 0.f;
    }
    bool write = true;
    int64_t dst;
    if (st.scatter) {
      const int64_t slot = m.slots[tok];
      write = slot >= 0 && slot < st.num_slots;
      dst = h * st.out_strides[1] + slot * st.out_strides[2];
    } else {
      dst = tok * st.out_strides[1] + h * st.out_strides[2];
    }
    uint64_t *out = reinterpret_cast<uint64_t *>(st.out) + dst / 2 + grp;
    const int64_t os0 = st.out_strides[0] / 2;
    for (int t0 = 0; t0 < m.T; t0 += kTBatch) {
      if (t0 > 0) {
#pragma unroll
        for (int k = 0; k < kTBatch; ++k)
          xv[k] = __builtin_nontemporal_load(reinterpret_cast<const Vec *>(xrow + min(t0 + k, m.T - 1) * xs0));
      }
#pragma unroll
      for (int k = 0; k < kTBatch; ++k) {
        if (t0 + k >= m.T) break;
        const Vec x = xv[k];
        uint32_t byte = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          byte |= lif_step_r(u[i], r[i], elem_to_f32<DT>(x[i]), beta[i], th[i], zth[i]) ? (1u << i) : 0u;
        const uint32_t lo = or_octet(sub < 4 ? byte << (8 * sub) : 0u);
        const uint32_t hi = or_octet(sub < 4 ? 0u : byte << (8 * (sub - 4)));
        if (write && sub == 0) out[(t0 + k) * os0] = (static_cast<uint64_t>(hi) << 32) | lo;
      }
    }
  }
}

}  // namespace spk

using namespace spk;

extern "C" int spk_lif_multistep(const void *x, int x_dtype, const int64_t x_strides[3],
                                 const void *beta, const void *threshold, int param_dtype,
                                 const float *mem0, void *spikes, int spike_dtype, float *u_out,
                                 int T, int64_t M, int N, void *stream) {
  if (T <= 0 || M < 0 || N <= 0) return fail(SPK_EINVAL, "bad sizes T=%d M=%lld N=%d", T, (long long)M, N);
  if (!valid_float_dtype(x_dtype) || !valid_float_dtype(param_dtype) || !valid_any_dtype(spike_dtype))
    return fail(SPK_EINVAL, "unsupported dtype (x %d, params %d, spikes %d)", x_dtype, param_dtype, spike_dtype);
  if (M == 0) return SPK_OK;
  LifParams p{x, x_dtype, beta, threshold, param_dtype, T};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int vec = x_dtype == SPK_F32 ? 4 : 8;
  const int esz = x_dtype == SPK_F32 ? 4 : 2;
  const bool vec_ok = spike_dtype == x_dtype && x_strides[2] == 1 && N % vec == 0 &&
                      (x_strides[0] * esz) % 16 == 0 && (x_strides[1] * esz) % 16 == 0 &&
                      (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(spikes) & 15) == 0;
  if (vec_ok) {
    const unsigned grid = grid_for(M * (N / vec), 256);
    if (x_dtype == SPK_BF16)
      lif_dense_vec_kernel<SPK_BF16><<<grid, 256, 0, s>>>(p, x_strides[0], x_strides[1], mem0, spikes, u_out, M, N);
    else if (x_dtype == SPK_F16)
      lif_dense_vec_kernel<SPK_F16><<<grid, 256, 0, s>>>(p, x_strides[0], x_strides[1], mem0, spikes, u_out, M, N);
    else
      lif_dense_vec_kernel<SPK_F32><<<grid, 256, 0, s>>>(p, x_strides[0], x_strides[1], mem0, spikes, u_out, M, N);
  } else {
    lif_dense_kernel<<<grid_for(M * N, 256), 256, 0, s>>>(
        p, x_strides[0], x_strides[1], x_strides[2], mem0, spikes, spike_dtype, u_out, M, N);
  }
  return check_launch("lif_multistep");
}

extern "C" int spk_lif_pack_write(const void *x, int x_dtype, const int64_t x_strides[4],
                                  const void *beta, const void *threshold, int param_dtype,
                                  int32_t *packed, const int64_t packed_strides[3],
                                  const int64_t *slot_mapping, int64_t num_slots, void *spikes,
                                  int spike_dtype, int T, int64_t n_tok, int H, int D,
                                  void *stream) {
  if (T <= 0 || n_tok < 0 || H <= 0 || D <= 0)
    return fail(SPK_EINVAL, "bad sizes T=%d n_tok=%lld H=%d D=%d", T, (long long)n_tok, H, D);
  if (D > 128) return fail(SPK_EUNSUPPORTED, "fused LIF-pack supports D <= 128, got %d", D);
  if (!valid_float_dtype(x_dtype) || !valid_float_dtype(param_dtype) ||
      (spikes && !valid_any_dtype(spike_dtype)))
    return fail(SPK_EINVAL, "unsupported dtype (x %d, params %d, spikes %d)", x_dtype, param_dtype, spike_dtype);
  if (n_tok == 0) return SPK_OK;
  LifParams p{x, x_dtype, beta, threshold, param_dtype, T};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(n_tok * H, 4);
  uint32_t *pk = reinterpret_cast<uint32_t *>(packed);
  const bool vec_ok = !spikes && (x_dtype == SPK_BF16 || x_dtype == SPK_F16) && D % 64 == 0 &&
                      x_strides[3] == 1 && (x_strides[0] % 8) == 0 && (x_strides[1] % 8) == 0 &&
                      (x_strides[2] % 8) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                      (packed_strides[0] % 2) == 0 && (packed_strides[1] % 2) == 0 &&
                      (packed_strides[2] % 2) == 0 && (reinterpret_cast<uintptr_t>(packed) & 7) == 0;
  if (vec_ok) {  // the one-site form of the several-sites kernel
    SpkLifSite site{};
    site.x = x;
    for (int i = 0; i < 4; ++i) site.x_strides[i] = x_strides[i];
    site.beta = beta;
    site.threshold = threshold;
    site.param_dtype = param_dtype;
    site.scatter = slot_mapping != nullptr;
    site.out = packed;
    for (int i = 0; i < 3; ++i) site.out_strides[i] = packed_strides[i];
    site.num_slots = num_slots;
    site.n_tok = n_tok;
    site.H = H;
    site.D = D;
    return spk_lif_pack_write_sites(&site, 1, x_dtype, T, slot_mapping, stream);
  } else if (D <= 64)
    lif_pack_kernel<1><<<grid, 256, 0, s>>>(p, x_strides[0], x_strides[1], x_strides[2], x_strides[3], pk,
                                            packed_strides[0], packed_strides[1], packed_strides[2],
                                            slot_mapping, num_slots, spikes, spike_dtype, n_tok, H, D);
  else
    lif_pack_kernel<2><<<grid, 256, 0, s>>>(p, x_strides[0], x_strides[1], x_strides[2], x_strides[3], pk,
                                            packed_strides[0], packed_strides[1], packed_strides[2],
                                            slot_mapping, num_slots, spikes, spike_dtype, n_tok, H, D);
  return check_launch("lif_pack_write");
}

extern "C" int spk_lif_pack_write_sites(const SpkLifSite *sites, int nsites, int x_dtype, int T,
                                        const int64_t *slot_mapping, void *stream) {
  if (!sites || nsites < 1 || nsites > kMaxSites)
    return fail(SPK_EINVAL, "nsites must be 1..%d, got %d", kMaxSites, nsites);
  if (T <= 0) return fail(SPK_EINVAL, "bad T=%d", T);
  if (!valid_float_dtype(x_dtype)) return fail(SPK_EINVAL, "unsupported x dtype %d", x_dtype);
  MultiSites m{};
  m.nsites = nsites;
  m.T = T;
  m.slots = slot_mapping;
  bool vec_ok = x_dtype == SPK_BF16 || x_dtype == SPK_F16;
  int64_t g = 0;
  for (int i = 0; i < nsites; ++i) {
    const SpkLifSite &s = sites[i];
    if (s.n_tok < 0 || s.H <= 0 || s.D <= 0)
      return fail(SPK_EINVAL, "site %d: bad sizes n_tok=%lld H=%d D=%d", i, (long long)s.n_tok, s.H, s.D);
    if (s.D > 128) return fail(SPK_EUNSUPPORTED, "fused LIF-pack supports D <= 128, got %d", s.D);
    if (!valid_float_dtype(s.param_dtype)) return fail(SPK_EINVAL, "site %d: param dtype %d", i, s.param_dtype);
    if (s.scatter && !slot_mapping) return fail(SPK_EINVAL, "site %d scatters but slot_mapping is NULL", i);
    vec_ok = vec_ok && s.D % 64 == 0 && s.x_strides[3] == 1 && (s.x_strides[0] % 8) == 0 &&
             (s.x_strides[1] % 8) == 0 && (s.x_strides[2] % 8) == 0 &&
             (reinterpret_cast<uintptr_t>(s.x) & 15) == 0 && (s.out_strides[0] % 2) == 0 &&
             (s.out_strides[1] % 2) == 0 && (s.out_strides[2] % 2) == 0 &&
             (reinterpret_cast<uintptr_t>(s.out) & 7) == 0;
    m.s[i] = s;
    m.gstart[i] = g;
    m.gcount[i] = s.n_tok * s.H * (s.D / 64);
    g += (m.gcount[i] + kGroupsPerWave - 1) / kGroupsPerWave * kGroupsPerWave;
  }
  m.gstart[nsites] = g;
  if (!vec_ok) {  // the general kernels, one launch per site
    for (int i = 0; i < nsites; ++i) {
      const SpkLifSite &s = sites[i];
      const int rc = spk_lif_pack_write(s.x, x_dtype, s.x_strides, s.beta, s.threshold, s.param_dtype,
                                        s.out, s.out_strides, s.scatter ? slot_mapping : nullptr,
                                        s.num_slots, nullptr, 0, T, s.n_tok, s.H, s.D, stream);
      if (rc != SPK_OK) return rc;
    }
    return SPK_OK;
  }
  if (g == 0) return SPK_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(g, 32);
  if (x_dtype == SPK_BF16) lif_pack_sites_kernel<SPK_BF16><<<grid, 256, 0, st>>>(m);
  else lif_pack_sites_kernel<SPK_F16><<<grid, 256, 0, st>>>(m);
  return check_launch("lif_pack_write_sites");
}

extern "C" int spk_pack(const void *x, int x_dtype, int64_t x_row_stride, int32_t *out, int64_t rows,
                        int C, void *stream) {
  if (rows < 0 || C <= 0) return fail(SPK_EINVAL, "bad sizes rows=%lld C=%d", (long long)rows, C);
  if (!valid_any_dtype(x_dtype)) return fail(SPK_EINVAL, "unsupported dtype %d", x_dtype);
  if (rows == 0) return SPK_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int esz = x_dtype == SPK_U8 ? 1 : (x_dtype == SPK_F16 || x_dtype == SPK_BF16) ? 2 : 4;
  if (C % 64 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && ((x_row_stride * esz) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(out) & 7) == 0) {
    const int64_t chunks = rows * (C / 64);
    const int per_block = 4 * (64 / (64 * esz / 16));  // chunks per 4-wave block
    const unsigned grid = grid_for(chunks, per_block);
    const char *xb = static_cast<const char *>(x);
    uint64_t *o = reinterpret_cast<uint64_t *>(out);
    const int64_t rs = x_row_stride * esz;
    switch (x_dtype) {
      case SPK_F32: pack_vec_kernel<SPK_F32><<<grid, 256, 0, s>>>(xb, rs, o, rows, C); break;
      case SPK_F16: pack_vec_kernel<SPK_F16><<<grid, 256, 0, s>>>(xb, rs, o, rows, C); break;
      case SPK_BF16: pack_vec_kernel<SPK_BF16><<<grid, 256, 0, s>>>(xb, rs, o, rows, C); break;
      case SPK_U8: pack_vec_kernel<SPK_U8><<<grid, 256, 0, s>>>(xb, rs, o, rows, C); break;
      default: pack_vec_kernel<SPK_I32><<<grid, 256, 0, s>>>(xb, rs, o, rows, C); break;
    }
    return check_launch("pack");
  }
  pack_kernel<<<grid_for(rows, 4), 256, 0, s>>>(
      x, x_dtype, x_row_stride, reinterpret_cast<uint32_t *>(out), rows, C);
  return check_launch("pack");
}

extern "C" int spk_unpack(const int32_t *words, int64_t rows, int C, void *out, int out_dtype,
                          void *stream) {
  if (rows < 0 || C <= 0) return fail(SPK_EINVAL, "bad sizes rows=%lld C=%d", (long long)rows, C);
  if (!valid_any_dtype(out_dtype)) return fail(SPK_EINVAL, "unsupported dtype %d", out_dtype);
  if (rows == 0) return SPK_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int esz = out_dtype == SPK_U8 ? 1 : (out_dtype == SPK_F16 || out_dtype == SPK_BF16) ? 2 : 4;
  if (C % 64 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(words) & 7) == 0) {
    const int64_t lanes = rows * (C / 64) * (4 * esz);  // 16 output bytes per lane
    const unsigned grid = grid_for(lanes, 256);
    const uint64_t *w = reinterpret_cast<const uint64_t *>(words);
    char *o = static_cast<char *>(out);
    switch (out_dtype) {
      case SPK_F32: unpack_vec_kernel<SPK_F32><<<grid, 256, 0, s>>>(w, rows, C, o); break;
      case SPK_F16: unpack_vec_kernel<SPK_F16><<<grid, 256, 0, s>>>(w, rows, C, o); break;
      case SPK_BF16: unpack_vec_kernel<SPK_BF16><<<grid, 256, 0, s>>>(w, rows, C, o); break;
      case SPK_U8: unpack_vec_kernel<SPK_U8><<<grid, 256, 0, s>>>(w, rows, C, o); break;
      default: unpack_vec_kernel<SPK_I32><<<grid, 256, 0, s>>>(w, rows, C, o); break;
    }
    return check_launch("unpack");
  }
  unpack_kernel<<<grid_for(rows * C, 256), 256, 0, s>>>(
      reinterpret_cast<const uint32_t *>(words), rows, C, out, out_dtype);
  return check_launch("unpack");
}
