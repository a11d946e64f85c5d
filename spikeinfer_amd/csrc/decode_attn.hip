// Paged popcount decode attention for gfx950.
//
// Reference semantics: spikeinfer/kernels/spike_attention.py:67-150 (Triton
// kernel) and :247-282 (SDPA oracle).  For every (sequence n, query head h,
// timestep t) the output is softmax_j(popc(q & k_j) * scale) @ bits(v_j) over
// the sequence's first seq_len positions, walked through its block table.
//
// MI355X design (this file: the general path, every head_dim <= 128 and GQA
// ratio <= 16):
//   * one workgroup per (partition of the context, t, kv head, sequence);
//     it serves all n_rep query heads of the kv head, so each K/V byte is read
//     from HBM once, not n_rep times;
//   * scores are integers, so the softmax uses the fixed offset c_q =
//     popc(q) (an upper bound of every count): weight(d) = exp(-d*scale) with
//     d = popc(q & ~k) = c_q - count in [0, head_dim].  No running max, no
//     rescaling, and partition partial sums combine by plain addition;
//   * the 1 + head_dim weights live in an LDS table, so a score costs two
//     bitwise ops and two v_bcnt per word plus one LDS read;
//   * value side: lane = channel, v bit selects the weight, fixed summation
//     order (bit-reproducible run to run).
#include "decode_attn.hpp"

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace spk {

template <int W>
__device__ __forceinline__ int popc_andn(const uint32_t (&q)[W], const uint32_t (&k)[W]) {
  int d = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) d += __popc(q[w] & ~k[w]);
  return d;
}

template <int W, int REP>
__global__ __launch_bounds__(kAttnThreads) void decode_attn_general(AttnParams p) {
  constexpr int CPL = (W + 1) / 2;  // channels per lane (64 lanes)
  // x = (sequence, timestep, kv head) unit, y = partition: consecutive block
  // ids (dealt round-robin to the 8 XCDs) are sibling units of similar
  // length, and every unit's first partition is launched before any tail.
  const int part = blockIdx.y;
  const int kvh = blockIdx.x % p.Hkv;
  const int t = (blockIdx.x / p.Hkv) % p.T;
  const int n = blockIdx.x / (p.Hkv * p.T);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const int len = seq_len(p, n);
  const int nparts_seq = len <= 0 ? 1 : (len + p.part_len - 1) / p.part_len;
  if (part >= nparts_seq) return;
  const int start = part * p.part_len;
  const int end = min(len, start + p.part_len);

  __shared__ float wtab[129];
  __shared__ float P[REP][kAttnThreads];
  __shared__ uint32_t Vs[kAttnThreads][W];
  __shared__ float red_l[4][REP];
  __shared__ float red_acc[4][REP][CPL * 64];

  const int hd = p.head_dim;
  for (int d = tid; d <= hd; d += kAttnThreads) wtab[d] = expf(-static_cast<float>(d) * p.scale);

  // Query words of the n_rep heads sharing this kv head (uniform per block).
  uint32_t qw[REP][W];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
#pragma unroll
    for (int w = 0; w < W; ++w) {
      qw[h][w] = 0;
      if (h < p.nrep)
        qw[h][w] = p.q[t * p.qs0 + n * p.qs1 + (kvh * p.nrep + h) * p.qs2 + w];
    }
  }

  float acc[REP][CPL];
  float lsum[REP];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    lsum[h] = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) acc[h][c] = 0.f;
  }

  const uint32_t *kbase = p.k + t * p.ks0 + kvh * p.ks1;
  const uint32_t *vbase = p.v + t * p.vs0 + kvh * p.vs1;
  const int bs_mask = (1 << p.bs_log2) - 1;
  __syncthreads();

  for (int c0 = start; c0 < end; c0 += kAttnThreads) {
    // Phase 1: one token per thread -> n_rep weights and the v words in LDS.
    const int j = c0 + tid;
    uint32_t kw[W], vw[W];
#pragma unroll
    for (int w = 0; w < W; ++w) kw[w] = vw[w] = 0;
    bool valid = j < end;
    if (valid) {
      const int phys = p.bt[n * p.bts0 + (j >> p.bs_log2) * p.bts1];
      const int64_t slot = (static_cast<int64_t>(phys) << p.bs_log2) | (j & bs_mask);
      valid = slot >= 0 && slot < p.num_slots;
      if (valid) {
#pragma unroll
        for (int w = 0; w < W; ++w) {
          kw[w] = kbase[slot * p.ks2 + w];
          vw[w] = vbase[slot * p.vs2 + w];
        }
      }
    }
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      const float pv = valid ? wtab[popc_andn<W>(qw[h], kw)] : 0.f;
      P[h][tid] = pv;
      lsum[h] += pv;
    }
#pragma unroll
    for (int w = 0; w < W; ++w) Vs[tid][w] = valid ? vw[w] : 0u;
    __syncthreads();

    // Phase 2: each wave owns 64 of the chunk's tokens; lane = channel.
    const int i0 = wave * 64;
    const int i1 = min(i0 + 64, end - c0);
    for (int i = i0; i < i1; ++i) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ch = lane + 64 * c;
        const uint32_t word = (ch >> 5) < W ? Vs[i][(ch >> 5) < W ? (ch >> 5) : 0] : 0u;
        const bool bit = (word >> (ch & 31)) & 1u;
#pragma unroll
        for (int h = 0; h < REP; ++h) acc[h][c] += bit ? P[h][i] : 0.f;
      }
    }
    __syncthreads();
  }

  // Reduce the four waves' partial sums in a fixed order.
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    float l = lsum[h];
    for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
    if (lane == 0) red_l[wave][h] = l;
#pragma unroll
    for (int c = 0; c < CPL; ++c) red_acc[wave][h][lane + 64 * c] = acc[h][c];
  }
  __syncthreads();

  const bool single = nparts_seq == 1 && !p.partials_only;
  for (int idx = tid; idx < p.nrep * hd; idx += kAttnThreads) {
    const int h = idx / hd;
    const int ch = idx % hd;
    const float a = ((red_acc[0][h][ch] + red_acc[1][h][ch]) + red_acc[2][h][ch]) + red_acc[3][h][ch];
    const float l = ((red_l[0][h] + red_l[1][h]) + red_l[2][h]) + red_l[3][h];
    const int hq = kvh * p.nrep + h;
    if (single) {
      const float o = len <= 0 ? 0.f : a / l;
      store_f32_as(p.out, t * p.os0 + n * p.os1 + hq * p.os2 + ch * p.os3, p.out_dtype, o);
    } else {
      float *dst = p.ws + ((((int64_t)part * p.T + t) * p.N + n) * p.Hq + hq) * (hd + 1);
      dst[ch] = a;
      if (ch == 0) dst[hd] = l;
    }
  }
}

// Sums the partitions of every split sequence (fixed order) and normalises:
// one thread per output element (t, n, hq, channel), so the few split rows of
// a batch fill the GPU without one workgroup per row.
__global__ __launch_bounds__(256) void decode_attn_combine(AttnParams p) {
  const int hd = p.head_dim;
  const int64_t total = (int64_t)p.T * p.N * p.Hq * hd;
  const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int ch = static_cast<int>(e % hd);
  const int64_t row = e / hd;  // (t, n, hq)
  const int hq = static_cast<int>(row % p.Hq);
  const int n = static_cast<int>((row / p.Hq) % p.N);
  const int t = static_cast<int>(row / ((int64_t)p.Hq * p.N));
  const int len = seq_len(p, n);
  const int nparts = len <= 0 ? 1 : (len + p.part_len - 1) / p.part_len;
  if (nparts <= 1 && !p.partials_only) return;  // the attention kernel wrote it
  const int64_t stride_part = (int64_t)p.T * p.N * p.Hq * (hd + 1);
  const float *src = p.ws + row * (hd + 1);
  float a = 0.f, l = 0.f;
  for (int q = 0; q < min(nparts, p.num_parts); ++q) {
    a += src[q * stride_part + ch];
    l += src[q * stride_part + hd];
  }
  store_f32_as(p.out, t * p.os0 + n * p.os1 + hq * p.os2 + ch * p.os3, p.out_dtype,
               len <= 0 ? 0.f : a / l);
}

// Integer scores popc(q & k) for every valid position (score-path check).
template <int W>
__global__ __launch_bounds__(256) void decode_scores_kernel(AttnParams p, int32_t *scores,
                                                            int max_len) {
  const int t = blockIdx.y / p.Hkv;
  const int kvh = blockIdx.y % p.Hkv;
  const int n = blockIdx.z;
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  const int len = seq_len(p, n);
  if (j >= len || j >= max_len) return;
  const int phys = p.bt[n * p.bts0 + (j >> p.bs_log2) * p.bts1];
  const int64_t slot = (static_cast<int64_t>(phys) << p.bs_log2) | (j & ((1 << p.bs_log2) - 1));
  if (slot < 0 || slot >= p.num_slots) return;
  uint32_t kw[W];
  for (int w = 0; w < W; ++w) kw[w] = p.k[t * p.ks0 + kvh * p.ks1 + slot * p.ks2 + w];
  for (int h = 0; h < p.nrep; ++h) {
    const int hq = kvh * p.nrep + h;
    int c = 0;
    for (int w = 0; w < W; ++w) c += __popc(p.q[t * p.qs0 + n * p.qs1 + hq * p.qs2 + w] & kw[w]);
    scores[(((int64_t)t * p.N + n) * p.Hq + hq) * max_len + j] = c;
  }
}

// Launch of the general path; REP is the smallest instantiated bound >= nrep.
template <int W>
static void launch_general(const AttnParams &p, dim3 grid, hipStream_t s) {
  if (p.nrep <= 1) decode_attn_general<W, 1><<<grid, kAttnThreads, 0, s>>>(p);
  else if (p.nrep <= 2) decode_attn_general<W, 2><<<grid, kAttnThreads, 0, s>>>(p);
  else if (p.nrep <= 4) decode_attn_general<W, 4><<<grid, kAttnThreads, 0, s>>>(p);
  else if (p.nrep <= 8) decode_attn_general<W, 8><<<grid, kAttnThreads, 0, s>>>(p);
  else decode_attn_general<W, 16><<<grid, kAttnThreads, 0, s>>>(p);
}

}  // namespace spk

using namespace spk;

static int check_common(int T, int N, int Hq, int Hkv, int head_dim, int block_size) {
  if (T <= 0 || N < 0 || Hq <= 0 || Hkv <= 0)
    return fail(SPK_EINVAL, "bad sizes T=%d N=%d Hq=%d Hkv=%d", T, N, Hq, Hkv);
  if (Hq % Hkv != 0) return fail(SPK_EINVAL, "Hq=%d is not a multiple of Hkv=%d", Hq, Hkv);
  if (Hq / Hkv > kMaxRep)
    return fail(SPK_EUNSUPPORTED, "GQA ratio %d exceeds %d", Hq / Hkv, kMaxRep);
  if (head_dim <= 0 || head_dim > 128)
    return fail(SPK_EUNSUPPORTED, "head_dim=%d (supported: 1..128)", head_dim);
  if (!is_pow2(block_size))
    return fail(SPK_EINVAL, "block_size=%d is not a power of two", block_size);
  return SPK_OK;
}

extern "C" size_t spk_decode_attn_workspace_bytes(int T, int N, int Hq, int Hkv, int head_dim,
                                                  int block_size, int max_blocks) {
  if (T <= 0 || N <= 0 || Hkv <= 0 || max_blocks <= 0 || block_size <= 0) return 0;
  const int64_t ctx_max = (int64_t)max_blocks * block_size;
  const int part = choose_part_len(block_size);
  const int64_t nparts = (ctx_max + part - 1) / part;
  // Partial sums of split contexts, then the launch order of long contexts.
  const size_t partials = nparts <= 1 ? 0 : (size_t)nparts * T * N * Hq * (head_dim + 1) * sizeof(float);
  const int64_t items = nparts * N;
  const size_t order = plan_in_workspace(ctx_max, items) ? ((size_t)items * T * Hkv + 1) * sizeof(int32_t) : 0;
  return partials + order;
}

// Shared by spk_decode_attn and spk_qkv_decode_attn: validation, parameters,
// path choice and launches.  fz != nullptr selects the fused q/k/v path
// (matrix-core kernel only; its x dtype in fused_dtype).
static int decode_attn_impl(const int32_t *q, const int64_t q_strides[4], const int32_t *k_cache,
                            const int64_t k_strides[4], const int32_t *v_cache,
                            const int64_t v_strides[4], int64_t num_slots,
                            const int32_t *block_tables, int64_t bt_stride0, int64_t bt_stride1,
                            const int32_t *seq_lens, void *out, int out_dtype,
                            const int64_t out_strides[4], int T, int N, int Hq, int Hkv,
                            int head_dim, int block_size, int max_blocks, float scale,
                            void *workspace, size_t workspace_bytes, void *stream,
                            const FusedParams *fz, int fused_dtype, int forced_part_len = 0,
                            float *partials = nullptr, size_t partials_bytes = 0) {
  int rc = check_common(T, N, Hq, Hkv, head_dim, block_size);
  if (rc) return rc;
  if (!partials && !valid_float_dtype(out_dtype))
    return fail(SPK_EINVAL, "out dtype %d not a float type", out_dtype);
  if ((!fz && q_strides[3] != 1) || k_strides[3] != 1 || v_strides[3] != 1)
    return fail(SPK_EINVAL, "packed word axis must be contiguous");
  if (!(scale > 0.f) || scale * head_dim > 80.f)
    return fail(SPK_EINVAL, "scale=%g outside (0, 80/head_dim]", (double)scale);
  if (max_blocks <= 0) return fail(SPK_EINVAL, "max_blocks=%d", max_blocks);
  const int64_t ctx_max = (int64_t)max_blocks * block_size;
  if (partials) {
    if (forced_part_len < block_size || forced_part_len % block_size || forced_part_len > 32768)
      return fail(SPK_EINVAL, "part_len=%d must be a multiple of block_size=%d in [%d, 32768]",
                  forced_part_len, block_size, block_size);
    const size_t need_p = (size_t)((ctx_max + forced_part_len - 1) / forced_part_len) * T * N * Hq *
                          (head_dim + 1) * sizeof(float);
    if (partials_bytes < need_p)
      return fail(SPK_EINVAL, "partials buffer of %zu bytes, need %zu", partials_bytes, need_p);
  }
  if (N == 0) return SPK_OK;
  const size_t need = partials ? 0 : spk_decode_attn_workspace_bytes(T, N, Hq, Hkv, head_dim, block_size, max_blocks);
  if ((int64_t)N * T * Hkv * ((ctx_max + 32767) / 32768 + 1) >= (int64_t(1) << 30))
    return fail(SPK_EUNSUPPORTED, "decode_attn: %d sequences x %d units is too many work items", N, T * Hkv);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(SPK_EINVAL, "workspace of %zu bytes, need %zu", workspace_bytes, need);

  AttnParams p{};
  if (!fz) {
    p.q = reinterpret_cast<const uint32_t *>(q);
    p.qs0 = q_strides[0]; p.qs1 = q_strides[1]; p.qs2 = q_strides[2];
  }
  p.k = reinterpret_cast<const uint32_t *>(k_cache);
  p.ks0 = k_strides[0]; p.ks1 = k_strides[1]; p.ks2 = k_strides[2];
  p.v = reinterpret_cast<const uint32_t *>(v_cache);
  p.vs0 = v_strides[0]; p.vs1 = v_strides[1]; p.vs2 = v_strides[2];
  p.num_slots = num_slots;
  p.bt = block_tables; p.bts0 = bt_stride0; p.bts1 = bt_stride1;
  p.lens = seq_lens;
  p.out = out; p.out_dtype = out_dtype;
  p.os0 = out_strides[0]; p.os1 = out_strides[1]; p.os2 = out_strides[2]; p.os3 = out_strides[3];
  p.out_vec = out && (out_dtype == SPK_F32 || out_dtype == SPK_BF16 || out_dtype == SPK_F16) &&
              p.os3 == 1 && p.os0 % 4 == 0 && p.os1 % 4 == 0 && p.os2 % 4 == 0 &&
              (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  p.T = T; p.N = N; p.Hq = Hq; p.Hkv = Hkv; p.head_dim = head_dim;
  p.bs_log2 = ilog2(block_size); p.nrep = Hq / Hkv; p.scale = scale;
  p.ctx_cap = (int)std::min<int64_t>(ctx_max, INT32_MAX);
  p.part_len = partials ? forced_part_len : choose_part_len(block_size);
  p.num_parts = (int)((ctx_max + p.part_len - 1) / p.part_len);
  p.ws = partials ? partials : static_cast<float *>(workspace);
  p.partials_only = partials != nullptr;
  if (p.ws == nullptr && need > 0) return fail(SPK_EINVAL, "workspace required");
  if (fz) p.fz = *fz;

  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(N * T * Hkv, p.num_parts);
  const int W = (head_dim + 31) / 32;
  const char *path = getenv("SPIKEINFER_AMD_ATTN_PATH");
  const bool force_general = !fz && path && strcmp(path, "general") == 0;
  if (!force_general && mfma_path_supported(p)) {
    build_digit_table(scale, p.digits);
    const size_t partial_floats = p.num_parts > 1 ? (size_t)p.num_parts * T * N * Hq * (head_dim + 1) : 0;
    // The partials entry orders its items only when the kernel can do it
    // itself (it has no workspace for a planner's list).
    const bool plan = plan_launch(ctx_max) &&
                      (!partials || (int64_t)p.num_parts * N <= kInlinePlanItems);
    int32_t *order = !partials && plan_in_workspace(ctx_max, (int64_t)p.num_parts * N)
                         ? reinterpret_cast<int32_t *>(p.ws + partial_floats) : nullptr;
    // Unplanned launches of short contexts (ctx_max below the planning
    // threshold, so every item is short): the 2-wave launch, two waves per
    // unit.  Otherwise 4-wave workgroups; a planned launch runs the items of
    // at most kPairMaxLen tokens two units at a time in the same per-unit
    // order (pair mode), which measured faster than the 2-wave launch at
    // fixed 8k (-1.4 %) and ragged contexts up to 8k (-6 %).
    const int waves = !fz && head_dim == 64 && !plan && ctx_max <= kPairMaxLen ? 2 : 4;
    launch_decode_mfma(p, plan, order, s, fz ? fused_dtype : 0, waves);
  } else if (fz) {
    return fail(SPK_EUNSUPPORTED, "qkv_decode_attn: needs head_dim 64, Hq/Hkv <= 8, aligned caches");
  } else switch (W) {
    case 1: launch_general<1>(p, grid, s); break;
    case 2: launch_general<2>(p, grid, s); break;
    case 3: launch_general<3>(p, grid, s); break;
    default: launch_general<4>(p, grid, s); break;
  }
  if ((rc = check_launch("decode_attn"))) return rc;
  if (p.num_parts > 1 && !partials) {
    const int64_t elems = (int64_t)T * N * Hq * head_dim;
    decode_attn_combine<<<static_cast<unsigned>((elems + 255) / 256), 256, 0, s>>>(p);
    if ((rc = check_launch("decode_attn_combine"))) return rc;
  }
  return SPK_OK;
}

extern "C" int spk_decode_attn(const int32_t *q, const int64_t q_strides[4], const int32_t *k_cache,
                               const int64_t k_strides[4], const int32_t *v_cache,
                               const int64_t v_strides[4], int64_t num_slots,
                               const int32_t *block_tables, int64_t bt_stride0, int64_t bt_stride1,
                               const int32_t *seq_lens, void *out, int out_dtype,
                               const int64_t out_strides[4], int T, int N, int Hq, int Hkv,
                               int head_dim, int block_size, int max_blocks, float scale,
                               void *workspace, size_t workspace_bytes, void *stream) {
  return decode_attn_impl(q, q_strides, k_cache, k_strides, v_cache, v_strides, num_slots,
                          block_tables, bt_stride0, bt_stride1, seq_lens, out, out_dtype,
                          out_strides, T, N, Hq, Hkv, head_dim, block_size, max_blocks, scale,
                          workspace, workspace_bytes, stream, nullptr, 0);
}

// ---- the allocation-free variant of spk_decode_attn ---------------------
// The partial sums and the launch-order list live in this file-scope device
// array instead of a caller workspace.  Each GPU the library runs on holds its
// own copy (kNoAllocScratchBytes, until the process ends).  Host code never
// passes `scratch` itself to a kernel: its name in host code is a stand-in,
// not a device address; the device address comes from hipGetSymbolAddress,
// looked up once per device with that device current.
constexpr size_t kNoAllocScratchBytes = SPK_DECODE_ATTN_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static int scratch_on_current_device(void **out) {
  constexpr int kMaxDevices = 64;
  static void *ptrs[kMaxDevices] = {};
  static std::mutex mu;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SPK_EHIP, "decode_attn_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(SPK_EUNSUPPORTED, "decode_attn_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(SPK_EHIP, "decode_attn_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
    ptrs[dev] = ptr;
  }
  *out = ptrs[dev];
  return SPK_OK;
}

extern "C" int spk_decode_attn_noalloc(const int32_t *q, const int64_t q_strides[4],
                                       const int32_t *k_cache, const int64_t k_strides[4],
                                       const int32_t *v_cache, const int64_t v_strides[4],
                                       int64_t num_slots, const int32_t *block_tables,
                                       int64_t bt_stride0, int64_t bt_stride1,
                                       const int32_t *seq_lens, void *out, int out_dtype,
                                       const int64_t out_strides[4], int T, int N, int Hq,
                                       int Hkv, int head_dim, int block_size, int max_blocks,
                                       float scale, void *stream) {
  const size_t need = spk_decode_attn_workspace_bytes(T, N, Hq, Hkv, head_dim, block_size, max_blocks);
  if (need > kNoAllocScratchBytes)
    return fail(SPK_EINVAL,
                "decode_attn_noalloc: this shape needs %zu bytes of scratch, more than the "
                "library's fixed %zu (use spk_decode_attn with a workspace)",
                need, kNoAllocScratchBytes);
  void *ws = nullptr;
  if (need > 0) {
    const int rc = scratch_on_current_device(&ws);
    if (rc) return rc;
  }
  // Nothing in the scratch needs clearing: every partial the combine reads
  // and every entry of the launch order is written by this call first.
  return decode_attn_impl(q, q_strides, k_cache, k_strides, v_cache, v_strides, num_slots,
                          block_tables, bt_stride0, bt_stride1, seq_lens, out, out_dtype,
                          out_strides, T, N, Hq, Hkv, head_dim, block_size, max_blocks, scale,
                          ws, need, stream, nullptr, 0);
}

extern "C" int spk_decode_attn_partials(const int32_t *q, const int64_t q_strides[4],
                                        const int32_t *k_cache, const int64_t k_strides[4],
                                        const int32_t *v_cache, const int64_t v_strides[4],
                                        int64_t num_slots, const int32_t *block_tables,
                                        int64_t bt_stride0, int64_t bt_stride1,
                                        const int32_t *seq_lens, int T, int N, int Hq, int Hkv,
                                        int head_dim, int block_size, int max_blocks, float scale,
                                        int part_len, float *partials, size_t partials_bytes,
                                        void *stream) {
  if (!partials) return fail(SPK_EINVAL, "decode_attn_partials: null partials buffer");
  const int64_t ostr[4] = {0, 0, 0, 0};
  return decode_attn_impl(q, q_strides, k_cache, k_strides, v_cache, v_strides, num_slots,
                          block_tables, bt_stride0, bt_stride1, seq_lens, nullptr, SPK_F32, ostr,
                          T, N, Hq, Hkv, head_dim, block_size, max_blocks, scale, nullptr, 0,
                          stream, nullptr, 0, part_len, partials, partials_bytes);
}

extern "C" int spk_decode_attn_combine(const float *partials, size_t partials_bytes, int num_parts,
                                       int part_len, const int32_t *seq_lens, void *out, int out_dtype,
                                       const int64_t out_strides[4], int T, int N, int Hq,
                                       int head_dim, void *stream) {
  if (T <= 0 || N < 0 || Hq <= 0 || head_dim <= 0 || num_parts <= 0 || part_len <= 0)
    return fail(SPK_EINVAL, "decode_attn_combine: bad sizes T=%d N=%d Hq=%d D=%d parts=%d part_len=%d",
                T, N, Hq, head_dim, num_parts, part_len);
  if (!valid_float_dtype(out_dtype)) return fail(SPK_EINVAL, "out dtype %d not a float type", out_dtype);
  if (N == 0) return SPK_OK;
  if (!partials || !seq_lens || !out) return fail(SPK_EINVAL, "decode_attn_combine: null pointer");
  const size_t need = (size_t)num_parts * T * N * Hq * (head_dim + 1) * sizeof(float);
  if (partials_bytes < need)
    return fail(SPK_EINVAL, "decode_attn_combine: partials buffer has %zu bytes, %d partitions need %zu",
                partials_bytes, num_parts, need);
  AttnParams p{};
  p.lens = seq_lens;
  // Partitions past num_parts do not exist in the buffer: lengths beyond
  // num_parts * part_len are clamped to it.
  p.ctx_cap = (int)std::min<int64_t>((int64_t)num_parts * part_len, INT32_MAX);
  p.out = out; p.out_dtype = out_dtype;
  p.os0 = out_strides[0]; p.os1 = out_strides[1]; p.os2 = out_strides[2]; p.os3 = out_strides[3];
  p.T = T; p.N = N; p.Hq = Hq; p.head_dim = head_dim;
  p.part_len = part_len; p.num_parts = num_parts;
  p.ws = const_cast<float *>(partials);
  p.partials_only = 1;
  const int64_t elems = (int64_t)T * N * Hq * head_dim;
  decode_attn_combine<<<static_cast<unsigned>((elems + 255) / 256), 256, 0,
                        static_cast<hipStream_t>(stream)>>>(p);
  return check_launch("decode_attn_combine");
}

extern "C" int spk_qkv_decode_attn(const void *x, int x_dtype, const int64_t x_strides[2],
                                   const void *cos, const void *sin, const int64_t *positions,
                                   int64_t table_rows, const void *beta, const void *threshold,
                                   int param_dtype, const int64_t *slot_mapping, int32_t *k_cache,
                                   int32_t *v_cache, const int64_t cache_strides[4],
                                   int64_t num_slots, const int32_t *block_tables,
                                   int64_t bt_stride0, int64_t bt_stride1, const int32_t *seq_lens,
                                   void *out, int out_dtype, const int64_t out_strides[4], int T,
                                   int N, int Hq, int Hkv, int head_dim, int block_size,
                                   int max_blocks, float scale, void *workspace,
                                   size_t workspace_bytes, void *stream) {
  if (x_dtype != SPK_BF16 && x_dtype != SPK_F16)
    return fail(SPK_EUNSUPPORTED, "qkv_decode_attn: input dtype %d (bf16 or f16 only)", x_dtype);
  if (!valid_float_dtype(param_dtype))
    return fail(SPK_EINVAL, "qkv_decode_attn: parameter dtype %d is not a float type", param_dtype);
  if (param_dtype != SPK_F32)
    return fail(SPK_EUNSUPPORTED, "qkv_decode_attn: LIF parameters must be fp32 (dtype %d given)",
                param_dtype);
  if (T < 1 || T > kMaxFusedT)
    return fail(SPK_EUNSUPPORTED, "qkv_decode_attn: T=%d (1..%d)", T, kMaxFusedT);
  if (head_dim != 64)
    return fail(SPK_EUNSUPPORTED, "qkv_decode_attn: head_dim=%d (64 only)", head_dim);
  if (N > 0 && (!x || !cos || !sin || !positions || !beta || !threshold || !slot_mapping ||
                !k_cache || !v_cache || table_rows < 1))
    return fail(SPK_EINVAL, "qkv_decode_attn: null pointer or empty rotary table");
  if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 7 ||
      (cache_strides[0] | cache_strides[1] | cache_strides[2]) & 1)
    return fail(SPK_EINVAL, "qkv_decode_attn: caches must be 8-byte aligned with even strides");
  FusedParams fz{};
  fz.x = x;
  fz.xs0 = x_strides[0];
  fz.xs1 = x_strides[1];
  fz.cos = cos;
  fz.sin = sin;
  fz.pos = positions;
  fz.table_rows = table_rows;
  fz.beta = beta;
  fz.th = threshold;
  fz.param_dtype = param_dtype;
  fz.slots = slot_mapping;
  fz.k_out = reinterpret_cast<uint32_t *>(k_cache);
  fz.v_out = reinterpret_cast<uint32_t *>(v_cache);
  return decode_attn_impl(nullptr, nullptr, k_cache, cache_strides, v_cache, cache_strides,
                          num_slots, block_tables, bt_stride0, bt_stride1, seq_lens, out,
                          out_dtype, out_strides, T, N, Hq, Hkv, head_dim, block_size, max_blocks,
                          scale, workspace, workspace_bytes, stream, &fz, x_dtype);
}

extern "C" int spk_decode_scores(const int32_t *q, const int64_t q_strides[4],
                                 const int32_t *k_cache, const int64_t k_strides[4],
                                 int64_t num_slots, const int32_t *block_tables,
                                 int64_t bt_stride0, int64_t bt_stride1, const int32_t *seq_lens,
                                 int32_t *scores, int max_len, int T, int N, int Hq, int Hkv,
                                 int head_dim, int block_size, void *stream) {
  int rc = check_common(T, N, Hq, Hkv, head_dim, block_size);
  if (rc) return rc;
  if (q_strides[3] != 1 || k_strides[3] != 1) return fail(SPK_EINVAL, "packed word axis must be contiguous");
  if (max_len <= 0 || N == 0) return SPK_OK;
  AttnParams p{};
  p.q = reinterpret_cast<const uint32_t *>(q);
  p.qs0 = q_strides[0]; p.qs1 = q_strides[1]; p.qs2 = q_strides[2];
  p.k = reinterpret_cast<const uint32_t *>(k_cache);
  p.ks0 = k_strides[0]; p.ks1 = k_strides[1]; p.ks2 = k_strides[2];
  p.num_slots = num_slots;
  p.bt = block_tables; p.bts0 = bt_stride0; p.bts1 = bt_stride1;
  p.lens = seq_lens;
  p.T = T; p.N = N; p.Hq = Hq; p.Hkv = Hkv; p.head_dim = head_dim;
  p.bs_log2 = ilog2(block_size); p.nrep = Hq / Hkv;
  p.ctx_cap = max_len;  // positions past max_len have no score slot
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid((max_len + 255) / 256, T * Hkv, N);
  switch ((head_dim + 31) / 32) {
    case 1: decode_scores_kernel<1><<<grid, 256, 0, s>>>(p, scores, max_len); break;
    case 2: decode_scores_kernel<2><<<grid, 256, 0, s>>>(p, scores, max_len); break;
    case 3: decode_scores_kernel<3><<<grid, 256, 0, s>>>(p, scores, max_len); break;
    default: decode_scores_kernel<4><<<grid, 256, 0, s>>>(p, scores, max_len); break;
  }
  return check_launch("decode_scores");
}
