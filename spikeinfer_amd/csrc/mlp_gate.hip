// Fused MLP gate of the decode step: the gate|up projection of the
// post-attention norm output, the gate LIF over the T timesteps, and the
// spike * up product, in one launch.
//
// Reference semantics (spikeinfer/modeling_fast.py:186-190, lif_triton.py:96-101):
//   gu = x @ W_gu^T                      (bf16 out: fp32 sums, rounded)
//   s_t = LIF_t(gu_gate)                 (per channel, t = 0..T-1)
//   y   = round(s_t * gu_up)             (the product in the model dtype)
// spk_lif_gate_mul applied to the output of a bf16 GEMM computes the same; this
// kernel replaces both launches at decode sizes.
//
// MI355X design.  At decode the GEMM has M = T * n_tok <= 256 rows and is bound
// by moving x and W into the CUs, not by the matrix cores: a CU must read its
// rows of x and its columns of W, at ~90 GB/s of L2 hits per CU.
//   * A workgroup owns 16 tokens (all T timesteps: T * 16 rows of x) and a
//     range of 16-channel pairs (a gate tile and the matching up tile).  The
//     x rows, the whole K, sit in LDS (T * 16 * H * 2 bytes, 115 KB at
//     H = 896), loaded once with global_load_lds into a swizzled layout
//     (16-byte chunk c of row r at chunk c ^ (r % 16): the 16 rows a 16-lane
//     group reads fall on 16 distinct bank groups).
//   * W is repacked once at load in MFMA-fragment order (spk_mlp_gate_pack
//     layout below), so a wave's B operand for one k-step of one tile is one
//     contiguous, fully coalesced 1 KB load, straight into registers.
//   * 8 waves share the workgroup's (pair, K-quarter) units, two units of
//     loads in flight per wave (~224 KB per CU).
//   * v_mfma_f32_16x16x32_bf16: D lane l, acc j = row 4(l/16) + j, column
//     l % 16.  With the x rows of timestep t in row tile t, the T values of one
//     (token, channel) land in one lane: the LIF runs in registers.
//   * K-quarters of a pair computed by different waves are summed in a fixed
//     order through LDS (deterministic).
// Grid: token groups x 64 column ranges; the token groups of one range are
// consecutive on one XCD (block b -> XCD b % 8), so W comes from HBM once.
#include "common.hpp"
#include "lif_math.hpp"
#include "norm_rows.hpp"

namespace spk {
namespace mlp {

typedef __bf16 v8b __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
#define SPK_LDS __attribute__((address_space(3)))

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kTok = 16;       // tokens per workgroup
constexpr int kMaxT = 4;       // timesteps (row tiles) per workgroup
constexpr int kRanges = 64;    // column ranges per token group
constexpr int kMaxPairsPerRange = 8;
constexpr int kLdsBytes = 160 * 1024;
constexpr int kSlotFloats = 2 * kMaxT * 4 * 64;  // one partial: 2 tiles x T row tiles x 4 x 64 lanes
constexpr int kStageOff = 2 * kWaves * kSlotFloats * 4;  // the y staging tiles, after the slots
constexpr int kStageBytes = kMaxT * 16 * 16 * 2;          // one wave's tile
static_assert(kStageOff + kWaves * kStageBytes <= kLdsBytes, "slots and staging fit the LDS");

// Packed W_gu (spk_mlp_gate_pack): for pair p (channels 16p..16p+15), k-step
// ks (K 32ks..32ks+31) and tile g (0 gate, 1 up), 1 KB at ((p*KS + ks)*2 + g)
// KB: lane l's 16 bytes are W[row][32ks + 8(l/16) .. +7], row = 16p + l%16
// (+ I for up).

// T is a template parameter: a runtime test per row tile would put branches
// between the MFMAs (and the accumulator copies they bring cost registers).
// NORM: the x rows are add_rmsnorm(nin.h, nin.delta, nin.w), computed in the
// prologue; the workgroups of the last column range (never empty) write h +
// delta to nin.h_out.
template <int KQ, int T, bool NORM>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void mlp_gate_lif_kernel(
    const uint16_t *x, const v4u *wp, const float *beta_p, const float *th_p, uint16_t *y, int n,
    int I, int MG, NormIn nin) {
  constexpr int KS = 4 * KQ;       // k-steps of 32 (H = 32 KS)
  constexpr int H = 32 * KS;
  constexpr int kChunks = 4 * KS;  // 16-byte chunks per x row
  extern __shared__ __align__(16) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.x, xcd = b & 7, s = b >> 3;
  const int m = s % MG, r = (s / MG) * 8 + xcd;
  const int P = I / 16;
  const int p0 = r * P / kRanges, np = (r + 1) * P / kRanges - p0;
  if (np <= 0) return;  // uniform over the workgroup
  // The LIF parameters of the pair this wave finishes (wave e < np: pair
  // p0 + e), loaded first so their latency hides under the whole K loop.
  const int ch = 16 * (p0 + min(wave, np - 1)) + (lane & 15);
  const float beta = clamp01(beta_p[ch]);
  const float th = th_p[ch];

  // Units (pair, K-quarter): wave w takes [u0, u1), at most 4 of them, over at
  // most two pairs.
  const int U = 4 * np;
  const int u0 = wave * U / kWaves, u1 = (wave + 1) * U / kWaves, nu = u1 - u0;
  // W arrives with nontemporal loads (graph of 24 distinct weights: 15.66
  // -> 15.10 us a launch).
  auto load_unit = [&](int u, v4u (&dst)[KQ][2]) {
    const v4u *src = wp + (static_cast<int64_t>((p0 + u / 4) * KS + (u % 4) * KQ) * 2) * 64 + lane;
#pragma unroll
    for (int ks = 0; ks < KQ; ++ks)
#pragma unroll
      for (int g = 0; g < 2; ++g) dst[ks][g] = __builtin_nontemporal_load(src + (ks * 2 + g) * 64);
  };
  // x rows of the token group into LDS: row rr = 16 t + i holds token 16m + i
  // (clamped to n - 1) at timestep t; chunk c of it at chunk c ^ (rr % 16).
  const int rows = T * kTok;
  if constexpr (NORM) {
    norm_rows<kWaves, T * kTok / kWaves>(
        nin, rows, H, r == kRanges - 1, wave, lane,
        [&](int rr) { return static_cast<int64_t>(rr >> 4) * n + min(m * kTok + (rr & 15), n - 1); },
        [&](int rr) { return m * kTok + (rr & 15) < n; },
        [&](int rr, int v, const NormRowBf16::v8u16 &yv) {
          *reinterpret_cast<NormRowBf16::v8u16 *>(smem + rr * (kChunks * 16) + 16 * (v ^ (rr & 15))) = yv;
        });
  } else {
    const int total = rows * kChunks;  // a multiple of 64
    for (int base = wave * 64; base < total; base += kWaves * 64) {
      const int g = base + lane;
      const int rr = g / kChunks, pc = g - rr * kChunks;
      const int c = pc ^ (rr & 15);
      const int t = rr >> 4, tok = min(m * kTok + (rr & 15), n - 1);
      __builtin_amdgcn_global_load_lds(
          reinterpret_cast<const void *>(x + (static_cast<int64_t>(t) * n + tok) * H + 8 * c),
          (SPK_LDS void *)(smem + base * 16), 16, 0, 0);
    }
  }
  // Then the first two units of W; the wait below lets those stay in flight
  // (vmcnt counts in issue order, so at most their loads outstanding means
  // every x chunk of this wave has landed).
  v4u bA[KQ][2], bB[KQ][2];
  if (nu > 0) load_unit(u0, bA);
  if (nu > 1) load_unit(u0 + 1, bB);
  constexpr int kOne = 2 * KQ;  // loads per unit
  static_assert(2 * kOne <= 63, "vmcnt holds 6 bits");
  if (nu > 1) __builtin_amdgcn_s_waitcnt(0x3f70 | ((2 * kOne) & 15) | (((2 * kOne) >> 4) << 14));
  else if (nu > 0) __builtin_amdgcn_s_waitcnt(0x3f70 | (kOne & 15) | ((kOne >> 4) << 14));
  else __builtin_amdgcn_s_waitcnt(0x3f70);
  __syncthreads();

  const int r16 = lane & 15, kq = lane >> 4;
  v4f accg[kMaxT], accu[kMaxT], saveg[kMaxT], saveu[kMaxT];
#pragma unroll
  for (int t = 0; t < kMaxT; ++t) accg[t] = accu[t] = saveg[t] = saveu[t] = v4f{};
  bool split = false;  // the wave's units span two pairs: the first one's sums are in save*

  auto compute = [&](int u, const v4u (&bq)[KQ][2]) {
#pragma unroll
    for (int ks = 0; ks < KQ; ++ks) {
      const int c = 4 * ((u % 4) * KQ + ks) + kq;
      const v8b bg = __builtin_bit_cast(v8b, bq[ks][0]);
      const v8b bu = __builtin_bit_cast(v8b, bq[ks][1]);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int rr = 16 * t + r16;
        const v8b a = *reinterpret_cast<const v8b *>(smem + rr * (kChunks * 16) + 16 * (c ^ r16));
        accg[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bg, accg[t], 0, 0, 0);
        accu[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bu, accu[t], 0, 0, 0);
      }
    }
  };
  auto next_pair = [&](int u) {  // unit u starts a new pair after the wave's first
    if (u > u0 && (u % 4) == 0) {
#pragma unroll
      for (int t = 0; t < kMaxT; ++t) {
        saveg[t] = accg[t];
        saveu[t] = accu[t];
        accg[t] = accu[t] = v4f{};
      }
      split = true;
    }
  };
  // Units j = 0..3, buffers alternating A, B; unit j + 2 reuses unit j's buffer.
  if (nu > 0) {
    next_pair(u0);
    compute(u0, bA);
    if (nu > 2) load_unit(u0 + 2, bA);
  }
  if (nu > 1) {
    next_pair(u0 + 1);
    compute(u0 + 1, bB);
    if (nu > 3) load_unit(u0 + 3, bB);
  }
  if (nu > 2) {
    next_pair(u0 + 2);
    compute(u0 + 2, bA);
  }
  if (nu > 3) {
    next_pair(u0 + 3);
    compute(u0 + 3, bB);
  }

  // Partials through LDS (the x rows are no longer read): slot 2w + 1 holds
  // the sums of the wave's last pair, slot 2w those of its first when split.
  __syncthreads();
  // A lane's accumulator of (tile g, row tile t) is one 16-byte chunk.
  v4f *slots = reinterpret_cast<v4f *>(smem);
  auto put = [&](int slot, const v4f (&g)[kMaxT], const v4f (&u)[kMaxT]) {
    v4f *d = slots + slot * (kSlotFloats / 4);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      d[(0 * kMaxT + t) * 64 + lane] = g[t];
      d[(1 * kMaxT + t) * 64 + lane] = u[t];
    }
  };
  if (nu > 0) {
    put(2 * wave + 1, accg, accu);
    if (split) put(2 * wave, saveg, saveu);
  }
  __syncthreads();

  // Epilogue: wave e < np finishes pair p0 + e, summing its partials in wave
  // order, then runs the LIF over t and writes y = round(s * up).
  if (wave >= np) return;
  const int pp = wave;
  float sg[kMaxT][4], su[kMaxT][4];
#pragma unroll
  for (int t = 0; t < kMaxT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) sg[t][j] = su[t][j] = 0.f;
  for (int w = 0; w < kWaves; ++w) {
    const int a0 = w * U / kWaves, a1 = (w + 1) * U / kWaves;
    if (a1 <= a0) continue;
    const int pf = a0 / 4, pl = (a1 - 1) / 4;
    int slot = -1;
    if (pf == pp && pf != pl) slot = 2 * w;
    else if (pl == pp) slot = 2 * w + 1;
    if (slot < 0) continue;
    const v4f *d = slots + slot * (kSlotFloats / 4);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const v4f a = d[(0 * kMaxT + t) * 64 + lane], c = d[(1 * kMaxT + t) * 64 + lane];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sg[t][j] += a[j];
        su[t][j] += c[j];
      }
    }
  }
  // The pair's y tile (T x 16 tokens x 16 channels, bf16) is staged in the
  // wave's 2 KB above the partial slots, then each (t, token) row's 32 bytes
  // go out as two 16-byte stores (16 two-byte stores a lane took ~2 us).
  uint16_t *stg = reinterpret_cast<uint16_t *>(smem + kStageOff + wave * kStageBytes);
  const float zth = 0.f * th;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float u = 0.f;
    bool r = 0.f - th > 0.f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float g = round_to<SPK_BF16>(sg[t][j]);
      const float up = round_to<SPK_BF16>(su[t][j]);
      const bool spike = lif_step_r(u, r, g, beta, th, zth);
      stg[(16 * t + 4 * kq + j) * 16 + r16] = f32_to_elem<SPK_BF16>((spike ? 1.f : 0.f) * up);
    }
  }
  wave_lds_sync();  // lanes read rows other lanes wrote
  const int tok = m * kTok + (lane & 15), t = lane >> 4;  // row (t, tok) of the tile
  if (t < T && tok < n) {
    const v4u *src = reinterpret_cast<const v4u *>(stg + lane * 16);
    const v4u lo = src[0], hi = src[1];
    v4u *dst = reinterpret_cast<v4u *>(y + (static_cast<int64_t>(t) * n + tok) * I + 16 * (p0 + pp));
    dst[0] = lo;
    dst[1] = hi;
  }
}

// Packs W_gu [2I, H] (gate rows, then up rows) into the fragment order above.
__global__ __launch_bounds__(256) void mlp_gate_pack_kernel(const uint16_t *w, v4u *out, int I, int H) {
  const int KS = H / 32;
  const int64_t total = static_cast<int64_t>(I / 16) * KS * 2 * 64;
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int l = static_cast<int>(e & 63);
    const int64_t blk = e >> 6;
    const int g = static_cast<int>(blk & 1);
    const int64_t pk = blk >> 1;
    const int ks = static_cast<int>(pk % KS);
    const int p = static_cast<int>(pk / KS);
    const int64_t row = static_cast<int64_t>(g) * I + 16 * p + (l & 15);
    out[e] = *reinterpret_cast<const v4u *>(w + row * H + 32 * ks + 8 * (l >> 4));
  }
}

}  // namespace mlp

static bool mlp_shape_ok(int T, int n_tok, int hidden, int inter) {
  if (T < 1 || T > mlp::kMaxT || n_tok < 1 || hidden % 128 || inter % 16) return false;
  const int KQ = hidden / 128;
  if (KQ < 4 || KQ > 8) return false;
  if (static_cast<int64_t>(T) * mlp::kTok * hidden * 2 > mlp::kLdsBytes) return false;
  const int P = inter / 16;
  return P >= mlp::kRanges && P <= mlp::kRanges * mlp::kMaxPairsPerRange;
}

extern "C" size_t spk_mlp_gate_packed_bytes(int hidden, int inter) {
  return static_cast<size_t>(2) * inter * hidden * 2;
}

extern "C" int spk_mlp_gate_pack(const void *w_gu, int inter, int hidden, int dtype, void *w_packed,
                                 void *stream) {
  if (dtype != SPK_BF16) return fail(SPK_EUNSUPPORTED, "mlp_gate_pack: bf16 weights only");
  if (inter <= 0 || hidden <= 0 || inter % 16 || hidden % 32)
    return fail(SPK_EINVAL, "mlp_gate_pack: inter=%d hidden=%d (need multiples of 16 and 32)", inter, hidden);
  if ((reinterpret_cast<uintptr_t>(w_gu) & 15) || (reinterpret_cast<uintptr_t>(w_packed) & 15))
    return fail(SPK_EINVAL, "mlp_gate_pack: pointers must be 16-byte aligned");
  mlp::mlp_gate_pack_kernel<<<1024, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t *>(w_gu), static_cast<mlp::v4u *>(w_packed), inter, hidden);
  return check_launch("mlp_gate_pack");
}

// Validation shared by both entry points; then the launch, rows from x or
// (nin) normed in the prologue.
static int mlp_gate_launch(const void *x, const NormIn *nin, const void *w_packed, const void *beta,
                           const void *threshold, int param_dtype, void *y, int T, int n_tok, int hidden,
                           int inter, int dtype, void *stream) {
  if (dtype != SPK_BF16) return fail(SPK_EUNSUPPORTED, "mlp_gate_lif: bf16 only");
  if (!valid_float_dtype(param_dtype))
    return fail(SPK_EINVAL, "mlp_gate_lif: parameter dtype %d is not a float type", param_dtype);
  if (param_dtype != SPK_F32)
    return fail(SPK_EUNSUPPORTED, "mlp_gate_lif: LIF parameters must be fp32 (dtype %d given)",
                param_dtype);
  if (!mlp_shape_ok(T, n_tok, hidden, inter))
    return fail(SPK_EUNSUPPORTED, "mlp_gate_lif: T=%d n_tok=%d hidden=%d inter=%d not supported", T,
                n_tok, hidden, inter);
  if ((!nin && (reinterpret_cast<uintptr_t>(x) & 15)) || (reinterpret_cast<uintptr_t>(w_packed) & 15))
    return fail(SPK_EINVAL, "mlp_gate_lif: x and packed weights must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(y) & 15)  // (the tile rows go out as 16-byte stores)
    return fail(SPK_EUNSUPPORTED, "mlp_gate_lif: y must be 16-byte aligned");
  const int MG = (n_tok + mlp::kTok - 1) / mlp::kTok;
  const dim3 grid(MG * mlp::kRanges);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto *xp = static_cast<const uint16_t *>(x);
  const auto *wp = static_cast<const mlp::v4u *>(w_packed);
  auto *yp = static_cast<uint16_t *>(y);
  const NormIn none{};
#define SPK_MLP_LAUNCH1(KQ, TT, NORM)                                                                \
  {                                                                                                \
    static bool attr = false;                                                                      \
    if (!attr) {                                                                                   \
      if (hipFuncSetAttribute(reinterpret_cast<const void *>(mlp::mlp_gate_lif_kernel<KQ, TT, NORM>), \
                              hipFuncAttributeMaxDynamicSharedMemorySize, mlp::kLdsBytes) != hipSuccess) \
        return fail(SPK_EHIP, "mlp_gate_lif: cannot reserve %d bytes of LDS", mlp::kLdsBytes);  \
      attr = true;                                                                                 \
    }                                                                                              \
    mlp::mlp_gate_lif_kernel<KQ, TT, NORM><<<grid, mlp::kThreads, mlp::kLdsBytes, s>>>(             \
        xp, wp, static_cast<const float *>(beta), static_cast<const float *>(threshold), yp, n_tok,  \
        inter, MG, nin ? *nin : none);                                                             \
  }
#define SPK_MLP_LAUNCH(KQ, TT)                                                                       \
  if (nin) SPK_MLP_LAUNCH1(KQ, TT, true) else SPK_MLP_LAUNCH1(KQ, TT, false)
#define SPK_MLP_CASE(KQ)                                                                             \
  case KQ:                                                                                         \
    if (T == 1) SPK_MLP_LAUNCH(KQ, 1)                                                             \
    else if (T == 2) SPK_MLP_LAUNCH(KQ, 2)                                                        \
    else if (T == 3) SPK_MLP_LAUNCH(KQ, 3)                                                        \
    else SPK_MLP_LAUNCH(KQ, 4)                                                                     \
    break;
  switch (hidden / 128) {
    SPK_MLP_CASE(4)
    SPK_MLP_CASE(5)
    SPK_MLP_CASE(6)
    SPK_MLP_CASE(7)
    SPK_MLP_CASE(8)
  }
#undef SPK_MLP_CASE
#undef SPK_MLP_LAUNCH
#undef SPK_MLP_LAUNCH1
  return check_launch("mlp_gate_lif");
}

extern "C" int spk_mlp_gate_lif(const void *x, const void *w_packed, const void *beta,
                                const void *threshold, int param_dtype, void *y, int T, int n_tok,
                                int hidden, int inter, int dtype, void *stream) {
  return mlp_gate_launch(x, nullptr, w_packed, beta, threshold, param_dtype, y, T, n_tok, hidden, inter, dtype,
                         stream);
}

extern "C" int spk_norm_mlp_gate_lif(const void *h, const void *delta, const void *norm_weight, void *h_out,
                                     float eps, const void *w_packed, const void *beta, const void *threshold,
                                     int param_dtype, void *y, int T, int n_tok, int hidden, int inter,
                                     int dtype, void *stream) {
  if (!h || !delta || !norm_weight) return fail(SPK_EINVAL, "norm_mlp_gate_lif: null pointer");
  const auto al = [](const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  if (!al(h) || !al(delta) || !al(norm_weight) || (h_out && !al(h_out)))
    return fail(SPK_EINVAL, "norm_mlp_gate_lif: h, delta, norm weight and h_out must be 16-byte aligned");
  if (h_out && (h_out == h || h_out == delta))
    return fail(SPK_EINVAL, "norm_mlp_gate_lif: h_out must not alias h or delta");
  if (hidden > 1024) return fail(SPK_EUNSUPPORTED, "norm_mlp_gate_lif: hidden=%d (at most 1024)", hidden);
  NormIn nin{static_cast<const uint16_t *>(h), static_cast<const uint16_t *>(delta),
             static_cast<const uint16_t *>(norm_weight), static_cast<uint16_t *>(h_out), eps};
  return mlp_gate_launch(nullptr, &nin, w_packed, beta, threshold, param_dtype, y, T, n_tok, hidden, inter,
                         dtype, stream);
}

}  // namespace spk
