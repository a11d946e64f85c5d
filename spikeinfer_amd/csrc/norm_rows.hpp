// Residual add + RMSNorm of whole rows by one wave each, shared by the
// add_rmsnorm kernel and the decode GEMMs that start from a normed input
// (their prologue: the rows they multiply are computed here instead of being
// read from a separate add_rmsnorm launch).
#pragma once

#include "common.hpp"
#include "lif_math.hpp"

namespace spk {

// Sum over the wave, the same value in every lane: DPP adds within each row of
// 16 lanes (pairs, quads, half rows, rows), then the four row sums by readlane.
__device__ __forceinline__ float wave_sum(float v) {
  auto dpp = [](float x, int ctrl) -> float {
    switch (ctrl) {  // the control must be a constant: one instantiation each
      case 0xB1: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
      case 0x4E: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
      case 0x141: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));
      default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));
    }
  };
  v += dpp(v, 0xB1);   // quad_perm [1,0,3,2]
  v += dpp(v, 0x4E);   // quad_perm [2,3,0,1]
  v += dpp(v, 0x141);  // row_half_mirror
  v += dpp(v, 0x140);  // row_mirror
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// One bf16 row of Qwen2RMSNorm after a residual add, in add_rmsnorm's
// arithmetic (so the values are identical to it): lane l holds the row's
// 16-byte vectors l and l + 64, xs = round(h + delta), r = rsqrt(sum(xs^2) /
// hidden + eps) with the lane sums over its vectors in order and wave_sum
// across lanes, y = round(w * round(xs * r)).  Rows of at most 1024 values.
// Loads of several rows are issued before any is reduced: load() then finish().
struct NormRowBf16 {
  typedef unsigned short v8u16 __attribute__((ext_vector_type(8)));
  v8u16 xs[2], ds[2];
  __device__ __forceinline__ void load(const uint16_t *h, const uint16_t *delta, int nv, int lane) {
    const v8u16 *hr = reinterpret_cast<const v8u16 *>(h);
    const v8u16 *dr = reinterpret_cast<const v8u16 *>(delta);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int v = min(lane + 64 * k, nv - 1);
      xs[k] = hr[v];
      ds[k] = dr[v];
    }
  }
  // put(v, y) gets output vector v (v < nv); h_out (if non-null) the sums.
  template <typename Put>
  __device__ __forceinline__ void finish(const v8u16 (&ws)[2], int nv, int hidden, float eps, int lane,
                                         uint16_t *h_out, Put &&put) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int v = lane + 64 * k;
      const bool mine = v < nv;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        xs[k][i] = f32_to_elem<SPK_BF16>(elem_to_f32<SPK_BF16>(xs[k][i]) + elem_to_f32<SPK_BF16>(ds[k][i]));
      if (h_out && mine) reinterpret_cast<v8u16 *>(h_out)[v] = xs[k];
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float f = elem_to_f32<SPK_BF16>(xs[k][i]);
        part += f * f;
      }
      ss += mine ? part : 0.f;
    }
    const float r = rsqrtf(wave_sum(ss) * (1.f / static_cast<float>(hidden)) + eps);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int v = lane + 64 * k;
      if (v >= nv) continue;
      v8u16 y;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float n = round_to<SPK_BF16>(elem_to_f32<SPK_BF16>(xs[k][i]) * r);
        y[i] = f32_to_elem<SPK_BF16>(elem_to_f32<SPK_BF16>(ws[k][i]) * n);
      }
      put(v, y);
    }
  }
};

// Inputs of a GEMM whose rows are add_rmsnorm(h, delta, w) (bf16): h_out, when
// set, receives h + delta (the caller lets one workgroup per row group write).
struct NormIn {
  const uint16_t *h, *delta, *w;
  uint16_t *h_out;
  float eps;
};

// The wave's rows rr = wave, wave + NW, ... (< rows, at most kMaxRows of them)
// of a normed input, each written by put(rr, v, y); row rr reads global row
// grow(rr) and writes h_out there only when own(rr).
template <int NW, int kMaxRows, typename Grow, typename Own, typename Put>
__device__ __forceinline__ void norm_rows(const NormIn &in, int rows, int hidden, bool write_h, int wave,
                                          int lane, Grow &&grow, Own &&own, Put &&put) {
  typedef NormRowBf16::v8u16 v8u16;
  const int nv = hidden / 8;
  v8u16 ws[2];
  const v8u16 *wr = reinterpret_cast<const v8u16 *>(in.w);
#pragma unroll
  for (int k = 0; k < 2; ++k) ws[k] = wr[min(lane + 64 * k, nv - 1)];
  NormRowBf16 row[kMaxRows];
#pragma unroll
  for (int j = 0; j < kMaxRows; ++j) {
    const int rr = wave + NW * j;
    if (rr < rows) {
      const int64_t g = grow(rr);
      row[j].load(in.h + g * hidden, in.delta + g * hidden, nv, lane);
    }
  }
#pragma unroll
  for (int j = 0; j < kMaxRows; ++j) {
    const int rr = wave + NW * j;
    if (rr < rows) {
      const int64_t g = grow(rr);
      uint16_t *ho = write_h && in.h_out && own(rr) ? in.h_out + g * hidden : nullptr;
      row[j].finish(ws, nv, hidden, in.eps, lane, ho, [&](int v, const v8u16 &y) { put(rr, v, y); });
    }
  }
}

}  // namespace spk
