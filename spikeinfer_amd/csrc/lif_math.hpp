// The LIF membrane step shared by every kernel that runs the neuron.
//
// Reference: spikeinfer/kernels/lif_triton.py:96-101.  Files including this
// are compiled with -ffp-contract=off so `beta*u + cur` rounds twice, exactly
// as PyTorch eager evaluates it.
#pragma once

#include "common.hpp"

namespace spk {

// One LIF step on the fp32 membrane; returns the spike.  The delayed reset
// uses the membrane of the previous step.
__device__ __forceinline__ bool lif_step(float &u, float cur, float beta, float th) {
  const float r = (u - th > 0.f) ? 1.f : 0.f;
  u = (beta * u + cur) - r * th;
  return u - th > 0.f;
}

__device__ __forceinline__ float clamp01(float b) { return fminf(fmaxf(b, 0.f), 1.f); }

// ---- element types of the 16-byte vector paths ------------------------------
template <int DT> struct Elem;
template <> struct Elem<SPK_F32> { typedef float T; static constexpr int kVec = 4; };
template <> struct Elem<SPK_F16> { typedef uint16_t T; static constexpr int kVec = 8; };
template <> struct Elem<SPK_BF16> { typedef uint16_t T; static constexpr int kVec = 8; };

template <int DT>
__device__ __forceinline__ float elem_to_f32(typename Elem<DT>::T v) {
  if constexpr (DT == SPK_F32) return v;
  else if constexpr (DT == SPK_BF16) return bf16_bits_to_f32(v);
  else return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

// fp32 -> element with round-to-nearest-even (the rounding of a torch
// elementwise op whose result has this dtype).
template <int DT>
__device__ __forceinline__ typename Elem<DT>::T f32_to_elem(float f) {
  if constexpr (DT == SPK_F32) return f;
  else if constexpr (DT == SPK_BF16) return f32_to_bf16_bits(f);
  else return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// The fp32 value of f after rounding to the element type.
template <int DT>
__device__ __forceinline__ float round_to(float f) {
  return elem_to_f32<DT>(f32_to_elem<DT>(f));
}

template <int DT>
__device__ __forceinline__ typename Elem<DT>::T spike_elem(bool s) {
  if constexpr (DT == SPK_F32) return s ? 1.f : 0.f;
  else if constexpr (DT == SPK_BF16) return s ? 0x3f80 : 0;
  else return s ? 0x3c00 : 0;
}

}  // namespace spk
