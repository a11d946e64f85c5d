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

// The same recurrence carrying the reset flag: r is the previous step's
// spike (u - th > 0 on the same u), which the reset of this step needs, so it
// is not recomputed; r * th is th or zth = 0 * th (the same value, signed
// zero included).  Start with r = (u0 - th > 0) and zth = 0.f * th.
__device__ __forceinline__ bool lif_step_r(float &u, bool &r, float cur, float beta, float th, float zth) {
  u = (beta * u + cur) - (r ? th : zth);
  r = u - th > 0.f;
  return r;
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

// V consecutive per-channel parameters from p[off .. off + V) of dtype `dt`,
// as fp32: 16-byte vector loads when the run is 16-byte aligned (the usual
// case: contiguous fp32/bf16/f16 parameter vectors and off % V == 0), scalar
// loads otherwise.
template <int V>
__device__ __forceinline__ void load_params(const void *p, int dt, int64_t off, float (&out)[V]) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  if (dt == SPK_F32 && ((a + off * 4) & 15) == 0 && V % 4 == 0) {
    typedef float F4 __attribute__((ext_vector_type(4)));
    const F4 *q = reinterpret_cast<const F4 *>(static_cast<const float *>(p) + off);
#pragma unroll
    for (int v = 0; v < V / 4; ++v) {
      const F4 x = q[v];
#pragma unroll
      for (int j = 0; j < 4; ++j) out[4 * v + j] = x[j];
    }
  } else if ((dt == SPK_BF16 || dt == SPK_F16) && ((a + off * 2) & 15) == 0 && V % 8 == 0) {
    typedef uint16_t H8 __attribute__((ext_vector_type(8)));
    const H8 *q = reinterpret_cast<const H8 *>(static_cast<const uint16_t *>(p) + off);
#pragma unroll
    for (int v = 0; v < V / 8; ++v) {
      const H8 x = q[v];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        // Through a scalar: a bit-cast applied to the vector element itself
        // has been compiled as a cast of element 0 for every j.
        const uint16_t e = x[j];
        out[8 * v + j] = dt == SPK_BF16 ? bf16_bits_to_f32(e)
                                        : static_cast<float>(__builtin_bit_cast(_Float16, e));
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) out[j] = load_as_f32(p, off + j, dt);
  }
}

}  // namespace spk
