// Shared helpers for the gfx950 spiking decode kernels: error reporting across
// the C ABI, element loads/stores by dtype code, launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/spikeinfer_amd.h"

namespace spk {

// Per-thread message of the last failed call, returned by spk_last_error().
std::string &last_error_slot();

inline int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  last_error_slot() = buf;
  return code;
}

// Reports a launch error (bad configuration, missing code object) as SPK_EHIP.
inline int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(SPK_EHIP, "%s: %s", what, hipGetErrorString(e));
  return SPK_OK;
}

inline bool is_pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }
inline int ilog2(int x) {
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

// ---- element access by dtype code -----------------------------------------

// Orders a wave's LDS writes before reads of what other lanes of the same
// wave wrote (release fence, wave barrier, acquire fence).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// fp32 -> bf16 with round-to-nearest-even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float load_as_f32(const void *p, int64_t i, int dtype) {
  switch (dtype) {
    case SPK_F32: return static_cast<const float *>(p)[i];
    case SPK_F16: return static_cast<float>(static_cast<const _Float16 *>(p)[i]);
    case SPK_BF16: return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
    case SPK_U8: return static_cast<float>(static_cast<const uint8_t *>(p)[i]);
    default: return static_cast<float>(static_cast<const int32_t *>(p)[i]);
  }
}

__device__ __forceinline__ bool load_nonzero(const void *p, int64_t i, int dtype) {
  switch (dtype) {
    // Bit tests rather than float compares: -0.0 and +0.0 both pack as 0,
    // anything else (including NaN) packs as 1, matching `x != 0`.
    case SPK_F32: return (static_cast<const uint32_t *>(p)[i] & 0x7fffffffu) != 0;
    case SPK_F16:
    case SPK_BF16: return (static_cast<const uint16_t *>(p)[i] & 0x7fffu) != 0;
    case SPK_U8: return static_cast<const uint8_t *>(p)[i] != 0;
    default: return static_cast<const int32_t *>(p)[i] != 0;
  }
}

__device__ __forceinline__ void store_f32_as(void *p, int64_t i, int dtype, float v) {
  switch (dtype) {
    case SPK_F32: static_cast<float *>(p)[i] = v; break;
    case SPK_F16: static_cast<_Float16 *>(p)[i] = static_cast<_Float16>(v); break;
    case SPK_BF16: static_cast<uint16_t *>(p)[i] = f32_to_bf16_bits(v); break;
    case SPK_U8: static_cast<uint8_t *>(p)[i] = static_cast<uint8_t>(v); break;
    default: static_cast<int32_t *>(p)[i] = static_cast<int32_t>(v); break;
  }
}

// Stores a 0/1 spike without going through a float conversion.
__device__ __forceinline__ void store_spike(void *p, int64_t i, int dtype, bool s) {
  switch (dtype) {
    case SPK_F32: static_cast<uint32_t *>(p)[i] = s ? 0x3f800000u : 0u; break;
    case SPK_F16: static_cast<uint16_t *>(p)[i] = s ? 0x3c00u : 0u; break;
    case SPK_BF16: static_cast<uint16_t *>(p)[i] = s ? 0x3f80u : 0u; break;
    case SPK_U8: static_cast<uint8_t *>(p)[i] = s ? 1u : 0u; break;
    default: static_cast<int32_t *>(p)[i] = s ? 1 : 0; break;
  }
}

inline bool valid_float_dtype(int d) { return d == SPK_F32 || d == SPK_F16 || d == SPK_BF16; }
inline bool valid_any_dtype(int d) { return d >= SPK_F32 && d <= SPK_I32; }

}  // namespace spk
