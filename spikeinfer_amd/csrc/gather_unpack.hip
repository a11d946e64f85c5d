// Prefill reader of the paged spike cache: one sequence's first seq_len cached
// tokens, walked through its block table, unpacked to dense 0/1 spikes.
//
// Reference: gather_kv_unpacked (spikeinfer/kernels/spike_attention.py:224-244),
// which is a slot-matrix index_select on the packed words followed by
// unpack_spikes (packing.py:136-152) -- two launches and a packed temporary per
// cache.  Here one launch serves K and V together: thread = (cache, t, head,
// token, 8-channel chunk); it reads the chunk's byte of the token's packed word
// straight from its slot and writes the 8 dense elements as one vector store,
// so the only HBM traffic is the packed words once and the dense output once.
#include "common.hpp"

namespace spk {
namespace {

// 8 spikes (bits of `b`) as 8 elements of dtype DT, written at `dst`
// (16-byte aligned for 2- and 4-byte types, 8-byte for u8).
template <int DT>
__device__ __forceinline__ void store8(char *dst, uint32_t b) {
  if constexpr (DT == SPK_F32 || DT == SPK_I32) {
    const uint32_t one = DT == SPK_F32 ? 0x3f800000u : 1u;
    uint4 lo, hi;
    lo.x = (b & 1u) ? one : 0u;  lo.y = (b & 2u) ? one : 0u;
    lo.z = (b & 4u) ? one : 0u;  lo.w = (b & 8u) ? one : 0u;
    hi.x = (b & 16u) ? one : 0u; hi.y = (b & 32u) ? one : 0u;
    hi.z = (b & 64u) ? one : 0u; hi.w = (b & 128u) ? one : 0u;
    reinterpret_cast<uint4 *>(dst)[0] = lo;
    reinterpret_cast<uint4 *>(dst)[1] = hi;
  } else if constexpr (DT == SPK_U8) {
    // Spread bit i to byte i: multiply-free with two masks per half.
    uint32_t lo = (b & 0xfu), hi = (b >> 4) & 0xfu;
    lo = (lo | (lo << 7) | (lo << 14) | (lo << 21)) & 0x01010101u;
    hi = (hi | (hi << 7) | (hi << 14) | (hi << 21)) & 0x01010101u;
    reinterpret_cast<uint2 *>(dst)[0] = make_uint2(lo, hi);
  } else {
    const uint32_t one = DT == SPK_BF16 ? 0x3f80u : 0x3c00u;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = ((b >> (2 * i)) & 1u ? one : 0u) | (((b >> (2 * i + 1)) & 1u ? one : 0u) << 16);
    reinterpret_cast<uint4 *>(dst)[0] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

struct GatherParams {
  const uint32_t *cache[2];  // K, V (V may be null)
  char *out[2];              // [T, H, S, D] contiguous each
  int64_t cs0, cs1, cs2;     // cache strides (elements): t, head, slot; word axis contiguous
  int64_t num_slots;
  const int32_t *table;      // this sequence's block-table row
  int64_t bt_stride;
  int n_table;               // entries in the row
  int S;                     // tokens to read
  int T, H, D, bs_log2;
  int ncache;
};

// Vector form: D % 8 == 0, output rows 16-byte aligned (8-byte for u8).
template <int DT>
__global__ __launch_bounds__(256) void gather_unpack_vec_kernel(GatherParams p) {
  constexpr int kEsz = (DT == SPK_F32 || DT == SPK_I32) ? 4 : (DT == SPK_U8 ? 1 : 2);
  const int chunks = p.D >> 3;
  const int64_t per_cache = (int64_t)p.T * p.H * p.S * chunks;
  const int64_t total = per_cache * p.ncache;
  const uint32_t nblocks = static_cast<uint32_t>(min<int64_t>(p.num_slots >> p.bs_log2, 0xffffffffll));
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int which = i >= per_cache;
    int64_t r = i - which * per_cache;
    const int c = static_cast<int>(r % chunks);
    r /= chunks;
    const int j = static_cast<int>(r % p.S);
    const int64_t plane = r / p.S;  // t * H + h
    const int h = static_cast<int>(plane % p.H), t = static_cast<int>(plane / p.H);
    const int blk = j >> p.bs_log2;
    uint32_t b = 0;
    if (blk < p.n_table) {
      const uint32_t phys = static_cast<uint32_t>(p.table[blk * p.bt_stride]);
      if (phys < nblocks) {
        const int64_t slot = (static_cast<int64_t>(phys) << p.bs_log2) | (j & ((1 << p.bs_log2) - 1));
        const uint32_t w = p.cache[which][t * p.cs0 + h * p.cs1 + slot * p.cs2 + (c >> 2)];
        b = (w >> (8 * (c & 3))) & 0xffu;
      }
    }
    char *dst = p.out[which] + (((plane * p.S + j) * p.D) + 8 * c) * kEsz;
    store8<DT>(dst, b);
  }
}

// Any D: one element per thread.
__global__ __launch_bounds__(256) void gather_unpack_kernel(GatherParams p, int dtype) {
  const int64_t per_cache = (int64_t)p.T * p.H * p.S * p.D;
  const int64_t total = per_cache * p.ncache;
  const uint32_t nblocks = static_cast<uint32_t>(min<int64_t>(p.num_slots >> p.bs_log2, 0xffffffffll));
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int which = i >= per_cache;
    const int64_t e = i - which * per_cache;
    const int ch = static_cast<int>(e % p.D);
    const int64_t r = e / p.D;
    const int j = static_cast<int>(r % p.S);
    const int64_t plane = r / p.S;
    const int h = static_cast<int>(plane % p.H), t = static_cast<int>(plane / p.H);
    const int blk = j >> p.bs_log2;
    bool s = false;
    if (blk < p.n_table) {
      const uint32_t phys = static_cast<uint32_t>(p.table[blk * p.bt_stride]);
      if (phys < nblocks) {
        const int64_t slot = (static_cast<int64_t>(phys) << p.bs_log2) | (j & ((1 << p.bs_log2) - 1));
        s = (p.cache[which][t * p.cs0 + h * p.cs1 + slot * p.cs2 + (ch >> 5)] >> (ch & 31)) & 1u;
      }
    }
    store_spike(p.out[which], e, dtype, s);
  }
}

unsigned grid_of(int64_t items) {
  int64_t g = (items + 255) / 256;
  return static_cast<unsigned>(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

}  // namespace
}  // namespace spk

using namespace spk;

extern "C" int spk_gather_unpack(const int32_t *k_cache, const int32_t *v_cache,
                                 const int64_t cache_strides[4], int64_t num_slots,
                                 const int32_t *block_table, int64_t bt_stride, int n_table,
                                 int seq_len, void *k_out, void *v_out, int out_dtype, int T,
                                 int H, int head_dim, int block_size, void *stream) {
  if (T <= 0 || H <= 0 || head_dim <= 0 || seq_len < 0 || n_table < 0)
    return fail(SPK_EINVAL, "gather_unpack: bad sizes T=%d H=%d D=%d seq_len=%d", T, H, head_dim, seq_len);
  if (!is_pow2(block_size)) return fail(SPK_EINVAL, "gather_unpack: block_size=%d is not a power of two", block_size);
  if (!valid_any_dtype(out_dtype)) return fail(SPK_EINVAL, "gather_unpack: out dtype %d", out_dtype);
  if (cache_strides[3] != 1) return fail(SPK_EINVAL, "gather_unpack: packed word axis must be contiguous");
  if (!k_cache || !k_out || (v_cache == nullptr) != (v_out == nullptr))
    return fail(SPK_EINVAL, "gather_unpack: k cache/output required, v cache and output together");
  if (seq_len == 0) return SPK_OK;
  GatherParams p{};
  p.cache[0] = reinterpret_cast<const uint32_t *>(k_cache);
  p.cache[1] = reinterpret_cast<const uint32_t *>(v_cache);
  p.out[0] = static_cast<char *>(k_out);
  p.out[1] = static_cast<char *>(v_out);
  p.cs0 = cache_strides[0]; p.cs1 = cache_strides[1]; p.cs2 = cache_strides[2];
  p.num_slots = num_slots;
  p.table = block_table; p.bt_stride = bt_stride; p.n_table = n_table;
  p.S = seq_len; p.T = T; p.H = H; p.D = head_dim; p.bs_log2 = ilog2(block_size);
  p.ncache = v_cache ? 2 : 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int esz = (out_dtype == SPK_F32 || out_dtype == SPK_I32) ? 4 : (out_dtype == SPK_U8 ? 1 : 2);
  const uintptr_t al = (reinterpret_cast<uintptr_t>(k_out) | reinterpret_cast<uintptr_t>(v_out));
  const bool vec = head_dim % 8 == 0 && (al % (esz == 1 ? 8 : 16)) == 0;
  if (vec) {
    const unsigned g = grid_of((int64_t)T * H * seq_len * (head_dim / 8) * p.ncache);
    switch (out_dtype) {
      case SPK_F32: gather_unpack_vec_kernel<SPK_F32><<<g, 256, 0, s>>>(p); break;
      case SPK_F16: gather_unpack_vec_kernel<SPK_F16><<<g, 256, 0, s>>>(p); break;
      case SPK_BF16: gather_unpack_vec_kernel<SPK_BF16><<<g, 256, 0, s>>>(p); break;
      case SPK_U8: gather_unpack_vec_kernel<SPK_U8><<<g, 256, 0, s>>>(p); break;
      default: gather_unpack_vec_kernel<SPK_I32><<<g, 256, 0, s>>>(p); break;
    }
  } else {
    gather_unpack_kernel<<<grid_of((int64_t)T * H * seq_len * head_dim * p.ncache), 256, 0, s>>>(p, out_dtype);
  }
  return check_launch("gather_unpack");
}
