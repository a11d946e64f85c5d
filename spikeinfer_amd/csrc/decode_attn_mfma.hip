// Paged popcount decode attention, matrix-core path (head_dim 64, GQA <= 8).
//
// Same result as the general path (spike_attention.py:67-150 semantics, fixed
// softmax offset popc(q)), with the value side on the gfx950 matrix cores.
//
// Why MFMA: per 16-byte K+V token unit the value side needs n_rep*64 = 448
// multiply-adds (GQA 7:1).  At 8 TB/s that is ~224 T MAC/s, far above what
// the fp32 VALU issues, so a lane-per-channel loop cannot approach the HBM
// roofline.  Here each 64-token step of a wave is one K=64 contraction:
//
//   D[32 x 32] += A[32 x 64] * B[64 x 32]     (v_mfma_scale_f32_32x32x64_f8f6f4)
//
//   A rows  = (head h < 8, digit s < 4): row 4h+s holds, per token, digit s of
//             the weight w(d) = exp(-d*scale), d = popc(q_h & ~k).  The weight
//             is split into four e4m3 digits, w = sum_s q_s * 2^-(8+4s)
//             (relative error <= ~1e-6), looked up in a 65-entry LDS table.
//   B cols  = 32 of the 64 channels; element = fp4 e2m1 0b0001 (= 0.5) where
//             the v bit is set.  Two MFMAs cover the 64 channels.
//
// Bits become MFMA operands through LDS transpose reads:
//   * v words are staged token-major (8 B per token).  ds_read_b64_tr_b4 on 16
//     token rows hands lane i the nibble i (channels 4i..4i+3) of all 16 rows,
//     so `(w >> s) & 0x11111111` is directly eight fp4 elements of channel
//     4i+s over eight tokens;
//   * the 8 digit words of a token (32 bytes, byte 4h+s) are staged
//     token-major; ds_read_b64_tr_b8 transposes 8x16-byte blocks so lane m
//     receives byte column m (= A row m) for 8 tokens.
// Operand layouts (measured on gfx950): A lane l holds row l%32, byte k is
// K = 32*(l/32)+k; B (fp4) lane l holds column l%32, nibble k is
// K = 32*(k/16) + 16*(l/32) + k%16; D lane l, acc j is row
// 8*(j/4) + 4*(l/32) + j%4, column l%32.
#include "decode_attn.hpp"

namespace spk {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
#define SPK_LDS __attribute__((address_space(3)))

namespace mfma {

constexpr int kWaves = 4;
constexpr int kStepTokens = 64;
constexpr int kMaxPartBlocks = 512;  // block-table entries staged per partition

struct alignas(16) WaveStage {
  uint64_t v[kStepTokens];          // token-major v words        (512 B)
  uint32_t a[kStepTokens * 8];      // token-major digit words, 8 heads (2 KB)
};

constexpr int kReduceFloats = (kWaves - 1) * 64 * 12;  // 8 values + 4 l per lane
constexpr int kSmemBytes =
    (kWaves * (int)sizeof(WaveStage) > kReduceFloats * 4) ? kWaves * (int)sizeof(WaveStage)
                                                            : kReduceFloats * 4;

// x to OCP e4m3 (bias 7, subnormal step 2^-9, sign bit 0x80), round to
// nearest even; returns the code and stores the value it encodes.  The digit
// split feeds it signed residuals (rounding up leaves a negative remainder).
__device__ inline uint32_t e4m3_encode(float x, float *val) {
  const uint32_t sign = x < 0.f ? 0x80u : 0u;
  const float a = fabsf(x);
  float v;
  uint32_t code;
  if (!(a > 0.f)) {
    v = 0.f;
    code = 0;
  } else if (a < 0.015625f) {  // below 2^-6: subnormal
    const float m = rintf(a * 512.f);
    if (m >= 8.f) { v = 0.015625f; code = 0x08; }
    else { v = m * (1.f / 512.f); code = static_cast<uint32_t>(m); }
  } else {
    int e;
    frexpf(a, &e);
    int E = e - 1;  // a in [2^E, 2^(E+1))
    float m = rintf((ldexpf(a, -E) - 1.f) * 8.f);
    if (m >= 8.f) { m = 0.f; ++E; }
    if (E > 8) { E = 8; m = 6.f; }  // saturate at 448 (never reached: |x| <= 256)
    v = ldexpf(1.f + m * 0.125f, E);
    code = static_cast<uint32_t>(((E + 7) << 3) | static_cast<int>(m));
  }
  *val = sign ? -v : v;
  return code | (code ? sign : 0u);
}

__device__ __forceinline__ v2i tr_b4(const SPK_LDS char *p) {
  return __builtin_amdgcn_ds_read_tr4_b64_v2i32((SPK_LDS v2i *)p);
}
__device__ __forceinline__ v2i tr_b8(const SPK_LDS char *p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((SPK_LDS v2i *)p);
}

// Stages one 64-token step of a wave: weight digits and v words into the
// wave's LDS stage, weights into lsum.  MASKED handles a partial last step.
template <int NREP, bool MASKED>
__device__ __forceinline__ void stage_step(WaveStage &st, int lane, uint64_t kw, uint64_t vw,
                                           bool valid, const uint32_t (&q0)[8],
                                           const uint32_t (&q1)[8], const uint2 *tab,
                                           float (&lsum)[8]) {
  const uint32_t klo = static_cast<uint32_t>(kw), khi = static_cast<uint32_t>(kw >> 32);
  uint32_t dig[8];
#pragma unroll
  for (int h = 0; h < 8; ++h) {
    if (h < NREP) {
      const int d = __popc(q0[h] & ~klo) + __popc(q1[h] & ~khi);
      const uint2 e = tab[d];
      dig[h] = (!MASKED || valid) ? e.x : 0u;
      lsum[h] += (!MASKED || valid) ? __uint_as_float(e.y) : 0.f;
    } else {
      dig[h] = 0u;
    }
  }
  st.v[lane] = (!MASKED || valid) ? vw : 0ull;
  uint4 *arow = reinterpret_cast<uint4 *>(&st.a[lane * 8]);
  arow[0] = make_uint4(dig[0], dig[1], dig[2], dig[3]);
  arow[1] = make_uint4(dig[4], dig[5], dig[6], dig[7]);
}

// Wave-level ordering of the private stage: LDS writes before the
// cross-lane transpose reads, and those reads before the next step's writes.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Transposes the staged step into MFMA operands and accumulates.
__device__ __forceinline__ void contract_step(const WaveStage &st, int lane, v16f &acc0,
                                              v16f &acc1) {
  const int g = lane >> 5;          // K group of the MFMA operands
  const int i16 = lane & 15;        // lane within its 16-lane transpose group
  const int win = (lane >> 4) & 1;  // 16-byte window of a digit row / channel offset
  const SPK_LDS char *lds_v = (const SPK_LDS char *)st.v;
  const SPK_LDS char *lds_a = (const SPK_LDS char *)st.a;
  v8i A;
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    const int row = 32 * g + 8 * qd + ((i16 >> 1) & 7);
    const v2i r = tr_b8(lds_a + row * 32 + win * 16 + (i16 & 1) * 8);
    A[2 * qd] = r.x;
    A[2 * qd + 1] = r.y;
  }
  const v2i w0 = tr_b4(lds_v + (16 * g + i16) * 8);
  const v2i w1 = tr_b4(lds_v + (32 + 16 * g + i16) * 8);
  const uint32_t wv[4] = {static_cast<uint32_t>(w0.x), static_cast<uint32_t>(w0.y),
                          static_cast<uint32_t>(w1.x), static_cast<uint32_t>(w1.y)};
  v8i B0 = {}, B1 = {};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    B0[i] = static_cast<int>((wv[i] >> win) & 0x11111111u);
    B1[i] = static_cast<int>((wv[i] >> (2 + win)) & 0x11111111u);
  }
  acc0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A, B0, acc0, 0, 4, 0, 127, 0, 127);
  acc1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A, B1, acc1, 0, 4, 0, 127, 0, 127);
}

// One workgroup = 4 waves = one (partition, t, kv head, sequence); waves take
// the partition's 64-token steps round-robin (two steps of loads in flight
// per wave) and reduce at the end in a fixed order.
template <int NREP>
__global__ __launch_bounds__(kWaves * 64) void decode_attn_mfma_kernel(AttnParams p) {
  const int part = blockIdx.x;
  const int t = blockIdx.y / p.Hkv;
  const int kvh = blockIdx.y % p.Hkv;
  const int n = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const int len = p.lens[n];
  const int nparts_seq = len <= 0 ? 1 : (len + p.part_len - 1) / p.part_len;
  if (part >= nparts_seq) return;
  const int start = part * p.part_len;
  const int end = min(len, start + p.part_len);

  __shared__ uint2 tab[65];            // per d: 4 e4m3 digits, bits of their value
  __shared__ int32_t blocks[kMaxPartBlocks];  // this partition's physical blocks
  __shared__ __align__(16) char smem[kSmemBytes];
  WaveStage &st = reinterpret_cast<WaveStage *>(smem)[wave];

  if (tid <= 64) {
    float x = expf(-static_cast<float>(tid) * p.scale) * 256.f;
    uint32_t digits = 0;
    float wsum = 0.f;
    for (int s = 0; s < 4; ++s) {
      float q;
      digits |= e4m3_encode(x, &q) << (8 * s);
      wsum += ldexpf(q, -(8 + 4 * s));
      x = (x - q) * 16.f;
    }
    tab[tid] = make_uint2(digits, __float_as_uint(wsum));
  }
  const int nblk = end > start ? ((end - start - 1) >> p.bs_log2) + 1 : 0;
  const int blk0 = start >> p.bs_log2;
  for (int b = tid; b < nblk; b += kWaves * 64) blocks[b] = p.bt[n * p.bts0 + (blk0 + b) * p.bts1];

  uint32_t q0[8], q1[8];
#pragma unroll
  for (int h = 0; h < 8; ++h) {
    q0[h] = q1[h] = 0u;
    if (h < NREP) {
      const uint32_t *qp = p.q + t * p.qs0 + n * p.qs1 + (kvh * NREP + h) * p.qs2;
      q0[h] = qp[0];
      q1[h] = qp[1];
    }
  }
  __syncthreads();

  const uint64_t *kbase = reinterpret_cast<const uint64_t *>(p.k + t * p.ks0 + kvh * p.ks1);
  const uint64_t *vbase = reinterpret_cast<const uint64_t *>(p.v + t * p.vs0 + kvh * p.vs1);
  const int bs_mask = (1 << p.bs_log2) - 1;
  const uint64_t num_slots = static_cast<uint64_t>(p.num_slots);

  // Token j of this partition -> its K/V words.  Slots outside the cache are
  // never dereferenced: they read slot 0 and are masked (tail step) or, for a
  // corrupt table, give an unspecified but fault-free result.
  auto load = [&](int j, uint64_t &kw, uint64_t &vw) {
    const int jj = min(j, end - 1);
    const int phys = blocks[(jj - start) >> p.bs_log2];
    uint64_t slot = (static_cast<uint64_t>(static_cast<uint32_t>(phys)) << p.bs_log2) |
                    static_cast<uint64_t>(jj & bs_mask);
    slot = slot < num_slots ? slot : 0;
    kw = __builtin_nontemporal_load(kbase + slot);
    vw = __builtin_nontemporal_load(vbase + slot);
  };

  v16f acc0 = {}, acc1 = {};
  float lsum[8];
#pragma unroll
  for (int h = 0; h < 8; ++h) lsum[h] = 0.f;

  constexpr int kStride = kWaves * kStepTokens;
  // Steps of this wave: full ones (every token valid), then at most one tail.
  const int first = start + wave * kStepTokens;
  const int span = end - first;
  const int nfull = span > 0 ? (span / kStride) + ((span % kStride) >= kStepTokens ? 1 : 0) : 0;
  const int ntotal = span > 0 ? (span + kStride - 1) / kStride : 0;

  uint64_t ka = 0, va = 0, kb = 0, vb = 0;
  if (ntotal > 0) load(first + lane, ka, va);
  if (ntotal > 1) load(first + kStride + lane, kb, vb);
  for (int i = 0; i < ntotal; ++i) {
    uint64_t kc = 0, vc = 0;
    if (i + 2 < ntotal) load(first + (i + 2) * kStride + lane, kc, vc);
    if (i < nfull) {
      stage_step<NREP, false>(st, lane, ka, va, true, q0, q1, tab, lsum);
    } else {
      const bool valid = first + i * kStride + lane < end;
      stage_step<NREP, true>(st, lane, ka, va, valid, q0, q1, tab, lsum);
    }
    wave_sync();
    contract_step(st, lane, acc0, acc1);
    wave_sync();
    ka = kb; va = vb;
    kb = kc; vb = vc;
  }

  // Per lane: column n = lane%32 of both tiles; rows 4h+s with
  // h = 2*qd + lane/32, s = j%4, for acc index j = 4*qd + s.  The digit scale
  // 2^-(8+4s) and the fp4 value 0.5 of a set bit fold into one factor.
  float val[8];
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float f = ldexpf(1.f, -(7 + 4 * s));
      a0 += acc0[4 * qd + s] * f;
      a1 += acc1[4 * qd + s] * f;
    }
    val[2 * qd] = a0;
    val[2 * qd + 1] = a1;
  }
  float lw[8];
#pragma unroll
  for (int h = 0; h < 8; ++h) {
    float l = lsum[h];
    for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
    lw[h] = l;
  }

  // Cross-wave reduction (fixed order) through LDS, reusing the stage area.
  __syncthreads();
  float *red = reinterpret_cast<float *>(smem);
  if (wave > 0) {
    float *dst = red + ((wave - 1) * 64 + lane) * 12;
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = val[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[8 + i] = lw[2 * i + (lane >> 5)];
  }
  __syncthreads();
  if (wave != 0) return;
  float lh[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) lh[i] = lw[2 * i + (lane >> 5)];
  for (int w = 1; w < kWaves; ++w) {
    const float *src = red + ((w - 1) * 64 + lane) * 12;
#pragma unroll
    for (int i = 0; i < 8; ++i) val[i] += src[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) lh[i] += src[8 + i];
  }

  const int col = lane & 31;
  const bool single = nparts_seq == 1;
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    const int h = 2 * qd + (lane >> 5);
    if (h >= NREP) continue;
    const int hq = kvh * NREP + h;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int ch = 4 * (col & 15) + 2 * u + (col >> 4);
      const float a = val[2 * qd + u];
      if (single) {
        const float o = len <= 0 ? 0.f : a / lh[qd];
        store_f32_as(p.out, t * p.os0 + n * p.os1 + hq * p.os2 + ch * p.os3, p.out_dtype, o);
      } else {
        float *dst = p.ws + ((((int64_t)part * p.T + t) * p.N + n) * p.Hq + hq) * 65;
        dst[ch] = a;
        if (ch == 0) dst[64] = lh[qd];
      }
    }
  }
}

}  // namespace mfma

bool mfma_path_supported(const AttnParams &p) {
  const auto al8 = [](const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 7) == 0; };
  return p.head_dim == 64 && p.nrep <= 8 && p.ks2 == 2 && p.vs2 == 2 &&
         (p.ks0 % 2) == 0 && (p.ks1 % 2) == 0 && (p.vs0 % 2) == 0 && (p.vs1 % 2) == 0 &&
         al8(p.k) && al8(p.v) &&
         ((p.part_len + (1 << p.bs_log2) - 1) >> p.bs_log2) <= mfma::kMaxPartBlocks;
}

void launch_decode_mfma(const AttnParams &p, dim3 grid, hipStream_t s) {
  const int threads = mfma::kWaves * 64;
  switch (p.nrep) {
    case 1: mfma::decode_attn_mfma_kernel<1><<<grid, threads, 0, s>>>(p); break;
    case 2: mfma::decode_attn_mfma_kernel<2><<<grid, threads, 0, s>>>(p); break;
    case 3: mfma::decode_attn_mfma_kernel<3><<<grid, threads, 0, s>>>(p); break;
    case 4: mfma::decode_attn_mfma_kernel<4><<<grid, threads, 0, s>>>(p); break;
    case 5: mfma::decode_attn_mfma_kernel<5><<<grid, threads, 0, s>>>(p); break;
    case 6: mfma::decode_attn_mfma_kernel<6><<<grid, threads, 0, s>>>(p); break;
    case 7: mfma::decode_attn_mfma_kernel<7><<<grid, threads, 0, s>>>(p); break;
    default: mfma::decode_attn_mfma_kernel<8><<<grid, threads, 0, s>>>(p); break;
  }
}

}  // namespace spk
