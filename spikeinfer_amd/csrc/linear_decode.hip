// Small-M linear layer of the decode step: y = x @ W^T (+ bias), bf16, for the
// q/k/v, o, down and lm_head projections (spikeinfer/modeling_fast.py:121-135,
// :150-166, :190, :335-355) at decode batch sizes (M = T * n_tok <= 256 rows).
// Three launch shapes: the tiled kernel below (K <= 1280), a wide-N variant
// (the lm_head) and a long-K variant with 16-row groups (the down projection).
//
// MI355X design (the same ground rules as the fused MLP gate in mlp_gate.hip):
// at these sizes a projection is bound by moving x and W into the CUs and by
// latency, not by the matrix cores.
//   * A workgroup owns a 32- or 64-row group of x, the whole K, in LDS (at
//     most 160 KB), loaded once by global_load_lds into a layout swizzled by
//     row (16-byte chunk c of row r at chunk c ^ (r % 16)).
//   * W is repacked once at load in MFMA-fragment order (spk_linear_pack):
//     one k-step (32 K) of one 16-column tile is one contiguous 1 KB block, so a
//     wave's B operand arrives with one coalesced 16-byte load per lane.
//   * The workgroup's 16-column tiles are split into (tile, K-eighth) units
//     over its 8 waves; each wave issues all of its units' loads at once and
//     the eight partial sums of a tile are added in a fixed order through LDS
//     (deterministic).
//   * v_mfma_f32_16x16x32_bf16: D lane l, acc j = row 4(l/16) + j of the row
//     tile, column l % 16.
// Grid: row groups x column ranges (ranges chosen so the launch has about 256
// workgroups); the row groups of one range are consecutive on one XCD (block b
// -> XCD b % 8), so W comes from HBM once.
#include <algorithm>

#include "common.hpp"
#include "lif_math.hpp"
#include "norm_rows.hpp"

namespace spk {
namespace lin {

typedef __bf16 v8b __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
#define SPK_LDS __attribute__((address_space(3)))

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kRows = 64;            // rows of x per workgroup, at most (4 row tiles)
constexpr int kParts = 8;            // K split of a tile into units
constexpr int kMaxUnitsPerWave = 2;  // tiles per range <= 2 (3 for the 32-row groups, below)
constexpr int kMaxPartSteps = 5;     // k-steps per part: K <= 8 * 5 * 32 = 1280
constexpr int kLdsBytes = 160 * 1024;
// One partial: RT row tiles x 4 x 64 lanes; the y staging follows the slots.
template <int RT> constexpr int slot_floats() { return RT * 4 * 64; }
template <int RT, int MU> constexpr int stage_off() { return kWaves * MU * slot_floats<RT>() * 4; }
constexpr int kStageBytes = 16 * 16 * 2;                               // one wave's 16 x 16 tile
static_assert(stage_off<4, 2>() + kWaves * kStageBytes <= kLdsBytes, "slots and staging fit the LDS");

// Packed W (spk_linear_pack): for tile p (rows 16p..16p+15 of W) and k-step
// ks, 1 KB at (p * KS + ks) KB: lane l's 16 bytes are W[16p + l%16][32ks +
// 8(l/16) .. +7].

// NORM: the rows are add_rmsnorm(nin.h, nin.delta, nin.w) (x unused), computed
// in the prologue; the workgroups of the last column range (never empty) write
// h + delta to nin.h_out.
// RT: row tiles of 16 per workgroup (2 or 4); MU: tiles per column range,
// at most (2, or 3 with 32-row groups).
template <bool NORM, int RT, int MU>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(RT == 4 ? 2 : 4))) void linear_kernel(
    const uint16_t *x, const v4u *wp, const uint16_t *bias, uint16_t *y, int M, int N, int K,
    int MG, int R, NormIn nin) {
  extern __shared__ __align__(16) char smem[];
  const int KS = K / 32, kChunks = K / 8;  // k-steps, 16-byte chunks per row
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.x, xcd = b & 7, s = b >> 3;
  const int m = s % MG, r = (s / MG) * 8 + xcd;
  const int P = N / 16;
  const int p0 = r * P / R, np = (r + 1) * P / R - p0;
  if (np <= 0) return;  // uniform over the workgroup
  static_assert(!NORM || RT == 4, "the norm prologue runs 64-row groups");
  constexpr int kR = 16 * RT, kSF = slot_floats<RT>();
  const int m0 = m * kR;

  // The bias of the epilogue's columns, loaded first (its latency hides under
  // the whole launch).
  float bv[MU];
#pragma unroll
  for (int e = 0; e < MU; ++e)
    bv[e] = bias ? elem_to_f32<SPK_BF16>(bias[16 * (p0 + min(e, np - 1)) + (lane & 15)]) : 0.f;
  // Units (tile, part): wave w takes units w, w + 8 (and w + 16) (np <= MU tiles).
  // W arrives with nontemporal loads: the row groups of a range run on one
  // XCD at about the same time, and streaming W past the caches measured
  // faster in the decode step (with the MLP gate's: 1.570 -> 1.549 ms).
  const int U = np * kParts;
  auto part_range = [&](int part, int &k0, int &k1) {
    k0 = part * KS / kParts;
    k1 = (part + 1) * KS / kParts;
  };
  v4u bq[MU][kMaxPartSteps];
#pragma unroll
  for (int j = 0; j < MU; ++j) {
    const int u = wave + kWaves * j;
    if (u < U) {
      int k0, k1;
      part_range(u % kParts, k0, k1);
      const v4u *src = wp + static_cast<int64_t>((p0 + u / kParts) * KS + k0) * 64 + lane;
#pragma unroll
      for (int ks = 0; ks < kMaxPartSteps; ++ks)
        if (ks < k1 - k0) bq[j][ks] = __builtin_nontemporal_load(src + ks * 64);
    }
  }

  // x rows m0..m0+16RT-1 (clamped to M - 1) into LDS, chunk c of row rr at c ^ (rr % 16).
  if constexpr (NORM) {
    norm_rows<kWaves, kRows / kWaves>(
        nin, kRows, K, r == R - 1, wave, lane, [&](int rr) { return static_cast<int64_t>(min(m0 + rr, M - 1)); },
        [&](int rr) { return m0 + rr < M; },
        [&](int rr, int v, const NormRowBf16::v8u16 &yv) {
          *reinterpret_cast<NormRowBf16::v8u16 *>(smem + rr * (kChunks * 16) + 16 * (v ^ (rr & 15))) = yv;
        });
  } else {
    const int total = kR * kChunks;  // a multiple of 64 (K % 128 == 0)
    for (int base = wave * 64; base < total; base += kWaves * 64) {
      const int g = base + lane;
      const int rr = g / kChunks, pc = g - rr * kChunks;
      const int c = pc ^ (rr & 15);
      const int row = min(m0 + rr, M - 1);
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(x + static_cast<int64_t>(row) * K + 8 * c),
                                       (SPK_LDS void *)(smem + base * 16), 16, 0, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)
  __syncthreads();

  const int r16 = lane & 15, kq = lane >> 4;
  v4f acc[MU][RT];
#pragma unroll
  for (int j = 0; j < MU; ++j)
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[j][t] = v4f{};
#pragma unroll
  for (int j = 0; j < MU; ++j) {
    const int u = wave + kWaves * j;
    if (u < U) {
      int k0, k1;
      part_range(u % kParts, k0, k1);
#pragma unroll
      for (int ks = 0; ks < kMaxPartSteps; ++ks) {
        if (ks < k1 - k0) {
          const int c = 4 * (k0 + ks) + kq;
          const v8b bw = __builtin_bit_cast(v8b, bq[j][ks]);
#pragma unroll
          for (int t = 0; t < RT; ++t) {
            const int rr = 16 * t + r16;
            const v8b a = *reinterpret_cast<const v8b *>(smem + rr * (kChunks * 16) + 16 * (c ^ r16));
            acc[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bw, acc[j][t], 0, 0, 0);
          }
        }
      }
    }
  }

  // Partials through LDS (x no longer read), slot = unit index; a lane's
  // accumulator of row tile t is one 16-byte chunk (t * 64 + lane).
  __syncthreads();
  v4f *slots = reinterpret_cast<v4f *>(smem);
#pragma unroll
  for (int j = 0; j < MU; ++j) {
    const int u = wave + kWaves * j;
    if (u < U) {
      v4f *d = slots + u * (kSF / 4);
#pragma unroll
      for (int t = 0; t < RT; ++t) d[t * 64 + lane] = acc[j][t];
    }
  }
  __syncthreads();

  // Epilogue: wave w finishes row tile w % RT of tile p0 + w / RT (w / RT < np),
  // summing its eight parts in order, adding the bias (loaded at the start)
  // and writing y (fp32 sum + bias, rounded once, as the GEMM epilogue).
  const int et = wave % RT, ee = wave / RT;
  if (ee >= np) return;
  float sum[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sum[i] = 0.f;
#pragma unroll
  for (int part = 0; part < kParts; ++part) {
    const v4f a = slots[(ee * kParts + part) * (kSF / 4) + et * 64 + lane];
#pragma unroll
    for (int i = 0; i < 4; ++i) sum[i] += a[i];
  }
  // The 16 x 16 bf16 tile is staged in the wave's 512 bytes above the
  // partial slots; its rows' 32 bytes then go out as two 16-byte stores.
  uint16_t *stg = reinterpret_cast<uint16_t *>(smem + stage_off<RT, MU>() + wave * kStageBytes);
#pragma unroll
  for (int i = 0; i < 4; ++i) stg[(4 * kq + i) * 16 + r16] = f32_to_elem<SPK_BF16>(sum[i] + bv[ee]);
  wave_lds_sync();  // lanes read rows other lanes wrote
  const int row = m0 + 16 * et + (lane >> 1);  // lane pair -> one row
  if (lane < 32 && row < M) {
    const v4u v = reinterpret_cast<const v4u *>(stg)[lane];
    reinterpret_cast<v4u *>(y + static_cast<int64_t>(row) * N + 16 * (p0 + ee))[lane & 1] = v;
  }
}

// Wide N (the lm_head: 151,936 columns) at M <= 64: the x rows stay in LDS for
// the whole launch and each wave runs whole-K pairs of 16-column tiles,
// streaming W through a register ring of up to 10 k-steps; no cross-wave sums.
// LDS rows are padded by one 16-byte chunk instead of swizzled (row stride
// = 16 mod 256 bytes: 16 consecutive rows still hit 16 distinct bank groups),
// so a k-step's fragment address is a per-row-tile base plus an immediate;
// with the swizzle every (k-step, row tile) address is its own register.
// Ring depth: up to 10 k-steps of W in flight per wave (a divisor of KS).
constexpr int ring_depth(int ks) {
  for (int d = 10; d > 1; --d)
    if (ks % d == 0) return d;
  return 1;
}
template <int KS>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void linear_wide_kernel(
    const uint16_t *x, const v4u *wp, const uint16_t *bias, uint16_t *y, int M, int N, bool vec) {
  extern __shared__ __align__(16) char smem[];
  constexpr int K = 32 * KS, kChunks = K / 8, kRowChunks = kChunks + 1;
  static_assert(kRows * kRowChunks * 16 <= kLdsBytes, "the padded x rows fit the LDS");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int PP = N / 32;  // tile pairs
  const int q0 = static_cast<int>(static_cast<int64_t>(blockIdx.x) * PP / gridDim.x);
  const int q1 = static_cast<int>(static_cast<int64_t>(blockIdx.x + 1) * PP / gridDim.x);
  // All 64 rows (clamped copies past M): a branch per row tile would put
  // control flow between every MFMA, which costs more registers than the
  // unused products cost time in this memory-bound kernel.
  for (int base = wave * 64; base < kRows * kRowChunks; base += kWaves * 64) {
    const int g = base + lane;
    const int rr = g / kRowChunks, pc = g - rr * kRowChunks;
    const int row = min(rr, M - 1);
    const int c = pc < kChunks ? pc : 0;  // the pad chunk loads a copy of chunk 0
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(x + static_cast<int64_t>(row) * K + 8 * c),
                                     (SPK_LDS void *)(smem + base * 16), 16, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)
  __syncthreads();
  const int r16 = lane & 15, kq = lane >> 4;
  const char *abase = smem + r16 * (kRowChunks * 16) + 16 * kq;  // row r16 of tile 0, chunk kq
  // W through a buffer resource: the lane's byte offset in a VGPR, the
  // k-step's (1 KB apart) in an SGPR, so the ring costs no address registers.
  // Every byte of W is read once per launch: nontemporal loads (aux 2), which
  // measured 63.3 -> 55.3 us for the lm_head (64 rows x 151,936 x 896).
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<v4u *>(wp), 0, -1, 0x00020000);
  auto wload = [&](int vofs, int ks) {
    return __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rs, vofs, ks * 1024, 2));
  };
  constexpr int D = ring_depth(KS);
  // Ring of D k-steps: slot ks % D is read by k-step ks's MFMAs and then
  // refilled with k-step ks + D; past the pair's last k-step it takes the
  // wave's next pair's first ones (KS is a multiple of D, so k-step j of the
  // next pair lands in slot j % D), and the ring never drains between pairs.
  int q = q0 + wave;
  if (q >= q1) return;  // no barrier below
  v4u r0[D], r1[D];
  {
    const int vofs0 = (2 * q * KS * 64 + lane) * 16, vofs1 = vofs0 + KS * 1024;
#pragma unroll
    for (int ks = 0; ks < D; ++ks) {
      r0[ks] = wload(vofs0, ks);
      r1[ks] = wload(vofs1, ks);
    }
  }
  for (; q < q1; q += kWaves) {
    const int vofs0 = (2 * q * KS * 64 + lane) * 16, vofs1 = vofs0 + KS * 1024;
    const bool more = q + kWaves < q1;
    const int nofs0 = vofs0 + 2 * kWaves * KS * 1024, nofs1 = nofs0 + KS * 1024;
    v4f acc0[4], acc1[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc0[t] = acc1[t] = v4f{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      // Keeps each k-step's LDS reads with its MFMAs: hoisted, the reads of
      // every k-step would be live at once and spill.
      __builtin_amdgcn_sched_barrier(0);
      const int slot = ks % D;
      const v8b w0 = __builtin_bit_cast(v8b, r0[slot]), w1 = __builtin_bit_cast(v8b, r1[slot]);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const v8b a = *reinterpret_cast<const v8b *>(abase + t * (16 * kRowChunks * 16) + 64 * ks);
        acc0[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, w0, acc0[t], 0, 0, 0);
        acc1[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, w1, acc1[t], 0, 0, 0);
      }
      if (ks + D < KS) {
        r0[slot] = wload(vofs0, ks + D);
        r1[slot] = wload(vofs1, ks + D);
      } else if (more) {  // the next pair's first k-steps, into the same slots
        r0[slot] = wload(nofs0, ks + D - KS);
        r1[slot] = wload(nofs1, ks + D - KS);
      }
    }
    const int col = 32 * q + r16;
    const float bv0 = bias ? elem_to_f32<SPK_BF16>(bias[col]) : 0.f;
    const float bv1 = bias ? elem_to_f32<SPK_BF16>(bias[col + 16]) : 0.f;
    constexpr int kXBytes = kRows * kRowChunks * 16;
    // The pair's 64 x 32 tile through a per-wave LDS stage, out as 16-byte row
    // pieces (64 B a row; 55.2 -> 53.3 us at the lm_head with the unbroken
    // ring, against 2-byte stores); a y that is not 16-byte aligned, or an x
    // that leaves no room for the stage, keeps the 2-byte stores.
    if constexpr (kXBytes + kWaves * 4096 <= kLdsBytes) {
      if (vec) {
        uint16_t *stg = reinterpret_cast<uint16_t *>(smem + kXBytes + wave * 4096);
        wave_lds_sync();  // the previous pair's reads are done
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int row = 16 * t + 4 * kq + i;
            stg[row * 32 + r16] = f32_to_elem<SPK_BF16>(acc0[t][i] + bv0);
            stg[row * 32 + 16 + r16] = f32_to_elem<SPK_BF16>(acc1[t][i] + bv1);
          }
        wave_lds_sync();  // lanes read rows other lanes wrote
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c = lane + 64 * j, row = c >> 2;
          const v4u v = reinterpret_cast<const v4u *>(stg)[c];
          if (row < M) *reinterpret_cast<v4u *>(y + static_cast<int64_t>(row) * N + 32 * q + 8 * (c & 3)) = v;
        }
        continue;
      }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * t + 4 * kq + i;
        if (row < M) {
          y[static_cast<int64_t>(row) * N + col] = f32_to_elem<SPK_BF16>(acc0[t][i] + bv0);
          y[static_cast<int64_t>(row) * N + col + 16] = f32_to_elem<SPK_BF16>(acc1[t][i] + bv1);
        }
      }
  }
}

// Long K (the down projection, K = 4864) at M <= 256: 16 rows of x per
// workgroup (16 * K * 2 <= 160 KB of LDS), 3-4 column tiles per workgroup, and
// the 8 waves split K into eighths.  Each wave streams its k-steps of W in
// chunks of 4 through a double buffer (branch-free: a chunk past the wave's
// range multiplies a zero B), then the eight partials of each tile are added
// in wave order through LDS.
constexpr int kTallRows = 16;
constexpr int kTallChunk = 4;  // k-steps per chunk
template <int NP>
__device__ __forceinline__ void linear_tall_run(const v4u *wp, uint16_t *y, int M, int N, int KS,
                                                int m0, int p0, char *smem) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kChunks = 4 * KS;  // 16-byte chunks per x row
  const int r16 = lane & 15, kq = lane >> 4;
  const int k0 = wave * KS / kWaves, nk = (wave + 1) * KS / kWaves - k0;
  const int nc = ((nk + kTallChunk - 1) / kTallChunk + 1) & ~1;  // chunks, even
  auto load = [&](int c, v4u (&b)[kTallChunk][NP]) {
#pragma unroll
    for (int j = 0; j < kTallChunk; ++j) {
      const int ks = k0 + min(c * kTallChunk + j, nk - 1);
#pragma unroll
      for (int t = 0; t < NP; ++t) b[j][t] = wp[(static_cast<int64_t>(p0 + t) * KS + ks) * 64 + lane];
    }
  };
  v4f acc[NP];
#pragma unroll
  for (int t = 0; t < NP; ++t) acc[t] = v4f{};
  auto compute = [&](int c, const v4u (&b)[kTallChunk][NP]) {
#pragma unroll
    for (int j = 0; j < kTallChunk; ++j) {
      const int kk = c * kTallChunk + j;
      const int ks = k0 + min(kk, nk - 1);
      const int ch = 4 * ks + kq;
      const v8b a = *reinterpret_cast<const v8b *>(smem + r16 * (kChunks * 16) + 16 * (ch ^ r16));
#pragma unroll
      for (int t = 0; t < NP; ++t) {
        const v4u bz = kk < nk ? b[j][t] : v4u{0u, 0u, 0u, 0u};
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(v8b, bz), acc[t], 0, 0, 0);
      }
    }
  };
  v4u bA[kTallChunk][NP], bB[kTallChunk][NP];
  load(0, bA);
  for (int c = 0; c < nc; c += 2) {
    load(c + 1, bB);
    compute(c, bA);
    load(c + 2, bA);  // past the end: clamped re-reads, never used
    compute(c + 1, bB);
  }
  __syncthreads();  // every wave is done with the x rows: the LDS takes the partials
  float *slots = reinterpret_cast<float *>(smem);
#pragma unroll
  for (int t = 0; t < NP; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) slots[((wave * NP + t) * 4 + i) * 64 + lane] = acc[t][i];
  __syncthreads();
  if (wave >= NP) return;
  float sum[4] = {0.f, 0.f, 0.f, 0.f};
  for (int w = 0; w < kWaves; ++w)
#pragma unroll
    for (int i = 0; i < 4; ++i) sum[i] += slots[((w * NP + wave) * 4 + i) * 64 + lane];
  const int col = 16 * (p0 + wave) + r16;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = m0 + 4 * kq + i;
    if (row < M) y[static_cast<int64_t>(row) * N + col] = f32_to_elem<SPK_BF16>(sum[i]);
  }
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void linear_tall_kernel(
    const uint16_t *x, const v4u *wp, uint16_t *y, int M, int N, int K, int MG, int R) {
  extern __shared__ __align__(16) char smem[];
  const int KS = K / 32, kChunks = K / 8;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.x, xcd = b & 7, s = b >> 3;
  const int m = s % MG, r = (s / MG) * 8 + xcd;
  const int P = N / 16;
  const int p0 = r * P / R, np = (r + 1) * P / R - p0;
  if (np <= 0) return;  // uniform over the workgroup
  const int m0 = m * kTallRows;
  for (int base = wave * 64; base < kTallRows * kChunks; base += kWaves * 64) {
    const int g = base + lane;
    const int rr = g / kChunks, pc = g - rr * kChunks;
    const int c = pc ^ (rr & 15);
    const int row = min(m0 + rr, M - 1);
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(x + static_cast<int64_t>(row) * K + 8 * c),
                                     (SPK_LDS void *)(smem + base * 16), 16, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)
  __syncthreads();
  if (np == 4) linear_tall_run<4>(wp, y, M, N, KS, m0, p0, smem);
  else if (np == 3) linear_tall_run<3>(wp, y, M, N, KS, m0, p0, smem);
  else if (np == 2) linear_tall_run<2>(wp, y, M, N, KS, m0, p0, smem);
  else linear_tall_run<1>(wp, y, M, N, KS, m0, p0, smem);
}

__global__ __launch_bounds__(256) void linear_pack_kernel(const uint16_t *w, v4u *out, int N, int K) {
  const int KS = K / 32;
  const int64_t total = static_cast<int64_t>(N / 16) * KS * 64;
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int l = static_cast<int>(e & 63);
    const int64_t blk = e >> 6;
    const int ks = static_cast<int>(blk % KS);
    const int64_t p = blk / KS;
    out[e] = *reinterpret_cast<const v4u *>(w + (16 * p + (l & 15)) * K + 32 * ks + 8 * (l >> 4));
  }
}

}  // namespace lin

extern "C" int spk_linear_pack(const void *w, int N, int K, int dtype, void *w_packed, void *stream) {
  if (dtype != SPK_BF16) return fail(SPK_EUNSUPPORTED, "linear_pack: bf16 weights only");
  if (N <= 0 || K <= 0 || N % 16 || K % 32)
    return fail(SPK_EINVAL, "linear_pack: N=%d K=%d (need multiples of 16 and 32)", N, K);
  if ((reinterpret_cast<uintptr_t>(w) & 15) || (reinterpret_cast<uintptr_t>(w_packed) & 15))
    return fail(SPK_EINVAL, "linear_pack: pointers must be 16-byte aligned");
  lin::linear_pack_kernel<<<1024, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t *>(w), static_cast<lin::v4u *>(w_packed), N, K);
  return check_launch("linear_pack");
}

// The tiled kernel (K <= 1280, M <= 256): rows from x, or (nin) normed in the
// prologue.
static int launch_linear_tiled(const void *x, const void *w_packed, const void *bias, void *y, int M, int N,
                               int K, const NormIn *nin, hipStream_t s) {
  // Column ranges: a multiple of 8 (one per XCD), about 256 workgroups in
  // all, at most two 16-column tiles each (three with 32-row groups).  32-row
  // groups (two workgroups fit a CU, so one's x fill overlaps the other's
  // MFMAs) whenever that grid stays within 256 workgroups, 64-row groups
  // otherwise.  Measured (graph of 24 distinct weights, K = 896): M = 32:
  // q/k/v 5.46 -> 4.25 us, o 5.17 -> 4.11 us; M = 256: o (N = 896) 5.37 ->
  // 5.14 us, q/k/v (N = 1152, three tiles a range) 6.90 -> 6.45 us.  The sum
  // of every element (eight K parts in order) is the same either way.
  const int P = N / 16;
  auto ranges = [&](int MG, int mu) {
    int R = ((256 / MG) + 7) / 8 * 8;
    if (R < 8) R = 8;
    while (R * mu < P) R += 8;
    return R;
  };
  const int MG2 = (M + 31) / 32;
  const int RT = !nin && MG2 * ranges(MG2, 3) <= 256 ? 2 : 4;
  const int rows = 16 * RT;
  const int MG = (M + rows - 1) / rows;
  const int R = ranges(MG, RT == 2 ? 3 : 2);
  const int MU = R * 2 >= P ? 2 : 3;  // 3 only where a range needs it (more registers)
  if (reinterpret_cast<uintptr_t>(y) & 15)  // (this kernel's tile rows go out as 16-byte stores)
    return fail(SPK_EUNSUPPORTED, "linear_decode: y must be 16-byte aligned for this shape");
  const NormIn none{};
  const lin::v4u *wp = static_cast<const lin::v4u *>(w_packed);
  const uint16_t *xb = static_cast<const uint16_t *>(x), *bb = static_cast<const uint16_t *>(bias);
  uint16_t *yb = static_cast<uint16_t *>(y);
  // Each launch takes the LDS it needs; the attribute (set once per kernel,
  // index k) lets any of them take all 160 KB.
  static bool attr[4] = {false, false, false, false};
  auto go = [&](auto kernel, int k, int lds, const NormIn &ni) -> int {
    if (!attr[k]) {
      if (hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                              lin::kLdsBytes) != hipSuccess)
        return fail(SPK_EHIP, "linear_decode: cannot reserve %d bytes of LDS", lin::kLdsBytes);
      attr[k] = true;
    }
    kernel<<<MG * R, lin::kThreads, lds, s>>>(xb, wp, bb, yb, M, N, K, MG, R, ni);
    return check_launch("linear_decode");
  };
  if (nin) return go(lin::linear_kernel<true, 4, 2>, 0, lin::kLdsBytes, *nin);
  if (RT == 4) return go(lin::linear_kernel<false, 4, 2>, 1, lin::kLdsBytes, none);
  const int x_bytes = rows * K * 2;
  if (MU == 2)
    return go(lin::linear_kernel<false, 2, 2>, 2,
              std::max(x_bytes, lin::stage_off<2, 2>() + lin::kWaves * lin::kStageBytes), none);
  return go(lin::linear_kernel<false, 2, 3>, 3, std::max(x_bytes, lin::stage_off<2, 3>() + lin::kWaves * lin::kStageBytes),
            none);
}

extern "C" int spk_linear_decode(const void *x, const void *w_packed, const void *bias, void *y,
                                 int M, int N, int K, int dtype, void *stream) {
  if (dtype != SPK_BF16) return fail(SPK_EUNSUPPORTED, "linear_decode: bf16 only");
  if (K > lin::kParts * lin::kMaxPartSteps * 32 && !bias && M >= 1 && M <= 4 * lin::kRows &&
      N >= 16 && N % 16 == 0 && K % 128 == 0 &&
      static_cast<int64_t>(lin::kTallRows) * K * 2 <= lin::kLdsBytes) {
    // Long K: 16-row groups, 3-4 tiles per range.
    if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(w_packed) & 15))
      return fail(SPK_EINVAL, "linear_decode: x and packed weights must be 16-byte aligned");
    const int MG = (M + lin::kTallRows - 1) / lin::kTallRows;
    int R = ((256 / MG) + 7) / 8 * 8;
    while (R * 4 < N / 16) R += 8;
    static bool attr = false;
    if (!attr) {
      if (hipFuncSetAttribute(reinterpret_cast<const void *>(lin::linear_tall_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lin::kLdsBytes) != hipSuccess)
        return fail(SPK_EHIP, "linear_decode: cannot reserve %d bytes of LDS", lin::kLdsBytes);
      attr = true;
    }
    lin::linear_tall_kernel<<<MG * R, lin::kThreads, lin::kLdsBytes, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint16_t *>(x), static_cast<const lin::v4u *>(w_packed),
        static_cast<uint16_t *>(y), M, N, K, MG, R);
    return check_launch("linear_decode");
  }
  if (M < 1 || M > 4 * lin::kRows || N < 16 || N % 16 || K % 128 ||
      K > lin::kParts * lin::kMaxPartSteps * 32 || static_cast<int64_t>(lin::kRows) * K * 2 > lin::kLdsBytes)
    return fail(SPK_EUNSUPPORTED, "linear_decode: M=%d N=%d K=%d not supported", M, N, K);
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(w_packed) & 15))
    return fail(SPK_EINVAL, "linear_decode: x and packed weights must be 16-byte aligned");
  const int MG = (M + lin::kRows - 1) / lin::kRows;
  // Column ranges: a multiple of 8 (one per XCD), about 256 workgroups in all,
  // and at most two 16-column tiles each.
  const int P = N / 16;
  int R = ((256 / MG) + 7) / 8 * 8;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (MG == 1 && P > lin::kMaxUnitsPerWave * R && N % 32 == 0) {
    // Wide N: 256 workgroups, each a range of tile pairs.  Rows of y are
    // N * 2 bytes (a multiple of 64), so an aligned y takes 16-byte stores.
    const bool vec = (reinterpret_cast<uintptr_t>(y) & 15) == 0;
#define SPK_WIDE_CASE(KS)                                                                              \
  case KS: {                                                                                         \
    static bool attr = false;                                                                        \
    if (!attr) {                                                                                     \
      if (hipFuncSetAttribute(reinterpret_cast<const void *>(lin::linear_wide_kernel<KS>),            \
                              hipFuncAttributeMaxDynamicSharedMemorySize, lin::kLdsBytes) != hipSuccess) \
        return fail(SPK_EHIP, "linear_decode: cannot reserve %d bytes of LDS", lin::kLdsBytes);      \
      attr = true;                                                                                   \
    }                                                                                                \
    lin::linear_wide_kernel<KS><<<256, lin::kThreads, lin::kLdsBytes, s>>>(                           \
        static_cast<const uint16_t *>(x), static_cast<const lin::v4u *>(w_packed),                   \
        static_cast<const uint16_t *>(bias), static_cast<uint16_t *>(y), M, N, vec);                 \
    return check_launch("linear_decode");                                                           \
  }
    // K = 1280 is not here: its padded x rows (164,864 B) exceed the LDS, and
    // the tiled kernel takes it.
    switch (K / 32) {
      SPK_WIDE_CASE(16)
      SPK_WIDE_CASE(20)
      SPK_WIDE_CASE(24)
      SPK_WIDE_CASE(28)
      SPK_WIDE_CASE(32)
      SPK_WIDE_CASE(36)
    }
#undef SPK_WIDE_CASE
  }
  return launch_linear_tiled(x, w_packed, bias, y, M, N, K, nullptr, s);
}

extern "C" int spk_norm_linear_decode(const void *h, const void *delta, const void *norm_weight, void *h_out,
                                      float eps, const void *w_packed, const void *bias, void *y, int M, int N,
                                      int K, int dtype, void *stream) {
  if (dtype != SPK_BF16) return fail(SPK_EUNSUPPORTED, "norm_linear_decode: bf16 only");
  if (M < 1 || M > 4 * lin::kRows || N < 16 || N % 16 || K % 128 || K > 1024 ||
      K > lin::kParts * lin::kMaxPartSteps * 32)
    return fail(SPK_EUNSUPPORTED, "norm_linear_decode: M=%d N=%d K=%d not supported", M, N, K);
  if (!h || !delta || !norm_weight || !w_packed || !y)
    return fail(SPK_EINVAL, "norm_linear_decode: null pointer");
  const auto al = [](const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  if (!al(h) || !al(delta) || !al(norm_weight) || !al(w_packed) || (h_out && !al(h_out)))
    return fail(SPK_EINVAL, "norm_linear_decode: h, delta, norm weight, h_out and packed weights must be 16-byte aligned");
  if (h_out && (h_out == h || h_out == delta))
    return fail(SPK_EINVAL, "norm_linear_decode: h_out must not alias h or delta");
  NormIn nin{static_cast<const uint16_t *>(h), static_cast<const uint16_t *>(delta),
             static_cast<const uint16_t *>(norm_weight), static_cast<uint16_t *>(h_out), eps};
  return launch_linear_tiled(nullptr, w_packed, bias, y, M, N, K, &nin, static_cast<hipStream_t>(stream));
}

}  // namespace spk
