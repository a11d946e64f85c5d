// Paged popcount decode attention, matrix-core path (head_dim 64, GQA <= 8).
//
// Same result as the general path (spike_attention.py:67-150 semantics, fixed
// softmax offset popc(q)), with the value side on the gfx950 matrix cores.
//
// Why MFMA: per 16-byte K+V token unit the value side needs n_rep*64 = 448
// multiply-adds (GQA 7:1).  At 8 TB/s that is ~224 T MAC/s, far above what
// the fp32 VALU issues, so a lane-per-channel loop cannot approach the HBM
// roofline.  Here each 128-token step of a wave is one K=128 contraction per
// output tile:
//
//   D[16 x 16] += A[16 x 128] * B[128 x 16]   (v_mfma_scale_f32_16x16x128_f8f6f4)
//
//   A rows  = (head h, digit s < 4) of one row tile (heads 4rt..4rt+3): row
//             4(h-4rt)+s holds, per token, digit s of the weight
//             w(d) = exp(-d*scale), d = popc(q_h & ~k).  The weight is split
//             into four e4m3 digits, w = sum_s q_s * 2^-(8+4s) (relative error
//             <= ~1e-6), looked up in a 129-entry LDS table (built once per
//             scale on the host, passed in the arguments).
//   B cols  = 16 channels 4c+ts (c < 16) of channel tile ts; element = fp4
//             with the v bit in place (0.5, 1.0 or 2.0 per set bit); a fifth,
//             all-ones tile accumulates the softmax denominators.
//   Two row tiles x five column tiles = 10 MFMAs per step (each about half
//   the issue time of a 32x32x64 one, measured).
//
// Bits become MFMA operands through LDS transpose reads:
//   * v words are staged token-major (8 B per token).  ds_read_b64_tr_b4 on 16
//     token rows hands lane i of each 16-lane group nibble i (channels
//     4i..4i+3) of all 16 rows, so `w & (0x11111111 << s)` is eight fp4
//     elements of channel 4i+s over eight tokens (bit 3, the fp4 sign, is
//     first shifted down to bit 2);
//   * the 8 digit words of a token (32 bytes, byte 4h+s) are staged
//     token-major; ds_read_b64_tr_b8 transposes 8x16-byte blocks so lane m
//     receives byte column m (= A row m) for 8 tokens.
// Operand layouts of the 16x16x128 f8 x f4 MFMA (measured on gfx950 with
// one-hot probes): A lane l holds row l%16, byte k is
// K = 16*(l/16) + k%16 + 64*(k/16); B (fp4) lane l holds column l%16, nibble
// n is K = 32*(l/16) + n; D lane l, acc j is row 4*(l/16) + j, column l%16.
#include "decode_attn.hpp"
#include "lif_math.hpp"

#include <cmath>
#include <type_traits>

namespace spk {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
#define SPK_LDS __attribute__((address_space(3)))

namespace mfma {

constexpr int kWaves = 4;  // waves per workgroup, except the short-context launch (KW = 2)

constexpr int kStepTokens = 128;      // tokens per wave step (2 per lane)
constexpr int kMaxPartBlocks = kMaxStagedBlocks;  // block-table entries staged per partition

// Stage of one wave step.  Row r holds token 2r (r < 64) or token
// 2(r-64)+1 (r >= 64) of the step, so lane l writes rows l and l+64 and every
// staging write and transpose read touches consecutive 8/16-byte chunks (no
// LDS bank conflicts).  Digit rows are 32 bytes (byte 4h+s = digit s of head
// h), stored as two 16-byte windows: a[w][r] = bytes 16w..16w+15 of row r.
// W64 = head_dim / 64 v words per token, v[w][r] = word w of row r.
template <int W64>
struct alignas(16) WaveStage {
  uint64_t v[W64][kStepTokens];       // v words of each row            (1 KB each)
  uint4 a[2][kStepTokens];            // digit rows, window-major            (4 KB)
};

// The workgroup's stages (each wave's also holds its cross-wave reduction
// values, 8 * W64 + 2 floats a lane, after its last step).
template <int W64, int KW>
constexpr int kSmemBytes = KW * (int)sizeof(WaveStage<W64>);

__device__ __forceinline__ v2i tr_b4(const SPK_LDS char *p) {
  return __builtin_amdgcn_ds_read_tr4_b64_v2i32((SPK_LDS v2i *)p);
}
__device__ __forceinline__ v2i tr_b8(const SPK_LDS char *p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((SPK_LDS v2i *)p);
}

// popc(a) + popc(b) as v_bcnt with its accumulator operand.  Written out
// because the compiler otherwise distributes the table-index scaling over both
// counts (two extra shifts per lookup on the hottest path).
__device__ __forceinline__ uint32_t popc2(uint32_t a, uint32_t b) {
  uint32_t d;
  asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(d) : "v"(b), "v"(__popc(a)));
  return d;
}

// popc(a) + acc, the same accumulate form.
__device__ __forceinline__ uint32_t bcnt_add(uint32_t a, uint32_t acc) {
  uint32_t d;
  asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(d) : "v"(a), "v"(acc));
  return d;
}

// Digit words of one token for the NREP heads; zero when masked off.
// q[w][h] = 32-bit word w of head h's packed query.
template <int NREP, int W64, bool MASKED>
__device__ __forceinline__ void token_digits(const uint64_t (&kw)[W64], bool valid,
                                             const uint32_t (&q)[2 * W64][8], const uint32_t *tab,
                                             uint32_t (&dig)[8]) {
  uint32_t kn[2 * W64];
#pragma unroll
  for (int w = 0; w < W64; ++w) {
    kn[2 * w] = ~static_cast<uint32_t>(kw[w]);
    kn[2 * w + 1] = ~static_cast<uint32_t>(kw[w] >> 32);
  }
#pragma unroll
  for (int h = 0; h < 8; ++h) {
    if (h < NREP) {
      uint32_t d = popc2(q[0][h] & kn[0], q[1][h] & kn[1]);
#pragma unroll
      for (int w = 2; w < 2 * W64; ++w) d = bcnt_add(q[w][h] & kn[w], d);
      dig[h] = (!MASKED || valid) ? tab[d] : 0u;
    } else {
      dig[h] = 0u;
    }
  }
}

// Stages one 128-token step of a wave (lane l holds tokens 2l and 2l+1,
// staged as rows l and l+64):
// weight digits and v words into the wave's LDS stage.
template <int NREP, int W64, bool MASKED>
__device__ __forceinline__ void stage_step(WaveStage<W64> &st, int lane,
                                           const uint64_t (&kw)[2][W64],
                                           const uint64_t (&vw)[2][W64], const bool (&valid)[2],
                                           const uint32_t (&q)[2 * W64][8], const uint32_t *tab) {
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    uint32_t dig[8];
    token_digits<NREP, W64, MASKED>(kw[e], valid[e], q, tab, dig);
    const int row = lane + 64 * e;
    st.a[0][row] = make_uint4(dig[0], dig[1], dig[2], dig[3]);
    if (NREP > 4) st.a[1][row] = make_uint4(dig[4], dig[5], dig[6], dig[7]);
#pragma unroll
    for (int w = 0; w < W64; ++w) st.v[w][row] = (!MASKED || valid[e]) ? vw[e][w] : 0ull;
  }
}

// Wave-level ordering of the private stage: LDS writes before the
// cross-lane transpose reads, and those reads before the next step's writes.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Contracts the 128 staged rows of a step with 16x16x128 MFMAs: K index k
// reads stage row srow(k) = (k%32 < 16 ? 0 : 64) + 16*(k/32) + k%16 (any
// order shared by A and B gives the same sums; this one lets every 16-lane
// transpose group read its own contiguous rows).
//   A, row tile rt (heads 4rt..4rt+3): lane l holds row l%16 = (head, digit),
//     bytes 0..15 -> K 16q..16q+15 and bytes 16..31 -> K 64+16q.. (q = l/16),
//     read as four 8-row tr_b8 transposes of the tile's 16-byte window;
//   B, channel tile s (0..3): lane l holds column l%16 = channel 4*(l%16)+s,
//     nibble n -> K 32p + n (p = l/16), from two tr_b4 transposes (rows
//     16p.. and 64+16p..); bit s of each nibble is kept in place for s < 3
//     (fp4 0.5, 1.0, 2.0) and shifted to bit 2 for s = 3 (2.0);
//   the all-ones B tile accumulates the softmax denominators.
// With W64 = 2 the channel tiles of v word hv are acc[rt][4*hv + s]
// (channel 64*hv + 4*(l%16) + s); the A operand is shared.
// The contraction is split in read_ops (LDS -> registers) and mma_ops so
// that a step's MFMAs can run while the next step is staged.

// Operands of one staged step, held in registers so that the stage can take
// the next step's rows while these MFMAs run.
template <int W64>
struct StepOps {
  v8i A[2];          // digit rows of row tiles 0 and 1
  uint32_t w[W64][4];  // transposed v words (nibble i = channels 4i..4i+3)
};

template <int RT, int W64>  // row tiles: heads 4rt..4rt+3 for rt < RT
__device__ __forceinline__ void read_ops(const WaveStage<W64> &st, int lane, StepOps<W64> &o) {
  const int q = lane >> 4;
  const int i16 = lane & 15;
  const int r0 = ((q & 1) ? 64 : 0) + 16 * (q >> 1);  // rows of A bytes 0..15; +32 for 16..31
  const int sub = (i16 >> 1) & 7, hb = (i16 & 1) * 8;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const SPK_LDS char *lds_a = (const SPK_LDS char *)&st.a[rt][0];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int row = r0 + 32 * (c >> 1) + 8 * (c & 1) + sub;
      const v2i r = tr_b8(lds_a + row * 16 + hb);
      o.A[rt][2 * c] = r.x;
      o.A[rt][2 * c + 1] = r.y;
    }
  }
#pragma unroll
  for (int hv = 0; hv < W64; ++hv) {
    const SPK_LDS char *lds_v = (const SPK_LDS char *)st.v[hv];
    const v2i w0 = tr_b4(lds_v + (16 * q + i16) * 8);
    const v2i w1 = tr_b4(lds_v + (64 + 16 * q + i16) * 8);
    o.w[hv][0] = static_cast<uint32_t>(w0.x);
    o.w[hv][1] = static_cast<uint32_t>(w0.y);
    o.w[hv][2] = static_cast<uint32_t>(w1.x);
    o.w[hv][3] = static_cast<uint32_t>(w1.y);
  }
}

typedef int v4i_ __attribute__((ext_vector_type(4)));  // the denominators' B operand (4 VGPRs)
template <int RT, int W64>
__device__ __forceinline__ void mma_ops(const StepOps<W64> &o, v4f (&acc)[2][4 * W64], v4f (&accl)[2],
                                        const v4i_ &ones) {
  constexpr uint32_t kMask[4] = {0x11111111u, 0x22222222u, 0x44444444u, 0x44444444u};
#pragma unroll
  for (int hv = 0; hv < W64; ++hv) {
#pragma unroll
    for (int ts = 0; ts < 4; ++ts) {
      v8i B = {};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        B[i] = static_cast<int>((ts == 3 ? o.w[hv][i] >> 1 : o.w[hv][i]) & kMask[ts]);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
        acc[rt][4 * hv + ts] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            o.A[rt], B, acc[rt][4 * hv + ts], 0, 4, 0, 127, 0, 127);
    }
  }
  const v8i Bl = {ones[0], ones[1], ones[2], ones[3], 0, 0, 0, 0};
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
    accl[rt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(o.A[rt], Bl, accl[rt], 0, 4, 0, 127, 0, 127);
}

// Longest-processing-time-first order of the launch's blocks, computed by
// every workgroup for itself.  An item ((sequence, partition), i = part * N +
// sequence) takes ups blocks, one per unit, or -- with PAIRS (the 4-wave plain
// kernel) and at most kPairMaxLen tokens -- ceil(ups / 2) blocks of two units
// each, whose waves then take twice the steps.  Items are ordered by the
// steps each of their waves takes (a paired item's tokens count twice), in
// buckets 256 tokens wide whose low bit marks paired items, ties in item
// order; the blocks of an item are consecutive.  Items are counted into an
// LDS histogram, the buckets scanned largest first in blocks, and block b's
// item found by a block-wide prefix count of its bucket's members.  When
// every sequence has the same length and one partition, the order is the
// item order, known after one vote.
//
// Returns block b's item, or -1 when the block has none (uniform over the
// block); *sub_out gets the unit (or, paired, the unit pair) within the
// item, *pair_out whether it is paired, *len_out its sequence length (as
// seq_len computes it).  Needs N * num_parts <= kInlinePlanItems; `sh` holds
// kMaxBuckets + 10 ints and is free again after the call.
constexpr int kMaxBuckets = 2 * 130;  // (steps per wave in 256-token units + 2) x paired
constexpr int kPlanKeys = 8;          // per-thread item keys kept in registers between the passes
// Bucket of an item of `size` tokens.  An empty item (size <= 0: nothing to
// sum, zeros out) is paired whenever pairs are on, so no item takes more than
// ceil(ups / 2) blocks when every item is short (the host sizes such a grid
// to N * num_parts * ceil(ups / 2)).
template <bool PAIRS>
__device__ __forceinline__ int plan_bucket(int size) {
  if (size <= 0) return PAIRS ? 1 : 0;
  const bool paired = PAIRS && size <= kPairMaxLen;
  const int eff = paired ? 2 * size : size;
  return 2 * (((eff + 255) >> 8) + 1) + (paired ? 1 : 0);
}
template <int KW, bool PAIRS>
__device__ __forceinline__ int plan_slot(const AttnParams &p, int b, int ups, int *sh, int *len_out,
                                         int *sub_out, bool *pair_out) {
  constexpr int kThreads = KW * 64;
  int *count = sh, *wsum = sh + kMaxBuckets, *res = wsum + KW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int M = p.N * p.num_parts;
  const int A = (ups + 1) >> 1;  // blocks of a paired item
  const int nb = 2 * (((max(p.part_len, PAIRS ? 2 * kPairMaxLen : 0) + 255) >> 8) + 2);
  auto bpi = [&](int bucket) { return (bucket & 1) ? A : ups; };  // blocks per item
  // Bucket of item i, -1 when the sequence has no such partition; `len` gets
  // the sequence's length.
  auto key = [&](int i, int &len) {
    const int n = i % p.N, part = i / p.N;
    len = seq_len(p, n);
    const int nparts = len <= 0 ? 1 : (len + p.part_len - 1) / p.part_len;
    if (part >= nparts) return -1;
    return plan_bucket<PAIRS>(min(p.part_len, len - part * p.part_len));
  };
  const int per = (M + kThreads - 1) / kThreads;
  const int i0 = min(M, tid * per), i1 = min(M, i0 + per);
  // The thread's first kPlanKeys keys and lengths are loaded once, before the
  // first barrier, and reused by the second pass (one dependent memory round
  // trip fewer in the prologue of every workgroup).
  int kc[kPlanKeys], lc[kPlanKeys];
#pragma unroll
  for (int k = 0; k < kPlanKeys; ++k) {
    kc[k] = -1;
    lc[k] = 0;
  }
  if (p.num_parts == 1 && per > 1) {
    // One partition per sequence (item i is sequence i), several items a
    // thread: the loads are unconditional (past the thread's range they
    // re-read its last item, in bounds), so they are in flight together --
    // a branch per key made the compiler wait for each load before the next.
#pragma unroll
    for (int k = 0; k < kPlanKeys; ++k) lc[k] = seq_len(p, min(i0 + k, max(i1 - 1, 0)));
#pragma unroll
    for (int k = 0; k < kPlanKeys; ++k)
      if (i0 + k < i1) kc[k] = plan_bucket<PAIRS>(min(p.part_len, lc[k]));
  } else {
#pragma unroll
    for (int k = 0; k < kPlanKeys; ++k) kc[k] = i0 + k < i1 ? key(i0 + k, lc[k]) : -1;
  }
  // Equal lengths (one partition each): the order is the item order, known
  // after one vote -- the histogram passes and their barriers are skipped.
  if (p.num_parts == 1) {
    const int l0 = seq_len(p, 0);
    bool same = per <= kPlanKeys;
#pragma unroll
    for (int k = 0; k < kPlanKeys; ++k) same = same && (i0 + k >= i1 || lc[k] == l0);
    if (__syncthreads_and(same)) {
      const int bk = plan_bucket<PAIRS>(min(p.part_len, l0));
      const int q = b / bpi(bk);
      *len_out = l0;
      *sub_out = b - q * bpi(bk);
      *pair_out = (bk & 1) != 0;
      return q < M ? q : -1;
    }
  }
  auto key_at = [&](int i, int &len) {
    const int k = i - i0;
#pragma unroll
    for (int c = 0; c < kPlanKeys; ++c)
      if (c == k) {
        len = lc[c];
        return kc[c];
      }
    return key(i, len);
  };
  for (int bk = tid; bk < nb; bk += kThreads) count[bk] = 0;
  __syncthreads();
  for (int i = i0; i < i1; ++i) {
    int len;
    const int k = key_at(i, len);
    if (k >= 0) atomicAdd(&count[k], 1);
  }
  __syncthreads();
  if (wave == 0) {  // largest bucket first, in blocks: lane holds list positions 5*lane..5*lane+4
    constexpr int kPer = (kMaxBuckets + 63) / 64;
    int c[kPer], sum = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int pos = kPer * lane + k;
      const int bk = nb - 1 - pos;
      c[k] = pos < nb ? count[bk] * bpi(bk) : 0;
      sum += c[k];
    }
    int incl = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o);
      if (lane >= o) incl += y;
    }
    int run = incl - sum;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      if (run <= b && b < run + c[k]) {
        const int bk = nb - 1 - (kPer * lane + k);
        res[0] = bk;
        res[1] = (b - run) / bpi(bk);  // rank within the bucket
        res[4] = (b - run) % bpi(bk);  // block within the item
      }
      run += c[k];
    }
    if (lane == 63 && b >= incl) res[0] = -1;
  }
  __syncthreads();
  const int sel = res[0], j = res[1];
  *sub_out = res[4];
  *pair_out = (sel & 1) != 0;
  if (sel < 0) return -1;
  int mine = 0;
  for (int i = i0; i < i1; ++i) {
    int len;
    mine += key_at(i, len) == sel;
  }
  int incl = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int before = incl - mine;
  for (int w = 0; w < wave; ++w) before += wsum[w];
  if (before <= j && j < before + mine) {
    int r = j - before;
    for (int i = i0; i < i1; ++i) {
      int len;
      if (key_at(i, len) == sel && r-- == 0) {
        res[2] = i;
        res[3] = len;  // the slot's sequence length: no reload after the plan
      }
    }
  }
  __syncthreads();
  *len_out = res[3];
  return res[2];
}

// One workgroup = KW waves (4, or 2 for short contexts) = one (partition, t, kv head, sequence); waves take
// the partition's 128-token steps round-robin (two steps of loads in flight
// per wave) and reduce at the end in a fixed order.
// Fused path: the unit's spikes at timestep t from the q/k/v currents, as
// spk_qkv_rope_lif_pack computes them (the same RoPE roundings and LIF
// recurrence over timesteps 0..t).  Each wave takes two heads a round: lane
// half lane/32 one head, lane%32 the channel pair (c, c + 32), so a ballot
// of each half's spikes is that head's packed word.  fw[h] for the NREP q
// heads, fw[NREP] for k, fw[NREP + 1] for v.  fused_load issues every load
// of the unit at once (ahead of the block-table staging); fused_spikes then
// computes, overlapping the first K/V loads.
template <int XDT>
struct FusedIn {
  typedef typename Elem<XDT>::T E;
  static constexpr int kRounds = 2;  // (NREP + 2) heads <= 10, 8 per round
  E xl[kRounds][kMaxFusedT], xh[kRounds][kMaxFusedT];
  float blo[kRounds], bhi[kRounds], tlo[kRounds], thi[kRounds];
  float clo[kRounds], chi[kRounds], slo[kRounds], shi[kRounds];
};

// Every load is unconditional (lanes of a round past the last head read the
// last head's currents, timesteps past t re-read timestep t; both are
// dropped): with a branch per load the compiler waited for each in turn.
// beta / th are fp32 (the host converts other dtypes, exactly).
template <int NREP, int XDT>
__device__ __forceinline__ void fused_load(const AttnParams &p, int n, int t, int kvh, int wave,
                                           int lane, FusedIn<XDT> &in) {
  typedef typename Elem<XDT>::T E;
  const FusedParams &f = p.fz;
  const int64_t q = f.pos[n];
  const int64_t prow = q < 0 ? 0 : (q >= f.table_rows ? f.table_rows - 1 : q);
  const int c = lane & 31;
  const E *cosr = static_cast<const E *>(f.cos) + prow * 64;
  const E *sinr = static_cast<const E *>(f.sin) + prow * 64;
  const E *xtok = static_cast<const E *>(f.x) + n * f.xs1;
  const float *beta = static_cast<const float *>(f.beta);
  const float *th = static_cast<const float *>(f.th);
#pragma unroll
  for (int r = 0; r < (NREP + 2 + 7) / 8; ++r) {
    const int hi = min(r * 8 + wave * 2 + (lane >> 5), NREP + 1);
    const int site = hi < NREP ? 0 : (hi == NREP ? 1 : 2);
    const int col = (hi < NREP ? kvh * NREP + hi : (hi == NREP ? p.Hq + kvh : p.Hq + p.Hkv + kvh)) * 64;
#pragma unroll
    for (int k = 0; k < kMaxFusedT; ++k) {
      in.xl[r][k] = xtok[min(k, t) * f.xs0 + col + c];
      in.xh[r][k] = xtok[min(k, t) * f.xs0 + col + c + 32];
    }
    in.blo[r] = clamp01(beta[site * 64 + c]);
    in.bhi[r] = clamp01(beta[site * 64 + c + 32]);
    in.tlo[r] = th[site * 64 + c];
    in.thi[r] = th[site * 64 + c + 32];
    in.clo[r] = elem_to_f32<XDT>(cosr[c]);
    in.chi[r] = elem_to_f32<XDT>(cosr[c + 32]);
    in.slo[r] = elem_to_f32<XDT>(sinr[c]);
    in.shi[r] = elem_to_f32<XDT>(sinr[c + 32]);
  }
}

template <int NREP, int XDT>
__device__ __forceinline__ void fused_spikes(const FusedIn<XDT> &in, int t, int wave, int lane,
                                             uint64_t *fw) {
  const int c = lane & 31;
#pragma unroll
  for (int r = 0; r < (NREP + 2 + 7) / 8; ++r) {
    const int hi = r * 8 + wave * 2 + (lane >> 5);
    const bool rope = hi <= NREP;  // q and k heads; v has none
    bool s_lo = false, s_hi = false;
    float ulo = 0.f, uhi = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxFusedT; ++k) {
      if (k > t) break;
      float lo = elem_to_f32<XDT>(in.xl[r][k]), hi2 = elem_to_f32<XDT>(in.xh[r][k]);
      if (rope) {
        const float rl = round_to<XDT>(round_to<XDT>(lo * in.clo[r]) + round_to<XDT>(-hi2 * in.slo[r]));
        const float rh = round_to<XDT>(round_to<XDT>(hi2 * in.chi[r]) + round_to<XDT>(lo * in.shi[r]));
        lo = rl;
        hi2 = rh;
      }
      s_lo = lif_step(ulo, lo, in.blo[r], in.tlo[r]);
      s_hi = lif_step(uhi, hi2, in.bhi[r], in.thi[r]);
    }
    const uint64_t ml = __ballot(s_lo), mh = __ballot(s_hi);
    if (hi < NREP + 2 && c == 0) {
      const int sft = (lane >> 5) * 32;
      fw[hi] = ((ml >> sft) & 0xffffffffull) | (((mh >> sft) & 0xffffffffull) << 32);
    }
  }
}

// XDT = 0: queries come packed in p.q.  XDT = SPK_BF16 / SPK_F16: the fused
// path, which derives this unit's q and current k/v spikes from p.fz
// (head_dim 64 only).  W64 = head_dim / 64 (1 or 2).
template <int NREP, int XDT, int W64, int KW>
__global__ __launch_bounds__(KW * 64) __attribute__((amdgpu_waves_per_eu(XDT == 0 && W64 == 1 ? 4 : 3))) void decode_attn_mfma_kernel(AttnParams p) {
  static_assert(W64 == 1 || (W64 == 2 && XDT == 0), "fused path: head_dim 64 only");
  static_assert(KW == kWaves || (KW == 2 && XDT == 0 && W64 == 1), "2-wave launch: plain path, head_dim 64");
  // Unplanned launch: x = (sequence, timestep, kv head) unit, y = partition.
  // Either way consecutive block ids (dealt round-robin to the 8 XCDs) are
  // sibling units of equal length.
  // Pair mode (PAIRS: the 4-wave plain kernel): a short item's units run two
  // waves each, two units per workgroup (waves 2s, 2s + 1: unit 2 * pair + s).
  constexpr bool PAIRS = KW == 4 && XDT == 0 && W64 == 1;
  const int units = p.N * p.T * p.Hkv;
  const int ups = p.T * p.Hkv;  // units per item
  int unit = blockIdx.x, part = blockIdx.y;
  int planned_len = 0;  // planned launch: the chosen item's sequence length
  bool pair = false;
  int pj = 0;  // pair mode: the unit pair of the item
  __shared__ __align__(16) char smem[kSmemBytes<W64, KW>];
  if (p.plan_inline) {  // planned launch: longest work items first
    int sub;
    const int i = plan_slot<KW, PAIRS>(p, blockIdx.x, ups, reinterpret_cast<int *>(smem), &planned_len,
                                       &sub, &pair);
    if (i < 0) return;
    unit = (i % p.N) * ups + (pair ? 0 : sub);
    pj = sub;
    part = i / p.N;
  } else if (p.order) {
    // The planner's entry for this block (see decode_attn_plan).
    if ((int)blockIdx.x >= p.order[units * p.num_parts]) return;
    const int e = p.order[blockIdx.x];
    const int rest = e & ((1 << 30) - 1);
    const int item = rest / ups, sub = rest - item * ups;
    pair = PAIRS && ((e >> 30) & 1);
    pj = sub;
    part = item / p.N;
    unit = (item % p.N) * ups + (pair ? 0 : sub);
  }
  const int n = unit / ups;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const int len = p.plan_inline ? planned_len : seq_len(p, n);
  const int nparts_seq = len <= 0 ? 1 : (len + p.part_len - 1) / p.part_len;
  if (part >= nparts_seq) return;
  const int start = part * p.part_len;
  const int end = min(len, start + p.part_len);
  if constexpr (PAIRS) {
    // An unplanned 4-wave launch (the partials entry past kInlinePlanItems
    // items) pairs a short item's units too, so it keeps the 2-wave order:
    // the block of even unit 2s runs units 2s and 2s + 1, the odd one exits.
    if (!p.plan_inline && !p.order && end - start <= kPairMaxLen) {
      if ((unit % ups) & 1) return;
      pair = true;
      pj = (unit % ups) >> 1;
    }
  }
  int my_r = unit % ups;  // this wave's unit within the item
  bool has_unit = true;
  if (pair) {
    my_r = 2 * pj + (wave >> 1);
    has_unit = my_r < ups;  // an odd ups leaves the last pair half empty
  }
  // (wave-uniform; readfirstlane keeps the cache addresses in scalar registers)
  const int kvh = __builtin_amdgcn_readfirstlane((has_unit ? my_r : 0) % p.Hkv);
  const int t = __builtin_amdgcn_readfirstlane((has_unit ? my_r : 0) / p.Hkv);
  // Short items (at most kPairMaxLen tokens, head_dim 64) sum in the 2-wave
  // order in every launch: the 2-wave launch, pairs in the 4-wave plain
  // kernel, and in the fused kernel waves 0 and 1 alone (waves 2 and 3 only
  // help derive the spikes).
  const bool half = XDT != 0 && end - start <= kPairMaxLen;
  const int kw_unit = KW == 2 || pair || half ? 2 : KW;  // waves per unit
  const int wave_in = pair ? (wave & 1) : wave;         // wave index within the unit
  const int leader = pair ? (wave & 2) : 0;             // the unit's reducing wave
  if (half && wave >= 2) has_unit = false;              // (its spike work is done above the loop)

  FusedIn<XDT == 0 ? SPK_BF16 : XDT> fin;
  if constexpr (XDT != 0) fused_load<NREP, XDT>(p, n, t, kvh, wave, lane, fin);

  __shared__ uint32_t tab[kDigitEntries];     // per d: 4 e4m3 digits of exp(-d*scale)
  __shared__ int32_t blocks[kMaxPartBlocks];  // this partition's physical blocks
  WaveStage<W64> &st = reinterpret_cast<WaveStage<W64> *>(smem)[wave];

  if (tid <= 64 * W64) tab[tid] = p.digits[tid];
  const int nblk = end > start ? ((end - start - 1) >> p.bs_log2) + 1 : 0;
  const int blk0 = start >> p.bs_log2;
  // Physical blocks outside the cache are replaced by block 0 here, once, so
  // the loads below never leave [0, num_slots) (a pair never straddles a block).
  const uint32_t num_blocks = static_cast<uint32_t>(min<int64_t>(p.num_slots >> p.bs_log2, 0xffffffffll));
  for (int b = tid; b < nblk; b += KW * 64) {
    const uint32_t phys = static_cast<uint32_t>(p.bt[n * p.bts0 + (blk0 + b) * p.bts1]);
    blocks[b] = static_cast<int32_t>(phys < num_blocks ? phys : 0u);
  }

  uint32_t q[2 * W64][8];  // q[w][h]: 32-bit word w of head h's packed query
  __shared__ uint64_t fw[10];  // fused path: packed spikes of the unit's q heads, then k, v
  if constexpr (XDT == 0) {
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      const uint32_t *qp = p.q + t * p.qs0 + n * p.qs1 + (kvh * NREP + h) * p.qs2;
#pragma unroll
      for (int w = 0; w < 2 * W64; ++w)  // wave-uniform: kept in SGPRs
        q[w][h] = h < NREP ? static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(qp[w]))) : 0u;
    }
  }
  __syncthreads();
  uint64_t kcur = 0, vcur = 0;  // fused path: the current token's k/v words
  bool subst = false;            // ... used in place of the loaded ones
  const uint64_t *kbase = reinterpret_cast<const uint64_t *>(p.k + t * p.ks0 + kvh * p.ks1);
  const uint64_t *vbase = reinterpret_cast<const uint64_t *>(p.v + t * p.vs0 + kvh * p.vs1);
  const int bs_mask = (1 << p.bs_log2) - 1;

  // Tokens j, j+1 of this partition (j even, same block as block_size >= 2)
  // -> their K/V words, W64 16-byte loads each (the pair's 16 * W64 bytes are
  // contiguous).  Pairs past the partition re-read its last pair (clamped) so
  // the loads stay unconditional; the staged block ids are inside the cache,
  // so every slot is.
  const int last_pair = (end - 1) & ~1;
  // Element offset (in u64 words / W64) of the pair's first slot.
  // Byte offset of the pair's words in its (t, kv head) slab (the host keeps
  // every slab under 4 GiB, so offsets are 32-bit and the loads are buffer
  // loads from a scalar base: no 64-bit address arithmetic per step).
  constexpr int kSlotShift = W64 == 1 ? 3 : 4;  // log2(bytes per token)
  auto slot_of = [&](int j) -> uint32_t {
    const int jj = min(j, last_pair);
    const uint32_t phys = static_cast<uint32_t>(blocks[(jj - start) >> p.bs_log2]);
    return ((phys << p.bs_log2) | static_cast<uint32_t>(jj & bs_mask)) << kSlotShift;
  };
  const auto krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t *>(kbase), 0, 0x7fffffff, 0x00020000);
  const auto vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t *>(vbase), 0, 0x7fffffff, 0x00020000);
  auto issue = [&](uint32_t off, uint64_t (&kw)[2][W64], uint64_t (&vw)[2][W64]) {
    typedef unsigned long long v2u64 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int i = 0; i < W64; ++i) {  // u64 2i, 2i+1 of the pair: token (2i+c)/W64, word (2i+c)%W64
      // aux 2: the nontemporal hint of the earlier global loads
      const v2u64 k2 = __builtin_bit_cast(v2u64, __builtin_amdgcn_raw_buffer_load_b128(krs, off + 16 * i, 0, 2));
      const v2u64 v2 = __builtin_bit_cast(v2u64, __builtin_amdgcn_raw_buffer_load_b128(vrs, off + 16 * i, 0, 2));
      kw[(2 * i) / W64][(2 * i) % W64] = k2.x;
      kw[(2 * i + 1) / W64][(2 * i + 1) % W64] = k2.y;
      vw[(2 * i) / W64][(2 * i) % W64] = v2.x;
      vw[(2 * i + 1) / W64][(2 * i + 1) % W64] = v2.y;
    }
  };
  auto load = [&](int j, uint64_t (&kw)[2][W64], uint64_t (&vw)[2][W64]) { issue(slot_of(j), kw, vw); };

  v4f acc[2][4 * W64] = {}, accl[2] = {};

  const int kStride = kw_unit * kStepTokens;
  const int first = start + wave_in * kStepTokens;
  const int span = has_unit ? end - first : 0;
  const int nfull = span > 0 ? (span / kStride) + ((span % kStride) >= kStepTokens ? 1 : 0) : 0;
  const int ntotal = span > 0 ? (span + kStride - 1) / kStride : 0;

  const int cur_pair = (len - 1) & ~1, cur_e = (len - 1) & 1;
  constexpr int kRT = NREP > 4 ? 2 : 1;
  StepOps<W64> ops = {};  // zero before the first step: its MFMAs add nothing
  // The denominators' constant B operand (fp4 1.0 in every nibble), made
  // opaque so it stays in four VGPRs for the whole loop: as a literal the
  // compiler rebuilt it from SGPRs every step (two 64-bit moves a step;
  // config 4 120.05 -> 119.25 us, ten interleaved runs).
  v4i_ ones = {0x11111111, 0x11111111, 0x11111111, 0x11111111};
  asm volatile("" : "+v"(ones));
  auto step = [&](const uint64_t (&kin)[2][W64], const uint64_t (&vin)[2][W64], bool masked, int j0,
                  auto &&after_stage) {
    // Nothing of this step moves ahead of the previous one: left free, the
    // scheduler hoists a later step's popcounts next to its just-issued loads
    // and the wait for them empties the prefetch ring (measured: -3.5 %).
    __builtin_amdgcn_sched_barrier(0);
    uint64_t kw[2][W64], vw[2][W64];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int w = 0; w < W64; ++w) {
        kw[e][w] = kin[e][w];
        vw[e][w] = vin[e][w];
      }
    if constexpr (XDT != 0) {  // the current token's words, not yet in the cache
      if (subst && min(j0 + 2 * lane, last_pair) == cur_pair) {
        kw[cur_e][0] = kcur;
        vw[cur_e][0] = vcur;
      }
    }
    if (!masked) {
      const bool all[2] = {true, true};
      stage_step<NREP, W64, false>(st, lane, kw, vw, all, q, tab);
    } else {
      const bool valid[2] = {j0 + 2 * lane < end, j0 + 2 * lane + 1 < end};
      stage_step<NREP, W64, true>(st, lane, kw, vw, valid, q, tab);
    }
    after_stage();  // this step's words are consumed: the ring buffer takes new loads
    // The previous step's MFMAs (operands already in registers) interleave
    // with this step's popcounts and staging writes.
    mma_ops<kRT, W64>(ops, acc, accl, ones);
    wave_sync();
    read_ops<kRT, W64>(st, lane, ops);
    wave_sync();
  };

  uint64_t k0[2][W64], v0[2][W64], k1[2][W64], v1[2][W64];
  const int lo = 2 * lane;
  // A wave with no tokens (short or empty partition) issues no loads: only
  // then is every pair index inside the staged block range [0, nblk).
  if (ntotal > 0) {
    load(first + lo, k0, v0);
    load(first + kStride + lo, k1, v1);
  }
  // Fused path: the spikes, computed while those first loads are in flight.
  if constexpr (XDT != 0) {
    fused_spikes<NREP, XDT>(fin, t, wave, lane, fw);
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      q[0][h] = h < NREP ? static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(fw[h]))) : 0u;
      q[1][h] = h < NREP ? static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(fw[h] >> 32))) : 0u;
    }
    kcur = fw[NREP];
    vcur = fw[NREP + 1];
    // The partition holding the current token (position len - 1) stores its
    // words in the token's cache slot, once per (t, kv head), and uses them
    // in registers where the block table maps that position to the same slot
    // (elsewhere it reads the cache, as the two separate launches would).
    const int cur = len - 1;
    if (cur >= start && cur < end) {
      const int64_t slot = p.fz.slots[n];
      if (slot >= 0 && slot < p.num_slots) {
        if (tid == 0) {
          *reinterpret_cast<uint64_t *>(p.fz.k_out + t * p.ks0 + kvh * p.ks1 + slot * p.ks2) = kcur;
          *reinterpret_cast<uint64_t *>(p.fz.v_out + t * p.vs0 + kvh * p.vs1 + slot * p.vs2) = vcur;
        }
        const uint32_t phys = static_cast<uint32_t>(blocks[(cur - start) >> p.bs_log2]);
        const int64_t tslot = (static_cast<int64_t>(phys) << p.bs_log2) | (cur & ((1 << p.bs_log2) - 1));
        subst = tslot == slot;
      }
    }
  }
  // Two register buffers in a fixed ring: a step consumes its buffer, then
  // refills it with the loads of the step after next, whose slot was read
  // from the staged block table one step earlier (so the load address never
  // waits behind this step's LDS traffic).
  auto none = [] {};
  int i = 0;
  // The slot of this lane's pair at step s (token first + s * kStride + lo).
  // In the 4-wave kernel, when the block size divides the step's token
  // stride, the lane's block moves by a constant each step and its offset in
  // the block stays: an add, a clamp into the staged table, one LDS read and
  // a merge (5 VALU a step fewer than slot_of; config 4 120.7 -> 120.4 us,
  // fixed 8k 56.05 -> 55.6 us, twelve interleaved runs).  Steps past the
  // partition clamp to its last staged block (inside the cache; their words
  // are never used).  Called only when the wave has steps (nblk >= 1).  The
  // 2-wave kernel keeps slot_of: there the extra registers cost config 3
  // 4.7 %.
  const bool stride_blocks = KW == 4 && kStride >= (1 << p.bs_log2);
  const int lb4 = ((first + lo - start) >> p.bs_log2) * 4;  // byte offset in blocks[] at step 0
  const int sb4 = (kStride >> p.bs_log2) * 4;
  const int last4 = (nblk - 1) * 4;
  const uint32_t lane_low = static_cast<uint32_t>((first + lo) & bs_mask) << kSlotShift;
  // The main loop, instantiated for both slot forms (a branch per step
  // splits the loop body and costs registers).
  auto main_loop = [&](auto fast) {
  auto slot_step = [&](int st_i) -> uint32_t {
    if constexpr (!decltype(fast)::value) {
      return slot_of(first + st_i * kStride + lo);
    } else {
      const int b4 = min(lb4 + st_i * sb4, last4);
      const uint32_t phys = *reinterpret_cast<const uint32_t *>(reinterpret_cast<const char *>(blocks) + b4);
      return (phys << (p.bs_log2 + kSlotShift)) | lane_low;
    }
  };
  uint32_t snext = ntotal > 0 ? slot_step(2) : 0;
  for (; i + 2 <= nfull; i += 2) {
    // Waves with more steps left issue first (s_setprio): the longer units of
    // a CU's mix keep their pace as it drains.  Measured: config 4 119.2 ->
    // 118.6 us, fixed 8k 56.3 -> 55.7 us (medians, one box).
    const int rem = ntotal - i;  // wave-uniform
    if (rem > 48) __builtin_amdgcn_s_setprio(3);
    else if (rem > 24) __builtin_amdgcn_s_setprio(2);
    else if (rem > 8) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
    step(k0, v0, false, first + i * kStride, [&] {
      issue(snext, k0, v0);
      snext = slot_step(i + 3);
    });
    step(k1, v1, false, first + (i + 1) * kStride, [&] {
      issue(snext, k1, v1);
      snext = slot_step(i + 4);
    });
  }
  };
  if constexpr (KW == 4) {
    if (stride_blocks) main_loop(std::true_type{});
    else main_loop(std::false_type{});
  } else {
    main_loop(std::false_type{});
  }
  if (i < nfull) step(k0, v0, false, first + i * kStride, none);
  if (nfull < ntotal) {  // the partial last step: buffer nfull % 2
    const int j0 = first + nfull * kStride;
    if (nfull % 2 == 0) step(k0, v0, true, j0, none);
    else step(k1, v1, true, j0, none);
  }

  mma_ops<kRT, W64>(ops, acc, accl, ones);  // the last staged step

  // Per lane: row tile rt holds head 4rt + lane/16 with its four digits in
  // acc[rt][c][d] (digit d carries 2^-(8+4d)); column lane%16 of channel
  // tile c = 4*hv + ts is channel 64*hv + 4*(lane%16) + ts, whose set bits
  // were 0.5, 1.0, 2.0, 2.0 for ts = 0..3 (the ones tile: 0.5).
  constexpr int kVals = 8 * W64;  // values per lane: 2 row tiles x 4 W64 channel tiles
  float val[kVals], lh[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    float l = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) l += accl[rt][d] * ldexpf(1.f, -(7 + 4 * d));
    lh[rt] = l;
#pragma unroll
    for (int c = 0; c < 4 * W64; ++c) {
      const int ts = c & 3;
      const float m = ts == 0 ? 1.f : (ts == 1 ? 0.5f : 0.25f);
      float a = 0.f;
#pragma unroll
      for (int d = 0; d < 4; ++d) a += acc[rt][c][d] * (m * ldexpf(1.f, -(7 + 4 * d)));
      val[4 * W64 * rt + c] = a;
    }
  }

  // Cross-wave reduction (fixed order) through LDS: a wave writes its values
  // into its own stage, which no other wave reads (so no barrier before the
  // writes), and each unit's leader adds its other waves' values in wave
  // order after one barrier.
  constexpr int kRed = kVals + 2;
  static_assert(64 * kRed * 4 <= (int)sizeof(WaveStage<W64>), "a wave's values fit its stage");
  auto red_of = [&](int w) { return reinterpret_cast<float *>(smem + w * sizeof(WaveStage<W64>)) + lane * kRed; };
  if (wave != leader) {
    float *dst = red_of(wave);
#pragma unroll
    for (int k = 0; k < kVals; ++k) dst[k] = val[k];
#pragma unroll
    for (int k = 0; k < 2; ++k) dst[kVals + k] = lh[k];
  }
  __syncthreads();
  if (wave != leader || !has_unit) return;
  for (int w = leader + 1; w < leader + kw_unit; ++w) {
    const float *src = red_of(w);
#pragma unroll
    for (int k = 0; k < kVals; ++k) val[k] += src[k];
#pragma unroll
    for (int k = 0; k < 2; ++k) lh[k] += src[kVals + k];
  }

  const bool single = nparts_seq == 1 && !p.partials_only;
  if (single && p.out_vec) {
    // A lane's values of one head are 4 consecutive channels per 64-channel
    // group: one 16-byte (fp32) or 8-byte (16-bit) store each.
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int h = 4 * rt + (lane >> 4);
      if (h >= NREP) continue;
      const int64_t row = t * p.os0 + n * p.os1 + (kvh * NREP + h) * p.os2;
#pragma unroll
      for (int g = 0; g < W64; ++g) {
        float o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = len <= 0 ? 0.f : val[4 * W64 * rt + 4 * g + c] / lh[rt];
        const int64_t at = row + 64 * g + 4 * (lane & 15);
        if (p.out_dtype == SPK_F32) {
          *reinterpret_cast<v4f *>(static_cast<float *>(p.out) + at) = v4f{o[0], o[1], o[2], o[3]};
        } else {
          typedef unsigned v2u __attribute__((ext_vector_type(2)));
          uint32_t w[2];
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            uint16_t lo, hi;
            if (p.out_dtype == SPK_BF16) {
              lo = f32_to_bf16_bits(o[2 * c]);
              hi = f32_to_bf16_bits(o[2 * c + 1]);
            } else {
              lo = __builtin_bit_cast(uint16_t, static_cast<_Float16>(o[2 * c]));
              hi = __builtin_bit_cast(uint16_t, static_cast<_Float16>(o[2 * c + 1]));
            }
            w[c] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
          }
          *reinterpret_cast<v2u *>(static_cast<uint16_t *>(p.out) + at) = v2u{w[0], w[1]};
        }
      }
    }
    return;
  }
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int h = 4 * rt + (lane >> 4);
    if (h >= NREP) continue;
    const int hq = kvh * NREP + h;
#pragma unroll
    for (int c = 0; c < 4 * W64; ++c) {
      const int ch = 64 * (c >> 2) + 4 * (lane & 15) + (c & 3);
      const float a = val[4 * W64 * rt + c];
      if (single) {
        const float o = len <= 0 ? 0.f : a / lh[rt];
        store_f32_as(p.out, t * p.os0 + n * p.os1 + hq * p.os2 + ch * p.os3, p.out_dtype, o);
      } else {  // partials: head_dim values, then the denominator
        float *dst = p.ws + ((((int64_t)part * p.T + t) * p.N + n) * p.Hq + hq) * (64 * W64 + 1);
        dst[ch] = a;
        if (ch == 0) dst[64 * W64] = lh[rt];
      }
    }
  }
}

}  // namespace mfma

// x to OCP e4m3 (bias 7, subnormal step 2^-9, sign bit 0x80), round to
// nearest even; returns the code and stores the value it encodes.  The digit
// split feeds it signed residuals (rounding up leaves a negative remainder).
static uint32_t e4m3_encode(float x, float *val) {
  const uint32_t sign = x < 0.f ? 0x80u : 0u;
  const float a = std::fabs(x);
  float v;
  uint32_t code;
  if (!(a > 0.f)) {
    v = 0.f;
    code = 0;
  } else if (a < 0.015625f) {  // below 2^-6: subnormal
    const float m = std::nearbyint(a * 512.f);
    if (m >= 8.f) { v = 0.015625f; code = 0x08; }
    else { v = m * (1.f / 512.f); code = static_cast<uint32_t>(m); }
  } else {
    int e;
    std::frexp(a, &e);
    int E = e - 1;  // a in [2^E, 2^(E+1))
    float m = std::nearbyint((std::ldexp(a, -E) - 1.f) * 8.f);
    if (m >= 8.f) { m = 0.f; ++E; }
    if (E > 8) { E = 8; m = 6.f; }  // saturate at 448 (never reached: |x| <= 256)
    v = std::ldexp(1.f + m * 0.125f, E);
    code = static_cast<uint32_t>(((E + 7) << 3) | static_cast<int>(m));
  }
  *val = sign ? -v : v;
  return code | (code ? sign : 0u);
}

void build_digit_table(float scale, uint32_t digits[kDigitEntries]) {
  static thread_local float last_scale = -1.f;
  static thread_local uint32_t last[kDigitEntries];
  if (scale != last_scale) {
    for (int d = 0; d < kDigitEntries; ++d) {
      float x = std::exp(-static_cast<float>(d) * scale) * 256.f;
      uint32_t w = 0;
      for (int s = 0; s < 4; ++s) {
        float q;
        w |= e4m3_encode(x, &q) << (8 * s);
        x = (x - q) * 16.f;
      }
      last[d] = w;
    }
    last_scale = scale;
  }
  for (int d = 0; d < kDigitEntries; ++d) digits[d] = last[d];
}

bool mfma_path_supported(const AttnParams &p) {
  const auto al16 = [](const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  const int w32 = p.head_dim / 32;  // 32-bit words per token: slots must be dense
  return (p.head_dim == 64 || p.head_dim == 128) && p.nrep <= 8 && p.bs_log2 >= 1 &&
         p.ks2 == w32 && p.vs2 == w32 &&
         (p.ks0 % 4) == 0 && (p.ks1 % 4) == 0 && (p.vs0 % 4) == 0 && (p.vs1 % 4) == 0 &&
         al16(p.k) && al16(p.v) &&
         // a (t, kv head) slab within the 2 GiB of the kernel's buffer loads
         p.num_slots <= (int64_t(0x7fffffff) >> (p.head_dim == 64 ? 3 : 4)) &&
         ((p.part_len + (1 << p.bs_log2) - 1) >> p.bs_log2) <= mfma::kMaxPartBlocks;
}

namespace mfma {

// Longest-processing-time-first launch order, written by one workgroup for
// launches with more items than plan_slot handles.  The same order as
// plan_slot: items by the steps each of their waves takes (bucket from
// plan_bucket; `pairs` as PAIRS there), largest first, the blocks of an item
// adjacent.  Entry order[b] = (item * UPS + sub) | (paired << 30), item = part
// * N + sequence, sub = the unit, or the unit pair of a paired item.  Items
// past a sequence's length are left out (their blocks exit); order[N * UPS *
// num_parts] gets the number of entries.  Ties are placed in arbitrary order:
// each item computes the same sums wherever it runs, so outputs do not depend
// on it.
__global__ __launch_bounds__(1024) void decode_attn_plan(const int32_t *lens, int ctx_cap, int N, int UPS,
                                                        int part_len, int num_parts, int pairs,
                                                        int32_t *order) {
  __shared__ int count[kMaxBuckets];
  __shared__ int offset[kMaxBuckets];
  const int tid = threadIdx.x;
  const int A = (UPS + 1) >> 1;
  const int nb = 2 * (((max(part_len, pairs ? 2 * kPairMaxLen : 0) + 255) >> 8) + 2);
  for (int b = tid; b < nb; b += blockDim.x) count[b] = 0;
  __syncthreads();
  auto bucket = [&](int len, int part) {
    const int size = min(part_len, len - part * part_len);
    return pairs ? plan_bucket<true>(size) : plan_bucket<false>(size);
  };
  auto bpi = [&](int bk) { return (bk & 1) ? A : UPS; };
  auto exists = [&](int len, int part) {
    const int nparts = len <= 0 ? 1 : (len + part_len - 1) / part_len;
    return part < nparts;
  };
  for (int i = tid; i < N * num_parts; i += blockDim.x) {
    const int n = i % N, part = i / N;
    const int len = min(lens[n], ctx_cap);
    if (exists(len, part)) {
      const int bk = bucket(len, part);
      atomicAdd(&count[bk], bpi(bk));
    }
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int b = nb - 1; b >= 0; --b) {
      offset[b] = run;
      run += count[b];
    }
    order[N * UPS * num_parts] = run;
  }
  __syncthreads();
  for (int i = tid; i < N * num_parts; i += blockDim.x) {
    const int n = i % N, part = i / N;
    const int len = min(lens[n], ctx_cap);
    if (!exists(len, part)) continue;
    const int bk = bucket(len, part);
    const int at = atomicAdd(&offset[bk], bpi(bk));
    for (int sub = 0; sub < bpi(bk); ++sub) order[at + sub] = (i * UPS + sub) | ((bk & 1) << 30);
  }
}

}  // namespace mfma

void launch_decode_mfma(AttnParams p, bool plan, int32_t *order, hipStream_t s, int fused_dtype,
                        int waves) {
  const bool two = waves == 2 && fused_dtype == 0 && p.head_dim == 64;
  const int threads = (two ? 2 : mfma::kWaves) * 64;
  const int units = p.N * p.T * p.Hkv;
  dim3 grid(units, p.num_parts);
  p.order = nullptr;
  p.plan_inline = 0;
  const bool pairs = !two && fused_dtype == 0 && p.head_dim == 64;  // as PAIRS in the kernel
  // A planned launch whose table holds at most kPairMaxLen tokens has only
  // paired items: ceil(T * Hkv / 2) workgroups each, no more.
  const int planned_blocks = pairs && p.ctx_cap <= kPairMaxLen
                                 ? p.N * p.num_parts * ((p.T * p.Hkv + 1) / 2)
                                 : units * p.num_parts;
  if (plan && !order) {
    p.plan_inline = 1;
    grid = dim3(planned_blocks);
  } else if (plan) {
    mfma::decode_attn_plan<<<1, 1024, 0, s>>>(p.lens, p.ctx_cap, p.N, p.T * p.Hkv, p.part_len, p.num_parts,
                                              pairs ? 1 : 0, order);
    p.order = order;
    grid = dim3(planned_blocks);
  }
#define SPK_NREP_CASES(XDT, W64, KW)                                                              \
  switch (p.nrep) {                                                                               \
    case 1: mfma::decode_attn_mfma_kernel<1, XDT, W64, KW><<<grid, threads, 0, s>>>(p); break;    \
    case 2: mfma::decode_attn_mfma_kernel<2, XDT, W64, KW><<<grid, threads, 0, s>>>(p); break;    \
    case 3: mfma::decode_attn_mfma_kernel<3, XDT, W64, KW><<<grid, threads, 0, s>>>(p); break;    \
    case 4: mfma::decode_attn_mfma_kernel<4, XDT, W64, KW><<<grid, threads, 0, s>>>(p); break;    \
    case 5: mfma::decode_attn_mfma_kernel<5, XDT, W64, KW><<<grid, threads, 0, s>>>(p); break;    \
    case 6: mfma::decode_attn_mfma_kernel<6, XDT, W64, KW><<<grid, threads, 0, s>>>(p); break;    \
    case 7: mfma::decode_attn_mfma_kernel<7, XDT, W64, KW><<<grid, threads, 0, s>>>(p); break;    \
    default: mfma::decode_attn_mfma_kernel<8, XDT, W64, KW><<<grid, threads, 0, s>>>(p); break;   \
  }
  if (fused_dtype == SPK_BF16) {  // the caller allows the fused path at head_dim 64 only
    SPK_NREP_CASES(SPK_BF16, 1, 4)
  } else if (fused_dtype == SPK_F16) {
    SPK_NREP_CASES(SPK_F16, 1, 4)
  } else if (p.head_dim == 128) {
    SPK_NREP_CASES(0, 2, 4)
  } else if (two) {
    SPK_NREP_CASES(0, 1, 2)
  } else {
    SPK_NREP_CASES(0, 1, 4)
  }
#undef SPK_NREP_CASES
}

}  // namespace spk
