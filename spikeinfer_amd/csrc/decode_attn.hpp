// Parameters and helpers shared by the two decode-attention paths
// (decode_attn.hip: general VALU path; decode_attn_mfma.hip: matrix cores).
#pragma once

#include "common.hpp"

#include <cstdlib>
#include <cstring>

namespace spk {

constexpr int kAttnThreads = 256;   // 4 waves
// Block-table entries of one partition staged in LDS by the matrix-core
// kernel; choose_part_len never makes a partition span more blocks.
constexpr int kMaxStagedBlocks = 2048;
// Matrix-core path: items (partitions) of at most this many tokens sum their
// tokens in the order of the 2-wave launch -- two waves per unit, 128-token
// steps alternating -- in every launch shape (the 4-wave kernel runs two such
// units per workgroup); longer items use four waves per unit.  The order is a
// function of the item's own size, so a sequence's output does not depend on
// the batch.
constexpr int kPairMaxLen = 8192;
constexpr int kMaxRep = 16;
constexpr int kMaxFusedT = 8;  // timesteps the fused q/k/v path keeps in registers
constexpr int kDigitEntries = 129;  // d = 0..128 (head_dim 64 or 128)

// Inputs of the fused q/k/v-spike path (spk_qkv_decode_attn): the q/k/v
// projection currents of the decode tokens, from which each workgroup derives
// its own heads' spikes (RoPE -> LIF), writing the current token's k/v words
// to the cache.
struct FusedParams {
  const void *x;            // [T, n_tok, (Hq + 2 Hkv) * 64] currents (bf16 or f16)
  int64_t xs0, xs1;         // timestep and token strides, in elements
  const void *cos, *sin;    // [table_rows, 64] rotary tables of x's dtype
  const int64_t *pos;       // [n_tok] positions (rows of the tables)
  int64_t table_rows;
  const void *beta, *th;    // [3, 64]: q, k and v sites
  int param_dtype;
  const int64_t *slots;     // [n_tok] cache slot of each token's k/v words
  uint32_t *k_out, *v_out;  // the caches (same layout as AttnParams::k / v)
};

struct AttnParams {
  const uint32_t *q;
  int64_t qs0, qs1, qs2;
  const uint32_t *k;
  int64_t ks0, ks1, ks2;
  const uint32_t *v;
  int64_t vs0, vs1, vs2;
  int64_t num_slots;
  const int32_t *bt;
  int64_t bts0, bts1;
  const int32_t *lens;
  void *out;
  int out_dtype;
  int64_t os0, os1, os2, os3;
  int T, N, Hq, Hkv, head_dim, bs_log2, nrep;
  // Tokens the block table can address (max_blocks * block_size, at most
  // INT_MAX): every kernel reads seq_lens through seq_len(), which clamps to
  // it, so a length past the table never indexes beyond the table's row or
  // the sized partitions.
  int ctx_cap;
  float scale;
  int part_len;      // tokens per partition (multiple of 256 and of block size)
  int num_parts;     // partitions per sequence at most
  float *ws;         // [num_parts][T][N][Hq][head_dim + 1] partial sums
  // Optional launch order (matrix-core path, split contexts): order[b] is the
  // work item (part * units + unit) of block b, longest first; order[items]
  // holds the number of items.  nullptr: block (unit, part) = (x, y).
  const int32_t *order;
  // Matrix-core path: the main kernel computes the longest-first order itself
  // (N * num_parts <= kInlinePlanItems) instead of reading `order`.
  int plan_inline;
  // Every (sequence, partition) writes its partial sums to `ws`, also when the
  // sequence has a single partition (spk_decode_attn_partials); the combine
  // then normalises every row.
  int partials_only;
  // The output rows take whole 4-channel vectors: fp32/bf16/f16 out, unit
  // channel stride, the other strides multiples of 4 and `out` 16-byte
  // aligned (the matrix-core epilogue then stores 16 or 8 bytes a lane).
  int out_vec;
  // Matrix-core path: for d = popc(q & ~k) in 0..head_dim (<= 128), the four
  // e4m3 digits of exp(-d*scale) * 2^8 (byte s weighs 2^-(4s)), built on the
  // host once per scale (build_digit_table) and copied into LDS by every
  // workgroup.
  uint32_t digits[kDigitEntries];
  FusedParams fz;  // used by the fused instantiations only
};

// Length of sequence n as the kernels use it: seq_lens[n] clamped to the
// tokens the block table can address.
__device__ __forceinline__ int seq_len(const AttnParams &p, int n) { return min(p.lens[n], p.ctx_cap); }

// Fills digits[0..128] for `scale` (host; reuses the last table when unchanged).
void build_digit_table(float scale, uint32_t digits[kDigitEntries]);

// Partition length: 32768 tokens, or fewer when a partition would stage
// more than kMaxStagedBlocks block-table entries.  It depends on the block
// size only -- never on the batch -- so a sequence is cut (and its sums
// ordered) the same way whatever else is decoded with it.
inline int choose_part_len(int block_size) {
  int part = 32768;
  while (part > block_size * kMaxStagedBlocks && part > 256) part >>= 1;
  return part < block_size ? block_size : part;  // partitions start on a block
}

// Matrix-core path for head_dim 64, n_rep <= 8 (decode_attn_mfma.hip).
// Returns false when the shape or alignment does not qualify.
bool mfma_path_supported(const AttnParams &p);
// Contexts from 3072 tokens (table capacity, plan_launch) are launched
// longest first.  Up to kInlinePlanItems (sequence, partition) items the main
// kernel orders them itself; beyond, a planner kernel first writes the order
// into `order` (items + 1 ints of workspace, plan_in_workspace).  Below the
// threshold the plan's prologue costs more than the order gains (measured:
// ragged contexts up to 2000 tokens 15.2 -> 16.7 us with a plan, up to 4000
// 24.1 -> 22.1 us).
inline bool plan_launch(int64_t ctx_max) { return ctx_max >= 3072; }
constexpr int kInlinePlanItems = 4096;
// SPIKEINFER_AMD_ATTN_PLAN=workspace forces the planner kernel for any
// planned launch (tests check that both orders give the same bytes).
inline bool plan_in_workspace(int64_t ctx_max, int64_t items) {
  const char *e = getenv("SPIKEINFER_AMD_ATTN_PLAN");
  const bool force = e && strcmp(e, "workspace") == 0;
  return plan_launch(ctx_max) && (items > kInlinePlanItems || force);
}
// Launches the matrix-core kernel; `plan` orders it longest first, from
// `order` when not null (after the planner kernel fills it: items * T * Hkv
// + 1 ints), else in-kernel.
// fused_dtype: 0 for q from p.q, else the dtype (SPK_BF16 / SPK_F16) of p.fz.x.
// waves: 4, or 2 for the short-context launch (plain path, head_dim 64 only;
// otherwise 4 is used).
void launch_decode_mfma(AttnParams p, bool plan, int32_t *order, hipStream_t s, int fused_dtype = 0,
                        int waves = 4);

}  // namespace spk
