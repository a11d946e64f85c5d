/*
 * spikeinfer_amd.h -- C ABI of the MI355X (gfx950) spiking decode hot path.
 *
 * Two kernels families sit behind this ABI:
 *   - paged popcount decode attention over bit-packed spike keys/values;
 *   - the LIF neuron (multi-step membrane update, threshold, delayed subtract
 *     reset), optionally fused with bit-packing and the paged-cache scatter.
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers owned by the caller.  Nothing here
 *     allocates device memory; scratch space, where needed, is passed in.
 *   - Launches are asynchronous on `stream` (a hipStream_t, passed as void*);
 *     no entry point synchronises or reads device memory on the host, so every
 *     call may be recorded into a hipGraph.
 *   - Strides are in ELEMENTS of the tensor they describe.  Packed spike
 *     tensors are int32 words: bit i of word w is channel 32*w + i.  The last
 *     (word) axis of a packed tensor must be contiguous (stride 1).
 *   - Return value: 0 on success, SPK_EINVAL for a rejected argument,
 *     SPK_EUNSUPPORTED for a valid but unimplemented shape, SPK_EHIP when the
 *     HIP runtime reported an error.  spk_last_error() gives the message of
 *     the last failure on the calling thread.
 */
#ifndef SPIKEINFER_AMD_H
#define SPIKEINFER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum spk_status {
  SPK_OK = 0,
  SPK_EINVAL = 1,
  SPK_EUNSUPPORTED = 2,
  SPK_EHIP = 3,
};

/* Element types used by the dtype arguments. */
enum spk_dtype {
  SPK_F32 = 0,
  SPK_F16 = 1,
  SPK_BF16 = 2,
  SPK_U8 = 3,
  SPK_I32 = 4,
};

/* Message of the last failing call on this thread ("" if none). */
const char *spk_last_error(void);

/* ABI version, bumped on any signature change (2: spk_decode_advance draws; 3: spk_decode_attn_combine takes the partials size, spk_norm_* GEMMs). */
int spk_abi_version(void);

/*
 * Paged popcount decode attention, one query position per sequence.
 *
 * Replaces the Triton launch in paged_spike_attn_decode
 * (spikeinfer/kernels/spike_attention.py:153-221, kernel :67-150).
 *
 *   q        int32 [T, N, Hq, W]          packed query spikes (any strides,
 *                                         word axis contiguous)
 *   k, v     int32 [T, Hkv, slots, W]     paged packed caches
 *   block_tables int32 [N, max_blocks]    logical -> physical block
 *   seq_lens int32 [N]                    cached length incl. this token
 *   out      [T, N, Hq, head_dim]         out_dtype in {F32, F16, BF16}
 *
 * For sequence n, query head h, timestep t: kv head = h / (Hq/Hkv); token
 * position p < seq_lens[n] lives in slot block_tables[n][p/bs]*bs + p%bs; the
 * score is popcount(q & k) * scale; out = softmax(scores) @ unpacked(v).
 * W must equal ceil(head_dim/32); head_dim <= 128; block_size a power of two.
 * A sequence with seq_len <= 0 gets an all-zero output row; a seq_len past
 * max_blocks*block_size is clamped to it (the table addresses no more).  Slots outside
 * [0, num_slots) are never dereferenced, so a corrupt block table cannot
 * fault the GPU (the output rows of such a sequence are unspecified).  scale must satisfy
 * 0 < scale*head_dim <= 80 (the softmax uses the fixed offset popcount(q)).
 *
 * Precision: head_dim 64 or 128 with Hq/Hkv <= 8 runs on the matrix cores,
 * with each softmax weight exp(-d*scale) (d = popcount(q & ~k)) held as four
 * e4m3 digits: relative error <= ~1e-6 while the weight * 2^8 is in the e4m3
 * normal range, i.e. for every d at head_dim 64 and for d <= 109 at head_dim
 * 128 with scale 1/sqrt(128).  Beyond that (queries with nearly all 128 bits
 * set against keys far from them) the first digit is subnormal and the
 * relative error grows to ~4.5e-5 (worst at d = 123); outputs stay far inside
 * max-abs 1e-3.  Other shapes run the VALU path in fp32.
 *
 * `workspace` must hold spk_decode_attn_workspace_bytes(...) bytes (it may be
 * NULL when that is 0).  It holds per-partition partial sums when long
 * contexts are split across workgroups.
 */
int spk_decode_attn(const int32_t *q, const int64_t q_strides[4],
                    const int32_t *k_cache, const int64_t k_strides[4],
                    const int32_t *v_cache, const int64_t v_strides[4],
                    int64_t num_slots, const int32_t *block_tables, int64_t bt_stride0,
                    int64_t bt_stride1, const int32_t *seq_lens, void *out,
                    int out_dtype, const int64_t out_strides[4], int T, int N,
                    int Hq, int Hkv, int head_dim, int block_size,
                    int max_blocks, float scale, void *workspace,
                    size_t workspace_bytes, void *stream);

/*
 * spk_decode_attn without a workspace argument, for callers that cannot
 * allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  Same
 * arguments and results as spk_decode_attn; the partial sums and launch-order
 * list it may need live in a fixed device array of the library,
 * SPK_DECODE_ATTN_SCRATCH_BYTES per GPU (held until the process ends).
 * Shapes whose spk_decode_attn_workspace_bytes exceeds that are rejected with
 * SPK_EINVAL.  Calls allocate nothing; every call on one GPU shares that
 * GPU's array, so calls that overlap in time on one GPU (e.g. on two streams)
 * race and must be ordered by the caller.
 */
#define SPK_DECODE_ATTN_SCRATCH_BYTES (16u << 20)
int spk_decode_attn_noalloc(const int32_t *q, const int64_t q_strides[4],
                            const int32_t *k_cache, const int64_t k_strides[4],
                            const int32_t *v_cache, const int64_t v_strides[4],
                            int64_t num_slots, const int32_t *block_tables,
                            int64_t bt_stride0, int64_t bt_stride1,
                            const int32_t *seq_lens, void *out, int out_dtype,
                            const int64_t out_strides[4], int T, int N, int Hq,
                            int Hkv, int head_dim, int block_size, int max_blocks,
                            float scale, void *stream);

/* Bytes of workspace spk_decode_attn needs for this launch shape. */
size_t spk_decode_attn_workspace_bytes(int T, int N, int Hq, int Hkv,
                                       int head_dim, int block_size,
                                       int max_blocks);

/*
 * The split-context halves of spk_decode_attn as separate operators.  The
 * reference has no split (its kernel walks each context in one program,
 * spike_attention.py:67-150, docs/architecture.md:225-228); these exist so a
 * context split into partitions -- within one launch, or across launches or
 * devices -- can be combined by the caller.
 *
 * spk_decode_attn_partials: same inputs and indexing as spk_decode_attn; the
 * context of every sequence is cut into partitions of part_len tokens
 * (a multiple of block_size, at most 32768) and partition p of row (t, n, h)
 * writes, unnormalised,
 *   partials[(((p*T + t)*N + n)*Hq + h)*(head_dim + 1) + c] = sum_j w_j * v_j[c]
 *   ... + head_dim]                                        = sum_j w_j
 * with w_j = exp(-popcount(q & ~k_j) * scale), j over the partition's tokens.
 * The weights share the fixed offset popcount(q), so partials of any
 * partitioning add.  partials_bytes must cover
 * ceil(max_blocks*block_size / part_len) * T*N*Hq*(head_dim+1) floats;
 * partitions at or past a sequence's length are not written.
 *
 * spk_decode_attn_combine: out[t, n, h, c] = sum_p a / sum_p l over the
 * partitions p < ceil(seq_lens[n] / part_len) (at most num_parts), summed in
 * partition order; a sequence with seq_len <= 0 gets zeros.  partials_bytes
 * must cover num_parts * T*N*Hq*(head_dim+1) floats (SPK_EINVAL otherwise).
 */
int spk_decode_attn_partials(const int32_t *q, const int64_t q_strides[4],
                             const int32_t *k_cache, const int64_t k_strides[4],
                             const int32_t *v_cache, const int64_t v_strides[4],
                             int64_t num_slots, const int32_t *block_tables,
                             int64_t bt_stride0, int64_t bt_stride1,
                             const int32_t *seq_lens, int T, int N, int Hq, int Hkv,
                             int head_dim, int block_size, int max_blocks, float scale,
                             int part_len, float *partials, size_t partials_bytes,
                             void *stream);
int spk_decode_attn_combine(const float *partials, size_t partials_bytes, int num_parts,
                            int part_len, const int32_t *seq_lens, void *out, int out_dtype,
                            const int64_t out_strides[4], int T, int N, int Hq,
                            int head_dim, void *stream);

/*
 * Prefill reader: one sequence's first seq_len cached tokens as dense 0/1
 * spikes, K and V in one launch.  Replaces gather_kv_unpacked
 * (spikeinfer/kernels/spike_attention.py:224-244: slot-matrix index_select,
 * then unpack_spikes, once per cache).
 *
 *   k_cache, v_cache int32 [T, H, num_slots, W] at cache_strides (v_cache may
 *            be NULL, then v_out must be too)
 *   block_table  the sequence's row, n_table entries at stride bt_stride
 *   k_out, v_out [T, H, seq_len, head_dim] contiguous in out_dtype (any type)
 * Token p reads slot table[p/bs]*bs + p%bs; positions past the table or whose
 * block lies outside the cache read as zeros.
 */
int spk_gather_unpack(const int32_t *k_cache, const int32_t *v_cache,
                      const int64_t cache_strides[4], int64_t num_slots,
                      const int32_t *block_table, int64_t bt_stride, int n_table,
                      int seq_len, void *k_out, void *v_out, int out_dtype, int T,
                      int H, int head_dim, int block_size, void *stream);

/*
 * Raw integer attention scores popcount(q & k) for every (t, n, h, position
 * < seq_len), written to scores[((t*N + n)*Hq + h)*max_len + p] (positions at
 * or past seq_len are left untouched).  Same indexing as spk_decode_attn; used
 * to check the score path bit-exactly.  No reference counterpart: the Triton
 * kernel keeps scores in registers (spike_attention.py:113-123).
 */
int spk_decode_scores(const int32_t *q, const int64_t q_strides[4],
                      const int32_t *k_cache, const int64_t k_strides[4],
                      int64_t num_slots, const int32_t *block_tables, int64_t bt_stride0,
                      int64_t bt_stride1, const int32_t *seq_lens,
                      int32_t *scores, int max_len, int T, int N, int Hq,
                      int Hkv, int head_dim, int block_size, void *stream);

/*
 * Multi-step LIF over [T, M, N] (N = channel axis beta/threshold broadcast
 * over).  Replaces the Triton launch in lif_multistep
 * (spikeinfer/kernels/lif_triton.py:141-233, kernel :48-105).
 *
 *   x        x_dtype [T, M, N] at strides x_strides (elements)
 *   beta, threshold  param_dtype [N] contiguous; beta is clamped to [0, 1]
 *   mem0     F32 [M, N] contiguous initial membrane, or NULL for zeros
 *   spikes   spike_dtype [T, M, N] contiguous, 0/1
 *   u_out    F32 [M, N] contiguous final membrane, or NULL
 *
 * Per element, for t = 0..T-1, in fp32 with no fused multiply-add:
 *   r = (u - th > 0);  u = (beta*u + x_t) - r*th;  s_t = (u - th > 0).
 */
int spk_lif_multistep(const void *x, int x_dtype, const int64_t x_strides[3],
                      const void *beta, const void *threshold, int param_dtype,
                      const float *mem0, void *spikes, int spike_dtype,
                      float *u_out, int T, int64_t M, int N, void *stream);

/*
 * Fused LIF + bit-pack (+ paged cache scatter) for one q/k/v site.  Replaces
 * the composition lif_multistep -> pack_spikes -> index_copy_
 * (spikeinfer/modeling_fast.py:132-134, spikeinfer/attention.py:138-139 and
 * :146-149, spikeinfer/kernels/packing.py:84-111).
 *
 *   x        x_dtype [T, n_tok, H, D] at x_strides (elements), e.g. the
 *            permuted projection output without a copy
 *   beta, threshold  param_dtype [D]
 *   Packed output goes to exactly one of:
 *     packed  int32 [T, n_tok, H, W] at packed_strides (word axis contiguous)
 *             when slot_mapping == NULL (the packed-query buffer), or
 *     packed  int32 [T, H, slots, W] at packed_strides when slot_mapping is
 *             given: token i is written to slot slot_mapping[i] (int64);
 *             a slot outside [0, num_slots) skips the token.
 *   spikes   optional dense 0/1 output [T, n_tok, H, D] contiguous in
 *            spike_dtype (NULL to skip); the prefill path feeds it to SDPA.
 * W = ceil(D/32); bits past D in the last word are zero.
 */
int spk_lif_pack_write(const void *x, int x_dtype, const int64_t x_strides[4],
                       const void *beta, const void *threshold,
                       int param_dtype, int32_t *packed,
                       const int64_t packed_strides[3],
                       const int64_t *slot_mapping, int64_t num_slots,
                       void *spikes,
                       int spike_dtype, int T, int64_t n_tok, int H, int D,
                       void *stream);

/*
 * One LIF site of spk_lif_pack_write_sites: the arguments of one
 * spk_lif_pack_write call (x dtype and T shared by all sites of a launch).
 *   x            [T, n_tok, H, D] at x_strides (elements)
 *   beta, threshold  param_dtype [D]
 *   out          int32 packed output at out_strides: [T, n_tok, H, W] when
 *                scatter == 0, the paged cache [T, H, num_slots, W] when
 *                scatter != 0 (token i -> slot slot_mapping[i]; slots outside
 *                [0, num_slots) skip the token)
 */
typedef struct SpkLifSite {
  const void *x;
  int64_t x_strides[4];
  const void *beta;
  const void *threshold;
  int param_dtype;
  int scatter;
  int32_t *out;
  int64_t out_strides[3];
  int64_t num_slots;
  int64_t n_tok;
  int H;
  int D;
} SpkLifSite;

/*
 * Several fused LIF + pack (+ cache scatter) sites in ONE launch, e.g. the
 * q, k and v sites of an attention layer: the k/v sites scatter into their
 * caches by slot_mapping (int64 [n_tok]), the q site writes the packed-query
 * buffer.  Same results as one spk_lif_pack_write per site; one launch
 * instead of three keeps the small k/v sites from running alone on a mostly
 * idle GPU.  Replaces attention.py:138-149 with modeling_fast.py:132-134
 * (three lif_multistep, pack_spikes, two index_copy_).  1 <= nsites <= 4.
 */
int spk_lif_pack_write_sites(const SpkLifSite *sites, int nsites, int x_dtype, int T,
                             const int64_t *slot_mapping, void *stream);

/*
 * Bit-pack rows: x [rows, C] (row stride x_row_stride elements, channel
 * stride 1) of any supported dtype -> int32 [rows, W] contiguous, nonzero ->
 * 1.  Replaces _pack_kernel (spikeinfer/kernels/packing.py:57-81, 114-133).
 */
int spk_pack(const void *x, int x_dtype, int64_t x_row_stride, int32_t *out,
             int64_t rows, int C, void *stream);

/*
 * Unpack rows: int32 [rows, W] contiguous -> [rows, C] contiguous 0/1 in
 * out_dtype.  Replaces unpack_spikes (spikeinfer/kernels/packing.py:136-152).
 */
int spk_unpack(const int32_t *words, int64_t rows, int C, void *out,
               int out_dtype, void *stream);

/* ------------------------------------------------------------------------
 * Decoder-step operators around the GEMMs (whole-step decode, hipGraph).
 * ------------------------------------------------------------------------ */

/*
 * Decode attention that derives its own spikes: for the N decode tokens,
 * RoPE -> LIF -> pack of each unit's q heads and current k/v head (exactly as
 * spk_qkv_rope_lif_pack computes them), the current k/v words written to the
 * token's cache slot, then the same attention as spk_decode_attn over
 * seq_lens[i] tokens (the current one included).  One launch replaces
 * spk_qkv_rope_lif_pack + spk_decode_attn on a decode-only batch
 * (spikeinfer/modeling_fast.py:121-135 + attention.py:138-149 + the Triton
 * launch in spike_attention.py:204-220).
 *
 *   x        x_dtype (BF16/F16) [T, N, (Hq + 2*Hkv) * 64], channel stride 1,
 *            strides {t, token} in elements (the q/k/v projection output)
 *   cos, sin x_dtype [table_rows, 64] tables; token i uses row positions[i]
 *   beta, threshold  param_dtype [3, 64]: q, k and v sites; param_dtype
 *            must be SPK_F32 (convert other dtypes first: it is exact)
 *   slot_mapping int64 [N]: cache slot of each token's k/v words (outside
 *            [0, num_slots): not written)
 *   k_cache, v_cache int32 [T, Hkv, num_slots, 2] at cache_strides
 *   block_tables, seq_lens, out, workspace: as spk_decode_attn.
 * head_dim must be 64, Hq/Hkv <= 8 and T <= 8 (SPK_EUNSUPPORTED otherwise).
 */
int spk_qkv_decode_attn(const void *x, int x_dtype, const int64_t x_strides[2], const void *cos,
                        const void *sin, const int64_t *positions, int64_t table_rows,
                        const void *beta, const void *threshold, int param_dtype,
                        const int64_t *slot_mapping, int32_t *k_cache, int32_t *v_cache,
                        const int64_t cache_strides[4], int64_t num_slots,
                        const int32_t *block_tables, int64_t bt_stride0, int64_t bt_stride1,
                        const int32_t *seq_lens, void *out, int out_dtype,
                        const int64_t out_strides[4], int T, int N, int Hq, int Hkv, int head_dim,
                        int block_size, int max_blocks, float scale, void *workspace,
                        size_t workspace_bytes, void *stream);

/*
 * Residual add + RMSNorm over rows of `hidden` contiguous elements, dtype in
 * {F32, F16, BF16}.  When delta != NULL, h <- round(h + delta) in place; then
 * out = round(weight * round(x * rsqrt(mean(x^2) + eps))), x = float(h).
 * Replaces `h = h + sublayer(...)` followed by Qwen2RMSNorm
 * (spikeinfer/modeling_fast.py:206-211).  Buffers 16-byte aligned.
 */
int spk_add_rmsnorm(void *h, const void *delta, const void *weight, void *out,
                    int dtype, int64_t rows, int hidden, float eps, void *stream);

/*
 * Embedding lookup + the first layer's RMSNorm, broadcast over T: for token
 * i, e = embed[clamp(ids[i], 0, vocab - 1)] (a row of `hidden`); for every
 * t < T, h[t, i] = e and out[t, i] = round(weight * round(e * rsqrt(mean(e^2)
 * + eps))).  h and out are [T, n, hidden] contiguous.  Replaces
 * `embed_tokens(ids)` broadcast to T steps and the first input_layernorm
 * (spikeinfer/modeling_fast.py:300, :311, :206).  Out-of-range ids read the
 * nearest row (torch raises instead).
 */
int spk_embed_rmsnorm(const int64_t *ids, const void *embed, int64_t vocab, const void *weight,
                      void *h, void *out, int dtype, int T, int64_t n, int hidden, float eps,
                      void *stream);

/*
 * Final residual add, RMSNorm and rate-coded readout: h [T, rows, hidden]
 * contiguous (plus delta of the same shape when not NULL, rounded to dtype; h
 * is only read) -> out [rows, hidden] = round(sum_t RMSNorm(h_t) * (1/T)),
 * 1 <= T <= 8.  Replaces `h = h + mlp(...)` of the last layer and
 * `self.norm(h).mean(dim=0)` (spikeinfer/modeling_fast.py:210, :319).
 */
int spk_rmsnorm_mean_t(const void *h, const void *delta, const void *weight, void *out,
                       int dtype, int T, int64_t rows, int hidden, float eps, void *stream);

/*
 * Fused q/k/v site of one attention layer: RoPE -> LIF -> bit-pack -> packed
 * q buffer and paged k/v cache slots.  Replaces _apply_rope_t + three
 * lif_multistep calls (spikeinfer/modeling_fast.py:89-99, :121-135) and the
 * packing / cache scatter of paged_attention (spikeinfer/attention.py:138-149).
 *
 *   x        x_dtype (BF16/F16) [T, n_tok, (Hq + 2*Hkv) * D], channel stride 1,
 *            strides {t, token} in elements: q heads, then k, then v heads
 *            (the concatenated q/k/v projection output)
 *   cos, sin x_dtype [n_tok, D] contiguous (rotary tables of each token), or,
 *            when positions != NULL, [table_rows, D] tables whose row
 *            positions[i] serves token i (out-of-range positions read the
 *            nearest row)
 *   beta, threshold  param_dtype [3, D] contiguous: q, k and v sites
 *   q_packed int32 [T, n_q, Hq, W] at q_strides: tokens [0, n_q) (the decode
 *            prefix) are packed here
 *   k_cache, v_cache int32 [T, Hkv, num_slots, W] at cache_strides; token i
 *            goes to slot_mapping[i] (outside [0, num_slots): skipped)
 *   dense_q/k/v optional x_dtype [T, H, n_tok, D] contiguous 0/1 spikes (the
 *            prefill path's SDPA operands), NULL to skip
 * RoPE is evaluated as the composition rounds it: round(round(x*cos) +
 * round(rotate_half(x)*sin)).  D is a power of two in [64, 512].
 */
int spk_qkv_rope_lif_pack(const void *x, int x_dtype, const int64_t x_strides[2],
                          const void *cos, const void *sin, const int64_t *positions,
                          int64_t table_rows, const void *beta,
                          const void *threshold, int param_dtype, int32_t *q_packed,
                          const int64_t q_strides[3], int64_t n_q, int32_t *k_cache,
                          int32_t *v_cache, const int64_t cache_strides[3],
                          const int64_t *slot_mapping, int64_t num_slots, void *dense_q,
                          void *dense_k, void *dense_v, int T, int64_t n_tok, int Hq,
                          int Hkv, int D, void *stream);

/*
 * MLP gate: x [T, rows, 2*I] (gate in columns [0, I), up in [I, 2I); strides
 * {t, row} in elements, channel stride 1) -> out [T, rows, I] contiguous =
 * round(LIF(gate) * up).  Replaces lif_multistep(gate_proj(x)) * up_proj(x)
 * (spikeinfer/modeling_fast.py:186-190) after one concatenated GEMM.
 */
int spk_lif_gate_mul(const void *x, int dtype, const int64_t x_strides[2],
                     const void *beta, const void *threshold, int param_dtype,
                     void *out, int T, int64_t rows, int I, void *stream);

/*
 * Fused MLP gate for decode sizes: the gate|up projection, the gate LIF over T
 * and the spike * up product in one launch, replacing
 * lif_multistep(gate_proj(x)) * up_proj(x) (spikeinfer/modeling_fast.py:186-190),
 * i.e. a bf16 GEMM on the concatenated weight followed by spk_lif_gate_mul.
 *
 * spk_mlp_gate_pack reorders W_gu [2*I, hidden] (gate rows, then up rows; bf16,
 * contiguous) into the kernel's operand order, spk_mlp_gate_packed_bytes(hidden,
 * I) bytes at w_packed; done once per weight.
 * spk_mlp_gate_lif: x [T, n_tok, hidden] bf16 contiguous -> y [T, n_tok, I] bf16
 * contiguous; beta, threshold [I] with param_dtype SPK_F32 (other dtypes:
 * convert first, exactly).  Supports T <= 4, hidden a multiple of 128 in [512, 1024] (and
 * T * 16 * hidden * 2 <= 160 KiB), I / 16 in [64, 512]; returns SPK_EUNSUPPORTED
 * otherwise (the caller then runs the GEMM and spk_lif_gate_mul).  The GEMM sums
 * are fp32 in a fixed order, rounded to bf16 before the LIF, as the two-launch
 * path rounds the GEMM output.
 */
size_t spk_mlp_gate_packed_bytes(int hidden, int inter);

/*
 * Small-M linear layer: y [M, N] = x [M, K] @ W^T (+ bias [N]), bf16, row-major
 * contiguous; the q/k/v and o projections of a decode step
 * (spikeinfer/modeling_fast.py:121-135, :150-166) in place of a library GEMM.
 * spk_linear_pack reorders W [N, K] (bf16, contiguous) into the kernel's operand
 * order (N * K * 2 bytes at w_packed), once per weight.  spk_linear_decode
 * supports M <= 256, N a multiple of 16, K a multiple of 128 up to 1280, or up
 * to 5120 without a bias (the down projection), bf16 (SPK_EUNSUPPORTED
 * otherwise); sums are fp32 in a fixed order, bias added, then rounded once.
 * x and w_packed 16-byte aligned; a y off 16 bytes is SPK_EUNSUPPORTED for
 * the short-K path (its tiles go out as 16-byte rows).  The same holds for
 * spk_mlp_gate_lif's y.
 */
int spk_linear_pack(const void *w, int N, int K, int dtype, void *w_packed, void *stream);
int spk_linear_decode(const void *x, const void *w_packed, const void *bias, void *y, int M, int N,
                      int K, int dtype, void *stream);
int spk_mlp_gate_pack(const void *w_gu, int inter, int hidden, int dtype, void *w_packed,
                      void *stream);
int spk_mlp_gate_lif(const void *x, const void *w_packed, const void *beta,
                     const void *threshold, int param_dtype, void *y, int T, int n_tok,
                     int hidden, int inter, int dtype, void *stream);

/*
 * The same GEMMs starting from the residual stream instead of a normed input:
 * the rows are add_rmsnorm(h, delta, norm_weight) (bf16, computed in the
 * launch's prologue with spk_add_rmsnorm's arithmetic, so the results are
 * identical to spk_add_rmsnorm followed by spk_linear_decode /
 * spk_mlp_gate_lif), replacing the post-attention / next-layer RMSNorm and
 * residual add (spikeinfer/modeling_fast.py:206-211) that precede the MLP and
 * the q/k/v projections (:121-135, :186-190).  h_out (may be NULL; must not
 * alias h or delta) receives round(h + delta).  h, delta: [rows, hidden]
 * contiguous (rows = M, or T * n_tok), hidden <= 1024; 16-byte aligned.
 * spk_norm_linear_decode supports the tiled shapes of spk_linear_decode (K =
 * hidden a multiple of 128 up to 1024).
 */
int spk_norm_linear_decode(const void *h, const void *delta, const void *norm_weight, void *h_out,
                           float eps, const void *w_packed, const void *bias, void *y, int M, int N,
                           int K, int dtype, void *stream);
int spk_norm_mlp_gate_lif(const void *h, const void *delta, const void *norm_weight, void *h_out,
                          float eps, const void *w_packed, const void *beta, const void *threshold,
                          int param_dtype, void *y, int T, int n_tok, int hidden, int inter, int dtype,
                          void *stream);

/*
 * Device-side advance of a decode batch after sampling: for rows i < n_live,
 * where n_live = n_rows, or min(n_rows, *live) when `live` is given (a device
 * count, so a captured step serves any live batch up to n_rows),
 * input_ids[i] = next_tokens[i], positions[i] += 1, seq_lens[i] =
 * positions[i] + 1, slot_mapping[i] = table[i][pos / bs] * bs + pos % bs
 * (spikeinfer/engine/model_runner.py:89-100, block_manager.py:71-77).  A row
 * whose next position is past its table stays put.  When history != NULL,
 * next_tokens[i] is also stored at history[i * hist_cap + *step] and *step is
 * incremented.  When uniforms != NULL (rng_seeds and step required), every row
 * i < n_rows also gets the next step's sampling draw uniforms[i] =
 * u(rng_seeds[i], *step after the increment): SplitMix64's output function on
 * seed + (step + 1) * 0x9E3779B97F4A7C15, top 24 bits / 2^24 -- a captured
 * step then needs no torch RNG (whose per-replay seed/offset fills are two
 * extra launches).  No reference counterpart as a kernel: the reference
 * rebuilds these tensors on the host every step.
 */
int spk_decode_advance(const int64_t *next_tokens, int64_t *input_ids, int64_t *positions,
                       int32_t *seq_lens, int64_t *slot_mapping, const int32_t *block_tables,
                       int64_t bt_stride0, int64_t bt_stride1, int max_blocks,
                       int block_size, int n_rows, const int32_t *live, int64_t *history,
                       int32_t *step, int hist_cap, const int64_t *rng_seeds,
                       float *uniforms, void *stream);

/*
 * Batched sampler, one workgroup per row (spikeinfer/engine/sampler.py:48-177):
 * penalties over the row's generated tokens (repetition, then presence +
 * frequency), temperature, min_p, top_k, top_p, then a draw.  Per-row
 * parameters are device arrays of `rows` entries (NULL = disabled: top_k -1,
 * top_p 1, min_p 0, penalties neutral).  Rows with temperature < 1e-5 take the
 * argmax of the penalised logits (lowest index on ties).
 *
 * Equal logits are ordered by index (the reference leaves that order to
 * torch.topk).  The draw is the inverse CDF of the kept softmax weights at
 * uniforms[row] in [0, 1), tokens taken by logit descending, index ascending.  history int64 [rows,
 * history_stride] holds generated tokens, history_len[row *
 * history_len_stride] of them (stride 0: one count for every row; at most
 * 2048 are used).  vocab <= 262144.  Result: out_tokens int64 [rows].
 */
int spk_sample(const void *logits, int logits_dtype, int64_t row_stride, int rows, int vocab,
               const float *temperature, const int32_t *top_k, const float *top_p,
               const float *min_p, const float *repetition_penalty,
               const float *presence_penalty, const float *frequency_penalty,
               const int64_t *history, int64_t history_stride, const int32_t *history_len,
               int64_t history_len_stride, const float *uniforms, int64_t *out_tokens,
               void *stream);

/* LDS bytes one spk_sample workgroup uses (for occupancy planning). */
size_t spk_sample_shared_bytes(void);

/*
 * spk_sample with a device workspace (spk_sample_workspace_bytes(rows) bytes,
 * 16-byte aligned; no counterpart in the reference, whose sampler is torch
 * ops).  `stages` picks the sliced stages, which cut a row into 8 slices of
 * the vocabulary, one workgroup each:
 *   SPK_SAMPLE_STAGE_TOPK: rows with a top-k cut (0 < top_k <= 256,
 *     temperature >= 1e-5); the slices hand the row workgroup a candidate set
 *     holding the row's top_k largest;
 *   SPK_SAMPLE_STAGE_OPEN: rows with no top-k cut (top_k < 0 or >= vocab,
 *     temperature >= 1e-5) and a top-p or min-p cut (top_p < 1 or
 *     min_p > 0); two launches give the row maximum, then each slice's 64
 *     largest and its exact share of the row's probability mass,
 *     which decide the row when its top-p cut and draw fall inside the
 *     certified prefix of the merged lists (else the row workgroup takes the
 *     whole row).
 * The tokens are those spk_sample returns whatever the stages; a stage only
 * pays off when the batch holds rows of its kind (each costs launches).  A
 * NULL workspace or stages 0 is spk_sample.  Calls sharing a workspace must
 * be ordered (one stream).
 */
#define SPK_SAMPLE_STAGE_TOPK 1
#define SPK_SAMPLE_STAGE_OPEN 2
size_t spk_sample_workspace_bytes(int rows);
int spk_sample_ws(const void *logits, int logits_dtype, int64_t row_stride, int rows, int vocab,
                  const float *temperature, const int32_t *top_k, const float *top_p,
                  const float *min_p, const float *repetition_penalty,
                  const float *presence_penalty, const float *frequency_penalty,
                  const int64_t *history, int64_t history_stride, const int32_t *history_len,
                  int64_t history_len_stride, const float *uniforms, int64_t *out_tokens,
                  void *workspace, size_t workspace_bytes, int stages, void *stream);



#ifdef __cplusplus
}
#endif

#endif /* SPIKEINFER_AMD_H */
