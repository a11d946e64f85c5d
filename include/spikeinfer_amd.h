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

/* ABI version, bumped on any signature change. */
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
 * A sequence with seq_len <= 0 gets an all-zero output row.  Slots outside
 * [0, num_slots) are never dereferenced, so a corrupt block table cannot
 * fault the GPU (the output rows of such a sequence are unspecified).  scale must satisfy
 * 0 < scale*head_dim <= 80 (the softmax uses the fixed offset popcount(q)).
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

/* Bytes of workspace spk_decode_attn needs for this launch shape. */
size_t spk_decode_attn_workspace_bytes(int T, int N, int Hq, int Hkv,
                                       int head_dim, int block_size,
                                       int max_blocks);

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

#ifdef __cplusplus
}
#endif

#endif /* SPIKEINFER_AMD_H */
