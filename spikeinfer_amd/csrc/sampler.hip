// Batched token sampler: the C-ABI entry (the kernels are in
// sampler_kernel.hpp, instantiated per logits dtype in sampler_f32.hip,
// sampler_f16.hip and sampler_bf16.hip so they compile in parallel).
#include "sampler_kernel.hpp"

namespace spk {
namespace smp {
extern template int launch<SPK_F32, true>(const Args &, int, hipStream_t);
extern template int launch<SPK_F32, false>(const Args &, int, hipStream_t);
extern template int launch<SPK_F16, true>(const Args &, int, hipStream_t);
extern template int launch<SPK_F16, false>(const Args &, int, hipStream_t);
extern template int launch<SPK_BF16, true>(const Args &, int, hipStream_t);
extern template int launch<SPK_BF16, false>(const Args &, int, hipStream_t);
}  // namespace smp
}  // namespace spk

using namespace spk;

extern "C" size_t spk_sample_shared_bytes(void) { return sizeof(smp::Shared); }

extern "C" size_t spk_sample_workspace_bytes(int rows) { return rows > 0 ? smp::slice_ws_bytes(rows) : 0; }

extern "C" int spk_sample_ws(const void *logits, int logits_dtype, int64_t row_stride, int rows,
                             int vocab, const float *temperature, const int32_t *top_k,
                             const float *top_p, const float *min_p, const float *repetition_penalty,
                             const float *presence_penalty, const float *frequency_penalty,
                             const int64_t *history, int64_t history_stride, const int32_t *history_len,
                             int64_t history_len_stride, const float *uniforms, int64_t *out_tokens,
                             void *workspace, size_t workspace_bytes, int stages, void *stream) {
  if (!valid_float_dtype(logits_dtype))
    return fail(SPK_EINVAL, "sample: logits dtype %d is not a float type", logits_dtype);
  if (!logits || !temperature || !out_tokens) return fail(SPK_EINVAL, "sample: null pointer");
  if (rows < 0 || vocab < 1 || vocab > smp::kMaxVocab || row_stride < vocab)
    return fail(SPK_EINVAL, "sample: vocab=%d must be in [1, %d] and row_stride >= vocab", vocab,
                smp::kMaxVocab);
  if (history && (!history_len || history_stride < 1))
    return fail(SPK_EINVAL, "sample: history needs history_len and a row stride >= 1");
  if (stages & ~(SPK_SAMPLE_STAGE_TOPK | SPK_SAMPLE_STAGE_OPEN))
    return fail(SPK_EINVAL, "sample: unknown stage bits %d", stages);
  if (rows == 0) return SPK_OK;
  if (workspace && workspace_bytes < smp::slice_ws_bytes(rows))
    return fail(SPK_EINVAL, "sample: workspace of %zu bytes, %zu needed for %d rows", workspace_bytes,
                smp::slice_ws_bytes(rows), rows);
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 15))
    return fail(SPK_EINVAL, "sample: workspace must be 16-byte aligned");
  smp::Args a{logits, row_stride, vocab, temperature, top_k, top_p, min_p, repetition_penalty,
              presence_penalty, frequency_penalty, history, history_stride, history_len,
              history_len_stride, uniforms, out_tokens, workspace, stages};
  const size_t esz = logits_dtype == SPK_F32 ? 4 : 2;
  const bool vec = (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && (row_stride * esz) % 16 == 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (logits_dtype) {
    case SPK_F32: return vec ? smp::launch<SPK_F32, true>(a, rows, s) : smp::launch<SPK_F32, false>(a, rows, s);
    case SPK_F16: return vec ? smp::launch<SPK_F16, true>(a, rows, s) : smp::launch<SPK_F16, false>(a, rows, s);
    default: return vec ? smp::launch<SPK_BF16, true>(a, rows, s) : smp::launch<SPK_BF16, false>(a, rows, s);
  }
}

extern "C" int spk_sample(const void *logits, int logits_dtype, int64_t row_stride, int rows,
                          int vocab, const float *temperature, const int32_t *top_k,
                          const float *top_p, const float *min_p, const float *repetition_penalty,
                          const float *presence_penalty, const float *frequency_penalty,
                          const int64_t *history, int64_t history_stride, const int32_t *history_len,
                          int64_t history_len_stride, const float *uniforms, int64_t *out_tokens,
                          void *stream) {
  return spk_sample_ws(logits, logits_dtype, row_stride, rows, vocab, temperature, top_k, top_p, min_p,
                       repetition_penalty, presence_penalty, frequency_penalty, history, history_stride,
                       history_len, history_len_stride, uniforms, out_tokens, nullptr, 0, 0, stream);
}
