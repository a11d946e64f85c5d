// Sampler kernels for bf16 logits (see sampler_kernel.hpp).
#include "sampler_kernel.hpp"

namespace spk {
namespace smp {
SPK_SAMPLER_INSTANTIATE(SPK_BF16)
}  // namespace smp
}  // namespace spk
