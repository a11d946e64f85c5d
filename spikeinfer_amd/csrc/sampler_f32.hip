// Sampler kernels for f32 logits (see sampler_kernel.hpp).
#include "sampler_kernel.hpp"

namespace spk {
namespace smp {
SPK_SAMPLER_INSTANTIATE(SPK_F32)
}  // namespace smp
}  // namespace spk
