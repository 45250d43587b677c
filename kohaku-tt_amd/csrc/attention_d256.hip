// Attention forward kernels for head dims padded to 256 (attention_kernels.hpp).
#include "attention_kernels.hpp"

namespace kmi {
namespace fwd {
template hipError_t launch_all<bf16, 256>(const AttnParams&, const Plan&, hipStream_t);
template hipError_t launch_all<f16, 256>(const AttnParams&, const Plan&, hipStream_t);
}  // namespace fwd
}  // namespace kmi
