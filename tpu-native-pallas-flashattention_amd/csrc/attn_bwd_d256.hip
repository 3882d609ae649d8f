// 16-bit instantiations of the backward kernels (attn_bwd.hpp) at head_dim
// 256, in a translation unit of their own with the default code generation:
// at this width the dQ and dK/dV accumulators (128 and 256 registers per
// lane) live in AGPRs as the compiler's MFMA accumulators, which the
// -amdgpu-mfma-vgpr-form=1 build of the 16-bit dK/dV unit would forbid.
#include "attn_bwd.hpp"

namespace pf {

hipError_t launch_bwd_d256(int kernel, const BwdParams& p, int dtype, bool causal, hipStream_t stream) {
  if (dtype != kBF16 && dtype != kF16) return hipErrorInvalidValue;
  const bool bf = dtype == kBF16;
  switch (kernel) {
    case 0: return bf ? bwd::delta_typed<bf16_t, 256>(p, stream) : bwd::delta_typed<f16_t, 256>(p, stream);
    case 1: return bf ? bwd::dq_typed<bf16_t, 256>(p, causal, stream) : bwd::dq_typed<f16_t, 256>(p, causal, stream);
    case 2:
      return bf ? bwd::dkv_typed<bf16_t, 256>(p, causal, stream) : bwd::dkv_typed<f16_t, 256>(p, causal, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pf
