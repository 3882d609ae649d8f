// Float32 instantiations of the backward kernels (attn_bwd.hpp). Kept apart
// from the 16-bit dK/dV unit: with float32 operands the dK/dV kernel needs
// more than 256 registers, and -amdgpu-mfma-vgpr-form=1 crashes this compiler
// there.
#include "attn_bwd.hpp"

namespace pf {

hipError_t launch_bwd_delta_f32(const BwdParams& p, int head_dim, hipStream_t stream) {
  if (head_dim == 128) return bwd::delta_typed<float, 128>(p, stream);
  if (head_dim == 64) return bwd::delta_typed<float, 64>(p, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_dq_f32(const BwdParams& p, int head_dim, bool causal, hipStream_t stream) {
  if (head_dim == 128) return bwd::dq_typed<float, 128>(p, causal, stream);
  if (head_dim == 64) return bwd::dq_typed<float, 64>(p, causal, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_dkv_f32(const BwdParams& p, int head_dim, bool causal, hipStream_t stream) {
  if (head_dim == 128) return bwd::dkv_typed<float, 128>(p, causal, stream);
  if (head_dim == 64) return bwd::dkv_typed<float, 64>(p, causal, stream);
  return hipErrorInvalidValue;
}

}  // namespace pf
