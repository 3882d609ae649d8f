// 16-bit instantiations of the dK/dV kernel (attn_bwd.hpp), built with
// -amdgpu-mfma-vgpr-form=1: at this kernel's register pressure the default
// lets the allocator park the dK/dV accumulators in AGPRs and copy them to
// VGPRs around every MFMA (320 extra moves per step).
#include "attn_bwd.hpp"

namespace pf {

hipError_t launch_bwd_dkv16(const BwdParams& p, int dtype, int head_dim, bool causal, hipStream_t stream) {
  if (head_dim == 128) {
    if (dtype == kBF16) return bwd::dkv_typed<bf16_t, 128>(p, causal, stream);
    if (dtype == kF16) return bwd::dkv_typed<f16_t, 128>(p, causal, stream);
  } else if (head_dim == 64) {
    if (dtype == kBF16) return bwd::dkv_typed<bf16_t, 64>(p, causal, stream);
    if (dtype == kF16) return bwd::dkv_typed<f16_t, 64>(p, causal, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace pf
