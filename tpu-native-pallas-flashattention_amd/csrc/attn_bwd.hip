// Backward launch entry points (kernels in attn_bwd.hpp). The 16-bit delta and
// dQ instantiations at head_dim 64 and 128 live in this translation unit; the
// 16-bit dK/dV kernel is built in attn_bwd_dkv16.hip, the float32 ones in
// attn_bwd_f32.hip and the 16-bit head_dim 256 ones in attn_bwd_d256.hip, each
// with its own code-generation flags (see the Makefile).
#include "attn_bwd.hpp"

namespace pf {

hipError_t launch_bwd_delta_f32(const BwdParams& p, int head_dim, hipStream_t stream);
hipError_t launch_bwd_dq_f32(const BwdParams& p, int head_dim, bool causal, hipStream_t stream);
hipError_t launch_bwd_dkv_f32(const BwdParams& p, int head_dim, bool causal, hipStream_t stream);
hipError_t launch_bwd_dkv16(const BwdParams& p, int dtype, int head_dim, bool causal, hipStream_t stream);
// kernel 0 = delta, 1 = dQ, 2 = dK/dV
hipError_t launch_bwd_d256(int kernel, const BwdParams& p, int dtype, bool causal, hipStream_t stream);

#define PF_DISPATCH16(FN, ...)                                                 \
  do {                                                                         \
    if (head_dim == 128) {                                                     \
      if (dtype == kBF16) return bwd::FN<bf16_t, 128>(__VA_ARGS__);            \
      if (dtype == kF16) return bwd::FN<f16_t, 128>(__VA_ARGS__);              \
    } else if (head_dim == 64) {                                               \
      if (dtype == kBF16) return bwd::FN<bf16_t, 64>(__VA_ARGS__);             \
      if (dtype == kF16) return bwd::FN<f16_t, 64>(__VA_ARGS__);               \
    }                                                                          \
    return hipErrorInvalidValue;                                               \
  } while (0)

hipError_t launch_attn_bwd_delta(const BwdParams& p, int dtype, int head_dim, hipStream_t stream) {
  if (dtype == kF32) return launch_bwd_delta_f32(p, head_dim, stream);
  if (head_dim == 256) return launch_bwd_d256(0, p, dtype, false, stream);
  PF_DISPATCH16(delta_typed, p, stream);
}

hipError_t launch_attn_bwd_dq(const BwdParams& p, int dtype, int head_dim, bool causal,
                              hipStream_t stream) {
  if (dtype == kF32) return launch_bwd_dq_f32(p, head_dim, causal, stream);
  if (head_dim == 256) return launch_bwd_d256(1, p, dtype, causal, stream);
  PF_DISPATCH16(dq_typed, p, causal, stream);
}

hipError_t launch_attn_bwd_dkv(const BwdParams& p, int dtype, int head_dim, bool causal,
                               hipStream_t stream) {
  if (dtype == kF32) return launch_bwd_dkv_f32(p, head_dim, causal, stream);
  if (head_dim == 256) return launch_bwd_d256(2, p, dtype, causal, stream);
  return launch_bwd_dkv16(p, dtype, head_dim, causal, stream);
}

}  // namespace pf
