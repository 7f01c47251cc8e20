// attention_fwd8.hip -- host launch of the block-scaled FP8 flash-attention
// forward (attention_fwd8.hpp).
#include "attention_fwd8.hpp"

#include <cmath>

namespace wave {
namespace attention {

hipError_t launch_fwd_fp8(const Fp8FwdArgs &a, hipStream_t stream) {
  Fp8Params p{};
  p.Q = static_cast<const uint8_t *>(a.Q);
  p.K = static_cast<const uint8_t *>(a.K);
  p.V = static_cast<const uint8_t *>(a.V);
  p.Qs = static_cast<const uint8_t *>(a.Q_scale);
  p.Ks = static_cast<const uint8_t *>(a.K_scale);
  p.Vs = static_cast<const uint8_t *>(a.V_scale);
  p.O = static_cast<uint16_t *>(a.O);
  p.batch = a.batch;
  p.q_heads = a.q_heads;
  p.kv_heads = a.kv_heads;
  p.seq_q = a.seq_q;
  p.seq_k = a.seq_k;
  p.q_blocks = (a.seq_q + k8Rows - 1) / k8Rows;
  p.causal = a.causal;
  const float scale = a.scale > 0.f ? a.scale : 1.0f / std::sqrt((float)kD);
  p.scale_log2 = scale * kLog2e;
  p.lse = a.lse;
  const dim3 grid(p.q_blocks * a.batch * a.q_heads), block(64 * k8Waves);
  if (a.out_dtype == kF16) {
    if (a.causal)
      hipLaunchKernelGGL((fwd8_kernel<kF16, true>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((fwd8_kernel<kF16, false>), grid, block, 0, stream, p);
  } else {
    if (a.causal)
      hipLaunchKernelGGL((fwd8_kernel<kBF16, true>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((fwd8_kernel<kBF16, false>), grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

} // namespace attention
} // namespace wave
