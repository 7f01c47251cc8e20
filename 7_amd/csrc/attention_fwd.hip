// attention_fwd.hip -- instantiation and host launch of the gfx950
// flash-attention forward kernels: the 12-wave three-group kernel
// (attention_fwd3.hpp), the 8-wave ping-pong kernel (attention_kernels.hpp)
// and the 4-wave kernel (attention_fwd4.hpp).
#include "attention_fwd3.hpp"
#include "attention_fwd4.hpp"
#include "attention_kernels.hpp"

#include <cmath>

namespace wave {
namespace attention {

hipError_t launch_fwd(const FwdArgs &a, hipStream_t stream) {
  Params p{};
  p.Q = static_cast<const uint16_t *>(a.Q);
  p.K = static_cast<const uint16_t *>(a.K);
  p.V = static_cast<const uint16_t *>(a.V);
  p.O = static_cast<uint16_t *>(a.O);
  p.batch = a.batch;
  p.q_heads = a.q_heads;
  p.kv_heads = a.kv_heads;
  p.seq_q = a.seq_q;
  p.seq_k = a.seq_k;
  const int rows = a.waves == kR3Waves ? kR3Rows : 32 * kPPWaves;  // 4 waves: 256 too
  p.q_blocks = (a.seq_q + rows - 1) / rows;
  p.causal = a.causal;
  const float scale = a.scale > 0.f ? a.scale : 1.0f / std::sqrt((float)a.head_dim);
  p.scale_log2 = scale * kLog2e;
  p.lse = a.lse;
  // Fixed-max mode: |s * scale| <= head_dim * qk_max_abs^2 * scale, in log2
  // units (wave_flash_attention.py:108-113 with scale = 1/sqrt(128)).
  p.fixed_max = (float)((double)kLog2e * scale * a.head_dim * a.qk_max_abs * a.qk_max_abs);
  const bool fixed = a.qk_max_abs > 0.f;
  if (a.waves == kF4Waves) {
    // 4 waves x 64 query rows per CTA (the same 256-row blocks).
    const dim3 grid(p.q_blocks * a.batch * a.q_heads), block(64 * kF4Waves);
    if (a.dtype == kF16) {
      if (fixed)
        hipLaunchKernelGGL((fwd4_kernel<kF16, true>), grid, block, 0, stream, p);
      else
        hipLaunchKernelGGL((fwd4_kernel<kF16, false>), grid, block, 0, stream, p);
    } else {
      if (fixed)
        hipLaunchKernelGGL((fwd4_kernel<kBF16, true>), grid, block, 0, stream, p);
      else
        hipLaunchKernelGGL((fwd4_kernel<kBF16, false>), grid, block, 0, stream, p);
    }
    return hipGetLastError();
  }
  if (a.waves == kR3Waves) {
    // 12 waves x 32 query rows per CTA, three rotating groups of 4 waves.
    const dim3 grid(p.q_blocks * a.batch * a.q_heads), block(64 * kR3Waves);
    if (a.dtype == kF16) {
      if (fixed)
        hipLaunchKernelGGL((fwd3_kernel<kF16, true>), grid, block, 0, stream, p);
      else
        hipLaunchKernelGGL((fwd3_kernel<kF16, false>), grid, block, 0, stream, p);
    } else {
      if (fixed)
        hipLaunchKernelGGL((fwd3_kernel<kBF16, true>), grid, block, 0, stream, p);
      else
        hipLaunchKernelGGL((fwd3_kernel<kBF16, false>), grid, block, 0, stream, p);
    }
    return hipGetLastError();
  }
  // 8 waves x 32 query rows per CTA, two ping-pong groups of 4 waves.
  const dim3 grid(p.q_blocks * a.batch * a.q_heads), block(64 * kPPWaves);
  if (a.dtype == kF16) {
    if (fixed)
      hipLaunchKernelGGL((fwd_pp_kernel<kF16, true>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((fwd_pp_kernel<kF16, false>), grid, block, 0, stream, p);
  } else {
    if (fixed)
      hipLaunchKernelGGL((fwd_pp_kernel<kBF16, true>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((fwd_pp_kernel<kBF16, false>), grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

} // namespace attention
} // namespace wave
