// fa_small.hip -- host launch of the single-workgroup flash_attention_f32
// kernel (body in fa_small.hpp): one wave, the row weights in dynamic LDS.
#include "attention.hpp"
#include "fa_small.hpp"

namespace wave {
namespace attention {

constexpr int kSmallThreads = 64;

__global__ __launch_bounds__(kSmallThreads) void small_kernel(const _Float16 *Q,
                                                              const _Float16 *K,
                                                              const _Float16 *V, float *O,
                                                              int block_m, int seq_n,
                                                              int head_dim) {
  extern __shared__ float lds[];  // kSmallThreads reduction slots, then seq_n weights
  small_cta(Q, K, V, O, block_m, seq_n, head_dim, lds + kSmallThreads, lds);
}

hipError_t launch_small(const void *Q, const void *K, const void *V, float *O,
                        int block_m, int seq_n, int head_dim,
                        hipStream_t stream) {
  hipLaunchKernelGGL(small_kernel, dim3(1), dim3(kSmallThreads),
                     (size_t)(kSmallThreads + seq_n) * sizeof(float), stream,
                     static_cast<const _Float16 *>(Q), static_cast<const _Float16 *>(K),
                     static_cast<const _Float16 *>(V), O, block_m, seq_n, head_dim);
  return hipGetLastError();
}

} // namespace attention
} // namespace wave
