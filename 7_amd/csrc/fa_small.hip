// fa_small.hip -- host launch of the single-workgroup flash_attention_f32
// kernel (body in fa_small.hpp): one wave per 16-query x 128-column unit,
// up to 16 waves, on the matrix cores; no LDS.
#include "attention.hpp"
#include "fa_small.hpp"

namespace wave {
namespace attention {

constexpr int kSmallMaxWaves = 16;

__global__ __launch_bounds__(64 * kSmallMaxWaves) void small_kernel(const _Float16 *Q,
                                                                    const _Float16 *K,
                                                                    const _Float16 *V, float *O,
                                                                    int block_m, int seq_n,
                                                                    int head_dim) {
  // Whole waves only: the scalar path (and its LDS) is never taken.
  small_cta(Q, K, V, O, block_m, seq_n, head_dim, nullptr, nullptr);
}

hipError_t launch_small(const void *Q, const void *K, const void *V, float *O,
                        int block_m, int seq_n, int head_dim,
                        hipStream_t stream) {
  const int units = (block_m + 15) / 16 * ((head_dim + kSmallCols - 1) / kSmallCols);
  const int waves = units < kSmallMaxWaves ? units : kSmallMaxWaves;
  hipLaunchKernelGGL(small_kernel, dim3(1), dim3(64 * waves), 0, stream,
                     static_cast<const _Float16 *>(Q), static_cast<const _Float16 *>(K),
                     static_cast<const _Float16 *>(V), O, block_m, seq_n, head_dim);
  return hipGetLastError();
}

} // namespace attention
} // namespace wave
