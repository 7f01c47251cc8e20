// fa_small.hip -- the single-workgroup `flash_attention_f32` kernel ABI
// (python/mlir/dialects/wave_attention.py:1406-1441; launched with grid
// (1,1,1) and one wave by tools/wave-fa-calibrate/wave-fa-calibrate-runner.cpp
// :346-361).  Q arrives pre-scaled by log2(e)/sqrt(D) (wave_attention.py:
// 225-245), so O[m] = sum_n 2^(s_n - max) V[n] / sum_n 2^(s_n - max) with
// s_n = Q[m].K[n] (wave_attention.py:248-278).  This configuration is a
// latency-bound parity case (a 16 x D query block); one wave processes the
// rows in turn: lanes split the keys for the scores and the head dimension
// for P.V, with the weights of the current row staged in LDS.
#include "attention.hpp"
#include "wave_common.hpp"

namespace wave {
namespace attention {

__global__ __launch_bounds__(64) void small_kernel(const _Float16 *Q,
                                                   const _Float16 *K,
                                                   const _Float16 *V, float *O,
                                                   int block_m, int seq_n,
                                                   int head_dim) {
  extern __shared__ float weights[];  // seq_n
  const int lane = threadIdx.x;
  for (int m = 0; m < block_m; ++m) {
    const _Float16 *q = Q + (size_t)m * head_dim;
    float mx = -__builtin_inff();
    for (int n = lane; n < seq_n; n += 64) {
      const _Float16 *k = K + (size_t)n * head_dim;
      float s = 0.f;
      for (int d = 0; d < head_dim; ++d)
        s = __builtin_fmaf((float)q[d], (float)k[d], s);
      weights[n] = s;
      mx = fmaxf(mx, s);
    }
    for (int off = 32; off > 0; off >>= 1)
      mx = fmaxf(mx, __shfl_xor(mx, off));
    float sum = 0.f;
    for (int n = lane; n < seq_n; n += 64) {
      const float w = exp2f(weights[n] - mx);
      weights[n] = w;
      sum += w;
    }
    for (int off = 32; off > 0; off >>= 1)
      sum += __shfl_xor(sum, off);
    __syncthreads();
    const float inv = 1.0f / sum;
    for (int d = lane; d < head_dim; d += 64) {
      float acc = 0.f;
      for (int n = 0; n < seq_n; ++n)
        acc = __builtin_fmaf(weights[n], (float)V[(size_t)n * head_dim + d], acc);
      O[(size_t)m * head_dim + d] = acc * inv;
    }
    __syncthreads();
  }
}

hipError_t launch_small(const void *Q, const void *K, const void *V, float *O,
                        int block_m, int seq_n, int head_dim,
                        hipStream_t stream) {
  hipLaunchKernelGGL(small_kernel, dim3(1), dim3(64), (size_t)seq_n * sizeof(float),
                     stream, static_cast<const _Float16 *>(Q),
                     static_cast<const _Float16 *>(K),
                     static_cast<const _Float16 *>(V), O, block_m, seq_n,
                     head_dim);
  return hipGetLastError();
}

} // namespace attention
} // namespace wave
