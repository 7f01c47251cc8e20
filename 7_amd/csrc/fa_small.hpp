// fa_small.hpp -- device body of the single-workgroup `flash_attention_f32`
// kernel (python/mlir/dialects/wave_attention.py:1406-1441; launched with
// grid (1,1,1) by tools/wave-fa-calibrate/wave-fa-calibrate-runner.cpp
// :346-361).  Q arrives pre-scaled by log2(e)/sqrt(D) (wave_attention.py:
// 225-245), so O[m] = sum_n 2^(s_n - max) V[n] / sum_n 2^(s_n - max) with
// s_n = Q[m].K[n] (wave_attention.py:248-278).  This configuration is a
// latency-bound parity case (a 16 x D query block); the workgroup processes
// the rows in turn: threads split the keys for the scores and the head
// dimension for P.V, with the weights of the current row staged in LDS.
// Any block size works (the runner's --threads); reductions go through LDS.
#pragma once

#include <hip/hip_runtime.h>

namespace wave {
namespace attention {

// weights: seq_n floats of LDS; red: blockDim.x floats of LDS.
__device__ __forceinline__ void small_cta(const _Float16 *Q, const _Float16 *K,
                                          const _Float16 *V, float *O, int block_m,
                                          int seq_n, int head_dim, float *weights,
                                          float *red) {
  const int t = threadIdx.x, nt = blockDim.x;
  // Block-wide reduction of v with op; every thread gets the result.
  auto reduce = [&](float v, bool is_max) {
    red[t] = v;
    __syncthreads();
    if (t == 0) {
      float r = red[0];
      for (int i = 1; i < nt; ++i)
        r = is_max ? fmaxf(r, red[i]) : r + red[i];
      red[0] = r;
    }
    __syncthreads();
    const float r = red[0];
    __syncthreads();
    return r;
  };
  for (int m = 0; m < block_m; ++m) {
    const _Float16 *q = Q + (size_t)m * head_dim;
    float mx = -__builtin_inff();
    for (int n = t; n < seq_n; n += nt) {
      const _Float16 *k = K + (size_t)n * head_dim;
      float s = 0.f;
      for (int d = 0; d < head_dim; ++d)
        s = __builtin_fmaf((float)q[d], (float)k[d], s);
      weights[n] = s;
      mx = fmaxf(mx, s);
    }
    mx = reduce(mx, true);
    float sum = 0.f;
    for (int n = t; n < seq_n; n += nt) {
      const float w = exp2f(weights[n] - mx);
      weights[n] = w;
      sum += w;
    }
    sum = reduce(sum, false);  // its barriers also publish the weights
    const float inv = 1.0f / sum;
    for (int d = t; d < head_dim; d += nt) {
      float acc = 0.f;
      for (int n = 0; n < seq_n; ++n)
        acc = __builtin_fmaf(weights[n], (float)V[(size_t)n * head_dim + d], acc);
      O[(size_t)m * head_dim + d] = acc * inv;
    }
    __syncthreads();  // weights are rewritten by the next row
  }
}

} // namespace attention
} // namespace wave
