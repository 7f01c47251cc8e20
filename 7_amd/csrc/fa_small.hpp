// fa_small.hpp -- device body of the single-workgroup `flash_attention_f32`
// kernel (python/mlir/dialects/wave_attention.py:1406-1441; launched with
// grid (1,1,1) by tools/wave-fa-calibrate/wave-fa-calibrate-runner.cpp
// :346-361).  Q arrives pre-scaled by log2(e)/sqrt(D) (wave_attention.py:
// 225-245), so O[m] = sum_n 2^(s_n - max) V[n] / sum_n 2^(s_n - max) with
// s_n = Q[m].K[n] (wave_attention.py:248-278).
//
// Blocks of whole waves (64 * w threads) run on the matrix cores.  A unit
// is 16 query rows x up to 128 output columns; wave w takes units w, w + W,
// ....  Per block of 32 keys the wave computes S^T = K Q^T with two
// v_mfma_f32_16x16x32_f16 (keys are the A rows, queries the B columns), so
// lane l ends up with the eight scores of query l%16 against keys
// 4*(l/16) + {0..3} and 16 + 4*(l/16) + {0..3}.  Those eight values are
// exactly the B operand P^T of O^T += V^T P^T when the MFMA's K slots are
// read in that key order, so P goes from the score registers to the PV
// MFMA without any lane exchange (as the reference, P enters the product
// as f16).  The online-softmax row max and the final row sum are reductions
// over the four lanes l%16 + 16*{0..3}: two xor shuffles.  Keys, queries and
// head-dim columns beyond the problem are zero-filled at load (keys masked
// to -inf), so any seq_n, block_m and head_dim work.
//
// Blocks narrower than a wave (the runner's default --threads 32) take a
// scalar path: threads split the keys for the scores and the head dimension
// for P.V, with LDS tree reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wave_common.hpp"

namespace wave {
namespace attention {

// Output columns per unit: 8 accumulator tiles of 16.
constexpr int kSmallCols = 128;

// 8 consecutive halves row[c .. c+7] of a row-major [rows x ld] f16 matrix
// as packed MFMA operand bits; elements at or beyond `cols`, or of an
// invalid row, read as zero.
__device__ __forceinline__ u32x4 small_load8(const _Float16 *base, int row, bool row_ok, int c,
                                             int ld, int cols) {
  u32x4 r = {0u, 0u, 0u, 0u};
  if (!row_ok || c >= cols)
    return r;
  const _Float16 *p = base + (size_t)row * ld + c;
  if (c + 8 <= cols && ((reinterpret_cast<uintptr_t>(p) & 15u) == 0))
    return *reinterpret_cast<const u32x4 *>(p);
  const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (c + e < cols)
      w[e >> 1] |= (uint32_t)h[e] << (16 * (e & 1));
  r[0] = w[0];
  r[1] = w[1];
  r[2] = w[2];
  r[3] = w[3];
  return r;
}

__device__ __forceinline__ uint32_t small_pack_f16(float lo, float hi) {
  const _Float16 a = (_Float16)lo, b = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) |
         ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

__device__ __forceinline__ float small_wave_max4(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  return fmaxf(v, __shfl_xor(v, 32));
}

__device__ __forceinline__ float small_wave_sum4(float v) {
  v += __shfl_xor(v, 16);
  return v + __shfl_xor(v, 32);
}

// One unit: O[q0 .. q0+16)[c0 .. c0+128) on the calling (full) wave.
__device__ __forceinline__ void small_mfma_unit(const _Float16 *Q, const _Float16 *K,
                                                const _Float16 *V, float *O, int block_m,
                                                int seq_n, int D, int q0, int c0) {
  const int lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int qrow = q0 + col;
  const bool q_ok = qrow < block_m;
  const int tiles = min(kSmallCols, D - c0 + 15) / 16;  // accumulator tiles in use
  f32x4 acc[kSmallCols / 16];
#pragma unroll
  for (int t = 0; t < kSmallCols / 16; ++t)
    acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_inff(), l = 0.f;

  for (int n0 = 0; n0 < seq_n; n0 += 32) {
    f32x4 s[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    for (int d0 = 0; d0 < D; d0 += 32) {
      const u32x4 qf = small_load8(Q, qrow, q_ok, d0 + 8 * grp, D, D);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int key = n0 + 16 * h + col;
        const u32x4 kf = small_load8(K, key, key < seq_n, d0 + 8 * grp, D, D);
        s[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, kf),
                                                      __builtin_bit_cast(f16x8, qf), s[h], 0,
                                                      0, 0);
      }
    }
    // Slot j of this lane: key n0 + 4*grp + j (j < 4), n0 + 16 + 4*grp + j-4.
    float p[8];
    float cmax = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = n0 + (j < 4 ? 4 * grp + j : 16 + 4 * grp + j - 4);
      p[j] = key < seq_n ? s[j >> 2][j & 3] : -__builtin_inff();
      cmax = fmaxf(cmax, p[j]);
    }
    const float m_new = fmaxf(m, small_wave_max4(cmax));  // finite: key n0 exists
    const float alpha = exp2f(m - m_new);
    m = m_new;
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = exp2f(p[j] - m_new);
      psum += p[j];
    }
    l = l * alpha + psum;
    const u32x4 pf = {small_pack_f16(p[0], p[1]), small_pack_f16(p[2], p[3]),
                      small_pack_f16(p[4], p[5]), small_pack_f16(p[6], p[7])};
#pragma unroll
    for (int t = 0; t < kSmallCols / 16; ++t) {
      if (t >= tiles)
        break;
      acc[t] *= alpha;
      // A = V^T: row c0 + 16t + col, K slots in the key order of pf.
      const int c = c0 + 16 * t + col;
      uint32_t w[4] = {0u, 0u, 0u, 0u};
      if (c < D) {
        const uint16_t *vh = reinterpret_cast<const uint16_t *>(V);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int key = n0 + (j < 4 ? 4 * grp + j : 16 + 4 * grp + j - 4);
          if (key < seq_n)
            w[j >> 1] |= (uint32_t)vh[(size_t)key * D + c] << (16 * (j & 1));
        }
      }
      const u32x4 vf = {w[0], w[1], w[2], w[3]};
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, vf),
                                                      __builtin_bit_cast(f16x8, pf), acc[t],
                                                      0, 0, 0);
    }
  }
  const float inv = 1.0f / small_wave_sum4(l);
  if (!q_ok)
    return;
#pragma unroll
  for (int t = 0; t < kSmallCols / 16; ++t) {
    if (t >= tiles)
      break;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = c0 + 16 * t + 4 * grp + i;  // O^T row = output column
      if (c < D)
        O[(size_t)qrow * D + c] = acc[t][i] * inv;
    }
  }
}

// Block-wide reduction through LDS in log2(blockDim) steps; every thread
// gets the result.  red: blockDim.x floats.
__device__ __forceinline__ float small_block_reduce(float v, bool is_max, float *red) {
  const int t = threadIdx.x, nt = blockDim.x;
  red[t] = v;
  __syncthreads();
  int span = 1;
  while (span < nt)
    span <<= 1;
  for (int s = span >> 1; s > 0; s >>= 1) {
    if (t < s && t + s < nt)
      red[t] = is_max ? fmaxf(red[t], red[t + s]) : red[t] + red[t + s];
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

// Scalar path for blocks narrower than one wave.  weights: seq_n floats of
// LDS; red: blockDim.x floats of LDS.
__device__ __forceinline__ void small_scalar(const _Float16 *Q, const _Float16 *K,
                                             const _Float16 *V, float *O, int block_m,
                                             int seq_n, int head_dim, float *weights,
                                             float *red) {
  const int t = threadIdx.x, nt = blockDim.x;
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
    mx = small_block_reduce(mx, true, red);
    float sum = 0.f;
    for (int n = t; n < seq_n; n += nt) {
      const float w = exp2f(weights[n] - mx);
      weights[n] = w;
      sum += w;
    }
    sum = small_block_reduce(sum, false, red);  // its barriers also publish the weights
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

// The whole kernel body.  weights / red are only touched on the scalar
// path (blockDim.x < 64); extra threads of a partial last wave idle.
__device__ __forceinline__ void small_cta(const _Float16 *Q, const _Float16 *K,
                                          const _Float16 *V, float *O, int block_m,
                                          int seq_n, int head_dim, float *weights,
                                          float *red) {
  const int waves = blockDim.x / 64;
  if (waves == 0) {
    small_scalar(Q, K, V, O, block_m, seq_n, head_dim, weights, red);
    return;
  }
  const int wave = threadIdx.x / 64;
  if (wave >= waves)
    return;
  const int col_groups = (head_dim + kSmallCols - 1) / kSmallCols;
  const int units = (block_m + 15) / 16 * col_groups;
  for (int u = wave; u < units; u += waves)
    small_mfma_unit(Q, K, V, O, block_m, seq_n, head_dim, 16 * (u / col_groups),
                    kSmallCols * (u % col_groups));
}

} // namespace attention
} // namespace wave
