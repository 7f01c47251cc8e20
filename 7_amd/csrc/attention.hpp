// attention.hpp -- host-side launch interface of the flash-attention kernels
// (attention_fwd.hip: production forward, head_dim 128; fa_small.hip: the
// single-workgroup flash_attention_f32 ABI).
#pragma once

#include <hip/hip_runtime.h>

namespace wave {
namespace attention {

struct FwdArgs {
  const void *Q = nullptr;  // [batch][q_heads][seq_q][head_dim]
  const void *K = nullptr;  // [batch][kv_heads][seq_k][head_dim]
  const void *V = nullptr;  // [batch][kv_heads][seq_k][head_dim]
  void *O = nullptr;        // [batch][q_heads][seq_q][head_dim]
  int batch = 1, q_heads = 1, kv_heads = 1, seq_q = 0, seq_k = 0;
  int head_dim = 128;
  int dtype = 1;            // wave::kF16 or wave::kBF16 (Q, K, V and O)
  int causal = 0;           // mask key > query (top-left aligned)
  float scale = 0.f;        // softmax scale; 0 selects 1/sqrt(head_dim)
  float qk_max_abs = 0.f;   // > 0: |Q|, |K| <= qk_max_abs, fixed-max kernel
  int waves = 8;            // 12: three-group kernel; 8: ping-pong kernel; 4: 4-wave kernel
  float *lse = nullptr;     // optional [batch][q_heads][seq_q] row log-sum-exp
};

hipError_t launch_fwd(const FwdArgs &args, hipStream_t stream);

// Backward (attention_bwd.hip): dQ, dK, dV of O = softmax(scale Q K^T) V from
// dO, O and the forward's lse.  Layouts as FwdArgs (seq_q = seq_k = seq);
// delta: caller scratch [batch][q_heads][seq] floats.  seq % 64 == 0.
struct BwdArgs {
  const void *Q = nullptr, *K = nullptr, *V = nullptr, *O = nullptr, *dO = nullptr;
  const float *lse = nullptr;  // [batch][q_heads][seq]: ln sum_k exp(scale q.k)
  float *delta = nullptr;      // [batch][q_heads][seq] scratch
  void *dQ = nullptr, *dK = nullptr, *dV = nullptr;
  int batch = 1, q_heads = 1, kv_heads = 1, seq = 0;
  int dtype = 1;
  int causal = 0;
  float scale = 0.f;           // 0 selects 1/sqrt(128)
};
hipError_t launch_bwd(const BwdArgs &args, hipStream_t stream);

// Block-scaled FP8 forward (attention_fwd8.hip): Q, K, V e4m3 bytes in the
// FwdArgs layouts (head_dim 128), e8m0 scales Q_scale [batch][q_heads][seq_q]
// [4] and K_scale [batch][kv_heads][seq_k][4] (blocks of 32 d), V_scale
// [batch][kv_heads][ceil(seq_k / 32)][128] (blocks of 32 keys); O f16 / bf16.
struct Fp8FwdArgs {
  const void *Q = nullptr, *K = nullptr, *V = nullptr;
  const void *Q_scale = nullptr, *K_scale = nullptr, *V_scale = nullptr;
  void *O = nullptr;
  int batch = 1, q_heads = 1, kv_heads = 1, seq_q = 0, seq_k = 0;
  int out_dtype = 1;        // wave::kF16 or wave::kBF16
  int causal = 0;
  float scale = 0.f;        // 0 selects 1/sqrt(128)
  float *lse = nullptr;
};
hipError_t launch_fwd_fp8(const Fp8FwdArgs &args, hipStream_t stream);

// flash_attention_f32 ABI: Q [block_m][head_dim] f16 already multiplied by
// log2(e)/sqrt(head_dim), K/V [seq_n][head_dim] f16, O [block_m][head_dim]
// f32 = sum_n 2^(s_n - max) V_n / sum_n 2^(s_n - max), s_n = Q.K_n.
hipError_t launch_small(const void *Q, const void *K, const void *V, float *O,
                        int block_m, int seq_n, int head_dim, hipStream_t stream);

} // namespace attention
} // namespace wave
