// gemm.hpp -- host-side launch interface of the tiled / Stream-K GEMM
// kernels in gemm.hip (used by the C ABI in wave_runtime.cpp).
#pragma once

#include <hip/hip_runtime.h>

namespace wave {
namespace gemm {

struct GemmArgs {
  const void *A = nullptr;  // [M x K] row-major, f16 or bf16
  const void *B = nullptr;  // [N x K] row-major, same type as A
  void *C = nullptr;        // [M x N] row-major or [N x M] (column-major)
  int M = 0, N = 0, K = 0;
  int in_dtype = 1;         // wave::kF16 / wave::kBF16
  int out_dtype = 1;        // wave::kF32 / kF16 / kBF16
  bool col_major = false;
  int group_m = 0;          // tile-row group size; 0 = default (4)
  void *scratch = nullptr;  // Stream-K fp32 partials (workers*2*256*256)
  void *counters = nullptr; // Stream-K per-tile arrival counters (zeroed)
  int workers = 0;          // > 0 selects the Stream-K kernel
  bool force_masked = false;
  // MXFP4 (in_dtype kMXFP4): A [M][K/2], B [N][K/2] packed fp4; e8m0 scales
  // group-major [K/32][M] and [K/32][N].
  const void *a_scale = nullptr;
  const void *b_scale = nullptr;
  // MXFP4 with B and both scales in the AITER preshuffled layouts.
  bool aiter = false;
  // Tile-packed C for the reference blocking (bm, bn, wave_m_tiles,
  // wave_n_tiles); computed in the column-major orientation.
  bool packed = false;
  int pk_bm = 1, pk_bn = 1, pk_wmt = 1, pk_wnt = 1;
};

constexpr int kTileEdge = 256;
constexpr int kKStage = 64;

int tiles_for(int extent);
int k_iterations(int K);
hipError_t launch(const GemmArgs &args, hipStream_t stream);
// MXFP4 scaled GEMM (gemm_mxfp4.hip): M, N % 256 == 0, K % 128 == 0.
hipError_t launch_mxfp4(const GemmArgs &args, hipStream_t stream);
// Short-M kernel (gemm_skinny.hip): M <= 128, K % 64 == 0, aligned.
bool skinny_supported(const GemmArgs &args);
hipError_t launch_skinny(const GemmArgs &args, hipStream_t stream);
// Split-K short-M kernel (gemm_skinny.hip): `bn`-column CTAs over
// `splits` K ranges, fp32 partials in `slots` (skinny_split_slot_bytes)
// reduced in the launch by each column block's last arriver, through
// `counters` (skinny_split_counter_count 64-bit words, 8-byte aligned, any
// contents before the launch: a word counts only under the launch's
// nonzero `epoch`; left zero).  skinny_split_plan: the plan for the shape
// on `cus` CUs,
// splits == 0 when the shape takes the unsplit kernel (pointers and C's
// leading dimension are checked by skinny_supported).
struct SplitPlan {
  int splits = 0;
  int bn = 128;
};
SplitPlan skinny_split_plan(int M, int N, int K, int cus);
size_t skinny_split_slot_bytes(int N, const SplitPlan &plan);
size_t skinny_split_counter_count(int N, const SplitPlan &plan);
hipError_t launch_skinny_split(const GemmArgs &args, const SplitPlan &plan, float *slots,
                               unsigned long long *counters, uint32_t epoch,
                               hipStream_t stream);

} // namespace gemm
} // namespace wave
