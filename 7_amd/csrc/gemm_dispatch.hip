// gemm_dispatch.hip -- host-side selection of the GEMM kernel variant
// (aligned DMA path vs masked path, dtype/layout, tiled vs Stream-K).
#include "gemm_kernels.hpp"

#ifndef WAVE_GEMM_GROUP_M
#define WAVE_GEMM_GROUP_M 4
#endif

#include <vector>

namespace wave {
namespace gemm {

#define WAVE_GEMM_EXTERN(IN, OUT, SK)                                          \
  extern template hipError_t launch_variant<IN, OUT, false, SK>(               \
      const Params &, int, hipStream_t);                                       \
  extern template hipError_t launch_variant<IN, OUT, true, SK>(                \
      const Params &, int, hipStream_t);
#define WAVE_GEMM_EXTERN_IN(IN)                                                \
  WAVE_GEMM_EXTERN(IN, kF32, false)                                            \
  WAVE_GEMM_EXTERN(IN, kF16, false)                                            \
  WAVE_GEMM_EXTERN(IN, kBF16, false)                                           \
  WAVE_GEMM_EXTERN(IN, kF32, true)                                             \
  WAVE_GEMM_EXTERN(IN, kF16, true)                                             \
  WAVE_GEMM_EXTERN(IN, kBF16, true)
WAVE_GEMM_EXTERN_IN(kF16)
WAVE_GEMM_EXTERN_IN(kBF16)

template <int IN, int OUT>
static hipError_t launch_out(const Params &p, bool cm, bool sk, int mode,
                             hipStream_t s) {
  if (sk)
    return cm ? launch_variant<IN, OUT, true, true>(p, mode, s)
              : launch_variant<IN, OUT, false, true>(p, mode, s);
  return cm ? launch_variant<IN, OUT, true, false>(p, mode, s)
            : launch_variant<IN, OUT, false, false>(p, mode, s);
}

template <int IN>
static hipError_t launch_in(const Params &p, int out, bool cm, bool sk,
                            int mode, hipStream_t s) {
  if (out == kF32)
    return launch_out<IN, kF32>(p, cm, sk, mode, s);
  if (out == kF16)
    return launch_out<IN, kF16>(p, cm, sk, mode, s);
  return launch_out<IN, kBF16>(p, cm, sk, mode, s);
}

static bool aligned_to(const void *ptr, size_t bytes) {
  return ((uintptr_t)ptr % bytes) == 0;
}

// Counter maintenance for the Stream-K workspace.  A fill kernel rather than
// hipMemsetAsync so the reset can sit inside a captured HIP graph.
__global__ void zero_u32_kernel(uint32_t *p, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n)
    p[i] = 0u;
}

hipError_t zero_counters(uint32_t *counters, size_t count, hipStream_t stream) {
  if (count == 0)
    return hipSuccess;
  hipLaunchKernelGGL(zero_u32_kernel, dim3((unsigned)((count + 255) / 256)),
                     dim3(256), 0, stream, counters, count);
  return hipGetLastError();
}

hipError_t count_nonzero(const uint32_t *counters, size_t count, int *result,
                         hipStream_t stream) {
  std::vector<uint32_t> host(count);
  hipError_t e = hipMemcpyAsync(host.data(), counters, count * sizeof(uint32_t),
                                hipMemcpyDeviceToHost, stream);
  if (e != hipSuccess)
    return e;
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess)
    return e;
  int n = 0;
  for (uint32_t v : host)
    n += v != 0u;
  *result = n;
  return hipSuccess;
}

int tiles_for(int extent) { return (extent + kTile - 1) / kTile; }
int k_iterations(int K) { return (K + kSKUnit - 1) / kSKUnit; }

hipError_t launch(const GemmArgs &g, hipStream_t stream) {
  if (g.workers == 0 && !g.force_masked && !g.packed && skinny_supported(g))
    return launch_skinny(g, stream);
  Params p{};
  p.A = static_cast<const uint16_t *>(g.A);
  p.B = static_cast<const uint16_t *>(g.B);
  p.C = g.C;
  p.M = g.M;
  p.N = g.N;
  p.K = g.K;
  p.tiles_m = tiles_for(g.M);
  p.tiles_n = tiles_for(g.N);
  p.group_m = g.group_m > 0 ? g.group_m : WAVE_GEMM_GROUP_M;
  if (p.group_m > p.tiles_m)
    p.group_m = p.tiles_m;
  const bool cm = g.col_major || g.packed;
  p.ldc = cm ? g.M : g.N;
  const size_t out_bytes = g.out_dtype == kF32 ? 4 : 2;
  p.c_vec_ok = (p.ldc % 4 == 0) && aligned_to(g.C, 4 * out_bytes);
  if (g.packed) {
    p.pk = 1;
    p.pk_bm = g.pk_bm;
    p.pk_bn = g.pk_bn;
    p.pk_wmt = g.pk_wmt;
    p.pk_wnt = g.pk_wnt;
    p.pk_nblocks = g.N / (16 * g.pk_bn * g.pk_wnt);
    p.c_vec_ok = aligned_to(g.C, 4 * out_bytes);  // M % 16 == 0: whole 4-row groups
  }
  p.scratch = static_cast<float *>(g.scratch);
  p.counters = static_cast<uint32_t *>(g.counters);
  p.workers = g.workers;
  // Whole tiles take the DMA path when K is a whole number of 64-deep stages
  // (the tiled and the Stream-K kernel).
  const bool sk = g.workers > 0;
  const int stage_k = TileCfg::BK;
  const bool fast = (g.M % kTile == 0) && (g.N % kTile == 0) &&
                    (g.K % stage_k == 0) && aligned_to(g.A, 16) &&
                    aligned_to(g.B, 16) && p.c_vec_ok && !g.force_masked;
  // Ragged M / N or K off the stage: the hybrid DMA path (rows every 8
  // bytes at least, so each 16-byte DMA access is dword-aligned), unless
  // the caller forces the bounds-checked one or C is tile-packed.
  const bool hybrid = !g.force_masked && !g.packed;
  int mode = 1;
  if (fast)
    mode = 0;
  else if (g.K % 8 == 0 && aligned_to(g.A, 16) && aligned_to(g.B, 16))
    mode = hybrid ? kModeHybrid8 : 8;
  else if (g.K % 4 == 0 && aligned_to(g.A, 8) && aligned_to(g.B, 8))
    mode = hybrid ? kModeHybrid4 : 4;
  if (g.in_dtype == kF16)
    return launch_in<kF16>(p, g.out_dtype, cm, sk, mode, stream);
  return launch_in<kBF16>(p, g.out_dtype, cm, sk, mode, stream);
}

} // namespace gemm
} // namespace wave
