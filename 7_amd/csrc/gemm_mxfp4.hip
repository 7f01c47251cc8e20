// gemm_mxfp4.hip -- host launch of the MXFP4 scaled GEMM: the tiled kernel
// of gemm_kernels.hpp with fp4 (e2m1) operands and e8m0 block scales, on
// v_mfma_scale_f32_32x32x64_f8f6f4.  This is the reference's `mxfp4` input
// type of wmma_f16_matmul_tiled (python/mlir/dialects/wave_matmul.py:187-206
// `mfma.scale ... f4`, :353-405 storage and scale layout, :996-1022
// reference math; runner tools/wave-matmul-calibrate/
// wave-matmul-calibrate-runner.cpp:1565-1595 decode and expected value):
//   C[m][n] = sum_k (a[m][k] * 2^(sa[k/32][m]-127)) * (b[n][k] * 2^(sb[k/32][n]-127))
// with fp32 accumulation; A, B row-major packed two fp4 per byte (low
// nibble = even k), scales group-major (the reference's canonical layout).
// With GemmArgs::aiter, B and both scale arrays come in the AITER
// preshuffled layouts instead (runner.cpp:1223-1283; wave_matmul.py:891-935):
// B byte (n, kb) at (((n/16 * K/64 + kb/32) * 2 + kb%32/16) * 16 + n%16) * 16
// + kb%16, scale (group g, row r) at (r/32 * G8 + g/8) * 256 + (g%4) * 64 +
// (r%16) * 4 + (g%8/4) * 2 + r%32/16 with rows padded to 256 and groups to
// a multiple of 8 (G8 = padded groups / 8).
#include "gemm_kernels.hpp"

namespace wave {
namespace gemm {

namespace {
template <int IN, int OUT>
hipError_t launch_out(const Params &p, bool cm, hipStream_t s) {
  const dim3 grid(p.tiles_m * p.tiles_n), block(CfgFor<IN>::THREADS);
  // Canonical layout with K a multiple of 256 values (64 16-bit units):
  // 64-deep stages (2-3 % faster at K = 8192 and 32768 than the 32-deep
  // ring, 4096^2 x K, one box).
  const bool deep = IN == kMXFP4 && p.K % 64 == 0;
  if (deep) {
    if constexpr (IN == kMXFP4) {
      if (cm)
        hipLaunchKernelGGL((tiled_kernel<IN, OUT, true, false, 8, false, false, true>), grid,
                           block, 0, s, p);
      else
        hipLaunchKernelGGL((tiled_kernel<IN, OUT, false, false, 8, false, false, true>), grid,
                           block, 0, s, p);
    }
  } else if (cm) {
    hipLaunchKernelGGL((tiled_kernel<IN, OUT, true, false, 8>), grid, block, 0, s, p);
  } else {
    hipLaunchKernelGGL((tiled_kernel<IN, OUT, false, false, 8>), grid, block, 0, s, p);
  }
  return hipGetLastError();
}
template <int IN>
hipError_t launch_in(const Params &p, int out_dtype, bool cm, hipStream_t s) {
  if (out_dtype == kF32)
    return launch_out<IN, kF32>(p, cm, s);
  if (out_dtype == kF16)
    return launch_out<IN, kF16>(p, cm, s);
  return launch_out<IN, kBF16>(p, cm, s);
}
} // namespace

hipError_t launch_mxfp4(const GemmArgs &g, hipStream_t stream) {
  Params p{};
  p.A = static_cast<const uint16_t *>(g.A);
  p.B = static_cast<const uint16_t *>(g.B);
  p.C = g.C;
  p.M = g.M;
  p.N = g.N;
  p.K = g.K / 4;  // 16-bit units: K/2 bytes per row
  p.a_scale = static_cast<const uint8_t *>(g.a_scale);
  p.b_scale = static_cast<const uint8_t *>(g.b_scale);
  p.tiles_m = g.M / kTile;
  p.tiles_n = g.N / kTile;
  p.group_m = g.group_m > 0 ? g.group_m : 4;
  if (p.group_m > p.tiles_m)
    p.group_m = p.tiles_m;
  p.ldc = g.col_major ? g.M : g.N;
  p.c_vec_ok = 1;
  if (g.aiter)
    return launch_in<kMXFP4A>(p, g.out_dtype, g.col_major, stream);
  return launch_in<kMXFP4>(p, g.out_dtype, g.col_major, stream);
}

} // namespace gemm
} // namespace wave
