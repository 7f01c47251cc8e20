// gemm_inst.hip -- explicit instantiation of one (input dtype, output dtype,
// tiled|Stream-K) slice of the GEMM kernels.  The Makefile compiles this file
// once per slice (WAVE_IN / WAVE_OUT / WAVE_SK) so the slices build in
// parallel.
#include "gemm_kernels.hpp"

namespace wave {
namespace gemm {
WAVE_GEMM_INSTANTIATE(WAVE_IN, WAVE_OUT, WAVE_SK)
} // namespace gemm
} // namespace wave
