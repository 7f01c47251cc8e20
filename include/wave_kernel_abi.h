/* wave_kernel_abi.h -- device-side kernel ABI of the reference-ABI code
 * objects (7_amd/hsaco/<name>.hsaco, built from 7_amd/csrc/ref_abi.hip).
 *
 * The reference compiles one kernel per shape and its runners launch it by
 * symbol through hipModuleLoad / hipModuleGetFunction /
 * hipModuleLaunchKernel with bare-pointer arguments
 * (gpu-to-llvm{use-bare-pointers-for-kernels=true}, examples/wave/
 * common.py:279-288).  The code objects built here export the same symbols
 * with the same argument lists, so a runner can load them in place of the
 * reference's HSACO.  The shape and element types are baked in when a code
 * object is built:
 *
 *   make -C 7_amd/csrc hsaco NAME=<name> DEFS="-DWAVE_ABI_GEMM -DWAVE_ABI_M=..
 *        -DWAVE_ABI_N=.. -DWAVE_ABI_K=.. -DWAVE_ABI_IN=kF16|kBF16
 *        -DWAVE_ABI_OUT=kF32|kF16|kBF16 -DWAVE_ABI_CM=0|1|2
 *        [-DWAVE_ABI_THREADS=64|128|256|512|1024]"
 *
 * The structs below are the explicit kernel-argument blocks (what
 * kernelParams points at, in order); nothing here is a host-callable
 * function.
 *
 * LDS.  The GEMM, MXFP4 and Stream-K kernels hold their LDS ring in the code
 * object's static group segment (*_STATIC_LDS below, the
 * .group_segment_fixed_size of the object) and take no dynamic LDS: launch
 * them with sharedMemBytes = 0, as the reference's launchers do
 * (tools/wave-matmul-calibrate/wave-matmul-calibrate.py:901-902; the
 * mlir-runner gpu.launch_func, python/mlir/dialects/wave_matmul.py
 * :6976-6982).  Static plus dynamic LDS may not exceed the 160 KiB of a
 * gfx950 CU, so a launch that adds dynamic LDS beyond WAVE_ABI_LDS_LIMIT -
 * *_STATIC_LDS is refused by the runtime.  The flash-attention kernels are
 * the other way round: no static LDS, and at least *_MIN_DYNAMIC_LDS bytes
 * of dynamic LDS (the reference's FA runner sets it with
 * hipFuncSetAttribute, wave-fa-gfx950-runner.cpp:425-428).
 *
 * A launch with another block size than the one stated, another grid than
 * the one stated (Stream-K, FA), less dynamic LDS than stated (FA), or
 * operands without the alignment the object's load path needs (16-byte A/B,
 * C aligned to 4 elements; hipMalloc'd buffers always have it) returns
 * without writing its outputs.
 */
#ifndef WAVE_KERNEL_ABI_H
#define WAVE_KERNEL_ABI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* LDS bytes a gfx950 workgroup can hold (static + dynamic). */
#define WAVE_ABI_LDS_LIMIT 163840

/* wmma_f16_matmul_tiled(const T* A, const T* B, C_t* C, int32 trip)
 * Replaces: the kernel emitted by python/mlir/dialects/wave_matmul.py
 *   :11415-11427 (args :6954-6982), launched by tools/wave-matmul-calibrate/
 *   wave-matmul-calibrate-runner.cpp:1852-1860 (args :1790-1791).
 * A [M][K], B [N][K] row-major (T = f16 or bf16); C [M][N] row-major,
 * column-major or tile-packed (C_t = f32, f16 or bf16); fp32 accumulation.
 * Launch: any grid (CTAs walk the 256x256 output tiles in a grid-stride
 *   loop; the runner's (M_blocks, N_blocks) works); block = the object's
 *   WAVE_ABI_THREADS (64 * BM * BN of the reference's blocking: 64, 128,
 *   256, 512 or 1024; WAVE_ABI_MATMUL_BLOCK when built without it), which
 *   is also its .max_flat_workgroup_size; static LDS
 *   WAVE_ABI_MATMUL_STATIC_LDS, dynamic LDS 0.  `trip` is accepted and
 *   unused (the K loop length follows from the baked K). */
#define WAVE_ABI_MATMUL_SYMBOL "wmma_f16_matmul_tiled"
#define WAVE_ABI_MATMUL_BLOCK 256
#define WAVE_ABI_MATMUL_STATIC_LDS 131072
#define WAVE_ABI_MATMUL_DYNAMIC_LDS 0
typedef struct {
  const void *A;
  const void *B;
  void *C;
  int32_t trip;
} wave_abi_matmul_args;

/* wmma_f16_matmul_tiled(const u8* A, const u8* B, C_t* C, const u8* A_scale,
 *                       const u8* B_scale, int32 trip), the mxfp4 input type
 * Replaces: the same kernel built with input_type="mxfp4"
 *   (python/mlir/dialects/wave_matmul.py:6965-6975 argument list, :187-206
 *   MFMA; runner wave-matmul-calibrate-runner.cpp:1792-1794 argument block).
 * A [M][K/2], B [N][K/2] packed e2m1 (low nibble = even k); A_scale
 * [K/32][M], B_scale [K/32][N] e8m0 (canonical layout), or B and the scales
 * in the AITER layouts when built with -DWAVE_ABI_MXFP4_AITER; C as above
 * (row- or column-major).
 * Built with: make hsaco NAME=mxfp4_<...> DEFS="-DWAVE_ABI_MXFP4 -DWAVE_ABI_M=..
 *   -DWAVE_ABI_N=.. -DWAVE_ABI_K=.. -DWAVE_ABI_OUT=kF32|kF16|kBF16 -DWAVE_ABI_CM=0|1
 *   [-DWAVE_ABI_MXFP4_AITER] [-DWAVE_ABI_THREADS=256]"
 *   (M, N % 256 == 0, K % 128 == 0).
 * Launch: any grid (grid-stride over the 256x256 tiles); block 512 (the
 *   reference's 8-wave MXFP4 block), or 256 when built so; static LDS
 *   WAVE_ABI_MXFP4_STATIC_LDS (AITER: WAVE_ABI_MXFP4_AITER_STATIC_LDS),
 *   dynamic LDS 0; A, B and the scales 16-byte aligned.  `trip` is accepted
 *   and unused. */
#define WAVE_ABI_MXFP4_SYMBOL "wmma_f16_matmul_tiled"
#define WAVE_ABI_MXFP4_BLOCK 512
#define WAVE_ABI_MXFP4_STATIC_LDS 139264
#define WAVE_ABI_MXFP4_AITER_STATIC_LDS 147456
#define WAVE_ABI_MXFP4_DYNAMIC_LDS 0
typedef struct {
  const void *A;
  const void *B;
  void *C;
  const void *A_scale;
  const void *B_scale;
  int32_t trip;
} wave_abi_mxfp4_args;

/* gfx950_f16_streamk_gemm(const f16* A, const f16* B, f16* C, f32* scratch,
 *                         u32* counters, int32 workers)
 * Replaces: python/mlir/dialects/wave_matmul.py:11556-11567, launched by
 *   wave-matmul-calibrate-runner.cpp:1811-1816; C column-major
 *   (runner.cpp:433-440).  scratch / counters as
 *   wave_gemm_streamk_workspace_bytes (include/wave_runtime.h); counters
 *   zero before the launch and zero again after it.
 * Launch: grid (workers), block WAVE_ABI_STREAMK_BLOCK; static LDS
 *   WAVE_ABI_STREAMK_STATIC_LDS (the ring plus the arrival word), dynamic
 *   LDS 0. */
#define WAVE_ABI_STREAMK_SYMBOL "gfx950_f16_streamk_gemm"
#define WAVE_ABI_STREAMK_BLOCK 256
#define WAVE_ABI_STREAMK_STATIC_LDS 131076
#define WAVE_ABI_STREAMK_DYNAMIC_LDS 0
typedef struct {
  const void *A;
  const void *B;
  void *C;
  float *scratch;
  uint32_t *counters;
  int32_t workers;
} wave_abi_streamk_args;

/* flash_attention_bf16_gfx950(const bf16* Q, const bf16* K, const bf16* V,
 *                             bf16* O)
 * Replaces: python/mlir/dialects/wave_flash_attention.py:1723-1728,
 *   launched by tools/wave-fa-calibrate/wave-fa-gfx950-runner.cpp:396-428.
 * Q, K, V, O [B*H][S][128] bf16; non-causal; scale 1/sqrt(128).
 * Launch: grid (S/256, B*H), block 512, no static LDS and at least
 *   WAVE_ABI_FA_MIN_DYNAMIC_LDS bytes of dynamic LDS (the runner's 8-wave
 *   setting --threads 512 --dynamic-lds 136192 works).
 * Built with -DWAVE_ABI_FA_WAVES=4 (the reference's waves=4 configuration,
 *   wave_flash_attention.py:44-93): block 256, dynamic LDS >=
 *   WAVE_ABI_FA4_MIN_DYNAMIC_LDS, so the runner's 4-wave default
 *   --threads 256 --dynamic-lds 68096 works; two such CTAs share a CU. */
#define WAVE_ABI_FA_SYMBOL "flash_attention_bf16_gfx950"
#define WAVE_ABI_FA_BLOCK 512
#define WAVE_ABI_FA_STATIC_LDS 0
#define WAVE_ABI_FA_MIN_DYNAMIC_LDS 102400
#define WAVE_ABI_FA4_BLOCK 256
#define WAVE_ABI_FA4_MIN_DYNAMIC_LDS 67584
typedef struct {
  const void *Q;
  const void *K;
  const void *V;
  void *O;
} wave_abi_fa_args;

/* flash_attention_f32(const f16* Q, const f16* K, const f16* V, f32* O)
 * Replaces: python/mlir/dialects/wave_attention.py:1436-1441, launched by
 *   tools/wave-fa-calibrate/wave-fa-calibrate-runner.cpp:346-361.
 * Q [block_m][D] f16 (pre-scaled by log2(e)/sqrt(D)), K, V [seq_n][D] f16,
 * O [block_m][D] f32.
 * Launch: grid (1,1,1), any block size up to WAVE_ABI_FA32_MAX_BLOCK;
 *   static LDS WAVE_ABI_FA32_STATIC_LDS(seq_n) (the softmax weights and a
 *   reduction buffer), no dynamic LDS. */
#define WAVE_ABI_FA32_SYMBOL "flash_attention_f32"
#define WAVE_ABI_FA32_MAX_BLOCK 1024
#define WAVE_ABI_FA32_STATIC_LDS(seq_n) (4 * ((seq_n) + 1024))
typedef struct {
  const void *Q;
  const void *K;
  const void *V;
  float *O;
} wave_abi_fa32_args;

#ifdef __cplusplus
}
#endif

#endif /* WAVE_KERNEL_ABI_H */
