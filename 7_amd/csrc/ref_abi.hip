// ref_abi.hip -- the reference's device-side kernel ABI, for code objects
// that its runners and host flows load with hipModuleLoad.
//
// The reference compiles one kernel per shape and launches it by symbol with
// bare-pointer arguments (gpu-to-llvm{use-bare-pointers-for-kernels=true};
// examples/wave/common.py:279-288).  This file gives the same symbols and
// argument lists; the shape and element types are compile-time constants set
// with -D when the code object is built (Makefile target `hsaco`):
//
//   wmma_f16_matmul_tiled(const T* A, const T* B, C_t* C, int32 trip)
//     (wave_matmul.py:11415-11427, :6954-6982; runner.cpp:1790-1791).
//     -DWAVE_ABI_GEMM -DWAVE_ABI_M= -DWAVE_ABI_N= -DWAVE_ABI_K=
//     -DWAVE_ABI_IN=kF16|kBF16 -DWAVE_ABI_OUT=kF32|kF16|kBF16
//     -DWAVE_ABI_CM=0|1|2 (row-major, column-major, tile-packed; tile-packed
//     also takes -DWAVE_ABI_PK_BM= _BN= _WMT= _WNT=, the reference blocking
//     whose tile order C follows) [-DWAVE_ABI_THREADS=64|128|256|512|1024]
//   wmma_f16_matmul_tiled(const u8* A, const u8* B, C_t* C, const u8* A_scale,
//                         const u8* B_scale, int32 trip)
//     the reference's mxfp4 input type (wave_matmul.py:6965-6975; runner.cpp
//     :1792-1794): packed e2m1 A [M][K/2], B [N][K/2], e8m0 scales
//     [K/32][M], [K/32][N].  -DWAVE_ABI_MXFP4 -DWAVE_ABI_M= -DWAVE_ABI_N=
//     -DWAVE_ABI_K= -DWAVE_ABI_OUT=kF32|kF16|kBF16 -DWAVE_ABI_CM=0|1
//     [-DWAVE_ABI_MXFP4_AITER: B and scales in the AITER layouts
//     (--mxfp4-input-layout aiter, runner.cpp:1223-1283)]
//     [-DWAVE_ABI_THREADS=512|256]
//   gfx950_f16_streamk_gemm(const f16* A, const f16* B, f16* C, f32* scratch,
//                           u32* counters, int32 workers)
//     (wave_matmul.py:11556-11567; runner.cpp:1811-1816; column-major C,
//     runner.cpp:433-440).  -DWAVE_ABI_SK -DWAVE_ABI_SK_M= _N= _K=
//   flash_attention_bf16_gfx950(const bf16* Q, const bf16* K, const bf16* V,
//                               bf16* O)
//     (wave_flash_attention.py:1723-1728; runner wave-fa-gfx950-runner.cpp
//     :396-402).  -DWAVE_ABI_FA -DWAVE_ABI_FA_B= -DWAVE_ABI_FA_H= -DWAVE_ABI_FA_S=
//     [-DWAVE_ABI_FA_QK_MAX_ABS=b: the fixed-max profile for |Q|, |K| <= b]
//     [-DWAVE_ABI_FA_WAVES=4: the reference's 4-wave configuration]
//   flash_attention_f32(const f16* Q, const f16* K, const f16* V, f32* O)
//     (wave_attention.py:1436-1441; runner wave-fa-calibrate-runner.cpp
//     :346-361).  -DWAVE_ABI_FA32 -DWAVE_ABI_FA32_M= _N= _D=
//
// Launch contract (what the reference's launchers pass):
//  * wmma_f16_matmul_tiled: any grid (the runner's (M_blocks, N_blocks) for
//    its tiling); CTAs walk this build's 256x256 tiles in a grid-stride loop.
//    Block WAVE_ABI_THREADS (default 256), i.e. 64 * BM * BN of the
//    reference's blocking.  LDS is static (the code object's group segment):
//    the reference's GEMM kernels declare theirs statically and both of its
//    launchers pass no dynamic LDS (wave-matmul-calibrate.py:901-902; the
//    mlir-runner gpu.launch_func, wave_matmul.py:6976-6982).  `trip` is
//    accepted and unused: the K loop length follows from the baked K.
//  * MXFP4 wmma_f16_matmul_tiled: any grid (grid-stride over the tiles),
//    block 512 (8 waves, the reference's gfx950-mxfp4-256x256-8wave block)
//    or 256, static LDS; M, N % 256 == 0 and K % 128 == 0 at build time; A,
//    B and both scale arrays 16-byte aligned.
//  * gfx950_f16_streamk_gemm: grid (workers), block 256, static LDS;
//    workspace as wave_gemm_streamk_workspace_bytes.
//  * flash_attention_bf16_gfx950: grid (S/256, B*H), block 512, >= 102400
//    bytes of dynamic LDS (the reference's 8-wave profile passes 136192 with
//    hipFuncSetAttribute); built with WAVE_ABI_FA_WAVES=4: block 256,
//    >= 67584 bytes (the runner's 4-wave default --threads 256
//    --dynamic-lds 68096).  Non-causal, one KV head per query head, scale
//    1/sqrt(128).
//  * flash_attention_f32: grid (1,1,1), any block size up to 1024: whole
//    waves run the matrix-core path, a block narrower than 64 (the runner's
//    default --threads 32) the scalar one; LDS is static.
// A launch with a smaller block than the one stated, another grid than the
// one stated (Stream-K, FA) or less dynamic LDS than stated (FA) returns
// without writing anything; so does a GEMM launch whose A/B (16 bytes) or C
// (4 elements) lack the alignment its load path needs (hipMalloc'd buffers
// always have it).  A larger block the runtime refuses (launch bounds).
#include "../../include/wave_kernel_abi.h"
#include "attention_fwd4.hpp"
#include "attention_kernels.hpp"
#include "fa_small.hpp"
#include "gemm_kernels.hpp"

using namespace wave;

// The published launch contract (include/wave_kernel_abi.h) is the LDS these
// kernels declare: the GEMM rings are static, the FA kernels check their
// dynamic LDS against these sizes.
static_assert(wave::gemm::TileCfg::SMEM == WAVE_ABI_MATMUL_STATIC_LDS, "GEMM ring");
static_assert(wave::gemm::Fp4Cfg::SMEM == WAVE_ABI_MXFP4_STATIC_LDS, "MXFP4 ring");
static_assert(wave::gemm::Fp4ACfg::SMEM == WAVE_ABI_MXFP4_AITER_STATIC_LDS, "AITER ring");
static_assert(wave::gemm::DefaultCfg::SMEM + 4 == WAVE_ABI_STREAMK_STATIC_LDS, "Stream-K ring");
static_assert(wave::attention::kPPSmem == WAVE_ABI_FA_MIN_DYNAMIC_LDS, "8-wave FA LDS");
static_assert(wave::attention::kF4Smem == WAVE_ABI_FA4_MIN_DYNAMIC_LDS, "4-wave FA LDS");

namespace {
[[maybe_unused]] __device__ __forceinline__ bool aligned16(const void *p) {
  return ((uintptr_t)p & 15u) == 0;
}
// The baked shape reaches the kernel body as an opaque scalar, so the body
// compiles exactly as in the shape-generic library kernels (constant shapes
// would let the compiler specialise the tile loops, at a register cost).
[[maybe_unused]] __device__ __forceinline__ int runtime_int(int v) {
  asm volatile("" : "+s"(v));
  return v;
}
// Dynamic LDS bytes of this launch: the hidden_dynamic_lds_size implicit
// kernel argument (code object v5, offset 120 of the implicit arguments).
[[maybe_unused]] __device__ __forceinline__ uint32_t dynamic_lds_bytes() {
  return *reinterpret_cast<const uint32_t *>(
      static_cast<const char *>(__builtin_amdgcn_implicitarg_ptr()) + 120);
}
} // namespace

#ifdef WAVE_ABI_GEMM
#ifndef WAVE_ABI_THREADS
#define WAVE_ABI_THREADS 256
#endif
// Waves per CTA: the reference's BM * BN (block = 64 * BM * BN threads).
constexpr int kAbiWaves = WAVE_ABI_THREADS / 64;
static_assert(WAVE_ABI_THREADS % 64 == 0 && (kAbiWaves == 1 || kAbiWaves == 2 ||
              kAbiWaves == 4 || kAbiWaves == 8 || kAbiWaves == 16),
              "block of 64, 128, 256, 512 or 1024 threads");
using AbiGemmCfg = wave::gemm::CfgFor<WAVE_ABI_IN, kAbiWaves>;
extern "C" __global__ __launch_bounds__(WAVE_ABI_THREADS, 1) void wmma_f16_matmul_tiled(
    const uint16_t *A, const uint16_t *B, void *C, int trip) {
  using namespace wave::gemm;
  // Static LDS (the code object's group segment): the reference's kernels
  // declare their LDS statically and its launchers pass no dynamic LDS
  // (wave-matmul-calibrate.py:901-902; wave_matmul.py:6976-6982).
  __shared__ __attribute__((aligned(1024))) uint8_t smem[AbiGemmCfg::SMEM];
  (void)trip;
  if (blockDim.x != WAVE_ABI_THREADS || blockDim.y != 1 || blockDim.z != 1)
    return;
  constexpr int M = WAVE_ABI_M, N = WAVE_ABI_N, K = WAVE_ABI_K;
  constexpr int CM = WAVE_ABI_CM;  // 0 row-major, 1 column-major, 2 tile-packed
  constexpr int OUT_BYTES = WAVE_ABI_OUT == kF32 ? 4 : 2;
  static_assert(M > 0 && N > 0 && K > 0 && CM >= 0 && CM <= 2, "shape / layout");
  Params p{};
  p.A = A;
  p.B = B;
  p.C = C;
  p.M = runtime_int(M);
  p.N = runtime_int(N);
  p.K = runtime_int(K);
  p.tiles_m = (p.M + kTile - 1) / kTile;
  p.tiles_n = (p.N + kTile - 1) / kTile;
  p.group_m = min(4, p.tiles_m);
  p.ldc = CM ? p.M : p.N;
#if WAVE_ABI_CM == 2
  // The reference blocking that fixes the tile order: BM * BN waves of
  // wave_m_tiles x wave_n_tiles 16x16 tiles per CTA.
  constexpr int PBM = WAVE_ABI_PK_BM, PBN = WAVE_ABI_PK_BN;
  constexpr int PWM = WAVE_ABI_PK_WMT, PWN = WAVE_ABI_PK_WNT;
  static_assert(PBM > 0 && PBN > 0 && PWM > 0 && PWN > 0 && M % (16 * PBM * PWM) == 0 &&
                N % (16 * PBN * PWN) == 0, "tile-packed blocking must divide M and N");
  p.pk = 1;
  p.pk_bm = runtime_int(PBM);
  p.pk_bn = runtime_int(PBN);
  p.pk_wmt = runtime_int(PWM);
  p.pk_wnt = runtime_int(PWN);
  p.pk_nblocks = runtime_int(N / (16 * PBN * PWN));
  p.c_vec_ok = ((uintptr_t)C % (4 * OUT_BYTES)) == 0;
#else
  p.c_vec_ok = (p.ldc % 4 == 0) && (((uintptr_t)C % (4 * OUT_BYTES)) == 0);
#endif
  // One load path per code object, chosen from the baked shape like the
  // host dispatcher does: the DMA fast path for whole tiles, else the masked
  // path with 16-byte (K % 8 == 0) or 2-byte loads.
  constexpr bool kFast = M % kTile == 0 && N % kTile == 0 && K % AbiGemmCfg::BK == 0 &&
                         (CM == 2 || (CM ? M : N) % 4 == 0);
  constexpr int kVec = kFast || K % 8 == 0 ? 8 : 1;
  if (kVec == 8 && !(aligned16(A) && aligned16(B)))
    return;
  if (kFast && !p.c_vec_ok)
    return;
  const int tiles = p.tiles_m * p.tiles_n;
  const int ctas = gridDim.x * gridDim.y;
  for (int raw = blockIdx.y * gridDim.x + blockIdx.x; raw < tiles; raw += ctas)
    tiled_cta<WAVE_ABI_IN, WAVE_ABI_OUT, CM != 0, !kFast, kVec, kAbiWaves, CM == 2>(p, raw,
                                                                                  smem);
}
#endif

#ifdef WAVE_ABI_MXFP4
#ifdef WAVE_ABI_MXFP4_AITER
constexpr int kAbiFp4 = kMXFP4A;  // AITER-preshuffled B and scales
#else
constexpr int kAbiFp4 = kMXFP4;
#endif
#ifndef WAVE_ABI_THREADS
#define WAVE_ABI_THREADS 512
#endif
static_assert(WAVE_ABI_THREADS == 256 || WAVE_ABI_THREADS == 512,
              "MXFP4 code objects run 4 or 8 waves");
using AbiFp4Cfg = wave::gemm::CfgFor<kAbiFp4, WAVE_ABI_THREADS / 64>;
extern "C" __global__ __launch_bounds__(AbiFp4Cfg::THREADS, 1) void wmma_f16_matmul_tiled(
    const uint8_t *A, const uint8_t *B, void *C, const uint8_t *A_scale, const uint8_t *B_scale,
    int trip) {
  using namespace wave::gemm;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[AbiFp4Cfg::SMEM];
  (void)trip;
  if (blockDim.x != AbiFp4Cfg::THREADS || blockDim.y != 1 || blockDim.z != 1)
    return;
  constexpr int M = WAVE_ABI_M, N = WAVE_ABI_N, K = WAVE_ABI_K;
  static_assert(M > 0 && N > 0 && M % kTile == 0 && N % kTile == 0 && K > 0 && K % 128 == 0,
                "MXFP4 code objects take whole 256x256 tiles and K % 128 == 0");
  static_assert((uint64_t)((K / 32 + 7) / 8 * 8) * (M > N ? M : N) < (1ull << 32),
                "scale offsets");
  constexpr bool CM = WAVE_ABI_CM != 0;
  constexpr int OUT_BYTES = WAVE_ABI_OUT == kF32 ? 4 : 2;
  if (!(aligned16(A) && aligned16(B) && aligned16(A_scale) && aligned16(B_scale)) ||
      ((uintptr_t)C % (4 * OUT_BYTES)) != 0)
    return;
  Params p{};
  p.A = reinterpret_cast<const uint16_t *>(A);
  p.B = reinterpret_cast<const uint16_t *>(B);
  p.C = C;
  p.a_scale = A_scale;
  p.b_scale = B_scale;
  p.M = runtime_int(M);
  p.N = runtime_int(N);
  p.K = runtime_int(K / 4);  // 16-bit units
  p.tiles_m = p.M / kTile;
  p.tiles_n = p.N / kTile;
  p.group_m = min(4, p.tiles_m);
  p.ldc = CM ? p.M : p.N;
  p.c_vec_ok = 1;
  const int tiles = p.tiles_m * p.tiles_n;
  const int ctas = gridDim.x * gridDim.y;
  // Canonical layout with K a multiple of 256: the 64-deep stages.
  constexpr bool kDeep = kAbiFp4 == kMXFP4 && K % 256 == 0;
  for (int raw = blockIdx.y * gridDim.x + blockIdx.x; raw < tiles; raw += ctas)
    tiled_cta<kAbiFp4, WAVE_ABI_OUT, CM, false, 8, WAVE_ABI_THREADS / 64, false, false, kDeep>(
        p, raw, smem);
}
#endif

#ifdef WAVE_ABI_SK
extern "C" __global__ __launch_bounds__(256, 1) void gfx950_f16_streamk_gemm(
    const uint16_t *A, const uint16_t *B, uint16_t *C, float *scratch, uint32_t *counters,
    int workers) {
  using namespace wave::gemm;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[DefaultCfg::SMEM];
  __shared__ int arrival;
  if (blockDim.x != 256 || blockDim.y != 1 || blockDim.z != 1 || workers <= 0 ||
      (int)gridDim.x != workers)
    return;
  constexpr int M = WAVE_ABI_SK_M, N = WAVE_ABI_SK_N, K = WAVE_ABI_SK_K;
  static_assert(M > 0 && N > 0 && K > 0, "shape");
  Params p{};
  p.A = A;
  p.B = B;
  p.C = C;
  p.M = runtime_int(M);
  p.N = runtime_int(N);
  p.K = runtime_int(K);
  p.tiles_m = (p.M + kTile - 1) / kTile;
  p.tiles_n = (p.N + kTile - 1) / kTile;
  p.group_m = min(4, p.tiles_m);
  p.ldc = p.M;  // column-major C
  p.c_vec_ok = (M % 4 == 0) && (((uintptr_t)C % 8) == 0);
  p.scratch = scratch;
  p.counters = counters;
  p.workers = workers;
  constexpr bool kFast = M % kTile == 0 && N % kTile == 0 && K % HybridTileCfgW<>::BK == 0 &&
                         M % 4 == 0;
  constexpr int kVec = kFast || K % 8 == 0 ? 8 : 1;
  if (kVec == 8 && !(aligned16(A) && aligned16(B)))
    return;
  if (kFast && !p.c_vec_ok)
    return;
  streamk_cta<kF16, kF16, true, !kFast, kVec>(p, blockIdx.x, smem, &arrival);
}
#endif

#ifdef WAVE_ABI_FA
#ifndef WAVE_ABI_FA_WAVES
#define WAVE_ABI_FA_WAVES 8
#endif
static_assert(WAVE_ABI_FA_WAVES == 4 || WAVE_ABI_FA_WAVES == 8, "waves must be 4 or 8");
// The 4-wave kernel is built for two CTAs per CU (64 KiB of LDS each).
extern "C" __global__ __launch_bounds__(64 * WAVE_ABI_FA_WAVES, WAVE_ABI_FA_WAVES == 4 ? 2 : 1)
void flash_attention_bf16_gfx950(
    const uint16_t *Q, const uint16_t *K, const uint16_t *V, uint16_t *O) {
  using namespace wave::attention;
  extern __shared__ __attribute__((aligned(1024))) uint8_t dsmem[];
  constexpr int B = WAVE_ABI_FA_B, H = WAVE_ABI_FA_H, S = WAVE_ABI_FA_S;
  static_assert(B > 0 && H > 0 && S > 0, "shape");
  // Both wave counts take 256 query rows per CTA (wave_flash_attention.py:23, :93).
  constexpr int kQBlocks = (S + 255) / 256;
  constexpr int kSmem = WAVE_ABI_FA_WAVES == 4 ? kF4Smem : kPPSmem;
  if (blockDim.x != 64 * WAVE_ABI_FA_WAVES || blockDim.y != 1 || blockDim.z != 1 ||
      (int)(gridDim.x * gridDim.y) != kQBlocks * B * H || dynamic_lds_bytes() < (uint32_t)kSmem)
    return;
  Params p{};
  p.Q = Q;
  p.K = K;
  p.V = V;
  p.O = O;
  p.batch = runtime_int(B);
  p.q_heads = runtime_int(H);
  p.kv_heads = p.q_heads;
  p.seq_q = runtime_int(S);
  p.seq_k = p.seq_q;
  p.q_blocks = runtime_int(kQBlocks);
  p.causal = runtime_int(0);
  // 1/sqrt(128) * log2(e), in the same float operations as the host path.
  p.scale_log2 = (1.0f / 11.313708498984761f) * kLog2e;
#ifdef WAVE_ABI_FA_QK_MAX_ABS
  // The reference's qk_max_abs profile (wave_flash_attention.py:108-113):
  // fixed row max log2(e) * sqrt(128) * qk_max_abs^2, no online max.
  constexpr double kB = WAVE_ABI_FA_QK_MAX_ABS;
  static_assert(kB > 0 && -2.0 * 1.4426950408889634 * 11.313708498984761 * kB * kB >= -126.0,
                "qk_max_abs outside the bf16 range");
  p.fixed_max = (float)(1.4426950408889634 * (1.0 / 11.313708498984761) * 128.0 * kB * kB);
  constexpr bool kFixed = true;
#else
  constexpr bool kFixed = false;
#endif
  const int raw = blockIdx.y * gridDim.x + blockIdx.x;
  if constexpr (WAVE_ABI_FA_WAVES == 4)
    fwd4_cta<kBF16, kFixed>(p, raw, dsmem);
  else
    fwd_pp_cta<kBF16, kFixed>(p, raw, dsmem);
}
#endif

#ifdef WAVE_ABI_FA32
extern "C" __global__ __launch_bounds__(1024) void flash_attention_f32(
    const _Float16 *Q, const _Float16 *K, const _Float16 *V, float *O) {
  constexpr int M = WAVE_ABI_FA32_M, N = WAVE_ABI_FA32_N, D = WAVE_ABI_FA32_D;
  static_assert(M > 0 && N > 0 && D > 0 && N <= 16384, "shape");
  __shared__ float weights[N];
  __shared__ float red[1024];
  if (blockDim.y != 1 || blockDim.z != 1)
    return;
  wave::attention::small_cta(Q, K, V, O, M, N, D, weights, red);
}
#endif
