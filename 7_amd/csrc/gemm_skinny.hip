// gemm_skinny.hip -- C = A . B^T for short M (M <= 128), the shape of
// BASELINE config 3a (128 x 8192 x 8192): the 256x256 tiles of
// gemm_kernels.hpp would leave half of every tile empty and run only N/256
// CTAs.  Here one CTA owns a 32-column block of N and all M rows (wave w:
// rows 32w .. 32w+31), over the whole K range, so N/32 CTAs stream B once
// from HBM while A (M x K, at most 2 MiB at K = 8192) stays in L2.  The
// roofline is HBM (arithmetic intensity ~124 FLOP/B at 128 x 8192 x 8192).
//
// The waves share nothing: each has its own LDS ring holding its 32 A rows
// and its own copy of the block's 32 B rows (the extra B copies come from
// L2), so it waits on its own DMA (vmcnt) and never on a barrier.  With the
// four waves sharing one ring through workgroup barriers the kernel measured
// 4 % slower (40.6 against 38.8 us at 128 x 8192 x 8192); the launch is
// bound by the DMA traffic per CU either way (without its MFMAs it takes
// 38.2 us).  A wave whose rows all lie past M exits at once.
//
// Requirements (checked by the dispatcher): M <= 128, K % 64 == 0, A and B
// 16-byte aligned, C vector-store aligned.  Rows past M or N are read
// clamped to the last row and never stored.
#include "gemm.hpp"
#include "wave_common.hpp"

namespace wave {
namespace gemm {

namespace {

constexpr int kBK = 64;
constexpr int kRB = 128;                 // bytes per operand row per stage
constexpr int kABytes = 32 * kRB;        // 4 KiB: the wave's A rows
constexpr int kStage = 2 * kABytes;      // + 4 KiB: B rows n0..n0+31
constexpr int kNS = 4;                   // stages in each wave's LDS ring
constexpr int kDmaPerWave = 8;           // 4 A issues + 4 B issues a stage

__device__ __forceinline__ uint32_t sw8(uint32_t r) { return (r ^ (r >> 3)) & 7u; }

struct SkinnyParams {
  const uint16_t *A, *B;
  void *C;
  int M, N, K, ldc;
};

template <int IN_DT, int OUT_DT, bool COL_MAJOR>
__global__ __launch_bounds__(256, 1) void skinny_kernel(SkinnyParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[4 * kNS * kStage];
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63;
  if ((int)(wave * 32) >= p.M)
    return;  // no rows of C for this wave (and no barrier in the kernel)
  const int n0 = blockIdx.x * 32;
  const uint32_t rowbytes = (uint32_t)p.K * 2u;

  // DMA issue i (i < 4) of a stage: local rows 8i .. 8i+7 (8 lanes a row,
  // 16-byte chunks XOR-swizzled by row) of the wave's A rows, then of B.
  uint32_t goa[4], gob[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t R = i * 8 + (lane >> 3);
    const uint32_t ch = ((lane & 7) ^ sw8(R)) << 4;
    goa[i] = (uint32_t)min((int)(wave * 32 + R), p.M - 1) * rowbytes + ch;
    gob[i] = (uint32_t)min(n0 + (int)R, p.N - 1) * rowbytes + ch;
  }
  const uint32_t ring = lds_addr(smem) + wave * (kNS * kStage);
  auto issue = [&](int s, int kt) {
    const uint32_t l = ring + s * kStage;
    const char *ab = reinterpret_cast<const char *>(p.A) + (size_t)kt * kRB;
    const char *bb = reinterpret_cast<const char *>(p.B) + (size_t)kt * kRB;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dma16(l + i * 1024, ab, goa[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dma16(l + kABytes + i * 1024, bb, gob[i]);
  };

  // Fragments: local row lane%32 of the wave's A rows and of B.
  const uint32_t r = lane & 31;
  const uint32_t off = r * kRB, swz = sw8(r) ^ (lane >> 5);
  const uint8_t *wsm = smem + wave * (kNS * kStage);
  f32x16 acc = f32x16{};
  auto compute = [&](int s) {
    const uint8_t *st = wsm + s * kStage;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint32_t x = 2 * kk;
      const u32x4 af = *reinterpret_cast<const u32x4 *>(st + off + ((x ^ swz) << 4));
      const u32x4 bf = *reinterpret_cast<const u32x4 *>(st + kABytes + off + ((x ^ swz) << 4));
      // Row-major C: MFMA rows = n (B), columns = m (A); column-major: swapped.
      if constexpr (COL_MAJOR)
        acc = mfma32x32x16<IN_DT>(af, bf, acc);
      else
        acc = mfma32x32x16<IN_DT>(bf, af, acc);
    }
  };

  const int nk = p.K / kBK;
  // Every iteration issues exactly one stage (the last stage is re-fetched
  // into the free slot near the end), so the vmcnt budget stays constant.
  // The slot refilled in iteration i was read in iteration i - 1; the
  // lgkmcnt wait makes those reads complete first.
#pragma unroll
  for (int s = 0; s + 1 < kNS; ++s)
    issue(s, min(s, nk - 1));
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerWave * (kNS - 2)) : "memory");
  int slot = 0;
  for (int i = 0; i < nk; ++i) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    issue(slot == 0 ? kNS - 1 : slot - 1, min(i + kNS - 1, nk - 1));
    compute(slot);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerWave * (kNS - 2)) : "memory");
    slot = slot == kNS - 1 ? 0 : slot + 1;
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");

  // Store: lane holds 4 consecutive values along C's contiguous dimension.
  const int mq = wave * 32 + (lane & 31), nq = n0 + (lane & 31);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int e0 = 8 * g + 4 * (lane >> 5);
    const f32x4 v = {acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]};
    // COL_MAJOR: values are m = 32w + e0 .. +3 at column nq; else n = n0 + e0
    // .. +3 at row mq.
    const int q = COL_MAJOR ? nq : mq;
    const int pp = COL_MAJOR ? (int)(wave * 32) + e0 : n0 + e0;
    const int qext = COL_MAJOR ? p.N : p.M, pext = COL_MAJOR ? p.M : p.N;
    if (q >= qext)
      continue;
    const size_t idx = (size_t)q * p.ldc + pp;
    if (pp + 3 < pext) {
      if constexpr (OUT_DT == kF32) {
        *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(p.C) + idx) = v;
      } else {
        u32x2 w = {pack2<OUT_DT>(v[0], v[1]), pack2<OUT_DT>(v[2], v[3])};
        *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(p.C) + idx) = w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (pp + e < pext) {
          if constexpr (OUT_DT == kF32)
            reinterpret_cast<float *>(p.C)[idx + e] = v[e];
          else
            reinterpret_cast<uint16_t *>(p.C)[idx + e] = to_bits<OUT_DT>(v[e]);
        }
    }
  }
}

template <int IN, int OUT>
hipError_t launch_out(const SkinnyParams &p, bool cm, hipStream_t s) {
  const dim3 grid((p.N + 31) / 32), block(256);
  if (cm)
    hipLaunchKernelGGL((skinny_kernel<IN, OUT, true>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((skinny_kernel<IN, OUT, false>), grid, block, 0, s, p);
  return hipGetLastError();
}

} // namespace

bool skinny_supported(const GemmArgs &g) {
  auto al = [](const void *ptr, size_t b) { return ((uintptr_t)ptr % b) == 0; };
  const size_t ob = g.out_dtype == 0 ? 4 : 2;
  const int ldc = g.col_major ? g.M : g.N;
  return g.workers == 0 && g.M <= 128 && g.K % kBK == 0 && g.N >= 1024 &&
         al(g.A, 16) && al(g.B, 16) && al(g.C, 4 * ob) && ldc % 4 == 0 &&
         (uint64_t)g.K * 2u * 128u < (1ull << 32) &&
         (uint64_t)g.N * g.K * 2u < (1ull << 32);
}

hipError_t launch_skinny(const GemmArgs &g, hipStream_t s) {
  SkinnyParams p{static_cast<const uint16_t *>(g.A), static_cast<const uint16_t *>(g.B),
                 g.C, g.M, g.N, g.K, g.col_major ? g.M : g.N};
  if (g.in_dtype == kF16) {
    if (g.out_dtype == kF32) return launch_out<kF16, kF32>(p, g.col_major, s);
    if (g.out_dtype == kF16) return launch_out<kF16, kF16>(p, g.col_major, s);
    return launch_out<kF16, kBF16>(p, g.col_major, s);
  }
  if (g.out_dtype == kF32) return launch_out<kBF16, kF32>(p, g.col_major, s);
  if (g.out_dtype == kF16) return launch_out<kBF16, kF16>(p, g.col_major, s);
  return launch_out<kBF16, kBF16>(p, g.col_major, s);
}

} // namespace gemm
} // namespace wave
