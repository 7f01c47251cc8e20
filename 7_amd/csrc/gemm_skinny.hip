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

// ------------------------------------------------------------ split-K
// The same product with wider column blocks and a K split: CTA (tile, split)
// owns C's BN-column block `tile` (BN = 128 or 64) and all M rows over one
// of `splits` contiguous K ranges (whole 64-deep stages, split j taking
// stages [j*q + min(j, r), +q + (j < r)) of nk = q*splits + r).  A CTA of
// the unsplit kernel streams all of A (M x K) through LDS for 32 columns;
// here it streams 1/splits of A for BN columns, so at 128 x 8192 x 8192
// with BN = 128 and 4 splits each CU moves 1 MiB a launch instead of 4 MiB
// and the L2 -> LDS traffic (which bounds the unsplit kernel) falls under
// B's HBM stream.
//
// The four waves share one LDS ring of stages holding A rows 0..127, then
// the block's BN B rows, each wave issuing a quarter of every stage; wave
// w computes a (128 / WM) x (BN / WN) block of C, WM x WN = 2 x 2 waves at
// BN = 128 and 4 x 1 at BN = 64.  One barrier a stage: after it every
// wave's DMA of the stage has landed and every wave has finished reading
// the slot the next issue overwrites.
//
// Reduction: each contributor takes an arrival ticket on the tile's first
// counter when its K range is done.  All but the last store their fp32
// partials (16-byte groups at f32x4 index group*256 + thread, fully
// coalesced) to their slots with device-scope stores and, once those are
// acknowledged, count themselves on the second counter; the last arriver
// waits for that count, reads the partials with device-scope loads (no
// release or acquire: the data never sits in a non-coherent cache), sums
// them in split order (its own from its accumulators),
// s = ((p_0 + p_1) + p_2) + p_3, so the result does not depend on arrival
// order, stores C, and resets both counters to zero.
// Splits of a tile take consecutive CTA numbers after the XCD renumbering
// (workgroup i runs on XCD i % 8), so they run on one XCD.
//
// Counter words are 64-bit: the launch's epoch (nonzero, from the host) in
// the high half, a count in the low half, and a word that carries any
// other epoch counts as zero.  So a workspace needs no clearing before a
// launch -- neither a fresh one nor one another launch left (which leaves
// zeros) -- and the launch is one kernel, not a fill kernel and this one
// (the fill and its kernel boundary cost 4-5 us at 128 x 8192 x 8192).
// The reset to zero keeps replays of a captured launch, whose epoch is
// fixed, correct.
constexpr int kXMaxSplits = 4;

typedef unsigned long long u64;
__device__ __forceinline__ uint32_t epoch_count(u64 w, uint32_t epoch) {
  return (uint32_t)(w >> 32) == epoch ? (uint32_t)w : 0u;
}
// Counts one arrival on *c for this launch and returns the count before it.
// The first guess is the zero every launch leaves, so the common first
// arrival takes one atomic round trip; each failed exchange means another
// contributor's succeeded (at most splits - 1) or the word was stale.
__device__ __forceinline__ uint32_t epoch_increment(u64 *c, uint32_t epoch) {
  u64 old = 0;
  for (;;) {
    const uint32_t n = epoch_count(old, epoch);
    if (__hip_atomic_compare_exchange_strong(c, &old, ((u64)epoch << 32) | (n + 1u),
                                             __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT))
      return n;
  }
}

template <int BN> struct SplitCfg {
  static_assert(BN == 128 || BN == 64, "column block");
  static constexpr int WN = BN == 128 ? 2 : 1, WM = 4 / WN;
  static constexpr int TI = 128 / WM / 32, TJ = BN / WN / 32;  // MFMA tiles a wave
  static constexpr int NG = TI * TJ * 4;      // 16-byte partial groups a thread
  static constexpr int AB = 128 * kRB;        // A rows of a stage: 16 KiB
  static constexpr int STAGE = AB + BN * kRB; // + B rows
  static constexpr int NS = BN == 128 ? 4 : 5;
  static constexpr int BI = BN / 32;          // B DMA issues per wave a stage
  static constexpr int DMA = 4 + BI;          // DMA issues per wave a stage
  static constexpr int SLOT = 128 * BN;       // floats per partial slot
};

struct SplitParams {
  const uint16_t *A, *B;
  void *C;
  float *slots;         // [tiles * splits][128 * BN]
  unsigned long long *counters;  // [tiles][2] arrived, published (epoch << 32 | count)
  int M, N, K, ldc, splits;
  uint32_t epoch;       // nonzero; the tag of this launch's counts
};

template <int IN_DT, int OUT_DT, bool COL_MAJOR, int BN>
__global__ __launch_bounds__(256, 1) void skinny_split_kernel(SplitParams p) {
  using X = SplitCfg<BN>;
  constexpr int TI = X::TI, TJ = X::TJ, NG = X::NG, NS = X::NS;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * X::STAGE];
  __shared__ uint32_t arrival;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63;
  int id = blockIdx.x;
  if ((gridDim.x & 7) == 0)
    id = (id & 7) * (int)(gridDim.x >> 3) + (id >> 3);
  const int tile = id / p.splits, split = id - tile * p.splits;
  const int n0 = tile * BN;
  const int nk = p.K / kBK;
  const int q = nk / p.splits, rem = nk - q * p.splits;
  const int k0 = split * q + min(split, rem), len = q + (split < rem ? 1 : 0);
  const uint32_t rowbytes = (uint32_t)p.K * 2u;

  // DMA issue i of a stage: local rows 32*wave + 8i .. +7 of A (i < 4),
  // then of B (i < BI; B rows 8 * (BI * wave + i) ..), 8 lanes a row,
  // 16-byte chunks XOR-swizzled by row.
  uint32_t goa[4], gob[X::BI], lb[X::BI];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t R = wave * 32 + i * 8 + (lane >> 3);
    goa[i] = (uint32_t)min((int)R, p.M - 1) * rowbytes + (((lane & 7) ^ sw8(R)) << 4);
  }
#pragma unroll
  for (int i = 0; i < X::BI; ++i) {
    const uint32_t R = (wave * X::BI + i) * 8 + (lane >> 3);
    gob[i] = (uint32_t)min(n0 + (int)R, p.N - 1) * rowbytes + (((lane & 7) ^ sw8(R)) << 4);
    lb[i] = X::AB + (wave * X::BI + i) * 1024;
  }
  const uint32_t ring = lds_addr(smem);
  auto issue = [&](int s, int kt) {
    const uint32_t l = ring + s * X::STAGE;
    const char *ab = reinterpret_cast<const char *>(p.A) + (size_t)kt * kRB;
    const char *bb = reinterpret_cast<const char *>(p.B) + (size_t)kt * kRB;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dma16(l + wave * 4096 + i * 1024, ab, goa[i]);
#pragma unroll
    for (int i = 0; i < X::BI; ++i)
      dma16(l + lb[i], bb, gob[i]);
  };

  const uint32_t wm = wave / X::WN, wn = wave % X::WN;
  const uint32_t rr = lane & 31, h = lane >> 5;
  constexpr int RM = 128 / X::WM, RN = BN / X::WN;  // rows / columns of a wave's block
  uint32_t offa[TI], swa[TI], offb[TJ], swb[TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    const uint32_t ra = wm * RM + i * 32 + rr;
    offa[i] = ra * kRB;
    swa[i] = sw8(ra) ^ h;
  }
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const uint32_t rb = wn * RN + j * 32 + rr;
    offb[j] = X::AB + rb * kRB;
    swb[j] = sw8(rb) ^ h;
  }
  // Waves whose rows all lie past M skip their MFMAs (they still carry
  // their share of the DMA and the barriers).
  const bool active = (int)(wm * RM) < p.M;
  f32x16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
      acc[i][j] = f32x16{};
  auto compute = [&](int s) {
    const uint8_t *st = smem + s * X::STAGE;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint32_t x = 2 * kk;
      u32x4 af[TI], bf[TJ];
#pragma unroll
      for (int i = 0; i < TI; ++i)
        af[i] = *reinterpret_cast<const u32x4 *>(st + offa[i] + ((x ^ swa[i]) << 4));
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        bf[j] = *reinterpret_cast<const u32x4 *>(st + offb[j] + ((x ^ swb[j]) << 4));
      // Row-major C: MFMA rows = n (B), columns = m (A); column-major: swapped.
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = COL_MAJOR ? mfma32x32x16<IN_DT>(af[i], bf[j], acc[i][j])
                                : mfma32x32x16<IN_DT>(bf[j], af[i], acc[i][j]);
    }
  };

  // Every iteration issues exactly one stage (the last stage is re-fetched
  // into the free slot near the end), so the vmcnt budget stays constant:
  // NS - 1 stages in flight after each issue.
#pragma unroll
  for (int s = 0; s + 1 < NS; ++s)
    issue(s, k0 + min(s, len - 1));
  int slot = 0;
  for (int i = 0; i < len; ++i) {
    vm_wait_barrier<X::DMA * (NS - 2)>();
    issue(slot == 0 ? NS - 1 : slot - 1, k0 + min(i + NS - 1, len - 1));
    if (active)
      compute(slot);
    slot = slot == NS - 1 ? 0 : slot + 1;
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");

  // 16-byte group g2 (0 .. NG-1) of the thread's partial: MFMA tile
  // (i, j) = (g2 / (4 TJ), g2 / 4 % TJ), accumulator registers
  // 4*(g2 % 4) .. +3.
  auto group = [&](int g2) {
    const f32x16 &a = acc[g2 / (4 * TJ)][(g2 / 4) % TJ];
    const int g = g2 & 3;
    return f32x4{a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]};
  };
  f32x4 out[NG];
  if (p.splits > 1) {
    // Arrival ticket first: the last of the tile's contributors to finish
    // its K range reduces and never publishes its own partial; the others
    // publish and then count themselves published with a release.
    if (threadIdx.x == 0)
      arrival = epoch_increment(&p.counters[2 * tile], p.epoch);
    __syncthreads();
    if (arrival != (uint32_t)p.splits - 1) {
      // Device-scope (sc1) stores: written through to the device's
      // coherence point, so the release below has no dirty L2 lines of
      // them to write back (35.4 against 37.4 us at 128 x 8192 x 8192).
      const __amdgpu_buffer_rsrc_t mine = coherent_rsrc(p.slots + (size_t)id * X::SLOT, X::SLOT * 4);
#pragma unroll
      for (int g2 = 0; g2 < NG; ++g2)
        coherent_store16(mine, (g2 * 256 + threadIdx.x) * 16, group(g2));
      // Every wave's partial stores are acknowledged at the coherence
      // point before the barrier, so thread 0's count, issued after it,
      // needs no release (whose L2 write-back measured 1-4 us a launch):
      // the reader's device-coherent loads below find them there.
      vm_wait_barrier();
      if (threadIdx.x == 0)
        epoch_increment(&p.counters[2 * tile + 1], p.epoch);
      return;
    }
    // Last arriver: every other contributor has taken its ticket, so it is
    // resident and finishes its publish without waiting on anything; the
    // wait below ends once the last of them has.  Both counters then go
    // back to zero (no contributor touches them again in this launch).  The
    // wait is bounded (2^20 polls, about a second): only a counter word that
    // already held this launch's epoch before it started (a chance of about
    // 2^-32 a word for arbitrary contents) could keep it from ending, and
    // then the launch still finishes.
    if (threadIdx.x == 0) {
      for (uint32_t poll = 0;
           poll < (1u << 20) &&
           epoch_count(__hip_atomic_load(&p.counters[2 * tile + 1], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT),
                       p.epoch) != (uint32_t)p.splits - 1;
           ++poll)
        __builtin_amdgcn_s_sleep(1);
      __hip_atomic_store(&p.counters[2 * tile], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&p.counters[2 * tile + 1], 0ull, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    // The other contributors' partials, all loads in flight at once: other
    // o (0 .. splits-2) is split o + (o >= split).  They are device-scope
    // (sc1) loads, the cache policy of agent-scope atomic loads, so they
    // read the coherence point the publishers' sc1 stores were
    // acknowledged at before their counts, and no acquire (an L2
    // invalidate, 1-3 us a launch) is needed; the barrier above issues
    // them after thread 0 has seen every count.
    const __amdgpu_buffer_rsrc_t peers =
        coherent_rsrc(p.slots + (size_t)tile * p.splits * X::SLOT, p.splits * X::SLOT * 4);
    f32x4 x[kXMaxSplits - 1][NG];
#pragma unroll
    for (int o = 0; o < kXMaxSplits - 1; ++o) {
      if (o + 1 < p.splits) {
        const int c = o + (o >= split ? 1 : 0);
#pragma unroll
        for (int g2 = 0; g2 < NG; ++g2)
          x[o][g2] = coherent_load16(
              peers, ((uint32_t)c * (X::SLOT / 4) + g2 * 256 + threadIdx.x) * 16);
      }
    }
    // Sum in split order; contributor c is this CTA's own (c == split) or
    // other c - (c > split).
#pragma unroll
    for (int g2 = 0; g2 < NG; ++g2) {
      const f32x4 own = group(g2);
      f32x4 s = split == 0 ? own : x[0][g2];
#pragma unroll
      for (int c = 1; c < kXMaxSplits; ++c) {
        if (c < p.splits) {
          const int lo = c < kXMaxSplits - 1 ? c : kXMaxSplits - 2;  // constant once unrolled
          const f32x4 v = c == split ? own : (c < split ? x[lo][g2] : x[c - 1][g2]);
          s += v;
        }
      }
      out[g2] = s;
    }
  } else {
#pragma unroll
    for (int g2 = 0; g2 < NG; ++g2)
      out[g2] = group(g2);
  }

  // Store: each 16-byte group holds 4 consecutive values along C's
  // contiguous dimension.
#pragma unroll
  for (int g2 = 0; g2 < NG; ++g2) {
    const int i = g2 / (4 * TJ), j = (g2 / 4) % TJ, g = g2 & 3;
    const int e0 = 8 * g + 4 * (int)h;
    // Row-major: n = n0 + RN wn + 32j + e0 .. +3 at row m = RM wm + 32i + rr;
    // column-major: m = RM wm + 32i + e0 .. +3 at column n = n0 + RN wn + 32j + rr.
    const int mb = (int)(wm * RM) + 32 * i, nb = n0 + (int)(wn * RN) + 32 * j;
    const int q = COL_MAJOR ? nb + (int)rr : mb + (int)rr;
    const int pp = COL_MAJOR ? mb + e0 : nb + e0;
    const int qext = COL_MAJOR ? p.N : p.M, pext = COL_MAJOR ? p.M : p.N;
    if (q >= qext)
      continue;
    const f32x4 v = out[g2];
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

template <int IN, int OUT, int BN>
hipError_t launch_split_bn(const SplitParams &p, bool cm, hipStream_t s) {
  const int tiles = (p.N + BN - 1) / BN;
  const dim3 grid((unsigned)(tiles * p.splits)), block(256);
  if (cm)
    hipLaunchKernelGGL((skinny_split_kernel<IN, OUT, true, BN>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((skinny_split_kernel<IN, OUT, false, BN>), grid, block, 0, s, p);
  return hipGetLastError();
}

template <int IN, int OUT>
hipError_t launch_split_out(const SplitParams &p, int bn, bool cm, hipStream_t s) {
  return bn == 128 ? launch_split_bn<IN, OUT, 128>(p, cm, s) : launch_split_bn<IN, OUT, 64>(p, cm, s);
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

SplitPlan skinny_split_plan(int M, int N, int K, int cus) {
  SplitPlan plan;
  if (M > 128 || N < 1024 || K % kBK != 0 || (uint64_t)K * 2u * 128u >= (1ull << 32) ||
      (uint64_t)N * K * 2u >= (1ull << 32))
    return plan;
  // 64-column blocks when they leave room for at least two splits, else
  // 128-column ones; at most 4 splits (at least 2 when the unsplit kernel
  // would take more than one round of CTAs), at least 8 stages a split.
  // The split pays its partial exchange (a few us at 256 CUs: the wait for
  // the last publisher, the partial loads, the sums), so it runs only where
  // each split keeps at least 4096 of K, or 2048 where M > 96 and the
  // unsplit kernel's N / 32 CTAs fill the CUs.  Measured (bf16, us,
  // unsplit / this plan, fill kernel included): 128 x N x 8192 with
  // N = 1024 31.2 / 21.5, 2048 33.7 / 21.2, 4096 34.8 / 23.7, 6144
  // 39.9 / 31.6, 8192 38.5 / 32.2, 12288 70.9 / 44.1, 16384 94.5 / 53.6,
  // 24576 153.2 / 105.7; 128 x N x 4096 with N = 8192 23.2 / 21.4, 16384
  // 44.3 / 31.3; M x 8192 x 8192 with M = 1 33.0 / 29.6, 32 34.7 / 30.7,
  // 64 35.5 / 31.5, 96 36.1 / 32.6; 100 x 5000 x 12288 49.5 / 32.3.  Not
  // split: 128 x 6144 x 4096 18.9 (20.8 in two splits), 32 x 8192 x 4096
  // 20.1 (19.8), 128 x 8192 x 2048 11.3 (16.2), 128 x 2048 x 2048 9.6
  // (13.2 in four).
  const int nk = K / kBK;
  const int unsplit = (N + 31) / 32;  // CTAs of the unsplit kernel
  for (int bn : {64, 128}) {
    const int tiles = (N + bn - 1) / bn;
    int s = cus / tiles;
    if (s > kXMaxSplits)
      s = kXMaxSplits;
    if (s < 2 && bn == 128 && unsplit > cus)
      s = 2;
    while (s > 1 && nk < 8 * s)
      --s;
    if (s < 2)
      continue;
    const int ks = K / s;
    if (ks < 2048 || (ks < 4096 && (M <= 96 || unsplit < cus)))
      return plan;
    plan.splits = s;
    plan.bn = bn;
    return plan;
  }
  return plan;
}

size_t skinny_split_slot_bytes(int N, const SplitPlan &plan) {
  return (size_t)((N + plan.bn - 1) / plan.bn) * plan.splits * 128 * plan.bn * sizeof(float);
}

size_t skinny_split_counter_count(int N, const SplitPlan &plan) {
  return 2 * (size_t)((N + plan.bn - 1) / plan.bn);  // arrived, published
}

hipError_t launch_skinny_split(const GemmArgs &g, const SplitPlan &plan, float *slots,
                               unsigned long long *counters, uint32_t epoch, hipStream_t s) {
  if (plan.splits < 1 || plan.splits > kXMaxSplits || g.K / kBK < plan.splits ||
      (plan.bn != 128 && plan.bn != 64) || epoch == 0)
    return hipErrorInvalidValue;
  SplitParams p{static_cast<const uint16_t *>(g.A), static_cast<const uint16_t *>(g.B),
                g.C, slots, counters, g.M, g.N, g.K, g.col_major ? g.M : g.N, plan.splits,
                epoch};
  const bool cm = g.col_major;
  const int bn = plan.bn;
  if (g.in_dtype == kF16) {
    if (g.out_dtype == kF32) return launch_split_out<kF16, kF32>(p, bn, cm, s);
    if (g.out_dtype == kF16) return launch_split_out<kF16, kF16>(p, bn, cm, s);
    return launch_split_out<kF16, kBF16>(p, bn, cm, s);
  }
  if (g.out_dtype == kF32) return launch_split_out<kBF16, kF32>(p, bn, cm, s);
  if (g.out_dtype == kF16) return launch_split_out<kBF16, kF16>(p, bn, cm, s);
  return launch_split_out<kBF16, kBF16>(p, bn, cm, s);
}

} // namespace gemm
} // namespace wave
