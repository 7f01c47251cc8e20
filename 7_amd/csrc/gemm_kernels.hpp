#pragma once
// gemm_kernels.hpp -- tiled f16/bf16 GEMM and its Stream-K variant for gfx950.
//
// C = A . B^T with A [M x K] and B [N x K], both row-major (K contiguous),
// fp32 accumulation, f32/f16/bf16 output in row-major (C[m*N+n]) or
// column-major (C[n*M+m]) layout.  This is the math of the reference kernel
// `wmma_f16_matmul_tiled` (python/mlir/dialects/wave_matmul.py:997-1022 for
// the element definition, :329-333 for the N x K storage of B) and of
// `gfx950_f16_streamk_gemm` (wave_matmul.py:77-165 partition,
// docs/Gfx950StreamKSameKernelReductionDesign.md:33-101 protocol).
//
// Design (one CTA = one 256x256 output tile, 4 waves of 64 lanes):
//  * K is consumed 64 elements at a time.  Each stage holds A and B tiles of
//    256 rows x 128 bytes (32 KiB each) in LDS; two stages double-buffer the
//    K loop (128 KiB of the 160 KiB LDS).
//  * Aligned shapes fill LDS with global_load_lds_dwordx4 (no VGPR staging);
//    ragged shapes stage through VGPRs with bounds checks and zero fill.
//  * LDS rows are 8 chunks of 16 bytes; chunk c of row r is stored at
//    position c ^ swz(r), swz(r) = (r ^ (r >> 3)) & 7, so the 16 rows read by
//    one ds_read_b128 quarter-wave hit distinct banks for both 32- and
//    64-bank LDS models.  The swizzle is applied on the global side of the
//    DMA (lane l fetches the chunk that belongs at LDS slot l).
//  * Each wave owns a 128x128 sub-tile = 4x4 MFMA 32x32x16 tiles (256 fp32
//    accumulators per lane).  MFMA operands are chosen so that each lane's
//    4 consecutive accumulator registers are 4 consecutive elements of C's
//    contiguous dimension (the "P" dimension: n for row-major, m for
//    column-major), giving 8/16-byte stores without an LDS transpose.
//  * Tiles are numbered so that consecutive CTAs on one XCD (the hardware
//    dispatches CTA i to XCD i % 8) form a group_m x tiles_n band, keeping
//    the A/B panels they share in that XCD's L2.

#include "gemm.hpp"
#include "wave_common.hpp"

namespace wave {
namespace gemm {

constexpr int kTile = 256;
constexpr int kBK = 64;
constexpr int kRowBytes = kBK * 2;                 // 128
constexpr int kOperandBytes = kTile * kRowBytes;   // 32 KiB
constexpr int kStageBytes = 2 * kOperandBytes;     // 64 KiB
constexpr int kSmemBytes = 2 * kStageBytes;        // 128 KiB
constexpr int kThreads = 256;
constexpr int kTileElems = kTile * kTile;

__device__ __forceinline__ uint32_t swz(uint32_t row) {
  return (row ^ (row >> 3)) & 7u;
}

struct Params {
  const uint16_t *A;
  const uint16_t *B;
  void *C;
  int M, N, K;
  int tiles_m, tiles_n;
  int group_m;
  int ldc;        // N for row-major C, M for column-major C
  int c_vec_ok;   // C base and ldc allow 4-element vector stores
  // Stream-K only
  float *scratch;
  uint32_t *counters;
  int workers;
};

// Linear CTA id -> (tile_m, tile_n).  XCD remap then grouped ordering.
__device__ __forceinline__ void tile_coords(int raw, int tiles_m, int tiles_n,
                                            int group_m, bool xcd_remap,
                                            int &tm, int &tn) {
  const int total = tiles_m * tiles_n;
  int pid = raw;
  if (xcd_remap && (total & 7) == 0)
    pid = (raw & 7) * (total >> 3) + (raw >> 3);
  const int per_group = group_m * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int in_group = pid - group * per_group;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

// Load 8 consecutive 16-bit elements of one row starting at column k, with
// zero fill past the row end.  VEC = elements per memory access (8: 16-byte
// loads, 4: 8-byte, 1: 2-byte), chosen by the host from K and the base
// pointer alignment.
template <int VEC>
__device__ __forceinline__ u32x4 load_chunk(const uint16_t *row, int k, int K) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (row == nullptr)
    return v;
  if (k + 8 <= K) {
    if constexpr (VEC == 8) {
      v = *reinterpret_cast<const u32x4 *>(row + k);
    } else if constexpr (VEC == 4) {
      u32x2 lo = *reinterpret_cast<const u32x2 *>(row + k);
      u32x2 hi = *reinterpret_cast<const u32x2 *>(row + k + 4);
      v = u32x4{lo.x, lo.y, hi.x, hi.y};
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] = (uint32_t)row[k + 2 * e] | ((uint32_t)row[k + 2 * e + 1] << 16);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t lo = (k + 2 * e < K) ? row[k + 2 * e] : 0u;
      uint32_t hi = (k + 2 * e + 1 < K) ? row[k + 2 * e + 1] : 0u;
      v[e] = lo | (hi << 16);
    }
  }
  return v;
}

// Accumulate C-tile (m0, n0) over K stages [kt_begin, kt_end) into acc.
template <int IN_DT, bool COL_MAJOR, bool MASKED, int VEC>
__device__ __forceinline__ void mainloop(const Params &p, int m0, int n0,
                                         int kt_begin, int kt_end,
                                         uint8_t *smem, f32x16 (&acc)[4][4]) {
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave_m = wave >> 1, wave_n = wave & 1;
  const uint32_t wp = COL_MAJOR ? wave_m : wave_n;
  const uint32_t wq = COL_MAJOR ? wave_n : wave_m;
  // P operand (rows of the MFMA result) comes from B for row-major C.
  constexpr uint32_t kPBuf = COL_MAJOR ? 0 : kOperandBytes;
  constexpr uint32_t kQBuf = COL_MAJOR ? kOperandBytes : 0;

  // Fragment read offsets: row r of the operand tile, chunk (2*kk + hi).
  uint32_t poff[4], pswz[4], qoff[4], qswz[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t pr = wp * 128 + t * 32 + (lane & 31);
    const uint32_t qr = wq * 128 + t * 32 + (lane & 31);
    poff[t] = kPBuf + pr * kRowBytes;
    qoff[t] = kQBuf + qr * kRowBytes;
    pswz[t] = swz(pr) ^ (lane >> 5);
    qswz[t] = swz(qr) ^ (lane >> 5);
  }

  // Fragments of one 16-wide K slice: 4 P tiles + 4 Q tiles, 16 bytes each.
  struct Frag {
    u32x4 p[4], q[4];
  };
  auto read_frags = [&](Frag &f, uint32_t stage, int kk) {
    const uint8_t *s = smem + stage * kStageBytes;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f.p[t] = *reinterpret_cast<const u32x4 *>(
          s + poff[t] + (((uint32_t)(2 * kk) ^ pswz[t]) << 4));
      f.q[t] = *reinterpret_cast<const u32x4 *>(
          s + qoff[t] + (((uint32_t)(2 * kk) ^ qswz[t]) << 4));
    }
  };
  auto mma = [&](const Frag &f) {
#pragma unroll
    for (int tp = 0; tp < 4; ++tp)
#pragma unroll
      for (int tq = 0; tq < 4; ++tq)
        acc[tp][tq] = mfma32x32x16<IN_DT>(f.p[tp], f.q[tq], acc[tp][tq]);
  };
  // Interleave the 8 fragment reads of the next slice with the 16 MFMAs of
  // the current one (1 LDS read : 2 MFMAs).
  auto interleave = [&]() {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
    }
  };
  // Slices 0..2 of `stage`, prefetching slices 1..3.  On return f[1] holds
  // slice 3, which the caller multiplies after the stage barrier while the
  // next stage's slice 0 is read into f[0].
  Frag f[2];
  auto body = [&](uint32_t stage) {
#pragma unroll
    for (int kk = 0; kk < 3; ++kk) {
      read_frags(f[(kk + 1) & 1], stage, kk + 1);
      mma(f[kk & 1]);
      interleave();
    }
  };

  const int nk = kt_end - kt_begin;
  if (nk <= 0)
    return;

  if constexpr (!MASKED) {
    // Global byte offsets of this lane's 8 DMA chunks (same for A and B).
    const uint32_t rowbytes = (uint32_t)p.K * 2u;
    uint32_t goff[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t r = wave * 64 + i * 8 + (lane >> 3);
      goff[i] = r * rowbytes + (((lane & 7) ^ swz(r)) << 4);
    }
    const char *a_tile =
        reinterpret_cast<const char *>(p.A) + (size_t)m0 * rowbytes;
    const char *b_tile =
        reinterpret_cast<const char *>(p.B) + (size_t)n0 * rowbytes;
    const uint32_t lds0 = lds_addr(smem) + wave * 8 * 1024;
    auto issue = [&](uint32_t stage, int kt) {
      const char *ab = a_tile + (size_t)kt * kRowBytes;
      const char *bb = b_tile + (size_t)kt * kRowBytes;
      const uint32_t l = lds0 + stage * kStageBytes;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        dma16(l + i * 1024, ab, goff[i]);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        dma16(l + kOperandBytes + i * 1024, bb, goff[i]);
    };
    issue(0, kt_begin);
    vm_wait_barrier();
    read_frags(f[0], 0, 0);
    // All but the last stage: the next stage's DMA is issued unconditionally
    // so it shares a basic block with (and is scheduled among) the MFMAs.
    for (int i = 0; i + 1 < nk; ++i) {
      const uint32_t stage = i & 1;
      issue(stage ^ 1, kt_begin + i + 1);
      body(stage);
      vm_wait_barrier();
      read_frags(f[0], stage ^ 1, 0);
      mma(f[1]);
      interleave();
    }
    body((nk - 1) & 1);
    mma(f[1]);
    vm_wait_barrier();
  } else {
    // VGPR-staged loads with bounds checks (ragged M/N/K, unaligned K).
    const uint16_t *arow[8], *brow[8];
    int kcol[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = wave * 64 + i * 8 + (lane >> 3);
      kcol[i] = (int)(((lane & 7) ^ swz(r)) * 8);
      arow[i] = (m0 + r < p.M) ? p.A + (size_t)(m0 + r) * p.K : nullptr;
      brow[i] = (n0 + r < p.N) ? p.B + (size_t)(n0 + r) * p.K : nullptr;
    }
    u32x4 ra[8], rb[8];
    auto load = [&](int kt) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ra[i] = load_chunk<VEC>(arow[i], kt * kBK + kcol[i], p.K);
        rb[i] = load_chunk<VEC>(brow[i], kt * kBK + kcol[i], p.K);
      }
    };
    auto store = [&](uint32_t stage) {
      uint8_t *s = smem + stage * kStageBytes + (wave * 8 * 1024) + lane * 16;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        *reinterpret_cast<u32x4 *>(s + i * 1024) = ra[i];
        *reinterpret_cast<u32x4 *>(s + kOperandBytes + i * 1024) = rb[i];
      }
    };
    load(kt_begin);
    store(0);
    lds_barrier();
    read_frags(f[0], 0, 0);
    for (int i = 0; i < nk; ++i) {
      const uint32_t stage = i & 1;
      if (i + 1 < nk)
        load(kt_begin + i + 1);
      body(stage);
      if (i + 1 < nk)
        store(stage ^ 1);
      lds_barrier();
      if (i + 1 < nk)
        read_frags(f[0], stage ^ 1, 0);
      mma(f[1]);
    }
  }
}

// Store 4 consecutive P-dimension values v at C[q*ldc + pp .. pp+3].
template <int OUT_DT>
__device__ __forceinline__ void store4(void *C, size_t idx, f32x4 v) {
  if constexpr (OUT_DT == kF32) {
    *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(C) + idx) = v;
  } else {
    u32x2 w = {pack2<OUT_DT>(v[0], v[1]), pack2<OUT_DT>(v[2], v[3])};
    *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(C) + idx) = w;
  }
}

template <int OUT_DT>
__device__ __forceinline__ void store1(void *C, size_t idx, float v) {
  if constexpr (OUT_DT == kF32)
    reinterpret_cast<float *>(C)[idx] = v;
  else
    reinterpret_cast<uint16_t *>(C)[idx] = to_bits<OUT_DT>(v);
}

// Write one lane's share of the 256x256 tile at (m0, n0).  `get(tp,tq,g)`
// returns the 4 values of accumulator group g of MFMA tile (tp, tq).
template <int OUT_DT, bool COL_MAJOR, bool MASKED, typename Get>
__device__ __forceinline__ void store_tile(const Params &p, int m0, int n0,
                                           Get get) {
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave_m = wave >> 1, wave_n = wave & 1;
  const int wp = COL_MAJOR ? wave_m : wave_n;
  const int wq = COL_MAJOR ? wave_n : wave_m;
  const int P0 = COL_MAJOR ? m0 : n0, Q0 = COL_MAJOR ? n0 : m0;
  const int Pext = COL_MAJOR ? p.M : p.N, Qext = COL_MAJOR ? p.N : p.M;
#pragma unroll
  for (int tq = 0; tq < 4; ++tq) {
    const int q = Q0 + wq * 128 + tq * 32 + (lane & 31);
#pragma unroll
    for (int tp = 0; tp < 4; ++tp) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int pp = P0 + wp * 128 + tp * 32 + 8 * g + 4 * (lane >> 5);
        const f32x4 v = get(tp, tq, g);
        const size_t idx = (size_t)q * p.ldc + pp;
        if constexpr (!MASKED) {
          store4<OUT_DT>(p.C, idx, v);
        } else {
          if (q < Qext) {
            if (p.c_vec_ok && pp + 3 < Pext) {
              store4<OUT_DT>(p.C, idx, v);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (pp + e < Pext)
                  store1<OUT_DT>(p.C, idx + e, v[e]);
            }
          }
        }
      }
    }
  }
}

template <int IN_DT, int OUT_DT, bool COL_MAJOR, bool MASKED, int VEC>
__global__ __launch_bounds__(kThreads, 1) void tiled_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmemBytes];
  int tm, tn;
  tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, p.group_m, true, tm, tn);
  const int m0 = tm * kTile, n0 = tn * kTile;
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = f32x16{};
  const int kt_n = (p.K + kBK - 1) / kBK;
  mainloop<IN_DT, COL_MAJOR, MASKED, VEC>(p, m0, n0, 0, kt_n, smem, acc);
  store_tile<OUT_DT, COL_MAJOR, MASKED>(p, m0, n0, [&](int tp, int tq, int g) {
    return f32x4{acc[tp][tq][4 * g], acc[tp][tq][4 * g + 1],
                 acc[tp][tq][4 * g + 2], acc[tp][tq][4 * g + 3]};
  });
}

// ---------------------------------------------------------------- Stream-K
// Work unit = (tile, 64-wide K stage); W = T * I units split into `workers`
// contiguous intervals (wave_matmul.py:88-101): worker w owns
// [w*q + min(w, r), +q + (w < r)) with q = W / workers, r = W % workers.
struct Interval {
  int begin, end;
};
__device__ __forceinline__ Interval sk_interval(int total, int workers, int w) {
  const int q = total / workers, r = total % workers;
  const int b = w * q + min(w, r);
  return {b, b + q + (w < r ? 1 : 0)};
}
// Owner of work unit `it` (wave_matmul.py:104-116).
__device__ __forceinline__ int sk_owner(int total, int workers, int it) {
  const int q = total / workers, r = total % workers;
  const int large_end = r * (q + 1);
  return it < large_end ? it / (q + 1) : r + (it - large_end) / q;
}
// Scratch slot that worker w uses for split tile `tile` (0 or 1): a worker
// interval has at most two split segments, its first and its last tile
// (wave_matmul.py:132-153).
__device__ __forceinline__ int sk_slot(int total, int workers, int w, int tile,
                                       int iters) {
  const Interval iv = sk_interval(total, workers, w);
  const int first = iv.begin / iters;
  if (tile == first)
    return 0;
  const bool first_whole = (iv.begin % iters == 0) && (iv.end >= (first + 1) * iters);
  return first_whole ? 0 : 1;
}

// Per-thread scratch layout: element e (0..4095 of this thread's 256x256
// share) of thread t lives at slot_base + e * 256 + t, so publishing and
// reducing are fully coalesced and need no coordinate math.
template <int IN_DT, int OUT_DT, bool COL_MAJOR, bool MASKED, int VEC>
__global__ __launch_bounds__(kThreads, 1) void streamk_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmemBytes];
  __shared__ int arrival;
  const int worker = blockIdx.x;
  const int tiles = p.tiles_m * p.tiles_n;
  const int iters = (p.K + kBK - 1) / kBK;
  const int total = tiles * iters;
  const Interval iv = sk_interval(total, p.workers, worker);
  const bool aligned = (total % p.workers == 0) && ((total / p.workers) % iters == 0);

  f32x16 acc[4][4];
  auto zero = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = f32x16{};
  };
  auto whole_tile = [&](int tile) {
    int tm, tn;
    tile_coords(tile, p.tiles_m, p.tiles_n, p.group_m, false, tm, tn);
    zero();
    mainloop<IN_DT, COL_MAJOR, MASKED, VEC>(p, tm * kTile, tn * kTile, 0,
                                            iters, smem, acc);
    store_tile<OUT_DT, COL_MAJOR, MASKED>(
        p, tm * kTile, tn * kTile, [&](int tp, int tq, int g) {
          return f32x4{acc[tp][tq][4 * g], acc[tp][tq][4 * g + 1],
                       acc[tp][tq][4 * g + 2], acc[tp][tq][4 * g + 3]};
        });
  };

  if (aligned) {
    // Every worker owns whole tiles: visit worker, worker + P, ... so the
    // tiles in flight at any moment are adjacent (no partials, no atomics).
    for (int tile = worker; tile < tiles; tile += p.workers)
      whole_tile(tile);
    return;
  }

  const int first_tile = iv.begin / iters;
  const int last_tile = (iv.end - 1) / iters;
  int slot = 0;
  for (int tile = first_tile; tile <= last_tile; ++tile) {
    const int kb = max(iv.begin, tile * iters) - tile * iters;
    const int ke = min(iv.end, (tile + 1) * iters) - tile * iters;
    if (kb == 0 && ke == iters) {
      whole_tile(tile);
      continue;
    }
    int tm, tn;
    tile_coords(tile, p.tiles_m, p.tiles_n, p.group_m, false, tm, tn);
    zero();
    mainloop<IN_DT, COL_MAJOR, MASKED, VEC>(p, tm * kTile, tn * kTile, kb, ke,
                                            smem, acc);
    // Publish this worker's fp32 partial.
    float *mine = p.scratch + ((size_t)worker * 2 + slot) * kTileElems;
#pragma unroll
    for (int tp = 0; tp < 4; ++tp)
#pragma unroll
      for (int tq = 0; tq < 4; ++tq)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          mine[((tp * 4 + tq) * 16 + r) * kThreads + threadIdx.x] = acc[tp][tq][r];
    ++slot;
    const int first_owner = sk_owner(total, p.workers, tile * iters);
    const int last_owner = sk_owner(total, p.workers, (tile + 1) * iters - 1);
    const int parts = last_owner - first_owner + 1;
    __threadfence();  // release the partial at device scope
    __syncthreads();
    if (threadIdx.x == 0)
      arrival = __hip_atomic_fetch_add(&p.counters[tile], 1u, __ATOMIC_ACQ_REL,
                                       __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrival != parts - 1)
      continue;
    // Last arriver: reduce all contributors' partials in worker order (a
    // fixed order, so the result does not depend on arrival order).
    __threadfence();  // acquire the other workers' partials
    store_tile<OUT_DT, COL_MAJOR, MASKED>(
        p, tm * kTile, tn * kTile, [&](int tp, int tq, int g) {
          f32x4 s = {0.f, 0.f, 0.f, 0.f};
          for (int c = first_owner; c <= last_owner; ++c) {
            const int cs = sk_slot(total, p.workers, c, tile, iters);
            const float *part =
                p.scratch + ((size_t)c * 2 + cs) * kTileElems;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              s[e] += __builtin_nontemporal_load(
                  part + ((tp * 4 + tq) * 16 + 4 * g + e) * kThreads +
                  threadIdx.x);
          }
          return s;
        });
    __syncthreads();
    if (threadIdx.x == 0)
      __hip_atomic_store(&p.counters[tile], 0u, __ATOMIC_RELEASE,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ------------------------------------------------------------- launchers
// mode: 0 = aligned fast path (LDS DMA), 8/4/1 = masked path with that many
// elements per global load.
template <int IN_DT, int OUT_DT, bool CM, bool SK>
hipError_t launch_variant(const Params &p, int mode, hipStream_t stream) {
  const dim3 block(kThreads);
  const dim3 grid(SK ? p.workers : p.tiles_m * p.tiles_n);
#define WAVE_LAUNCH(MASKED, VEC)                                               \
  do {                                                                         \
    if constexpr (SK)                                                          \
      hipLaunchKernelGGL((streamk_kernel<IN_DT, OUT_DT, CM, MASKED, VEC>),     \
                         grid, block, 0, stream, p);                           \
    else                                                                       \
      hipLaunchKernelGGL((tiled_kernel<IN_DT, OUT_DT, CM, MASKED, VEC>), grid, \
                         block, 0, stream, p);                                 \
  } while (0)
  switch (mode) {
  case 0: WAVE_LAUNCH(false, 8); break;
  case 8: WAVE_LAUNCH(true, 8); break;
  case 4: WAVE_LAUNCH(true, 4); break;
  default: WAVE_LAUNCH(true, 1); break;
  }
#undef WAVE_LAUNCH
  return hipGetLastError();
}

#define WAVE_GEMM_INSTANTIATE(IN, OUT, SK)                                     \
  template hipError_t launch_variant<IN, OUT, false, SK>(const Params &, int,   \
                                                         hipStream_t);         \
  template hipError_t launch_variant<IN, OUT, true, SK>(const Params &, int,    \
                                                        hipStream_t);

} // namespace gemm
} // namespace wave
