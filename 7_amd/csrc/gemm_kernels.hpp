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
//  * K is consumed BK (32 or 64) elements per LDS stage.  A stage holds A and
//    B tiles of 256 rows x 2*BK bytes; NSTAGE stages form a ring (BK=32 x 4
//    or BK=64 x 2 = 128 KiB of the 160 KiB LDS), so the DMA for stage i+3
//    (resp. i+1) is in flight while stage i is multiplied.
//  * Aligned shapes fill LDS with global_load_lds_dwordx4 (no VGPR staging);
//    ragged shapes stage through VGPRs with bounds checks and zero fill.
//  * LDS rows are BK/8 chunks of 16 bytes; chunk c of row r is stored at
//    c ^ swz(r) so the rows read together by one ds_read_b128 hit distinct
//    banks (rocprofv3 SQ_LDS_BANK_CONFLICT = 0).  The swizzle is applied on
//    the global side of the DMA (lane l fetches the chunk that belongs at
//    LDS slot l).
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

#include <type_traits>

#ifndef WAVE_GEMM_BK
#define WAVE_GEMM_BK 32
#endif
#ifndef WAVE_GEMM_NSTAGE
#define WAVE_GEMM_NSTAGE 4
#endif
#ifndef WAVE_GEMM_WAVES
#define WAVE_GEMM_WAVES 4
#endif
#ifndef WAVE_GEMM_READ_ORDER
#define WAVE_GEMM_READ_ORDER 0
#endif
#ifndef WAVE_GEMM_PRE_RG
#define WAVE_GEMM_PRE_RG 4  // MFMA groups that carry the pre-barrier reads
#endif
// MFMA shape of the tiled f16/bf16 kernel's whole-tile path: 32 selects
// v_mfma_f32_32x32x16, 16 selects v_mfma_f32_16x16x32.  Ragged tiles,
// Stream-K and MXFP4 always use the 32x32 shapes.
#ifndef WAVE_GEMM_MF
#define WAVE_GEMM_MF 16
#endif
// With one MFMA slice per stage (16x16x32 at BK = 32): MFMA groups of a
// step that carry the next stage's fragment reads (0 = all of them).
#ifndef WAVE_GEMM_KS1_RG
#define WAVE_GEMM_KS1_RG 0
#endif

namespace wave {
namespace gemm {

constexpr int kTile = 256;
constexpr int kTileElems = kTile * kTile;
constexpr int kSKUnit = 64;  // Stream-K work unit: 64 K elements of one tile

// LDS ring geometry for BK elements of K per stage and NSTAGE stages, and
// the wave grid: WAVES waves, WPN along P (the MFMA row / C-contiguous
// dimension) x WQN along Q, each owning TP x TQ MFMA tiles of MF x MF.
// SCALE_: bytes per stage of MXFP4 e8m0 scales after the A and B tiles.
// MF_: MFMA tile edge, 32 (32x32x16: K slice 16) or 16 (16x16x32: K slice
// 32).  Accumulator register r of lane l holds D[8*(r/4) + 4*(l/MF) + r%4]
// [l%MF] of its tile in both shapes (NG = MF*MF/256 groups of 4).
template <int BK_, int NSTAGE_, int WAVES_, int SCALE_ = 0, int MF_ = 32> struct Cfg {
  static constexpr int BK = BK_;
  static constexpr int SCALE = SCALE_;
  static constexpr int NSTAGE = NSTAGE_;
  static constexpr int WAVES = WAVES_;
  static constexpr int MF = MF_;
  static constexpr int THREADS = 64 * WAVES;
  // Compute grid: VW virtual waves, WPN along P x WQN along Q.  With fewer
  // than 4 waves each wave runs PASSES = VW / WAVES virtual waves in turn
  // (one K loop each, all of them over the same LDS ring).
  static constexpr int VW = WAVES < 4 ? 4 : WAVES;
  static constexpr int PASSES = VW / WAVES;
  static constexpr int WPN = VW >= 16 ? 4 : 2, WQN = VW / WPN;
  static constexpr int TP = 256 / WPN / MF, TQ = 256 / WQN / MF;
  static_assert((MF == 32 || MF == 16) && TP >= 1 && TQ >= 1, "MFMA tile shape");
  static_assert(WAVES == 1 || WAVES == 2 || WAVES == 4 || WAVES == 8 || WAVES == 16,
                "1, 2, 4, 8 or 16 waves");
  static constexpr int NG = MF * MF / 256;       // 4-register accumulator groups
  using Acc = std::conditional_t<MF == 32, f32x16, f32x4>;
  static constexpr int KSL = 512 / MF;           // K elements per MFMA slice
  static constexpr int CHS = KSL / 8;            // 16-byte row chunks per slice
  static constexpr int RB = BK * 2;              // bytes per operand row
  static constexpr int CPR = BK / 8;             // 16-byte chunks per row
  static constexpr int KS = BK / KSL;            // MFMA K slices per stage
  static_assert(KS >= 1 && BK % KSL == 0, "BK holds whole MFMA slices");
  static constexpr int OPB = kTile * RB;         // bytes per operand tile
  static constexpr int STAGE = 2 * OPB + SCALE;  // A + B (+ scales)
  static constexpr int SMEM = NSTAGE * STAGE;
  static constexpr int DMA = OPB / 1024 / WAVES; // DMA issues per wave per operand
  static_assert(OPB == 128 * 128 * (BK / 32), "super-row layout covers BK 32/64");
  static_assert(SMEM <= 160 * 1024, "LDS ring exceeds 160 KiB");
};
// Ragged tiles (bounds-checked path) with W waves per CTA (0: the library's
// default wave count).
template <int W = 0>
using DefaultCfgW = Cfg<WAVE_GEMM_BK, WAVE_GEMM_NSTAGE, W == 0 ? WAVE_GEMM_WAVES : W>;
using DefaultCfg = DefaultCfgW<>;
// Whole tiles of the tiled f16/bf16 kernel (same ring and wave grid).  With
// 8 or 16 waves (two or four per SIMD: 256 or 128 registers a wave) the
// 16x16 path's two fragment sets do not fit next to its accumulators (8
// waves: 12 VGPR spills), so those CTAs keep the 32x32 shape unless
// WAVE_GEMM_MF8 says otherwise for 8 waves.
#ifndef WAVE_GEMM_MF8
#define WAVE_GEMM_MF8 32
#endif
// 4-wave whole tiles take 64-deep stages in two buffers (one barrier per
// stage, whole-line DMA): 8192^3 f16 1321-1331 -> 1382-1391 TFLOP/s against
// 32-deep stages in four, one box, two runs.  Other wave counts keep the
// 32-deep ring.
#ifndef WAVE_GEMM_TILE_BK
#define WAVE_GEMM_TILE_BK 64
#endif
template <int W = 0, int WV = (W == 0 ? WAVE_GEMM_WAVES : W)>
using TileCfgW = Cfg<WV == 4 ? WAVE_GEMM_TILE_BK : WAVE_GEMM_BK,
                     WV == 4 && WAVE_GEMM_TILE_BK == 64 ? 2 : WAVE_GEMM_NSTAGE, WV, 0,
                     WV >= 16 ? 32 : WV == 8 ? WAVE_GEMM_MF8 : WAVE_GEMM_MF>;
using TileCfg = TileCfgW<>;
// 32-deep stages for the hybrid path (ragged tiles and K on the DMA ring) of
// wave counts other than 4.
template <int W = 0>
using HybridCfgW = Cfg<WAVE_GEMM_BK, WAVE_GEMM_NSTAGE, W == 0 ? WAVE_GEMM_WAVES : W, 0,
                       WAVE_GEMM_MF>;
// The hybrid path and Stream-K's whole-tile ranges: the 64-deep two-buffer
// ring where whole tiles run it (4 waves), else HybridCfgW.
template <int W = 0, int WV = (W == 0 ? WAVE_GEMM_WAVES : W)>
using HybridTileCfgW =
    std::conditional_t<WV == 4 && WAVE_GEMM_TILE_BK == 64, TileCfgW<W>, HybridCfgW<W>>;
// MXFP4: the same ring with K counted in 16-bit units (one 64-byte row
// chunk = 128 fp4 values per stage, one MFMA 32x32x64 per 32-byte slice)
// and 2 KiB of scales per stage: four 32-value groups x (256 A + 256 B)
// rows, laid out [group][A rows | B rows].  8 waves (two per SIMD, 128x64
// outputs each) measured 2-8 % faster than 4 for these short-latency MFMAs.
#ifndef WAVE_FP4_WAVES
#define WAVE_FP4_WAVES 8
#endif
// MFMA shape of the MXFP4 path: 32 (32x32x64) or 16 (16x16x128).
#ifndef WAVE_FP4_MF
#define WAVE_FP4_MF 32
#endif
template <int W = 0>
using Fp4CfgW = Cfg<32, 4, W == 0 ? WAVE_FP4_WAVES : W, 4 * 512, WAVE_FP4_MF>;
using Fp4Cfg = Fp4CfgW<>;
// Canonical MXFP4 with K a multiple of 256 values: 64-deep stages (256
// values, 128 bytes a row, 4 KiB of scales) in two buffers, the same LDS.
template <int W = 0>
using Fp4Cfg64W = Cfg<64, 2, W == 0 ? WAVE_FP4_WAVES : W, 8 * 512, WAVE_FP4_MF>;
// MXFP4 with AITER-preshuffled B and scales: the scale area holds whole
// 256-byte AITER scale blocks (32 rows x 8 groups), 8 for A and 8 for B.
template <int W = 0>
using Fp4ACfgW = Cfg<32, 4, W == 0 ? WAVE_FP4_WAVES : W, 16 * 256, WAVE_FP4_MF>;
using Fp4ACfg = Fp4ACfgW<>;

// LDS geometry of an operand tile.  The tile is stored as 128-byte
// "super-rows" of eight 16-byte slots: with BK = 64 super-row R is tile row
// R; with BK = 32 it holds row R in slots 0-3 and row R + 128 in slots 4-7.
// Logical slot lc of super-row R lives at physical slot lc ^ Geo<C>::swz(R).
// Fragment reads, timed by a probe that repeats one ds_read_b128 lane
// pattern from precomputed addresses (ns per wave access per CU; a linear
// 1 KiB read: 2.0):
//  * 32x32 fragments (32 consecutive rows at one chunk): swz_rr(R) =
//    (R ^ R>>3) & 7 1.92, (R >> 1) & 7 1.82 (rocprofv3: 4 LDS cycles per
//    read, no conflict);
//  * 16x16 fragments (16 consecutive rows x 4 chunks): (R >> 1) & 7 1.77
//    (conflict-free), swz_rr 3.39, 2*((R>>2)&3) + ((R>>4)&1) (the previous
//    16x16 swizzle) 3.49, none 6.70.  With 64 banks of 4 bytes, rows R and
//    R + 2 of 128 bytes fall on the same banks, so a swizzle has to differ
//    between them: (R >> 1) & 7 gives the 16 rows 16 distinct 16-byte bank
//    groups.  8192^3 f16 with it: +0.5 % (wave-bench, same box, 3 passes).
__device__ __forceinline__ uint32_t swz_rr(uint32_t R) { return (R ^ (R >> 3)) & 7u; }
__device__ __forceinline__ uint32_t swz_16(uint32_t R) { return (R >> 1) & 7u; }

template <class C> struct Geo {
  static __device__ __forceinline__ uint32_t swz(uint32_t R) {
    return C::MF == 16 ? swz_16(R) : swz_rr(R);
  }
  // (tile row, 16-byte chunk) -> (super-row, logical slot)
  static __device__ __forceinline__ uint32_t super_row(uint32_t row) {
    return C::CPR == 8 ? row : (row & 127u);
  }
  static __device__ __forceinline__ uint32_t slot_base(uint32_t row) {
    return C::CPR == 8 ? 0u : ((row >> 7) << 2);
  }
  // Inverse, for the loaders: physical slot p of super-row R holds tile row
  // row_of(R, p) chunk chunk_of(R, p).
  static __device__ __forceinline__ uint32_t logical(uint32_t R, uint32_t p) {
    return p ^ swz(R);
  }
  static __device__ __forceinline__ uint32_t row_of(uint32_t R, uint32_t p) {
    return C::CPR == 8 ? R : R + 128u * (logical(R, p) >> 2);
  }
  static __device__ __forceinline__ uint32_t chunk_of(uint32_t R, uint32_t p) {
    return C::CPR == 8 ? logical(R, p) : (logical(R, p) & 3u);
  }
};

struct Params {
  const uint16_t *A;
  const uint16_t *B;
  void *C;
  int M, N, K;    // MXFP4: K counted in 16-bit units (fp4 K / 4)
  // MXFP4 only: e8m0 scales, group-major [K/32][M] and [K/32][N]
  const uint8_t *a_scale, *b_scale;
  int tiles_m, tiles_n;
  int group_m;
  int ldc;        // N for row-major C, M for column-major C
  int c_vec_ok;   // C base and ldc allow 4-element vector stores
  // Stream-K only
  float *scratch;
  uint32_t *counters;
  int workers;
  // Tile-packed C (pk != 0; column-major MFMA orientation): the reference
  // blocking whose 16x16 tile order C follows, and its CTA columns
  // pk_nblocks = N / (16 * pk_bn * pk_wnt).
  int pk, pk_bm, pk_bn, pk_wmt, pk_wnt, pk_nblocks;
};

// Tile-packed C, the reference's output_layout "tile-packed"
// (wave_matmul.py:1279-1347 C pointers, :6351-6405 fragment stores; decoded
// by the runner's getOutputCoordinate, wave-matmul-calibrate-runner.cpp
// :772-834).  C is a sequence of 16x16 tiles, ordered by the reference's CTA
// (row-major over its M_blocks x N_blocks grid), then wave (m_wave * BN +
// n_wave), then wave tile (i * wave_n_tiles + j); inside a tile, element
// (mi, nj) sits at (mi / 4) * 64 + nj * 4 + mi % 4 -- the 16x16 MFMA
// accumulator order (lane (mi / 4) * 16 + nj, register mi % 4).  The index
// is a sum of an m part and an n part.
__device__ __forceinline__ size_t packed_m_part(const Params &p, int m) {
  const int mt = m >> 4, mi = m & 15;
  const int mtpb = p.pk_bm * p.pk_wmt;
  const int wg = mt / mtpb, r = mt - wg * mtpb;
  const int mw = r / p.pk_wmt, i = r - mw * p.pk_wmt;
  const size_t wave_elems = (size_t)p.pk_wmt * p.pk_wnt * 256;
  const size_t cta_elems = wave_elems * p.pk_bm * p.pk_bn;
  return (size_t)wg * p.pk_nblocks * cta_elems + (size_t)mw * p.pk_bn * wave_elems +
         (size_t)i * p.pk_wnt * 256 + (size_t)((mi >> 2) * 64 + (mi & 3));
}
__device__ __forceinline__ size_t packed_n_part(const Params &p, int n) {
  const int nt = n >> 4, nj = n & 15;
  const int ntpb = p.pk_bn * p.pk_wnt;
  const int wg = nt / ntpb, r = nt - wg * ntpb;
  const int nw = r / p.pk_wnt, j = r - nw * p.pk_wnt;
  const size_t wave_elems = (size_t)p.pk_wmt * p.pk_wnt * 256;
  const size_t cta_elems = wave_elems * p.pk_bm * p.pk_bn;
  return (size_t)wg * cta_elems + (size_t)nw * wave_elems + (size_t)j * 256 + (size_t)nj * 4;
}

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

// The hybrid path's K remainder: K % 4 == 0 and rows 8-byte aligned, so each
// 8-element chunk (k % 8 == 0) is whole, half (4 elements) or past K.  Both
// 8-byte halves are loaded from in-bounds addresses (column 0 for a half past
// K) and zeroed by a select: no branch, so the loads issue back to back
// under one wait (the branchy load_chunk waited out one round trip per
// load: config 3b spent 20-25 us on its 4-element tail).
__device__ __forceinline__ u32x4 load_chunk_k4(const uint16_t *row, int k, int K) {
  const bool v0 = k + 4 <= K, v1 = k + 8 <= K;
  const u32x2 lo = *reinterpret_cast<const u32x2 *>(row + (v0 ? k : 0));
  const u32x2 hi = *reinterpret_cast<const u32x2 *>(row + (v1 ? k + 4 : 0));
  return u32x4{v0 ? lo.x : 0u, v0 ? lo.y : 0u, v1 ? hi.x : 0u, v1 ? hi.y : 0u};
}

// Accumulate C-tile (m0, n0) over K steps [kt_begin, kt_end) (in units of
// C::BK elements) into acc.
// HYBRID (with !MASKED; one MFMA slice per stage, or the 64-deep two-buffer
// ring): the DMA ring for tiles
// that cross M or N and for K that is not a multiple of BK.  Rows past M / N
// are fetched from the last valid row instead (their products only reach C
// rows / columns that are never stored), the stages wholly inside K run the
// DMA pipeline, and a K remainder is one more stage copied through VGPRs
// with zero fill past K (VEC elements per access, as the masked path).  Every
// DMA access is dword-aligned when K is even and A, B are 4-byte aligned.
template <class C, int IN_DT, bool COL_MAJOR, bool MASKED, int VEC, bool HYBRID = false>
__device__ __forceinline__ void mainloop(const Params &p, int m0, int n0,
                                         int kt_begin, int kt_end,
                                         uint8_t *smem,
                                         typename C::Acc (&acc)[C::TP][C::TQ],
                                         uint32_t pass = 0) {
  // The tile origin is uniform for every caller; readfirstlane keeps it, and
  // the DMA bases derived from it, in SGPRs (the DMA's scalar base operand)
  // where a caller's control flow hides that (Stream-K's ticket loop).
  m0 = __builtin_amdgcn_readfirstlane(m0);
  n0 = __builtin_amdgcn_readfirstlane(n0);
  constexpr int TP = C::TP, TQ = C::TQ, NREAD = TP + TQ, MF = C::MF;
  static_assert(C::KS >= 2 || !MASKED, "the bounds-checked path needs two slices a stage");
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63;
  // Virtual wave of this pass (fewer than 4 waves: PASSES > 1).
  const uint32_t vw = wave + pass * C::WAVES;
  const uint32_t wp = vw % C::WPN, wq = vw / C::WPN;
  // P operand (rows of the MFMA result) comes from B for row-major C.
  constexpr uint32_t kPBuf = COL_MAJOR ? 0 : C::OPB;
  constexpr uint32_t kQBuf = COL_MAJOR ? C::OPB : 0;

  // AITER (kMXFP4A): B arrives preshuffled, so the B tile sits in LDS as
  // 16 row blocks of 1 KiB, each [4 chunks of 16 B][16 rows] (one K stage
  // of one 16-row block is one contiguous KiB of the AITER buffer).
  constexpr bool kAiter = IN_DT == kMXFP4A;
  constexpr bool kPAiter = kAiter && !COL_MAJOR, kQAiter = kAiter && COL_MAJOR;
  // Fragment read offsets: lane l reads row r = (tile base) + l%MF of the
  // operand tile, chunk CHS*kk + hi with hi = l/MF.
  // slot = (slot_base + CHS*kk + hi) ^ swz(R) = (CHS*kk) ^ [slot_base ^ hi ^ swz(R)]
  // AITER B tile: (r/16)*1024 + (CHS*kk + hi)*256 + (r%16)*16.
  auto aiter_off = [&](uint32_t buf, uint32_t r) {
    return buf + (r >> 4) * 1024u + (lane / MF) * 256u + (r & 15u) * 16u;
  };
  uint32_t poff[TP], pswz[TP], qoff[TQ], qswz[TQ];
#pragma unroll
  for (int t = 0; t < TP; ++t) {
    const uint32_t pr = wp * (TP * MF) + t * MF + (lane % MF);
    const uint32_t pR = Geo<C>::super_row(pr);
    poff[t] = kPAiter ? aiter_off(kPBuf, pr) : kPBuf + pR * 128u;
    pswz[t] = Geo<C>::swz(pR) ^ Geo<C>::slot_base(pr) ^ (lane / MF);
  }
#pragma unroll
  for (int t = 0; t < TQ; ++t) {
    const uint32_t qr = wq * (TQ * MF) + t * MF + (lane % MF);
    const uint32_t qR = Geo<C>::super_row(qr);
    qoff[t] = kQAiter ? aiter_off(kQBuf, qr) : kQBuf + qR * 128u;
    qswz[t] = Geo<C>::swz(qR) ^ Geo<C>::slot_base(qr) ^ (lane / MF);
  }

  // MXFP4: offsets of this lane's P / Q tile rows in a stage's scale area.
  // Canonical: [group][A rows | B rows], 512 bytes per 32-value group.
  // AITER: [A blocks | B blocks] of 256 bytes per 32 rows, byte
  // g*64 + (r%16)*4 + (kt&1)*2 + (r%32)/16 for group g of the stage (the
  // block covers 8 groups = two stages).
  uint32_t psc[TP], qsc[TQ];
  auto aiter_sc = [&](bool is_b, uint32_t r) {
    return 2 * C::OPB + (is_b ? 2048u : 0u) + (r >> 5) * 256u + (lane / MF) * 64u +
           (r & 15u) * 4u + ((r >> 4) & 1u);
  };
  if constexpr (IN_DT == kMXFP4) {
#pragma unroll
    for (int t = 0; t < TP; ++t)
      psc[t] = 2 * C::OPB + (COL_MAJOR ? 0u : 256u) + wp * (TP * MF) + t * MF + (lane % MF);
#pragma unroll
    for (int t = 0; t < TQ; ++t)
      qsc[t] = 2 * C::OPB + (COL_MAJOR ? 256u : 0u) + wq * (TQ * MF) + t * MF + (lane % MF);
  } else if constexpr (kAiter) {
#pragma unroll
    for (int t = 0; t < TP; ++t)
      psc[t] = aiter_sc(!COL_MAJOR, wp * (TP * MF) + t * MF + (lane % MF));
#pragma unroll
    for (int t = 0; t < TQ; ++t)
      qsc[t] = aiter_sc(COL_MAJOR, wq * (TQ * MF) + t * MF + (lane % MF));
  }

  // Fragments of one K slice: TP P tiles + TQ Q tiles, 16 bytes each
  // (MXFP4: 64 fp4 values per slice, plus each lane's e8m0 scale byte).
  struct Frag {
    u32x4 p[TP], q[TQ];
    uint32_t sp[TP], sq[TQ];
  };
  // Fragment j of a slice: j < TQ -> Q tile j, else P tile j - TQ.  With
  // WAVE_GEMM_READ_ORDER 1 (4 x 4 tiles) the reads run P0, Q0-Q3, P1-P3, so
  // the first MFMA row of the next slice finds P0 read a whole step early.
  auto read_one = [&](Frag &f, uint32_t stage, int kk, int jr) {
    constexpr bool kP0First = WAVE_GEMM_READ_ORDER == 1 && TP == 4 && TQ == 4;
    const int j = !kP0First ? jr : jr == 0 ? TQ : jr <= TQ ? jr - 1 : jr;
    const uint8_t *s = smem + stage * C::STAGE;
    const uint32_t x = (uint32_t)(C::CHS * kk);
    if (j < TQ)
      f.q[j] = *reinterpret_cast<const u32x4 *>(
          s + qoff[j] + (kQAiter ? x * 256u : ((x ^ qswz[j]) << 4)));
    else
      f.p[j - TQ] = *reinterpret_cast<const u32x4 *>(
          s + poff[j - TQ] + (kPAiter ? x * 256u : ((x ^ pswz[j - TQ]) << 4)));
    if constexpr (IN_DT == kMXFP4) {
      // Lane part h = l/MF holds the slice's 32-value group CHS*kk + h.
      const uint8_t *sg = s + (x + lane / MF) * 512u;
      if (j < TQ)
        f.sq[j] = sg[qsc[j]];
      else
        f.sp[j - TQ] = sg[psc[j - TQ]];
    } else if constexpr (kAiter) {
      // Group CHS*kk + h of the stage; the stage's half of the AITER block is
      // kt & 1 = stage & 1 (the ring has an even number of stages).
      const uint8_t *sg = s + x * 64u + (stage & 1u) * 2u;
      if (j < TQ)
        f.sq[j] = sg[qsc[j]];
      else
        f.sp[j - TQ] = sg[psc[j - TQ]];
    }
  };
  auto read_frags = [&](Frag &f, uint32_t stage, int kk) {
#pragma unroll
    for (int j = 0; j < NREAD; ++j)
      read_one(f, stage, kk, j);
  };
  // One K slice as TP explicitly ordered groups: group tp issues its share
  // of the LDS reads of the next slice's fragments (Q tiles first: the next
  // slice's first MFMA row needs all of them), the TQ MFMAs of P row tp,
  // and hook(tp) (the DMA issues assigned to that group).  sched_barrier
  // keeps the compiler from regrouping them, so DMA and LDS traffic stay
  // spread through the MFMA stream.
  // RG: the reads are spread over the first RG groups only.
  // The 64-deep two-buffer path spreads each group's LDS reads and DMA
  // issues between its MFMAs (reads before the 1st and 3rd, DMA after the
  // 4th and 6th): a timing copy measured 2580 cycles a stage against 2700
  // with the reads together before the group and the two issues after its
  // 4th and 8th MFMAs (2815 with both issues after the 8th); the other
  // placements tried (reads before the 1st and 5th, issues after 2nd/6th,
  // 3rd/7th, 4th/8th) fell in between.
  constexpr bool kSpread = C::KS == 2 && C::NSTAGE == 2 && MF == 16 && !is_fp4(IN_DT) && TQ == 8;
  auto step = [&](const Frag &cur, Frag &nxt, bool read, uint32_t nstage,
                  int nkk, auto hook, auto rg_tag) {
    constexpr int RG = decltype(rg_tag)::value;
    static_assert(RG >= 1 && RG <= TP, "every read group is one of the step's TP groups");
#pragma unroll
    for (int tp = 0; tp < TP; ++tp) {
      // kSpread: the group's later reads go after its second MFMA.
      const int j0 = tp * NREAD / RG, j2 = (tp + 1) * NREAD / RG;
      const int j1 = kSpread ? (j0 + j2) / 2 : j2;
      // The two-buffer path's odd step (the one with the two-argument DMA
      // hook) holds its stage barrier: its first two MFMAs use registers
      // only, so the barrier waits behind them, and group 0's reads follow.
      constexpr bool kLateBar = std::is_invocable_v<decltype(hook), int, int>;
      if (read && tp < RG && !(kLateBar && tp == 0)) {
#pragma unroll
        for (int j = j0; j < j1; ++j)
          read_one(nxt, nstage, nkk, j);
      }
#pragma unroll
      for (int tq = 0; tq < TQ; ++tq) {
        if (kLateBar && tp == 0 && tq == 2) {
          vm_wait_barrier<0>();
          if (read && tp < RG) {
#pragma unroll
            for (int j = j0; j < j2; ++j)
              read_one(nxt, nstage, nkk, j);
          }
        } else if (kSpread && read && tp < RG && tq == 2 && !(kLateBar && tp == 0)) {
#pragma unroll
          for (int j = j1; j < j2; ++j)
            read_one(nxt, nstage, nkk, j);
        }
        if constexpr (is_fp4(IN_DT) && MF == 32)
          acc[tp][tq] = mfma_fp4_32x32x64(cur.p[tp], cur.q[tq], acc[tp][tq], cur.sp[tp],
                                          cur.sq[tq]);
        else if constexpr (is_fp4(IN_DT))
          mfma_fp4_16x16x128_acc(acc[tp][tq], cur.p[tp], cur.q[tq], cur.sp[tp], cur.sq[tq]);
        else if constexpr (MF == 32)
          acc[tp][tq] = mfma32x32x16<IN_DT>(cur.p[tp], cur.q[tq], acc[tp][tq]);
        else
          mfma16x16x32_acc<IN_DT>(acc[tp][tq], cur.p[tp], cur.q[tq]);
        // A two-argument hook (two DMA issues) runs after the group's 4th
        // and 6th MFMAs.
        if constexpr (std::is_invocable_v<decltype(hook), int, int>) {
          static_assert(TQ == 8, "issue positions within an 8-MFMA group");
          if (tq == 3 || tq == 5)
            hook(tp, tq == 5 ? 1 : 0);
        }
      }
      if constexpr (!std::is_invocable_v<decltype(hook), int, int>)
        hook(tp);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto no_hook = [](int) {};
  // Slices 0..KS-2 of `stage`, prefetching slices 1..KS-1.  On return
  // f[kLast] holds the last slice, which the caller multiplies after the
  // stage barrier while the next stage's slice 0 is read into f[0].
  Frag f[2];
  constexpr int kLast = (C::KS - 1) & 1;
  // The step just before a stage barrier spreads its fragment reads over its
  // first WAVE_GEMM_PRE_RG groups.
  auto body_h = [&](uint32_t stage, auto hook) {
#pragma unroll
    for (int kk = 0; kk + 1 < C::KS; ++kk) {
      if (kk + 2 < C::KS)
        step(f[kk & 1], f[(kk + 1) & 1], true, stage, kk + 1,
             [&](int tp) { hook(kk * TP + tp); }, std::integral_constant<int, TP>{});
      else
        step(f[kk & 1], f[(kk + 1) & 1], true, stage, kk + 1,
             [&](int tp) { hook(kk * TP + tp); },
             std::integral_constant<int, (WAVE_GEMM_PRE_RG < TP ? WAVE_GEMM_PRE_RG : TP)>{});
    }
  };
  auto body = [&](uint32_t stage) { body_h(stage, no_hook); };

  constexpr bool kTwoBuf = C::KS == 2 && C::NSTAGE == 2 && MF == 16 && !is_fp4(IN_DT);
  static_assert(!HYBRID || (!MASKED && (C::KS == 1 || kTwoBuf) && !is_fp4(IN_DT)),
                "the hybrid path is the one-slice or the 64-deep 16-bit DMA path");
  // HYBRID: the DMA pipeline covers the stages wholly inside K.
  const int kt_last = HYBRID ? min(kt_end, p.K / C::BK) : kt_end;
  const int nk = kt_last - kt_begin;
  const bool tail = HYBRID && kt_end > kt_last && kt_last >= kt_begin;
  if (nk <= 0 && !tail)
    return;

  if constexpr (!MASKED) {
    // Global byte offsets of this lane's DMA chunks (same for A and B).
    const uint32_t rowbytes = (uint32_t)p.K * 2u;
    uint32_t goff[C::DMA];
    // HYBRID: B's offsets differ (rows clamped to N instead of M).
    uint32_t goff_bh[HYBRID ? C::DMA : 1];
#pragma unroll
    for (int i = 0; i < C::DMA; ++i) {
      // Lane l of DMA issue i fills physical slot l%8 of super-row R.
      const uint32_t R = (wave * C::DMA + i) * 8 + (lane >> 3), ps = lane & 7;
      const uint32_t row = Geo<C>::row_of(R, ps), cb = Geo<C>::chunk_of(R, ps) << 4;
      if constexpr (HYBRID) {
        goff[i] = min(row, (uint32_t)(p.M - m0 - 1)) * rowbytes + cb;
        goff_bh[i] = min(row, (uint32_t)(p.N - n0 - 1)) * rowbytes + cb;
      } else {
        goff[i] = row * rowbytes + cb;
      }
    }
    const char *a_tile =
        reinterpret_cast<const char *>(p.A) + (size_t)m0 * rowbytes;
    const char *b_tile =
        reinterpret_cast<const char *>(p.B) + (size_t)n0 * rowbytes;
    const uint32_t lds0 = lds_addr(smem) + wave * C::DMA * 1024;
    // MXFP4 scales: a stage has 8 scale jobs, (group j/2 of the stage) x
    // (A if j is even, else B), 256 rows = 4 bytes a lane each; wave w runs
    // jobs w*SJ .. w*SJ+SJ-1 into [group][A rows | B rows] of the stage's
    // scale area.  All 64 lanes take part, so the loop body stays one basic
    // block and its explicit instruction order holds.
    // AITER: 16 jobs, (A if j < 8, else B) x the 256-byte scale block of
    // rows 32*(j%8) .. +31 that holds the stage's groups.
    static_assert(!kAiter || C::NSTAGE % 2 == 0, "AITER scale half follows stage parity");
    constexpr int SJ = IN_DT == kMXFP4 ? (C::BK / 4) / C::WAVES : kAiter ? 16 / C::WAVES : 0;
    uint32_t lds_sc[SJ > 0 ? SJ : 1], g_sc[SJ > 0 ? SJ : 1];
    // AITER scale blocks per 32-row block: ceil(groups / 8), groups = K/32
    // (p.K counts 16-bit units, 4 fp4 values each).
    const uint32_t g8 = ((uint32_t)p.K + 63u) / 64u;
    if constexpr (IN_DT == kMXFP4) {
#pragma unroll
      for (int s = 0; s < SJ; ++s) {
        const uint32_t j = wave * SJ + s, grp = j >> 1;
        lds_sc[s] = lds_addr(smem) + 2 * C::OPB + grp * 512 + (j & 1) * 256;
        g_sc[s] = grp * (uint32_t)((j & 1) ? p.N : p.M) + ((j & 1) ? n0 : m0) + lane * 4;
      }
    } else if constexpr (kAiter) {
#pragma unroll
      for (int s = 0; s < SJ; ++s) {
        const uint32_t j = wave * SJ + s, u = j & 7u;
        lds_sc[s] = lds_addr(smem) + 2 * C::OPB + (j >> 3) * 2048u + u * 256u;
        g_sc[s] = ((uint32_t)((j >> 3) ? n0 : m0) / 32u + u) * g8 * 256u + lane * 4u;
      }
    }
    // AITER B: per-lane offset of its 16 bytes in the 1 KiB run of row
    // block (wave*DMA + i); a row block spans 16 rows x 2*p.K bytes.
    uint32_t goff_b[C::DMA];
#pragma unroll
    for (int i = 0; i < C::DMA; ++i) {
      if constexpr (HYBRID)
        goff_b[i] = goff_bh[i];
      else
        goff_b[i] = kAiter ? (wave * C::DMA + i) * 32u * (uint32_t)p.K + lane * 16u : goff[i];
    }
    // DMA d of one stage (0 <= d < 2*DMA): A chunks first, then B; MXFP4
    // adds d = 2*DMA (A scales) and 2*DMA + 1 (B scales).
    auto issue_one = [&](uint32_t stage, int kt, int d) {
      const uint32_t l = lds0 + stage * C::STAGE;
      if (d < C::DMA) {
        dma16(l + d * 1024, a_tile + (size_t)kt * C::RB, goff[d]);
      } else if (d < 2 * C::DMA) {
        dma16(l + C::OPB + (d - C::DMA) * 1024,
              b_tile + (size_t)kt * (kAiter ? 1024 : C::RB), goff_b[d - C::DMA]);
      } else if constexpr (IN_DT == kMXFP4) {
        const int s = d - 2 * C::DMA;
        const bool is_b = ((wave * SJ + s) & 1) != 0;
        const uint32_t g0 = (uint32_t)kt * (C::BK / 8u) * (uint32_t)(is_b ? p.N : p.M);
        dma4(lds_sc[s] + stage * C::STAGE, is_b ? (const void *)p.b_scale : p.a_scale,
             g_sc[s] + g0);
      } else if constexpr (kAiter) {
        const int s = d - 2 * C::DMA;
        const bool is_b = ((wave * SJ + s) >> 3) != 0;
        dma4(lds_sc[s] + stage * C::STAGE, is_b ? (const void *)p.b_scale : p.a_scale,
             g_sc[s] + ((uint32_t)kt >> 1) * 256u);
      }
    };
    constexpr int kDmaPerStage = 2 * C::DMA + SJ;
    auto issue = [&](uint32_t stage, int kt) {
#pragma unroll
      for (int d = 0; d < kDmaPerStage; ++d)
        issue_one(stage, kt, d);
    };
    // Steady-state DMA schedule: the D2 issues of the prefetched stage are
    // spread over the G1 MFMA row groups before the stage barrier and (with
    // three or more stages) the G2 = TP groups after it: issue d follows
    // group d*G/D2.  At the barrier of iteration i stage i+1 must be
    // complete; issued after it are stages i+2 .. i+NSTAGE-2 and the P
    // pre-barrier issues of stage i+NSTAGE-1, hence vmcnt(D2*(NSTAGE-3)+P).
    constexpr int D2 = kDmaPerStage;
    constexpr int G1 = (C::KS - 1) * TP;
    constexpr int G2 = C::NSTAGE >= 3 ? TP : 0;
    constexpr int G = G1 + G2;
    constexpr int P = (G1 * D2 + G - 1) / G;  // #d with d*G/D2 < G1
    constexpr int kVm = D2 * (C::NSTAGE - 3) + P;
    static_assert(kVm >= 0 && kVm < 64, "vmcnt budget");
    auto issue_groups = [&](uint32_t stage, int kt, int g) {
#pragma unroll
      for (int d = 0; d < D2; ++d)
        if (d * G / D2 == g)
          issue_one(stage, kt, d);
    };
    // HYBRID K remainder: stage kt_last copied through VGPRs into ring slot
    // 0 (zero past K; rows past M / N clamped to the last valid row, as the
    // DMA clamps them), then its MFMA steps (one per slice).  Runs after the
    // pipeline's final wait + barrier, so no DMA is in flight and no wave
    // still reads the ring.
    auto tail_stage = [&]() {
      if constexpr (HYBRID) {
#pragma unroll
        for (int i = 0; i < C::DMA; ++i) {
          const uint32_t R = (wave * C::DMA + i) * 8 + (lane >> 3), ps = lane & 7;
          const int r = (int)Geo<C>::row_of(R, ps);
          const int kc = kt_last * C::BK + (int)(Geo<C>::chunk_of(R, ps) * 8);
          const uint16_t *ar = p.A + (size_t)min(m0 + r, p.M - 1) * p.K;
          const uint16_t *br = p.B + (size_t)min(n0 + r, p.N - 1) * p.K;
          const u32x4 va = load_chunk_k4(ar, kc, p.K);
          const u32x4 vb = load_chunk_k4(br, kc, p.K);
          uint8_t *d = smem + (wave * C::DMA + i) * 1024 + lane * 16;
          *reinterpret_cast<u32x4 *>(d) = va;
          *reinterpret_cast<u32x4 *>(d + C::OPB) = vb;
        }
        lds_barrier();
        read_frags(f[0], 0, 0);
        // Asm MFMA hazard: the accumulators' VALU zero fill (K < BK: no
        // pipeline ran) stays 2+ wait states ahead.
        asm volatile("s_nop 4" ::: "memory");
        if constexpr (C::KS == 2) {
          step(f[0], f[1], true, 0, 1, no_hook, std::integral_constant<int, TP>{});
          step(f[1], f[0], false, 0, 0, no_hook, std::integral_constant<int, TP>{});
        } else {
          step(f[0], f[1], false, 0, 0, no_hook, std::integral_constant<int, TP>{});
        }
        mfma_asm_drain();
        lds_barrier();  // fragment reads done before the ring is reused
      }
    };
    if (nk <= 0) {
      tail_stage();
      return;
    }
    // Prologue: stages 0 .. NSTAGE-2 in flight, wait for stage 0.
#pragma unroll
    for (int s = 0; s + 1 < C::NSTAGE; ++s)
      if (s < nk)
        issue(s, kt_begin + s);
    vm_wait_barrier();
    uint32_t stage = 0;
    int i = 0;
    if constexpr (C::KS == 1) {
      // One MFMA slice per stage: each step is one barrier (stage i+1 has
      // landed) and one MFMA pass that multiplies stage i, reads stage
      // i+1's fragments and issues stage i+NSTAGE-1's DMA (issue d after
      // group d * TP / D2).  The fragments alternate between f[0] and f[1],
      // two steps per loop trip, and every step is the same code: past the
      // last stage the DMA re-issues the last stage into the slot of stage
      // i-1 (no later step reads it) and the last step's fragment reads
      // land in f[] unused.  An odd stage count gets one leading step on
      // zero fragments (stage -1), which adds exact zeros to the
      // accumulators.
      constexpr int kRg = WAVE_GEMM_KS1_RG > 0 ? WAVE_GEMM_KS1_RG : TP;
      static_assert(kRg >= 1 && kRg <= TP, "read groups within the step");
      const auto rg = std::integral_constant<int, kRg>{};
      auto next = [&](Frag &cur, Frag &nxt) {
        const uint32_t ahead = (stage + C::NSTAGE - 1) % C::NSTAGE;
        const int kt_ahead = min(kt_begin + i + C::NSTAGE - 1, kt_last - 1);
        vm_wait_barrier<kVm>();
        stage = (stage + 1) % C::NSTAGE;
        step(cur, nxt, true, stage, 0,
             [&](int tp) { issue_groups(ahead, kt_ahead, tp); }, rg);
        ++i;
      };
      if (nk & 1) {
        f[0] = Frag{};
        stage = C::NSTAGE - 1;
        i = -1;
      } else {
        read_frags(f[0], 0, 0);
      }
      // The accumulators' zero fill is VALU: keep it 2+ wait states ahead
      // of the first asm MFMA.
      asm volatile("s_nop 4" ::: "memory");
      for (int t = i; t < nk; t += 2) {
        next(f[0], f[1]);
        next(f[1], f[0]);
      }
      mfma_asm_drain();
      vm_wait_barrier();
      if (tail)
        tail_stage();
      return;
    }
    if constexpr (kTwoBuf) {
      // 64-deep stages in two LDS buffers (the geometry of hipBLASLt's
      // kernel for this shape): every DMA instruction fetches 8 whole
      // 128-byte row segments (a 32-deep stage gives 16 half ones, and the
      // DMA then measured to stall the MFMA stream more).
      // Stage k sits in buffer k & 1 and is multiplied as two slices: the
      // even step (slice (k, 0) from registers, reading slice (k, 1)) needs
      // no barrier, since nothing it reads is new; the barrier in the odd
      // step (after its first two MFMAs, which use registers only: 1.7 %
      // fewer cycles a stage than a barrier before the step) waits for
      // stage k+1 (vmcnt(0)) and for every wave's reads of buffer k & 1, so
      // the rest of the odd step (slice (k, 1), reading (k+1, 0)) refills
      // that buffer with stage k+2, two DMA issues in each of its groups.  Cover for a stage's DMA: the rest of an odd step plus
      // an even step; one barrier per 64-deep stage.  Past the end the DMA
      // re-fetches the last stage into the free buffer.
      constexpr int D2 = kDmaPerStage;
      // Stage k+2's 16 DMA issues go two into each of the odd step's groups,
      // between its MFMAs (see kSpread): each issue stalls the wave's MFMA
      // stream.  Spread over 4 or 2 groups they measured 1 and 5 % slower
      // (the DMA backs up); moving 4 or 8 of them into the even step k+1,
      // 5-7 % slower (the even step's groups then wait on LDS).
      static_assert(D2 == 2 * TP, "one DMA issue per half group");
      issue(0, kt_begin);
      issue(1, kt_begin + min(1, nk - 1));
      vm_wait_barrier<D2>();  // stage 0 has landed
      read_frags(f[0], 0, 0);
      asm volatile("s_nop 4" ::: "memory");  // VALU zero fill -> asm MFMA
      const auto rg = std::integral_constant<int, TP>{};
      // The odd step always reads the next stage's first slice: after the
      // last stage those reads land, unused, in registers no MFMA reads (from
      // the other buffer, in bounds), and no read sits behind a branch.
      for (int k = 0; k < nk; ++k) {
        const uint32_t buf = (uint32_t)(k & 1);
        step(f[0], f[1], true, buf, 1, no_hook, rg);
        // (the stage barrier sits inside the odd step, after its 2nd MFMA)
        step(f[1], f[0], true, buf ^ 1u, 0,
             [&](int tp, int sub) { issue_one(buf, kt_begin + min(k + 2, nk - 1), 2 * tp + sub); },
             rg);
      }
      mfma_asm_drain();
      vm_wait_barrier();
      if (tail)
        tail_stage();
      return;
    }
    if constexpr (C::KS == 4 && C::NSTAGE == 2 && IN_DT == kMXFP4) {
      // MXFP4, 64-deep stages in two buffers: stage k (buffer k & 1) is
      // four 32x32x64 slices.  Steps 0-2 multiply slices 0-2 and read
      // slices 1-3; the barrier before step 3 waits for stage k+1 and for
      // every wave's reads of buffer k & 1, so step 3 (slice 3, reading
      // stage k+1's slice 0) refills that buffer with the first half of
      // stage k+2's DMA issues and step 0 of stage k+1 with the rest: three
      // to four steps of cover, against one to two on the 32-deep ring.
      // Past the end the DMA re-fetches the last stage; the last step's
      // reads of that copy land in registers no MFMA reads.
      constexpr int D2 = kDmaPerStage, DH = D2 / 2;
      auto issue_part = [&](uint32_t buf, int k, int first, int count, int tp) {
#pragma unroll
        for (int d = 0; d < count; ++d)
          if (d * TP / count == tp)
            issue_one(buf, kt_begin + min(k, nk - 1), first + d);
      };
      issue(0, kt_begin);
#pragma unroll
      for (int d = 0; d < DH; ++d)
        issue_one(1, kt_begin + min(1, nk - 1), d);
      vm_wait_barrier<DH>();  // stage 0 has landed
      read_frags(f[0], 0, 0);
      const auto rg = std::integral_constant<int, TP>{};
      for (int k = 0; k < nk; ++k) {
        const uint32_t buf = (uint32_t)(k & 1);
        step(f[0], f[1], true, buf, 1,
             [&](int tp) { issue_part(buf ^ 1u, k + 1, DH, D2 - DH, tp); }, rg);
        step(f[1], f[0], true, buf, 2, no_hook, rg);
        step(f[0], f[1], true, buf, 3, no_hook, rg);
        vm_wait_barrier<0>();
        step(f[1], f[0], true, buf ^ 1u, 0, [&](int tp) { issue_part(buf, k + 2, 0, DH, tp); },
             rg);
      }
      vm_wait_barrier();
      return;
    }
    read_frags(f[0], 0, 0);
    if constexpr (MF == 16)  // asm MFMAs: the one-slice path's hazard rules
      asm volatile("s_nop 4" ::: "memory");
    for (; i + C::NSTAGE - 1 < nk; ++i) {
      const uint32_t ahead = (stage + C::NSTAGE - 1) % C::NSTAGE;
      const int kt_ahead = kt_begin + i + C::NSTAGE - 1;
      body_h(stage, [&](int g) { issue_groups(ahead, kt_ahead, g); });
      if constexpr (G1 == 0 || G2 == 0) {
        // All issues fit before the barrier (or none did): none pending.
        if constexpr (G1 == 0)
          issue(ahead, kt_ahead);
      }
      vm_wait_barrier<kVm>();
      stage = (stage + 1) % C::NSTAGE;
      step(f[kLast], f[0], true, stage, 0,
           [&](int tp) { issue_groups(ahead, kt_ahead, G1 + tp); },
           std::integral_constant<int, TP>{});
    }
    // Drain: nothing more to issue; wait for everything.
    for (; i + 1 < nk; ++i) {
      body(stage);
      vm_wait_barrier();
      stage = (stage + 1) % C::NSTAGE;
      step(f[kLast], f[0], true, stage, 0, no_hook, std::integral_constant<int, TP>{});
    }
    body(stage);
    step(f[kLast], f[0], false, 0, 0, no_hook, std::integral_constant<int, TP>{});
    if constexpr (MF == 16)
      mfma_asm_drain();
    vm_wait_barrier();
  } else {
    // VGPR-staged loads with bounds checks (ragged M/N/K, unaligned K);
    // two LDS stages, the next stage held in VGPRs during the current one.
    // With 1 or 2 waves a stage is 16 or 8 chunks per operand and thread;
    // those CTAs copy the next stage after the current one's MFMAs instead,
    // 4 chunks at a time, so the staging registers stay within budget.
    constexpr int kChunks = C::DMA;  // per operand per thread
    constexpr bool kPrefetch = kChunks <= 4;
    constexpr int kHeld = kPrefetch ? kChunks : 4;
    // Source row (nullptr past the operand's end) and K column of chunk i.
    auto chunk_src = [&](int i, bool is_b, int &kc) -> const uint16_t * {
      const uint32_t R = (wave * C::DMA + i) * 8 + (lane >> 3), ps = lane & 7;
      const int r = (int)Geo<C>::row_of(R, ps);
      kc = (int)(Geo<C>::chunk_of(R, ps) * 8);
      if (is_b)
        return (n0 + r < p.N) ? p.B + (size_t)(n0 + r) * p.K : nullptr;
      return (m0 + r < p.M) ? p.A + (size_t)(m0 + r) * p.K : nullptr;
    };
    const uint16_t *arow[kHeld], *brow[kHeld];
    int kcol[kHeld];
    if constexpr (kPrefetch) {
#pragma unroll
      for (int i = 0; i < kChunks; ++i) {
        arow[i] = chunk_src(i, false, kcol[i]);
        brow[i] = chunk_src(i, true, kcol[i]);
      }
    }
    u32x4 ra[kHeld], rb[kHeld];
    // Chunks i0 .. i0 + kHeld - 1 of K step kt into VGPRs, then into LDS.
    auto load = [&](int kt, int i0) {
#pragma unroll
      for (int i = 0; i < kHeld; ++i) {
        if constexpr (!kPrefetch) {
          arow[i] = chunk_src(i0 + i, false, kcol[i]);
          brow[i] = chunk_src(i0 + i, true, kcol[i]);
        }
        ra[i] = load_chunk<VEC>(arow[i], kt * C::BK + kcol[i], p.K);
        rb[i] = load_chunk<VEC>(brow[i], kt * C::BK + kcol[i], p.K);
      }
    };
    auto store = [&](uint32_t stage, int i0) {
      uint8_t *s = smem + stage * C::STAGE + ((wave * C::DMA + i0) * 1024) + lane * 16;
#pragma unroll
      for (int i = 0; i < kHeld; ++i) {
        *reinterpret_cast<u32x4 *>(s + i * 1024) = ra[i];
        *reinterpret_cast<u32x4 *>(s + C::OPB + i * 1024) = rb[i];
      }
    };
    auto copy = [&](int kt, uint32_t stage) {
      for (int i0 = 0; i0 < kChunks; i0 += kHeld) {
        load(kt, i0);
        store(stage, i0);
      }
    };
    copy(kt_begin, 0);
    lds_barrier();
    read_frags(f[0], 0, 0);
    for (int i = 0; i < nk; ++i) {
      const uint32_t stage = i & 1;
      if (kPrefetch && i + 1 < nk)
        load(kt_begin + i + 1, 0);
      body(stage);
      if (i + 1 < nk) {
        if constexpr (kPrefetch)
          store(stage ^ 1, 0);
        else
          copy(kt_begin + i + 1, stage ^ 1);
      }
      lds_barrier();
      step(f[kLast], f[0], i + 1 < nk, stage ^ 1, 0, no_hook,
           std::integral_constant<int, TP>{});
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
// PACKED: C is tile-packed (column-major orientation: pp is m and q is n;
// pp % 4 == 0, so the 4 values are 4 consecutive elements in tile-packed
// order too).
template <class C, int OUT_DT, bool COL_MAJOR, bool MASKED, bool PACKED = false, typename Get>
__device__ __forceinline__ void store_tile(const Params &p, int m0, int n0,
                                           Get get, uint32_t pass = 0) {
  static_assert(!PACKED || COL_MAJOR, "tile-packed C uses the column-major orientation");
  const uint32_t wave = (threadIdx.x >> 6) + pass * C::WAVES;  // virtual wave
  const uint32_t lane = threadIdx.x & 63;
  const int wp = wave % C::WPN, wq = wave / C::WPN;
  const int P0 = COL_MAJOR ? m0 : n0, Q0 = COL_MAJOR ? n0 : m0;
  const int Pext = COL_MAJOR ? p.M : p.N, Qext = COL_MAJOR ? p.N : p.M;
  constexpr int MF = C::MF;
#pragma unroll
  for (int tq = 0; tq < C::TQ; ++tq) {
    const int q = Q0 + wq * (C::TQ * MF) + tq * MF + (lane % MF);
#pragma unroll
    for (int tp = 0; tp < C::TP; ++tp) {
#pragma unroll
      for (int g = 0; g < C::NG; ++g) {
        const int pp = P0 + wp * (C::TP * MF) + tp * MF + 8 * g + 4 * (lane / MF);
        const f32x4 v = get(tp, tq, g);
        const size_t idx = PACKED ? packed_m_part(p, pp) + packed_n_part(p, q)
                                  : (size_t)q * p.ldc + pp;
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

// Whole-tile store of a 16-bit output through LDS.  The MFMA layout leaves
// each lane 4 consecutive P values of one Q line, so a direct store
// instruction writes 8 bytes into each of 32 lines; here the tile is first
// transposed into 256 LDS lines of 512 bytes (128 KiB) and then written as
// whole 512-byte line runs, 16 bytes a lane.  In LDS line r, 16-byte chunk c
// sits at c ^ (r mod 32) and its two 8-byte halves are swapped when bit 4
// of r is set: the 32 lanes of one scattered write (32 lines, one chunk
// half each) then cover all 64 banks, and the line reads are contiguous.
// Needs: the mainloop's LDS reads and DMA finished, a whole tile, C 16-byte
// aligned and ldc * 2 a multiple of 16 bytes.  MASKED: any tile and any C;
// the line runs are cut at M / N, and a 16-byte piece that is partly outside
// or not 16-byte aligned in C is written element by element.
template <class C, int OUT_DT, bool COL_MAJOR, bool MASKED = false, typename Get>
__device__ __forceinline__ void store_tile_lds(const Params &p, int m0, int n0, uint8_t *smem,
                                               Get get) {
  static_assert(OUT_DT != kF32, "16-bit outputs only");
  constexpr int LINE = 512, CH = 32;
  static_assert(C::SMEM >= 256 * LINE, "LDS ring smaller than the output tile");
  const uint32_t tid = threadIdx.x;
  const uint32_t wave = tid >> 6, lane = tid & 63;
  const int wp = wave % C::WPN, wq = wave / C::WPN;
  const int P0 = COL_MAJOR ? m0 : n0, Q0 = COL_MAJOR ? n0 : m0;
  char *out = reinterpret_cast<char *>(p.C);
  constexpr int MF = C::MF;
#pragma unroll
  for (int tq = 0; tq < C::TQ; ++tq) {
    const uint32_t r = (uint32_t)(wq * (C::TQ * MF) + tq * MF) + (lane % MF);
#pragma unroll
    for (int tp = 0; tp < C::TP; ++tp) {
#pragma unroll
      for (int g = 0; g < C::NG; ++g) {
        // Elements e .. e+3 of line r, e = wp*TP*MF + tp*MF + 8g + 4*(lane/MF):
        // chunk e/8, half (e/4)%2.
        const uint32_t e = wp * (C::TP * MF) + tp * MF + 8 * g + 4 * (lane / MF);
        const uint32_t c = e >> 3;
        const uint32_t half = ((e >> 2) ^ (r >> 4)) & 1u;
        const f32x4 v = get(tp, tq, g);
        *reinterpret_cast<u32x2 *>(smem + r * LINE + ((c ^ (r % CH)) * 16) + half * 8) =
            u32x2{pack2<OUT_DT>(v[0], v[1]), pack2<OUT_DT>(v[2], v[3])};
      }
    }
  }
  lds_barrier();
  constexpr int PER = 256 * CH / C::THREADS;
  const int Pext = COL_MAJOR ? p.M : p.N, Qext = COL_MAJOR ? p.N : p.M;
  const bool vec16 = ((((uintptr_t)p.C | (uintptr_t)p.ldc * 2) & 15) == 0);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint32_t flat = i * C::THREADS + tid;
    const uint32_t r = flat / CH, c = flat % CH;
    u32x4 v = *reinterpret_cast<const u32x4 *>(smem + r * LINE + ((c ^ (r % CH)) * 16));
    if ((r >> 4) & 1u)
      v = u32x4{v[2], v[3], v[0], v[1]};
    const size_t q = (size_t)(Q0 + (int)r);
    // Whole tiles store non-temporally: C is not read again by this launch.
    // With plain stores one round of tiles leaves its C lines (32 MiB for 256
    // f16 tiles) dirty in L2, and their write-back slows the next round's K
    // loop (wave-bench, same box: 8192^3 f16 1479-1482 -> 1510-1514 TFLOP/s,
    // rand_int inputs 1701 -> 1863-1875, 16384x8192x4096 1403 -> 1447-1451,
    // MXFP4 4096^2 x 32768 +1-2 %).  The bounds-checked branch (the hybrid
    // path's ragged tiles) keeps plain stores: config 3b measured 1.3 %
    // slower with non-temporal ones.
    if constexpr (!MASKED) {
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(out + (q * p.ldc + P0) * 2 + c * 16));
    } else {
      const int pc = P0 + 8 * (int)c;
      if ((int)q < Qext && pc < Pext) {
        uint16_t *dst = reinterpret_cast<uint16_t *>(p.C) + q * p.ldc + pc;
        if (vec16 && pc + 8 <= Pext) {
          *reinterpret_cast<u32x4 *>(dst) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (pc + e < Pext)
              dst[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
  }
  // Every wave's line reads are done before LDS is written again (the next
  // tile's DMA ring in a grid-stride caller).
  lds_barrier();
}

// Store one finished tile: 16-bit output goes through LDS (store_tile_lds):
// whole tiles when C allows 16-byte line runs, ragged tiles always (with
// bounds checks on the line runs, which also keeps the per-accumulator
// bounds logic and its registers out of the kernel; not with 16 waves,
// whose 128 registers a wave it overflows); f32 output, twice the bytes, is
// bound by HBM writes either way and is stored directly (measured faster).
// Tile-packed C is stored directly: each wave's 64 lanes already write one
// contiguous 16x16 tile.
template <class C, int OUT_DT, bool COL_MAJOR, bool MASKED, bool PACKED = false, typename Get>
__device__ __forceinline__ void store_out(const Params &p, int m0, int n0, uint8_t *smem,
                                          Get get) {
  if constexpr (MASKED && !PACKED && OUT_DT != kF32 && C::WAVES < 16) {
    store_tile_lds<C, OUT_DT, COL_MAJOR, true>(p, m0, n0, smem, get);
    return;
  } else if constexpr (!MASKED && !PACKED && OUT_DT != kF32) {
    if ((((uintptr_t)p.C | (uintptr_t)p.ldc * 2) & 15) == 0) {
      store_tile_lds<C, OUT_DT, COL_MAJOR>(p, m0, n0, smem, get);
      return;
    }
  }
  store_tile<C, OUT_DT, COL_MAJOR, MASKED, PACKED>(p, m0, n0, get);
}

// One 256x256 output tile: CTA `raw` of a grid of tiles_m * tiles_n CTAs,
// with W waves (0: the library default).  smem: CfgFor<IN_DT, W>::SMEM bytes
// of 1024-byte-aligned LDS.
template <int IN_DT, int W = 0>
using CfgFor = std::conditional_t<IN_DT == kMXFP4, Fp4CfgW<W>,
                                  std::conditional_t<IN_DT == kMXFP4A, Fp4ACfgW<W>, TileCfgW<W>>>;

// HYBRID: every tile on the DMA ring (see mainloop), edge tiles stored with
// bounds checks.
// DEEP (canonical MXFP4, K a multiple of 256 values): 64-deep stages.
template <int IN_DT, int OUT_DT, bool COL_MAJOR, bool MASKED, int VEC, int W = 0,
          bool PACKED = false, bool HYBRID = false, bool DEEP = false>
__device__ __forceinline__ void tiled_cta(const Params &p, int raw, uint8_t *smem) {
  static_assert(!DEEP || IN_DT == kMXFP4, "64-deep MXFP4 stages: canonical layout");
  // Whole tiles run TileCfg's MFMA shape; ragged tiles the 32x32 one.
  using C = std::conditional_t<
      MASKED, DefaultCfgW<W>,
      std::conditional_t<HYBRID, HybridTileCfgW<W>,
                         std::conditional_t<DEEP, Fp4Cfg64W<W>, CfgFor<IN_DT, W>>>>;
  static_assert(!HYBRID || (!MASKED && !PACKED), "hybrid: row- or column-major C");
  static_assert(C::SMEM == CfgFor<IN_DT, W>::SMEM && C::THREADS == CfgFor<IN_DT, W>::THREADS,
                "one LDS size and block size per input type");
  static_assert(!is_fp4(IN_DT) || !MASKED, "MXFP4 takes whole tiles only");
  static_assert(!is_fp4(IN_DT) || C::WAVES == 4 || C::WAVES == 8, "MXFP4 runs 4 or 8 waves");
  int tm, tn;
  tile_coords(raw, p.tiles_m, p.tiles_n, p.group_m, true, tm, tn);
  // The tile origin is uniform; readfirstlane keeps it (and the DMA bases
  // derived from it) in SGPRs, as the DMA's scalar base operand requires.
  const int m0 = __builtin_amdgcn_readfirstlane(tm * kTile);
  const int n0 = __builtin_amdgcn_readfirstlane(tn * kTile);
  typename C::Acc acc[C::TP][C::TQ];
  auto zero = [&]() {
#pragma unroll
    for (int i = 0; i < C::TP; ++i)
#pragma unroll
      for (int j = 0; j < C::TQ; ++j)
        acc[i][j] = typename C::Acc{};
  };
  const int kt_n = (p.K + C::BK - 1) / C::BK;
  auto get = [&](int tp, int tq, int g) {
    return f32x4{acc[tp][tq][4 * g], acc[tp][tq][4 * g + 1],
                 acc[tp][tq][4 * g + 2], acc[tp][tq][4 * g + 3]};
  };
  if constexpr (HYBRID) {
    zero();
    mainloop<C, IN_DT, COL_MAJOR, false, VEC, true>(p, m0, n0, 0, kt_n, smem, acc);
    if constexpr (OUT_DT != kF32)
      store_tile_lds<C, OUT_DT, COL_MAJOR, true>(p, m0, n0, smem, get);
    else
      store_tile<C, OUT_DT, COL_MAJOR, true>(p, m0, n0, get);
  } else if constexpr (C::PASSES == 1) {
    zero();
    mainloop<C, IN_DT, COL_MAJOR, MASKED, VEC>(p, m0, n0, 0, kt_n, smem, acc);
    store_out<C, OUT_DT, COL_MAJOR, MASKED, PACKED>(p, m0, n0, smem, get);
  } else {
    // Fewer than 4 waves: one K loop per virtual wave, each stored directly.
    for (uint32_t pass = 0; pass < (uint32_t)C::PASSES; ++pass) {
      zero();
      mainloop<C, IN_DT, COL_MAJOR, MASKED, VEC>(p, m0, n0, 0, kt_n, smem, acc, pass);
      store_tile<C, OUT_DT, COL_MAJOR, MASKED, PACKED>(p, m0, n0, get, pass);
    }
  }
}

template <int IN_DT, int OUT_DT, bool COL_MAJOR, bool MASKED, int VEC, bool PACKED = false,
          bool HYBRID = false, bool DEEP = false>
__global__ __launch_bounds__(CfgFor<IN_DT>::THREADS, 1) void tiled_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[CfgFor<IN_DT>::SMEM];
  tiled_cta<IN_DT, OUT_DT, COL_MAJOR, MASKED, VEC, 0, PACKED, HYBRID, DEEP>(p, blockIdx.x, smem);
}

// ---------------------------------------------------------------- Stream-K
// Work unit = (tile, 64-wide K step); W = T * I units split into `workers`
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

// Per-thread scratch layout: 16-byte group j (0 .. 65536/THREADS/4 - 1) of
// thread t's share of the 256x256 tile lives at f32x4 index
// slot_base/4 + j * THREADS + t, so publishing and reducing are fully
// coalesced 16-byte accesses and need no coordinate math.
// Worker `worker` of p.workers.  smem: DefaultCfg::SMEM bytes of
// 1024-byte-aligned LDS; arrival: one int of LDS.  HYBRID (with !MASKED):
// ragged M / N or K off the stage on the DMA ring, as for the tiled kernel,
// with bounds-checked stores.
template <int IN_DT, int OUT_DT, bool COL_MAJOR, bool MASKED, int VEC, bool HYBRID = false>
__device__ __forceinline__ void streamk_cta(const Params &p, int worker, uint8_t *smem,
                                            int *arrival) {
  // Whole-tile ranges run the 16x16 MFMA shape (64-deep stages); ragged
  // tiles the 32x32 one.
  using C = std::conditional_t<MASKED, DefaultCfg, HybridTileCfgW<>>;
  static_assert(!(HYBRID && MASKED), "hybrid runs the DMA mainloop");
  constexpr bool SM = MASKED || HYBRID;  // bounds-checked stores
  static_assert(C::SMEM == DefaultCfg::SMEM && C::THREADS == DefaultCfg::THREADS,
                "one LDS size and block size");
  // XCD-aware worker numbering, as for tiled CTAs: the dispatcher places
  // workgroup i on XCD i % 8, so renumbering makes the workers of one XCD
  // consecutive; their work units, and so their tiles, are then adjacent and
  // share A/B panels in that XCD's L2.  Every use of the worker index below
  // (intervals, owners, partial slots) takes the renumbered one.
  if ((p.workers & 7) == 0)
    worker = (worker & 7) * (p.workers >> 3) + (worker >> 3);
  const int tiles = p.tiles_m * p.tiles_n;
  const int iters = (p.K + kSKUnit - 1) / kSKUnit;
  const int ksteps = (p.K + C::BK - 1) / C::BK;  // mainloop steps per tile
  constexpr int kStepsPerUnit = kSKUnit / C::BK;
  const int total = tiles * iters;
  const Interval iv = sk_interval(total, p.workers, worker);
  const bool aligned = (total % p.workers == 0) && ((total / p.workers) % iters == 0);

  constexpr int TP = C::TP, TQ = C::TQ, NT = C::THREADS;
  typename C::Acc acc[TP][TQ];
  auto zero = [&]() {
#pragma unroll
    for (int i = 0; i < TP; ++i)
#pragma unroll
      for (int j = 0; j < TQ; ++j)
        acc[i][j] = typename C::Acc{};
  };
  auto get = [&](int tp, int tq, int g) {
    return f32x4{acc[tp][tq][4 * g], acc[tp][tq][4 * g + 1], acc[tp][tq][4 * g + 2],
                 acc[tp][tq][4 * g + 3]};
  };
  // Aligned: every worker owns whole tiles and visits worker, worker + P,
  // ... so the tiles in flight at any moment are adjacent (no partials, no
  // atomics).  Split: the tiles of the worker's interval, in order.  Both
  // share one mainloop call site, so its code is inlined once (two copies
  // of the hybrid ring spilled 79 VGPRs).
  const int tile_lo = aligned ? worker : iv.begin / iters;
  const int tile_hi = aligned ? tiles - 1 : (iv.end - 1) / iters;
  const int tile_step = aligned ? p.workers : 1;
  int slot = 0;
  for (int tile = tile_lo; tile <= tile_hi; tile += tile_step) {
    const int kb = aligned ? 0 : max(iv.begin, tile * iters) - tile * iters;
    const int ke = aligned ? iters : min(iv.end, (tile + 1) * iters) - tile * iters;
    int tm, tn;
    tile_coords(tile, p.tiles_m, p.tiles_n, p.group_m, false, tm, tn);
    zero();
    mainloop<C, IN_DT, COL_MAJOR, MASKED, VEC, HYBRID>(
        p, tm * kTile, tn * kTile, kb * kStepsPerUnit,
        min(ke * kStepsPerUnit, ksteps), smem, acc);
    if (kb == 0 && ke == iters) {
      store_out<C, OUT_DT, COL_MAJOR, SM>(p, tm * kTile, tn * kTile, smem, get);
      continue;
    }
    // Publish this worker's fp32 partial: 16-byte group g of MFMA tile
    // (tp, tq) of thread t at f32x4 index ((tp*TQ + tq)*NG + g)*NT + t, so
    // every store and load instruction covers 4 KiB contiguously.  Plain
    // stores: the accumulators go out of AGPRs directly (device-coherent
    // buffer stores need them in VGPRs and spilled 146 VGPRs here).
    f32x4 *mine = reinterpret_cast<f32x4 *>(p.scratch + ((size_t)worker * 2 + slot) * kTileElems);
#pragma unroll
    for (int tp = 0; tp < TP; ++tp)
#pragma unroll
      for (int tq = 0; tq < TQ; ++tq)
#pragma unroll
        for (int g = 0; g < C::NG; ++g)
          mine[((tp * TQ + tq) * C::NG + g) * NT + threadIdx.x] =
              f32x4{acc[tp][tq][4 * g], acc[tp][tq][4 * g + 1], acc[tp][tq][4 * g + 2],
                    acc[tp][tq][4 * g + 3]};
    ++slot;
    const int first_owner = sk_owner(total, p.workers, tile * iters);
    const int last_owner = sk_owner(total, p.workers, (tile + 1) * iters - 1);
    const int parts = last_owner - first_owner + 1;
    // Every wave waits for its partial stores (vmcnt(0): acknowledged by
    // L2) before the barrier; thread 0's agent-scope release ticket then
    // writes the XCD's L2 back, which publishes all of them at once.  The
    // last arriver reads the partials with device-coherent (sc1) loads,
    // issued after the barrier that follows its ticket: they read the
    // coherence point, so it needs no acquire (an L2 invalidate).
    vm_wait_barrier();
    if (threadIdx.x == 0)
      *arrival = __hip_atomic_fetch_add(&p.counters[tile], 1u, __ATOMIC_RELEASE,
                                        __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*arrival != parts - 1)
      continue;
    // Last arriver: reduce all contributors' partials (its own included,
    // reloaded) in worker order, a fixed order, so the result does not
    // depend on arrival order: s = ((0 + p_first) + p_second) + ....
    auto part_of = [&](int c) {
      return coherent_rsrc(
          p.scratch + ((size_t)c * 2 + sk_slot(total, p.workers, c, tile, iters)) * kTileElems,
          kTileElems * 4);
    };
    // Partial group (tp, tq, g) of this thread: byte offset tid16 + at()
    // (the asm keeps tid16 from being hoisted, live, across the mainloop).
    uint32_t tid16 = threadIdx.x * 16;
    asm volatile("" : "+v"(tid16));
    auto at = [&](int tp, int tq, int g) {
      return (uint32_t)((tp * TQ + tq) * C::NG + g) * NT * 16u;
    };
    if (parts >= 2) {
      if (parts > 2) {
        // More than two contributors: fold all but the last, in worker
        // order from +0, into the first one's slot (read before it is
        // overwritten, by the same thread, at the same index; no worker
        // writes that slot again in this launch).  The pass below then adds
        // the last one to (+0 + fold), which equals the fold exactly (a sum
        // begun at +0 is never -0), so the result is the serial
        // ((0 + p_first) + p_second) + ... bit for bit.  kFold groups of
        // two contributors are in flight per round trip; accumulating
        // inside the store callback instead spilled 96-141 VGPRs.
        constexpr int kGroups = TP * TQ * C::NG, kFold = 8;
        static_assert(kGroups % kFold == 0, "whole fold batches");
        const __amdgpu_buffer_rsrc_t dst = part_of(first_owner);
        auto off = [&](int q) { return (uint32_t)q * NT * 16u; };
        for (int q0 = 0; q0 < kGroups; q0 += kFold) {
          f32x4 r[kFold];
#pragma unroll
          for (int j = 0; j < kFold; ++j)
            r[j] = f32x4{0.f, 0.f, 0.f, 0.f};
          int c = first_owner;
          for (; c + 1 < last_owner; c += 2) {
            const __amdgpu_buffer_rsrc_t x = part_of(c), y = part_of(c + 1);
            f32x4 a[kFold], b[kFold];
#pragma unroll
            for (int j = 0; j < kFold; ++j) {
              a[j] = coherent_load16(x, tid16, off(q0 + j));
              b[j] = coherent_load16(y, tid16, off(q0 + j));
            }
#pragma unroll
            for (int j = 0; j < kFold; ++j) {
              r[j] += a[j];
              r[j] += b[j];
            }
          }
          if (c < last_owner) {
            const __amdgpu_buffer_rsrc_t x = part_of(c);
#pragma unroll
            for (int j = 0; j < kFold; ++j)
              r[j] += coherent_load16(x, tid16, off(q0 + j));
          }
#pragma unroll
          for (int j = 0; j < kFold; ++j)
            coherent_store16(dst, tid16, r[j], off(q0 + j));
        }
        // The pass below reads these groups back (same thread, same
        // offsets): let the stores complete first.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      // s = (0 + X) + Y with X the first slot (p_first, or the fold) and Y
      // the last contributor's partial.  The last arriver still holds its
      // own partial in its accumulators, so one of the two comes from
      // registers when it is the first contributor of two (X) or the last
      // one (Y); only a middle contributor of three or more reads both
      // slots.  (Reading the accumulators after the MFMAs: the publish's
      // reads of them above already covered the asm MFMA hazard.)
      // A batch of partial groups (KB MFMA tiles of a row, over TB rows) is
      // loaded at the first of them, before that batch's stores (which the
      // compiler cannot move loads across), so 16 loads are in flight at
      // once: kBatch tiles from both slots, or twice as many from one.  A
      // contributor loop inside the callback waited out one memory round
      // trip per group: ~140 us a tile.  Stored directly: the LDS-staged
      // epilogue costs VGPR spills here.
      constexpr int kBatch = 8 / C::NG < TP ? 8 / C::NG : TP;
      static_assert(TP % kBatch == 0, "whole batches per row");
      const __amdgpu_buffer_rsrc_t pa = part_of(first_owner), pb = part_of(last_owner);
      auto reduce = [&](auto role) {
        // R: 0 both slots, 1 X from registers, 2 Y from registers.
        constexpr int R = decltype(role)::value;
        constexpr int KB = R == 0 ? kBatch : (2 * kBatch <= TP ? 2 * kBatch : TP);
        constexpr int TB = (R != 0 && KB == kBatch) ? 2 : 1;  // then KB == TP
        static_assert(TP % KB == 0 && TQ % TB == 0 && (TB == 1 || KB == TP), "batches");
        f32x4 rx[TB][KB][C::NG], ry[TB][KB][C::NG];
        store_tile<C, OUT_DT, COL_MAJOR, SM>(
            p, tm * kTile, tn * kTile, [&](int tp, int tq, int g) {
              if (g == 0 && tp % KB == 0 && tq % TB == 0) {
#pragma unroll
                for (int u = 0; u < TB; ++u)
#pragma unroll
                  for (int j = 0; j < KB; ++j)
#pragma unroll
                    for (int h = 0; h < C::NG; ++h) {
                      if constexpr (R != 1)
                        rx[u][j][h] = coherent_load16(pa, tid16, at(tp + j, tq + u, h));
                      if constexpr (R != 2)
                        ry[u][j][h] = coherent_load16(pb, tid16, at(tp + j, tq + u, h));
                    }
                // Buffer loads do not alias C's global stores for the
                // compiler, which would otherwise hoist every batch's loads
                // to the top (spilling); keep each batch at its place.
                asm volatile("" ::: "memory");
              }
              f32x4 s = {0.f, 0.f, 0.f, 0.f};
              if constexpr (R == 1)
                s += get(tp, tq, g);
              else
                s += rx[tq % TB][tp % KB][g];
              if constexpr (R == 2)
                s += get(tp, tq, g);
              else
                s += ry[tq % TB][tp % KB][g];
              return s;
            });
      };
      // (The VGPR-staged 32x32 path keeps reading both slots: three
      // variants there spill 211 VGPRs.)
      if (!MASKED && worker == last_owner)
        reduce(std::integral_constant<int, MASKED ? 0 : 2>{});
      else if (!MASKED && parts == 2)
        reduce(std::integral_constant<int, MASKED ? 0 : 1>{});
      else
        reduce(std::integral_constant<int, 0>{});
    } else {
      store_tile<C, OUT_DT, COL_MAJOR, SM>(
          p, tm * kTile, tn * kTile, [&](int tp, int tq, int g) {
            f32x4 s = {0.f, 0.f, 0.f, 0.f};
            for (int c = first_owner; c <= last_owner; ++c)
              s += coherent_load16(part_of(c), tid16, at(tp, tq, g));
            return s;
          });
    }
    // Counter back to zero for the next launch (ordered after this one by
    // the kernel boundary, so no release is needed).
    __syncthreads();
    if (threadIdx.x == 0)
      __hip_atomic_store(&p.counters[tile], 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int IN_DT, int OUT_DT, bool COL_MAJOR, bool MASKED, int VEC, bool HYBRID = false>
__global__ __launch_bounds__(DefaultCfg::THREADS, 1) void streamk_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[DefaultCfg::SMEM];
  __shared__ int arrival;
  streamk_cta<IN_DT, OUT_DT, COL_MAJOR, MASKED, VEC, HYBRID>(p, blockIdx.x, smem, &arrival);
}

// ------------------------------------------------------------- launchers
// mode: 0 = aligned fast path (LDS DMA), 8/4/1 = masked path with that many
// elements per global load, kModeHybrid8/4 = hybrid DMA path whose K tail
// loads 8/4 elements at a time (tile-packed C runs the masked path with the
// same load width instead).
constexpr int kModeHybrid8 = 18, kModeHybrid4 = 14;
template <int IN_DT, int OUT_DT, bool CM, bool SK>
hipError_t launch_variant(const Params &p, int mode, hipStream_t stream) {
  const dim3 block(DefaultCfg::THREADS);
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
  // Tile-packed C (tiled kernel, column-major orientation only).
#define WAVE_LAUNCH_PACKED(MASKED, VEC)                                        \
  hipLaunchKernelGGL((tiled_kernel<IN_DT, OUT_DT, true, MASKED, VEC, true>), grid, block, 0, \
                     stream, p)
  if constexpr (CM && !SK) {
    if (p.pk) {
      switch (mode) {
      case 0: WAVE_LAUNCH_PACKED(false, 8); break;
      case 8: case kModeHybrid8: WAVE_LAUNCH_PACKED(true, 8); break;
      case 4: case kModeHybrid4: WAVE_LAUNCH_PACKED(true, 4); break;
      default: WAVE_LAUNCH_PACKED(true, 1); break;
      }
      return hipGetLastError();
    }
  }
  // Hybrid DMA path.
  if (mode == kModeHybrid8 || mode == kModeHybrid4) {
    if constexpr (SK) {
      if (mode == kModeHybrid8)
        hipLaunchKernelGGL((streamk_kernel<IN_DT, OUT_DT, CM, false, 8, true>), grid, block, 0,
                           stream, p);
      else
        hipLaunchKernelGGL((streamk_kernel<IN_DT, OUT_DT, CM, false, 4, true>), grid, block, 0,
                           stream, p);
    } else {
      if (mode == kModeHybrid8)
        hipLaunchKernelGGL((tiled_kernel<IN_DT, OUT_DT, CM, false, 8, false, true>), grid, block,
                           0, stream, p);
      else
        hipLaunchKernelGGL((tiled_kernel<IN_DT, OUT_DT, CM, false, 4, false, true>), grid, block,
                           0, stream, p);
    }
    return hipGetLastError();
  }
  switch (mode) {
  case 0: WAVE_LAUNCH(false, 8); break;
  case 8: case kModeHybrid8: WAVE_LAUNCH(true, 8); break;
  case 4: case kModeHybrid4: WAVE_LAUNCH(true, 4); break;
  default: WAVE_LAUNCH(true, 1); break;
  }
#undef WAVE_LAUNCH
#undef WAVE_LAUNCH_PACKED
  return hipGetLastError();
}

#define WAVE_GEMM_INSTANTIATE(IN, OUT, SK)                                     \
  template hipError_t launch_variant<IN, OUT, false, SK>(const Params &, int,   \
                                                         hipStream_t);         \
  template hipError_t launch_variant<IN, OUT, true, SK>(const Params &, int,    \
                                                        hipStream_t);

} // namespace gemm
} // namespace wave
