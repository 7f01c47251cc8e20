// attention_kernels.hpp -- flash-attention forward for gfx950, head_dim 128.
//
// O = softmax(Q K^T * scale) V per (batch, query head), with optional causal
// mask and grouped-query heads (kv_head = q_head / (Hq / Hkv)).  This is the
// math of the reference kernel `flash_attention_bf16_gfx950`
// (python/mlir/dialects/wave_flash_attention.py:586-728 softmax, :814 PV,
// :1034-1095 store; layout Q,K,V,O = [B*H][S][128], runner
// tools/wave-fa-calibrate/wave-fa-gfx950-runner.cpp:396-402), generalised to
// f16 / bf16, causal masking and GQA.
//
// Design (one CTA = 256 query rows of one head, 8 waves of 64 lanes, one
// CTA per CU):
//  * Each wave owns 32 query rows and computes S^T = K . Q^T with
//    v_mfma_f32_32x32x16 (A = K rows from LDS, B = Q fragments held in
//    VGPRs for the whole kernel).  In that orientation lane l owns query
//    l%32 and 32 of the 64 keys of a tile, so the row max and row sum are
//    in-lane reductions plus one exchange with lane l^32, and the online
//    softmax rescale of O is a per-lane multiply.
//  * O^T += V^T . P^T with A = V^T from LDS and B = P^T taken straight from
//    the S^T accumulators (packed to 16 bits): accumulator registers 8s..8s+7
//    of a 32-key block hold keys {16s+4h+0..3, 16s+8+4h+0..3} for lane half
//    h, which is exactly one MFMA K slice once V^T is stored with each
//    16-key group permuted as [0-3, 8-11, 4-7, 12-15].
//  * K tiles (64 keys x 256 B) arrive by global_load_lds_dwordx4 with an XOR
//    swizzle (chunk c of row r at c ^ (r & 15)) into a 4-tile ring; V tiles
//    are loaded into VGPRs, transposed in registers and written to LDS as
//    V^T rows of 64 keys (+16 B padding, 144 B pitch) into a 2-tile ring.
//  * The two groups of 4 waves alternate between a matrix-only segment (the
//    MFMAs of S(t+1) and O += V(t) P(t)) and a vector-only segment (the
//    softmax of the next tile), one segment apart, so every SIMD pairs one
//    wave's MFMA stream with the other wave's softmax (fwd_pp_kernel).
//  * exp2 with the scale folded into one FMA; the running max is only
//    raised (and O rescaled) when a tile's max exceeds it by more than 8
//    (log2 units), as in the reference's lazy rescale
//    (wave_flash_attention.py:557-583); P stays below 2^8.  Row sums are
//    v_dot2 products of the packed 16-bit P with ones, so they sum exactly
//    the values that multiply V.
//  * CTAs of one head are placed on the same XCD so its K/V stay in that
//    XCD's L2; causal grids start with the longest query blocks.
#pragma once

#include "attention.hpp"
#include "wave_common.hpp"

#include <type_traits>

namespace wave {
namespace attention {

constexpr int kD = 128;
constexpr float kLn2 = 0.69314718055994531f;
constexpr int kBN = 64;                          // keys per tile
constexpr int kKRowBytes = kD * 2;               // 256
constexpr int kKBytes = kBN * kKRowBytes;        // 16 KiB
constexpr int kVtPitch = kBN * 2 + 16;           // 144 B per d row of V^T
constexpr int kVtBytes = kD * kVtPitch;          // 18 KiB
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleThreshold = 8.0f;

struct Params {
  const uint16_t *Q, *K, *V;
  uint16_t *O;
  int batch, q_heads, kv_heads, seq_q, seq_k;
  int q_blocks;   // ceil(seq_q / (32 * NW))
  int causal;
  float scale_log2;  // softmax scale * log2(e)
  float fixed_max;   // fixed-max kernels: the row max of every row (log2 units)
  float *lse;        // optional [batch*q_heads][seq_q]: ln sum_k exp(scale * q.k)
};

// Linear CTA id -> (batch*head, query block).
__device__ __forceinline__ void block_coords(const Params &p, int raw, int &bh, int &qb) {
  const int total = p.q_blocks * p.batch * p.q_heads;
  // Dispatch puts CTA i on XCD i % 8; make consecutive pids share an XCD.
  int pid = raw;
  if ((total & 7) == 0)
    pid = (raw & 7) * (total >> 3) + (raw >> 3);
  bh = pid / p.q_blocks;
  qb = pid - bh * p.q_blocks;
  if (p.causal)
    qb = p.q_blocks - 1 - qb;  // longest rows first
}

// ------------------------------------------------------------------------
// fwd_pp_kernel: 8 waves x 32 query rows per CTA (256 rows, one CTA per
// CU), run as two groups of four waves -- A = waves 0-3, B = waves 4-7;
// wave w shares SIMD w % 4 with wave w + 4 -- that the workgroup barriers
// keep one segment apart ("ping-pong"):
//
//   segment   2t          2t+1        2t+2
//   group A   G(t)        SM(t+1)     G(t+1)
//   group B   SM(t)       G(t)        SM(t+1)
//
// G(t), matrix only: S(t+1) = K(t+1) . Q^T and O^T += V(t)^T . P(t)^T,
// 32 MFMAs fed from LDS.  SM(t), vector only: mask and row max of S(t),
// the lazy rescale of O, P(t) = exp2(S(t) * c - m) packed to 16 bits, the
// row sums of P(t) (v_dot2 on the packed values), half of a V^T transpose
// and this wave's share of a K DMA.  Each SIMD therefore always pairs one
// wave's MFMA stream with the other wave's softmax.  All 8 waves share each
// K and V^T tile, so per query row the K/V traffic from L2 and the
// transpose work are half of fwd_kernel's.
//
// Buffers (the unrolled loop makes every index a compile-time constant):
//  * K ring of 4 tiles, tile j in buffer j % 4, read in G(j-1) (segments
//    2j-2 and 2j-1).  Both groups issue K(j) in SM(j-3) (segments 2j-5 and
//    2j-6), after the last read of K(j-4); each wave's next V wait (next
//    SM) completes its share before the barrier that precedes G(j-1).
//  * V^T ring of 2 tiles, V^T(j) read in G(j) (segments 2j, 2j+1).  A
//    writes its half (d rows 0-63) in SM(j) (segment 2j-1), B its half (d
//    rows 64-127) in SM(j-1) (segment 2j-2); the buffer's previous tile
//    V^T(j-2) was last read in segment 2j-3.
// Both groups run the same code: B joins one extra barrier before its loop
// (its idle segment 0); after the last G only A joins a barrier (it pairs
// with the end of B's last SM).  Barriers per wave: 2 * ntiles + 1.
constexpr int kPPWaves = 8;
constexpr int kKRingPP = 4;
#ifndef WAVE_FA_PF
#define WAVE_FA_PF 4  // LDS fragment prefetch depth (MFMAs) in G
#endif
#ifndef WAVE_FA_TAIL
#define WAVE_FA_TAIL 8  // PV MFMAs of G(t) issued at the start of SM(t+1)
#endif
template <int N> using I_ = std::integral_constant<int, N>;

template <int DT>
__device__ __forceinline__ float dot2_ones(uint32_t pk, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  if constexpr (DT == kF16)
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, pk),
                                  __builtin_bit_cast(h2, kOnePair<DT>), acc, false);
  else
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, pk),
                                           __builtin_bit_cast(b2, kOnePair<DT>), acc, false);
}

// 16-byte LDS load / 4- and 8-byte LDS stores at a 32-bit LDS byte address.
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) uint32_t lds_u32;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
__device__ __forceinline__ u32x4 lds_load16(uint32_t a) { return *(lds_u32x4 *)(uintptr_t)a; }
__device__ __forceinline__ void lds_store4(uint32_t a, uint32_t v) { *(lds_u32 *)(uintptr_t)a = v; }
__device__ __forceinline__ void lds_store8(uint32_t a, u32x2 v) { *(lds_u32x2 *)(uintptr_t)a = v; }
// Hide v's value from constant folding, so that base + constant address
// expressions keep the constant in the instruction's 16-bit offset field.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}
// The same, but never merged with another use: each call yields a value the
// compiler cannot share, so expressions built on it are recomputed where
// they are used instead of being kept live in registers.
__device__ __forceinline__ uint32_t fresh(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// LDS of one CTA: K ring [4][64 keys][256 B] (XOR-swizzled chunks), V^T ring
// [2][128 d][144 B].
constexpr int kPPSmem = kKRingPP * kKBytes + 2 * kVtBytes;

// CTA `raw` of a grid of q_blocks * batch * q_heads CTAs of 512 threads.
// smem: kPPSmem bytes of 1024-byte-aligned LDS.  FIXED: the caller bounds
// |Q|, |K| so that every scaled score lies in [-fixed_max, fixed_max]; the
// running max is then the constant fixed_max and the softmax segment skips
// the row max and the rescale (the reference's qk_max_abs mode,
// wave_flash_attention.py:63-75, :108-113, :586-622).
template <int DT, bool FIXED = false>
__device__ __forceinline__ void fwd_pp_cta(const Params &p, int raw, uint8_t *smem) {
  constexpr int kRows = 32 * kPPWaves;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t grp = wave >> 2;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t half = lane >> 5;
  int bh, qb;
  block_coords(p, raw, bh, qb);
  const int b = bh / p.q_heads, hq = bh - b * p.q_heads;
  const int hkv = hq / (p.q_heads / p.kv_heads);
  const uint16_t *Qh = p.Q + ((size_t)bh * p.seq_q) * kD;
  const uint16_t *Kh = p.K + ((size_t)(b * p.kv_heads + hkv) * p.seq_k) * kD;
  const char *Vh =
      reinterpret_cast<const char *>(p.V + ((size_t)(b * p.kv_heads + hkv) * p.seq_k) * kD);
  uint16_t *Oh = p.O + ((size_t)bh * p.seq_q) * kD;

  const int q0 = qb * kRows;
  const int qw = q0 + wave * 32;
  const int my_q = qw + (lane & 31);

  u32x4 qf[8];
  {
    const bool ok = my_q < p.seq_q;
    const uint16_t *qrow = Qh + (size_t)(ok ? my_q : 0) * kD + 8 * half;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      qf[kk] = ok ? *reinterpret_cast<const u32x4 *>(qrow + 16 * kk)
                  : u32x4{0u, 0u, 0u, 0u};
  }

  int kend = p.seq_k;
  if (p.causal)
    kend = min(kend, q0 + kRows);
  const int ntiles = (kend + kBN - 1) / kBN;

  // K DMA: wave w fills rows 8w .. 8w+7 of a tile (2 x 1 KiB).  Rows past
  // seq_k re-read the last key (masked out of the softmax).  Tiles past the
  // last one are issued too (clamped, never read), so the DMA needs no
  // branch; the kernel drains them before it ends.
  uint32_t kgoff[2];
  int krow[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    krow[i] = (wave * 2 + i) * 4 + (lane >> 4);
    kgoff[i] = ((lane & 15) ^ (krow[i] & 15)) << 4;
  }
  const uint32_t lds0 = lds_addr(smem);
  auto issue_k = [&](int kt) {
    const uint32_t l = lds0 + (kt & (kKRingPP - 1)) * kKBytes + wave * 2048;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = min(kt * kBN + krow[i], p.seq_k - 1);
      dma16(l + i * 1024, Kh, (uint32_t)key * kKRowBytes + kgoff[i]);
    }
  };

  // V: group g transposes d rows 64g .. 64g+63.  Thread tg of the group
  // loads keys 2kp, 2kp+1 (kp = tg % 32) of d chunk dc = 8g + tg / 32.
  const int tg = threadIdx.x & 255;
  const int kp = tg & 31, dc = 8 * grp + (tg >> 5);
  u32x4 vr[2], vr1[2];
  auto load_v_to = [&](int kt, u32x4(&dst)[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t key = (uint32_t)min(kt * kBN + 2 * kp + i, p.seq_k - 1);
      dst[i] = *reinterpret_cast<const u32x4 *>(Vh + key * kKRowBytes + 16 * dc);
    }
  };
  auto load_v = [&](int kt) { load_v_to(kt, vr); };
  // V^T column of key 2kp: 16-key groups stored as [0-3, 8-11, 4-7, 12-15].
  const int k2 = 2 * kp, blk = (k2 >> 2) & 3;
  const int vpos = 16 * (k2 >> 4) + 4 * (((blk & 1) << 1) | (blk >> 1)) + (k2 & 3);
  constexpr uint32_t kVtOff = kKRingPP * kKBytes;
  // Per-lane LDS bases; buffer, fragment and row offsets (< 64 KiB) are
  // added as immediates.
  const uint32_t kr = lane & 31;
  const uint32_t vt_store = opaque(lds0 + kVtOff + (uint32_t)(8 * dc) * kVtPitch + 2 * vpos);
  const uint32_t vt_read = opaque(lds0 + kVtOff + kr * kVtPitch + 16 * half);
  uint32_t kread[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    kread[kk] = opaque(lds0 + kr * kKRowBytes + (((2 * kk + half) ^ (kr & 15)) << 4));
  // V^T(t+1+grp) is stored in SM(t+1): buffer ((t+1) & 1) ^ grp.
  const uint32_t vst_par[2] = {opaque(vt_store + grp * kVtBytes),
                               opaque(vt_store + (grp ^ 1) * kVtBytes)};

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = f32x16{};
  float lsum = 0.f;
  float m = FIXED ? p.fixed_max : -__builtin_inff();
  const float c = p.scale_log2;
  // pin(x): x must be computed before this point (keeps each segment's work
  // on its side of the barrier that follows).
  auto pin = [](auto x) { asm volatile("" ::"v"(x)); };

  auto kfrag = [&](uint32_t kb, int i) {  // i = 2*kk + j: key row 32j + kr
    return lds_load16(kread[i >> 1] + kb * kKBytes + (i & 1) * 32 * kKRowBytes);
  };
  auto vfrag = [&](uint32_t vb, int i) {  // i = 4*(2*j + sl) + dt
    const int g = i >> 2, dt = i & 3;
    return lds_load16(vt_read + vb * kVtBytes + dt * 32 * kVtPitch + 32 * g);
  };
  u32x4 pf[2][2];

  // G(t): S(t+1) (when NEXT) from K buffer KB and O += V^T(t) P(t) from
  // V^T buffer VB as one explicit pipeline: the LDS fragment of MFMA
  // i + kPF is read in step i.  MFMA order (NEXT): S0 PV0 S1 PV1 ...
  // S(15-kTail) PV(15-kTail), then S(16-kTail) .. S15, then the kTail PV
  // MFMAs PV(16-kTail) .. PV15, which are issued at the start of the next
  // SM (pv_tail) with their fragments already in registers.
  constexpr int kPF = WAVE_FA_PF, kTail = WAVE_FA_TAIL;
  static_assert(kTail >= 0 && kTail <= 16 && kPF >= 1, "G pipeline shape");
  u32x4 tailf[kTail > 0 ? kTail : 1];
  auto seg_g = [&](auto next_tag, auto kb_tag, auto vb_tag, f32x16 (&sn)[2]) {
    constexpr bool NEXT = decltype(next_tag)::value;
    constexpr uint32_t KB = decltype(kb_tag)::value;
    constexpr uint32_t VB = decltype(vb_tag)::value;
    constexpr int NM = NEXT ? 32 : 16;           // MFMAs incl. the deferred tail
    constexpr int NI = NM - (NEXT ? kTail : 0);  // issued here
    constexpr int NP = 16 - kTail;               // S/PV pairs at the front
    // Position i -> (is S, step index).
    auto is_s = [&](int i) { return NEXT && (i < 2 * NP ? !(i & 1) : i < 2 * NP + kTail); };
    auto step = [&](int i) {
      if (!NEXT)
        return i;
      return i < 2 * NP ? i >> 1 : i < 2 * NP + kTail ? i - NP : i - NP - kTail;
    };
    auto frag = [&](int i) { return is_s(i) ? kfrag(KB, step(i)) : vfrag(VB, step(i)); };
    u32x4 f[NM];
#pragma unroll
    for (int i = 0; i < kPF && i < NM; ++i)
      f[i] = frag(i);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      if (i + kPF < NM)
        f[i + kPF] = frag(i + kPF);
      const int si = step(i);
      if (is_s(i)) {
        sn[si & 1] = mfma32x32x16<DT>(f[i], qf[si >> 1], si < 2 ? f32x16{} : sn[si & 1]);
      } else {
        const int g = si >> 2, dt = si & 3;
        o[dt] = mfma32x32x16<DT>(f[i], pf[g >> 1][g & 1], o[dt]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // Tail fragments the pipeline has not read yet (kTail > kPF).
#pragma unroll
    for (int i = NI + kPF; i < NM; ++i)
      f[i] = frag(i);
    if constexpr (NEXT) {
#pragma unroll
      for (int k = 0; k < kTail; ++k)
        tailf[k] = f[NI + k];
    }
  };
  // The deferred PV MFMAs PV(16-kTail) .. PV15 of the previous G.
  auto pv_tail = [&]() {
#pragma unroll
    for (int k = 0; k < kTail; ++k) {
      const int v = 16 - kTail + k;
      const int g = v >> 2, dt = v & 3;
      o[dt] = mfma32x32x16<DT>(tailf[k], pf[g >> 1][g & 1], o[dt]);
    }
  };

  auto mask = [&](f32x16 (&sc)[2], int t) {
    const int k0 = t * kBN;
    const bool edge = (k0 + kBN > p.seq_k) || (p.causal && k0 + kBN - 1 > qw);
    if (edge) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 32 * j + 8 * (r >> 2) + 4 * half + (r & 3);
          if (key >= p.seq_k || (p.causal && key > my_q))
            sc[j][r] = -__builtin_inff();
        }
    }
  };
  // Lazy rescale: raise the running max only when it grows by > 8 (log2).
  auto update_max = [&](float mx) {
    const bool need = mx > m + kRescaleThreshold;
    if (__builtin_amdgcn_ballot_w64(need)) {
      const float mn = fmaxf(m, mx);
      const float alpha = (m == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(m - mn);
      m = mn;
      lsum *= alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[i] *= alpha;
    }
  };
  // Softmax of tile t (scores in sc): max, rescale, P(t) -> pf, row sums.
  auto softmax = [&](f32x16 (&sc)[2], int t) {
    mask(sc, t);
    if constexpr (!FIXED) {
      // Four independent max chains (a short dependency path), then the
      // other half of the row from lane l ^ 32.
      float mq[4] = {sc[0][0], sc[0][1], sc[1][0], sc[1][1]};
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 2; r < 16; ++r)
          mq[2 * j + (r & 1)] = fmaxf(mq[2 * j + (r & 1)], sc[j][r]);
      float lo, hi;
      half_pair(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3])), lo, hi);
      update_max(fmaxf(lo, hi) * c);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][8 * sl + 2 * e], c, -m));
          const float p1 =
              __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][8 * sl + 2 * e + 1], c, -m));
          pf[j][sl][e] = pack2<DT>(p0, p1);
        }
    // Row sums in two independent v_dot2 chains.
    float l1 = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lsum = dot2_ones<DT>(pf[j][0][e], lsum);
        l1 = dot2_ones<DT>(pf[j][1][e], l1);
      }
    lsum += l1;
    pin(lsum);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int sl = 0; sl < 2; ++sl)
        pin(pf[j][sl]);
  };
  // This group's half of a V^T tile (from vr) at store base vst.
  auto store_vt_from = [&](uint32_t vst, const u32x4(&src)[2]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lds_store4(vst + 2 * e * kVtPitch, __builtin_amdgcn_perm(src[1][e], src[0][e], 0x05040100u));
      lds_store4(vst + (2 * e + 1) * kVtPitch,
                 __builtin_amdgcn_perm(src[1][e], src[0][e], 0x07060302u));
    }
  };
  auto store_vt = [&](uint32_t vst) { store_vt_from(vst, vr); };

  // One iteration t < ntiles - 1: G(t), barrier, SM(t+1), barrier.
  // PH = t % 4 fixes the buffer offsets.
  auto iter = [&](auto ph_tag, int t, f32x16 (&sn)[2]) {
    constexpr int PH = decltype(ph_tag)::value;
    load_v(t + 1 + (int)grp);
    seg_g(std::true_type{}, std::integral_constant<uint32_t, (PH + 1) % kKRingPP>{},
          std::integral_constant<uint32_t, PH & 1>{}, sn);
    // G only reads LDS, and the next writer of what it read (a V^T or K
    // buffer) comes after the barrier that ends the following SM, which
    // waits for LDS.  So this barrier does not wait for G's last fragment
    // reads (the deferred tail's), which complete under the next SM.
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    pv_tail();
    softmax(sn, t + 1);
    store_vt(vst_par[(PH + 1) & 1]);  // first use of vr: waits for the loads
    issue_k(t + 4);                   // after the V wait (see the K ring)
    lds_barrier();
  };

  // ---- prologue (all waves): K(0..3), V^T(0), B's half of V^T(1), S(0)
  // and its softmax --------------------------------------------------------
  f32x16 sa[2];
  // Group B's V(1) is loaded with V(0), so the prologue waits on memory once.
  issue_k(0);
  issue_k(1);
  issue_k(2);
  load_v(0);
  if (grp == 1)
    load_v_to(1, vr1);
  vm_wait_barrier();
  store_vt(vt_store);
  if (grp == 1)
    store_vt_from(vt_store + kVtBytes, vr1);
#pragma unroll
  for (int i = 0; i < 16; ++i)
    sa[i & 1] = mfma32x32x16<DT>(kfrag(0, i), qf[i >> 1], i < 2 ? f32x16{} : sa[i & 1]);
  issue_k(3);
  softmax(sa, 0);
  lds_barrier();
  if (grp == 1)  // group B's idle segment 0
    lds_barrier();

  // ---- main loop, unrolled by 4 (K ring); leaves with t = ntiles - 1 -----
  int t = 0;
  for (;; t += 4) {
    if (t + 1 >= ntiles)
      break;
    iter(I_<0>{}, t, sa);
    if (t + 2 >= ntiles) {
      t += 1;
      break;
    }
    iter(I_<1>{}, t + 1, sa);
    if (t + 3 >= ntiles) {
      t += 2;
      break;
    }
    iter(I_<2>{}, t + 2, sa);
    if (t + 4 >= ntiles) {
      t += 3;
      break;
    }
    iter(I_<3>{}, t + 3, sa);
  }
  // Last tile: G = PV(t) only (V^T buffer t & 1).
  if (t & 1)
    seg_g(std::false_type{}, std::integral_constant<uint32_t, 0>{},
          std::integral_constant<uint32_t, 1>{}, sa);
  else
    seg_g(std::false_type{}, std::integral_constant<uint32_t, 0>{},
          std::integral_constant<uint32_t, 0>{}, sa);
  if (grp == 0)
    lds_barrier();
  // K DMA issued for tiles past the end may still be in flight: let it land
  // before the workgroup's LDS can be handed to another workgroup.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Normalise and store O[my_q][d], d = 32*dt + 8*(r/4) + 4*half + r%4.
  // Lanes l and l^32 hold the sums of complementary key halves.
  float s_lo, s_hi;
  half_pair(lsum, s_lo, s_hi);
  const float total = s_lo + s_hi;
  const float inv = total > 0.f ? 1.0f / total : 0.f;
  // sum_k 2^(c*s_k) = total * 2^m, so ln sum_k e^(scale*s_k) = (m + log2 total) ln 2.
  if (p.lse != nullptr && half == 0 && my_q < p.seq_q)
    p.lse[(size_t)bh * p.seq_q + my_q] = (m + __builtin_log2f(total)) * kLn2;
  // The wave's 32 rows go through LDS so that each store writes 4 whole
  // 256-byte rows (1 KiB) instead of 8-byte pieces of 32 rows.  Staging
  // area: this wave's own K DMA rows of the four ring tiles (2 KiB each,
  // row r in tile r / 8): after its vmcnt(0) nothing else writes them, and
  // no wave reads K after its last G.  16-byte chunk c of row r sits at
  // c ^ (r & 15).
  {
    const uint32_t r = lane & 31;
    const uint32_t wb = lds0 + wave * 2048;
    const uint32_t wrow = wb + (r >> 3) * kKBytes + (r & 7) * 256 + half * 8;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const u32x2 w = {pack2<DT>(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv),
                         pack2<DT>(o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv)};
        const uint32_t c = (uint32_t)(4 * dt + g);
        lds_store8(wrow + ((c ^ (r & 15)) << 4), w);
      }
    const uint32_t c = lane & 15;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const uint32_t rr = it * 4 + (lane >> 4);
      const u32x4 v = lds_load16(wb + (rr >> 3) * kKBytes + (rr & 7) * 256 + ((c ^ (rr & 15)) << 4));
      if (qw + (int)rr < p.seq_q)
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(Oh + (size_t)(qw + rr) * kD + 8 * c));
    }
  }
}

template <int DT, bool FIXED>
__global__ __launch_bounds__(512, 1) void fwd_pp_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kPPSmem];
  fwd_pp_cta<DT, FIXED>(p, blockIdx.x, smem);
}

} // namespace attention
} // namespace wave
