// attention_fwd3.hpp -- flash-attention forward for gfx950 with three
// rotating wave groups (12 waves, 384 query rows per CTA).
//
// Same math and conventions as fwd_pp_cta (attention_kernels.hpp): per wave
// 32 query rows, S^T = K . Q^T with v_mfma_f32_32x32x16 (Q fragments held in
// VGPRs), P^T straight from the S^T accumulators, V^T in LDS with each
// 16-key group permuted as [0-3, 8-11, 4-7, 12-15], lazy rescale at 8
// (log2 units), v_dot2 row sums of the packed P, optional fixed max, causal
// mask and grouped-query heads (the reference kernel's math,
// python/mlir/dialects/wave_flash_attention.py:586-728, :814, :1034-1095).
//
// Why three groups.  In the two-group kernel one SIMD pairs one wave's MFMA
// segment G (32 MFMAs of 32 cycles) with one wave's softmax segment SM, and
// SM -- about 117 VALU and 32 v_exp_f32 per wave and key tile -- runs at a
// single wave's issue rate (an FMA every ~5.4 cycles; the SIMD retires about
// two waves' worth), so SM (~1550 cycles) sets the pace and the MFMA pipe
// idles a third of the time.  Here each SIMD holds three waves, one of each
// group, and the workgroup barriers keep the groups one segment apart:
//
//   segment   3t        3t+1      3t+2      3t+3
//   group 0   G(t)      SM1(t+1)  SM2(t+1)  G(t+1)
//   group 1   SM2(t)    G(t)      SM1(t+1)  SM2(t+1)
//   group 2   SM1(t)    SM2(t)    G(t)      SM1(t+1)
//
// so every SIMD runs one wave's MFMA stream next to two waves' softmax
// halves.  G(t): O^T += V^T(t) P(t)^T (16 MFMAs) and then S(t+1) = K(t+1)
// Q^T (16 MFMAs); PV first, so P(t) is dead before S(t+1) is live (the
// per-wave live set has to fit 168 registers: 512 per SIMD lane / 3).
// SM1(t+1): mask, row max, lazy rescale, exp2 and pack of the first 32 keys.
// SM2(t+1): exp2 and pack of the other 32 keys, row sums, and (groups 0 and
// 1) this group's half of a V^T tile.
//
// Buffers (the loop is unrolled by 4, so every buffer index is a
// compile-time constant):
//  * K ring of 4 tiles, K(j) in buffer j % 4, read by the three G(j-1) in
//    segments 3j-3 .. 3j-1.  Group 2 alone issues the K DMA in steady state:
//    K(j) in SM1(j-3) (segment 3j-9; buffer free since K(j-4)'s last read in
//    3j-13), each wave 4 x 1 KiB, and waits for it at the end of its G(j-2)
//    (segment 3j-4, vmcnt(4): K(j+1)'s four issues may still fly).  The
//    prologue issues K(0..3) from all waves and waits for all of it.
//  * V^T ring of 2 tiles, V^T(j) in buffer j % 2, read by the three G(j) in
//    segments 3j .. 3j+2.  Group g in {0, 1} loads the V rows of its half
//    (d rows 64g .. 64g+63) of tile t+1+g at the end of its G(t) and stores
//    them transposed in its SM2(t+1): group 0 in segment 3t+2 = 3j-1,
//    group 1 in 3t+3 = 3j-3, both after V^T(j-2)'s last read (3j-4) and
//    before the first read of V^T(j) (3j).  The prologue stores V^T(0) and
//    group 1's half of V^T(1).
// Measured (MI355X, same box and process, against fwd_pp_kernel): B2 H64
// S8192 bf16 1175 against 1197 TFLOP/s, B4 H32 S4096 f16 1030 against 1100
// (that grid is 5.5 rounds of 384-row CTAs on 256 CUs).  Per-segment stamps
// show G MFMA-bound and the groups' softmax halves no shorter than the
// two-group kernel's segments once three waves share a SIMD, so the library
// keeps the 8-wave kernel as its default and offers this one as waves = 12.
//
// Every barrier waits for the wave's LDS operations (lgkmcnt(0)): a group's
// G reads are complete when its last MFMA issues, and its writes (V^T) have
// to be visible one segment later.  Barriers per wave: 2 (prologue) + 3 *
// ntiles + 1 (epilogue): group g joins g barriers before its first G and
// 2 - g after its last one.
#pragma once

#include "attention_kernels.hpp"

namespace wave {
namespace attention {

constexpr int kR3Waves = 12;
constexpr int kR3Rows = 32 * kR3Waves;  // 384 query rows per CTA
constexpr int kKRing3 = 4;
constexpr int kR3VtOff = kKRing3 * kKBytes;
// LDS of one CTA: K ring [4][16 KiB] (fragment-major, see fwd3_cta), V^T
// ring [2][128 d][144 B]; the epilogue reuses it to stage O (8 KiB a wave).
constexpr int kR3Smem = kR3VtOff + 2 * kVtBytes;
static_assert(kR3Waves * 32 * kKRowBytes <= kR3Smem, "O staging fits the rings");

// CTA `raw` of a grid of q_blocks * batch * q_heads CTAs of 768 threads
// (q_blocks = ceil(seq_q / 384)).  smem: kR3Smem bytes of 1024-byte-aligned
// LDS.  FIXED as in fwd_pp_cta.
template <int DT, bool FIXED = false>
__device__ __forceinline__ void fwd3_cta(const Params &p, int raw, uint8_t *smem) {
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t grp = uniform(wave >> 2);
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

  const int q0 = qb * kR3Rows;
  const int qw = q0 + (int)wave * 32;
  const int my_q = qw + (int)(lane & 31);

  u32x4 qf[8];
  {
    const bool ok = my_q < p.seq_q;
    const uint16_t *qrow = Qh + (size_t)(ok ? my_q : 0) * kD + 8 * half;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      qf[kk] = ok ? *reinterpret_cast<const u32x4 *>(qrow + 16 * kk) : u32x4{0u, 0u, 0u, 0u};
  }

  int kend = p.seq_k;
  if (p.causal)
    kend = min(kend, q0 + kR3Rows);
  const int ntiles = (kend + kBN - 1) / kBN;

  // K tiles sit in LDS fragment-major: window w = 2kk + j (1 KiB) of a tile
  // holds, at slot 32h + r, the 16-byte chunk 2kk + h of key row 32j + r
  // (kk = Q chunk pair 0..7, j = 32-key block, h = lane half, r = 0..31).
  // The S^T fragment of lane (r, h) for (kk, j) is then one base register
  // plus an immediate offset (2048 kk + 1024 j), and the 64 lanes of a read
  // cover one contiguous 1 KiB (no bank conflict).  One DMA fills one
  // window: lane l fetches chunk 2kk + l/32 of key row 32j + l%32.  Rows
  // past seq_k re-read the last key (masked out of the softmax); tiles past
  // the last one are issued too (clamped, never read), so the DMA needs no
  // branch, and the kernel drains them before it ends.
  const uint32_t lds0 = lds_addr(smem);
  auto issue_k_window = [&](int kt, uint32_t w, uint32_t ln) {
    const uint32_t l = lds0 + (uint32_t)(kt & (kKRing3 - 1)) * kKBytes + w * 1024u;
    const uint32_t key = (uint32_t)min(kt * kBN + (int)(32u * (w & 1u) + (ln & 31u)),
                                       p.seq_k - 1);
    dma16(l, Kh, key * kKRowBytes + ((w & ~1u) + (ln >> 5)) * 16u);
  };
  // Steady state: group 2's wave u issues windows 4u .. 4u+3.  The lane id
  // is rebuilt here, so no per-lane term of the DMA stays live between
  // tiles.
  auto issue_k_g2 = [&](int kt) {
    const uint32_t u = wave - 8u;
    const uint32_t ln = fresh(threadIdx.x) & 63u;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i)
      issue_k_window(kt, 4u * u + i, ln);
  };

  // V: group g < 2 transposes d rows 64g .. 64g+63.  Thread tg of the group
  // loads keys 2kp, 2kp+1 (kp = tg % 32) of d chunk dc = 8g + tg / 32.  The
  // per-lane terms of the load address are rebuilt at each load from a fresh
  // thread id (a 32-bit offset from the uniform V base), so none of them
  // stays live through G.
  const int tg = (int)(threadIdx.x & 255);
  const int kp = tg & 31, dc = 8 * (int)(grp & 1u) + (tg >> 5);
  u32x4 vr[2];
  auto load_v_to = [&](int kt, u32x4(&dst)[2]) {
    const uint32_t tid = fresh(threadIdx.x);
    const int kp_ = (int)(tid & 31u);
    const uint32_t col = 16u * (8u * (grp & 1u) + ((tid & 255u) >> 5));
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t key = (uint32_t)min(kt * kBN + 2 * kp_ + i, p.seq_k - 1);
      dst[i] = *reinterpret_cast<const u32x4 *>(Vh + (key * kKRowBytes + col));
    }
  };
  // V^T column of key 2kp: 16-key groups stored as [0-3, 8-11, 4-7, 12-15].
  const int k2 = 2 * kp, blk = (k2 >> 2) & 3;
  const int vpos = 16 * (k2 >> 4) + 4 * (((blk & 1) << 1) | (blk >> 1)) + (k2 & 3);
  const uint32_t kr = lane & 31;
  const uint32_t vt_store = opaque(lds0 + kR3VtOff + (uint32_t)(8 * dc) * kVtPitch + 2 * vpos);
  const uint32_t vt_read = opaque(lds0 + kR3VtOff + kr * kVtPitch + 16 * half);
  // This lane's slot in a K window (see the K layout above).
  const uint32_t kbase = opaque(lds0 + 16u * (32u * half + kr));

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = f32x16{};
  float lsum = 0.f;
  float m = FIXED ? p.fixed_max : -__builtin_inff();
  const float c = p.scale_log2;
  auto pin = [](auto x) { asm volatile("" ::"v"(x)); };

  auto kfrag = [&](uint32_t kb, int i) {  // i = 2*kk + j: key row 32j + kr, window i
    return lds_load16(kbase + kb * kKBytes + (uint32_t)i * 1024u);
  };
  // V^T fragment i = 4*(2*j + sl) + dt of the buffer at vt (vt_read plus the
  // buffer offset).
  auto vfrag = [&](uint32_t vt, int i) {
    const int g = i >> 2, dt = i & 3;
    return lds_load16(vt + dt * 32 * kVtPitch + 32 * g);
  };
  u32x4 pf[2][2];

  // G(t): O += V^T(t) P(t) from V^T buffer VB (16 MFMAs), then (NEXT)
  // S(t+1) from K buffer KB (16 MFMAs), as one explicit pipeline: the LDS
  // fragment of MFMA i + kPF is read in step i.
#ifndef WAVE_FA3_PF
#define WAVE_FA3_PF 4  // LDS fragment prefetch depth (MFMAs) in G
#endif
  constexpr int kPF = WAVE_FA3_PF;
  // vt: the V^T buffer's read base (vt_read + buffer * kVtBytes).
  auto seg_g = [&](auto next_tag, auto kb_tag, uint32_t vt, f32x16(&sn)[2]) {
    constexpr bool NEXT = decltype(next_tag)::value;
    constexpr uint32_t KB = decltype(kb_tag)::value;
    constexpr int NM = NEXT ? 32 : 16;
    auto frag = [&](int i) { return i < 16 ? vfrag(vt, i) : kfrag(KB, i - 16); };
    u32x4 f[NM];
#pragma unroll
    for (int i = 0; i < kPF; ++i)
      f[i] = frag(i);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      if (i + kPF < NM)
        f[i + kPF] = frag(i + kPF);
      if (i < 16) {
        const int g = i >> 2, dt = i & 3;
        o[dt] = mfma32x32x16<DT>(f[i], pf[g >> 1][g & 1], o[dt]);
      } else {
        const int si = i - 16;
        sn[si & 1] = mfma32x32x16<DT>(f[i], qf[si >> 1], si < 2 ? f32x16{} : sn[si & 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Edge tiles only; the lane terms and -inf are rebuilt here (fresh), so
  // they hold no registers through the rest of the loop.
  auto mask = [&](f32x16(&sc)[2], int t) {
    const int k0 = t * kBN;
    const bool edge = (k0 + kBN > p.seq_k) || (p.causal && k0 + kBN - 1 > qw);
    if (edge) {
      const uint32_t ln = fresh(threadIdx.x) & 63u;
      const int q = qw + (int)(ln & 31u);
      const int kb = k0 + 4 * (int)(ln >> 5);
      const float ninf = __builtin_bit_cast(float, fresh(0xff800000u));
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb + 32 * j + 8 * (r >> 2) + (r & 3);
          if (key >= p.seq_k || (p.causal && key > q))
            sc[j][r] = ninf;
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
  // P of the 32 keys of block j of tile t (scores sc[j]) -> pf[j].
  auto exp_block = [&](f32x16(&sc)[2], int j) {
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][8 * sl + 2 * e], c, -m));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][8 * sl + 2 * e + 1], c, -m));
        pf[j][sl][e] = pack2<DT>(p0, p1);
      }
  };
  // SM1(t): mask, row max and rescale, P of keys 0-31.
  auto softmax1 = [&](f32x16(&sc)[2], int t) {
    mask(sc, t);
    if constexpr (!FIXED) {
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
    exp_block(sc, 0);
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
      pin(pf[0][sl]);
    pin(m);
  };
  // SM2(t): P of keys 32-63, row sums of P(t) in two v_dot2 chains.
  auto softmax2 = [&](f32x16(&sc)[2]) {
    exp_block(sc, 1);
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
    for (int sl = 0; sl < 2; ++sl)
      pin(pf[1][sl]);
  };
  // This group's half of a V^T tile (from src) at store base vst.
  auto store_vt_from = [&](uint32_t vst, const u32x4(&src)[2]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lds_store4(vst + 2 * e * kVtPitch, __builtin_amdgcn_perm(src[1][e], src[0][e], 0x05040100u));
      lds_store4(vst + (2 * e + 1) * kVtPitch,
                 __builtin_amdgcn_perm(src[1][e], src[0][e], 0x07060302u));
    }
  };
  auto barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };

  // One iteration t < ntiles - 1: G(t), SM1(t+1), SM2(t+1), a barrier after
  // each.  PH = t % 4 fixes the buffer offsets.
  auto iter = [&](auto ph_tag, int t, f32x16(&sn)[2]) {
    constexpr int PH = decltype(ph_tag)::value;
    seg_g(std::true_type{}, std::integral_constant<uint32_t, (PH + 1) % kKRing3>{},
          vt_read + (uint32_t)(PH & 1) * kVtBytes, sn);
    if (grp < 2u)
      load_v_to(t + 1 + (int)grp, vr);
    else
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");  // K(t+2) has landed
    barrier();
    softmax1(sn, t + 1);
    if (grp == 2u)
      issue_k_g2(t + 4);
    barrier();
    softmax2(sn);
    // Group g < 2 stores V^T(t+1+g): buffer ((t+1) & 1) ^ g.
    if (grp < 2u)
      store_vt_from(vt_store + (((grp & 1u) ^ (uint32_t)((PH + 1) & 1)) * kVtBytes), vr);
    barrier();
  };

  // ---- prologue (all waves): K(0..3), V^T(0), group 1's half of V^T(1),
  // S(0) and its whole softmax -----------------------------------------------
  {
    // 64 K windows of tiles 0..3, window wave + 12 i for each wave.
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const uint32_t cc = wave + 12u * (uint32_t)i;
      if (cc < 64u)
        issue_k_window((int)(cc >> 4), cc & 15u, lane);
    }
  }
  u32x4 vr1[2];
  if (grp < 2u)
    load_v_to(0, vr);
  if (grp == 1u)
    load_v_to(1, vr1);
  vm_wait_barrier();
  if (grp < 2u)
    store_vt_from(vt_store + (grp & 1u) * 0u, vr);  // V^T(0): buffer 0
  if (grp == 1u)
    store_vt_from(vt_store + kVtBytes, vr1);        // V^T(1): buffer 1
  f32x16 sa[2];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    sa[i & 1] = mfma32x32x16<DT>(kfrag(0, i), qf[i >> 1], i < 2 ? f32x16{} : sa[i & 1]);
  softmax1(sa, 0);
  softmax2(sa);
  barrier();
  // Group g idles g segments so that the groups run one segment apart.
  if (grp >= 1u)
    barrier();
  if (grp == 2u)
    barrier();

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
  // Last tile: G = PV(t) only, from V^T buffer t & 1 (a runtime base: one
  // copy of the segment).
  seg_g(std::false_type{}, std::integral_constant<uint32_t, 0>{},
        vt_read + (uint32_t)(t & 1) * kVtBytes, sa);
  barrier();
  // Group g joins 2 - g more segments (the other groups' last G).
  if (grp == 0u)
    barrier();
  if (grp <= 1u)
    barrier();
  // Every wave's K DMA (tiles past the end included) and V loads have
  // landed and every LDS read is done: the rings are free for staging O.
  vm_wait_barrier();

  // Normalise and store O[my_q][d], d = 32*dt + 8*(r/4) + 4*half + r%4.
  // Lanes l and l^32 hold the sums of complementary key halves.
  float s_lo, s_hi;
  half_pair(lsum, s_lo, s_hi);
  const float total = s_lo + s_hi;
  const float inv = total > 0.f ? 1.0f / total : 0.f;
  // sum_k 2^(c*s_k) = total * 2^m, so ln sum_k e^(scale*s_k) = (m + log2 total) ln 2.
  if (p.lse != nullptr && half == 0 && my_q < p.seq_q)
    p.lse[(size_t)bh * p.seq_q + my_q] = (m + __builtin_log2f(total)) * kLn2;
  // The wave's 32 rows are staged in its own 8 KiB of the rings (row r at
  // r * 256, 16-byte chunk c at c ^ (r & 15)), then stored as whole
  // 256-byte rows, 4 rows (1 KiB) a store instruction, non-temporally.
  {
    const uint32_t r = lane & 31;
    const uint32_t wb = lds0 + wave * 8192u;
    const uint32_t wrow = wb + r * 256u + half * 8u;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const u32x2 w = {pack2<DT>(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv),
                         pack2<DT>(o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv)};
        const uint32_t ch = (uint32_t)(4 * dt + g);
        lds_store8(wrow + ((ch ^ (r & 15u)) << 4), w);
      }
    const uint32_t ch = lane & 15u;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const uint32_t rr = (uint32_t)it * 4u + (lane >> 4);
      const u32x4 v = lds_load16(wb + rr * 256u + ((ch ^ (rr & 15u)) << 4));
      if (qw + (int)rr < p.seq_q)
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(Oh + (size_t)(qw + rr) * kD + 8 * ch));
    }
  }
}

template <int DT, bool FIXED>
__global__ __launch_bounds__(64 * kR3Waves, 1) void fwd3_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kR3Smem];
  fwd3_cta<DT, FIXED>(p, blockIdx.x, smem);
}

} // namespace attention
} // namespace wave
