// attention_fwd8.hpp -- block-scaled FP8 flash-attention forward for gfx950,
// head_dim 128: the "block-scaled FP8 attention contract" the reference
// names as its next FA step (docs/PerfReferences/WaveGfx950FlashAttention.md:
// 94-99, "gfx950 FP8 MFMA needs an explicit scaled-input contract").
//
// Inputs are OCP MX-FP8: e4m3 elements with one e8m0 scale (2^(e - 127)) per
// 32 elements along the dimension each product contracts:
//   Q [B][Hq][S_q][128] e4m3, Q_scale [B][Hq][S_q][4]    (blocks of 32 d)
//   K [B][Hkv][S_k][128] e4m3, K_scale [B][Hkv][S_k][4]  (blocks of 32 d)
//   V [B][Hkv][S_k][128] e4m3, V_scale [B][Hkv][ceil(S_k/32)][128]
//                                                    (blocks of 32 keys)
// O [B][Hq][S_q][128] f16 or bf16 = softmax(scale * Q K^T) V of the decoded
// values, with the probabilities P rounded to e4m3 before the PV product.
//
// Same CTA shape and ping-pong schedule as fwd_pp_cta (attention_kernels.hpp):
// 8 waves x 32 query rows, two groups of four alternating a matrix-only
// segment G and a vector-only segment SM.  Both products run on
// v_mfma_scale_f32_32x32x64_f8f6f4 with the MX scales as its per-lane scale
// operands, so a 64-key tile is 4 + 4 MFMAs a wave (against 16 + 16 for 16-bit
// inputs).  With e4m3 operands that MFMA takes its 64-deep K dimension as two
// 32-element scale blocks: block b is bytes 16b .. 16b+15 of both lane halves
// of a row / column, scaled by the scale operand of lane half b (measured on
// gfx950 by a one-hot probe).  So:
//  * S^T(j) = K(j) . Q^T, j = 32-key block, d slice s = 0, 1: lane half h
//    supplies d 64s + 16h .. +15 (block 2s) and 64s + 32 + 16h .. +15 (block
//    2s + 1) of K row 32j + l%32 (A) and of Q row l%32 (B, held in VGPRs),
//    with the scales of d blocks 2s + h.
//  * O^T(dt) += V^T(dt) . P^T: the S^T accumulators give lane half h keys
//    32j + 8i + 4h + 0..3 (i = 0..3) of query l%32, i.e. 16 keys of each
//    32-key block j; packed to e4m3 (4 a dword, block j in bytes 16j ..) they
//    are the B operand as they stand, and A = the same keys of V column
//    32dt + l%32 at the same bytes (key 32j + 8i + 4h + e at byte
//    16j + 4i + e), scaled by V_scale of (key block h, d).
//  * P = exp2(c s - m + 4) is at most 2^8 (the running max is raised when a
//    tile's max exceeds it by more than 4), so it fits e4m3 (max 448) and
//    values down to 2^-13 of the running max stay representable; the PV
//    MFMA's B scale is the constant 2^-4.  Row sums are one more MFMA a
//    tile (a ones operand against the same e4m3 P).
//  * K and V both arrive by LDS DMA in 4-tile rings, 64 rows x 128 B a tile.
//    K: 16-byte chunk c of row r at c ^ ((r >> 1) & 7) (rows r and r + 1
//    share a 256-byte bank line, so the 16 rows one ds_read_b128 phase reads
//    hit 16 distinct chunk slots).  V stays row-major and the PV operand is
//    read with ds_read_b64_tr_b8 (gfx950's transposing LDS read: in each
//    16-lane group, source lane 2e + p addresses 8 bytes of a row and lane
//    i receives byte i % 8 of source lanes 2e + i / 8, e = 0..7 -- measured
//    by a probe on the box), so no transpose runs in the softmax segment.
#pragma once

#include "attention_kernels.hpp"

namespace wave {
namespace attention {

constexpr int k8Waves = 8;
constexpr int k8Rows = 32 * k8Waves;             // query rows a CTA
constexpr int k8KRowBytes = kD;                  // 128 B per K / V row
constexpr int k8KBytes = kBN * k8KRowBytes;      // 8 KiB per K tile
constexpr int k8KRing = 4;
constexpr int k8VtOff = k8KRing * k8KBytes;      // V ring: 4 tiles from 32 KiB
constexpr int k8StageOff = 2 * k8KRing * k8KBytes;  // 64 KiB
constexpr int k8StageBytes = 32 * kD * 2;        // one wave's 32 output rows
constexpr int k8Smem = k8StageOff + k8Waves * k8StageBytes;  // 128 KiB
constexpr float k8Threshold = 4.0f;              // lazy rescale (log2 units)
constexpr float k8PShift = 4.0f;                 // P = 2^4 * probability
constexpr int k8PScale = 127 - 4;                // e8m0 of 2^-4

struct Fp8Params {
  const uint8_t *Q, *K, *V;
  const uint8_t *Qs, *Ks, *Vs;  // e8m0 scales
  uint16_t *O;
  int batch, q_heads, kv_heads, seq_q, seq_k;
  int q_blocks;
  int causal;
  float scale_log2;
  float *lse;
};

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x2v __attribute__((ext_vector_type(2)));

// D[32x32] += (A * 2^(sa-127))[32x64] (B * 2^(sb-127))[64x32], e4m3 A and B;
// lane l supplies 32 bytes of row / column l%32 at K offset 32*(l/32) and in
// byte 0 of sa / sb the e8m0 scale of those 32 values.
__device__ __forceinline__ f32x16 mfma_fp8(i32x8 a, i32x8 b, f32x16 c, uint32_t sa, uint32_t sb) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, (int)sa, 0, (int)sb);
}

__device__ __forceinline__ i32x8 join8(u32x4 lo, u32x4 hi) {
  return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
               (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}


// Four floats -> four e4m3 bytes (RNE), first value in byte 0.
__device__ __forceinline__ uint32_t pack_fp8x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

template <int OUT_DT, bool CAUSAL>
__device__ __forceinline__ void fwd8_cta(const Fp8Params &p, int raw, uint8_t *smem) {
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t grp = wave >> 2;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t half = lane >> 5;
  const uint32_t kr = lane & 31;
  int bh, qb;
  {
    Params cp{};
    cp.q_blocks = p.q_blocks;
    cp.batch = p.batch;
    cp.q_heads = p.q_heads;
    cp.causal = CAUSAL;
    block_coords(cp, raw, bh, qb);
  }
  const int b = bh / p.q_heads, hq = bh - b * p.q_heads;
  const int hkv = hq / (p.q_heads / p.kv_heads);
  const size_t kvh = (size_t)(b * p.kv_heads + hkv);
  const uint8_t *Kh = p.K + kvh * p.seq_k * kD;
  const uint8_t *Vh = p.V + kvh * p.seq_k * kD;
  const int vsrows = (p.seq_k + 31) / 32;
  // Buffer resources over this head's K scales and V scales: 32-bit
  // offsets from an SGPR base, and reads past the end return 0 (keys past
  // seq_k are masked out of the softmax, so their scales only need to be
  // finite).
  const __amdgpu_buffer_rsrc_t ksrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(p.Ks + kvh * p.seq_k * 4), 0,
                                        p.seq_k * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t vsrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(p.Vs + kvh * vsrows * kD), 0,
                                        vsrows * kD, 0x00020000);
  uint16_t *Oh = p.O + ((size_t)bh * p.seq_q) * kD;

  const int q0 = qb * k8Rows;
  const int qw = q0 + wave * 32;
  const int my_q = qw + kr;

  // Q row my_q: d 64s + 16h .. +15 and 64s + 32 + 16h .. +15 (s = 0, 1) and
  // the scales of d blocks 2s + h.
  i32x8 qf[2];
  uint32_t qs[2];
  {
    const bool ok = my_q < p.seq_q;
    const uint8_t *qrow = p.Q + ((size_t)bh * p.seq_q + (ok ? my_q : 0)) * kD + 16 * half;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 lo = ok ? *reinterpret_cast<const u32x4 *>(qrow + 64 * s) : u32x4{0, 0, 0, 0};
      const u32x4 hi =
          ok ? *reinterpret_cast<const u32x4 *>(qrow + 64 * s + 32) : u32x4{0, 0, 0, 0};
      qf[s] = join8(lo, hi);
    }
    const uint32_t w =
        ok ? reinterpret_cast<const uint32_t *>(p.Qs)[(size_t)bh * p.seq_q + my_q] : 0x7F7F7F7Fu;
#pragma unroll
    for (int s = 0; s < 2; ++s)
      qs[s] = w >> (8 * (2 * s + half));
  }

  int kend = p.seq_k;
  if (CAUSAL)
    kend = min(kend, q0 + k8Rows);
  const int ntiles = (kend + kBN - 1) / kBN;

  // K DMA: wave w fills rows 8w .. 8w+7 of a tile (one 1 KiB issue).
  const int krow = wave * 8 + (lane >> 3);
  const uint32_t kgoff = ((lane & 7) ^ ((krow >> 1) & 7)) << 4;
  const uint32_t lds0 = lds_addr(smem);
  auto issue_k = [&](int kt) {
    const uint32_t l = lds0 + (kt & (k8KRing - 1)) * k8KBytes + wave * 1024;
    const int key = min(kt * kBN + krow, p.seq_k - 1);
    dma16(l, Kh, (uint32_t)key * k8KRowBytes + kgoff);
  };
  // K scales of tile kt for this lane's two key rows 32j + kr, shifted so
  // that byte 0 is d block 2s + h after a further shift by 16 s.
  // Every offset goes in the VGPR offset, which the buffer range check
  // covers (the SGPR offset is not checked).
  auto load_ks = [&](int kt, uint32_t (&dst)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      dst[j] = __builtin_amdgcn_raw_buffer_load_b32(
                   ksrs, (uint32_t)(kt * kBN + 32 * j + (int)kr) * 4, 0, 0) >>
               (8 * half);
  };
  // V scales of tile kt: key block 2kt + h, d = 32dt + kr.
  auto load_vs = [&](int kt, uint32_t (&dst)[4]) {
    const uint32_t off = (uint32_t)(2 * kt + (int)half) * kD + kr;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      dst[dt] = __builtin_amdgcn_raw_buffer_load_b8(vsrs, off + 32 * dt, 0, 0);
  };

  // V by LDS DMA into a 4-tile ring (64 rows x 128 B; wave w fills rows
  // 8w .. 8w+7, rows past seq_k re-read the last key), 16-byte chunk c of row
  // r at c ^ fv(r), fv(r) = 2 (((r >> 1) & 1) | ((r >> 3) & 1) << 1): the
  // eight rows one transposing read touches in each lane half (4h + 0..3,
  // 8 + 4h + 0..3) sit in distinct bank slots, and the two column halves
  // keep opposite chunk parity, so 32 lanes read 256 bytes without conflict.
  // V(t+3) is issued in iteration t into the slot of V(t-1), whose last
  // reader (group B's G(t-1)) finished two segments earlier.
  const int vrow = wave * 8 + (lane >> 3);
  auto fv = [](uint32_t r) { return 2u * (((r >> 1) & 1u) | (((r >> 3) & 1u) << 1)); };
  const uint32_t vgoff = ((lane & 7) ^ fv((uint32_t)vrow)) << 4;
  auto issue_v = [&](int kt) {
    const uint32_t l = lds0 + k8VtOff + (kt & 3) * k8KBytes + wave * 1024;
    const int key = min(kt * kBN + vrow, p.seq_k - 1);
    dma16(l, Vh, (uint32_t)key * k8KRowBytes + vgoff);
  };
  // ds_read_b64_tr_b8: in each 16-lane group source lane 2e + p addresses
  // V[row R(e)][d0 + 8p .. +7] and lane i then holds V[R(0..7)][d0 + i].
  // Read q: R(e) = 16q + 4h + (e & 3) + 8 (e >> 2), d0 = 32dt + 16 ((l >> 4) & 1),
  // i.e. operand bytes 8q .. 8q+7 are keys 16q + 4h + 0..3 and 16q + 8 + 4h +
  // 0..3 of column 32dt + l%32: the key order of the P operand.
  uint32_t vread[4];
  {
    const uint32_t rl = 4 * half + ((lane >> 1) & 3) + 8 * ((lane >> 3) & 1);
    const uint32_t cl = (lane >> 4) & 1;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      vread[dt] = opaque(lds0 + k8VtOff + rl * k8KRowBytes + (((2 * dt + cl) ^ fv(rl)) << 4) +
                         8 * (lane & 1));
  }
  // Fragment bases: K row kr of block j at +j*4096, d chunks 4s + h (bytes
  // 0-15 of the operand) and 4s + 2 + h (bytes 16-31); V^T row 32dt + kr,
  // bytes 32h .. +31.
  uint32_t kread[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < 2; ++i)
      kread[s][i] = opaque(lds0 + kr * k8KRowBytes +
                           (((4 * s + 2 * i + half) ^ ((kr >> 1) & 7)) << 4));
  auto kfrag = [&](uint32_t kb, int j, int s) {
    return join8(lds_load16(kread[s][0] + kb * k8KBytes + j * 32 * k8KRowBytes),
                 lds_load16(kread[s][1] + kb * k8KBytes + j * 32 * k8KRowBytes));
  };
  typedef __attribute__((address_space(3))) i32x2v lds_i2v;
  auto vfrag = [&](uint32_t vb, int dt) {
    const uint32_t a = vread[dt] + vb * k8KBytes;
    i32x2v r[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      r[q] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i2v *)(uintptr_t)(a + 16 * q * k8KRowBytes));
    return i32x8{r[0][0], r[0][1], r[1][0], r[1][1], r[2][0], r[2][1], r[3][0], r[3][1]};
  };

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = f32x16{};
  // Row sums of the e4m3 P on the MFMA: lacc = ones . P^T, so every
  // accumulator register of lane l holds the sum for query l%32 (only
  // register 0 is kept up to date through the rescales).  That takes 32
  // VALU adds a tile out of the softmax segment and puts one MFMA into the
  // matrix segment, which has room; the sums are then exactly those of the
  // values that multiply V.
  f32x16 lacc = f32x16{};
  const i32x8 ones8 = {0x38383838, 0x38383838, 0x38383838, 0x38383838,
                       0x38383838, 0x38383838, 0x38383838, 0x38383838};  // e4m3 1.0
  float m = -__builtin_inff();  // running max (log2 units), minus the P shift
  const float c = p.scale_log2;
  auto pin = [](auto x) { asm volatile("" ::"v"(x)); };
  i32x8 pf;                     // P^T operand: 32 e4m3 bytes
  // K and V scales by tile parity (every index is a compile-time constant in
  // the unrolled loop): ks[x] / vs[x] hold the scales of a tile with parity x.
  uint32_t ks[2][2], vs[2][4];

  // G(t): S(t+1) (when NEXT) from K buffer KB, O += V^T(t) P(t) from V^T
  // buffer VB; MFMA order S(0,0) PV0 S(0,1) PV1 S(1,0) PV2 S(1,1) PV3, the
  // LDS fragment of MFMA i + 2 read in step i.
  auto seg_g = [&](auto next_tag, auto kb_tag, auto vb_tag, f32x16(&sn)[2]) {
    constexpr bool NEXT = decltype(next_tag)::value;
    constexpr uint32_t KB = decltype(kb_tag)::value;
    constexpr uint32_t VB = decltype(vb_tag)::value;  // also the parity of t
    constexpr int NM = NEXT ? 8 : 4;
    auto is_s = [&](int i) { return NEXT && !(i & 1); };
    auto idx = [&](int i) { return NEXT ? i >> 1 : i; };
    auto frag = [&](int i) {
      const int x = idx(i);
      return is_s(i) ? kfrag(KB, x >> 1, x & 1) : vfrag(VB, x);
    };
    constexpr int kPF = 2;
    i32x8 f[NM];
#pragma unroll
    for (int i = 0; i < kPF && i < NM; ++i)
      f[i] = frag(i);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      if (i + kPF < NM)
        f[i + kPF] = frag(i + kPF);
      const int x = idx(i);
      if (is_s(i)) {
        const int j = x >> 1, s = x & 1;
        sn[j] = mfma_fp8(f[i], qf[s], s == 0 ? f32x16{} : sn[j], ks[(VB & 1) ^ 1][j] >> (16 * s),
                         qs[s]);
      } else {
        o[x] = mfma_fp8(f[i], pf, o[x], vs[VB & 1][x], (uint32_t)k8PScale);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    lacc = mfma_fp8(ones8, pf, lacc, 127u, (uint32_t)k8PScale);
  };

  auto mask = [&](f32x16(&sc)[2], int t) {
    const int k0 = t * kBN;
    const bool edge = (k0 + kBN > p.seq_k) || (CAUSAL && k0 + kBN - 1 > qw);
    if (edge) {
      // Lane terms rebuilt here (fresh): hoisted out of the loop they would
      // hold 32 VGPRs of per-r key offsets.
      const int kl = k0 + 4 * (int)(fresh(threadIdx.x) >> 5 & 1);
      const int lim = CAUSAL ? min(p.seq_k - 1, qw + (int)(fresh(threadIdx.x) & 31)) : p.seq_k - 1;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kl + 32 * j + 8 * (r >> 2) + (r & 3) > lim)
            sc[j][r] = -__builtin_inff();
    }
  };
  auto update_max = [&](float mx) {
    const bool need = mx > m + k8Threshold;
    if (__builtin_amdgcn_ballot_w64(need)) {
      const float mn = fmaxf(m, mx);
      const float alpha = (m == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(m - mn);
      m = mn;
      lacc[0] *= alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[i] *= alpha;
    }
  };
  // Softmax of tile t: P = 2^4 * exp2(c s - m) to e4m3, the P^T operand;
  // fp32 row sums.
  auto softmax = [&](f32x16(&sc)[2], int t) {
    mask(sc, t);
    float mq[4] = {sc[0][0], sc[0][1], sc[1][0], sc[1][1]};
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 2; r < 16; ++r)
        mq[2 * j + (r & 1)] = fmaxf(mq[2 * j + (r & 1)], sc[j][r]);
    float lo, hi;
    half_pair(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3])), lo, hi);
    update_max(fmaxf(lo, hi) * c);
    const float mb = m - k8PShift;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][4 * i + e], c, -mb));
        pf[4 * j + i] = (int)pack_fp8x4(v[0], v[1], v[2], v[3]);
      }
    pin(pf);
  };

  // One iteration t < ntiles - 1: G(t), barrier, SM(t+1), barrier.
  auto iter = [&](auto ph_tag, int t, f32x16(&sn)[2]) {
    constexpr int PH = decltype(ph_tag)::value;
    load_ks(t + 2, ks[PH & 1]);
    load_vs(t + 1, vs[(PH + 1) & 1]);
    seg_g(std::true_type{}, std::integral_constant<uint32_t, (PH + 1) % k8KRing>{},
          std::integral_constant<uint32_t, PH>{}, sn);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    softmax(sn, t + 1);
    issue_k(t + 4);
    issue_v(t + 3);
    vm_wait_barrier<2>();
  };

  // ---- prologue: K(0..3), V(0..2), S(0), softmax(0)
  f32x16 sa[2];
  issue_k(0);
  issue_k(1);
  issue_k(2);
  issue_v(0);
  issue_v(1);
  issue_v(2);
  load_ks(0, ks[0]);
  load_ks(1, ks[1]);
  load_vs(0, vs[0]);
  vm_wait_barrier();
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int j = x >> 1, s = x & 1;
    sa[j] = mfma_fp8(kfrag(0, j, s), qf[s], s == 0 ? f32x16{} : sa[j], ks[0][j] >> (16 * s),
                     qs[s]);
  }
  issue_k(3);
  softmax(sa, 0);
  lds_barrier();
  if (grp == 1)  // group B's idle segment 0
    lds_barrier();

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
  // Last tile: G = PV(t) only (V buffer t & 3, scales of parity t & 1).
  switch (t & 3) {
  case 0: seg_g(std::false_type{}, std::integral_constant<uint32_t, 0>{}, std::integral_constant<uint32_t, 0>{}, sa); break;
  case 1: seg_g(std::false_type{}, std::integral_constant<uint32_t, 0>{}, std::integral_constant<uint32_t, 1>{}, sa); break;
  case 2: seg_g(std::false_type{}, std::integral_constant<uint32_t, 0>{}, std::integral_constant<uint32_t, 2>{}, sa); break;
  default: seg_g(std::false_type{}, std::integral_constant<uint32_t, 0>{}, std::integral_constant<uint32_t, 3>{}, sa); break;
  }
  // K DMA issued for tiles past the end may still be in flight: let it land
  // before the workgroup's LDS can be handed to another workgroup.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (grp == 0)
    lds_barrier();

  // Normalise (both O and the row sums took the 2^-4 off P in their MFMAs)
  // and store O[my_q][d], d = 32dt + 8(r/4) + 4h + r%4.
  const float total = lacc[0];
  const float inv = total > 0.f ? 1.0f / total : 0.f;
  if (p.lse != nullptr && half == 0 && my_q < p.seq_q)
    p.lse[(size_t)bh * p.seq_q + my_q] = (m + __builtin_log2f(total)) * kLn2;
  // Through this wave's own staging area (rows of 256 B, 16-byte chunk c of
  // row r at c ^ (r & 15)), so each global store writes whole rows.
  {
    const uint32_t wb = lds0 + k8StageOff + wave * k8StageBytes;
    const uint32_t wrow = wb + kr * 256 + half * 8;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const u32x2 w = {pack2<OUT_DT>(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv),
                         pack2<OUT_DT>(o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv)};
        const uint32_t cc = (uint32_t)(4 * dt + g);
        lds_store8(wrow + ((cc ^ (kr & 15)) << 4), w);
      }
    const uint32_t cc = lane & 15;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const uint32_t rr = it * 4 + (lane >> 4);
      const u32x4 v = lds_load16(wb + rr * 256 + ((cc ^ (rr & 15)) << 4));
      if (qw + (int)rr < p.seq_q)
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(Oh + (size_t)(qw + rr) * kD + 8 * cc));
    }
  }
}

template <int OUT_DT, bool CAUSAL>
__global__ __launch_bounds__(512, 1) void fwd8_kernel(Fp8Params p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[k8Smem];
  fwd8_cta<OUT_DT, CAUSAL>(p, blockIdx.x, smem);
}

} // namespace attention
} // namespace wave
