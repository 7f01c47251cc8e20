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
// Design (one CTA = 32*NW query rows of one head, NW waves of 64 lanes):
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
//    swizzle (chunk c of row r at c ^ (r & 15)); V tiles are loaded into
//    VGPRs one tile ahead, transposed in registers and written to LDS as
//    V^T rows of 64 keys (+16 B padding, 144 B pitch).  Two buffers each;
//    K runs one tile ahead of V (see the pipeline below).
//  * Software pipeline inside each wave: the MFMAs of S(t+1) are
//    interleaved with the exp2 VALU work of tile t, and the PV MFMAs of
//    tile t with the row max of tile t+1, so the matrix pipe and the VALU
//    stay busy at the same time.
//  * exp2 with the scale folded into one FMA; the running max is only
//    raised (and O rescaled) when a tile's max exceeds it by more than 8
//    (log2 units), as in the reference's lazy rescale
//    (wave_flash_attention.py:557-583); P stays below 2^8.
//  * CTAs of one head are placed on the same XCD so its K/V stay in that
//    XCD's L2; causal grids start with the longest query blocks.
#pragma once

#include "attention.hpp"
#include "wave_common.hpp"

namespace wave {
namespace attention {

constexpr int kD = 128;
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
};

template <int NW>
__device__ __forceinline__ void block_coords(const Params &p, int &bh, int &qb) {
  const int total = p.q_blocks * p.batch * p.q_heads;
  const int raw = blockIdx.x;
  // Dispatch puts CTA i on XCD i % 8; make consecutive pids share an XCD.
  int pid = raw;
  if ((total & 7) == 0)
    pid = (raw & 7) * (total >> 3) + (raw >> 3);
  bh = pid / p.q_blocks;
  qb = pid - bh * p.q_blocks;
  if (p.causal)
    qb = p.q_blocks - 1 - qb;  // longest rows first
}

template <int DT, int NW>
__global__ __launch_bounds__(NW * 64, 2) void fwd_kernel(Params p) {
  static_assert(NW == 4, "V^T transpose mapping assumes 256 threads");
  // LDS: K ring [2][64 keys][256 B] (XOR-swizzled chunks), then the V^T
  // ring [2][128 d][144 B].
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * kKBytes + 2 * kVtBytes];
  constexpr int kRows = 32 * NW;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t half = lane >> 5;
  int bh, qb;
  block_coords<NW>(p, bh, qb);
  const int b = bh / p.q_heads, hq = bh - b * p.q_heads;
  const int hkv = hq / (p.q_heads / p.kv_heads);
  const uint16_t *Qh = p.Q + ((size_t)bh * p.seq_q) * kD;
  const uint16_t *Kh = p.K + ((size_t)(b * p.kv_heads + hkv) * p.seq_k) * kD;
  const char *Vh =
      reinterpret_cast<const char *>(p.V + ((size_t)(b * p.kv_heads + hkv) * p.seq_k) * kD);
  uint16_t *Oh = p.O + ((size_t)bh * p.seq_q) * kD;

  const int q0 = qb * kRows;
  const int qw = q0 + wave * 32;             // this wave's first query
  const int my_q = qw + (lane & 31);          // this lane's query

  // Q^T fragments: lane supplies Q[my_q][16*kk + 8*half .. +8].
  u32x4 qf[8];
  {
    const bool ok = my_q < p.seq_q;
    const uint16_t *qrow = Qh + (size_t)(ok ? my_q : 0) * kD + 8 * half;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      qf[kk] = ok ? *reinterpret_cast<const u32x4 *>(qrow + 16 * kk)
                  : u32x4{0u, 0u, 0u, 0u};
  }

  // Key range.  Causal: keys <= last query of the block.
  int kend = p.seq_k;
  if (p.causal)
    kend = min(kend, q0 + kRows);
  const int ntiles = (kend + kBN - 1) / kBN;

  // K DMA: wave w fills rows 16w .. 16w+15 of the tile (4 x 1 KiB).  Rows
  // past seq_k re-read the last key (masked out of the softmax).
  uint32_t kgoff[4];
  int krow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    krow[i] = (wave * 4 + i) * 4 + (lane >> 4);
    kgoff[i] = ((lane & 15) ^ (krow[i] & 15)) << 4;
  }
  const uint32_t lds0 = lds_addr(smem);
  auto issue_k = [&](uint32_t buf, int kt) {
    const int k0 = kt * kBN;
    const uint32_t l = lds0 + buf * kKBytes + wave * 4 * 1024;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = min(k0 + krow[i], p.seq_k - 1);
      dma16(l + i * 1024, Kh, (uint32_t)key * kKRowBytes + kgoff[i]);
    }
  };

  // V: thread t loads keys 4g..4g+3 (g = t % 16) of d-chunk c = t / 16 into
  // VGPRs one tile ahead.  Keys past seq_k re-read the last key: their P is 0.
  const int vg = threadIdx.x & 15, vc = threadIdx.x >> 4;
  u32x4 vr[4];
  auto load_v = [&](int kt) {
    const int k0 = kt * kBN + 4 * vg;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t key = (uint32_t)min(k0 + i, p.seq_k - 1);
      vr[i] = *reinterpret_cast<const u32x4 *>(Vh + key * kKRowBytes + 16 * vc);
    }
  };
  // V^T position of key group g: 16-key group G = g/4 stored as
  // [0-3, 8-11, 4-7, 12-15].
  const int vpos = 16 * (vg >> 2) + 4 * ((vg & 1) * 2 + ((vg >> 1) & 1));
  uint8_t *const vt0 = smem + 2 * kKBytes;
  auto store_v = [&](uint32_t buf) {
    uint8_t *s = vt0 + buf * kVtBytes + vpos * 2;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // d = 8*vc + 2e (low halves) and 8*vc + 2e + 1 (high halves).
      const uint32_t lo01 = __builtin_amdgcn_perm(vr[1][e], vr[0][e], 0x05040100u);
      const uint32_t lo23 = __builtin_amdgcn_perm(vr[3][e], vr[2][e], 0x05040100u);
      const uint32_t hi01 = __builtin_amdgcn_perm(vr[1][e], vr[0][e], 0x07060302u);
      const uint32_t hi23 = __builtin_amdgcn_perm(vr[3][e], vr[2][e], 0x07060302u);
      const int d = 8 * vc + 2 * e;
      *reinterpret_cast<u32x2 *>(s + d * kVtPitch) = u32x2{lo01, lo23};
      *reinterpret_cast<u32x2 *>(s + (d + 1) * kVtPitch) = u32x2{hi01, hi23};
    }
  };

  const uint32_t kr = lane & 31;                     // key row within block
  const uint32_t vt_row = (lane & 31) * kVtPitch;    // d row within d-tile

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = f32x16{};
  // Row sums on the matrix pipe: ones[32 x 16] . P^T gives, in every
  // accumulator register of lane l, the sum of P over the slice for query
  // l%32.  Only register 0 is read (and rescaled); it sums exactly the
  // 16-bit P values that multiply V.
  f32x16 lacc = f32x16{};
  const u32x4 ones = {kOnePair<DT>, kOnePair<DT>, kOnePair<DT>, kOnePair<DT>};
  float m = -__builtin_inff();
  const float c = p.scale_log2;

  // ---- stage primitives ---------------------------------------------------
  // S^T = K . Q^T for the 2 blocks of 32 keys of the tile in K buffer kb.
  auto s_mfma = [&](f32x16 (&sc)[2], uint32_t kb) {
    const uint8_t *ks = smem + kb * kKBytes;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      sc[j] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t row = j * 32 + kr;
        const uint32_t chunk = (2 * kk + half) ^ (row & 15);
        const u32x4 kf =
            *reinterpret_cast<const u32x4 *>(ks + row * kKRowBytes + (chunk << 4));
        sc[j] = mfma32x32x16<DT>(kf, qf[kk], sc[j]);
      }
  };
  // Masks of tile t: causal (key > query) and keys past seq_k.
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
  auto rowmax = [&](const f32x16 (&sc)[2]) {
    float mx = sc[0][0];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        mx = fmaxf(mx, sc[j][r]);
    return fmaxf(mx, __shfl_xor(mx, 32)) * c;
  };
  // Lazy rescale: raise the running max only when it grows by > 8 (log2).
  auto update_max = [&](float mx) {
    const bool need = mx > m + kRescaleThreshold;
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
  // P = exp2(s*c - m), packed to 16 bits as the B operand of O^T += V^T P^T.
  auto exp_pack = [&](const f32x16 (&sc)[2], u32x4 (&pf)[2][2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][8 * sl + 2 * e], c, -m));
          const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][8 * sl + 2 * e + 1], c, -m));
          pf[j][sl][e] = pack2<DT>(p0, p1);
        }
  };
  // O^T += V^T . P^T over 4 d-tiles x 4 key slices (V^T buffer vb), and the
  // row sums alongside.
  auto pv_mfma = [&](const u32x4 (&pf)[2][2], uint32_t vb) {
    const uint8_t *vs = vt0 + vb * kVtBytes;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const u32x4 vf = *reinterpret_cast<const u32x4 *>(
              vs + dt * 32 * kVtPitch + vt_row + (16 * (2 * j + sl) + 8 * half) * 2);
          o[dt] = mfma32x32x16<DT>(vf, pf[j][sl], o[dt]);
        }
        lacc = mfma32x32x16<DT>(ones, pf[j][sl], lacc);
      }
  };

  // ---- fused pipeline phases ----------------------------------------------
  // pin(x): an empty asm use, so x is computed in the step that produces it
  // (without it, IR-level sinking moves the VALU work next to its uses).
  auto pin = [](auto x) { asm volatile("" ::"v"(x)); };
  // Each phase is written as explicit steps of one MFMA plus a share of the
  // VALU work of the other tile; sched_barrier keeps the steps in order so
  // the two pipes overlap.  LDS fragment reads run 4 steps ahead.
  //
  // Phase 1: S(t+1) = K(t+1) . Q^T (16 MFMAs) with P(t) = exp2(S(t)*c - m)
  // packed to 16 bits (2 elements per step).
  auto phase1 = [&](f32x16 (&sn)[2], uint32_t kb, const f32x16 (&sc)[2],
                    u32x4 (&pf)[2][2]) {
    const uint8_t *ks = smem + kb * kKBytes;
    auto kfrag = [&](int i) {  // i = 2*kk + j
      const uint32_t row = (i & 1) * 32 + kr;
      const uint32_t chunk = (2 * (i >> 1) + half) ^ (row & 15);
      return *reinterpret_cast<const u32x4 *>(ks + row * kKRowBytes + (chunk << 4));
    };
    u32x4 kf[16];
    sn[0] = f32x16{};
    sn[1] = f32x16{};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      kf[i] = kfrag(i);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i + 4 < 16)
        kf[i + 4] = kfrag(i + 4);
      sn[i & 1] = mfma32x32x16<DT>(kf[i], qf[i >> 1], sn[i & 1]);
      const int j = i >> 3, r = (2 * i) & 15;
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][r], c, -m));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][r + 1], c, -m));
      pf[j][r >> 3][(r & 7) >> 1] = pack2<DT>(p0, p1);
      pin(pf[j][r >> 3][(r & 7) >> 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Phase 2: O^T += V(t)^T . P(t)^T and the row sums (20 MFMAs) with the
  // row max of S(t+1) and the register transpose of V(t+1) for its LDS
  // store.  Returns the scaled row max of S(t+1).
  auto phase2 = [&](const u32x4 (&pf)[2][2], uint32_t vb, const f32x16 (&sn)[2],
                    bool with_next) {
    const uint8_t *vs = vt0 + vb * kVtBytes;
    auto vfrag = [&](int i) {  // i = 4*(2*j + sl) + dt
      const int g = i >> 2, dt = i & 3;
      return *reinterpret_cast<const u32x4 *>(vs + dt * 32 * kVtPitch + vt_row +
                                              (16 * g + 8 * half) * 2);
    };
    u32x4 vf[16];
    float mx = -__builtin_inff();
    uint32_t tr[16];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      vf[i] = vfrag(i);
#pragma unroll
    for (int q = 0; q < 20; ++q) {
      const int g = q / 5, w = q % 5;
      const u32x4 &pb = pf[g >> 1][g & 1];
      if (w < 4) {
        const int i = 4 * g + w;
        if (i + 4 < 16)
          vf[i + 4] = vfrag(i + 4);
        o[w] = mfma32x32x16<DT>(vf[i], pb, o[w]);
      } else {
        lacc = mfma32x32x16<DT>(ones, pb, lacc);
      }
      if (with_next) {
        // 32 S values -> 16 max3 steps, then 16 perms of the V transpose.
        if (q < 16) {
          mx = __builtin_fmaxf(__builtin_fmaxf(mx, sn[q >> 3][(2 * q) & 15]),
                               sn[q >> 3][((2 * q) & 15) + 1]);
          pin(mx);
        }
        if (q >= 4) {
          const int e = (q - 4) >> 2, k = (q - 4) & 3;
          // k: 0 lo01, 1 lo23, 2 hi01, 3 hi23 of dword e
          const int a = (k & 1) ? 3 : 1, b2 = (k & 1) ? 2 : 0;
          tr[q - 4] = __builtin_amdgcn_perm(vr[a][e], vr[b2][e],
                                            (k & 2) ? 0x07060302u : 0x05040100u);
          pin(tr[q - 4]);
          // Dword e of the transpose is complete: store its two V^T rows
          // now (the buffer's last reader, PV(t-1), finished before the
          // previous barrier), so only 4 transposed registers are live.
          if (k == 3) {
            uint8_t *sv = vt0 + (vb ^ 1) * kVtBytes + vpos * 2;
            const int d = 8 * vc + 2 * e;
            *reinterpret_cast<u32x2 *>(sv + d * kVtPitch) = u32x2{tr[4 * e], tr[4 * e + 1]};
            *reinterpret_cast<u32x2 *>(sv + (d + 1) * kVtPitch) =
                u32x2{tr[4 * e + 2], tr[4 * e + 3]};
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    return fmaxf(mx, __shfl_xor(mx, 32)) * c;
  };

  // ---- software pipeline over key tiles --------------------------------------
  // Iteration t: the matrix pipe computes S(t+1) while the VALU turns S(t)
  // into P(t) (phase 1), then the matrix pipe computes O += V(t) P(t) while
  // the VALU reduces S(t+1) to its row max and transposes V(t+1) (phase 2).
  // K runs one tile ahead of V: K(t+2) and V(t+1) are loaded during
  // iteration t into the buffers that K(t) and V(t-1) left.
  // The loop is unrolled by two with the score arrays swapping roles, so no
  // register copies carry S(t+1) into the next iteration.
  f32x16 sa[2], sb[2];
  u32x4 pf[2][2];
  issue_k(0, 0);
  load_v(0);
  vm_wait_barrier();
  if (ntiles > 1)
    issue_k(1, 1);
  s_mfma(sa, 0);
  store_v(0);
  mask(sa, 0);
  update_max(rowmax(sa));
  vm_wait_barrier();
  // cur = t & 1 is passed as a constant (t is even for sc = sa).
  auto iteration = [&](int t, uint32_t cur, const f32x16 (&sc)[2], f32x16 (&sn)[2]) {
    load_v(t + 1);
    if (t + 2 < ntiles)
      issue_k(cur, t + 2);
    phase1(sn, cur ^ 1, sc, pf);
    mask(sn, t + 1);
    const float mx = phase2(pf, cur, sn, true);
    update_max(mx);
    vm_wait_barrier();
  };
  int t = 0;
  for (; t + 2 < ntiles; t += 2) {
    iteration(t, 0, sa, sb);
    iteration(t + 1, 1, sb, sa);
  }
  if (t + 1 < ntiles) {
    iteration(t, 0, sa, sb);
    exp_pack(sb, pf);
    pv_mfma(pf, 1);
  } else {
    exp_pack(sa, pf);
    pv_mfma(pf, 0);
  }
  const float lsum = lacc[0];

  // Normalise and store O[my_q][d], d = 32*dt + 8*(r/4) + 4*half + r%4.
  const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
  if (my_q < p.seq_q) {
    uint16_t *orow = Oh + (size_t)my_q * kD + 4 * half;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const u32x2 w = {pack2<DT>(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv),
                         pack2<DT>(o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv)};
        *reinterpret_cast<u32x2 *>(orow + 32 * dt + 8 * g) = w;
      }
  }
}

// ------------------------------------------------------------------------
// fwd64_kernel: 4 waves x 64 query rows (two 32-row query blocks per wave),
// 32-key tiles, one CTA per CU.  Each K and V^T fragment read from LDS feeds
// two MFMAs (one per query block), halving LDS read traffic per MFMA
// relative to fwd_kernel.  Same per-lane softmax orientation, V^T key
// permutation, MFMA row sums, lazy rescale and two-phase intra-wave
// pipeline.  K: 3-buffer LDS ring (DMA two tiles ahead); V: loaded one tile
// ahead into VGPRs with explicitly counted loads, transposed into a 2-buffer
// V^T ring with an 80-byte pitch (16 consecutive d rows -> distinct banks).
constexpr int kBN2 = 32;                            // keys per tile
constexpr int kK2Bytes = kBN2 * kKRowBytes;         // 8 KiB
constexpr int kVt2Pitch = kBN2 * 2 + 16;            // 80 B per d row of V^T
constexpr int kVt2Bytes = kD * kVt2Pitch;           // 10 KiB
constexpr int kKRing = 3;

// Global load of 16 bytes per lane whose completion the caller waits for
// with vm_wait_regs (the compiler does not track it).
__device__ __forceinline__ u32x4 gload16(const void *base, uint32_t voff) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(v) : "v"(voff), "s"(base));
  return v;
}
// s_waitcnt vmcnt(N) that also "redefines" a and b, so no use of them can be
// scheduled before the wait.
template <int N>
__device__ __forceinline__ void vm_wait_regs(u32x4 &a, u32x4 &b) {
  asm volatile("s_waitcnt vmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N) : "memory");
}

template <int DT>
__global__ __launch_bounds__(256, 1) void fwd64_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kKRing * kK2Bytes + 2 * kVt2Bytes];
  constexpr int kRows = 256;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t half = lane >> 5;
  int bh, qb_idx;
  block_coords<4>(p, bh, qb_idx);
  const int b = bh / p.q_heads, hq = bh - b * p.q_heads;
  const int hkv = hq / (p.q_heads / p.kv_heads);
  const uint16_t *Qh = p.Q + ((size_t)bh * p.seq_q) * kD;
  const char *Kh = reinterpret_cast<const char *>(
      p.K + ((size_t)(b * p.kv_heads + hkv) * p.seq_k) * kD);
  const char *Vh = reinterpret_cast<const char *>(
      p.V + ((size_t)(b * p.kv_heads + hkv) * p.seq_k) * kD);
  uint16_t *Oh = p.O + ((size_t)bh * p.seq_q) * kD;

  const int q0 = qb_idx * kRows;
  const int qw = q0 + wave * 64;  // this wave's first query
  int my_q[2];
  my_q[0] = qw + (lane & 31);
  my_q[1] = qw + 32 + (lane & 31);

  // Q^T fragments of both query blocks.
  u32x4 qf[2][8];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const bool ok = my_q[g] < p.seq_q;
    const uint16_t *qrow = Qh + (size_t)(ok ? my_q[g] : 0) * kD + 8 * half;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      qf[g][kk] = ok ? *reinterpret_cast<const u32x4 *>(qrow + 16 * kk)
                     : u32x4{0u, 0u, 0u, 0u};
  }

  int kend = p.seq_k;
  if (p.causal)
    kend = min(kend, q0 + kRows);
  const int ntiles = (kend + kBN2 - 1) / kBN2;

  // K DMA: wave w fills rows 8w .. 8w+7 of the 32-row tile (2 x 1 KiB).
  uint32_t kgoff[2];
  int krow[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    krow[i] = (wave * 2 + i) * 4 + (lane >> 4);
    kgoff[i] = ((lane & 15) ^ (krow[i] & 15)) << 4;
  }
  const uint32_t lds0 = lds_addr(smem);
  auto issue_k = [&](uint32_t buf, int kt) {
    const uint32_t l = lds0 + buf * kK2Bytes + wave * 2 * 1024;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = min(kt * kBN2 + krow[i], p.seq_k - 1);
      dma16(l + i * 1024, Kh, (uint32_t)key * kKRowBytes + kgoff[i]);
    }
  };
  // V: thread t loads keys 2g, 2g+1 (g = t % 16) of d-chunk c = t / 16.
  const int vg = threadIdx.x & 15, vc = threadIdx.x >> 4;
  u32x4 vr[2];
  auto load_v = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t key = (uint32_t)min(kt * kBN2 + 2 * vg + i, p.seq_k - 1);
      vr[i] = gload16(Vh, key * kKRowBytes + 16 * vc);
    }
  };
  // V^T position of keys 2g, 2g+1: 16-key groups stored as [0-3,8-11,4-7,12-15].
  const int vk = (2 * vg) & 15;
  const int vpos = 16 * (vg >> 3) + (vk < 4 ? vk : vk < 8 ? vk + 4 : vk < 12 ? vk - 4 : vk);
  uint8_t *const vt0 = smem + kKRing * kK2Bytes;
  uint32_t tr[8];
  auto transpose_v = [&](int e) {  // dword e: d = 8*vc + 2e (lo), +1 (hi)
    tr[2 * e] = __builtin_amdgcn_perm(vr[1][e], vr[0][e], 0x05040100u);
    tr[2 * e + 1] = __builtin_amdgcn_perm(vr[1][e], vr[0][e], 0x07060302u);
  };
  auto store_vt = [&](uint32_t buf) {
    uint8_t *s = vt0 + buf * kVt2Bytes + vpos * 2;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = 8 * vc + 2 * e;
      *reinterpret_cast<uint32_t *>(s + d * kVt2Pitch) = tr[2 * e];
      *reinterpret_cast<uint32_t *>(s + (d + 1) * kVt2Pitch) = tr[2 * e + 1];
    }
  };

  const uint32_t kr = lane & 31;
  const uint32_t vt_row = (lane & 31) * kVt2Pitch;
  f32x16 o[2][4];
  f32x16 lacc[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    lacc[g] = f32x16{};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[g][i] = f32x16{};
  }
  const u32x4 ones = {kOnePair<DT>, kOnePair<DT>, kOnePair<DT>, kOnePair<DT>};
  float m[2] = {-__builtin_inff(), -__builtin_inff()};
  const float c = p.scale_log2;
  auto pin = [](auto x) { asm volatile("" ::"v"(x)); };

  auto kfrag = [&](uint32_t kb, int kk) {
    const uint32_t chunk = (2 * kk + half) ^ (kr & 15);
    return *reinterpret_cast<const u32x4 *>(smem + kb * kK2Bytes + kr * kKRowBytes +
                                            (chunk << 4));
  };
  auto mask = [&](f32x16 (&sc)[2], int t) {
    const int k0 = t * kBN2;
    const bool edge = (k0 + kBN2 > p.seq_k) || (p.causal && k0 + kBN2 - 1 > qw);
    if (edge) {
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
          if (key >= p.seq_k || (p.causal && key > my_q[g]))
            sc[g][r] = -__builtin_inff();
        }
    }
  };
  auto update_max = [&](int g, float mx) {
    const bool need = mx > m[g] + kRescaleThreshold;
    if (__builtin_amdgcn_ballot_w64(need)) {
      const float mn = fmaxf(m[g], mx);
      const float alpha = (m[g] == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(m[g] - mn);
      m[g] = mn;
      lacc[g][0] *= alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[g][i] *= alpha;
    }
  };
  auto rowmax = [&](const f32x16 &s) {
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r)
      mx = fmaxf(mx, s[r]);
    return fmaxf(mx, __shfl_xor(mx, 32)) * c;
  };

  // Phase 1: S(t+1) (16 MFMAs: 8 K fragments x 2 query blocks) with
  // P(t) = exp2(S(t)*c - m) (2 elements per step).
  u32x4 pf[2][2];
  auto phase1 = [&](f32x16 (&sn)[2], uint32_t kb, const f32x16 (&sc)[2]) {
    u32x4 kf[8];
    sn[0] = f32x16{};
    sn[1] = f32x16{};
    kf[0] = kfrag(kb, 0);
    kf[1] = kfrag(kb, 1);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kk = i >> 1, g = i & 1;
      if (g == 0 && kk + 2 < 8)
        kf[kk + 2] = kfrag(kb, kk + 2);
      sn[g] = mfma32x32x16<DT>(kf[kk], qf[g][kk], sn[g]);
      const int e = 2 * i, eg = e >> 4, r = e & 15;
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[eg][r], c, -m[eg]));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[eg][r + 1], c, -m[eg]));
      pf[eg][r >> 3][(r & 7) >> 1] = pack2<DT>(p0, p1);
      pin(pf[eg][r >> 3][(r & 7) >> 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Phase 2: O^T += V^T(t) P^T(t) and row sums (20 MFMAs) with the row max
  // of S(t+1) and the transpose of V(t+1).  Returns both scaled maxima.
  float mxo[2];
  auto phase2 = [&](uint32_t vb, const f32x16 (&sn)[2], bool with_next) {
    const uint8_t *vs = vt0 + vb * kVt2Bytes;
    auto vfrag = [&](int sl, int dt) {
      return *reinterpret_cast<const u32x4 *>(vs + dt * 32 * kVt2Pitch + vt_row +
                                              (16 * sl + 8 * half) * 2);
    };
    u32x4 vf[8];
    float mx[2] = {-__builtin_inff(), -__builtin_inff()};
    vf[0] = vfrag(0, 0);
    vf[1] = vfrag(0, 1);
    int q = 0;
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
#pragma unroll
      for (int x = 0; x < 5; ++x) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          if (x < 4) {
            const int fi = sl * 4 + x;
            if (g == 0 && fi + 2 < 8)
              vf[fi + 2] = vfrag((fi + 2) >> 2, (fi + 2) & 3);
            o[g][x] = mfma32x32x16<DT>(vf[fi], pf[g][sl], o[g][x]);
          } else {
            lacc[g] = mfma32x32x16<DT>(ones, pf[g][sl], lacc[g]);
          }
          if (with_next) {
            if (q < 16) {
              const int mg = q >> 3, r = (2 * q) & 15;
              mx[mg] = __builtin_fmaxf(__builtin_fmaxf(mx[mg], sn[mg][r]), sn[mg][r + 1]);
              pin(mx[mg]);
            } else {
              transpose_v(q - 16);
              pin(tr[2 * (q - 16)]);
              pin(tr[2 * (q - 16) + 1]);
            }
          }
          ++q;
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    mxo[0] = fmaxf(mx[0], __shfl_xor(mx[0], 32)) * c;
    mxo[1] = fmaxf(mx[1], __shfl_xor(mx[1], 32)) * c;
  };

  // ---- pipeline -----------------------------------------------------------
  f32x16 sc[2], sn[2];
  issue_k(0, 0);
  load_v(0);
  vm_wait_regs<0>(vr[0], vr[1]);
  lds_barrier();
  issue_k(1, min(1, ntiles - 1));
  issue_k(2, min(2, ntiles - 1));
  {
    // S(0), first row maxima, V^T(0).
    sc[0] = f32x16{};
    sc[1] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const u32x4 kf = kfrag(0, kk);
      sc[0] = mfma32x32x16<DT>(kf, qf[0][kk], sc[0]);
      sc[1] = mfma32x32x16<DT>(kf, qf[1][kk], sc[1]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
      transpose_v(e);
    store_vt(0);
    mask(sc, 0);
    update_max(0, rowmax(sc[0]));
    update_max(1, rowmax(sc[1]));
  }
  vm_wait_barrier<2>();
  for (int t = 0; t + 1 < ntiles; ++t) {
    const uint32_t vcur = t & 1;
    load_v(t + 1);
    issue_k(t % kKRing, min(t + 3, ntiles - 1));
    phase1(sn, (t + 1) % kKRing, sc);
    mask(sn, t + 1);
    vm_wait_regs<2>(vr[0], vr[1]);  // V(t+1) landed; K DMA may stay in flight
    phase2(vcur, sn, true);
    store_vt(vcur ^ 1);
    update_max(0, mxo[0]);
    update_max(1, mxo[1]);
    sc[0] = sn[0];
    sc[1] = sn[1];
    vm_wait_barrier<2>();
  }
  // Last tile: P and O += V P.
#pragma unroll
  for (int e = 0; e < 32; e += 2) {
    const int eg = e >> 4, r = e & 15;
    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[eg][r], c, -m[eg]));
    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[eg][r + 1], c, -m[eg]));
    pf[eg][r >> 3][(r & 7) >> 1] = pack2<DT>(p0, p1);
  }
  phase2((ntiles - 1) & 1, sn, false);
  vm_wait_barrier();

#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const float lsum = lacc[g][0];
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    if (my_q[g] < p.seq_q) {
      uint16_t *orow = Oh + (size_t)my_q[g] * kD + 4 * half;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
          const u32x2 w = {pack2<DT>(o[g][dt][4 * gg] * inv, o[g][dt][4 * gg + 1] * inv),
                           pack2<DT>(o[g][dt][4 * gg + 2] * inv, o[g][dt][4 * gg + 3] * inv)};
          *reinterpret_cast<u32x2 *>(orow + 32 * dt + 8 * gg) = w;
        }
    }
  }
}

} // namespace attention
} // namespace wave
