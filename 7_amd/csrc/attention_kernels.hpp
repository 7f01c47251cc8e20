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
//    V^T rows of 64 keys (+16 B padding, 144 B pitch).  Two stages.
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
constexpr int kStageBytes = kKBytes + kVtBytes;  // 34 KiB
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
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * kStageBytes];
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
  const uint16_t *Vh = p.V + ((size_t)(b * p.kv_heads + hkv) * p.seq_k) * kD;
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

  // K DMA: wave w fills rows 16w .. 16w+15 of the tile (4 x 1 KiB).
  uint32_t kgoff[4];
  int krow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    krow[i] = (wave * 4 + i) * 4 + (lane >> 4);
    kgoff[i] = ((lane & 15) ^ (krow[i] & 15)) << 4;
  }
  const uint32_t lds0 = lds_addr(smem);
  auto issue_k = [&](uint32_t stage, int kt) {
    const int k0 = kt * kBN;
    const uint32_t l = lds0 + stage * kStageBytes + wave * 4 * 1024;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // Rows past seq_k re-read the last key (masked out of the softmax).
      const int key = min(k0 + krow[i], p.seq_k - 1);
      dma16(l + i * 1024, Kh, (uint32_t)key * kKRowBytes + kgoff[i]);
    }
  };

  // V: thread t loads keys 4g..4g+3 (g = t % 16) of d-chunk c = t / 16.
  const int vg = threadIdx.x & 15, vc = threadIdx.x >> 4;
  u32x4 vr[4];
  auto load_v = [&](int kt) {
    const int k0 = kt * kBN + 4 * vg;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = k0 + i;
      vr[i] = key < p.seq_k
                  ? *reinterpret_cast<const u32x4 *>(Vh + (size_t)key * kD + 8 * vc)
                  : u32x4{0u, 0u, 0u, 0u};
    }
  };
  // V^T position of key group g: 16-key group G = g/4 stored as
  // [0-3, 8-11, 4-7, 12-15].
  const int vpos = 16 * (vg >> 2) + 4 * ((vg & 1) * 2 + ((vg >> 1) & 1));
  auto store_v = [&](uint32_t stage) {
    uint8_t *s = smem + stage * kStageBytes + kKBytes + vpos * 2;
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

  // Fragment addressing (per lane).
  const uint32_t kr = lane & 31;                     // key row within block
  const uint32_t vt_row = (lane & 31) * kVtPitch;    // d row within d-tile

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = f32x16{};
  float m = -__builtin_inff();
  float lsum = 0.f;
  const float c = p.scale_log2;

  if (ntiles > 0) {
    issue_k(0, 0);
    load_v(0);
    store_v(0);
    vm_wait_barrier();
  }
  for (int t = 0; t < ntiles; ++t) {
    const uint32_t stage = t & 1;
    const bool more = t + 1 < ntiles;
    if (more) {
      issue_k(stage ^ 1, t + 1);
      load_v(t + 1);
    }
    const uint8_t *ks = smem + stage * kStageBytes;
    const uint8_t *vs = ks + kKBytes;
    const int k0 = t * kBN;
    // Waves whose queries all precede the tile skip it (causal).
    const bool active = !p.causal || k0 <= qw + 31;
    if (active) {
      // S^T = K . Q^T for 2 blocks of 32 keys.
      f32x16 s[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        s[j] = f32x16{};
        const uint32_t row = j * 32 + kr;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const uint32_t chunk = (2 * kk + half) ^ (row & 15);
          const u32x4 kf =
              *reinterpret_cast<const u32x4 *>(ks + row * kKRowBytes + (chunk << 4));
          s[j] = mfma32x32x16<DT>(kf, qf[kk], s[j]);
        }
      }
      // Masks: causal (key > query) and keys past seq_k.
      const bool edge = (k0 + kBN > p.seq_k) || (p.causal && k0 + kBN - 1 > qw);
      if (edge) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = k0 + 32 * j + 8 * (r >> 2) + 4 * half + (r & 3);
            if (key >= p.seq_k || (p.causal && key > my_q))
              s[j][r] = -__builtin_inff();
          }
      }
      float mx = s[0][0];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          mx = fmaxf(mx, s[j][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      mx *= c;
      // Lazy rescale: raise the running max only when it grows by > 8.
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
      // P = exp2(s*c - m), packed to 16 bits as the B operand of O^T += V^T P^T.
      u32x4 pf[2][2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int sl = 0; sl < 2; ++sl)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][8 * sl + 2 * e], c, -m));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][8 * sl + 2 * e + 1], c, -m));
            lsum += p0 + p1;
            pf[j][sl][e] = pack2<DT>(p0, p1);
          }
      // O^T += V^T . P^T over 4 d-tiles x 4 key slices.
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int sl = 0; sl < 2; ++sl) {
            const u32x4 vf = *reinterpret_cast<const u32x4 *>(
                vs + dt * 32 * kVtPitch + vt_row + (16 * (2 * j + sl) + 8 * half) * 2);
            o[dt] = mfma32x32x16<DT>(vf, pf[j][sl], o[dt]);
          }
    }
    if (more)
      store_v(stage ^ 1);
    vm_wait_barrier();
  }

  // Normalise and store O[my_q][d], d = 32*dt + 8*(r/4) + 4*half + r%4.
  const float ltot = lsum + __shfl_xor(lsum, 32);
  const float inv = ltot > 0.f ? 1.0f / ltot : 0.f;
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

} // namespace attention
} // namespace wave
