// attention_fwd4.hpp -- the 4-wave variant of the gfx950 flash-attention
// forward: the reference's `waves=4` configuration of
// flash_attention_bf16_gfx950 (python/mlir/dialects/wave_flash_attention.py
// :44-93 config, :114-135 threads and LDS: block 256, 256 query rows per
// CTA, grid (S/256, B*H)), whose runner default is --threads 256
// --dynamic-lds 68096 (tools/wave-fa-calibrate/wave-fa-gfx950-runner.cpp).
//
// Same math and conventions as fwd_pp_cta (attention_kernels.hpp): S^T =
// K . Q^T per wave, P^T straight from the S^T accumulators, V^T with each
// 16-key group permuted as [0-3, 8-11, 4-7, 12-15], lazy rescale at 8
// (log2 units), v_dot2 row sums of the packed P, optional fixed max.  The
// schedule differs:
//  * 4 waves x 32 query rows = 128 rows per pass; a CTA runs its 256 rows
//    as two passes over the keys.  64 KiB of LDS and at most 256 VGPRs let
//    two CTAs share a CU, so each SIMD holds two waves of different CTAs
//    whose MFMA and softmax work overlap.
//  * Within a wave, a two-phase pipeline per 64-key tile: phase 1 issues
//    the 16 MFMAs of S(t+1) with the exp2 / pack / row sum of P(t)
//    interleaved one element pair per MFMA; phase 2 issues the 16 MFMAs of
//    O += V(t) P(t) with the row max of S(t+1) and the register transpose
//    of V(t+1) interleaved (V^T rows stored as each transposed dword
//    completes).  sched_barrier keeps the pairs together.
//  * K: 2-tile LDS ring filled by global_load_lds_dwordx4 one tile ahead
//    (chunk c of key row r at c ^ (r & 15)).  V: loaded one tile ahead into
//    VGPRs, transposed in registers into a 2-tile V^T ring of 136-byte rows
//    (64 keys + 8 bytes).  That pitch keeps the ring within the runner's
//    LDS; it is 8-byte aligned, so a V^T fragment is two ds_read_b64 (the
//    32 rows of one read then cover all 64 banks).
#pragma once

#include "attention_kernels.hpp"

namespace wave {
namespace attention {

constexpr int kF4Waves = 4;
constexpr int kF4PassRows = 32 * kF4Waves;       // 128 query rows per pass
constexpr int kVt4Pitch = kBN * 2 + 8;           // 136 B per d row of V^T
constexpr int kVt4Bytes = kD * kVt4Pitch;        // 17 KiB
// LDS of one 4-wave CTA: K ring [2][64 keys][256 B], V^T ring
// [2][128 d][136 B] = 67584 bytes, within the runner's 68096.
constexpr int kF4Smem = 2 * kKBytes + 2 * kVt4Bytes;

// CTA `raw` of a grid of q_blocks * batch * q_heads CTAs of 256 threads
// (q_blocks = ceil(seq_q / 256)).  smem: kF4Smem bytes of 1024-byte-aligned
// LDS.  FIXED as in fwd_pp_cta.
template <int DT, bool FIXED = false>
__device__ __forceinline__ void fwd4_cta(const Params &p, int raw, uint8_t *smem) {
  int bh, qb;
  block_coords(p, raw, bh, qb);
  const int b = bh / p.q_heads, hq = bh - b * p.q_heads;
  const int hkv = hq / (p.q_heads / p.kv_heads);
  const uint16_t *Qh = p.Q + ((size_t)bh * p.seq_q) * kD;
  const uint16_t *Kh = p.K + ((size_t)(b * p.kv_heads + hkv) * p.seq_k) * kD;
  const char *Vh =
      reinterpret_cast<const char *>(p.V + ((size_t)(b * p.kv_heads + hkv) * p.seq_k) * kD);
  uint16_t *Oh = p.O + ((size_t)bh * p.seq_q) * kD;
  const uint32_t lds0 = lds_addr(smem);
  uint8_t *const vt0 = smem + 2 * kKBytes;
  const float c = p.scale_log2;
  auto pin = [](auto x) { asm volatile("" ::"v"(x)); };

#pragma unroll 1
  for (int pass = 0; pass < 2; ++pass) {
    const int q0 = qb * (2 * kF4PassRows) + pass * kF4PassRows;
    if (q0 >= p.seq_q)
      break;
    // Per-lane values are derived inside the pass (from a thread id the
    // compiler cannot hoist), so nothing per-lane stays live between passes.
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t wave = uniform(tid >> 6);
    const uint32_t lane = tid & 63;
    const uint32_t half = lane >> 5;
    const uint32_t kr = lane & 31;
    // K DMA: wave w fills rows 16w .. 16w+15 of the tile (4 x 1 KiB).  Rows
    // past seq_k re-read the last key (masked out of the softmax).
    uint32_t kgoff[4];
    int krow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      krow[i] = (wave * 4 + i) * 4 + (lane >> 4);
      kgoff[i] = ((lane & 15) ^ (krow[i] & 15)) << 4;
    }
    // V: thread t loads keys 4g..4g+3 (g = t % 16) of d-chunk c = t / 16 one
    // tile ahead.  Keys past seq_k re-read the last key: their P is 0.
    const int vg = tid & 15, vc = tid >> 4;
    // V^T key position of key group g: 16-key groups stored as
    // [0-3, 8-11, 4-7, 12-15].
    const int vpos = 16 * (vg >> 2) + 4 * ((vg & 1) * 2 + ((vg >> 1) & 1));
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
    // Key range.  Causal: keys <= last query of the pass.
    int kend = p.seq_k;
    if (p.causal)
      kend = min(kend, q0 + kF4PassRows);
    const int ntiles = (kend + kBN - 1) / kBN;

    auto issue_k = [&](uint32_t buf, int kt) {
      const int k0 = kt * kBN;
      const uint32_t l = lds0 + buf * kKBytes + wave * 4 * 1024;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = min(k0 + krow[i], p.seq_k - 1);
        dma16(l + i * 1024, Kh, (uint32_t)key * kKRowBytes + kgoff[i]);
      }
    };
    u32x4 vr[4];
    auto load_v = [&](int kt) {
      const int k0 = kt * kBN + 4 * vg;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t key = (uint32_t)min(k0 + i, p.seq_k - 1);
        vr[i] = *reinterpret_cast<const u32x4 *>(Vh + key * kKRowBytes + 16 * vc);
      }
    };
    // V^T rows d, d + 1 (d = 8*vc + 2e) of transposed dword e into buffer vb.
    auto store_vt_rows = [&](uint32_t vb, int e, uint32_t lo01, uint32_t lo23, uint32_t hi01,
                             uint32_t hi23) {
      uint8_t *sv = vt0 + vb * kVt4Bytes + vpos * 2;
      const int d = 8 * vc + 2 * e;
      *reinterpret_cast<u32x2 *>(sv + d * kVt4Pitch) = u32x2{lo01, lo23};
      *reinterpret_cast<u32x2 *>(sv + (d + 1) * kVt4Pitch) = u32x2{hi01, hi23};
    };
    auto store_v = [&](uint32_t vb) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        store_vt_rows(vb, e, __builtin_amdgcn_perm(vr[1][e], vr[0][e], 0x05040100u),
                      __builtin_amdgcn_perm(vr[3][e], vr[2][e], 0x05040100u),
                      __builtin_amdgcn_perm(vr[1][e], vr[0][e], 0x07060302u),
                      __builtin_amdgcn_perm(vr[3][e], vr[2][e], 0x07060302u));
    };

    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = f32x16{};
    // Partial row sum of the packed P values: this lane's 32 of each tile's
    // 64 keys (lane l ^ 32 holds the rest).
    float lsum = 0.f;
    float m = FIXED ? p.fixed_max : -__builtin_inff();

    auto s_mfma = [&](f32x16 (&sc)[2], uint32_t kb) {
      const uint8_t *ks = smem + kb * kKBytes;
      sc[0] = f32x16{};
      sc[1] = f32x16{};
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
      float mq[4] = {sc[0][0], sc[0][1], sc[1][0], sc[1][1]};
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 2; r < 16; ++r)
          mq[2 * j + (r & 1)] = fmaxf(mq[2 * j + (r & 1)], sc[j][r]);
      float lo, hi;
      half_pair(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3])), lo, hi);
      return fmaxf(lo, hi) * c;
    };
    // Lazy rescale: raise the running max only when it grows by > 8 (log2).
    auto update_max = [&](float mx) {
      if constexpr (!FIXED) {
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
      }
    };
    // Element pair i of P = exp2(s*c - m), packed to 16 bits and summed.
    auto p_pair = [&](const f32x16 (&sc)[2], u32x4 (&pf)[2][2], int i) {
      const int j = i >> 3, r = (2 * i) & 15;
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][r], c, -m));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][r + 1], c, -m));
      const uint32_t w = pack2<DT>(p0, p1);
      pf[j][r >> 3][(r & 7) >> 1] = w;
      lsum = dot2_ones<DT>(w, lsum);
      return w;
    };
    auto vfrag_at = [&](uint32_t vb, int i) {  // i = 4*(2*j + sl) + dt
      const int g = i >> 2, dt = i & 3;
      const uint8_t *a = vt0 + vb * kVt4Bytes + (dt * 32 + kr) * kVt4Pitch + (16 * g + 8 * half) * 2;
      const u32x2 lo = *reinterpret_cast<const u32x2 *>(a);
      const u32x2 hi = *reinterpret_cast<const u32x2 *>(a + 8);
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
    // O^T += V^T . P^T over 4 d-tiles x 4 key slices (V^T buffer vb).
    auto pv_mfma = [&](const u32x4 (&pf)[2][2], uint32_t vb) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        o[i & 3] = mfma32x32x16<DT>(vfrag_at(vb, i), pf[i >> 3][(i >> 2) & 1], o[i & 3]);
    };

    // Phase 1: S(t+1) = K(t+1) . Q^T (16 MFMAs) with P(t) (one element pair
    // per MFMA).  LDS fragment reads run 4 steps ahead.
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
        pin(p_pair(sc, pf, i));
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // Phase 2: O^T += V(t)^T . P(t)^T (16 MFMAs) with the row max of S(t+1)
    // (online mode) and the transpose of V(t+1) into the other V^T buffer.
    // Returns the scaled row max of S(t+1).
    auto phase2 = [&](const u32x4 (&pf)[2][2], uint32_t vb, const f32x16 (&sn)[2]) {
      u32x4 vf[16];
      float mx = -__builtin_inff();
      uint32_t tr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        vf[i] = vfrag_at(vb, i);
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        if (q + 4 < 16)
          vf[q + 4] = vfrag_at(vb, q + 4);
        o[q & 3] = mfma32x32x16<DT>(vf[q], pf[q >> 3][(q >> 2) & 1], o[q & 3]);
        if constexpr (!FIXED) {
          mx = __builtin_fmaxf(__builtin_fmaxf(mx, sn[q >> 3][(2 * q) & 15]),
                               sn[q >> 3][((2 * q) & 15) + 1]);
          pin(mx);
        }
        // Transpose: dword e = q / 4; k: 0 lo01, 1 lo23, 2 hi01, 3 hi23.
        const int e = q >> 2, k = q & 3;
        const int a = (k & 1) ? 3 : 1, b2 = (k & 1) ? 2 : 0;
        tr[k] = __builtin_amdgcn_perm(vr[a][e], vr[b2][e], (k & 2) ? 0x07060302u : 0x05040100u);
        pin(tr[k]);
        // Dword e of the transpose is complete: store its two V^T rows (the
        // buffer's last reader, PV(t-1), finished before the last barrier).
        if (k == 3)
          store_vt_rows(vb ^ 1, e, tr[0], tr[1], tr[2], tr[3]);
        __builtin_amdgcn_sched_barrier(0);
      }
      float lo, hi;
      half_pair(mx, lo, hi);
      return fmaxf(lo, hi) * c;
    };

    // ---- software pipeline over key tiles ----------------------------------
    // Iteration t: the matrix pipe computes S(t+1) while the VALU turns S(t)
    // into P(t) (phase 1), then O += V(t) P(t) while the VALU reduces S(t+1)
    // to its row max and transposes V(t+1) (phase 2).  K(t+2) and V(t+1)
    // are loaded during iteration t into the buffers K(t) and V(t-1) left.
    // The loop is unrolled by two with the score arrays swapping roles.
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
    auto iteration = [&](int t, uint32_t cur, const f32x16 (&sc)[2], f32x16 (&sn)[2]) {
      load_v(t + 1);
      if (t + 2 < ntiles)
        issue_k(cur, t + 2);
      phase1(sn, cur ^ 1, sc, pf);
      mask(sn, t + 1);
      const float mx = phase2(pf, cur, sn);
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
#pragma unroll
      for (int i = 0; i < 16; ++i)
        p_pair(sb, pf, i);
      pv_mfma(pf, 1);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        p_pair(sa, pf, i);
      pv_mfma(pf, 0);
    }

    // Normalise and store O[my_q][d], d = 32*dt + 8*(r/4) + 4*half + r%4.
    float s_lo, s_hi;
    half_pair(lsum, s_lo, s_hi);
    const float total = s_lo + s_hi;
    const float inv = total > 0.f ? 1.0f / total : 0.f;
    if (p.lse != nullptr && half == 0 && my_q < p.seq_q)
      p.lse[(size_t)bh * p.seq_q + my_q] = (m + __builtin_log2f(total)) * kLn2;
    // Staged through this wave's own K DMA rows of the two ring tiles (4 KiB
    // each, row r in tile r / 16; no wave reads K after the last barrier) so
    // that each store writes 4 whole 256-byte rows, as in fwd_pp_cta.
    {
      const uint32_t r = lane & 31;
      const uint32_t wb = lds0 + wave * 4096;
      const uint32_t wrow = wb + (r >> 4) * kKBytes + (r & 15) * 256 + half * 8;
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
        const u32x4 v =
            lds_load16(wb + (rr >> 4) * kKBytes + (rr & 15) * 256 + ((c ^ (rr & 15)) << 4));
        if (qw + (int)rr < p.seq_q)
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(Oh + (size_t)(qw + rr) * kD + 8 * c));
      }
    }
    // The next pass refills both rings: every wave's reads of this pass are
    // done first.
    lds_barrier();
  }
}

template <int DT, bool FIXED>
__global__ __launch_bounds__(64 * kF4Waves, 2) void fwd4_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kF4Smem];
  fwd4_cta<DT, FIXED>(p, blockIdx.x, smem);
}

} // namespace attention
} // namespace wave
