// attention_bwd.hip -- flash-attention backward for gfx950, head_dim 128.
//
// Gradients of O = softmax(scale * Q K^T) V (optional causal mask key >
// query, grouped-query heads kv_head = q_head / (Hq / Hkv)) given dO, O and
// the forward's row log-sum-exp lse = ln sum_k exp(scale * q.k):
//   P   = exp(scale * Q K^T - lse)         (recomputed, never stored)
//   dV  = P^T dO                          (summed over a KV head's q heads)
//   dP  = dO V^T
//   dS  = P o (dP - delta),  delta = rowsum(dO o O)
//   dQ  = scale * dS K,      dK = scale * dS^T Q
// The reference has no backward; this is the standard flash-attention-2
// recomputation scheme, checked against a float64 CPU restatement of the
// formulas above (oracle.py fa_backward) that is itself checked against
// torch autograd.
//
// Three kernels, deterministic (no atomics):
//  * bwd_delta_kernel: -delta[row] = -sum_d dO[row][d] * O[row][d] in fp32
//    (into the caller's scratch).
//  * bwd_kv_pp_kernel (seq a multiple of 128): one CTA (8 waves, two groups
//    of 4 one segment apart) per 128-key block of one KV head; it loops over
//    the query blocks of every q head of the group (causal: the blocks at or
//    after the key block), with each block's Q, dO, lse and -delta arriving
//    by LDS DMA, and accumulates dK, dV in registers.  bwd_kv_kernel (one
//    CTA of 4 waves per 64-key block, Q and dO staged through registers)
//    covers seq = 64 (mod 128).
//  * bwd_q_kernel: one CTA per 64-query block of one q head; it loops over
//    the key blocks (causal: up to the diagonal) and accumulates dQ.
// Every product is an "NT" product C[m][n] = sum_k A[m][k] B[n][k] of 32x32
// tiles on v_mfma_f32_32x32x16.  The operands fixed for a CTA (K, V in the
// dK/dV kernels; Q, dO in the dQ kernel) are held as MFMA fragments in
// registers; the rest are read as 16-byte row chunks from LDS.  Operands
// needed K-contiguous the other way (Q^T, dO^T, K^T as the B operand of
// dK, dV, dQ) are read from the row-major Q, dO, K tiles by transposing LDS
// reads (ds_read_b64_tr_b16), and P^T / dS^T (dS for dQ) go through LDS
// between the score products and the gradient products.  LDS tiles are
// unpadded with XOR-swizzled 16-byte chunks (swz below), conflict-free for
// every read these kernels make: 130 KiB (bwd_kv_pp_kernel, one CTA per
// CU), 48 KiB (bwd_kv_kernel) and 40 KiB (dQ) of LDS, two CTAs per CU
// (register-bound).
#include "attention.hpp"
#include "wave_common.hpp"

namespace wave {
namespace attention {

namespace {

constexpr int kBD = 128;               // head dim
constexpr int kBlk = 64;               // query or key rows per block
constexpr int kWide = kBlk * 256;      // [64][128] 16-bit tile: 16 KiB
constexpr int kNarrowS = kBlk * 128;   // [64][64] tile: 8 KiB
constexpr float kLog2eB = 1.4426950408889634f;

// Byte offset of (row r, byte b) in a tile of ROWB-byte rows: 16-byte chunk
// c of row r at c ^ swz(r).  256-byte rows: swz(r) = 4 (r % 4) + (r / 4) % 4,
// under which both access patterns of these tiles are free of LDS bank
// conflicts on gfx950 (measured: a 16-byte row-fragment read of 32
// consecutive rows, and the transposing 8-byte reads of tr_frag, which
// touch rows k .. k+3 and k+8 .. k+11 in one instruction; c ^ (r % 16)
// served the first but made the second 2.6x slower).  128-byte rows:
// swz(r) = (r / 2) % 8.
template <int ROWB> __device__ __forceinline__ uint32_t swz(uint32_t r) {
  return ROWB == 256 ? (((r & 3u) << 2) | ((r >> 2) & 3u)) : ((r >> 1) & 7u);
}
template <int ROWB> __device__ __forceinline__ uint32_t toff(uint32_t r, uint32_t b) {
  return r * ROWB + ((((b >> 4) ^ swz<ROWB>(r))) << 4) + (b & 15u);
}

struct BwdParams {
  const uint16_t *Q, *K, *V, *O, *dO;
  const float *lse;
  float *delta;
  uint16_t *dQ, *dK, *dV;
  int batch, q_heads, kv_heads, seq;
  int causal;
  float scale;        // softmax scale
  float scale_log2;   // scale * log2(e)
  float inv_scale;    // 1 / scale
};

// Two NT products over K = 128 that share their A rows: c0 += A0 . b0^T and
// c1 += A1 . b1^T, with A rows a0 .. a0+31 of two [rows][128] 16-bit LDS
// tiles (256-byte rows) and B as per-slice register fragments (lane l: row
// l % 32 of B, elements 16 kk + 8 (l / 32) .. +8).  The two accumulation
// chains alternate (each MFMA's predecessor on its chain is two MFMAs
// back), and each A fragment is read kPF slices ahead of its MFMA.
template <int DT, int kPF = 2>
__device__ __forceinline__ void mma2_nt_reg(f32x16 &c0, const uint8_t *A0, const u32x4 (&b0)[8],
                                            f32x16 &c1, const uint8_t *A1, const u32x4 (&b1)[8],
                                            uint32_t a0) {
  const uint32_t lane = threadIdx.x & 63, ra = a0 + (lane & 31);
  const uint32_t sw = (lane >> 5) ^ swz<256>(ra);
  auto frag = [&](const uint8_t *A, int kk) {
    return *reinterpret_cast<const u32x4 *>(A + ra * 256 + (((2u * kk) ^ sw) << 4));
  };
  u32x4 f0[8], f1[8];
#pragma unroll
  for (int kk = 0; kk < kPF; ++kk) {
    f0[kk] = frag(A0, kk);
    f1[kk] = frag(A1, kk);
  }
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    if (kk + kPF < 8) {
      f0[kk + kPF] = frag(A0, kk + kPF);
      f1[kk + kPF] = frag(A1, kk + kPF);
    }
    c0 = mfma32x32x16<DT>(f0[kk], b0[kk], c0);
    c1 = mfma32x32x16<DT>(f1[kk], b1[kk], c1);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The B operand of a gradient product from a row-major [K][128] 16-bit LDS
// tile R of 256-byte rows, columns c0 .. c0+31, slice kk (K rows 16 kk ..
// 16 kk + 15), by transposing reads (ds_read_b64_tr_b16: in each 16-lane
// group source lane 4a + p addresses R[k + a][c + 4p .. +3] and lane i then
// holds R[k .. k+3][c + i]).  Lane l reads rows 16 kk + 8 (l / 32) + 4 r +
// (l >> 2) % 4, columns c0 + 16 ((l >> 4) % 2) + 4 (l % 4), r = 0, 1: the 8
// K values of its B fragment, in order.  So no transposed copy of R is
// needed.
__device__ __forceinline__ u32x4 tr_frag(uint32_t rbase, int kk, uint32_t c0) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s4 lds_s4;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t rb = 16 * kk + 8 * (lane >> 5) + ((lane >> 2) & 3);
  const uint32_t cb = 2 * c0 + 32 * ((lane >> 4) & 1) + 8 * (lane & 3);
  const u32x2 lo = __builtin_bit_cast(
      u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4 *)(uintptr_t)(rbase + toff<256>(rb, cb))));
  const u32x2 hi = __builtin_bit_cast(
      u32x2,
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4 *)(uintptr_t)(rbase + toff<256>(rb + 4, cb))));
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

// 2 NT gradient chains over K = 64 (4 slices): for tile pair i < NT and
// t = 0, 1, acc[2i + t] += A_i . R_i[:, c_t .. c_t + 31], with A_i rows
// a0 .. a0+31 of a 128-byte-row LDS tile and R_i a row-major [64][128] LDS
// tile read transposed (tr_frag).  Steps (slice kk, pair i) run in order,
// two MFMAs each, and the fragments of step n + GPF are read before the
// MFMAs of step n.
template <int DT, int NT, int GPF = 1>
__device__ __forceinline__ void mma_grad(f32x16 (&acc)[2 * NT], const uint8_t *const (&A)[NT],
                                         uint32_t a0, const uint8_t *const (&R)[NT],
                                         uint32_t c0, uint32_t c1) {
  const uint32_t lane = threadIdx.x & 63, ra = a0 + (lane & 31);
  const uint32_t sw = (lane >> 5) ^ swz<128>(ra);
  constexpr int NS = 4 * NT, NB = GPF + 1;
  u32x4 fa[NB], fb[NB][2];
  auto load = [&](int n, int slot) {
    const int kk = n / NT, i = n % NT;
    fa[slot] = *reinterpret_cast<const u32x4 *>(A[i] + ra * 128 + (((2u * kk) ^ sw) << 4));
    fb[slot][0] = tr_frag(lds_addr(R[i]), kk, c0);
    fb[slot][1] = tr_frag(lds_addr(R[i]), kk, c1);
  };
#pragma unroll
  for (int n = 0; n < GPF && n < NS; ++n)
    load(n, n % NB);
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    if (n + GPF < NS)
      load(n + GPF, (n + GPF) % NB);
    const int i = n % NT;
    acc[2 * i] = mfma32x32x16<DT>(fa[n % NB], fb[n % NB][0], acc[2 * i]);
    acc[2 * i + 1] = mfma32x32x16<DT>(fa[n % NB], fb[n % NB][1], acc[2 * i + 1]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// One gradient product over K = 64 (4 slices) for 64 rows: acc[2a + t] +=
// A[32a .. 32a+31] . R[:, c_t .. c_t + 31] (a, t = 0, 1), A a 128-byte-row
// LDS tile (rows r and r + 32 share swz<128>), R a row-major [64][128] tile
// read transposed.  Per slice two A and two B fragments feed four MFMAs:
// 1 KiB of LDS reads an MFMA, against 1.5 KiB for mma_grad's two products
// of 32 rows each (whose A fragment feeds two MFMAs but each B one).  The
// fragments of slice kk + GPF are read before the MFMAs of slice kk.
template <int DT, int GPF = 1>
__device__ __forceinline__ void mma_grad_rows2(f32x16 (&acc)[4], const uint8_t *A,
                                               const uint8_t *R, uint32_t c0, uint32_t c1) {
  const uint32_t lane = threadIdx.x & 63, ra = lane & 31;
  const uint32_t sw = (lane >> 5) ^ swz<128>(ra);
  constexpr int NB = GPF + 1;
  u32x4 fa[NB][2], fb[NB][2];
  auto load = [&](int kk, int slot) {
    const uint32_t cb = ((2u * kk) ^ sw) << 4;
    fa[slot][0] = *reinterpret_cast<const u32x4 *>(A + ra * 128 + cb);
    fa[slot][1] = *reinterpret_cast<const u32x4 *>(A + (ra + 32) * 128 + cb);
    fb[slot][0] = tr_frag(lds_addr(R), kk, c0);
    fb[slot][1] = tr_frag(lds_addr(R), kk, c1);
  };
#pragma unroll
  for (int kk = 0; kk < GPF && kk < 4; ++kk)
    load(kk, kk % NB);
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    if (kk + GPF < 4)
      load(kk + GPF, (kk + GPF) % NB);
    const int sl = kk % NB;
    acc[0] = mfma32x32x16<DT>(fa[sl][0], fb[sl][0], acc[0]);
    acc[1] = mfma32x32x16<DT>(fa[sl][0], fb[sl][1], acc[1]);
    acc[2] = mfma32x32x16<DT>(fa[sl][1], fb[sl][0], acc[2]);
    acc[3] = mfma32x32x16<DT>(fa[sl][1], fb[sl][1], acc[3]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// MFMA fragments of 32 rows of a [rows][128] global block (row0 = the
// lane's row): lane l holds elements 16 kk + 8 (l / 32) .. +8 for kk < 8.
__device__ __forceinline__ void load_frags(const uint16_t *row, u32x4 (&f)[8]) {
  const uint32_t lane = threadIdx.x & 63;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    f[kk] = *reinterpret_cast<const u32x4 *>(row + 16 * kk + 8 * (lane >> 5));
}

// A [64][128] block of rows (row stride 128 elements) in flight through
// registers: fetch() issues the global loads, put() writes the rows to LDS
// (wide tile R).
// Thread t handles row pairs x 16-byte chunks: unit u = t + 256*i, row pair
// u / 16, chunk u % 16.
struct BlockRegs {
  u32x4 a[2], b[2];
  __device__ __forceinline__ void fetch(const uint16_t *src) {
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t u = t + 256u * i, rp = u >> 4, c = u & 15u;
      a[i] = *reinterpret_cast<const u32x4 *>(src + (size_t)(2 * rp) * kBD + 8 * c);
      b[i] = *reinterpret_cast<const u32x4 *>(src + (size_t)(2 * rp + 1) * kBD + 8 * c);
    }
  }
  __device__ __forceinline__ void put(uint8_t *R) const {
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t u = t + 256u * i, rp = u >> 4, c = u & 15u;
      *reinterpret_cast<u32x4 *>(R + toff<256>(2 * rp, 16 * c)) = a[i];
      *reinterpret_cast<u32x4 *>(R + toff<256>(2 * rp + 1, 16 * c)) = b[i];
    }
  }
};

// CTA id -> work index with the CTAs of one head on one XCD (the
// dispatcher places workgroup i on XCD i % 8), so they share that head's
// K/V or Q/dO rows in the XCD's L2.
__device__ __forceinline__ int xcd_pid(int raw, int total) {
  return (total & 7) == 0 ? (raw & 7) * (total >> 3) + (raw >> 3) : raw;
}

// Store a 32x32 fp32 accumulator tile (rows row0.., columns col0..) of a
// [rows][128] 16-bit output, times mul.
template <int DT>
__device__ __forceinline__ void store_tile32(uint16_t *dst, int row0, int col0, const f32x16 &acc,
                                             float mul) {
  const uint32_t lane = threadIdx.x & 63;
  const int col = col0 + (int)(lane & 31);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = row0 + 8 * (r >> 2) + 4 * (int)(lane >> 5) + (r & 3);
    dst[(size_t)row * kBD + col] = to_bits<DT>(acc[r] * mul);
  }
}

} // namespace

// delta[row] = -sum_d dO[row][d] * O[row][d] (stored negated: it is the
// start value of the dP accumulators); 16 lanes per row, 8 elements a lane.
template <int DT>
__global__ __launch_bounds__(256) void bwd_delta_kernel(BwdParams p, int rows) {
  const int row = (int)(blockIdx.x * 16 + (threadIdx.x >> 4));
  const int c = threadIdx.x & 15;
  float s = 0.f;
  if (row < rows) {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(p.dO + (size_t)row * kBD + 8 * c);
    const u32x4 b = *reinterpret_cast<const u32x4 *>(p.O + (size_t)row * kBD + 8 * c);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s += from_bits<DT>((uint16_t)(a[e] & 0xffffu)) * from_bits<DT>((uint16_t)(b[e] & 0xffffu));
      s += from_bits<DT>((uint16_t)(a[e] >> 16)) * from_bits<DT>((uint16_t)(b[e] >> 16));
    }
  }
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1)
    s += __shfl_xor(s, m, 16);
  if (row < rows && c == 0)
    p.delta[row] = -s;
}

// dK, dV of one 64-key block of one KV head.
template <int DT, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void bwd_kv_kernel(BwdParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kWide + 2 * kNarrowS];
  uint8_t *sQ = smem, *sdO = sQ + kWide, *sPt = sdO + kWide, *sdSt = sPt + kNarrowS;
  const int nb = p.seq / kBlk;
  const int pid = xcd_pid((int)blockIdx.x, (int)gridDim.x);
  const int kb = pid % nb, bhk = pid / nb;
  const int b = bhk / p.kv_heads, hkv = bhk - b * p.kv_heads;
  const int group = p.q_heads / p.kv_heads;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const size_t kv_off = ((size_t)bhk * p.seq + (size_t)kb * kBlk) * kBD;

  // Score tiles: wave w computes S[q][key] for q half w&1, key half w>>1;
  // lane l holds key kh2*32 + l%32 and queries qh2*32 + 8g + 4(l/32) + e.
  const int qh2 = wave & 1, kh2 = wave >> 1;
  // Gradient tiles: key half w&1, d quarters 2(w>>1), 2(w>>1)+1.
  const int kh = wave & 1, dq = wave >> 1;
  // K and V rows of this wave's key half as B fragments, for the whole CTA.
  u32x4 kf[8], vf[8];
  load_frags(p.K + kv_off + (size_t)(kh2 * 32 + (lane & 31)) * kBD, kf);
  load_frags(p.V + kv_off + (size_t)(kh2 * 32 + (lane & 31)) * kBD, vf);
  // Gradient accumulators: dV columns (2 dq) * 32 and (2 dq + 1) * 32, then
  // dK's.
  f32x16 g[4] = {f32x16{}, f32x16{}, f32x16{}, f32x16{}};
  const int key = kb * kBlk + kh2 * 32 + (int)(lane & 31);
  // Work items: (q head h of the group, query block qb), h major (causal:
  // the blocks at or after the key block); the next item's Q and dO rows
  // and its lse / delta are fetched while this one's products run.
  const int qb0 = CAUSAL ? kb : 0, items = group * (nb - qb0);
  auto rows_of = [&](int h, int q) {  // first row of item (h, q) in [B*Hq*S]
    return ((size_t)b * p.q_heads + (size_t)hkv * group + h) * p.seq + (size_t)q * kBlk;
  };
  // This wave's score rows of an item: lse and -delta of rows
  // qh2*32 + 8 g + 4 (l / 32) + e as the accumulators' start values.
  f32x16 s, dp;
  auto load_stats = [&](size_t rb) {
    const size_t r0 = rb + qh2 * 32 + 4 * (lane >> 5);
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const f32x4 a = *reinterpret_cast<const f32x4 *>(p.lse + r0 + 8 * g4);
      const f32x4 d = *reinterpret_cast<const f32x4 *>(p.delta + r0 + 8 * g4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s[4 * g4 + e] = a[e];
        dp[4 * g4 + e] = d[e];
      }
    }
  };
  int h = 0, qb = qb0;
  BlockRegs rq, rdo;
  rq.fetch(p.Q + rows_of(0, qb0) * kBD);
  rdo.fetch(p.dO + rows_of(0, qb0) * kBD);
  load_stats(rows_of(0, qb0));
  for (int it = 0; it < items; ++it) {
    int hn = h, qbn = qb + 1;
    if (qbn == nb) {
      qbn = qb0;
      ++hn;
    }
    const bool more = it + 1 < items;
    __syncthreads();  // the previous item's readers are done
    rq.put(sQ);
    rdo.put(sdO);
    if (more) {
      rq.fetch(p.Q + rows_of(hn, qbn) * kBD);
      rdo.fetch(p.dO + rows_of(hn, qbn) * kBD);
    }
    // The score accumulator starts at -lse / scale and dP's at -delta, so
    // exp2(c * s) = P and dp = dP - delta after the products.
#pragma unroll
    for (int r = 0; r < 16; ++r)
      s[r] *= -p.inv_scale;
    __syncthreads();
    mma2_nt_reg<DT>(s, sQ, kf, dp, sdO, vf, qh2 * 32);
    // P and dS; P^T / dS^T rows = keys, 4 consecutive queries per store.
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      float pv[4], dsv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * g4 + e;
        const int q = qb * kBlk + qh2 * 32 + 8 * g4 + 4 * (int)(lane >> 5) + e;
        float pr = __builtin_amdgcn_exp2f(s[r] * p.scale_log2);
        if (CAUSAL && key > q)
          pr = 0.f;
        pv[e] = pr;
        dsv[e] = pr * dp[r];
      }
      const uint32_t off =
          toff<128>(kh2 * 32 + (lane & 31), 2 * (qh2 * 32 + 8 * g4 + 4 * (lane >> 5)));
      *reinterpret_cast<u32x2 *>(sPt + off) = u32x2{pack2<DT>(pv[0], pv[1]), pack2<DT>(pv[2], pv[3])};
      *reinterpret_cast<u32x2 *>(sdSt + off) =
          u32x2{pack2<DT>(dsv[0], dsv[1]), pack2<DT>(dsv[2], dsv[3])};
    }
    __syncthreads();
    const uint8_t *const ga[2] = {sPt, sdSt};
    const uint8_t *const gr[2] = {sdO, sQ};
    mma_grad<DT, 2>(g, ga, kh * 32, gr, (2 * dq) * 32, (2 * dq + 1) * 32);
    if (more)
      load_stats(rows_of(hn, qbn));
    h = hn;
    qb = qbn;
  }
  uint16_t *dK = p.dK + kv_off, *dV = p.dV + kv_off;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    store_tile32<DT>(dV, kh * 32, (2 * dq + t) * 32, g[t], 1.f);
    store_tile32<DT>(dK, kh * 32, (2 * dq + t) * 32, g[2 + t], p.scale);
  }
}

// dK, dV of a 128-key block of one KV head as two groups of four waves:
// group g (waves 4g .. 4g+3) owns keys 64 g .. 64 g + 63 of the block and
// does for them what bwd_kv_kernel does for its 64 keys (same wave roles,
// same products), on the same work items.  The groups share each item's Q
// and dO rows and its rows' lse and -delta, which arrive by LDS DMA into a
// 3-buffer ring (so no global load is waited for inside the loop), and run
// one segment apart ("ping-pong"), so that on every SIMD one wave's MFMAs
// run next to the other group's softmax:
//
//   segment    2i              2i+1            2i+2
//   group 0    M2(i-1) M1(i)   SM(i)           M2(i) M1(i+1)
//   group 1    SM(i-1)         M2(i-1) M1(i)   SM(i)
//
// M1(i): S and dP of item i (A fragments from its Q / dO buffer); SM(i): P
// and dS of item i into the group's P^T / dS^T tiles; M2(i): dV, dK += the
// products of those tiles with Q / dO of item i (transposing reads).  Every
// segment ends with a workgroup barrier (2 * items + 2 of them for every
// wave).  Buffers: item i's Q / dO sit in ring slot i % 3, read from
// segment 2i (group 0's M1(i)) to 2i+3 (group 1's M2(i)); group 1's waves
// issue the DMA of item j+1 at the start of segment 2j (their SM(j-1),
// shorter than group 0's matrix segment beside it, which the DMA issues
// used to lengthen: 4-5 % of the kernel's time), after slot (j+1) % 3's
// previous item (j-2) was last read in segment 2j-1, and every wave waits
// for it at the end of segment 2j+1.  A group's P^T / dS^T are written in
// SM(i) and read in M2(i), the next segment of that group.
#ifndef WAVE_BWD_PF
#define WAVE_BWD_PF 3  // score products: A fragments read this many slices ahead
#endif
#ifndef WAVE_BWD_GPF
#define WAVE_BWD_GPF 2  // gradient products: fragments read this many steps ahead
#endif
template <int DT, bool CAUSAL>
__global__ __launch_bounds__(512, 1) void bwd_kv_pp_kernel(BwdParams p) {
  // One ring slot: an item's Q and dO rows (32 KiB), then its 64 rows' lse
  // and -delta (256 B each).
  constexpr uint32_t kStats = 2 * kWide, kQD = kStats + 512;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[3 * kQD + 4 * kNarrowS];
  const int nb = p.seq / kBlk, nkb = nb / 2;
  const int pid = xcd_pid((int)blockIdx.x, (int)gridDim.x);
  const int kb2 = pid % nkb, bhk = pid / nkb;
  const int b = bhk / p.kv_heads, hkv = bhk - b * p.kv_heads;
  const int group = p.q_heads / p.kv_heads;
  const uint32_t wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const uint32_t grp = wave >> 2, wg = wave & 3;
  const int kb = 2 * kb2 + (int)grp;  // this group's 64-key block
  const size_t kv_off = ((size_t)bhk * p.seq + (size_t)kb * kBlk) * kBD;
  uint8_t *sPt = smem + 3 * kQD + grp * 2 * kNarrowS, *sdSt = sPt + kNarrowS;
  const uint32_t lds0 = lds_addr(smem);
  // Wave roles within the group, as in bwd_kv_kernel.
  // Score products: query half qh2, key half kh2.  Gradient products: wave
  // role 0 accumulates dV, role 1 dK, each for all 64 keys of the group and
  // d columns 64 dq .. 64 dq + 63.
  const int qh2 = wg & 1, kh2 = wg >> 1, role = wg & 1, dq = wg >> 1;
  u32x4 kf[8], vf[8];
  load_frags(p.K + kv_off + (size_t)(kh2 * 32 + (lane & 31)) * kBD, kf);
  load_frags(p.V + kv_off + (size_t)(kh2 * 32 + (lane & 31)) * kBD, vf);
  f32x16 g[4] = {f32x16{}, f32x16{}, f32x16{}, f32x16{}};
  const int key = kb * kBlk + kh2 * 32 + (int)(lane & 31);
  // Work items (q head h, query block qb), h major; causal: the blocks at
  // or after group 0's key block (group 1's first one is wholly masked).
  const int qb0 = CAUSAL ? 2 * kb2 : 0, items = group * (nb - qb0);
  struct Cursor {
    int h, qb;
  };
  auto advance = [&](Cursor &c) {
    if (++c.qb == nb) {
      c.qb = qb0;
      ++c.h;
    }
  };
  auto rows_of = [&](const Cursor &c) {
    return ((size_t)b * p.q_heads + (size_t)hkv * group + c.h) * p.seq + (size_t)c.qb * kBlk;
  };
  // DMA of an item into ring slot `slot`, issued by group 1's waves: wave
  // wg fills Q and dO rows 16 wg .. 16 wg + 15 (four 1 KiB windows each),
  // lane l row 4 win + l / 16, slot l % 16, which holds chunk (l % 16) ^
  // swz(row); waves wg = 0 and 1 add the rows' lse and -delta (256 B each,
  // 4 bytes a lane).
  auto dma_item = [&](const Cursor &c, uint32_t slot) {
    const size_t rb = rows_of(c);
    const uint32_t l = lds0 + slot * kQD;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t win = 4 * wg + j, r = 4 * win + (lane >> 4);
      const uint32_t off = r * 256 + (((lane & 15) ^ swz<256>(r)) << 4);
      dma16(l + win * 1024, p.Q + rb * kBD, off);
      dma16(l + kWide + win * 1024, p.dO + rb * kBD, off);
    }
    if (wg < 2)
      dma4(l + kStats + wg * 256, wg == 0 ? (const void *)(p.lse + rb) : (const void *)(p.delta + rb),
           4 * lane);
  };
  f32x16 s, dp;
  // This wave's score rows' lse and -delta (rows qh2*32 + 8 g + 4 (l / 32)
  // + e) from the item's ring slot: the accumulators' start values.
  auto load_stats = [&](const uint8_t *q) {
    const float *r0 = reinterpret_cast<const float *>(q + kStats) + qh2 * 32 + 4 * (lane >> 5);
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const f32x4 a = *reinterpret_cast<const f32x4 *>(r0 + 8 * g4);
      const f32x4 d = *reinterpret_cast<const f32x4 *>(r0 + 64 + 8 * g4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s[4 * g4 + e] = a[e];
        dp[4 * g4 + e] = d[e];
      }
    }
  };
  Cursor dmac{0, qb0}, cur{0, qb0};
  if (grp == 1)
    dma_item(dmac, 0);
  advance(dmac);
  vm_wait_barrier();
  const int nseg = 2 * items + 2;
  for (int sg = 0; sg < nseg; ++sg) {
    if ((sg & 1) == 0 && (sg >> 1) + 1 < items) {
      if (grp == 1)
        dma_item(dmac, (uint32_t)(((sg >> 1) + 1) % 3));
      advance(dmac);
    }
    const int ls = sg - (int)grp;
    if (ls >= 0 && ls <= 2 * items) {
      const int i = ls >> 1;
      if ((ls & 1) == 0) {
        if (i >= 1) {  // M2(i-1)
          const uint8_t *q = smem + ((i - 1) % 3) * kQD;
          // dV += P^T dO, dK += dS^T Q (scaled at the store).
          mma_grad_rows2<DT, WAVE_BWD_GPF>(g, role ? sdSt : sPt, role ? q : q + kWide,
                                           (2 * dq) * 32, (2 * dq + 1) * 32);
        }
        if (i < items) {  // M1(i): S starts at -lse / scale, dP at -delta
          const uint8_t *q = smem + (i % 3) * kQD;
          load_stats(q);
#pragma unroll
          for (int r = 0; r < 16; ++r)
            s[r] *= -p.inv_scale;
          mma2_nt_reg<DT, WAVE_BWD_PF>(s, q, kf, dp, q + kWide, vf, qh2 * 32);
        }
      } else {  // SM(i)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          float pv[4], dsv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g4 + e;
            const int q = cur.qb * kBlk + qh2 * 32 + 8 * g4 + 4 * (int)(lane >> 5) + e;
            float pr = __builtin_amdgcn_exp2f(s[r] * p.scale_log2);
            if (CAUSAL && key > q)
              pr = 0.f;
            pv[e] = pr;
            dsv[e] = pr * dp[r];
          }
          const uint32_t off =
              toff<128>(kh2 * 32 + (lane & 31), 2 * (qh2 * 32 + 8 * g4 + 4 * (lane >> 5)));
          *reinterpret_cast<u32x2 *>(sPt + off) =
              u32x2{pack2<DT>(pv[0], pv[1]), pack2<DT>(pv[2], pv[3])};
          *reinterpret_cast<u32x2 *>(sdSt + off) =
              u32x2{pack2<DT>(dsv[0], dsv[1]), pack2<DT>(dsv[2], dsv[3])};
        }
        advance(cur);
      }
    }
    if (sg & 1)
      vm_wait_barrier();  // the DMA of item (sg >> 1) + 1 has landed
    else
      lds_barrier();
  }
  uint16_t *dst = (role ? p.dK : p.dV) + kv_off;
  const float sc = role ? p.scale : 1.f;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int t = 0; t < 2; ++t)
      store_tile32<DT>(dst, a * 32, (2 * dq + t) * 32, g[2 * a + t], sc);
}

// dQ of one 64-query block of one q head.
#ifndef WAVE_BWDQ_PF
#define WAVE_BWDQ_PF 2  // score products: A fragments read this many slices ahead
#endif
#ifndef WAVE_BWDQ_GPF
#define WAVE_BWDQ_GPF 1  // dQ product: fragments read this many steps ahead
#endif
template <int DT, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void bwd_q_kernel(BwdParams p) {
  // K and V rows of a key block arrive by LDS DMA into a 2-slot ring: the
  // DMA of block kb + 1 goes into the slot block kb - 1 used, after the
  // barrier that starts iteration kb, and is waited for at the barrier that
  // starts iteration kb + 1.
  constexpr uint32_t kKV = 2 * kWide;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * kKV + kNarrowS];
  uint8_t *sdS = smem + 2 * kKV;
  const int nb = p.seq / kBlk;
  const int pid = xcd_pid((int)blockIdx.x, (int)gridDim.x);
  const int qb = pid % nb, bh = pid / nb;
  const int b = bh / p.q_heads, hq = bh - b * p.q_heads;
  const int hkv = hq / (p.q_heads / p.kv_heads);
  const uint32_t wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const size_t q_off = ((size_t)bh * p.seq + (size_t)qb * kBlk) * kBD;
  // Score tiles: wave w computes S^T[key][q] for key half w&1, q half w>>1;
  // lane l holds query qh2*32 + l%32 and keys kh2*32 + 8g + 4(l/32) + e.
  const int kh2 = wave & 1, qh2 = wave >> 1;
  // dQ tiles: q half w&1, d quarters 2(w>>1), 2(w>>1)+1.
  const int qh = wave & 1, dq = wave >> 1;
  // Q and dO rows of this wave's query half as B fragments, for the whole CTA.
  u32x4 qf[8], dof[8];
  load_frags(p.Q + q_off + (size_t)(qh2 * 32 + (lane & 31)) * kBD, qf);
  load_frags(p.dO + q_off + (size_t)(qh2 * 32 + (lane & 31)) * kBD, dof);
  const int q = qb * kBlk + qh2 * 32 + (int)(lane & 31);
  const size_t row = (size_t)bh * p.seq + q;
  const float l2 = p.lse[row] * kLog2eB, ndl = p.delta[row];  // -delta
  f32x16 dqa[2] = {f32x16{}, f32x16{}};
  const size_t kv_base = (size_t)(b * p.kv_heads + hkv) * p.seq * kBD;
  const int kb_end = CAUSAL ? qb + 1 : nb;
  const uint32_t lds0 = lds_addr(smem);
  // DMA of key block kb into ring slot kb % 2: wave w fills K and V rows
  // 16w .. 16w+15 (four 1 KiB windows each), lane l row 4 win + l / 16,
  // slot l % 16, which holds chunk (l % 16) ^ swz(row).
  auto dma_block = [&](int kb) {
    const size_t r0 = kv_base + (size_t)kb * kBlk * kBD;
    const uint32_t l = lds0 + (kb & 1) * kKV;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t win = 4 * wave + j, r = 4 * win + (lane >> 4);
      const uint32_t off = r * 256 + (((lane & 15) ^ swz<256>(r)) << 4);
      dma16(l + win * 1024, p.K + r0, off);
      dma16(l + kWide + win * 1024, p.V + r0, off);
    }
  };
  dma_block(0);
  for (int kb = 0; kb < kb_end; ++kb) {
    // Block kb's DMA has landed everywhere, and every wave is done with
    // iteration kb - 1's LDS reads (of the slot block kb + 1 takes, and of
    // dS, which this iteration rewrites).
    vm_wait_barrier();
    if (kb + 1 < kb_end)
      dma_block(kb + 1);
    const uint8_t *sK = smem + (kb & 1) * kKV, *sV = sK + kWide;
    f32x16 st = {}, dpt = {};
    mma2_nt_reg<DT, WAVE_BWDQ_PF>(st, sK, qf, dpt, sV, dof, kh2 * 32);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float dsv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * g + e;
        const int key = kb * kBlk + kh2 * 32 + 8 * g + 4 * (int)(lane >> 5) + e;
        float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(st[r], p.scale_log2, -l2));
        if (CAUSAL && key > q)
          pr = 0.f;
        dsv[e] = pr * (dpt[r] + ndl);
      }
      // dS row q, 4 consecutive keys.
      const uint32_t off =
          toff<128>(qh2 * 32 + (lane & 31), 2 * (kh2 * 32 + 8 * g + 4 * (lane >> 5)));
      *reinterpret_cast<u32x2 *>(sdS + off) =
          u32x2{pack2<DT>(dsv[0], dsv[1]), pack2<DT>(dsv[2], dsv[3])};
    }
    __syncthreads();
    const uint8_t *const ga[1] = {sdS};
    const uint8_t *const gr[1] = {sK};
    mma_grad<DT, 1, WAVE_BWDQ_GPF>(dqa, ga, qh * 32, gr, (2 * dq) * 32, (2 * dq + 1) * 32);
  }
  uint16_t *dQ = p.dQ + q_off;
#pragma unroll
  for (int t = 0; t < 2; ++t)
    store_tile32<DT>(dQ, qh * 32, (2 * dq + t) * 32, dqa[t], p.scale);
}

namespace {
template <int DT, bool CAUSAL>
hipError_t launch_bwd_dt(const BwdParams &p, hipStream_t stream) {
  const int rows = p.batch * p.q_heads * p.seq;
  hipLaunchKernelGGL((bwd_delta_kernel<DT>), dim3((rows + 15) / 16), dim3(256), 0, stream, p,
                     rows);
  const int nb = p.seq / kBlk;
  if (nb % 2 == 0)
    hipLaunchKernelGGL((bwd_kv_pp_kernel<DT, CAUSAL>), dim3(nb / 2 * p.batch * p.kv_heads),
                       dim3(512), 0, stream, p);
  else
    hipLaunchKernelGGL((bwd_kv_kernel<DT, CAUSAL>), dim3(nb * p.batch * p.kv_heads), dim3(256),
                       0, stream, p);
  hipLaunchKernelGGL((bwd_q_kernel<DT, CAUSAL>), dim3(nb * p.batch * p.q_heads), dim3(256), 0,
                     stream, p);
  return hipGetLastError();
}
} // namespace

hipError_t launch_bwd(const BwdArgs &a, hipStream_t stream) {
  BwdParams p{};
  p.Q = static_cast<const uint16_t *>(a.Q);
  p.K = static_cast<const uint16_t *>(a.K);
  p.V = static_cast<const uint16_t *>(a.V);
  p.O = static_cast<const uint16_t *>(a.O);
  p.dO = static_cast<const uint16_t *>(a.dO);
  p.lse = a.lse;
  p.delta = a.delta;
  p.dQ = static_cast<uint16_t *>(a.dQ);
  p.dK = static_cast<uint16_t *>(a.dK);
  p.dV = static_cast<uint16_t *>(a.dV);
  p.batch = a.batch;
  p.q_heads = a.q_heads;
  p.kv_heads = a.kv_heads;
  p.seq = a.seq;
  p.causal = a.causal;
  p.scale = a.scale > 0.f ? a.scale : 1.0f / __builtin_sqrtf((float)kBD);
  p.scale_log2 = p.scale * kLog2eB;
  p.inv_scale = 1.0f / p.scale;
  if (a.dtype == kF16)
    return a.causal ? launch_bwd_dt<kF16, true>(p, stream) : launch_bwd_dt<kF16, false>(p, stream);
  return a.causal ? launch_bwd_dt<kBF16, true>(p, stream) : launch_bwd_dt<kBF16, false>(p, stream);
}

} // namespace attention
} // namespace wave
