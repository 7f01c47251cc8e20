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
//  * bwd_delta_kernel: delta[row] = sum_d dO[row][d] * O[row][d] in fp32.
//  * bwd_kv_kernel: one CTA (4 waves) per 64-key block of one KV head; it
//    loops over the query blocks of every q head of the group (causal: the
//    blocks at or after the key block) and accumulates dK, dV in registers.
//  * bwd_q_kernel: one CTA per 64-query block of one q head; it loops over
//    the key blocks (causal: up to the diagonal) and accumulates dQ.
// Every product is an "NT" product C[m][n] = sum_k A[m][k] B[n][k] of 32x32
// tiles on v_mfma_f32_32x32x16 with both operands read as 16-byte row chunks
// from LDS; the operands that the products need K-contiguous the other way
// (Q^T, dO^T, K^T) are written to LDS transposed when a block is loaded, and
// P^T / dS^T (dS for dQ) go through LDS between the score products and the
// gradient products.  LDS rows are padded by 16 bytes (272 B for 128-element
// rows, 144 B for 64-element rows) so the 32 rows a fragment read touches
// start in different bank groups.
#include "attention.hpp"
#include "wave_common.hpp"

namespace wave {
namespace attention {

namespace {

constexpr int kBD = 128;               // head dim
constexpr int kBlk = 64;               // query or key rows per block
constexpr int kRP = kBD * 2 + 16;      // 272: pitch of a [64][128] row tile
constexpr int kTP = kBlk * 2 + 16;     // 144: pitch of [128][64] and [64][64] tiles
constexpr int kRowTile = kBlk * kRP;   // 17408 bytes
constexpr int kColTile = kBD * kTP;    // 18432 bytes
constexpr int kSqTile = kBlk * kTP;    // 9216 bytes
constexpr float kLog2eB = 1.4426950408889634f;

struct BwdParams {
  const uint16_t *Q, *K, *V, *O, *dO;
  const float *lse;
  float *delta;
  uint16_t *dQ, *dK, *dV;
  int batch, q_heads, kv_heads, seq;
  int causal;
  float scale;        // softmax scale
  float scale_log2;   // scale * log2(e)
};

// acc += A[32 rows][K] * B[32 rows][K]^T, K = 16 * NK, both row-major in LDS
// with the given pitch (bytes), 16-bit elements.
template <int DT, int NK>
__device__ __forceinline__ void mma_nt(f32x16 &acc, const uint8_t *A, int pa, const uint8_t *B,
                                       int pb) {
  const uint32_t lane = threadIdx.x & 63;
  const uint8_t *ar = A + (lane & 31) * pa + (lane >> 5) * 16;
  const uint8_t *br = B + (lane & 31) * pb + (lane >> 5) * 16;
#pragma unroll
  for (int kk = 0; kk < NK; ++kk) {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(ar + 32 * kk);
    const u32x4 b = *reinterpret_cast<const u32x4 *>(br + 32 * kk);
    acc = mfma32x32x16<DT>(a, b, acc);
  }
}

// Load a [64][128] block of rows (row stride 128 elements) into LDS row-major
// (pitch kRP) and, when T != nullptr, transposed ([128][64], pitch kTP).
// Thread t handles row pairs x 16-byte chunks: unit u = t + 256*i, row pair
// u / 16, chunk u % 16.
__device__ __forceinline__ void load_block(const uint16_t *src, uint8_t *R, uint8_t *T) {
  const uint32_t t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t u = t + 256u * i, rp = u >> 4, c = u & 15u;
    const u32x4 a = *reinterpret_cast<const u32x4 *>(src + (size_t)(2 * rp) * kBD + 8 * c);
    const u32x4 b = *reinterpret_cast<const u32x4 *>(src + (size_t)(2 * rp + 1) * kBD + 8 * c);
    *reinterpret_cast<u32x4 *>(R + (2 * rp) * kRP + 16 * c) = a;
    *reinterpret_cast<u32x4 *>(R + (2 * rp + 1) * kRP + 16 * c) = b;
    if (T != nullptr) {
      // Element d = 8c + e of rows 2rp, 2rp+1 -> T[8c + e][2rp .. 2rp+1].
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        *reinterpret_cast<uint32_t *>(T + (8 * c + 2 * e) * kTP + 4 * rp) =
            __builtin_amdgcn_perm(b[e], a[e], 0x05040100u);
        *reinterpret_cast<uint32_t *>(T + (8 * c + 2 * e + 1) * kTP + 4 * rp) =
            __builtin_amdgcn_perm(b[e], a[e], 0x07060302u);
      }
    }
  }
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

// delta[row] = sum_d dO[row][d] * O[row][d]; 16 lanes per row, 8 elements
// a lane.
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
    p.delta[row] = s;
}

// dK, dV of one 64-key block of one KV head.
template <int DT, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void bwd_kv_kernel(BwdParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[4 * kRowTile + 2 * kColTile + 2 * kSqTile];
  uint8_t *sK = smem, *sV = sK + kRowTile, *sQ = sV + kRowTile, *sdO = sQ + kRowTile;
  uint8_t *sQt = sdO + kRowTile, *sdOt = sQt + kColTile;
  uint8_t *sPt = sdOt + kColTile, *sdSt = sPt + kSqTile;
  const int nb = p.seq / kBlk;
  const int kb = (int)blockIdx.x % nb, bhk = (int)blockIdx.x / nb;
  const int b = bhk / p.kv_heads, hkv = bhk - b * p.kv_heads;
  const int group = p.q_heads / p.kv_heads;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const size_t kv_off = ((size_t)bhk * p.seq + (size_t)kb * kBlk) * kBD;
  load_block(p.K + kv_off, sK, nullptr);
  load_block(p.V + kv_off, sV, nullptr);

  // Score tiles: wave w computes S[q][key] for q half w&1, key half w>>1;
  // lane l holds key kh2*32 + l%32 and queries qh2*32 + 8g + 4(l/32) + e.
  const int qh2 = wave & 1, kh2 = wave >> 1;
  // Gradient tiles: key half w&1, d quarters 2(w>>1), 2(w>>1)+1.
  const int kh = wave & 1, dq = wave >> 1;
  f32x16 dv[2] = {f32x16{}, f32x16{}}, dk[2] = {f32x16{}, f32x16{}};
  const int key = kb * kBlk + kh2 * 32 + (int)(lane & 31);
  for (int hq = hkv * group; hq < (hkv + 1) * group; ++hq) {
    const size_t bh = (size_t)b * p.q_heads + hq;
    for (int qb = CAUSAL ? kb : 0; qb < nb; ++qb) {
      __syncthreads();  // the previous block's readers are done
      const size_t q_off = (bh * p.seq + (size_t)qb * kBlk) * kBD;
      load_block(p.Q + q_off, sQ, sQt);
      load_block(p.dO + q_off, sdO, sdOt);
      // This lane's 16 query rows: lse (log2 units) and delta.
      float l2[16], dl[16];
      const size_t row0 = bh * p.seq + (size_t)qb * kBlk + qh2 * 32 + 4 * (lane >> 5);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 a = *reinterpret_cast<const f32x4 *>(p.lse + row0 + 8 * g);
        const f32x4 d = *reinterpret_cast<const f32x4 *>(p.delta + row0 + 8 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          l2[4 * g + e] = a[e] * kLog2eB;
          dl[4 * g + e] = d[e];
        }
      }
      __syncthreads();
      f32x16 s = {}, dp = {};
      mma_nt<DT, 8>(s, sQ + qh2 * 32 * kRP, kRP, sK + kh2 * 32 * kRP, kRP);
      mma_nt<DT, 8>(dp, sdO + qh2 * 32 * kRP, kRP, sV + kh2 * 32 * kRP, kRP);
      // P and dS; P^T / dS^T rows = keys, 4 consecutive queries per store.
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float pv[4], dsv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          const int q = qb * kBlk + qh2 * 32 + 8 * g + 4 * (int)(lane >> 5) + e;
          float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], p.scale_log2, -l2[r]));
          if (CAUSAL && key > q)
            pr = 0.f;
          pv[e] = pr;
          dsv[e] = pr * (dp[r] - dl[r]);
        }
        const uint32_t off = (kh2 * 32 + (lane & 31)) * kTP + 2 * (qh2 * 32 + 8 * g + 4 * (lane >> 5));
        *reinterpret_cast<u32x2 *>(sPt + off) = u32x2{pack2<DT>(pv[0], pv[1]), pack2<DT>(pv[2], pv[3])};
        *reinterpret_cast<u32x2 *>(sdSt + off) =
            u32x2{pack2<DT>(dsv[0], dsv[1]), pack2<DT>(dsv[2], dsv[3])};
      }
      __syncthreads();
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        mma_nt<DT, 4>(dv[t], sPt + kh * 32 * kTP, kTP, sdOt + (2 * dq + t) * 32 * kTP, kTP);
        mma_nt<DT, 4>(dk[t], sdSt + kh * 32 * kTP, kTP, sQt + (2 * dq + t) * 32 * kTP, kTP);
      }
    }
  }
  uint16_t *dK = p.dK + kv_off, *dV = p.dV + kv_off;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    store_tile32<DT>(dV, kh * 32, (2 * dq + t) * 32, dv[t], 1.f);
    store_tile32<DT>(dK, kh * 32, (2 * dq + t) * 32, dk[t], p.scale);
  }
}

// dQ of one 64-query block of one q head.
template <int DT, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void bwd_q_kernel(BwdParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[4 * kRowTile + kColTile + kSqTile];
  uint8_t *sQ = smem, *sdO = sQ + kRowTile, *sK = sdO + kRowTile, *sV = sK + kRowTile;
  uint8_t *sKt = sV + kRowTile, *sdS = sKt + kColTile;
  const int nb = p.seq / kBlk;
  const int qb = (int)blockIdx.x % nb, bh = (int)blockIdx.x / nb;
  const int b = bh / p.q_heads, hq = bh - b * p.q_heads;
  const int hkv = hq / (p.q_heads / p.kv_heads);
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const size_t q_off = ((size_t)bh * p.seq + (size_t)qb * kBlk) * kBD;
  load_block(p.Q + q_off, sQ, nullptr);
  load_block(p.dO + q_off, sdO, nullptr);
  // Score tiles: wave w computes S^T[key][q] for key half w&1, q half w>>1;
  // lane l holds query qh2*32 + l%32 and keys kh2*32 + 8g + 4(l/32) + e.
  const int kh2 = wave & 1, qh2 = wave >> 1;
  // dQ tiles: q half w&1, d quarters 2(w>>1), 2(w>>1)+1.
  const int qh = wave & 1, dq = wave >> 1;
  const int q = qb * kBlk + qh2 * 32 + (int)(lane & 31);
  const size_t row = (size_t)bh * p.seq + q;
  const float l2 = p.lse[row] * kLog2eB, dl = p.delta[row];
  f32x16 dqa[2] = {f32x16{}, f32x16{}};
  const size_t kv_base = (size_t)(b * p.kv_heads + hkv) * p.seq * kBD;
  const int kb_end = CAUSAL ? qb + 1 : nb;
  for (int kb = 0; kb < kb_end; ++kb) {
    __syncthreads();
    load_block(p.K + kv_base + (size_t)kb * kBlk * kBD, sK, sKt);
    load_block(p.V + kv_base + (size_t)kb * kBlk * kBD, sV, nullptr);
    __syncthreads();
    f32x16 st = {}, dpt = {};
    mma_nt<DT, 8>(st, sK + kh2 * 32 * kRP, kRP, sQ + qh2 * 32 * kRP, kRP);
    mma_nt<DT, 8>(dpt, sV + kh2 * 32 * kRP, kRP, sdO + qh2 * 32 * kRP, kRP);
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
        dsv[e] = pr * (dpt[r] - dl);
      }
      // dS row q, 4 consecutive keys.
      const uint32_t off = (qh2 * 32 + (lane & 31)) * kTP + 2 * (kh2 * 32 + 8 * g + 4 * (lane >> 5));
      *reinterpret_cast<u32x2 *>(sdS + off) =
          u32x2{pack2<DT>(dsv[0], dsv[1]), pack2<DT>(dsv[2], dsv[3])};
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 2; ++t)
      mma_nt<DT, 4>(dqa[t], sdS + qh * 32 * kTP, kTP, sKt + (2 * dq + t) * 32 * kTP, kTP);
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
  hipLaunchKernelGGL((bwd_kv_kernel<DT, CAUSAL>), dim3(nb * p.batch * p.kv_heads), dim3(256), 0,
                     stream, p);
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
  if (a.dtype == kF16)
    return a.causal ? launch_bwd_dt<kF16, true>(p, stream) : launch_bwd_dt<kF16, false>(p, stream);
  return a.causal ? launch_bwd_dt<kBF16, true>(p, stream) : launch_bwd_dt<kBF16, false>(p, stream);
}

} // namespace attention
} // namespace wave
