// oracle.cpp -- CPU restatement of the reference's generators and references.
//
// TEST INFRASTRUCTURE ONLY: the product (7_amd/) never links or loads this
// file.  Users: tests/ (parity checker), __graft_entry__.smoke() (checker),
// bench.py cpu_baseline leg (timed CPU baseline, kind "port").
//
// Reference files restated (all paths under the reference checkout):
//   tools/wave-matmul-calibrate/wave-matmul-calibrate-runner.cpp  ("runner")
//   python/mlir/dialects/wave_matmul.py                          ("wave_matmul")
//   python/mlir/dialects/wave_attention.py                       ("wave_attention")
//   tools/wave-fa-calibrate/wave-fa-calibrate-runner.cpp          ("fa-f32-runner")
//   tools/wave-fa-calibrate/wave-fa-gfx950-runner.cpp             ("fa-gfx950-runner")
//
// How each function is pinned (tests/test_oracle.py):
//   rand_state/next_rand/bucket_value   -> reference golden: seed-7 generator
//        fixtures from oracle/_ref (the runner's own randomInputValue compiled
//        from the reference sources) + closed-form value set {-2..2 step .25}.
//   rand_int / hpl                      -> reference golden vectors
//        (wave_matmul_rand_int_test.cpp:30-33, :467-472) and oracle/_ref.
//   f32_to_f16 / f16_to_f32 / f64_to_f16 -> numpy float16 (IEEE RNE) on all
//        65536 bit patterns and on random doubles; runner halfToFloat via _ref.
//   f32_to_bf16 / bf16_to_f32           -> runner floatToBF16Bits via _ref on
//        random floats; HPL bf16 golden bit patterns.
//   gemm_inputs                          -> rand_int/HPL goldens, _ref bytes.
//   gemm_nt / gemm_element               -> 2x2x4 rand_int golden {0,-2,2,-2}
//        (rand_int_test.cpp:78), bf16-ref 32.0 (test wave_matmul.py CHECK:1068),
//        f16-ref-rounding -132.5625/-132.5 (CHECK:1075), _ref
//        computeExpectedElement, float64 numpy matmul (exact for bucket data).
//   fa_f32_inputs / fa_f32_reference     -> _ref computeReference (fa-f32-runner),
//        numpy float64 softmax, zero-QK closed form (mean of V).
//   fa_gfx950_inputs / attention_rows    -> _ref computeAttentionRow, numpy
//        float64 softmax, zero-QK closed form, causal row 0 == V[0].
//   streamk_*                            -> exhaustive property check
//        (test/python/dialects/wave_matmul_streamk.py:13-57) + scratch/counter
//        goldens.

#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

template <typename F> void parallelFor(int begin, int end, int threads, F fn) {
  if (threads <= 1 || end - begin <= 1) {
    for (int i = begin; i < end; ++i)
      fn(i);
    return;
  }
  threads = std::min(threads, end - begin);
  std::vector<std::thread> pool;
  pool.reserve(threads);
  for (int t = 0; t < threads; ++t) {
    pool.emplace_back([=, &fn]() {
      for (int i = begin + t; i < end; i += threads)
        fn(i);
    });
  }
  for (std::thread &th : pool)
    th.join();
}

uint64_t xorShift(uint64_t s) { return s ^ (s << 13) ^ (s >> 17) ^ (s << 5); }

float toFloat(uint16_t bits, int dtype) {
  return dtype == ORACLE_BF16 ? oracle_bf16_to_f32(bits)
                              : oracle_f16_to_f32(bits);
}

uint16_t fromFloat(float v, int dtype) {
  return dtype == ORACLE_BF16 ? oracle_f32_to_bf16(v) : oracle_f32_to_f16(v);
}

std::vector<float> widen(const uint16_t *src, size_t n, int dtype) {
  std::vector<float> out(n);
  for (size_t i = 0; i < n; ++i)
    out[i] = toFloat(src[i], dtype);
  return out;
}

} // namespace

extern "C" {

// runner.cpp:681-684, wave_matmul.py:831
uint32_t oracle_rand_state(int seed, int stream) {
  return static_cast<uint32_t>(seed) ^
         (static_cast<uint32_t>(stream + 1) * 0x9E3779B9u);
}

// runner.cpp:686-689 (LCG constants of Numerical Recipes)
uint32_t oracle_next_rand(uint32_t *state) {
  *state = 1664525u * *state + 1013904223u;
  return *state;
}

// runner.cpp:691-694 (step 0.25); fa-gfx950-runner.cpp:188-192 and
// fa-f32-runner.cpp:183-187 use the same bucket with other steps.
float oracle_bucket_value(uint32_t *state, float step) {
  int bucket = static_cast<int>((oracle_next_rand(state) >> 24) % 17u) - 8;
  return static_cast<float>(bucket) * step;
}

// runner.cpp:700-706
float oracle_rand_int(size_t index) {
  uint64_t s = static_cast<uint64_t>(index) * 1664525ull + 1013904223ull;
  s = xorShift(xorShift(xorShift(s)));
  return static_cast<float>(static_cast<uint32_t>(s) % 5u) - 2.0f;
}

// runner.cpp:708-716
float oracle_hpl(size_t index) {
  uint64_t s = static_cast<uint64_t>(index) * 1664525ull + 1013904223ull;
  s = xorShift(xorShift(xorShift(s)));
  return static_cast<float>(static_cast<double>(static_cast<uint32_t>(s)) /
                                static_cast<double>(UINT32_MAX) -
                            0.5);
}

// IEEE-754 binary16 round-to-nearest-even from binary32 (the conversion the
// runner gets from `static_cast<_Float16>` at runner.cpp:660-665).  Written
// from the IEEE definition: keep 10 mantissa bits, round on the dropped bits.
uint16_t oracle_f32_to_f16(float v) {
  uint32_t x;
  std::memcpy(&x, &v, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) // inf / nan
    return static_cast<uint16_t>(sign | 0x7c00u |
                                 (absx > 0x7f800000u ? 0x200u : 0u));
  int exp = static_cast<int>(absx >> 23) - 127;
  if (exp > 15)
    return static_cast<uint16_t>(sign | 0x7c00u);
  uint32_t mant = (absx & 0x7fffffu) | (absx ? 0x800000u : 0u);
  if (exp >= -14) {
    // normal half: 10 kept bits, 13 dropped bits
    uint32_t half = (static_cast<uint32_t>(exp + 15) << 10) | ((mant >> 13) & 0x3ffu);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u)))
      ++half; // may carry into exponent / to inf, which is correct
    return static_cast<uint16_t>(sign | half);
  }
  if (absx == 0)
    return static_cast<uint16_t>(sign);
  // subnormal half: value = mant * 2^(exp-23); half unit = 2^-24
  int shift = -exp - 14 + 13; // bits to drop from the 24-bit mantissa
  if (shift > 24)
    return static_cast<uint16_t>(sign);
  uint32_t half = mant >> shift;
  uint32_t rem = mant & ((1u << shift) - 1u);
  uint32_t mid = 1u << (shift - 1);
  if (rem > mid || (rem == mid && (half & 1u)))
    ++half;
  return static_cast<uint16_t>(sign | half);
}

// Same rounding from binary64 (Python's struct.pack('<e'), used by
// wave_matmul.py:839-840 and wave_attention.py:221-222; also the runner's
// double -> _Float16 cast at fa-f32-runner.cpp:201-203).
uint16_t oracle_f64_to_f16(double v) {
  uint64_t x;
  std::memcpy(&x, &v, 8);
  uint32_t sign = static_cast<uint32_t>((x >> 48) & 0x8000u);
  uint64_t absx = x & 0x7fffffffffffffffull;
  if (absx >= 0x7ff0000000000000ull)
    return static_cast<uint16_t>(sign | 0x7c00u |
                                 (absx > 0x7ff0000000000000ull ? 0x200u : 0u));
  int exp = static_cast<int>(absx >> 52) - 1023;
  if (exp > 15)
    return static_cast<uint16_t>(sign | 0x7c00u);
  if (absx == 0)
    return static_cast<uint16_t>(sign);
  uint64_t mant = (absx & 0xfffffffffffffull) | 0x10000000000000ull; // 53 bits
  int shift;
  uint64_t base;
  if (exp >= -14) {
    shift = 42; // keep 11 bits (implicit + 10)
    base = static_cast<uint64_t>(exp + 15) << 10;
    uint64_t kept = (mant >> shift) & 0x3ffull;
    uint64_t rem = mant & ((1ull << shift) - 1);
    uint64_t mid = 1ull << (shift - 1);
    uint64_t half = base | kept;
    if (rem > mid || (rem == mid && (half & 1ull)))
      ++half;
    return static_cast<uint16_t>(sign | half);
  }
  shift = 42 + (-14 - exp);
  if (shift > 53)
    return static_cast<uint16_t>(sign);
  uint64_t half = mant >> shift;
  uint64_t rem = mant & ((1ull << shift) - 1);
  uint64_t mid = 1ull << (shift - 1);
  if (rem > mid || (rem == mid && (half & 1ull)))
    ++half;
  return static_cast<uint16_t>(sign | half);
}

// runner.cpp:633-658 (exact widening)
float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t mant = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      int e = 1;
      while ((mant & 0x400u) == 0) {
        mant <<= 1;
        --e;
      }
      mant &= 0x3ffu;
      bits = sign | (static_cast<uint32_t>(e + 112) << 23) | (mant << 13);
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 112) << 23) | (mant << 13);
  }
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

// runner.cpp:667-672 (no NaN special case, as in the reference)
uint16_t oracle_f32_to_bf16(float v) {
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  uint32_t rounded = bits + 0x7fffu + ((bits >> 16) & 1u);
  return static_cast<uint16_t>(rounded >> 16);
}

// runner.cpp:674-679
float oracle_bf16_to_f32(uint16_t h) {
  uint32_t bits = static_cast<uint32_t>(h) << 16;
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

// runner.cpp:1143-1186 (make16BitInputBytes) and wave_matmul.py:966-994
// (HALVES = the python builder's non-random fill).
void oracle_gemm_inputs(uint16_t *out, int rows, int k, int dtype, int seed,
                        int stream, int mode) {
  size_t elements = static_cast<size_t>(rows) * static_cast<size_t>(k);
  switch (mode) {
  case ORACLE_MODE_ALL_ONES: {
    uint16_t one = dtype == ORACLE_BF16 ? 0x3f80u : 0x3c00u; // runner.cpp:1058-1068
    for (size_t i = 0; i < elements; ++i)
      out[i] = one;
    return;
  }
  case ORACLE_MODE_HPL:
    for (size_t i = 0; i < elements; ++i)
      out[i] = fromFloat(oracle_hpl(i), dtype);
    return;
  case ORACLE_MODE_RAND_INT:
    for (size_t i = 0; i < elements; ++i) {
      float value = oracle_rand_int(i);
      size_t row = i / static_cast<size_t>(k);
      size_t col = i % static_cast<size_t>(k);
      if (stream == 1 && ((row ^ col) & 1u) == 0)
        value = -value;
      out[i] = fromFloat(value, dtype);
    }
    return;
  case ORACLE_MODE_HALVES: {
    size_t half = elements / 2;
    for (size_t i = 0; i < elements; ++i)
      out[i] = fromFloat(i < half ? 1.0f : 2.0f, dtype);
    return;
  }
  default: {
    uint32_t state = oracle_rand_state(seed, stream);
    for (size_t i = 0; i < elements; ++i)
      out[i] = fromFloat(oracle_bucket_value(&state, 0.25f), dtype);
    return;
  }
  }
}

// runner.cpp:1586-1597 (computeExpectedElement): float accumulator, k order,
// unfused multiply then add (this file is built with -ffp-contract=off).
float oracle_gemm_element(const uint16_t *a, const uint16_t *b, int k,
                          int dtype, int64_t row, int64_t col) {
  float acc = 0.0f;
  const uint16_t *ar = a + row * k;
  const uint16_t *br = b + col * k;
  for (int i = 0; i < k; ++i)
    acc += toFloat(ar[i], dtype) * toFloat(br[i], dtype);
  return acc;
}

} // extern "C"

namespace {

// 8 floats in one AVX register (GCC vector extension); element-wise
// arithmetic, so each lane is its own C element.
typedef float f8 __attribute__((vector_size(32)));

// acc[r][0..15] += a[r][i] * bt[i][0..15] for i in [kb, ke), 4 rows x 16
// columns held in registers: every element is the same float multiply then
// add, in ascending i, as the scalar loop (this file is built with
// -ffp-contract=off, so nothing is fused).
inline void microKernel4x16(const float *const a[4], const float *bt, size_t ldb, int kb,
                            int ke, float *acc, int ldacc) {
  f8 c[4][2];
  for (int r = 0; r < 4; ++r)
    for (int h = 0; h < 2; ++h)
      std::memcpy(&c[r][h], acc + r * ldacc + 8 * h, sizeof(f8));
  for (int i = kb; i < ke; ++i) {
    f8 b0, b1;
    std::memcpy(&b0, bt + i * ldb, sizeof(f8));
    std::memcpy(&b1, bt + i * ldb + 8, sizeof(f8));
    for (int r = 0; r < 4; ++r) {
      const float av = a[r][i];
      c[r][0] += av * b0;
      c[r][1] += av * b1;
    }
  }
  for (int r = 0; r < 4; ++r)
    for (int h = 0; h < 2; ++h)
      std::memcpy(acc + r * ldacc + 8 * h, &c[r][h], sizeof(f8));
}

// Rows [m0, m1) of C = A * B^T from decoded operands: `arow(r, dst)` writes
// row r of A (K floats) and bt is B^T [K][N].  Each C element is the
// runner's float accumulation in ascending k (runner.cpp:1586-1597), blocked
// over (n, k) so every element is still summed strictly in k order.  Whole
// 4 x 16 blocks run the register micro-kernel, edges the scalar loop (the
// same arithmetic per element).
template <typename ARow>
void gemmFloatRows(ARow arowOf, const float *bt, float *c, int m0,
                   int m1, int n, int k, int threads, int c_row0 = 0) {
  constexpr int NB = 128, KB = 256, MB = 32;
  int mBlocks = (m1 - m0 + MB - 1) / MB;
  parallelFor(0, mBlocks, threads, [&](int mb) {
    int rb = m0 + mb * MB;
    int re = std::min(rb + MB, m1);
    std::vector<float> arow(static_cast<size_t>(MB) * k);
    for (int r = rb; r < re; ++r)
      arowOf(r, arow.data() + static_cast<size_t>(r - rb) * k);
    std::vector<float> acc(static_cast<size_t>(MB) * NB);
    for (int nb = 0; nb < n; nb += NB) {
      int nw = std::min(NB, n - nb);
      std::fill(acc.begin(), acc.end(), 0.0f);
      for (int kb = 0; kb < k; kb += KB) {
        int ke = std::min(kb + KB, k);
        int r = rb;
        for (; r + 4 <= re; r += 4) {
          const float *a4[4];
          for (int q = 0; q < 4; ++q)
            a4[q] = arow.data() + static_cast<size_t>(r + q - rb) * k;
          int j = 0;
          for (; j + 16 <= nw; j += 16)
            microKernel4x16(a4, bt + nb + j, static_cast<size_t>(n), kb, ke,
                            acc.data() + static_cast<size_t>(r - rb) * NB + j, NB);
          for (int q = 0; q < 4; ++q) {
            float *accr = acc.data() + static_cast<size_t>(r + q - rb) * NB;
            for (int i = kb; i < ke; ++i) {
              const float av = a4[q][i];
              const float *btr = bt + static_cast<size_t>(i) * n + nb;
              for (int jj = j; jj < nw; ++jj)
                accr[jj] += av * btr[jj];
            }
          }
        }
        for (; r < re; ++r) {
          float *accr = acc.data() + static_cast<size_t>(r - rb) * NB;
          const float *ar = arow.data() + static_cast<size_t>(r - rb) * k;
          for (int i = kb; i < ke; ++i) {
            float av = ar[i];
            const float *btr = bt + static_cast<size_t>(i) * n + nb;
            for (int j = 0; j < nw; ++j)
              accr[j] += av * btr[j];
          }
        }
      }
      for (int r = rb; r < re; ++r)
        std::memcpy(c + static_cast<size_t>(r - c_row0) * n + nb,
                    acc.data() + static_cast<size_t>(r - rb) * NB,
                    sizeof(float) * nw);
    }
  });
}

} // namespace

extern "C" {

// B [N x K] (f16 or bf16) widened and transposed to B^T [K][N] floats, the
// operand layout gemmFloatRows streams.
void oracle_gemm_prepare_bt(const uint16_t *b, float *bt, int n, int k, int dtype,
                            int threads) {
  parallelFor(0, n, threads, [&](int col) {
    for (int i = 0; i < k; ++i)
      bt[static_cast<size_t>(i) * n + col] = toFloat(b[static_cast<size_t>(col) * k + i], dtype);
  });
}

// Rows [m0, m1) of C = A * B^T from A [M x K] (f16 or bf16) and a prepared
// B^T (oracle_gemm_prepare_bt), into c [m1 - m0][N] (row r at c + (r - m0) *
// N).  bench.py times this (and the preparation, apportioned per row) as the
// multithreaded CPU baseline.
void oracle_gemm_nt_rows_bt(const uint16_t *a, const float *bt, float *c, int m0, int m1,
                            int n, int k, int dtype, int threads) {
  gemmFloatRows(
      [&](int r, float *dst) {
        for (int i = 0; i < k; ++i)
          dst[i] = toFloat(a[static_cast<size_t>(r) * k + i], dtype);
      },
      bt, c, m0, m1, n, k, threads, m0);
}

// Rows [m0, m1) of C = A * B^T with A [M x K] and B [N x K] row-major (f16 or
// bf16).
void oracle_gemm_nt_rows(const uint16_t *a, const uint16_t *b, float *c,
                         int m0, int m1, int n, int k, int dtype, int threads) {
  std::vector<float> bt(static_cast<size_t>(k) * n);
  oracle_gemm_prepare_bt(b, bt.data(), n, k, dtype, threads);
  oracle_gemm_nt_rows_bt(a, bt.data(), c + static_cast<size_t>(m0) * n, m0, m1, n, k, dtype,
                         threads);
}

void oracle_gemm_nt(const uint16_t *a, const uint16_t *b, float *c, int m,
                    int n, int k, int dtype, int threads) {
  oracle_gemm_nt_rows(a, b, c, 0, m, n, k, dtype, threads);
}

// runner.cpp:738-745 (roundExpectedOutput): f32 -> f16 (RNE) or bf16.
void oracle_round_output(const float *in, void *out, size_t n, int out_dtype) {
  if (out_dtype == ORACLE_F32) {
    std::memcpy(out, in, n * sizeof(float));
    return;
  }
  uint16_t *o = static_cast<uint16_t *>(out);
  for (size_t i = 0; i < n; ++i)
    o[i] = fromFloat(in[i], out_dtype);
}

// fa-f32-runner.cpp:183-211 (fillRand + makeInputs) == wave_attention.py:210-245.
// Q is pre-scaled by log2(e)/sqrt(D) in double and rounded straight to f16.
void oracle_fa_f32_inputs(uint16_t *q, uint16_t *k, uint16_t *v, int block_m,
                          int seq_n, int head_dim, int seed) {
  size_t qn = static_cast<size_t>(block_m) * head_dim;
  size_t kvn = static_cast<size_t>(seq_n) * head_dim;
  double qScale = 1.4426950408889634 / std::sqrt(static_cast<double>(head_dim));
  uint32_t s = oracle_rand_state(seed, 0);
  for (size_t i = 0; i < qn; ++i) {
    float value = oracle_bucket_value(&s, 0.0625f);
    q[i] = oracle_f64_to_f16(static_cast<double>(value) * qScale);
  }
  s = oracle_rand_state(seed, 1);
  for (size_t i = 0; i < kvn; ++i)
    k[i] = oracle_f32_to_f16(oracle_bucket_value(&s, 0.0625f));
  s = oracle_rand_state(seed, 2);
  for (size_t i = 0; i < kvn; ++i)
    v[i] = oracle_f32_to_f16(oracle_bucket_value(&s, 0.125f));
}

// fa-f32-runner.cpp:220-249 (computeReference) == wave_attention.py:248-278:
// double scores, exp2 softmax against the row max, double P.V, / denom.
void oracle_fa_f32_reference(const uint16_t *q, const uint16_t *k,
                             const uint16_t *v, float *out, int block_m,
                             int seq_n, int head_dim) {
  std::vector<double> scores(seq_n), weights(seq_n);
  for (int m = 0; m < block_m; ++m) {
    for (int n = 0; n < seq_n; ++n) {
      double score = 0.0;
      for (int d = 0; d < head_dim; ++d)
        score += static_cast<double>(oracle_f16_to_f32(q[m * head_dim + d])) *
                 static_cast<double>(oracle_f16_to_f32(k[n * head_dim + d]));
      scores[n] = score;
    }
    double rowMax = *std::max_element(scores.begin(), scores.end());
    double denom = 0.0;
    for (int n = 0; n < seq_n; ++n) {
      weights[n] = std::exp2(scores[n] - rowMax);
      denom += weights[n];
    }
    for (int d = 0; d < head_dim; ++d) {
      double acc = 0.0;
      for (int n = 0; n < seq_n; ++n)
        acc += weights[n] *
               static_cast<double>(oracle_f16_to_f32(v[n * head_dim + d]));
      out[m * head_dim + d] = static_cast<float>(acc / denom);
    }
  }
}

// fa-gfx950-runner.cpp:194-202 and :410-417: bucket LCG per stream, Q/K step
// 0.125*input_scale, V step 0.25, rounded to bf16; --zero-qk zeroes Q and K.
void oracle_fa_gfx950_inputs(uint16_t *q, uint16_t *k, uint16_t *v,
                             size_t elements, int seed, int input_scale,
                             int zero_qk) {
  float qkScale = 0.125f * static_cast<float>(input_scale);
  uint16_t *dst[3] = {q, k, v};
  float step[3] = {qkScale, qkScale, 0.25f};
  for (int stream = 0; stream < 3; ++stream) {
    uint32_t s = oracle_rand_state(seed, stream);
    for (size_t i = 0; i < elements; ++i)
      dst[stream][i] = oracle_f32_to_bf16(oracle_bucket_value(&s, step[stream]));
  }
  if (zero_qk) {
    std::memset(q, 0, elements * 2);
    std::memset(k, 0, elements * 2);
  }
}

// fa-gfx950-runner.cpp:247-279 (computeAttentionRow), generalised with the
// two extensions the configs ask for (causal mask, grouped-query head map;
// neither exists in the reference, so those two are checked only against
// closed forms and numpy).  Layout: Q/O [B][Hq][Sq][D], K/V [B][Hkv][Sk][D].
// `heads` index the flattened (b*Hq + h) space.  Scores are double sums in d
// order, scaled, softmax with exp(score - max) in double, P.V in key order.
void oracle_attention_rows(const uint16_t *q, const uint16_t *k,
                           const uint16_t *v, int dtype, int batch,
                           int q_heads, int kv_heads, int seq_q, int seq_k,
                           int head_dim, int causal, double scale,
                           const int *heads, const int *rows, int count,
                           float *out, int threads) {
  (void)batch;
  int group = q_heads / kv_heads;
  parallelFor(0, count, threads, [&](int idx) {
    int flat = heads[idx];
    int b = flat / q_heads;
    int h = flat % q_heads;
    int kvh = h / group;
    int row = rows[idx];
    size_t qBase = (static_cast<size_t>(flat) * seq_q + row) * head_dim;
    size_t kvBase = (static_cast<size_t>(b) * kv_heads + kvh) *
                    static_cast<size_t>(seq_k) * head_dim;
    // bottom-right aligned causal mask: key j visible iff j <= row + (Sk-Sq)
    int limit = causal ? std::min(seq_k, row + (seq_k - seq_q) + 1) : seq_k;
    std::vector<double> scores(limit > 0 ? limit : 0);
    for (int key = 0; key < limit; ++key) {
      double score = 0.0;
      for (int d = 0; d < head_dim; ++d)
        score += static_cast<double>(toFloat(q[qBase + d], dtype)) *
                 static_cast<double>(
                     toFloat(k[kvBase + static_cast<size_t>(key) * head_dim + d], dtype));
      scores[key] = score * scale;
    }
    float *o = out + static_cast<size_t>(idx) * head_dim;
    if (limit <= 0) {
      for (int d = 0; d < head_dim; ++d)
        o[d] = 0.0f;
      return;
    }
    double rowMax = *std::max_element(scores.begin(), scores.end());
    double denom = 0.0;
    for (double &s : scores) {
      s = std::exp(s - rowMax);
      denom += s;
    }
    for (int d = 0; d < head_dim; ++d) {
      double sum = 0.0;
      for (int key = 0; key < limit; ++key)
        sum += scores[key] *
               static_cast<double>(
                   toFloat(v[kvBase + static_cast<size_t>(key) * head_dim + d], dtype));
      o[d] = static_cast<float>(sum / denom);
    }
  });
}

// fa-gfx950-runner.cpp:213-232 (referenceRows): all rows when S <= 512, else
// the sorted unique sample {0,31,32,127,S/2,S-128,S-1}.  Returns the count.
int oracle_fa_reference_rows(int sequence, int *rows) {
  if (sequence <= 512) {
    for (int r = 0; r < sequence; ++r)
      rows[r] = r;
    return sequence;
  }
  std::vector<int> r{0, 31, 32, 127, sequence / 2, sequence - 128, sequence - 1};
  std::sort(r.begin(), r.end());
  r.erase(std::unique(r.begin(), r.end()), r.end());
  std::copy(r.begin(), r.end(), rows);
  return static_cast<int>(r.size());
}

// fa-gfx950-runner.cpp:204-211 (referenceHeads)
int oracle_fa_reference_heads(int head_count, int *heads) {
  if (head_count <= 4) {
    for (int h = 0; h < head_count; ++h)
      heads[h] = h;
    return head_count;
  }
  heads[0] = 0;
  heads[1] = head_count / 2;
  heads[2] = head_count - 1;
  return 3;
}

// wave_matmul.py:88-100 (streamk_worker_interval).  Returns 0 or -1.
int oracle_streamk_worker_interval(int64_t total, int workers, int worker,
                                   int64_t *begin, int64_t *end) {
  if (total <= 0 || workers < 1 || workers > total || worker < 0 ||
      worker >= workers)
    return -1;
  int64_t q = total / workers, r = total % workers;
  *begin = worker * q + std::min<int64_t>(worker, r);
  *end = *begin + q + (worker < r ? 1 : 0);
  return 0;
}

// wave_matmul.py:103-114 (streamk_owner_for_iteration). -1 on bad input.
int64_t oracle_streamk_owner(int64_t total, int workers, int64_t iteration) {
  if (iteration < 0 || iteration >= total || workers < 1)
    return -1;
  int64_t q = total / workers, r = total % workers;
  if (q == 0)
    return -1;
  int64_t largeEnd = r * (q + 1);
  if (iteration < largeEnd)
    return iteration / (q + 1);
  return r + (iteration - largeEnd) / q;
}

// wave_matmul.py:132-155 (streamk_worker_segments).  slot = -1 for a whole
// tile, else the partial slot (0 or 1).  Returns segment count or -1.
int oracle_streamk_segments(int tile_count, int k_iterations, int workers,
                            int worker, int *tiles, int *k_begin, int *k_end,
                            int *slot, int max_segments) {
  if (tile_count <= 0 || k_iterations <= 0)
    return -1;
  int64_t total = static_cast<int64_t>(tile_count) * k_iterations;
  int64_t begin, end;
  if (oracle_streamk_worker_interval(total, workers, worker, &begin, &end))
    return -1;
  int64_t first = begin / k_iterations, last = (end - 1) / k_iterations;
  int count = 0, partial = 0;
  for (int64_t t = first; t <= last; ++t) {
    if (count >= max_segments)
      return -1;
    int64_t tb = t * k_iterations;
    int64_t kb = std::max(begin, tb) - tb;
    int64_t ke = std::min(end, tb + k_iterations) - tb;
    bool whole = kb == 0 && ke == k_iterations;
    tiles[count] = static_cast<int>(t);
    k_begin[count] = static_cast<int>(kb);
    k_end[count] = static_cast<int>(ke);
    slot[count] = whole ? -1 : partial;
    partial += whole ? 0 : 1;
    ++count;
  }
  if (partial > 2)
    return -1;
  return count;
}

int oracle_hardware_threads(void) {
  unsigned n = std::thread::hardware_concurrency();
  return n ? static_cast<int>(n) : 1;
}

// ---- MXFP4 ---------------------------------------------------------------

// OCP e2m1 decode: magnitude table {0, .5, 1, 1.5, 2, 3, 4, 6}, sign bit 3
// (runner.cpp:722-727).  The table follows from e2m1 (1 sign, 2 exponent
// bits with bias 1, 1 mantissa bit, subnormal at exponent 0).
float oracle_mxfp4_code_value(int code) {
  int e = (code >> 1) & 3, m = code & 1;
  float mag = e == 0 ? 0.5f * m : std::ldexp(1.0f + 0.5f * m, e - 1);
  return (code & 8) ? -mag : mag;
}

// e8m0 scale: 2^(raw - 127) (runner.cpp:729-731; wave_matmul.py:854-855).
float oracle_e8m0_value(int raw) {
  return static_cast<float>(std::ldexp(1.0, raw - 127));
}

// Packed codes for a `rows` x `k` operand, two per byte, low nibble = even
// element (runner.cpp:1135-1150; wave_matmul.py:883-888).  Modes:
//   RANDOM     runner: code = (nextRand >> 28) & 0xf on randState(seed, stream)
//   ALL_ONES   runner --all-ones: 0x22 (1.0, 1.0)
//   HALVES     Python non-random inputs: first half of the elements 1.0
//              (code 0x2), the rest 2.0 (code 0x4) (wave_matmul.py:985-989)
//   PY_RANDOM  Python random inputs: code 0x2 if bit 31 of the LCG state is
//              set, else 0x4 (wave_matmul.py:858-866)
void oracle_mxfp4_inputs(uint8_t *out, int rows, int k, int seed, int stream,
                         int mode) {
  size_t elements = static_cast<size_t>(rows) * static_cast<size_t>(k);
  uint32_t st = oracle_rand_state(seed, stream);
  size_t half = elements / 2;
  for (size_t i = 0; i < elements; i += 2) {
    uint8_t code[2];
    for (int h = 0; h < 2; ++h) {
      switch (mode) {
      case ORACLE_MODE_ALL_ONES:
        code[h] = 0x2;
        break;
      case ORACLE_MODE_HALVES:
        code[h] = i + h < half ? 0x2 : 0x4;
        break;
      case ORACLE_MODE_PY_RANDOM:
        code[h] = (oracle_next_rand(&st) >> 31) ? 0x2 : 0x4;
        break;
      default:
        code[h] = static_cast<uint8_t>((oracle_next_rand(&st) >> 28) & 0xfu);
        break;
      }
    }
    out[i / 2] = static_cast<uint8_t>(code[0] | (code[1] << 4));
  }
}

// Group-major [k/32][rows] e8m0 scales.  RANDOM: 124 + ((nextRand >> 29) & 3)
// on randState(seed, stream) (runner.cpp:1208-1220); ALL_ONES: 0x7f;
// HALVES / PY_RANDOM (the Python path, seed-independent,
// wave_matmul.py:937-950): (0x7f for the first rows/2 rows, else `low`) -
// group, with low 0x7e for A (stream 2) and 0x7d for B (stream 3).
void oracle_mxfp4_scales(uint8_t *out, int rows, int k, int seed, int stream,
                         int mode) {
  int groups = k / 32;
  size_t n = static_cast<size_t>(rows) * groups;
  if (mode == ORACLE_MODE_ALL_ONES) {
    std::memset(out, 0x7f, n);
    return;
  }
  if (mode == ORACLE_MODE_HALVES || mode == ORACLE_MODE_PY_RANDOM) {
    int low = stream == 3 ? 0x7d : 0x7e;
    for (int g = 0; g < groups; ++g)
      for (int r = 0; r < rows; ++r)
        out[static_cast<size_t>(g) * rows + r] =
            static_cast<uint8_t>((r < rows / 2 ? 0x7f : low) - g);
    return;
  }
  uint32_t st = oracle_rand_state(seed, stream);
  for (size_t i = 0; i < n; ++i)
    out[i] = static_cast<uint8_t>(124u + ((oracle_next_rand(&st) >> 29) & 3u));
}

} // extern "C"

namespace {
// Element (row, kk) of a packed operand times its group scale
// (runner.cpp:1565-1584 readMXFP4Input * e8m0ToFloat).
inline float mxfp4Scaled(const uint8_t *x, const uint8_t *sx, int rows, int k,
                         int64_t row, int kk) {
  uint8_t packed = x[(static_cast<size_t>(row) * k + kk) / 2];
  int code = (kk & 1) ? (packed >> 4) : (packed & 0xf);
  return oracle_mxfp4_code_value(code) *
         oracle_e8m0_value(sx[static_cast<size_t>(kk / 32) * rows + row]);
}
} // namespace

extern "C" {

// One C element, the runner's float accumulation (runner.cpp:1586-1597).
float oracle_gemm_mxfp4_element(const uint8_t *a, const uint8_t *b,
                                const uint8_t *sa, const uint8_t *sb, int m,
                                int n, int k, int64_t row, int64_t col) {
  float acc = 0.0f;
  for (int i = 0; i < k; ++i)
    acc += mxfp4Scaled(a, sa, m, k, row, i) * mxfp4Scaled(b, sb, n, k, col, i);
  return acc;
}

// Rows [m0, m1) of C [M][N] row-major, same float accumulation order.
void oracle_gemm_mxfp4_rows(const uint8_t *a, const uint8_t *b,
                            const uint8_t *sa, const uint8_t *sb, float *c,
                            int m0, int m1, int m, int n, int k, int threads) {
  std::vector<float> bt(static_cast<size_t>(k) * n);
  parallelFor(0, n, threads, [&](int col) {
    for (int i = 0; i < k; ++i)
      bt[static_cast<size_t>(i) * n + col] = mxfp4Scaled(b, sb, n, k, col, i);
  });
  gemmFloatRows(
      [&](int r, float *dst) {
        for (int i = 0; i < k; ++i)
          dst[i] = mxfp4Scaled(a, sa, m, k, r, i);
      },
      bt.data(), c, m0, m1, n, k, threads);
}

// AITER B layout (runner.cpp:1223-1246; wave_matmul.py:891-910): byte
// (row, kb) of the [N][K/2] operand goes to
// (((row/16 * K/64 + kb/32) * 2 + kb%32/16) * 16 + row%16) * 16 + kb%16.
void oracle_mxfp4_aiter_b(const uint8_t *in, uint8_t *out, int n, int k) {
  int storageK = k / 2, kBlocks = storageK / 32;
  for (int row = 0; row < n; ++row)
    for (int kb = 0; kb < storageK; ++kb) {
      size_t dst = ((((static_cast<size_t>(row / 16) * kBlocks + kb / 32) * 2 +
                      (kb % 32) / 16) * 16 + row % 16) * 16) + kb % 16;
      out[dst] = in[static_cast<size_t>(row) * storageK + kb];
    }
}

// AITER scale layout (runner.cpp:1248-1283; wave_matmul.py:913-935): rows
// padded to 256, groups to 8, pad bytes 0x7f; scale (group g, row r) goes to
// (r/32 * G8 + g/8) * 256 + (g%4) * 64 + (r%16) * 4 + (g%8/4) * 2 + r%32/16,
// G8 = padded groups / 8.  Returns the padded size; out may be NULL.
size_t oracle_mxfp4_aiter_scales(const uint8_t *in, uint8_t *out, int rows,
                                 int k) {
  int groups = k / 32;
  size_t paddedRows = (static_cast<size_t>(rows) + 255) / 256 * 256;
  size_t paddedGroups = (static_cast<size_t>(groups) + 7) / 8 * 8;
  size_t total = paddedRows * paddedGroups;
  if (!out)
    return total;
  std::memset(out, 0x7f, total);
  size_t g8 = paddedGroups / 8;
  for (int r = 0; r < rows; ++r)
    for (int g = 0; g < groups; ++g) {
      size_t dst = (static_cast<size_t>(r / 32) * g8 + g / 8) * 256 +
                   (g % 4) * 64 + (r % 16) * 4 + ((g % 8) / 4) * 2 + (r % 32) / 16;
      out[dst] = in[static_cast<size_t>(g) * rows + r];
    }
  return total;
}

} // extern "C"
