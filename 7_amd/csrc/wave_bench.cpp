// wave_bench.cpp -- C++ host driver for libwave_runtime.so, the counterpart
// of the reference's HIP runners (tools/wave-matmul-calibrate/
// wave-matmul-calibrate-runner.cpp:1836-1912, tools/wave-fa-calibrate/
// wave-fa-gfx950-runner.cpp:406-491): allocate device buffers, fill them with
// seeded synthetic inputs, launch through the C ABI, time `iters`
// back-to-back launches between two hipEvents (median over `repeats`), and
// print the runners' `key: value` lines (per_launch_us, tflops, ...).
//
//   wave-bench gemm [--m M] [--n N] [--k K] [--input-type f16|bf16|mxfp4]
//                   [--c-type f32|f16|bf16] [--output-layout row-major|column-major]
//                   [--streamk-workers W] [--iters N] [--warmup N] [--repeats R]
//                   [--seed S] [--input-mode uniform|normal|bucket|rand-int|hpl|all-ones]
//                   [--rand-int] [--hpl] [--all-ones] [--auto] [--check]
//   wave-bench fa   [--batch B] [--heads H] [--kv-heads H] [--sequence S]
//                   [--dtype f16|bf16] [--causal] [--iters N] [--warmup N]
//                   [--repeats R] [--seed S] [--check]
//
// Input modes: uniform [-1, 1) and N(0,1)/sqrt(K)
// (config 3) from a seeded std::mt19937_64; bucket, rand-int, hpl and
// all-ones restate the reference runner's generators (runner.cpp:681-716,
// :1143-1186), e.g. for comparison with its rand_int profile numbers.
// MXFP4 (--input-type mxfp4) takes the runner's random e2m1 codes and e8m0
// scales 124..127 (runner.cpp:1135-1150, :1208-1220) or, with --all-ones,
// codes 0x22 and scales 0x7f; rand-int and hpl are refused as the runner
// refuses them (runner.cpp:599-600).
// --check samples outputs against a host fp32 (GEMM) or double (FA)
// reference with the runner's tolerances (1e-2 + 1e-3*|expected|,
// runner.cpp:942, plus one ulp of a 16-bit output; 3e-2 for FA,
// wave-fa-gfx950-runner.cpp:388) and prints the runner's `output_check:`
// line; the full parity suite is tests/.
// Exit codes follow the runners: 2 for bad arguments, 1 for HIP failures or
// a failed check.
#include "../../include/wave_runtime.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

namespace {

[[noreturn]] void die(const std::string &msg) {
  std::fprintf(stderr, "%s\n", msg.c_str());
  std::exit(2);
}

void check_hip(hipError_t e, const char *what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    std::exit(1);
  }
}

void check_wave(int st, const char *what) {
  if (st == WAVE_OK)
    return;
  std::fprintf(stderr, "%s: %s (%s)\n", what, wave_status_string(st), wave_last_error());
  std::exit(st < 0 ? 2 : 1);
}

struct Opts {
  std::vector<std::string> args;
  size_t i = 0;
  bool flag(const char *name) {
    for (auto &a : args)
      if (a == name)
        return true;
    return false;
  }
  std::string str(const char *name, const std::string &def) {
    for (size_t k = 0; k + 1 < args.size(); ++k)
      if (args[k] == name)
        return args[k + 1];
    return def;
  }
  long num(const char *name, long def) {
    std::string v = str(name, "");
    if (v.empty())
      return def;
    char *end = nullptr;
    long r = std::strtol(v.c_str(), &end, 10);
    if (!end || *end)
      die(std::string("bad integer for ") + name);
    return r;
  }
};

int dtype_of(const std::string &s) {
  if (s == "f32")
    return WAVE_F32;
  if (s == "f16")
    return WAVE_F16;
  if (s == "bf16")
    return WAVE_BF16;
  die("unknown dtype " + s);
}

float from_bits(uint16_t b, int dtype) {
  if (dtype == WAVE_F16) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return (float)h;
  }
  uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint16_t to_bits(float v, int dtype) {
  if (dtype == WAVE_F16) {
    _Float16 h = (_Float16)v;
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
  }
  uint32_t u;
  std::memcpy(&u, &v, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

enum class Mode { Uniform, Normal, Bucket, RandInt, Hpl, AllOnes };

Mode mode_of(const std::string &s) {
  if (s == "uniform") return Mode::Uniform;
  if (s == "normal") return Mode::Normal;
  if (s == "bucket") return Mode::Bucket;
  if (s == "rand-int") return Mode::RandInt;
  if (s == "hpl") return Mode::Hpl;
  if (s == "all-ones") return Mode::AllOnes;
  die("unknown --input-mode " + s);
}

// The reference runner's index hash (runner.cpp:700-716).
uint32_t index_hash(size_t index) {
  uint64_t s = (uint64_t)index * 1664525ull + 1013904223ull;
  for (int r = 0; r < 3; ++r)
    s = s ^ (s << 13) ^ (s >> 17) ^ (s << 5);
  return (uint32_t)s;
}

// `rows` x `k` values of operand `stream` (0 = A, 1 = B), 16-bit storage.
std::vector<uint16_t> synth(size_t rows, size_t k, int dtype, uint64_t seed, int stream, Mode mode,
                            float scale) {
  const size_t n = rows * k;
  std::vector<uint16_t> out(n);
  std::mt19937_64 rng(seed + (uint64_t)stream);
  std::uniform_real_distribution<float> uni(-1.f, 1.f);
  std::normal_distribution<float> nor(0.f, 1.f);
  // Bucket LCG: seed ^ ((stream+1) * golden), values (bucket - 8) / 4.
  uint32_t state = (uint32_t)seed ^ ((uint32_t)(stream + 1) * 0x9E3779B9u);
  for (size_t i = 0; i < n; ++i) {
    float v = 0.f;
    switch (mode) {
    case Mode::Uniform: v = uni(rng) * scale; break;
    case Mode::Normal: v = nor(rng) * scale; break;
    case Mode::Bucket:
      state = 1664525u * state + 1013904223u;
      v = (float)((int)((state >> 24) % 17u) - 8) * 0.25f;
      break;
    case Mode::RandInt: {
      v = (float)(index_hash(i) % 5u) - 2.0f;
      const size_t r = i / k, c = i % k;
      if (stream == 1 && ((r ^ c) & 1u) == 0)
        v = -v;
      break;
    }
    case Mode::Hpl: v = (float)((double)index_hash(i) / (double)UINT32_MAX - 0.5); break;
    case Mode::AllOnes: v = 1.f; break;
    }
    out[i] = to_bits(v, dtype);
  }
  return out;
}

// Deterministic sample of `count` indices in [0, n), always including the
// first and last.
std::vector<size_t> sample_indices(size_t n, int count, uint64_t seed) {
  std::vector<size_t> idx = {0, n - 1};
  std::mt19937_64 rng(seed * 7919u + 13u);
  std::uniform_int_distribution<size_t> d(0, n - 1);
  for (int i = 0; i < count; ++i)
    idx.push_back(d(rng));
  return idx;
}

void *upload(const std::vector<uint16_t> &h) {
  void *d = nullptr;
  check_hip(hipMalloc(&d, h.size() * 2), "hipMalloc");
  check_hip(hipMemcpy(d, h.data(), h.size() * 2, hipMemcpyHostToDevice), "hipMemcpy");
  return d;
}

template <typename F> double median_us(F launch, int iters, int warmup, int repeats) {
  for (int i = 0; i < warmup; ++i)
    launch();
  check_hip(hipDeviceSynchronize(), "warmup sync");
  hipEvent_t a, b;
  check_hip(hipEventCreate(&a), "event");
  check_hip(hipEventCreate(&b), "event");
  std::vector<double> us;
  for (int r = 0; r < repeats; ++r) {
    check_hip(hipEventRecord(a, nullptr), "record");
    for (int i = 0; i < iters; ++i)
      launch();
    check_hip(hipEventRecord(b, nullptr), "record");
    check_hip(hipEventSynchronize(b), "sync");
    float ms = 0.f;
    check_hip(hipEventElapsedTime(&ms, a, b), "elapsed");
    us.push_back(ms * 1000.0 / iters);
  }
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  std::sort(us.begin(), us.end());
  return us[us.size() / 2];
}

double clock_mhz() {
  double tf = 0, mhz = 0;
  int cus = 0;
  check_wave(wave_device_mfma_peak(0, &tf, &mhz, &cus), "device");
  return mhz;
}

void print_device() {
  double tf = 0, mhz = 0;
  int cus = 0;
  check_wave(wave_device_mfma_peak(0, &tf, &mhz, &cus), "device");
  hipDeviceProp_t p;
  check_hip(hipGetDeviceProperties(&p, 0), "props");
  std::printf("device: %s (%s) cus=%d shader_clock_mhz=%.0f mfma_peak_tflops=%.1f\n", p.name,
              p.gcnArchName, cus, mhz, tf);
}

// The runner's LCG (runner.cpp:681-689).
uint32_t lcg_state(uint64_t seed, int stream) {
  return (uint32_t)seed ^ ((uint32_t)(stream + 1) * 0x9E3779B9u);
}
uint32_t lcg_next(uint32_t &s) { return s = 1664525u * s + 1013904223u; }

float fp4_value(unsigned code) {
  static const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
  return (code & 8u) ? -mag[code & 7u] : mag[code & 7u];
}

int run_gemm_mxfp4(Opts &o, int M, int N, int K, int out, int layout, const std::string &lay,
                   int iters, int warmup, int repeats, uint64_t seed) {
  std::string mode_name = o.str("--input-mode", "uniform");
  if (o.flag("--rand-int")) mode_name = "rand-int";
  if (o.flag("--hpl")) mode_name = "hpl";
  if (o.flag("--all-ones")) mode_name = "all-ones";
  if (mode_name == "rand-int" || mode_name == "hpl")
    die("--rand-int and --hpl are dense-input modes; MXFP4 takes random or all-ones");
  const bool ones = mode_name == "all-ones";
  if (K % 32)
    die("MXFP4 K must be a multiple of 32");
  auto codes = [&](size_t rows, int stream) {
    std::vector<uint8_t> v(rows * (size_t)K / 2, 0x22);
    uint32_t st = lcg_state(seed, stream);
    if (!ones)
      for (auto &b : v) {
        const unsigned lo = (lcg_next(st) >> 28) & 0xfu, hi = (lcg_next(st) >> 28) & 0xfu;
        b = (uint8_t)(lo | (hi << 4));
      }
    return v;
  };
  auto scales = [&](size_t rows, int stream) {
    std::vector<uint8_t> v(rows * (size_t)(K / 32), 0x7f);
    uint32_t st = lcg_state(seed, stream);
    if (!ones)
      for (auto &b : v)
        b = (uint8_t)(124u + ((lcg_next(st) >> 29) & 3u));
    return v;
  };
  const std::vector<uint8_t> hA = codes(M, 0), hB = codes(N, 1);
  const std::vector<uint8_t> hSA = scales(M, 2), hSB = scales(N, 3);
  auto up8 = [](const std::vector<uint8_t> &h) {
    void *d = nullptr;
    check_hip(hipMalloc(&d, h.size()), "hipMalloc");
    check_hip(hipMemcpy(d, h.data(), h.size(), hipMemcpyHostToDevice), "hipMemcpy");
    return d;
  };
  void *A = up8(hA), *B = up8(hB), *SA = up8(hSA), *SB = up8(hSB);
  void *C = nullptr;
  check_hip(hipMalloc(&C, (size_t)M * N * (out == WAVE_F32 ? 4 : 2)), "hipMalloc C");
  auto launch = [&]() {
    check_wave(wave_gemm_mxfp4_launch(A, B, C, SA, SB, M, N, K, out, layout, nullptr),
               "wave_gemm_mxfp4_launch");
  };
  const double us = median_us(launch, iters, warmup, repeats);
  print_device();
  std::printf("kernel: wmma_f16_matmul_tiled\n");
  std::printf("shape: m=%d n=%d k=%d input_type=mxfp4 c_type=%s output_layout=%s\n", M, N, K,
              o.str("--c-type", "f16").c_str(), lay.c_str());
  std::printf("mxfp4_input_layout: canonical\n");
  std::printf("input_mode: %s\n", ones ? "all-ones" : "random");
  std::printf("iters: %d repeats: %d\n", iters, repeats);
  std::printf("per_launch_us: %.3f\n", us);
  std::printf("median_per_launch_us: %.3f\n", us);
  std::printf("  hw_cycles_wallclock: %.0f\n", us * clock_mhz());
  std::printf("tflops: %.3f\n", 2.0 * M * N * (double)K / us * 1e-6);
  int rc = 0;
  if (o.flag("--check")) {
    // Sampled elements against the runner's float accumulation of decoded
    // values (runner.cpp:1565-1597), its tolerance plus one output ulp.
    const size_t ob = out == WAVE_F32 ? 4 : 2;
    std::vector<uint8_t> hC((size_t)M * N * ob);
    check_hip(hipMemcpy(hC.data(), C, hC.size(), hipMemcpyDeviceToHost), "hipMemcpy C");
    auto val = [&](const std::vector<uint8_t> &x, const std::vector<uint8_t> &sx, int rows,
                   int r, int kk) {
      const uint8_t b = x[((size_t)r * K + kk) / 2];
      return fp4_value((kk & 1) ? (b >> 4) : (b & 0xfu)) *
             std::ldexp(1.0f, (int)sx[(size_t)(kk / 32) * rows + r] - 127);
    };
    double worst = 0.0;
    for (size_t idx : sample_indices((size_t)M * N, 512, seed)) {
      const int m = layout == WAVE_ROW_MAJOR ? (int)(idx / N) : (int)(idx % M);
      const int n = layout == WAVE_ROW_MAJOR ? (int)(idx % N) : (int)(idx / M);
      float acc = 0.f;
      for (int kk = 0; kk < K; ++kk)
        acc += val(hA, hSA, M, m, kk) * val(hB, hSB, N, n, kk);
      double exp = acc, got;
      if (out == WAVE_F32) {
        float g;
        std::memcpy(&g, &hC[idx * 4], 4);
        got = g;
      } else {
        uint16_t g;
        std::memcpy(&g, &hC[idx * 2], 2);
        got = from_bits(g, out);
        exp = from_bits(to_bits(acc, out), out);
      }
      const double diff = std::fabs(got - exp);
      worst = std::max(worst, diff);
      const double ulp = out == WAVE_F32 ? 0.0
                         : std::ldexp(std::fabs(exp) > 0 ? std::fabs(exp) : 1.0,
                                      out == WAVE_BF16 ? -7 : -10);
      if (!(diff <= 1.0e-2 + 1.0e-3 * std::fabs(exp) + ulp)) {
        std::fprintf(stderr,
                     "output_check: failed m=%d n=%d expected=%.6f got=%.6f abs_diff=%.6f\n", m,
                     n, exp, got, diff);
        rc = 1;
        break;
      }
    }
    if (rc == 0)
      std::printf("output_check: passed mode=sampled elements=514 max_abs_diff=%.6f\n", worst);
  }
  for (void *p : {A, B, SA, SB, C})
    (void)hipFree(p);
  return rc;
}

int run_gemm(Opts &o) {
  const int M = (int)o.num("--m", 8192), N = (int)o.num("--n", 8192), K = (int)o.num("--k", 8192);
  if (o.str("--input-type", "f16") == "mxfp4") {
    const std::string lay = o.str("--output-layout", "row-major");
    if (lay != "row-major" && lay != "column-major")
      die("--output-layout must be row-major or column-major");
    const int iters = (int)o.num("--iters", 100), warmup = (int)o.num("--warmup", 10);
    const int repeats = (int)o.num("--repeats", 3);
    if (M <= 0 || N <= 0 || K <= 0 || iters <= 0 || warmup < 0 || repeats <= 0)
      die("invalid non-positive argument");
    return run_gemm_mxfp4(o, M, N, K, dtype_of(o.str("--c-type", "f16")),
                          lay == "row-major" ? WAVE_ROW_MAJOR : WAVE_COL_MAJOR, lay, iters,
                          warmup, repeats, (uint64_t)o.num("--seed", 7));
  }
  const int in = dtype_of(o.str("--input-type", "f16"));
  const int out = dtype_of(o.str("--c-type", "f16"));
  const std::string lay = o.str("--output-layout", "row-major");
  if (lay != "row-major" && lay != "column-major")
    die("--output-layout must be row-major or column-major");
  const int layout = lay == "row-major" ? WAVE_ROW_MAJOR : WAVE_COL_MAJOR;
  const int workers = (int)o.num("--streamk-workers", 0);
  const int iters = (int)o.num("--iters", 100), warmup = (int)o.num("--warmup", 10);
  const int repeats = (int)o.num("--repeats", 3);
  const uint64_t seed = (uint64_t)o.num("--seed", 7);
  if (M <= 0 || N <= 0 || K <= 0 || iters <= 0 || warmup < 0 || repeats <= 0)
    die("invalid non-positive argument");
  std::string mode_name = o.str("--input-mode", "uniform");
  if (o.flag("--rand-int")) mode_name = "rand-int";
  if (o.flag("--hpl")) mode_name = "hpl";
  if (o.flag("--all-ones")) mode_name = "all-ones";
  const Mode mode = mode_of(mode_name);
  const float scale = mode == Mode::Normal ? 1.0f / std::sqrt((float)K) : 1.0f;
  const std::vector<uint16_t> hA = synth(M, K, in, seed, 0, mode, scale);
  const std::vector<uint16_t> hB = synth(N, K, in, seed, 1, mode, scale);
  void *A = upload(hA);
  void *B = upload(hB);
  void *C = nullptr;
  check_hip(hipMalloc(&C, (size_t)M * N * (out == WAVE_F32 ? 4 : 2)), "hipMalloc C");
  float *scratch = nullptr;
  uint32_t *counters = nullptr;
  // --auto: wave_gemm_auto_launch with the workspace it asks for.
  const bool use_auto = o.flag("--auto");
  void *ws = nullptr;
  size_t ws_bytes = 0;
  if (use_auto) {
    if (workers > 0)
      die("--auto picks its own kernel; drop --streamk-workers");
    check_wave(wave_gemm_auto_workspace_bytes(M, N, K, &ws_bytes), "auto workspace");
    if (ws_bytes)
      check_hip(hipMalloc(&ws, ws_bytes), "hipMalloc workspace");
  }
  if (workers > 0) {
    size_t sb = 0, cb = 0;
    check_wave(wave_gemm_streamk_workspace_bytes(M, N, workers, &sb, &cb), "workspace");
    check_hip(hipMalloc((void **)&scratch, sb), "hipMalloc scratch");
    check_hip(hipMalloc((void **)&counters, cb), "hipMalloc counters");
    check_wave(wave_gemm_streamk_workspace_reset(counters, M, N, nullptr), "reset");
  }
  auto launch = [&]() {
    if (use_auto)
      check_wave(wave_gemm_auto_launch(A, B, C, M, N, K, in, out, layout, ws, ws_bytes, nullptr),
                 "wave_gemm_auto_launch");
    else if (workers > 0)
      check_wave(wave_gemm_streamk_launch(A, B, C, M, N, K, in, out, layout, scratch, counters,
                                          workers, nullptr),
                 "wave_gemm_streamk_launch");
    else
      check_wave(wave_gemm_launch(A, B, C, M, N, K, in, out, layout, nullptr),
                 "wave_gemm_launch");
  };
  const double us = median_us(launch, iters, warmup, repeats);
  print_device();
  std::printf("kernel: %s\n", use_auto ? "wave_gemm_auto_launch"
                              : workers > 0 ? "gfx950_f16_streamk_gemm" : "wmma_f16_matmul_tiled");
  if (use_auto)
    std::printf("auto_workspace_bytes: %zu\n", ws_bytes);
  std::printf("shape: m=%d n=%d k=%d input_type=%s c_type=%s output_layout=%s\n", M, N, K,
              o.str("--input-type", "f16").c_str(), o.str("--c-type", "f16").c_str(), lay.c_str());
  if (workers > 0)
    std::printf("streamk_workers: %d\n", workers);
  std::printf("input_mode: %s\n", mode_name.c_str());
  std::printf("iters: %d repeats: %d\n", iters, repeats);
  std::printf("per_launch_us: %.3f\n", us);
  std::printf("median_per_launch_us: %.3f\n", us);
  std::printf("  hw_cycles_wallclock: %.0f\n", us * clock_mhz());
  std::printf("tflops: %.3f\n", 2.0 * M * N * (double)K / us * 1e-6);
  if (o.flag("--check")) {
    // C from the last launch; sampled elements against an fp32 host dot
    // product rounded like the output (runner.cpp:738-745, :925-955).
    const size_t ob = out == WAVE_F32 ? 4 : 2;
    std::vector<uint8_t> hC((size_t)M * N * ob);
    check_hip(hipMemcpy(hC.data(), C, hC.size(), hipMemcpyDeviceToHost), "hipMemcpy C");
    double worst = 0.0;
    size_t worst_idx = 0;
    for (size_t idx : sample_indices((size_t)M * N, 512, seed)) {
      const int m = layout == WAVE_ROW_MAJOR ? (int)(idx / N) : (int)(idx % M);
      const int n = layout == WAVE_ROW_MAJOR ? (int)(idx % N) : (int)(idx / M);
      float acc = 0.f;
      for (int kk = 0; kk < K; ++kk)
        acc += from_bits(hA[(size_t)m * K + kk], in) * from_bits(hB[(size_t)n * K + kk], in);
      double exp = acc, got;
      if (out == WAVE_F32) {
        float g;
        std::memcpy(&g, &hC[idx * 4], 4);
        got = g;
      } else {
        uint16_t g;
        std::memcpy(&g, &hC[idx * 2], 2);
        got = from_bits(g, out);
        exp = from_bits(to_bits(acc, out), out);
      }
      const double diff = std::fabs(got - exp);
      if (diff > worst) {
        worst = diff;
        worst_idx = idx;
      }
      // The runner's bound plus one unit in the last place of the output
      // type: two valid fp32 summation orders can round a 16-bit output to
      // neighbouring values (one bf16 ulp is 0.25 at |C| ~ 40).
      const double ulp = out == WAVE_F32 ? 0.0
                         : std::ldexp(std::fabs(exp) > 0 ? std::fabs(exp) : 1.0,
                                      out == WAVE_BF16 ? -7 : -10);
      if (!(diff <= 1.0e-2 + 1.0e-3 * std::fabs(exp) + ulp)) {
        std::fprintf(stderr,
                     "output_check: failed m=%d n=%d expected=%.6f got=%.6f abs_diff=%.6f\n", m,
                     n, exp, got, diff);
        return 1;
      }
    }
    std::printf("output_check: passed mode=sampled elements=514 max_abs_diff=%.6f index=%zu\n",
                worst, worst_idx);
  }
  if (workers > 0) {
    int nz = wave_gemm_streamk_counters_check(counters, M, N, nullptr);
    if (nz != 0) {
      std::fprintf(stderr, "streamk_counter_check: failed nonzero=%d\n", nz);
      return 1;
    }
    std::printf("streamk_counter_check: passed\n");
    (void)hipFree(scratch);
    (void)hipFree(counters);
  }
  if (ws)
    (void)hipFree(ws);
  (void)hipFree(A);
  (void)hipFree(B);
  (void)hipFree(C);
  return 0;
}

int run_fa(Opts &o) {
  const int B = (int)o.num("--batch", 4), H = (int)o.num("--heads", 32);
  const int Hkv = (int)o.num("--kv-heads", H), S = (int)o.num("--sequence", 4096);
  const int D = 128;
  const int dt = dtype_of(o.str("--dtype", "f16"));
  const int causal = o.flag("--causal") ? 1 : 0;
  const int iters = (int)o.num("--iters", 20), warmup = (int)o.num("--warmup", 5);
  const int repeats = (int)o.num("--repeats", 3);
  const uint64_t seed = (uint64_t)o.num("--seed", 11);
  if (B <= 0 || H <= 0 || Hkv <= 0 || S <= 0 || iters <= 0 || repeats <= 0)
    die("invalid non-positive argument");
  const size_t nq = (size_t)B * H * S * D, nkv = (size_t)B * Hkv * S * D;
  const std::vector<uint16_t> hQ = synth(nq / D, D, dt, seed, 0, Mode::Normal, 1.f);
  const std::vector<uint16_t> hK = synth(nkv / D, D, dt, seed, 1, Mode::Normal, 1.f);
  const std::vector<uint16_t> hV = synth(nkv / D, D, dt, seed, 2, Mode::Normal, 1.f);
  void *Q = upload(hQ);
  void *Kd = upload(hK);
  void *V = upload(hV);
  void *O = nullptr;
  check_hip(hipMalloc(&O, nq * 2), "hipMalloc O");
  auto launch = [&]() {
    check_wave(wave_fa_fwd_launch(Q, Kd, V, O, B, H, Hkv, S, D, dt, causal, 0.f, nullptr),
               "wave_fa_fwd_launch");
  };
  const double us = median_us(launch, iters, warmup, repeats);
  // 4*B*H*S^2*D as the reference counts (wave-fa-gfx950-runner.cpp:465-467);
  // causal work is half of that.
  const double flops = 4.0 * B * H * (double)S * S * D * (causal ? 0.5 : 1.0);
  print_device();
  std::printf("kernel: flash_attention_bf16_gfx950\n");
  std::printf("shape: B=%d H=%d Hkv=%d N=%d D=%d dtype=%s causal=%d\n", B, H, Hkv, S, D,
              o.str("--dtype", "f16").c_str(), causal);
  std::printf("per_launch_us: %.3f\n", us);
  std::printf("median_per_launch_us: %.3f\n", us);
  std::printf("  hw_cycles_wallclock: %.0f\n", us * clock_mhz());
  std::printf("tflops: %.3f\n", flops / us * 1e-6);
  if (o.flag("--check")) {
    // The reference runner's sampled heads x rows (wave-fa-gfx950-runner.cpp
    // :204-232), double-precision softmax, tolerance 3e-2 (:388).
    std::vector<uint16_t> hO(nq);
    check_hip(hipMemcpy(hO.data(), O, nq * 2, hipMemcpyDeviceToHost), "hipMemcpy O");
    const int heads[3] = {0, (B * H) / 2, B * H - 1};
    const int rows[7] = {0, 31, 32, 127, S / 2, S - 128, S - 1};
    const double scale = 1.0 / std::sqrt((double)D);
    double worst = 0.0;
    for (int bh : heads)
      for (int r : rows) {
        if (r < 0 || r >= S)
          continue;
        const int b = bh / H, h = bh % H, hk = h / (H / Hkv);
        const size_t qb = ((size_t)bh * S + r) * D, kb = ((size_t)(b * Hkv + hk) * S) * D;
        const int kend = causal ? r + 1 : S;
        std::vector<double> w(kend);
        double mx = -1e300, sum = 0.0;
        for (int j = 0; j < kend; ++j) {
          double s = 0.0;
          for (int d = 0; d < D; ++d)
            s += (double)from_bits(hQ[qb + d], dt) * from_bits(hK[kb + (size_t)j * D + d], dt);
          w[j] = s * scale;
          mx = std::max(mx, w[j]);
        }
        for (int j = 0; j < kend; ++j)
          sum += (w[j] = std::exp(w[j] - mx));
        for (int d = 0; d < D; ++d) {
          double acc = 0.0;
          for (int j = 0; j < kend; ++j)
            acc += w[j] * from_bits(hV[kb + (size_t)j * D + d], dt);
          const double diff = std::fabs(acc / sum - from_bits(hO[qb + d], dt));
          worst = std::max(worst, diff);
          if (!(diff <= 3e-2)) {
            std::fprintf(stderr, "output_check: failed head=%d row=%d d=%d abs_diff=%.6f\n", bh,
                         r, d, diff);
            return 1;
          }
        }
      }
    std::printf("output_check: passed max_abs_diff=%.8f\n", worst);
  }
  (void)hipFree(Q);
  (void)hipFree(Kd);
  (void)hipFree(V);
  (void)hipFree(O);
  return 0;
}

} // namespace

int main(int argc, char **argv) {
  if (argc < 2 || (std::strcmp(argv[1], "gemm") && std::strcmp(argv[1], "fa"))) {
    std::fprintf(stderr, "usage: wave-bench gemm|fa [options]  (see wave_bench.cpp)\n");
    return 2;
  }
  Opts o;
  for (int i = 2; i < argc; ++i)
    o.args.push_back(argv[i]);
  return std::strcmp(argv[1], "gemm") == 0 ? run_gemm(o) : run_fa(o);
}
