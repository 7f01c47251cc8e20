// wave_bench.cpp -- C++ host driver for libwave_runtime.so, the counterpart
// of the reference's HIP runners (tools/wave-matmul-calibrate/
// wave-matmul-calibrate-runner.cpp:1836-1912, tools/wave-fa-calibrate/
// wave-fa-gfx950-runner.cpp:406-491): allocate device buffers, fill them with
// seeded synthetic inputs, launch through the C ABI, time `iters`
// back-to-back launches between two hipEvents (median over `repeats`), and
// print the runners' `key: value` lines (per_launch_us, tflops, ...).
//
//   wave-bench gemm [--m M] [--n N] [--k K] [--input-type f16|bf16]
//                   [--c-type f32|f16|bf16] [--output-layout row-major|column-major]
//                   [--streamk-workers W] [--iters N] [--warmup N] [--repeats R]
//                   [--seed S]
//   wave-bench fa   [--batch B] [--heads H] [--kv-heads H] [--sequence S]
//                   [--dtype f16|bf16] [--causal] [--iters N] [--warmup N]
//                   [--repeats R] [--seed S]
//
// Parity is checked by the test suite, not here.
// Exit codes follow the runners: 2 for bad arguments, 1 for HIP failures.
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

// Uniform [-1, 1) or N(0, 1) * scale values, 16-bit storage.
std::vector<uint16_t> synth(size_t n, int dtype, uint64_t seed, bool normal, float scale) {
  std::vector<uint16_t> out(n);
  std::mt19937_64 rng(seed);
  std::uniform_real_distribution<float> uni(-1.f, 1.f);
  std::normal_distribution<float> nor(0.f, 1.f);
  for (auto &v : out)
    v = to_bits((normal ? nor(rng) : uni(rng)) * scale, dtype);
  return out;
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

void print_device() {
  double tf = 0, mhz = 0;
  int cus = 0;
  check_wave(wave_device_mfma_peak(0, &tf, &mhz, &cus), "device");
  hipDeviceProp_t p;
  check_hip(hipGetDeviceProperties(&p, 0), "props");
  std::printf("device: %s (%s) cus=%d shader_clock_mhz=%.0f mfma_peak_tflops=%.1f\n", p.name,
              p.gcnArchName, cus, mhz, tf);
}

int run_gemm(Opts &o) {
  const int M = (int)o.num("--m", 8192), N = (int)o.num("--n", 8192), K = (int)o.num("--k", 8192);
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
  const bool normal = o.str("--input-mode", "uniform") == "normal";
  const float scale = normal ? 1.0f / std::sqrt((float)K) : 1.0f;
  void *A = upload(synth((size_t)M * K, in, seed, normal, scale));
  void *B = upload(synth((size_t)N * K, in, seed + 1, normal, scale));
  void *C = nullptr;
  check_hip(hipMalloc(&C, (size_t)M * N * (out == WAVE_F32 ? 4 : 2)), "hipMalloc C");
  float *scratch = nullptr;
  uint32_t *counters = nullptr;
  if (workers > 0) {
    size_t sb = 0, cb = 0;
    check_wave(wave_gemm_streamk_workspace_bytes(M, N, workers, &sb, &cb), "workspace");
    check_hip(hipMalloc((void **)&scratch, sb), "hipMalloc scratch");
    check_hip(hipMalloc((void **)&counters, cb), "hipMalloc counters");
    check_wave(wave_gemm_streamk_workspace_reset(counters, M, N, nullptr), "reset");
  }
  auto launch = [&]() {
    if (workers > 0)
      check_wave(wave_gemm_streamk_launch(A, B, C, M, N, K, in, out, layout, scratch, counters,
                                          workers, nullptr),
                 "wave_gemm_streamk_launch");
    else
      check_wave(wave_gemm_launch(A, B, C, M, N, K, in, out, layout, nullptr),
                 "wave_gemm_launch");
  };
  const double us = median_us(launch, iters, warmup, repeats);
  print_device();
  std::printf("kernel: %s\n", workers > 0 ? "gfx950_f16_streamk_gemm" : "wmma_f16_matmul_tiled");
  std::printf("shape: m=%d n=%d k=%d input_type=%s c_type=%s output_layout=%s\n", M, N, K,
              o.str("--input-type", "f16").c_str(), o.str("--c-type", "f16").c_str(), lay.c_str());
  if (workers > 0)
    std::printf("streamk_workers: %d\n", workers);
  std::printf("iters: %d repeats: %d\n", iters, repeats);
  std::printf("per_launch_us: %.3f\n", us);
  std::printf("tflops: %.3f\n", 2.0 * M * N * (double)K / us * 1e-6);
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
  void *Q = upload(synth(nq, dt, seed, true, 1.f));
  void *Kd = upload(synth(nkv, dt, seed + 1, true, 1.f));
  void *V = upload(synth(nkv, dt, seed + 2, true, 1.f));
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
  std::printf("tflops: %.3f\n", flops / us * 1e-6);
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
