// wave_runtime.cpp -- the C ABI of libwave_runtime.so (include/wave_runtime.h).
//
// Validates every request on the host before any HIP call, maps it onto the
// kernels in gemm_kernels.hpp / attention_kernels.hpp / fa_small.hip, and
// reports failures as status codes plus a per-thread message.  Also carries
// the reference's seven memref -> pointer shims (runtime/wave_runtime.cpp:
// 27-74) unchanged in behaviour.
#include "../../include/wave_runtime.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "attention.hpp"
#include "gemm.hpp"

namespace {

thread_local char g_error[512] = "";

int fail(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return status;
}

int hip_status(hipError_t e, const char *what) {
  if (e == hipSuccess)
    return WAVE_OK;
  return fail((int)e, "%s: %s", what, hipGetErrorString(e));
}

bool is_in_dtype(int t) { return t == WAVE_F16 || t == WAVE_BF16; }
bool is_out_dtype(int t) { return t == WAVE_F32 || t == WAVE_F16 || t == WAVE_BF16; }

// Shared GEMM argument checks.  Per-lane DMA offsets inside one 256-row
// panel are 32-bit: 256 * K * 2 bytes must stay below 2^32.
int check_gemm(const void *A, const void *B, const void *C, int M, int N, int K,
               int in_dtype, int out_dtype, int c_layout) {
  if (!A || !B || !C)
    return fail(WAVE_ERR_INVALID, "gemm: null A, B or C");
  if (M <= 0 || N <= 0 || K <= 0)
    return fail(WAVE_ERR_INVALID, "gemm: M=%d N=%d K=%d must be positive", M, N, K);
  if (!is_in_dtype(in_dtype))
    return fail(WAVE_ERR_INVALID, "gemm: input dtype %d is not f16/bf16", in_dtype);
  if (!is_out_dtype(out_dtype))
    return fail(WAVE_ERR_INVALID, "gemm: output dtype %d is not f32/f16/bf16", out_dtype);
  if (c_layout != WAVE_ROW_MAJOR && c_layout != WAVE_COL_MAJOR && c_layout != WAVE_TILE_PACKED)
    return fail(WAVE_ERR_INVALID, "gemm: layout %d is not row-major, column-major or "
                "tile-packed", c_layout);
  if ((uint64_t)K * 2u * 256u >= (1ull << 32))
    return fail(WAVE_ERR_UNSUPPORTED, "gemm: K=%d exceeds 2^23", K);
  return WAVE_OK;
}

// Every argument check of wave_gemm_streamk_launch (shared with the
// allocation-free entry point, which must reject a call before it touches
// its static workspace).
int check_streamk(const void *A, const void *B, const void *C, int M, int N, int K,
                  int in_dtype, int out_dtype, int c_layout, int workers) {
  int st = check_gemm(A, B, C, M, N, K, in_dtype, out_dtype, c_layout);
  if (st != WAVE_OK)
    return st;
  if (c_layout == WAVE_TILE_PACKED)
    return fail(WAVE_ERR_UNSUPPORTED, "streamk: tile-packed C is not supported (the "
                "reference's Stream-K ABI stores column-major C)");
  const int64_t work = (int64_t)wave::gemm::tiles_for(M) *
                       wave::gemm::tiles_for(N) * wave::gemm::k_iterations(K);
  if (work > INT32_MAX)
    return fail(WAVE_ERR_UNSUPPORTED, "streamk: %lld work units exceed i32",
                (long long)work);
  if (workers <= 0 || workers > work)
    return fail(WAVE_ERR_INVALID, "streamk: workers=%d must be in [1, %lld]",
                workers, (long long)work);
  return WAVE_OK;
}

int streamk_sizes(int M, int N, int workers, size_t *scratch, size_t *counters) {
  if (M <= 0 || N <= 0)
    return fail(WAVE_ERR_INVALID, "streamk: M=%d N=%d must be positive", M, N);
  if (workers <= 0)
    return fail(WAVE_ERR_INVALID, "streamk: workers=%d must be positive", workers);
  const size_t tiles = (size_t)wave::gemm::tiles_for(M) * wave::gemm::tiles_for(N);
  *scratch = (size_t)workers * 2u * 256u * 256u * sizeof(float);
  *counters = tiles * sizeof(uint32_t);
  return WAVE_OK;
}

// Shared MXFP4 checks and launch (canonical or AITER input layout).
int gemm_mxfp4(const void *A, const void *B, void *C, const void *A_scale,
               const void *B_scale, int M, int N, int K, int out_dtype, int c_layout,
               bool aiter, void *stream, const char *name) {
  if (!A || !B || !C || !A_scale || !B_scale)
    return fail(WAVE_ERR_INVALID, "gemm_mxfp4: null A, B, C or scale pointer");
  if (M <= 0 || N <= 0 || K <= 0)
    return fail(WAVE_ERR_INVALID, "gemm_mxfp4: M=%d N=%d K=%d must be positive", M, N, K);
  if (!is_out_dtype(out_dtype))
    return fail(WAVE_ERR_INVALID, "gemm_mxfp4: output dtype %d is not f32/f16/bf16",
                out_dtype);
  if (c_layout != WAVE_ROW_MAJOR && c_layout != WAVE_COL_MAJOR)
    return fail(WAVE_ERR_INVALID, "gemm_mxfp4: layout %d is not row/column-major", c_layout);
  if (K % 128)
    return fail(WAVE_ERR_INVALID, "gemm_mxfp4: K=%d is not a multiple of 128", K);
  if (M % 256 || N % 256)
    return fail(WAVE_ERR_UNSUPPORTED, "gemm_mxfp4: M=%d N=%d must be multiples of 256", M, N);
  const size_t out_bytes = out_dtype == WAVE_F32 ? 4 : 2;
  if (((uintptr_t)A | (uintptr_t)B | (uintptr_t)A_scale | (uintptr_t)B_scale) & 15u)
    return fail(WAVE_ERR_UNSUPPORTED, "gemm_mxfp4: A, B and scales must be 16-byte aligned");
  if ((uintptr_t)C % (4 * out_bytes))
    return fail(WAVE_ERR_UNSUPPORTED, "gemm_mxfp4: C must be aligned to 4 elements");
  // Per-lane scale offsets are 32-bit: (K/32 groups, padded to 8 for AITER)
  // x max(M, N) bytes.
  const uint64_t groups = aiter ? ((uint64_t)K / 32 + 7) / 8 * 8 : (uint64_t)K / 32;
  if (groups * (uint64_t)(M > N ? M : N) >= (1ull << 32))
    return fail(WAVE_ERR_UNSUPPORTED, "gemm_mxfp4: scale array exceeds 2^32 bytes");
  wave::gemm::GemmArgs g;
  g.A = A;
  g.B = B;
  g.C = C;
  g.a_scale = A_scale;
  g.b_scale = B_scale;
  g.M = M;
  g.N = N;
  g.K = K;
  g.in_dtype = 3;  // wave::kMXFP4
  g.aiter = aiter;
  g.out_dtype = out_dtype;
  g.col_major = c_layout == WAVE_COL_MAJOR;
  return hip_status(wave::gemm::launch_mxfp4(g, static_cast<hipStream_t>(stream)), name);
}

// ---- allocation-free Stream-K workspace ------------------------------------
// wave_gemm_streamk_noalloc_launch takes its workspace from `scratch`: the
// partial slots of up to kNoAllocWorkers workers (two fp32 256x256 tiles
// each, 64 MiB) followed by one uint32 counter per output tile for up to
// kNoAllocTiles tiles (16 KiB).  Each GPU the library runs on holds its own
// copy from module load until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not a device
// address): it uses the per-device address from hipGetSymbolAddress.
constexpr int kNoAllocWorkers = 128;
constexpr int kNoAllocTiles = 4096;
constexpr size_t kNoAllocSlotWords = (size_t)kNoAllocWorkers * 2u * 256u * 256u;
static __device__ __align__(256) uint32_t scratch[kNoAllocSlotWords + kNoAllocTiles];

constexpr int kNoAllocMaxDevices = 256;
std::mutex g_noalloc_mu;
void *g_noalloc_base[kNoAllocMaxDevices];  // per device: address of its `scratch`

// This device's `scratch`, looked up once per device with that device
// current (the first call on it).  The lookup may load this library's code
// object onto the device, which must not happen inside a stream capture: a
// first call made while `stream` is capturing is refused (make one call on
// the device outside capture first).
int noalloc_workspace(void **base, hipStream_t stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return hip_status(e, "wave_gemm_streamk_noalloc_launch: hipGetDevice");
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return fail(WAVE_ERR_UNSUPPORTED, "wave_gemm_streamk_noalloc_launch: device %d", dev);
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (!g_noalloc_base[dev]) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cap);
    if (e != hipSuccess)
      return hip_status(e, "wave_gemm_streamk_noalloc_launch: hipStreamIsCapturing");
    if (cap != hipStreamCaptureStatusNone)
      return fail(WAVE_ERR_UNSUPPORTED, "wave_gemm_streamk_noalloc_launch: the first call on "
                  "device %d is inside a stream capture; make one call on it outside capture "
                  "first (it resolves the static workspace's address)", dev);
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
      return hip_status(e, "wave_gemm_streamk_noalloc_launch: hipGetSymbolAddress(scratch)");
    g_noalloc_base[dev] = p;
  }
  *base = g_noalloc_base[dev];
  return WAVE_OK;
}

// Compute units of the current device (cached per device), for the
// shape-driven dispatch's Stream-K worker count.
int device_cus(int *cus) {
  static int cached[kNoAllocMaxDevices];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return hip_status(e, "hipGetDevice");
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return fail(WAVE_ERR_UNSUPPORTED, "device %d", dev);
  if (cached[dev] == 0) {
    int n = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess)
      return hip_status(e, "hipDeviceGetAttribute(multiProcessorCount)");
    cached[dev] = n > 0 ? n : 1;
  }
  *cus = cached[dev];
  return WAVE_OK;
}

// Stream-K workers the shape-driven dispatch uses for (M, N, K), or 0 for
// the tiled path: fewer 256x256 tiles than CUs, K >= 4096 (64 K units a
// tile), M > 128 (the short-M kernel's range).
int auto_workers(int M, int N, int K, int cus) {
  const int64_t tiles = (int64_t)wave::gemm::tiles_for(M) * wave::gemm::tiles_for(N);
  if (M <= 128 || K < 4096 || tiles >= cus)
    return 0;
  // With 2 * tiles = CUs every CU runs a worker; the split then pays off
  // from K = 8192 (measured, bf16: 4096x2048x4096 tiled 750 against
  // Stream-K 720 TFLOP/s, 8192x1024x8192 826 against 932); with fewer
  // workers than CUs from K = 4096 (2048^2 x 4096: 423 against 507).
  if (tiles * 2 >= cus && K < 8192)
    return 0;
  // Between CUs / 2 and CUs tiles the split leaves workers with uneven,
  // tile-straddling shares, which measured slower than one round of whole
  // tiles (bf16, microseconds, tiled against 256 workers: 3072^2 x 8192
  // 153 / 227, 4096 x 3072 x 8192 166 / 198); exactly CUs / 2 tiles split
  // into even halves (4096 x 2048 x 8192 148 / 130).
  if (tiles * 2 > cus)
    return 0;
  int64_t w = tiles * 2 < cus ? tiles * 2 : cus;
  // Fewer than CUs / 2 tiles: one worker per 2048 of K a tile, at least
  // two a tile, at most CUs / 2 (bf16, one box, microseconds at 2 * tiles
  // against this: 1024^2 x 16384 150 -> 101, 1024^2 x 32768 272 -> 136,
  // 2048 x 1024 x 16384 153 -> 125; over nine shapes with 16 to 64 tiles
  // at most 5 % off the best of 32 to 256 workers: 2048^2 x 16384 166
  // against 158 at 256).
  if (tiles * 4 <= cus) {
    const int64_t by_k = tiles * (K / 2048);
    const int64_t cap = cus / 2;
    const int64_t want = by_k < cap ? by_k : cap;
    if (want > w)
      w = want;
  }
  const int64_t work = tiles * wave::gemm::k_iterations(K);
  return (int)(w < work ? w : work);
}

template <typename T> void *to_global(wave_memref_1d *m) {
  return static_cast<void *>(static_cast<T *>(m->data) + m->offset);
}

} // namespace

namespace wave {
namespace gemm {
hipError_t zero_counters(uint32_t *counters, size_t count, hipStream_t stream);
hipError_t count_nonzero(const uint32_t *counters, size_t count, int *result,
                         hipStream_t stream);
} // namespace gemm
} // namespace wave

extern "C" {

void *_mlir_ciface_wave_memref_to_ptr_global_i32(wave_memref_1d *m) {
  return to_global<int32_t>(m);
}
void *_mlir_ciface_wave_memref_to_ptr_global_i8(wave_memref_1d *m) {
  return to_global<int8_t>(m);
}
void *_mlir_ciface_wave_memref_to_ptr_global_f32(wave_memref_1d *m) {
  return to_global<float>(m);
}
void *_mlir_ciface_wave_memref_to_ptr_global_f16(wave_memref_1d *m) {
  return to_global<uint16_t>(m);
}
void *_mlir_ciface_wave_memref_to_ptr_global_bf16(wave_memref_1d *m) {
  return to_global<uint16_t>(m);
}
void *_mlir_ciface_wave_memref_to_ptr_global_i64(wave_memref_1d *m) {
  return to_global<int64_t>(m);
}
void *_mlir_ciface_wave_memref_to_ptr_global_f64(wave_memref_1d *m) {
  return to_global<double>(m);
}

int wave_gemm_launch(const void *A, const void *B, void *C, int M, int N, int K,
                     int in_dtype, int out_dtype, int c_layout, void *stream) {
  if (c_layout == WAVE_TILE_PACKED)
    return wave_gemm_tile_packed_launch(A, B, C, M, N, K, in_dtype, out_dtype, 1, 1, 1, 1,
                                        stream);
  int st = check_gemm(A, B, C, M, N, K, in_dtype, out_dtype, c_layout);
  if (st != WAVE_OK)
    return st;
  wave::gemm::GemmArgs g;
  g.A = A;
  g.B = B;
  g.C = C;
  g.M = M;
  g.N = N;
  g.K = K;
  g.in_dtype = in_dtype;
  g.out_dtype = out_dtype;
  g.col_major = c_layout == WAVE_COL_MAJOR;
  return hip_status(wave::gemm::launch(g, static_cast<hipStream_t>(stream)),
                    "wave_gemm_launch");
}

int wave_gemm_tile_packed_launch(const void *A, const void *B, void *C, int M, int N, int K,
                                 int in_dtype, int out_dtype, int bm, int bn, int wave_m_tiles,
                                 int wave_n_tiles, void *stream) {
  int st = check_gemm(A, B, C, M, N, K, in_dtype, out_dtype, WAVE_TILE_PACKED);
  if (st != WAVE_OK)
    return st;
  if (bm < 1 || bn < 1 || wave_m_tiles < 1 || wave_n_tiles < 1 || bm > 32 || bn > 32 ||
      bm * bn > 32)
    return fail(WAVE_ERR_INVALID, "gemm tile-packed: bm=%d bn=%d wave_m_tiles=%d "
                "wave_n_tiles=%d must be >= 1 with bm*bn <= 32", bm, bn, wave_m_tiles,
                wave_n_tiles);
  const int64_t mb = 16ll * bm * wave_m_tiles, nb = 16ll * bn * wave_n_tiles;
  if (M % mb != 0 || N % nb != 0)
    return fail(WAVE_ERR_INVALID, "gemm tile-packed: M=%d N=%d are not multiples of the "
                "CTA block %lld x %lld", M, N, (long long)mb, (long long)nb);
  wave::gemm::GemmArgs g;
  g.A = A;
  g.B = B;
  g.C = C;
  g.M = M;
  g.N = N;
  g.K = K;
  g.in_dtype = in_dtype;
  g.out_dtype = out_dtype;
  g.packed = true;
  g.pk_bm = bm;
  g.pk_bn = bn;
  g.pk_wmt = wave_m_tiles;
  g.pk_wnt = wave_n_tiles;
  return hip_status(wave::gemm::launch(g, static_cast<hipStream_t>(stream)),
                    "wave_gemm_tile_packed_launch");
}

int wave_gemm_mxfp4_launch(const void *A, const void *B, void *C, const void *A_scale,
                           const void *B_scale, int M, int N, int K, int out_dtype,
                           int c_layout, void *stream) {
  return gemm_mxfp4(A, B, C, A_scale, B_scale, M, N, K, out_dtype, c_layout, false, stream,
                    "wave_gemm_mxfp4_launch");
}

int wave_gemm_mxfp4_aiter_launch(const void *A, const void *B, void *C, const void *A_scale,
                                 const void *B_scale, int M, int N, int K, int out_dtype,
                                 int c_layout, void *stream) {
  return gemm_mxfp4(A, B, C, A_scale, B_scale, M, N, K, out_dtype, c_layout, true, stream,
                    "wave_gemm_mxfp4_aiter_launch");
}

int wave_gemm_streamk_workspace_bytes(int M, int N, int workers,
                                      size_t *scratch_bytes,
                                      size_t *counter_bytes) {
  if (!scratch_bytes || !counter_bytes)
    return fail(WAVE_ERR_INVALID, "streamk: null size outputs");
  return streamk_sizes(M, N, workers, scratch_bytes, counter_bytes);
}

int wave_gemm_streamk_launch(const void *A, const void *B, void *C, int M,
                             int N, int K, int in_dtype, int out_dtype,
                             int c_layout, float *scratch, uint32_t *counters,
                             int workers, void *stream) {
  int st = check_streamk(A, B, C, M, N, K, in_dtype, out_dtype, c_layout, workers);
  if (st != WAVE_OK)
    return st;
  if (!scratch || !counters)
    return fail(WAVE_ERR_INVALID, "streamk: null scratch or counters");
  wave::gemm::GemmArgs g;
  g.A = A;
  g.B = B;
  g.C = C;
  g.M = M;
  g.N = N;
  g.K = K;
  g.in_dtype = in_dtype;
  g.out_dtype = out_dtype;
  g.col_major = c_layout == WAVE_COL_MAJOR;
  g.scratch = scratch;
  g.counters = counters;
  g.workers = workers;
  return hip_status(wave::gemm::launch(g, static_cast<hipStream_t>(stream)),
                    "wave_gemm_streamk_launch");
}

int wave_gemm_streamk_noalloc_launch(const void *A, const void *B, void *C, int M, int N,
                                     int K, int in_dtype, int out_dtype, int c_layout,
                                     int workers, void *stream) {
  if (workers <= 0)
    return fail(WAVE_ERR_INVALID, "streamk noalloc: workers=%d must be positive", workers);
  const int64_t tiles = M > 0 && N > 0
                            ? (int64_t)wave::gemm::tiles_for(M) * wave::gemm::tiles_for(N)
                            : 0;
  if (workers > kNoAllocWorkers || tiles > kNoAllocTiles)
    return fail(WAVE_ERR_UNSUPPORTED, "streamk noalloc: workers=%d and %lld output tiles "
                "exceed the static workspace (at most %d workers and %d 256x256 tiles)",
                workers, (long long)tiles, kNoAllocWorkers, kNoAllocTiles);
  // Every check of wave_gemm_streamk_launch runs before the counter reset
  // below writes the array that all calls on this GPU share.
  int st = check_streamk(A, B, C, M, N, K, in_dtype, out_dtype, c_layout, workers);
  if (st != WAVE_OK)
    return st;
  void *base = nullptr;
  st = noalloc_workspace(&base, static_cast<hipStream_t>(stream));
  if (st != WAVE_OK)
    return st;
  float *slots = static_cast<float *>(base);
  uint32_t *counters = static_cast<uint32_t *>(base) + kNoAllocSlotWords;
  // The array keeps the previous call's contents: zero this call's counters
  // (a fill kernel, so a captured graph holds no memset node).  The partial
  // slots need no clearing: every slot a launch reads it writes first.
  st = hip_status(wave::gemm::zero_counters(counters, (size_t)tiles,
                                            static_cast<hipStream_t>(stream)),
                  "wave_gemm_streamk_noalloc_launch: counter reset");
  if (st != WAVE_OK)
    return st;
  return wave_gemm_streamk_launch(A, B, C, M, N, K, in_dtype, out_dtype, c_layout, slots,
                                  counters, workers, stream);
}

// Launch epochs for counters that carry their launch's tag (the split-K
// short-M kernel): process-wide, never 0, and started from the clock, so
// that a workspace another process left behind is unlikely to hold one.
static uint32_t next_epoch() {
  static std::atomic<uint32_t> epoch{
      (uint32_t)std::chrono::steady_clock::now().time_since_epoch().count()};
  uint32_t e;
  do
    e = epoch.fetch_add(1u, std::memory_order_relaxed) + 1u;
  while (e == 0u);
  return e;
}

int wave_gemm_auto_workspace_bytes(int M, int N, int K, size_t *bytes) {
  if (!bytes)
    return fail(WAVE_ERR_INVALID, "gemm auto: null size output");
  if (M <= 0 || N <= 0 || K <= 0)
    return fail(WAVE_ERR_INVALID, "gemm auto: M=%d N=%d K=%d must be positive", M, N, K);
  int cus = 0;
  int st = device_cus(&cus);
  if (st != WAVE_OK)
    return st;
  const int workers = auto_workers(M, N, K, cus);
  const wave::gemm::SplitPlan plan = wave::gemm::skinny_split_plan(M, N, K, cus);
  *bytes = 0;
  if (plan.splits > 0)
    *bytes = wave::gemm::skinny_split_slot_bytes(N, plan) +
             wave::gemm::skinny_split_counter_count(N, plan) * sizeof(uint64_t);
  if (workers > 0) {
    size_t scratch = 0, counters = 0;
    st = streamk_sizes(M, N, workers, &scratch, &counters);
    if (st != WAVE_OK)
      return st;
    *bytes = scratch + counters;
  }
  return WAVE_OK;
}

int wave_gemm_auto_launch(const void *A, const void *B, void *C, int M, int N, int K,
                          int in_dtype, int out_dtype, int c_layout, void *workspace,
                          size_t workspace_bytes, void *stream) {
  int st = check_gemm(A, B, C, M, N, K, in_dtype, out_dtype, c_layout);
  if (st != WAVE_OK)
    return st;
  if (c_layout == WAVE_TILE_PACKED)
    return fail(WAVE_ERR_INVALID, "gemm auto: layout must be row- or column-major");
  int cus = 0;
  st = device_cus(&cus);
  if (st != WAVE_OK)
    return st;
  if (workspace && (uintptr_t)workspace % 16 != 0)
    return fail(WAVE_ERR_INVALID, "gemm auto: workspace must be 16-byte aligned");
  const wave::gemm::SplitPlan plan = wave::gemm::skinny_split_plan(M, N, K, cus);
  if (plan.splits > 0) {
    // Short M: the split-K short-M kernel when the workspace holds its
    // partial slots and counters and the operands suit the short-M kernel;
    // otherwise wave_gemm_launch (the unsplit short-M kernel or the tiled one).
    const size_t slot_bytes = wave::gemm::skinny_split_slot_bytes(N, plan);
    const size_t count = wave::gemm::skinny_split_counter_count(N, plan);
    wave::gemm::GemmArgs g;
    g.A = A;
    g.B = B;
    g.C = C;
    g.M = M;
    g.N = N;
    g.K = K;
    g.in_dtype = in_dtype;
    g.out_dtype = out_dtype;
    g.col_major = c_layout == WAVE_COL_MAJOR;
    if (!workspace || workspace_bytes < slot_bytes + count * sizeof(uint64_t) ||
        !wave::gemm::skinny_supported(g))
      return wave_gemm_launch(A, B, C, M, N, K, in_dtype, out_dtype, c_layout, stream);
    float *slots = static_cast<float *>(workspace);
    auto *counters = reinterpret_cast<unsigned long long *>(static_cast<char *>(workspace) +
                                                            slot_bytes);
    // No counter fill: the kernel's counts carry this launch's epoch.
    return hip_status(wave::gemm::launch_skinny_split(g, plan, slots, counters, next_epoch(),
                                                      static_cast<hipStream_t>(stream)),
                      "wave_gemm_auto_launch (split-K short-M)");
  }
  const int workers = auto_workers(M, N, K, cus);
  size_t scratch = 0, counter_bytes = 0;
  if (workers > 0) {
    st = streamk_sizes(M, N, workers, &scratch, &counter_bytes);
    if (st != WAVE_OK)
      return st;
  }
  if (workers == 0 || !workspace || workspace_bytes < scratch + counter_bytes)
    return wave_gemm_launch(A, B, C, M, N, K, in_dtype, out_dtype, c_layout, stream);
  float *slots = static_cast<float *>(workspace);
  uint32_t *counters = reinterpret_cast<uint32_t *>(static_cast<char *>(workspace) + scratch);
  st = hip_status(wave::gemm::zero_counters(counters, counter_bytes / sizeof(uint32_t),
                                            static_cast<hipStream_t>(stream)),
                  "wave_gemm_auto_launch: counter reset");
  if (st != WAVE_OK)
    return st;
  return wave_gemm_streamk_launch(A, B, C, M, N, K, in_dtype, out_dtype, c_layout, slots,
                                  counters, workers, stream);
}

int wave_gemm_streamk_workspace_reset(uint32_t *counters, int M, int N,
                                      void *stream) {
  if (!counters)
    return fail(WAVE_ERR_INVALID, "streamk reset: null counters");
  size_t scratch = 0, bytes = 0;
  int st = streamk_sizes(M, N, 1, &scratch, &bytes);
  if (st != WAVE_OK)
    return st;
  return hip_status(wave::gemm::zero_counters(counters, bytes / sizeof(uint32_t),
                                              static_cast<hipStream_t>(stream)),
                    "wave_gemm_streamk_workspace_reset");
}

int wave_gemm_streamk_counters_check(const uint32_t *counters, int M, int N,
                                     void *stream) {
  if (!counters)
    return fail(WAVE_ERR_INVALID, "streamk check: null counters");
  size_t scratch = 0, bytes = 0;
  int st = streamk_sizes(M, N, 1, &scratch, &bytes);
  if (st != WAVE_OK)
    return st;
  int nonzero = 0;
  st = hip_status(wave::gemm::count_nonzero(counters, bytes / sizeof(uint32_t),
                                            &nonzero,
                                            static_cast<hipStream_t>(stream)),
                  "wave_gemm_streamk_counters_check");
  return st != WAVE_OK ? st : nonzero;
}

namespace {
// Shared by the adaptive (qk_max_abs == 0) and fixed-max entry points.
// wave_flash_attention.py:63-75: qk_max_abs finite and positive, and the
// smallest probability 2^(-2 * bound) a normal number of the P type.
int check_qk_bound(float qk_max_abs, float scale, int head_dim, int dtype) {
  if (!(qk_max_abs > 0.f) || !std::isfinite(qk_max_abs))
    return fail(WAVE_ERR_INVALID, "fa: qk_max_abs must be finite and positive");
  const double s = scale > 0.f ? (double)scale : 1.0 / std::sqrt((double)head_dim);
  const double bound = 1.4426950408889634 * s * head_dim * (double)qk_max_abs * qk_max_abs;
  const double min_normal_log2 = dtype == WAVE_F16 ? -14.0 : -126.0;
  if (-2.0 * bound < min_normal_log2)
    return fail(WAVE_ERR_INVALID,
                "fa: qk_max_abs=%g fixed reference %.3g exceeds the %s range; use "
                "wave_fa_fwd_launch", (double)qk_max_abs, bound,
                dtype == WAVE_F16 ? "f16" : "bf16");
  return WAVE_OK;
}

int fa_fwd(const void *Q, const void *K, const void *V, void *O, int batch, int q_heads,
           int kv_heads, int seq, int head_dim, int dtype, int causal, float scale,
           float qk_max_abs, int waves, void *stream, const char *name, float *lse = nullptr) {
  if (waves != 4 && waves != 8 && waves != 12)
    return fail(WAVE_ERR_INVALID, "fa: waves=%d must be 4, 8 or 12", waves);
  if (!Q || !K || !V || !O)
    return fail(WAVE_ERR_INVALID, "fa: null Q, K, V or O");
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || seq <= 0)
    return fail(WAVE_ERR_INVALID, "fa: batch=%d q_heads=%d kv_heads=%d seq=%d must be positive",
                batch, q_heads, kv_heads, seq);
  if (q_heads % kv_heads != 0)
    return fail(WAVE_ERR_INVALID, "fa: q_heads=%d not a multiple of kv_heads=%d",
                q_heads, kv_heads);
  if (!is_in_dtype(dtype))
    return fail(WAVE_ERR_INVALID, "fa: dtype %d is not f16/bf16", dtype);
  if (causal != 0 && causal != 1)
    return fail(WAVE_ERR_INVALID, "fa: causal=%d must be 0 or 1", causal);
  if (!(scale >= 0.f) || scale != scale)
    return fail(WAVE_ERR_INVALID, "fa: scale must be >= 0");
  if (head_dim != 128)
    return fail(WAVE_ERR_UNSUPPORTED, "fa: head_dim=%d (only 128 is built)", head_dim);
  if ((int64_t)batch * q_heads * ((seq + 127) / 128) > INT32_MAX ||
      (uint64_t)seq * 256u >= (1ull << 32))
    return fail(WAVE_ERR_UNSUPPORTED, "fa: problem too large");
  if ((reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(K) |
       reinterpret_cast<uintptr_t>(V) | reinterpret_cast<uintptr_t>(O)) & 15)
    return fail(WAVE_ERR_INVALID, "fa: Q, K, V and O must be 16-byte aligned");
  wave::attention::FwdArgs a;
  a.Q = Q;
  a.K = K;
  a.V = V;
  a.O = O;
  a.batch = batch;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.seq_q = seq;
  a.seq_k = seq;
  a.head_dim = head_dim;
  a.dtype = dtype;
  a.causal = causal;
  a.scale = scale;
  a.qk_max_abs = qk_max_abs;
  a.waves = waves;
  a.lse = lse;
  return hip_status(wave::attention::launch_fwd(a, static_cast<hipStream_t>(stream)), name);
}
} // namespace

int wave_fa_fwd_lse_launch(const void *Q, const void *K, const void *V, void *O, float *lse,
                           int batch, int q_heads, int kv_heads, int seq, int head_dim,
                           int dtype, int causal, float scale, void *stream) {
  if (!lse)
    return fail(WAVE_ERR_INVALID, "wave_fa_fwd_lse_launch: null lse");
  if (reinterpret_cast<uintptr_t>(lse) & 15)
    return fail(WAVE_ERR_INVALID, "wave_fa_fwd_lse_launch: lse must be 16-byte aligned");
  return fa_fwd(Q, K, V, O, batch, q_heads, kv_heads, seq, head_dim, dtype, causal, scale, 0.f,
                8, stream, "wave_fa_fwd_lse_launch", lse);
}

int wave_fa_bwd_launch(const void *Q, const void *K, const void *V, const void *O,
                       const void *dO, const float *lse, float *delta, void *dQ, void *dK,
                       void *dV, int batch, int q_heads, int kv_heads, int seq, int head_dim,
                       int dtype, int causal, float scale, void *stream) {
  if (!Q || !K || !V || !O || !dO || !lse || !delta || !dQ || !dK || !dV)
    return fail(WAVE_ERR_INVALID, "fa_bwd: null pointer argument");
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || seq <= 0)
    return fail(WAVE_ERR_INVALID, "fa_bwd: batch=%d q_heads=%d kv_heads=%d seq=%d must be positive",
                batch, q_heads, kv_heads, seq);
  if (q_heads % kv_heads != 0)
    return fail(WAVE_ERR_INVALID, "fa_bwd: q_heads=%d not a multiple of kv_heads=%d", q_heads,
                kv_heads);
  if (!is_in_dtype(dtype))
    return fail(WAVE_ERR_INVALID, "fa_bwd: dtype %d is not f16/bf16", dtype);
  if (causal != 0 && causal != 1)
    return fail(WAVE_ERR_INVALID, "fa_bwd: causal=%d must be 0 or 1", causal);
  if (!(scale >= 0.f) || scale != scale)
    return fail(WAVE_ERR_INVALID, "fa_bwd: scale must be >= 0");
  if (head_dim != 128)
    return fail(WAVE_ERR_UNSUPPORTED, "fa_bwd: head_dim=%d (only 128 is built)", head_dim);
  if (seq % 64 != 0)
    return fail(WAVE_ERR_UNSUPPORTED, "fa_bwd: seq=%d must be a multiple of 64", seq);
  if ((int64_t)batch * q_heads * seq > INT32_MAX / 2)
    return fail(WAVE_ERR_UNSUPPORTED, "fa_bwd: problem too large");
  const uintptr_t bits = reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(K) |
                         reinterpret_cast<uintptr_t>(V) | reinterpret_cast<uintptr_t>(O) |
                         reinterpret_cast<uintptr_t>(dO) | reinterpret_cast<uintptr_t>(lse) |
                         reinterpret_cast<uintptr_t>(delta) | reinterpret_cast<uintptr_t>(dQ) |
                         reinterpret_cast<uintptr_t>(dK) | reinterpret_cast<uintptr_t>(dV);
  if (bits & 15)
    return fail(WAVE_ERR_INVALID, "fa_bwd: every buffer must be 16-byte aligned");
  wave::attention::BwdArgs a;
  a.Q = Q;
  a.K = K;
  a.V = V;
  a.O = O;
  a.dO = dO;
  a.lse = lse;
  a.delta = delta;
  a.dQ = dQ;
  a.dK = dK;
  a.dV = dV;
  a.batch = batch;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.seq = seq;
  a.dtype = dtype;
  a.causal = causal;
  a.scale = scale;
  return hip_status(wave::attention::launch_bwd(a, static_cast<hipStream_t>(stream)),
                    "wave_fa_bwd_launch");
}

int wave_fa_fwd_launch(const void *Q, const void *K, const void *V, void *O,
                       int batch, int q_heads, int kv_heads, int seq,
                       int head_dim, int dtype, int causal, float scale,
                       void *stream) {
  return fa_fwd(Q, K, V, O, batch, q_heads, kv_heads, seq, head_dim, dtype, causal, scale, 0.f,
                8, stream, "wave_fa_fwd_launch");
}

int wave_fa_fwd_bounded_launch(const void *Q, const void *K, const void *V, void *O,
                               int batch, int q_heads, int kv_heads, int seq,
                               int head_dim, int dtype, int causal, float scale,
                               float qk_max_abs, void *stream) {
  const int st = check_qk_bound(qk_max_abs, scale, head_dim, dtype);
  if (st != WAVE_OK)
    return st;
  return fa_fwd(Q, K, V, O, batch, q_heads, kv_heads, seq, head_dim, dtype, causal, scale,
                qk_max_abs, 8, stream, "wave_fa_fwd_bounded_launch");
}

int wave_fa_fwd_config_launch(const void *Q, const void *K, const void *V, void *O,
                              int batch, int q_heads, int kv_heads, int seq, int head_dim,
                              int dtype, int causal, float scale, float qk_max_abs, int waves,
                              void *stream) {
  if (qk_max_abs != 0.f) {
    const int st = check_qk_bound(qk_max_abs, scale, head_dim, dtype);
    if (st != WAVE_OK)
      return st;
  }
  return fa_fwd(Q, K, V, O, batch, q_heads, kv_heads, seq, head_dim, dtype, causal, scale,
                qk_max_abs, waves, stream, "wave_fa_fwd_config_launch");
}

int wave_fa_fwd_mxfp8_launch(const void *Q, const void *Q_scale, const void *K,
                             const void *K_scale, const void *V, const void *V_scale, void *O,
                             float *lse, int batch, int q_heads, int kv_heads, int seq,
                             int head_dim, int out_dtype, int causal, float scale,
                             void *stream) {
  if (!Q || !K || !V || !O || !Q_scale || !K_scale || !V_scale)
    return fail(WAVE_ERR_INVALID, "fa mxfp8: null Q, K, V, O or scale pointer");
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || seq <= 0)
    return fail(WAVE_ERR_INVALID,
                "fa mxfp8: batch=%d q_heads=%d kv_heads=%d seq=%d must be positive", batch,
                q_heads, kv_heads, seq);
  if (q_heads % kv_heads != 0)
    return fail(WAVE_ERR_INVALID, "fa mxfp8: q_heads=%d not a multiple of kv_heads=%d",
                q_heads, kv_heads);
  if (out_dtype != WAVE_F16 && out_dtype != WAVE_BF16)
    return fail(WAVE_ERR_INVALID, "fa mxfp8: out_dtype %d is not f16/bf16", out_dtype);
  if (causal != 0 && causal != 1)
    return fail(WAVE_ERR_INVALID, "fa mxfp8: causal=%d must be 0 or 1", causal);
  if (!(scale >= 0.f) || scale != scale)
    return fail(WAVE_ERR_INVALID, "fa mxfp8: scale must be >= 0");
  if (head_dim != 128)
    return fail(WAVE_ERR_UNSUPPORTED, "fa mxfp8: head_dim=%d (only 128 is built)", head_dim);
  // Per-head buffer resources hold seq * 128 bytes in 32 bits.
  if ((int64_t)batch * q_heads * ((seq + 255) / 256) > INT32_MAX || seq >= (1 << 24))
    return fail(WAVE_ERR_UNSUPPORTED, "fa mxfp8: problem too large");
  if ((reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(K) |
       reinterpret_cast<uintptr_t>(V) | reinterpret_cast<uintptr_t>(O)) & 15)
    return fail(WAVE_ERR_INVALID, "fa mxfp8: Q, K, V and O must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(Q_scale) | reinterpret_cast<uintptr_t>(K_scale) |
       reinterpret_cast<uintptr_t>(lse)) & 3)
    return fail(WAVE_ERR_INVALID, "fa mxfp8: Q_scale, K_scale and lse must be 4-byte aligned");
  wave::attention::Fp8FwdArgs a;
  a.Q = Q;
  a.K = K;
  a.V = V;
  a.Q_scale = Q_scale;
  a.K_scale = K_scale;
  a.V_scale = V_scale;
  a.O = O;
  a.batch = batch;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.seq_q = seq;
  a.seq_k = seq;
  a.out_dtype = out_dtype;
  a.causal = causal;
  a.scale = scale;
  a.lse = lse;
  return hip_status(wave::attention::launch_fwd_fp8(a, static_cast<hipStream_t>(stream)),
                    "wave_fa_fwd_mxfp8_launch");
}

int wave_fa_f32_launch(const void *Q, const void *K, const void *V, float *O,
                       int block_m, int seq_n, int head_dim, void *stream) {
  if (!Q || !K || !V || !O)
    return fail(WAVE_ERR_INVALID, "fa_f32: null Q, K, V or O");
  if (block_m <= 0 || seq_n <= 0 || head_dim <= 0)
    return fail(WAVE_ERR_INVALID, "fa_f32: block_m=%d seq_n=%d head_dim=%d must be positive",
                block_m, seq_n, head_dim);
  if ((int64_t)block_m * head_dim > INT32_MAX || (int64_t)seq_n * head_dim > INT32_MAX)
    return fail(WAVE_ERR_INVALID, "fa_f32: block_m=%d seq_n=%d head_dim=%d exceed 2^31 elements",
                block_m, seq_n, head_dim);
  return hip_status(wave::attention::launch_small(Q, K, V, O, block_m, seq_n, head_dim,
                                                  static_cast<hipStream_t>(stream)),
                    "wave_fa_f32_launch");
}

const char *wave_status_string(int status) {
  switch (status) {
  case WAVE_OK:
    return "ok";
  case WAVE_ERR_INVALID:
    return "invalid argument";
  case WAVE_ERR_UNSUPPORTED:
    return "unsupported configuration";
  case WAVE_ERR_WORKSPACE:
    return "Stream-K workspace not reset";
  default:
    return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
  }
}

const char *wave_last_error(void) { return g_error; }

int wave_device_mfma_peak(int device, double *tflops, double *clock_mhz,
                          int *compute_units) {
  if (!tflops || !clock_mhz || !compute_units)
    return fail(WAVE_ERR_INVALID, "device peak: null output");
  hipDeviceProp_t prop;
  int st = hip_status(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (st != WAVE_OK)
    return st;
  *compute_units = prop.multiProcessorCount;
  *clock_mhz = prop.clockRate / 1000.0;
  *tflops = (double)prop.multiProcessorCount * (prop.clockRate * 1e3) * 4096.0 * 1e-12;
  return WAVE_OK;
}

} // extern "C"
