/*
 * wave_runtime.h -- C ABI of libwave_runtime.so, the MI355X-native (gfx950)
 * drop-in for the reference's GEMM / Stream-K / flash-attention hot path.
 *
 * Plain pointers and sizes only: device buffers are caller-owned device
 * memory, `stream` is a hipStream_t passed as void* (NULL = the null
 * stream).  No entry point allocates; every launch entry point validates
 * its arguments before touching the GPU.
 *
 * Return codes: WAVE_OK (0); a negative WAVE_ERR_* for argument errors
 * (the reference runners exit 2 on these: wave-matmul-calibrate-runner.cpp
 * :65-68 `die`); a positive hipError_t value for HIP failures (the runners
 * exit 1: runner.cpp:620-625 `checkHip`).  wave_last_error() returns a
 * message for the last failure on the calling thread.
 */
#ifndef WAVE_RUNTIME_H
#define WAVE_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (f16/bf16 inputs; f32/f16/bf16 GEMM output). */
enum { WAVE_F32 = 0, WAVE_F16 = 1, WAVE_BF16 = 2 };
/* GEMM output layouts: C[m*N+n], C[n*M+m], or tile-packed: C as a
 * sequence of 16x16 tiles in the reference's CTA / wave / wave-tile order,
 * each tile in 16x16 MFMA accumulator order (runner.cpp:32
 * OutputLayout::RowMajor / ColumnMajor / TilePacked; see
 * wave_gemm_tile_packed_launch). */
enum { WAVE_ROW_MAJOR = 0, WAVE_COL_MAJOR = 1, WAVE_TILE_PACKED = 2 };
/* Status codes. */
enum {
  WAVE_OK = 0,
  WAVE_ERR_INVALID = -1,     /* bad argument (null pointer, size, dtype)  */
  WAVE_ERR_UNSUPPORTED = -2, /* valid request outside what is built       */
  WAVE_ERR_WORKSPACE = -3    /* Stream-K counters not zero / too small    */
};

/* ---- reference shims, byte-compatible --------------------------------
 * runtime/wave_runtime.cpp:27-74: MLIR StridedMemRefType<T,1> descriptor
 * -> device pointer data + offset (offset in elements of T). */
typedef struct {
  void *base;
  void *data;
  int64_t offset;
  int64_t sizes[1];
  int64_t strides[1];
} wave_memref_1d;

void *_mlir_ciface_wave_memref_to_ptr_global_i32(wave_memref_1d *m);
void *_mlir_ciface_wave_memref_to_ptr_global_i8(wave_memref_1d *m);
void *_mlir_ciface_wave_memref_to_ptr_global_f32(wave_memref_1d *m);
void *_mlir_ciface_wave_memref_to_ptr_global_f16(wave_memref_1d *m);
void *_mlir_ciface_wave_memref_to_ptr_global_bf16(wave_memref_1d *m);
void *_mlir_ciface_wave_memref_to_ptr_global_i64(wave_memref_1d *m);
void *_mlir_ciface_wave_memref_to_ptr_global_f64(wave_memref_1d *m);

/* ---- tiled GEMM --------------------------------------------------------
 * C = A . B^T: A [M x K] row-major, B [N x K] row-major (the reference's
 * "column-major K x N" B, python/mlir/dialects/wave_matmul.py:329-333),
 * fp32 accumulation, one RNE rounding to the output type.  Replaces the
 * kernel `wmma_f16_matmul_tiled(A, B, C, trip)` (wave_matmul.py:11415-11430,
 * launched by wave-matmul-calibrate-runner.cpp:1852-1856) for any M, N, K
 * > 0 and f16/bf16 input; the reference bakes M/N/K into each kernel and
 * requires the tiling to divide them. */
int wave_gemm_launch(const void *A, const void *B, void *C, int M, int N,
                     int K, int in_dtype, int out_dtype, int c_layout,
                     void *stream);
/* c_layout WAVE_TILE_PACKED in wave_gemm_launch is the tile-packed C of the
 * reference's default blocking (BM = BN = 1, one 16x16 tile per wave,
 * wave_matmul.py:288-300 `_MatmulConfig`): the 16x16 tiles in row-major
 * order over the (M/16) x (N/16) tile grid.  M, N % 16 == 0. */

/* The same product with C tile-packed for the reference blocking
 * (bm, bn, wave_m_tiles, wave_n_tiles): the reference's output_layout
 * "tile-packed" (wave_matmul.py:284, :1279-1347 C pointers, :6351-6405
 * fragment stores; decoded by the runner's getOutputCoordinate,
 * runner.cpp:772-834).  Element index of C[m][n], with mt = m/16,
 * nt = n/16, mi = m%16, nj = n%16, MB = 16*bm*wave_m_tiles,
 * NB = 16*bn*wave_n_tiles:
 *   CTA (m/MB, n/NB), row-major over the (M/MB) x (N/NB) grid;
 *   wave (mt % (bm*wave_m_tiles)) / wave_m_tiles * bn
 *        + (nt % (bn*wave_n_tiles)) / wave_n_tiles;
 *   wave tile (mt % wave_m_tiles) * wave_n_tiles + nt % wave_n_tiles;
 *   offset in the tile (mi/4)*64 + nj*4 + mi%4.
 * Requires bm, bn, wave_m_tiles, wave_n_tiles >= 1, bm*bn <= 32 (the
 * reference's wave limit), M % MB == 0 and N % NB == 0. */
int wave_gemm_tile_packed_launch(const void *A, const void *B, void *C, int M,
                                 int N, int K, int in_dtype, int out_dtype,
                                 int bm, int bn, int wave_m_tiles,
                                 int wave_n_tiles, void *stream);

/* ---- Stream-K GEMM ------------------------------------------------------
 * Same C as wave_gemm_launch, computed by `workers` persistent workgroups
 * over the (tile, 64-wide K step) work list (wave_matmul.py:77-165).
 * Replaces `gfx950_f16_streamk_gemm(A, B, C, scratch, counters, workers)`
 * (wave_matmul.py:11521-11567; runner.cpp:1781-1834).  The reference
 * requires f16 in/out, column-major C, M,N % 256 == 0 and K % 64 == 0
 * (runner.cpp:424-440); this one takes any shape, dtype and layout.
 * Workspace (caller-owned, runner.cpp:393-412): scratch holds two fp32
 * 256x256 tiles per worker and needs no initialisation; counters hold one
 * uint32 per 256x256 output tile and must be zero before the first launch;
 * each launch leaves them zero again.  One launch in flight per workspace. */
int wave_gemm_streamk_workspace_bytes(int M, int N, int workers,
                                      size_t *scratch_bytes,
                                      size_t *counter_bytes);
int wave_gemm_streamk_launch(const void *A, const void *B, void *C, int M,
                             int N, int K, int in_dtype, int out_dtype,
                             int c_layout, float *scratch, uint32_t *counters,
                             int workers, void *stream);
/* Allocation-free Stream-K.  No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The same product as
 * wave_gemm_streamk_launch, with the workspace taken from a static device
 * array of the library (64 MiB of partial slots + 16 KiB of counters, held
 * on each GPU the library runs on until the process ends).  Limits:
 * workers <= 128 and ceil(M/256) * ceil(N/256) <= 4096 output tiles;
 * larger requests return WAVE_ERR_UNSUPPORTED.  Each call first zeroes the
 * counters it uses with a fill kernel on `stream` and calls no hipMalloc,
 * hipFree or allocating library routine.  All calls on one GPU share the
 * array: calls that overlap on one GPU (on different streams) race.  The
 * first call on each device resolves the array's address
 * (hipGetSymbolAddress, which can load the library's code object): make it
 * outside any stream capture; a first call on a capturing stream returns
 * WAVE_ERR_UNSUPPORTED, and later calls may be captured into a HIP graph.
 * Every argument check precedes the counter reset, so a rejected call
 * leaves the array untouched. */
int wave_gemm_streamk_noalloc_launch(const void *A, const void *B, void *C,
                                     int M, int N, int K, int in_dtype,
                                     int out_dtype, int c_layout, int workers,
                                     void *stream);
/* Zero the counters (after a failed or interrupted launch; Stream-K design
 * doc docs/Gfx950StreamKSameKernelReductionDesign.md:98-101). */
int wave_gemm_streamk_workspace_reset(uint32_t *counters, int M, int N,
                                      void *stream);
/* Synchronise `stream` and count non-zero counters (runner.cpp:1718-1742
 * checkStreamKCounters).  Returns the count (0 = clean) or an error. */
int wave_gemm_streamk_counters_check(const uint32_t *counters, int M, int N,
                                     void *stream);

/* ---- shape-driven GEMM dispatch ------------------------------------------
 * No kernel symbol of the reference: the reference's harness picks its
 * tiled or Stream-K kernel per run (tools/wave-matmul-calibrate/
 * wave-matmul-perf-sweep.py:151-326 kernel matrix).  This entry point picks
 * for the caller: the tiled kernel (or, for M <= 128, the short-M kernel,
 * split over K into 2 to 4 ranges of 128-column blocks when N / 128 leaves
 * CUs idle: fp32 partials reduced in the launch by each block's last
 * arriver), or Stream-K with 2 * tiles workers when the 256x256 output tiles would leave
 * at least half the CUs idle (tiles <= CUs / 2) and K >= 4096 (K >= 8192
 * at exactly CUs / 2 tiles); with at most CUs / 4 tiles,
 * max(2 * tiles, min(tiles * (K / 2048), CUs / 2)) workers.  Stream-K
 * and the split short-M kernel take their workspace from `workspace`
 * (caller-owned, 16-byte aligned device memory of
 * wave_gemm_auto_workspace_bytes(M, N, K) bytes, 0 when the shape takes an
 * unsplit path; no initialisation needed: a Stream-K launch zeroes the
 * counters it uses with a fill kernel, and the split short-M kernel's
 * counters carry a per-launch tag, so whatever they hold counts as zero,
 * and it leaves them zero); with a smaller workspace the unsplit kernel
 * runs.  One launch in flight per workspace.  Same C as wave_gemm_launch
 * (c_layout row- or column-major). */
int wave_gemm_auto_workspace_bytes(int M, int N, int K, size_t *bytes);
int wave_gemm_auto_launch(const void *A, const void *B, void *C, int M, int N,
                          int K, int in_dtype, int out_dtype, int c_layout,
                          void *workspace, size_t workspace_bytes,
                          void *stream);

/* ---- MXFP4 scaled GEMM ----------------------------------------------------
 * C[m][n] = sum_k (a[m][k] * 2^(sa[k/32][m] - 127)) * (b[n][k] * 2^(sb[k/32][n] - 127))
 * with fp32 accumulation and one RNE rounding to out_dtype.  A [M][K/2] and
 * B [N][K/2] bytes, two OCP e2m1 (fp4) values per byte, low nibble = even k;
 * A_scale [K/32][M] and B_scale [K/32][N] e8m0 bytes, group-major (the
 * reference's canonical layout).  Replaces the `mxfp4` input type of
 * `wmma_f16_matmul_tiled(A, B, C, A_scale, B_scale, trip)`
 * (python/mlir/dialects/wave_matmul.py:187-206 `mfma.scale.f32.16x16x128.f4`,
 * :996-1022 reference math, :6965-6975 argument list; runner
 * wave-matmul-calibrate-runner.cpp:1565-1595 decode and expected value,
 * :1792-1794 argument block).  Requires M, N % 256 == 0, K % 128 == 0 (the
 * reference's MXFP4 K tile, runner.cpp:1098-1100), A, B and both scale
 * arrays 16-byte aligned, C aligned to 4 elements, and
 * (K/32) * max(M, N) < 2^32. */
int wave_gemm_mxfp4_launch(const void *A, const void *B, void *C,
                           const void *A_scale, const void *B_scale, int M,
                           int N, int K, int out_dtype, int c_layout,
                           void *stream);

/* The same product with the reference's AITER input layout
 * (--mxfp4-input-layout aiter; runner.cpp:1223-1283 makeAITERBBytes /
 * makeAITERScaleBytes, wave_matmul.py:891-935): A as above; B preshuffled,
 * byte (n, kb) of the [N][K/2] matrix at
 * (((n/16 * K/64 + kb/32) * 2 + kb%32/16) * 16 + n%16) * 16 + kb%16; both
 * scale arrays as 256-byte blocks of 32 rows x 8 groups, scale (g, r) at
 * (r/32 * G8 + g/8) * 256 + (g%4) * 64 + (r%16) * 4 + (g%8/4) * 2 + r%32/16,
 * rows padded to a multiple of 256 and groups to a multiple of 8 (G8 =
 * padded groups / 8; pad bytes are never read).  Same limits as
 * wave_gemm_mxfp4_launch. */
int wave_gemm_mxfp4_aiter_launch(const void *A, const void *B, void *C,
                                 const void *A_scale, const void *B_scale, int M,
                                 int N, int K, int out_dtype, int c_layout,
                                 void *stream);

/* ---- flash-attention forward --------------------------------------------
 * O = softmax(Q K^T * scale) V.  Q, O: [batch][q_heads][seq][head_dim];
 * K, V: [batch][kv_heads][seq][head_dim]; dtype f16 or bf16 for all four;
 * fp32 row max / sum.  kv head = q head / (q_heads / kv_heads).  causal
 * masks key > query.  scale <= 0 selects 1/sqrt(head_dim).  Replaces the
 * kernel `flash_attention_bf16_gfx950(Q, K, V, O)` (wave_flash_attention.py
 * :1697-1728; wave-fa-gfx950-runner.cpp:396-402: grid (seq/256,
 * batch*heads)), which is bf16, non-causal, q_heads == kv_heads and
 * seq % 256 == 0 only.  head_dim must be 128. */
int wave_fa_fwd_launch(const void *Q, const void *K, const void *V, void *O,
                       int batch, int q_heads, int kv_heads, int seq,
                       int head_dim, int dtype, int causal, float scale,
                       void *stream);

/* Fixed-max variant: the caller guarantees |Q|, |K| <= qk_max_abs, so every
 * scaled score lies within bound = log2(e) * scale * head_dim *
 * qk_max_abs^2 (log2 units) and the kernel uses that bound as the row max of
 * every row: no online max, no rescale.  Replaces the reference's
 * `qk_max_abs` mode of `flash_attention_bf16_gfx950`
 * (wave_flash_attention.py:63-75 validation, :108-113 bound, :586-622
 * softmax).  Returns WAVE_ERR_INVALID when qk_max_abs is not finite and
 * positive or when 2^(-2 * bound) is below the smallest normal of dtype
 * (2^-126 for bf16, 2^-14 for f16), as the reference rejects it. */
int wave_fa_fwd_bounded_launch(const void *Q, const void *K, const void *V, void *O,
                               int batch, int q_heads, int kv_heads, int seq,
                               int head_dim, int dtype, int causal, float scale,
                               float qk_max_abs, void *stream);

/* Both knobs of the reference's Gfx950FlashAttentionConfig
 * (wave_flash_attention.py:44-93, :114-135) in one call: waves = 8 runs the
 * kernel of wave_fa_fwd_launch; waves = 4 runs the reference's 4-wave
 * configuration (256 threads, 64 query rows per wave, the same 256-row
 * blocks and grid).  qk_max_abs = 0 selects the online softmax; > 0 the
 * fixed-max mode, validated as in wave_fa_fwd_bounded_launch.  Other
 * arguments as wave_fa_fwd_launch.  Returns WAVE_ERR_INVALID for waves
 * other than 4 or 8. */
int wave_fa_fwd_config_launch(const void *Q, const void *K, const void *V, void *O,
                              int batch, int q_heads, int kv_heads, int seq,
                              int head_dim, int dtype, int causal, float scale,
                              float qk_max_abs, int waves, void *stream);

/* The online-softmax forward of wave_fa_fwd_launch that also writes each
 * query row's log-sum-exp, lse[b][h][q] = ln sum_k exp(scale * Q[q].K[k])
 * over the unmasked keys (float32, 16-byte aligned), for the backward below.
 * No counterpart in the reference (its forward returns O only); the lse
 * convention is flash-attention's. */
int wave_fa_fwd_lse_launch(const void *Q, const void *K, const void *V, void *O, float *lse,
                           int batch, int q_heads, int kv_heads, int seq, int head_dim,
                           int dtype, int causal, float scale, void *stream);

/* ---- block-scaled FP8 flash-attention forward ----------------------------
 * O = softmax(scale * Qd Kd^T) Vd, where Qd, Kd, Vd are OCP MX-FP8 inputs
 * decoded: e4m3 bytes times 2^(e - 127) of their e8m0 block scale, one scale
 * per 32 elements along the dimension each product contracts.
 *   Q [batch][q_heads][seq][128], Q_scale [batch][q_heads][seq][4]   (d blocks)
 *   K [batch][kv_heads][seq][128], K_scale [batch][kv_heads][seq][4] (d blocks)
 *   V [batch][kv_heads][seq][128], V_scale [batch][kv_heads][ceil(seq/32)][128]
 *                                                              (key blocks)
 * O [batch][q_heads][seq][128] in out_dtype (f16 or bf16).  The
 * probabilities are rounded to e4m3 for the PV product (as 2^4 times the
 * probability, at most 2^8, after the running max); fp32 accumulation, fp32
 * row sums.  causal, GQA, scale (<= 0: 1/sqrt(128)) and the optional lse
 * output (nullptr for none) as wave_fa_fwd_lse_launch.  Q, K, V, O 16-byte
 * aligned, Q_scale and K_scale 4-byte aligned; head_dim must be 128.  No
 * kernel of the reference: its FA notes name a block-scaled FP8 attention
 * contract as the next step (docs/PerfReferences/
 * WaveGfx950FlashAttention.md:94-99). */
int wave_fa_fwd_mxfp8_launch(const void *Q, const void *Q_scale, const void *K,
                             const void *K_scale, const void *V, const void *V_scale,
                             void *O, float *lse, int batch, int q_heads, int kv_heads,
                             int seq, int head_dim, int out_dtype, int causal, float scale,
                             void *stream);

/* ---- flash-attention backward --------------------------------------------
 * dQ, dK, dV of O = softmax(scale * Q K^T) V (causal and GQA as the forward;
 * dK, dV sum over the q heads of each KV head) from dO, O and the lse of
 * wave_fa_fwd_lse_launch: P = exp(scale Q K^T - lse), dV = P^T dO,
 * dS = P o (dO V^T - rowsum(dO o O)), dQ = scale dS K, dK = scale dS^T Q,
 * fp32 accumulation, one rounding to dtype.  Layouts as the forward; delta is
 * caller scratch of batch * q_heads * seq floats.  Requires seq % 64 == 0,
 * head_dim 128 and 16-byte aligned buffers.  The reference has no backward:
 * no counterpart to replace. */
int wave_fa_bwd_launch(const void *Q, const void *K, const void *V, const void *O,
                       const void *dO, const float *lse, float *delta, void *dQ, void *dK,
                       void *dV, int batch, int q_heads, int kv_heads, int seq, int head_dim,
                       int dtype, int causal, float scale, void *stream);

/* ---- flash_attention_f32 ------------------------------------------------
 * Replaces `flash_attention_f32(Q, K, V, O)` (wave_attention.py:1406-1441;
 * wave-fa-calibrate-runner.cpp:346-361): Q [block_m][head_dim] f16
 * pre-scaled by log2(e)/sqrt(head_dim), K, V [seq_n][head_dim] f16,
 * O [block_m][head_dim] f32 = softmax2(Q K^T) V with exp2; P enters the
 * P.V product as f16, as in the reference.  Any positive sizes (each of Q
 * and K below 2^31 elements). */
int wave_fa_f32_launch(const void *Q, const void *K, const void *V, float *O,
                       int block_m, int seq_n, int head_dim, void *stream);

/* ---- diagnostics ---------------------------------------------------------- */
const char *wave_status_string(int status);
const char *wave_last_error(void);
/* Dense f16/bf16 MFMA peak (TFLOP/s) of `device` derived from
 * hipDeviceProp_t (CUs x clock x 4096 FLOP/clk/CU) and its clock in MHz. */
int wave_device_mfma_peak(int device, double *tflops, double *clock_mhz,
                          int *compute_units);

#ifdef __cplusplus
}
#endif
#endif /* WAVE_RUNTIME_H */
