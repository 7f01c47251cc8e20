/*
 * oracle.h -- CPU restatement of the reference's input generators and CPU
 * references for the GEMM / Stream-K / flash-attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (7_amd/) links, loads or
 * calls this library.  It is used by tests/ (as the parity checker), by
 * __graft_entry__.smoke() (as the checker) and by bench.py's cpu_baseline leg
 * (as the timed CPU baseline).  Every function cites the reference file:line
 * whose behaviour it restates.
 *
 * Parity pinning (see the pin list in oracle.cpp's header comment): every
 * function here is checked in tests/test_oracle.py against the reference's own
 * golden values, the reference's runner CPU code compiled from
 * /root/reference (oracle/_ref, via tests/golden/make_golden.py fixtures), or
 * closed forms / brute force.
 */
#ifndef WAVE_ORACLE_H
#define WAVE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes shared with the product's C ABI */
enum { ORACLE_F32 = 0, ORACLE_F16 = 1, ORACLE_BF16 = 2 };
/* GEMM input modes (runner.cpp:1143-1186 + wave_matmul.py:966-994) */
enum {
  ORACLE_MODE_RANDOM = 0,    /* bucket LCG, runner default                 */
  ORACLE_MODE_ALL_ONES = 1,  /* --all-ones                                  */
  ORACLE_MODE_RAND_INT = 2,  /* --rand-int (hipBLASLt rand_int)             */
  ORACLE_MODE_HPL = 3,       /* --hpl                                       */
  ORACLE_MODE_HALVES = 4,    /* python non-random: first half 1, rest 2     */
  ORACLE_MODE_PY_RANDOM = 5  /* python MXFP4 random codes (0x2 / 0x4)       */
};

/* ---- scalar generators and rounding ---------------------------------- */
uint32_t oracle_rand_state(int seed, int stream);
uint32_t oracle_next_rand(uint32_t *state);
float oracle_bucket_value(uint32_t *state, float step);
float oracle_rand_int(size_t index);
float oracle_hpl(size_t index);
uint16_t oracle_f32_to_f16(float v);
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_bf16(float v);
float oracle_bf16_to_f32(uint16_t h);
uint16_t oracle_f64_to_f16(double v);

/* ---- GEMM ------------------------------------------------------------- */
void oracle_gemm_inputs(uint16_t *out, int rows, int k, int dtype, int seed,
                        int stream, int mode);
void oracle_gemm_nt(const uint16_t *a, const uint16_t *b, float *c, int m,
                    int n, int k, int dtype, int threads);
void oracle_gemm_nt_rows(const uint16_t *a, const uint16_t *b, float *c,
                         int m0, int m1, int n, int k, int dtype, int threads);
void oracle_gemm_prepare_bt(const uint16_t *b, float *bt, int n, int k, int dtype,
                            int threads);
void oracle_gemm_nt_rows_bt(const uint16_t *a, const float *bt, float *c, int m0, int m1,
                            int n, int k, int dtype, int threads);
float oracle_gemm_element(const uint16_t *a, const uint16_t *b, int k,
                          int dtype, int64_t row, int64_t col);
void oracle_round_output(const float *in, void *out, size_t n, int out_dtype);

/* ---- MXFP4 scaled GEMM (runner.cpp:718-732, :1135-1150, :1208-1283,
 *      :1565-1597; wave_matmul.py:854-950, :996-1022) ------------------- */
float oracle_mxfp4_code_value(int code);
float oracle_e8m0_value(int raw);
void oracle_mxfp4_inputs(uint8_t *out, int rows, int k, int seed, int stream,
                         int mode);
void oracle_mxfp4_scales(uint8_t *out, int rows, int k, int seed, int stream,
                         int mode);
float oracle_gemm_mxfp4_element(const uint8_t *a, const uint8_t *b,
                                const uint8_t *sa, const uint8_t *sb, int m,
                                int n, int k, int64_t row, int64_t col);
void oracle_gemm_mxfp4_rows(const uint8_t *a, const uint8_t *b,
                            const uint8_t *sa, const uint8_t *sb, float *c,
                            int m0, int m1, int m, int n, int k, int threads);
void oracle_mxfp4_aiter_b(const uint8_t *in, uint8_t *out, int n, int k);
size_t oracle_mxfp4_aiter_scales(const uint8_t *in, uint8_t *out, int rows,
                                 int k);

/* ---- flash attention ---------------------------------------------------- */
void oracle_fa_f32_inputs(uint16_t *q, uint16_t *k, uint16_t *v, int block_m,
                          int seq_n, int head_dim, int seed);
void oracle_fa_f32_reference(const uint16_t *q, const uint16_t *k,
                             const uint16_t *v, float *out, int block_m,
                             int seq_n, int head_dim);
void oracle_fa_gfx950_inputs(uint16_t *q, uint16_t *k, uint16_t *v,
                             size_t elements, int seed, int input_scale,
                             int zero_qk);
void oracle_attention_rows(const uint16_t *q, const uint16_t *k,
                           const uint16_t *v, int dtype, int batch,
                           int q_heads, int kv_heads, int seq_q, int seq_k,
                           int head_dim, int causal, double scale,
                           const int *heads, const int *rows, int count,
                           float *out, int threads);
int oracle_fa_reference_rows(int sequence, int *rows);
int oracle_fa_reference_heads(int head_count, int *heads);

/* ---- Stream-K partition (wave_matmul.py:77-165) ----------------------- */
int oracle_streamk_worker_interval(int64_t total, int workers, int worker,
                                   int64_t *begin, int64_t *end);
int64_t oracle_streamk_owner(int64_t total, int workers, int64_t iteration);
int oracle_streamk_segments(int tile_count, int k_iterations, int workers,
                            int worker, int *tiles, int *k_begin, int *k_end,
                            int *slot, int max_segments);

/* ---- misc ---------------------------------------------------------------- */
int oracle_hardware_threads(void);

#ifdef __cplusplus
}
#endif
#endif
