// wave_common.hpp -- shared CDNA4 (gfx950) device helpers for the GEMM and
// flash-attention kernels: vector types, MFMA wrappers, LDS address helpers,
// the asynchronous global->LDS DMA issue, and output conversions.
//
// Everything here is written for wave64 gfx950 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wave {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Element type codes of the C ABI (include/wave_runtime.h).
// kMXFP4: packed e2m1 with group-major e8m0 scales (canonical layout);
// kMXFP4A: the same values with B and both scale arrays in the AITER
// preshuffled layouts.
enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2, kMXFP4 = 3, kMXFP4A = 4 };
constexpr bool is_fp4(int dt) { return dt == kMXFP4 || dt == kMXFP4A; }

// v_mfma_f32_32x32x16_{f16,bf16}: D[32x32] += A[32x16] * B[16x32].
// Lane l supplies A[l%32][8*(l/32) .. +8] and B[8*(l/32) .. +8][l%32] as
// eight packed 16-bit values; accumulator register r of lane l holds
// D[8*(r/4) + 4*(l/32) + r%4][l%32].
template <int DT>
__device__ __forceinline__ f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == kF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
        0);
}

// v_mfma_f32_16x16x32_{f16,bf16} on an AGPR accumulator, in place:
// D[16x16] += A[16x32] * B[32x16].  Lane l supplies A[l%16][8*(l/16) .. +8]
// and B[8*(l/16) .. +8][l%16]; accumulator register r of lane l holds
// D[4*(l/16) + r][l%16].  Issued from inline asm: with the builtin, hipcc
// copies srcC into a scratch AGPR tuple for most of a 64-tile (256-AGPR)
// accumulator grid and spills.  The compiler's hazard checks do not see an
// asm MFMA, so the caller keeps two rules: an accumulator written by VALU
// (its zero fill) is at least 2 wait states old when an MFMA reads it, and
// mfma_asm_drain() separates the last MFMA from any other access to its
// accumulators.  srcA/srcB need nothing beyond the s_waitcnt the compiler
// inserts for their LDS loads (the MFMA reads them at issue).
template <int DT>
__device__ __forceinline__ void mfma16x16x32_acc(f32x4 &acc, u32x4 a, u32x4 b) {
  if constexpr (DT == kF16)
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// 24 wait states: more than the 8-pass MFMA's result latency (passes + 3).
__device__ __forceinline__ void mfma_asm_drain() {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
}

// v_mfma_scale_f32_32x32x64_f8f6f4 with fp4 (e2m1) A and B: D[32x32] +=
// (A * sa)[32x64] * (B * sb)[64x32].  Lane l supplies 32 fp4 values (16
// bytes, two per byte, low nibble first) of row l%32 (A) / column l%32 (B)
// at K offset 32*(l/32), and in byte 0 of sa / sb the e8m0 scale
// 2^(raw-127) of exactly those 32 values; the accumulator layout is that of
// the 16-bit 32x32 MFMA above (layout checked by the MXFP4 parity tests).
__device__ __forceinline__ f32x16 mfma_fp4_32x32x64(u32x4 a, u32x4 b, f32x16 c, uint32_t sa,
                                                    uint32_t sb) {
  typedef int i32x8 __attribute__((ext_vector_type(8)));
  const i32x8 av = {(int)a[0], (int)a[1], (int)a[2], (int)a[3], 0, 0, 0, 0};
  const i32x8 bv = {(int)b[0], (int)b[1], (int)b[2], (int)b[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 4, 4, 0, (int)sa, 0,
                                                         (int)sb);
}

// v_mfma_scale_f32_16x16x128_f8f6f4 with fp4 (e2m1) A and B on an AGPR
// accumulator, in place: D[16x16] += (A * sa)[16x128] * (B * sb)[128x16].
// Lane l supplies 32 fp4 values (16 bytes, low nibble first) of row l%16
// (A) / column l%16 (B) at K offset 32*(l/16), and in byte 0 of sa / sb the
// e8m0 scale of exactly those 32 values; accumulator layout as
// mfma16x16x32_acc, and the same asm hazard rules.
__device__ __forceinline__ void mfma_fp4_16x16x128_acc(f32x4 &acc, u32x4 a, u32x4 b,
                                                       uint32_t sa, uint32_t sb) {
  asm volatile("v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel_hi:[0,0,0] "
               "cbsz:4 blgp:4"
               : "+a"(acc)
               : "v"(a), "v"(b), "v"(sa), "v"(sb));
}

// x from this lane (a) and from lane l ^ 32 (b), ordered by lane half: in
// every lane a holds the lower-half lane's value and b the upper-half
// lane's, so a + b and max(a, b) are bit-identical across the pair.  One
// v_permlane32_swap_b32 (gfx950: swaps the upper 32 lanes of its first
// operand with the lower 32 lanes of its second) instead of an LDS
// permute.  Inline asm with two registers: hipcc folds the builtin's two
// results into one register when both operands are the same value.  The
// s_nops give the swap's VALU read/write hazards their wait states.
__device__ __forceinline__ void half_pair(float x, float &a, float &b) {
  uint32_t lo = __builtin_bit_cast(uint32_t, x), hi = lo;
  asm volatile("s_nop 2\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 2" : "+v"(lo), "+v"(hi));
  a = __builtin_bit_cast(float, lo);
  b = __builtin_bit_cast(float, hi);
}

// 32-bit LDS byte address of a __shared__ object (address space 3).
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}

// Direct global->LDS copy of 16 bytes per lane (global_load_lds_dwordx4).
// Lane l's 16 bytes land at LDS byte lds + 16*l, so one call fills a
// contiguous 1 KiB LDS window.  `lds` and `base` must be wave-uniform; the
// per-lane source is base + voff.  Issued from inline asm so that the
// compiler does not insert its own conservative vmcnt waits in front of the
// LDS reads of the *other* buffer; callers synchronise explicitly with
// vm_wait_barrier().  No memory clobber: the DMA only writes an LDS buffer
// that no instruction between two barriers reads, so LDS reads of the
// current buffer may be scheduled around it.  M0 is written here and nowhere
// else in these kernels.
__device__ __forceinline__ void dma16(uint32_t lds, const void *base,
                                      uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\t"
               "s_nop 0\n\t"
               "global_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds), "v"(voff), "s"(base));
}

// The same with 4 bytes per lane: 64 lanes fill 256 bytes of LDS at
// lds + 4 * lane.
__device__ __forceinline__ void dma4(uint32_t lds, const void *base, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\t"
               "s_nop 0\n\t"
               "global_load_lds_dword %1, %2"
               :
               : "s"(lds), "v"(voff), "s"(base));
}

// Wait until this wave's outstanding vector-memory operations (including the
// LDS DMA above) have completed, then join the workgroup barrier.  The asm
// memory clobber also stops the compiler moving LDS accesses across it.
// VMCNT: how many of this wave's most recent vector-memory operations may
// still be in flight (DMA issued in order completes in order).
template <int VMCNT = 0> __device__ __forceinline__ void vm_wait_barrier() {
  static_assert(VMCNT >= 0 && VMCNT < 64, "vmcnt field is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(VMCNT)
               : "memory");
}

// Device-coherent 16-byte loads and stores through a buffer resource over
// [base, base + bytes).  Cache policy sc1 (sc0 clear) is what gfx950 gives
// agent-scope atomic accesses: they read and write the device's coherence
// point, never a stale or dirty line of one XCD's L2, so data that CTAs on
// different XCDs exchange within a launch this way needs no L2 write-back
// (release) or invalidate (acquire) around it -- only the waits that order
// the accesses: the writer's vmcnt(0) before it signals, the reader's loads
// issued after it has seen the signal.
constexpr int kCoherentDevice = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void *base,
                                                                uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}
// The byte offset is voff (per lane, range-checked against `bytes`) plus
// soff (wave-uniform, an SGPR or constant; not range-checked, so callers
// keep voff + soff inside the buffer by construction).  Splitting a
// per-thread base from a per-access constant keeps one offset VGPR for a
// whole run of accesses.
__device__ __forceinline__ f32x4 coherent_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                 uint32_t soff = 0) {
  return __builtin_bit_cast(
      f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kCoherentDevice));
}
__device__ __forceinline__ void coherent_store16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                 f32x4 v, uint32_t soff = 0) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, voff, soff,
                                         kCoherentDevice);
}

__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
  return __builtin_amdgcn_readfirstlane(v);
}

// Round-to-nearest-even float -> 16-bit storage.
template <int DT> __device__ __forceinline__ uint16_t to_bits(float v) {
  if constexpr (DT == kF16)
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  else
    return __builtin_bit_cast(uint16_t, (__bf16)v);
}

template <int DT> __device__ __forceinline__ float from_bits(uint16_t v) {
  if constexpr (DT == kF16)
    return (float)__builtin_bit_cast(_Float16, v);
  else
    return __builtin_bit_cast(float, (uint32_t)v << 16);
}

// Pack two floats into one dword of 16-bit values (lo, hi), RNE: one
// v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
template <int DT> __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  if constexpr (DT == kF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// 16-bit bit pattern of 1.0 in both halves of a dword.
template <int DT> constexpr uint32_t kOnePair = DT == kF16 ? 0x3C003C00u : 0x3F803F80u;

} // namespace wave
