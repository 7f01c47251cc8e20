"""ctypes front end for oracle/liboracle.so -- the CPU restatement of the
reference's input generators and CPU references.

TEST INFRASTRUCTURE ONLY.  Importable from tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg; the product package never imports it.  See
oracle.cpp for the reference file:line each function restates and how each
is pinned.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

F32, F16, BF16 = 0, 1, 2
MODE_RANDOM, MODE_ALL_ONES, MODE_RAND_INT, MODE_HPL, MODE_HALVES = 0, 1, 2, 3, 4
MODE_PY_RANDOM = 5

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t


def build() -> None:
    """Compile liboracle.so (and oracle/_ref when the reference is present)."""
    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "oracle_rand_state": (ctypes.c_uint32, [_I, _I]),
            "oracle_next_rand": (ctypes.c_uint32, [ctypes.POINTER(ctypes.c_uint32)]),
            "oracle_bucket_value": (ctypes.c_float, [ctypes.POINTER(ctypes.c_uint32), ctypes.c_float]),
            "oracle_rand_int": (ctypes.c_float, [_SZ]),
            "oracle_hpl": (ctypes.c_float, [_SZ]),
            "oracle_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "oracle_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "oracle_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "oracle_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "oracle_f64_to_f16": (ctypes.c_uint16, [ctypes.c_double]),
            "oracle_gemm_inputs": (None, [_P, _I, _I, _I, _I, _I, _I]),
            "oracle_gemm_nt": (None, [_P, _P, _P, _I, _I, _I, _I, _I]),
            "oracle_gemm_nt_rows": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _I]),
            "oracle_gemm_prepare_bt": (None, [_P, _P, _I, _I, _I, _I]),
            "oracle_gemm_nt_rows_bt": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _I]),
            "oracle_gemm_element": (ctypes.c_float, [_P, _P, _I, _I, _I64, _I64]),
            "oracle_round_output": (None, [_P, _P, _SZ, _I]),
            "oracle_mxfp4_code_value": (ctypes.c_float, [_I]),
            "oracle_e8m0_value": (ctypes.c_float, [_I]),
            "oracle_mxfp4_inputs": (None, [_P, _I, _I, _I, _I, _I]),
            "oracle_mxfp4_scales": (None, [_P, _I, _I, _I, _I, _I]),
            "oracle_gemm_mxfp4_element": (ctypes.c_float, [_P, _P, _P, _P, _I, _I, _I, _I64,
                                                           _I64]),
            "oracle_gemm_mxfp4_rows": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
            "oracle_mxfp4_aiter_b": (None, [_P, _P, _I, _I]),
            "oracle_mxfp4_aiter_scales": (_SZ, [_P, _P, _I, _I]),
            "oracle_fa_f32_inputs": (None, [_P, _P, _P, _I, _I, _I, _I]),
            "oracle_fa_f32_reference": (None, [_P, _P, _P, _P, _I, _I, _I]),
            "oracle_fa_gfx950_inputs": (None, [_P, _P, _P, _SZ, _I, _I, _I]),
            "oracle_attention_rows": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                                             ctypes.c_double, _P, _P, _I, _P, _I]),
            "oracle_fa_reference_rows": (_I, [_I, _P]),
            "oracle_fa_reference_heads": (_I, [_I, _P]),
            "oracle_streamk_worker_interval": (_I, [_I64, _I, _I, ctypes.POINTER(_I64), ctypes.POINTER(_I64)]),
            "oracle_streamk_owner": (_I64, [_I64, _I, _I64]),
            "oracle_streamk_segments": (_I, [_I, _I, _I, _I, _P, _P, _P, _P, _I]),
            "oracle_hardware_threads": (_I, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def hardware_threads() -> int:
    return lib().oracle_hardware_threads()


# ---- generators --------------------------------------------------------
def gemm_inputs(rows: int, k: int, dtype: int = F16, seed: int = 0, stream: int = 0,
                mode: int = MODE_RANDOM) -> np.ndarray:
    out = np.empty(rows * k, dtype=np.uint16)
    lib().oracle_gemm_inputs(_ptr(out), rows, k, dtype, seed, stream, mode)
    return out.reshape(rows, k)


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bits_to_f32(bits: np.ndarray, dtype: int) -> np.ndarray:
    return bf16_bits_to_f32(bits) if dtype == BF16 else f16_bits_to_f32(bits)


def round_output(c: np.ndarray, out_dtype: int) -> np.ndarray:
    c = np.ascontiguousarray(c, dtype=np.float32)
    if out_dtype == F32:
        return c.copy()
    out = np.empty(c.shape, dtype=np.uint16)
    lib().oracle_round_output(_ptr(c), _ptr(out), c.size, out_dtype)
    return out


# ---- GEMM reference ------------------------------------------------------
def gemm_nt(a: np.ndarray, b: np.ndarray, dtype: int = F16, threads: int | None = None) -> np.ndarray:
    """C[M,N] = A[M,K] . B[N,K]^T, float accumulation in ascending k."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    m, k = a.shape
    n, k2 = b.shape
    assert k == k2
    c = np.empty((m, n), dtype=np.float32)
    lib().oracle_gemm_nt(_ptr(a), _ptr(b), _ptr(c), m, n, k, dtype,
                         threads or hardware_threads())
    return c


def gemm_nt_rows(a: np.ndarray, b: np.ndarray, m0: int, m1: int, dtype: int = F16,
                 threads: int | None = None) -> np.ndarray:
    """Rows [m0, m1) of A . B^T (same arithmetic as gemm_nt)."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    m, k = a.shape
    n = b.shape[0]
    c = np.zeros((m, n), dtype=np.float32)
    lib().oracle_gemm_nt_rows(_ptr(a), _ptr(b), _ptr(c), m0, m1, n, k, dtype,
                              threads or hardware_threads())
    return c[m0:m1]


def gemm_prepare_bt(b: np.ndarray, dtype: int = F16, threads: int | None = None) -> np.ndarray:
    """B [N x K] (16-bit bits) widened to float and transposed, [K][N]: the
    operand gemm_nt_rows_bt takes."""
    b = np.ascontiguousarray(b, dtype=np.uint16)
    n, k = b.shape
    bt = np.empty((k, n), dtype=np.float32)
    lib().oracle_gemm_prepare_bt(_ptr(b), _ptr(bt), n, k, dtype, threads or hardware_threads())
    return bt


def gemm_nt_rows_bt(a: np.ndarray, bt: np.ndarray, m0: int, m1: int, dtype: int = F16,
                    threads: int | None = None, out: np.ndarray | None = None) -> np.ndarray:
    """Rows [m0, m1) of A . B^T from a prepared B^T (gemm_prepare_bt); same
    arithmetic as gemm_nt.  `out`: a float32 [m1 - m0, N] buffer to write."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    bt = np.ascontiguousarray(bt, dtype=np.float32)
    k, n = bt.shape
    assert a.shape[1] == k and 0 <= m0 <= m1 <= a.shape[0]
    if out is None:
        out = np.empty((m1 - m0, n), dtype=np.float32)
    assert out.shape == (m1 - m0, n) and out.dtype == np.float32 and out.flags.c_contiguous
    lib().oracle_gemm_nt_rows_bt(_ptr(a), _ptr(bt), _ptr(out), m0, m1, n, k, dtype,
                                 threads or hardware_threads())
    return out


def gemm_elements(a: np.ndarray, b: np.ndarray, rows, cols, dtype: int = F16) -> np.ndarray:
    """Sampled C[rows[i], cols[i]] with the runner's per-element arithmetic."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    k = a.shape[1]
    L = lib()
    return np.array([L.oracle_gemm_element(_ptr(a), _ptr(b), k, dtype, int(r), int(c))
                     for r, c in zip(rows, cols)], dtype=np.float32)


# ---- MXFP4 ------------------------------------------------------------------------
def mxfp4_inputs(rows: int, k: int, seed: int = 0, stream: int = 0,
                 mode: int = MODE_RANDOM) -> np.ndarray:
    """Packed e2m1 codes [rows, k/2] (low nibble = even k)."""
    out = np.empty(rows * k // 2, dtype=np.uint8)
    lib().oracle_mxfp4_inputs(_ptr(out), rows, k, seed, stream, mode)
    return out.reshape(rows, k // 2)


def mxfp4_scales(rows: int, k: int, seed: int = 0, stream: int = 2,
                 mode: int = MODE_RANDOM) -> np.ndarray:
    """Group-major e8m0 scales [k/32, rows] (stream 2 = A, 3 = B)."""
    out = np.empty(rows * (k // 32), dtype=np.uint8)
    lib().oracle_mxfp4_scales(_ptr(out), rows, k, seed, stream, mode)
    return out.reshape(k // 32, rows)


def mxfp4_operands(m: int, n: int, k: int, seed: int = 0, mode: int = MODE_RANDOM):
    """(A, B, A_scale, B_scale) as the runner (RANDOM / ALL_ONES) or the
    Python builder (HALVES / PY_RANDOM) makes them."""
    return (mxfp4_inputs(m, k, seed, 0, mode), mxfp4_inputs(n, k, seed, 1, mode),
            mxfp4_scales(m, k, seed, 2, mode), mxfp4_scales(n, k, seed, 3, mode))


def gemm_mxfp4_rows(a, b, sa, sb, m0: int, m1: int, threads: int | None = None) -> np.ndarray:
    """Rows [m0, m1) of the MXFP4 product, the runner's float accumulation."""
    a, b, sa, sb = (np.ascontiguousarray(x, dtype=np.uint8) for x in (a, b, sa, sb))
    m, n, k = a.shape[0], b.shape[0], 2 * a.shape[1]
    c = np.zeros((m, n), dtype=np.float32)
    lib().oracle_gemm_mxfp4_rows(_ptr(a), _ptr(b), _ptr(sa), _ptr(sb), _ptr(c), m0, m1, m, n,
                                 k, threads or hardware_threads())
    return c[m0:m1]


def gemm_mxfp4(a, b, sa, sb, threads: int | None = None) -> np.ndarray:
    return gemm_mxfp4_rows(a, b, sa, sb, 0, a.shape[0], threads)


def gemm_mxfp4_elements(a, b, sa, sb, rows, cols) -> np.ndarray:
    a, b, sa, sb = (np.ascontiguousarray(x, dtype=np.uint8) for x in (a, b, sa, sb))
    m, n, k = a.shape[0], b.shape[0], 2 * a.shape[1]
    L = lib()
    return np.array([L.oracle_gemm_mxfp4_element(_ptr(a), _ptr(b), _ptr(sa), _ptr(sb), m, n,
                                                 k, int(r), int(c))
                     for r, c in zip(rows, cols)], dtype=np.float32)


def mxfp4_aiter_b(b: np.ndarray, n: int, k: int) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(b.size, dtype=np.uint8)
    lib().oracle_mxfp4_aiter_b(_ptr(b), _ptr(out), n, k)
    return out


def mxfp4_aiter_scales(s: np.ndarray, rows: int, k: int) -> np.ndarray:
    s = np.ascontiguousarray(s, dtype=np.uint8)
    size = lib().oracle_mxfp4_aiter_scales(_ptr(s), None, rows, k)
    out = np.empty(size, dtype=np.uint8)
    lib().oracle_mxfp4_aiter_scales(_ptr(s), _ptr(out), rows, k)
    return out


# ---- flash attention ----------------------------------------------------------
def fa_f32_inputs(block_m: int, seq_n: int, head_dim: int, seed: int = 0):
    q = np.empty(block_m * head_dim, dtype=np.uint16)
    k = np.empty(seq_n * head_dim, dtype=np.uint16)
    v = np.empty(seq_n * head_dim, dtype=np.uint16)
    lib().oracle_fa_f32_inputs(_ptr(q), _ptr(k), _ptr(v), block_m, seq_n, head_dim, seed)
    return q.reshape(block_m, head_dim), k.reshape(seq_n, head_dim), v.reshape(seq_n, head_dim)


def fa_f32_reference(q, k, v) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    block_m, head_dim = q.shape
    seq_n = k.shape[0]
    out = np.empty((block_m, head_dim), dtype=np.float32)
    lib().oracle_fa_f32_reference(_ptr(q), _ptr(k), _ptr(v), _ptr(out), block_m, seq_n, head_dim)
    return out


def fa_gfx950_inputs(elements: int, seed: int = 0, input_scale: int = 1, zero_qk: bool = False):
    q = np.empty(elements, dtype=np.uint16)
    k = np.empty(elements, dtype=np.uint16)
    v = np.empty(elements, dtype=np.uint16)
    lib().oracle_fa_gfx950_inputs(_ptr(q), _ptr(k), _ptr(v), elements, seed, input_scale,
                                  int(zero_qk))
    return q, k, v


def attention_rows(q, k, v, *, dtype: int, batch: int, q_heads: int, kv_heads: int,
                   seq_q: int, seq_k: int, head_dim: int, causal: bool, scale: float,
                   heads, rows, threads: int | None = None) -> np.ndarray:
    """Double-precision softmax(QK^T*scale)V for the (flat head, row) pairs."""
    q = np.ascontiguousarray(q, dtype=np.uint16).ravel()
    k = np.ascontiguousarray(k, dtype=np.uint16).ravel()
    v = np.ascontiguousarray(v, dtype=np.uint16).ravel()
    heads = np.ascontiguousarray(heads, dtype=np.int32)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    assert heads.shape == rows.shape
    out = np.empty((len(rows), head_dim), dtype=np.float32)
    lib().oracle_attention_rows(_ptr(q), _ptr(k), _ptr(v), dtype, batch, q_heads, kv_heads,
                                seq_q, seq_k, head_dim, int(causal), float(scale),
                                _ptr(heads), _ptr(rows), len(rows), _ptr(out),
                                threads or hardware_threads())
    return out


def fa_reference_rows(sequence: int) -> list[int]:
    buf = np.zeros(max(sequence, 8), dtype=np.int32)
    n = lib().oracle_fa_reference_rows(sequence, _ptr(buf))
    return buf[:n].tolist()


def fa_reference_heads(head_count: int) -> list[int]:
    buf = np.zeros(max(head_count, 4), dtype=np.int32)
    n = lib().oracle_fa_reference_heads(head_count, _ptr(buf))
    return buf[:n].tolist()


# ---- Tile-packed C ------------------------------------------------------------
def tile_packed_coords(m: int, n: int, bm: int, bn: int, wave_m_tiles: int,
                       wave_n_tiles: int) -> tuple[np.ndarray, np.ndarray]:
    """(m, n) of every element index of a tile-packed C, decoded as the
    runner's getOutputCoordinate does for wave64 MFMA accumulators
    (tools/wave-matmul-calibrate/wave-matmul-calibrate-runner.cpp:772-834):
    index -> CTA (row-major over the M_blocks x N_blocks grid), wave
    (m_wave * bn + n_wave), wave tile (i * wave_n_tiles + j), then lane =
    slot / 4 and register slot % 4, i.e. row (lane / 16) * 4 + register and
    column lane % 16 of the 16x16 tile."""
    m_rows, n_cols = 16 * bm * wave_m_tiles, 16 * bn * wave_n_tiles
    if m % m_rows or n % n_cols:
        raise ValueError("tile-packed blocking must divide M and N")
    n_blocks = n // n_cols
    wave_elems = wave_m_tiles * wave_n_tiles * 256
    cta_elems = bm * bn * wave_elems
    idx = np.arange(m * n, dtype=np.int64)
    cta, cta_rem = idx // cta_elems, idx % cta_elems
    wg_m, wg_n = cta // n_blocks, cta % n_blocks
    wave, wave_rem = cta_rem // wave_elems, cta_rem % wave_elems
    tile, slot = wave_rem // 256, wave_rem % 256
    m_wave, n_wave = wave // bn, wave % bn
    lane, reg = slot // 4, slot % 4
    m_tile = wg_m * (bm * wave_m_tiles) + m_wave * wave_m_tiles + tile // wave_n_tiles
    n_tile = wg_n * (bn * wave_n_tiles) + n_wave * wave_n_tiles + tile % wave_n_tiles
    return m_tile * 16 + (lane // 16) * 4 + reg, n_tile * 16 + lane % 16


def to_tile_packed(c: np.ndarray, bm: int, bn: int, wave_m_tiles: int,
                   wave_n_tiles: int) -> np.ndarray:
    """The row-major [M, N] array c in tile-packed order (1-D)."""
    mm, nn = tile_packed_coords(c.shape[0], c.shape[1], bm, bn, wave_m_tiles, wave_n_tiles)
    return np.ascontiguousarray(c)[mm, nn]


# ---- Stream-K partition -------------------------------------------------------
def streamk_worker_interval(total: int, workers: int, worker: int) -> tuple[int, int]:
    b, e = _I64(), _I64()
    if lib().oracle_streamk_worker_interval(total, workers, worker, ctypes.byref(b), ctypes.byref(e)):
        raise ValueError("bad Stream-K interval arguments")
    return b.value, e.value


def streamk_owner_for_iteration(total: int, workers: int, iteration: int) -> int:
    r = lib().oracle_streamk_owner(total, workers, iteration)
    if r < 0:
        raise ValueError("bad Stream-K owner arguments")
    return r


def streamk_worker_segments(tile_count: int, k_iterations: int, workers: int, worker: int):
    cap = 64
    t = np.zeros(cap, np.int32)
    kb = np.zeros(cap, np.int32)
    ke = np.zeros(cap, np.int32)
    sl = np.zeros(cap, np.int32)
    n = lib().oracle_streamk_segments(tile_count, k_iterations, workers, worker,
                                      _ptr(t), _ptr(kb), _ptr(ke), _ptr(sl), cap)
    if n < 0:
        raise ValueError("bad Stream-K segment arguments")
    return [(int(t[i]), int(kb[i]), int(ke[i]), None if sl[i] < 0 else int(sl[i]))
            for i in range(n)]


def fa_backward(q, k, v, do, *, scale: float | None = None, causal: bool = False,
                o_delta=None):
    """Float64 flash-attention forward and backward for q [B, Hq, S, D], k/v
    [B, Hkv, S, D], do [B, Hq, S, D] (arrays of the dtype-rounded values).

    Returns (o, lse, dq, dk, dv): o = softmax(scale Q K^T) V with key > query
    masked when causal, lse = ln sum_k exp(scale q.k) per row, and the
    gradients dV = P^T dO, dS = P o (dO V^T - rowsum(dO o O)), dQ = scale dS K,
    dK = scale dS^T Q, with dK and dV summed over the q heads of each KV head.
    No reference counterpart (the reference has no backward): these are the
    textbook gradients of softmax attention, pinned against torch autograd
    in tests/test_oracle_fa_bwd.py.  o_delta: the O to use in
    rowsum(dO o O) (a kernel's own rounded output), default the exact one."""
    q, k, v, do = (np.asarray(x, dtype=np.float64) for x in (q, k, v, do))
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    sc = 1.0 / np.sqrt(D) if not scale else float(scale)
    kk = np.repeat(k, g, axis=1)
    vv = np.repeat(v, g, axis=1)
    kt = np.swapaxes(kk, -1, -2)
    s = sc * np.matmul(q, kt)
    if causal:
        mask = np.triu(np.ones((S, S), dtype=bool), 1)
        s = np.where(mask, -np.inf, s)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    tot = e.sum(axis=-1, keepdims=True)
    p = e / tot
    lse = (m + np.log(tot))[..., 0]
    o = np.matmul(p, vv)
    dvv = np.matmul(np.swapaxes(p, -1, -2), do)
    dp = np.matmul(do, np.swapaxes(vv, -1, -2))
    o_d = o if o_delta is None else np.asarray(o_delta, dtype=np.float64)
    delta = (do * o_d).sum(axis=-1, keepdims=True)
    ds = p * (dp - delta)
    dq = sc * np.matmul(ds, kk)
    dkk = sc * np.matmul(np.swapaxes(ds, -1, -2), q)
    dk = dkk.reshape(B, Hkv, g, S, D).sum(axis=2)
    dv = dvv.reshape(B, Hkv, g, S, D).sum(axis=2)
    return o, lse, dq, dk, dv


# ---- block-scaled FP8 (OCP MX-FP8) ---------------------------------------------
# No reference counterpart: the reference only names a block-scaled FP8 attention
# contract as future work (docs/PerfReferences/WaveGfx950FlashAttention.md:94-99).
# The formats are the OCP ones (OCP 8-bit Floating Point Specification, E4M3;
# OCP Microscaling Formats (MX) v1.0, E8M0 scales over blocks of 32).  Pinned
# in tests/test_mxfp8_oracle.py: every e4m3 code against torch's float8_e4m3fn
# conversion, e8m0 against its closed form, and the attention against
# attention computed by torch in float64 on the same decoded values.

def _e4m3_table() -> np.ndarray:
    t = np.empty(256, dtype=np.float64)
    for b in range(256):
        sign = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 7
        if e == 0xF and m == 7:
            t[b] = np.nan
        elif e == 0:
            t[b] = sign * m * 2.0 ** -9
        else:
            t[b] = sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


_E4M3 = _e4m3_table()


def e4m3_to_float(b: np.ndarray) -> np.ndarray:
    """OCP E4M3 bytes -> float64: sign, 4-bit exponent (bias 7), 3-bit
    mantissa; exponent 0 is subnormal (m * 2^-9); 0x7F / 0xFF are NaN."""
    return _E4M3[np.asarray(b, dtype=np.uint8)]


def e8m0_to_float(b: np.ndarray) -> np.ndarray:
    """E8M0 scale bytes -> 2^(b - 127) (255 is NaN)."""
    b = np.asarray(b, dtype=np.uint8).astype(np.float64)
    return np.where(b == 255, np.nan, np.exp2(b - 127.0))


def mxfp8_decode(elems: np.ndarray, scales: np.ndarray, axis: int) -> np.ndarray:
    """Decode MX-FP8: each e4m3 element times the e8m0 scale of its block of
    32 along `axis` (scales has that axis divided by 32, rounded up)."""
    x = e4m3_to_float(elems)
    sc = np.repeat(e8m0_to_float(scales), 32, axis=axis)
    sc = np.take(sc, np.arange(x.shape[axis]), axis=axis)
    return x * sc


def attention_forward(q, k, v, *, scale: float | None = None, causal: bool = False):
    """Float64 softmax(scale Q K^T) V for q [B, Hq, S, D], k / v [B, Hkv, S, D]
    (kv head = q head / (Hq / Hkv)), key > query masked when causal.  Returns
    (o, lse) with lse = ln sum_k exp(scale q.k)."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    B, Hq, S, D = q.shape
    g = Hq // k.shape[1]
    sc = 1.0 / np.sqrt(D) if not scale else float(scale)
    kk = np.repeat(k, g, axis=1)
    vv = np.repeat(v, g, axis=1)
    s = sc * np.matmul(q, np.swapaxes(kk, -1, -2))
    if causal:
        s = np.where(np.triu(np.ones((S, S), dtype=bool), 1), -np.inf, s)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    tot = e.sum(axis=-1, keepdims=True)
    return np.matmul(e / tot, vv), (m + np.log(tot))[..., 0]

