"""Record golden vectors from the reference runners' own CPU code.

Runs ONLY in the build container, where /root/reference exists and
oracle/_ref/*.so have been compiled from the reference runner sources by
oracle/Makefile.  Writes small JSON fixtures next to this script; the tests
compare the repo's own oracle (oracle/liboracle.so) against them, so parity of
the oracle is pinned to the reference's code even where the reference is
absent (the GPU box).

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import ctypes
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = os.path.join(ROOT, "oracle", "_ref")

P = ctypes.c_void_p


def load(name: str) -> ctypes.CDLL:
    path = os.path.join(REF, name)
    if not os.path.exists(path):
        sys.exit(f"{path} missing: run `make -C oracle ref` in the build container")
    return ctypes.CDLL(path)


def ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def matmul_vectors() -> dict:
    L = load("libref_matmul.so")
    L.ref_random_input_value.restype = ctypes.c_float
    L.ref_random_input_value.argtypes = [ctypes.POINTER(ctypes.c_uint32)]
    L.ref_rand_state.restype = ctypes.c_uint32
    L.ref_rand_state.argtypes = [ctypes.c_int, ctypes.c_int]
    L.ref_hipblaslt_rand_int.restype = ctypes.c_float
    L.ref_hipblaslt_rand_int.argtypes = [ctypes.c_size_t]
    L.ref_hipblaslt_hpl.restype = ctypes.c_float
    L.ref_hipblaslt_hpl.argtypes = [ctypes.c_size_t]
    L.ref_float_to_half_bits.restype = ctypes.c_uint16
    L.ref_float_to_half_bits.argtypes = [ctypes.c_float]
    L.ref_float_to_bf16_bits.restype = ctypes.c_uint16
    L.ref_float_to_bf16_bits.argtypes = [ctypes.c_float]
    L.ref_half_to_float.restype = ctypes.c_float
    L.ref_half_to_float.argtypes = [ctypes.c_uint16]
    L.ref_make_input_bytes.argtypes = [ctypes.c_int] * 8 + [P]
    L.ref_gemm_expected.argtypes = [ctypes.c_int] * 7 + [P]
    L.ref_output_coordinate.argtypes = [ctypes.c_int] * 3 + [P, P]
    L.ref_streamk_workspace.argtypes = [ctypes.c_int] * 4 + [P, P, P, P]

    out: dict = {}
    # bucket LCG (runner.cpp:681-694), seeds 0/7/91, streams 0..2
    buckets = {}
    for seed in (0, 7, 91):
        for stream in (0, 1, 2):
            st = ctypes.c_uint32(L.ref_rand_state(seed, stream))
            buckets[f"{seed}:{stream}"] = {
                "state0": st.value,
                "values": [L.ref_random_input_value(ctypes.byref(st)) for _ in range(64)],
            }
    out["bucket"] = buckets
    out["rand_int"] = [L.ref_hipblaslt_rand_int(i) for i in range(256)]
    out["hpl"] = [L.ref_hipblaslt_hpl(i) for i in range(256)]

    rng = np.random.default_rng(1234)
    floats = np.concatenate([
        rng.standard_normal(2000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(500) * 1e-5).astype(np.float32),  # f16 subnormal range
        (rng.standard_normal(500) * 3e4).astype(np.float32),   # near f16 overflow
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, -2.98e-8, 6.1e-5], dtype=np.float32),
    ])
    out["convert_inputs"] = [float(x) for x in floats]
    out["f16_bits"] = [int(L.ref_float_to_half_bits(float(x))) for x in floats]
    out["bf16_bits"] = [int(L.ref_float_to_bf16_bits(float(x))) for x in floats]
    halves = np.arange(0, 65536, 7, dtype=np.uint16)
    out["half_to_float_inputs"] = [int(h) for h in halves]
    out["half_to_float"] = [L.ref_half_to_float(int(h)) for h in halves]

    # makeInputBytes for every (dtype, mode, stream) on a 3x5 and a 7x9 shape
    inputs = {}
    for dtype, dname in ((1, "f16"), (2, "bf16")):
        for mode, (ones, rint, hpl) in {"random": (0, 0, 0), "all_ones": (1, 0, 0),
                                         "rand_int": (0, 1, 0), "hpl": (0, 0, 1)}.items():
            for rows, k in ((3, 5), (7, 9)):
                for stream in (0, 1):
                    buf = np.zeros(rows * k * 2, dtype=np.uint8)
                    L.ref_make_input_bytes(rows, k, dtype, 7, stream, ones, rint, hpl, ptr(buf))
                    inputs[f"{dname}:{mode}:{rows}x{k}:{stream}"] = buf.view(np.uint16).tolist()
    out["inputs_seed7"] = inputs

    # computeExpectedElement + roundExpectedOutput (runner.cpp:1586-1597, :738)
    gemms = {}
    cases = [
        # (m, n, k, dtype, seed, mode, out_type)
        (32, 32, 64, 1, 7, 0, 0),     # config 1 (f16 in, f32 out, seed 7)
        (32, 32, 64, 1, 7, 0, 1),     # config 1 with f16 out
        (32, 32, 64, 2, 7, 0, 0),     # bf16 in
        (64, 96, 64, 1, 37, 0, 0),    # wave_mfma_tiled.mlir shape, seed 37
        (2, 2, 4, 1, 0, 2, 0),        # rand_int golden {0,-2,2,-2}
        (2, 2, 4, 2, 0, 2, 0),
        (8, 8, 16, 1, 0, 3, 0),       # HPL
        (8, 8, 16, 2, 0, 3, 2),       # HPL bf16 out
        (16, 16, 512, 1, 91, 0, 1),   # f16 rounding case, seed 91
        (16, 24, 48, 1, 3, 2, 1),     # rand_int f16 out
    ]
    for (m, n, k, dtype, seed, mode, ot) in cases:
        buf = np.zeros(m * n, dtype=np.float64)
        L.ref_gemm_expected(m, n, k, dtype, seed, mode, ot, ptr(buf))
        gemms[f"{m}x{n}x{k}:{dtype}:{seed}:{mode}:{ot}"] = buf.tolist()
    out["gemm_expected"] = gemms

    coords = {}
    for ws, wmma in ((64, 0), (32, 1), (32, 0)):
        mm = ctypes.c_int()
        nn = ctypes.c_int()
        vals = []
        for idx in range(256):
            L.ref_output_coordinate(ws, wmma, idx, ctypes.byref(mm), ctypes.byref(nn))
            vals.append([mm.value, nn.value])
        coords[f"{ws}:{wmma}"] = vals
    out["output_coordinates"] = coords

    # Tile-packed C: the runner's getOutputCoordinate over whole blockings
    # (small ones in full; the 16-wave profile's as a sample plus a digest).
    L.ref_tile_packed_coordinate.argtypes = [ctypes.c_int] * 7 + [P, P]
    packed = {}
    for (m, n, bm, bn, wmt, wnt) in ((32, 64, 1, 2, 2, 1), (64, 96, 2, 1, 2, 3),
                                     (128, 64, 2, 2, 1, 2), (1024, 512, 4, 4, 4, 4)):
        mm = ctypes.c_int()
        nn = ctypes.c_int()
        coords = np.zeros((m * n, 2), np.int32)
        for idx in range(m * n):
            L.ref_tile_packed_coordinate(m, n, bm, bn, wmt, wnt, idx, ctypes.byref(mm),
                                         ctypes.byref(nn))
            coords[idx] = (mm.value, nn.value)
        key = f"{m}x{n}:{bm}:{bn}:{wmt}:{wnt}"
        if m * n <= 8192:
            packed[key] = {"coords": coords.tolist()}
        else:
            sample = list(range(0, m * n, 4093)) + [m * n - 1]
            packed[key] = {"sample_index": sample, "sample": coords[sample].tolist(),
                           "sha256": hashlib.sha256(coords.tobytes()).hexdigest()}
    out["tile_packed_coordinates"] = packed

    ws = {}
    for (m, n, k, w) in ((512, 256, 256, 5), (512, 512, 256, 2), (8192, 8192, 8192, 256),
                         (2048, 2048, 8192, 128)):
        sc = ctypes.c_uint64()
        cn = ctypes.c_uint64()
        gx = ctypes.c_int()
        bl = ctypes.c_int()
        L.ref_streamk_workspace(m, n, k, w, ctypes.byref(sc), ctypes.byref(cn),
                                ctypes.byref(gx), ctypes.byref(bl))
        ws[f"{m}x{n}x{k}:{w}"] = [sc.value, cn.value, gx.value, bl.value]
    out["streamk_workspace"] = ws
    return out


def mxfp4_vectors() -> dict:
    """The runner's MXFP4 generators, expected outputs and AITER shuffles
    (runner.cpp:1135-1150, :1208-1283, :1436-1456, :1565-1597)."""
    L = load("libref_matmul.so")
    L.ref_mxfp4_input_bytes.argtypes = [ctypes.c_int] * 5 + [P]
    L.ref_mxfp4_scale_bytes.argtypes = [ctypes.c_int] * 5 + [P]
    L.ref_mxfp4_code_to_float.restype = ctypes.c_float
    L.ref_mxfp4_code_to_float.argtypes = [ctypes.c_int]
    L.ref_e8m0_to_float.restype = ctypes.c_float
    L.ref_e8m0_to_float.argtypes = [ctypes.c_int]
    L.ref_gemm_mxfp4_expected.argtypes = [ctypes.c_int] * 6 + [P]
    L.ref_mxfp4_aiter_b.argtypes = [P, ctypes.c_int, ctypes.c_int, P]
    L.ref_mxfp4_aiter_scales.restype = ctypes.c_size_t
    L.ref_mxfp4_aiter_scales.argtypes = [P, ctypes.c_int, ctypes.c_int, P]

    out: dict = {}
    out["code_to_float"] = [L.ref_mxfp4_code_to_float(c) for c in range(16)]
    out["e8m0_to_float"] = [L.ref_e8m0_to_float(r) for r in range(100, 140)]
    inputs, scales = {}, {}
    for seed in (0, 7):
        for ones in (0, 1):
            for (rows, k) in ((4, 64), (16, 128)):
                for stream in (0, 1):
                    buf = np.zeros(rows * k // 2, np.uint8)
                    L.ref_mxfp4_input_bytes(rows, k, seed, stream, ones, ptr(buf))
                    inputs[f"{seed}:{ones}:{rows}x{k}:{stream}"] = buf.tolist()
                for stream in (2, 3):
                    buf = np.zeros(rows * k // 32, np.uint8)
                    L.ref_mxfp4_scale_bytes(rows, k, seed, stream, ones, ptr(buf))
                    scales[f"{seed}:{ones}:{rows}x{k}:{stream}"] = buf.tolist()
    out["inputs"] = inputs
    out["scales"] = scales
    gemms = {}
    for (m, n, k, seed, ones, ot) in ((16, 16, 128, 7, 0, 0), (32, 16, 256, 0, 0, 0),
                                      (16, 32, 128, 7, 0, 1), (16, 16, 128, 3, 0, 2),
                                      (16, 16, 256, 7, 1, 0)):
        buf = np.zeros(m * n, np.float64)
        L.ref_gemm_mxfp4_expected(m, n, k, seed, ones, ot, ptr(buf))
        gemms[f"{m}x{n}x{k}:{seed}:{ones}:{ot}"] = buf.tolist()
    out["gemm_expected"] = gemms
    rng = np.random.default_rng(5)
    b = rng.integers(0, 256, 32 * 64, dtype=np.uint8)
    sb = np.zeros(32 * 64, np.uint8)
    L.ref_mxfp4_aiter_b(ptr(b), 32, 128, ptr(sb))
    out["aiter_b"] = {"n": 32, "k": 128, "in": b.tolist(), "out": sb.tolist()}
    s = rng.integers(0, 256, 40 * 12, dtype=np.uint8)  # 40 rows, K = 384 (12 groups)
    size = L.ref_mxfp4_aiter_scales(ptr(s), 40, 384, None)
    ss = np.zeros(size, np.uint8)
    L.ref_mxfp4_aiter_scales(ptr(s), 40, 384, ptr(ss))
    out["aiter_scales"] = {"rows": 40, "k": 384, "in": s.tolist(), "out": ss.tolist()}
    return out


def fa_vectors() -> dict:
    out: dict = {}
    L32 = load("libref_fa_f32.so")
    L32.ref_fa_f32_inputs_and_reference.argtypes = [ctypes.c_int] * 4 + [P] * 4
    f32 = {}
    for (bm, sn, hd, seed) in ((16, 16, 32, 11), (16, 32, 32, 11), (16, 32, 16, 11),
                               (16, 64, 64, 0), (16, 128, 128, 5)):
        q = np.zeros(bm * hd, np.uint16)
        k = np.zeros(sn * hd, np.uint16)
        v = np.zeros(sn * hd, np.uint16)
        o = np.zeros(bm * hd, np.float32)
        L32.ref_fa_f32_inputs_and_reference(bm, sn, hd, seed, ptr(q), ptr(k), ptr(v), ptr(o))
        f32[f"{bm}:{sn}:{hd}:{seed}"] = {"q": q.tolist(), "k": k.tolist(), "v": v.tolist(),
                                        "o": o.tolist()}
    out["fa_f32"] = f32

    L950 = load("libref_fa_gfx950.so")
    L950.ref_fa_gfx950_make_input.argtypes = [ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_float, P]
    L950.ref_fa_gfx950_attention_row.argtypes = [ctypes.c_int] * 3 + [P] * 3 + [ctypes.c_int] * 2 + [P]
    g = {}
    for (b, h, s, seed, iscale) in ((1, 1, 256, 0, 1), (1, 2, 256, 3, 4), (2, 1, 512, 9, 1)):
        n = b * h * s * 128
        q = np.zeros(n, np.uint16)
        k = np.zeros(n, np.uint16)
        v = np.zeros(n, np.uint16)
        L950.ref_fa_gfx950_make_input(n, seed, 0, 0.125 * iscale, ptr(q))
        L950.ref_fa_gfx950_make_input(n, seed, 1, 0.125 * iscale, ptr(k))
        L950.ref_fa_gfx950_make_input(n, seed, 2, 0.25, ptr(v))
        rows = [0, 1, 31, 32, 127, s // 2, s - 1]
        heads = list(range(b * h))
        res = {}
        for hh in heads:
            for r in rows:
                o = np.zeros(128, np.float32)
                L950.ref_fa_gfx950_attention_row(b, h, s, ptr(q), ptr(k), ptr(v), hh, r, ptr(o))
                res[f"{hh}:{r}"] = o.tolist()
        g[f"{b}:{h}:{s}:{seed}:{iscale}"] = {
            "sha256_q": hashlib.sha256(q.tobytes()).hexdigest(),
            "sha256_k": hashlib.sha256(k.tobytes()).hexdigest(),
            "sha256_v": hashlib.sha256(v.tobytes()).hexdigest(),
            "head0_q": q[:256].tolist(),
            "rows": res,
        }
    out["fa_gfx950"] = g
    return out


def main() -> None:
    with open(os.path.join(HERE, "matmul_runner_vectors.json"), "w") as f:
        json.dump(matmul_vectors(), f, separators=(",", ":"))
    with open(os.path.join(HERE, "mxfp4_runner_vectors.json"), "w") as f:
        json.dump(mxfp4_vectors(), f, separators=(",", ":"))
    with open(os.path.join(HERE, "fa_runner_vectors.json"), "w") as f:
        json.dump(fa_vectors(), f, separators=(",", ":"))
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
