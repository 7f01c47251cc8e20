"""Pin the MXFP4 part of the CPU oracle before trusting it.

Checks, chosen so that a plausible slip (nibble order, scale indexed
row-major instead of group-major, wrong e2m1 table entry or sign bit, scale
bias off by one, wrong LCG shift) fails one of them:

* golden values printed by the reference's own test
  (test/python/dialects/wave_matmul.py:812-833, :910-921, CHECK :1069-1074),
* fixtures recorded from the reference runner's own CPU code compiled from
  the reference sources (tests/golden/make_golden.py `mxfp4_vectors`),
* closed forms: the OCP e2m1 encoding, e8m0 = 2^(raw-127), and an
  independent numpy float64 product (exact for these dyadic operands).
"""

import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def mx():
    with open(os.path.join(HERE, "golden", "mxfp4_runner_vectors.json")) as f:
        return json.load(f)


def decode(oracle, packed, scales):
    """Independent numpy decode of [rows, K/2] codes with [K/32, rows] scales."""
    table = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float64)
    codes = np.empty((packed.shape[0], packed.shape[1] * 2), np.uint8)
    codes[:, 0::2] = packed & 0xF
    codes[:, 1::2] = packed >> 4
    vals = table[codes & 7] * np.where(codes & 8, -1.0, 1.0)
    sc = np.exp2(scales.astype(np.float64) - 127).T  # [rows, groups]
    return vals * np.repeat(sc, 32, axis=1)


def test_e2m1_and_e8m0_decode(oracle, mx):
    L = oracle.lib()
    got = [L.oracle_mxfp4_code_value(c) for c in range(16)]
    assert got == mx["code_to_float"]
    # OCP MX e2m1: sign | 2-bit exponent (bias 1) | 1-bit mantissa.
    for c in range(16):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        mag = m * 0.5 if e == 0 else (1 + m / 2) * 2.0 ** (e - 1)
        assert got[c] == (-mag if s else mag)
    assert [L.oracle_e8m0_value(r) for r in range(100, 140)] == mx["e8m0_to_float"]
    assert L.oracle_e8m0_value(127) == 1.0 and L.oracle_e8m0_value(124) == 0.125


def test_runner_inputs_and_scales_match_reference(oracle, mx):
    for key, want in mx["inputs"].items():
        seed, ones, shape, stream = key.split(":")
        rows, k = map(int, shape.split("x"))
        mode = oracle.MODE_ALL_ONES if int(ones) else oracle.MODE_RANDOM
        got = oracle.mxfp4_inputs(rows, k, int(seed), int(stream), mode)
        assert got.ravel().tolist() == want, key
    for key, want in mx["scales"].items():
        seed, ones, shape, stream = key.split(":")
        rows, k = map(int, shape.split("x"))
        mode = oracle.MODE_ALL_ONES if int(ones) else oracle.MODE_RANDOM
        got = oracle.mxfp4_scales(rows, k, int(seed), int(stream), mode)
        assert got.ravel().tolist() == want, key
    # the runner's random scales stay in its test domain 124..127
    s = oracle.mxfp4_scales(256, 1024, 7, 2)
    assert set(np.unique(s).tolist()) == {124, 125, 126, 127}


def test_python_builder_goldens(oracle):
    # CHECK: mxfp4-scales 64 64 127 122  (16x16x128)
    a, b, sa, sb = oracle.mxfp4_operands(16, 16, 128, 0, oracle.MODE_HALVES)
    assert sa.size == 64 and sb.size == 64
    assert sa.ravel()[0] == 127 and sb.ravel()[-1] == 122
    # CHECK: mxfp4-ref 256 42.5 21.25  (non-random inputs)
    c = oracle.gemm_mxfp4(a, b, sa, sb)
    assert c.size == 256 and c.ravel()[0] == 42.5 and c.ravel()[-1] == 21.25
    # CHECK: mxfp4-packed-random 1024 1024 68 34  (seed 7), seed 8 differs
    a7 = oracle.mxfp4_inputs(16, 128, 7, 0, oracle.MODE_PY_RANDOM)
    b7 = oracle.mxfp4_inputs(16, 128, 7, 1, oracle.MODE_PY_RANDOM)
    a8 = oracle.mxfp4_inputs(16, 128, 8, 0, oracle.MODE_PY_RANDOM)
    assert a7.size * 2 == 2048 and a7.ravel()[0] == 68 and b7.ravel()[-1] == 34
    assert not np.array_equal(a7, a8)
    # CHECK: mxfp4-random-ref 256 92.703125 12.6484375
    a, b, sa, sb = oracle.mxfp4_operands(16, 16, 128, 7, oracle.MODE_PY_RANDOM)
    c = oracle.gemm_mxfp4(a, b, sa, sb)
    assert c.ravel()[0] == 92.703125 and c.ravel()[-1] == 12.6484375


def test_gemm_matches_runner_expected(oracle, mx):
    for key, want in mx["gemm_expected"].items():
        shape, seed, ones, ot = key.split(":")
        m, n, k = map(int, shape.split("x"))
        mode = oracle.MODE_ALL_ONES if int(ones) else oracle.MODE_RANDOM
        a, b, sa, sb = oracle.mxfp4_operands(m, n, k, int(seed), mode)
        c = oracle.gemm_mxfp4(a, b, sa, sb)
        ot = int(ot)
        got = oracle.round_output(c, ot)
        if ot != oracle.F32:
            got = oracle.bits_to_f32(got, ot)
        assert np.array_equal(got.astype(np.float64).ravel(), np.array(want)), key


def test_gemm_vs_numpy_decode_and_elements(oracle):
    # Random runner data at K <= 1024: every partial sum is a multiple of
    # 2^-8 below 2^24 * 2^-8, so float accumulation is exact and must equal
    # the float64 product of an independent decode.
    m, n, k = 48, 40, 512
    a, b, sa, sb = oracle.mxfp4_operands(m, n, k, 11)
    c = oracle.gemm_mxfp4(a, b, sa, sb)
    ref = decode(oracle, a, sa) @ decode(oracle, b, sb).T
    assert np.array_equal(c.astype(np.float64), ref)
    rows, cols = [0, 5, 47, 13], [0, 39, 7, 20]
    assert np.array_equal(oracle.gemm_mxfp4_elements(a, b, sa, sb, rows, cols),
                          c[rows, cols])
    # Row slices agree with the whole product.
    assert np.array_equal(oracle.gemm_mxfp4_rows(a, b, sa, sb, 16, 33), c[16:33])


def test_aiter_shuffles_match_reference(oracle, mx):
    rec = mx["aiter_b"]
    got = oracle.mxfp4_aiter_b(np.array(rec["in"], np.uint8), rec["n"], rec["k"])
    assert got.tolist() == rec["out"]
    rec = mx["aiter_scales"]
    got = oracle.mxfp4_aiter_scales(np.array(rec["in"], np.uint8), rec["rows"], rec["k"])
    assert got.tolist() == rec["out"]
    # CHECK: mxfp4-aiter-shuffle 2048 8192 (B 32x128, scales 257 rows x 16 groups)
    inp = np.arange(32 * 64, dtype=np.int64) % 251
    sh = oracle.mxfp4_aiter_b(inp.astype(np.uint8), 32, 128)
    assert sh.size == 2048 and sorted(sh.tolist()) == sorted(inp.tolist())
    sin = (np.arange(257 * 16) % 251).astype(np.uint8)
    ss = oracle.mxfp4_aiter_scales(sin, 257, 512)
    assert ss.size == 8192
    # a permutation of the input plus 0x7f padding
    assert np.count_nonzero(ss != 0x7F) == np.count_nonzero(sin != 0x7F)
