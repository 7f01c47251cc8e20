"""Pin the CPU oracle (oracle/liboracle.so) before trusting it.

Each check is chosen so a plausible mistake in the restatement (wrong LCG
constant or shift, wrong rounding, transposed B, wrong accumulation type, a
dropped softmax term, a wrong causal/GQA index) fails one of them:

* golden values written in the reference's own tests
  (test/Integration/Inputs/wave_matmul_rand_int_test.cpp, test/python/...),
* fixtures recorded from the reference runners' own CPU code, compiled from
  the reference sources (tests/golden/make_golden.py, oracle/_ref),
* closed forms / independent numpy computations.
"""

import json
import math
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")


@pytest.fixture(scope="module")
def mm():
    with open(os.path.join(GOLD, "matmul_runner_vectors.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def fa():
    with open(os.path.join(GOLD, "fa_runner_vectors.json")) as f:
        return json.load(f)


# ---- generators -----------------------------------------------------------------
def test_bucket_lcg_matches_reference_runner(oracle, mm):
    L = oracle.lib()
    import ctypes
    for key, rec in mm["bucket"].items():
        seed, stream = map(int, key.split(":"))
        st = ctypes.c_uint32(L.oracle_rand_state(seed, stream))
        assert st.value == rec["state0"]
        vals = [L.oracle_bucket_value(ctypes.byref(st), 0.25) for _ in range(64)]
        assert vals == rec["values"], key
        # closed form: 17 buckets of 0.25 in [-2, 2]
        assert all(v in [0.25 * b for b in range(-8, 9)] for v in vals)


def test_rand_int_reference_goldens(oracle, mm):
    # wave_matmul_rand_int_test.cpp:30-33 (3x5 A and B, seed-independent)
    exp_a = [-2, -2, 0, 0, 1, 0, 1, 2, -1, -2, 0, -1, -2, -2, 0]
    exp_b = [2, -2, -0.0, 0, -1, 0, -1, 2, 1, -2, -0.0, -1, 2, -2, -0.0]
    for dtype in (oracle.F16, oracle.BF16):
        a = oracle.bits_to_f32(oracle.gemm_inputs(3, 5, dtype, 0, 0, oracle.MODE_RAND_INT), dtype)
        b = oracle.bits_to_f32(oracle.gemm_inputs(3, 5, dtype, 0, 1, oracle.MODE_RAND_INT), dtype)
        a91 = oracle.bits_to_f32(oracle.gemm_inputs(3, 5, dtype, 91, 0, oracle.MODE_RAND_INT), dtype)
        assert a.ravel().tolist() == exp_a
        assert b.ravel().tolist() == exp_b
        assert [math.copysign(1, x) for x in b.ravel()] == [math.copysign(1, x) for x in exp_b]
        assert np.array_equal(a, a91)  # seed-independent (:38-41)
    L = oracle.lib()
    assert [L.oracle_rand_int(i) for i in range(256)] == mm["rand_int"]


def test_hpl_reference_goldens(oracle, mm):
    # wave_matmul_rand_int_test.cpp:467-472
    f16 = [0xb5dc, 0x33a1, 0xb028, 0xb61c, 0x2a95, 0x3581, 0xb509, 0xb583,
           0xb537, 0xaaa8, 0x365c, 0xb48d, 0xa801, 0x2b96, 0x304a]
    bf16 = [0xbebb, 0x3e74, 0xbe05, 0xbec3, 0x3d53, 0x3eb0, 0xbea1, 0xbeb0,
            0xbea7, 0xbd55, 0x3ecb, 0xbe92, 0xbd00, 0x3d73, 0x3e09]
    for dtype, exp in ((oracle.F16, f16), (oracle.BF16, bf16)):
        a = oracle.gemm_inputs(3, 5, dtype, 0, 0, oracle.MODE_HPL).ravel().tolist()
        b = oracle.gemm_inputs(3, 5, dtype, 0, 1, oracle.MODE_HPL).ravel().tolist()
        assert a == exp and b == exp
    L = oracle.lib()
    assert [L.oracle_hpl(i) for i in range(256)] == mm["hpl"]


def test_gemm_inputs_match_reference_bytes(oracle, mm):
    modes = {"random": oracle.MODE_RANDOM, "all_ones": oracle.MODE_ALL_ONES,
             "rand_int": oracle.MODE_RAND_INT, "hpl": oracle.MODE_HPL}
    for key, exp in mm["inputs_seed7"].items():
        dname, mode, shape, stream = key.split(":")
        rows, k = map(int, shape.split("x"))
        dtype = oracle.F16 if dname == "f16" else oracle.BF16
        got = oracle.gemm_inputs(rows, k, dtype, 7, int(stream), modes[mode])
        assert got.ravel().tolist() == exp, key


def test_python_halves_fill_closed_form(oracle):
    # wave_matmul.py:987-991: first half of M*K elements 1.0, the rest 2.0
    a = oracle.bits_to_f32(oracle.gemm_inputs(5, 7, oracle.F16, 0, 0, oracle.MODE_HALVES), oracle.F16)
    flat = a.ravel()
    assert flat[:17].tolist() == [1.0] * 17 and flat[17:].tolist() == [2.0] * 18


# ---- rounding -------------------------------------------------------------------
def test_f16_conversion_matches_reference_and_ieee(oracle, mm):
    L = oracle.lib()
    got = [L.oracle_f32_to_f16(x) for x in mm["convert_inputs"]]
    assert got == mm["f16_bits"]
    got = [L.oracle_f32_to_bf16(x) for x in mm["convert_inputs"]]
    assert got == mm["bf16_bits"]
    got = np.array([L.oracle_f16_to_f32(h) for h in mm["half_to_float_inputs"]], np.float32)
    exp = np.array(mm["half_to_float"], np.float32)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))
    # every f16 bit pattern: widening equals numpy, narrowing round-trips
    bits = np.arange(65536, dtype=np.uint16)
    wide = np.array([L.oracle_f16_to_f32(int(h)) for h in bits], dtype=np.float32)
    ref = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(wide[finite], ref[finite])
    back = np.array([L.oracle_f32_to_f16(float(w)) for w in wide[finite]], dtype=np.uint16)
    assert np.array_equal(back, bits[finite])
    # random doubles/floats vs numpy's IEEE round-to-nearest-even
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.standard_normal(3000) * 100, rng.standard_normal(3000) * 1e-5,
                         (rng.integers(0, 2048, 500) + 0.5) * 2.0 ** -24,  # subnormal ties
                         (rng.integers(1024, 2048, 500) + 0.5)])           # normal ties
    got64 = np.array([L.oracle_f64_to_f16(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got64, xs.astype(np.float16).view(np.uint16))
    xs32 = xs.astype(np.float32)
    got32 = np.array([L.oracle_f32_to_f16(float(x)) for x in xs32], dtype=np.uint16)
    assert np.array_equal(got32, xs32.astype(np.float16).view(np.uint16))


# ---- GEMM reference -------------------------------------------------------------------
def _mode_of(m):
    return {0: 0, 2: 2, 3: 3, 1: 1}[m]


def test_gemm_reference_matches_runner_cpu_reference(oracle, mm):
    for key, exp in mm["gemm_expected"].items():
        shape, dtype, seed, mode, ot = key.split(":")
        m, n, k = map(int, shape.split("x"))
        dtype, seed, mode, ot = int(dtype), int(seed), int(mode), int(ot)
        a = oracle.gemm_inputs(m, k, dtype, seed, 0, mode)
        b = oracle.gemm_inputs(n, k, dtype, seed, 1, mode)
        c = oracle.gemm_nt(a, b, dtype, threads=2)
        if ot == oracle.F32:
            got = c.astype(np.float64).ravel()
        else:
            got = oracle.bits_to_f32(oracle.round_output(c, ot), ot).astype(np.float64).ravel()
        assert np.array_equal(got, np.array(exp)), key
        # the element-wise path agrees with the blocked path
        rows = [0, m - 1, m // 2]
        cols = [0, n - 1, n // 3]
        assert np.array_equal(oracle.gemm_elements(a, b, rows, cols, dtype), c[rows, cols])


def test_gemm_reference_small_goldens(oracle):
    # rand_int_test.cpp:78: 2x2x4 rand_int -> {0, -2, 2, -2}
    for dtype in (oracle.F16, oracle.BF16):
        a = oracle.gemm_inputs(2, 4, dtype, 0, 0, oracle.MODE_RAND_INT)
        b = oracle.gemm_inputs(2, 4, dtype, 0, 1, oracle.MODE_RAND_INT)
        assert oracle.gemm_nt(a, b, dtype).ravel().tolist() == [0, -2, 2, -2]
    # test/python/dialects/wave_matmul.py:803-814 + CHECK:1068 "bf16-ref 256 32.0"
    a = oracle.gemm_inputs(16, 32, oracle.BF16, 0, 0, oracle.MODE_HALVES)
    b = oracle.gemm_inputs(16, 32, oracle.BF16, 0, 1, oracle.MODE_HALVES)
    c = oracle.gemm_nt(a, b, oracle.BF16)
    assert c.size == 256 and c.ravel()[0] == 32.0
    # CHECK:1075 "f16-ref-rounding -132.5625 -132.5" (16x16x512, seed 91)
    a = oracle.gemm_inputs(16, 512, oracle.F16, 91, 0)
    b = oracle.gemm_inputs(16, 512, oracle.F16, 91, 1)
    c32 = oracle.gemm_nt(a, b, oracle.F16).ravel()
    c16 = oracle.bits_to_f32(oracle.round_output(c32, oracle.F16), oracle.F16)
    pair = next((x, y) for x, y in zip(c32, c16) if x != y)
    assert pair == (-132.5625, -132.5)


def test_gemm_reference_vs_numpy_exact_and_layout(oracle):
    # bucket inputs: every product is a multiple of 1/16, sums exact in f32,
    # so float64 numpy must agree bit-for-bit; a non-square shape catches a
    # transposed B (N x K storage, wave_matmul.py:329-333).
    m, n, k = 48, 80, 96
    for dtype in (oracle.F16, oracle.BF16):
        a = oracle.gemm_inputs(m, k, dtype, 3, 0)
        b = oracle.gemm_inputs(n, k, dtype, 3, 1)
        ref = oracle.bits_to_f32(a, dtype).astype(np.float64) @ oracle.bits_to_f32(b, dtype).astype(np.float64).T
        assert np.array_equal(oracle.gemm_nt(a, b, dtype), ref.astype(np.float32))
        rows = oracle.gemm_nt_rows(a, b, 10, 20, dtype)
        assert np.array_equal(rows, ref[10:20].astype(np.float32))


def test_blocked_gemm_sums_each_element_in_k_order(oracle):
    """The blocked GEMM (register micro-kernel for whole 4 x 16 blocks, the
    scalar loop at the edges) and the prepared-B^T entry the CPU baseline
    times give, on inexact normal inputs where any change of summation
    order or a fused multiply-add shows in the bits, exactly the runner's
    per-element float accumulation (oracle_gemm_element, runner.cpp
    :1586-1597); every output row and column sits in a block or an edge."""
    rng = np.random.default_rng(1)
    m, n, k = 70, 90, 300
    for dtype in (oracle.F16, oracle.BF16):
        af = rng.standard_normal((m, k)).astype(np.float32)
        bf = rng.standard_normal((n, k)).astype(np.float32)
        a = oracle.round_output(af, dtype).reshape(m, k)
        b = oracle.round_output(bf, dtype).reshape(n, k)
        ref = np.array([[oracle.gemm_elements(a, b, [r], [c], dtype)[0] for c in range(n)]
                        for r in range(m)], dtype=np.float32)
        assert np.array_equal(oracle.gemm_nt(a, b, dtype, threads=3), ref)
        bt = oracle.gemm_prepare_bt(b, dtype, threads=2)
        assert np.array_equal(bt, oracle.bits_to_f32(b, dtype).reshape(n, k).T)
        assert np.array_equal(oracle.gemm_nt_rows_bt(a, bt, 5, 66, dtype, threads=4), ref[5:66])
        # fused multiply-add or float64 accumulation would differ somewhere
        fused = (oracle.bits_to_f32(a, dtype).reshape(m, k).astype(np.float64)
                 @ oracle.bits_to_f32(b, dtype).reshape(n, k).astype(np.float64).T)
        assert not np.array_equal(fused.astype(np.float32), ref)


def test_output_coordinate_goldens(mm):
    # rand_int_test.cpp:112-141: MFMA wave64 fragment index -> (m, n)
    c = mm["output_coordinates"]["64:0"]
    assert c[0] == [0, 0] and c[3] == [3, 0] and c[4] == [0, 1]
    assert c[64] == [4, 0] and c[255] == [15, 15]
    # closed form of the gfx950 16x16x32 accumulator layout (wave_matmul.py:6534-6545)
    for idx, (m, n) in enumerate(c):
        lane, r = divmod(idx, 4)
        assert (m, n) == ((lane // 16) * 4 + r, lane % 16)


def test_tile_packed_matches_runner(oracle, mm):
    """oracle.tile_packed_coords against the runner's own getOutputCoordinate
    (runner.cpp:772-834, recorded through oracle/_ref) on four blockings,
    including the reference's tile-packed test (32x64, bm=1 bn=2
    wave_m_tiles=2, wave_matmul_rand_int_runtime.mlir:7-8) and the 16-wave
    profile's (bm=bn=4, 4x4 wave tiles)."""
    import hashlib
    for key, rec in mm["tile_packed_coordinates"].items():
        shape, bm, bn, wmt, wnt = key.split(":")
        m, n = map(int, shape.split("x"))
        mm_, nn_ = oracle.tile_packed_coords(m, n, int(bm), int(bn), int(wmt), int(wnt))
        coords = np.stack([mm_, nn_], axis=1).astype(np.int32)
        if "coords" in rec:
            assert coords.tolist() == rec["coords"], key
        else:
            assert coords[rec["sample_index"]].tolist() == rec["sample"], key
            assert hashlib.sha256(coords.tobytes()).hexdigest() == rec["sha256"], key


def test_tile_packed_is_a_permutation_of_16x16_tiles(oracle):
    """Properties that fix the layout independently of the runner: every
    (m, n) appears once; each run of 256 indices is one 16x16 tile; inside a
    tile the 4 consecutive indices of a lane are 4 consecutive rows of one
    column (the MFMA 16x16 accumulator registers)."""
    m, n = 128, 192
    mm_, nn_ = oracle.tile_packed_coords(m, n, 2, 1, 2, 3)
    assert len(set(zip(mm_.tolist(), nn_.tolist()))) == m * n
    assert mm_.min() == 0 and mm_.max() == m - 1 and nn_.max() == n - 1
    t_m, t_n = (mm_ // 16).reshape(-1, 256), (nn_ // 16).reshape(-1, 256)
    assert (t_m == t_m[:, :1]).all() and (t_n == t_n[:, :1]).all()
    q_m, q_n = mm_.reshape(-1, 4), nn_.reshape(-1, 4)
    assert (np.diff(q_m, axis=1) == 1).all() and (q_n == q_n[:, :1]).all()
    with pytest.raises(ValueError):
        oracle.tile_packed_coords(48, 64, 2, 1, 2, 1)  # 48 % 64 != 0
    c = np.arange(32 * 64, dtype=np.float32).reshape(32, 64)
    p = oracle.to_tile_packed(c, 1, 2, 2, 1)
    assert p[:8].tolist() == [0.0, 64.0, 128.0, 192.0, 1.0, 65.0, 129.0, 193.0]


# ---- flash attention reference -----------------------------------------------------------
def test_fa_f32_matches_runner(oracle, fa):
    for key, rec in fa["fa_f32"].items():
        bm, sn, hd, seed = map(int, key.split(":"))
        q, k, v = oracle.fa_f32_inputs(bm, sn, hd, seed)
        assert q.ravel().tolist() == rec["q"], key
        assert k.ravel().tolist() == rec["k"], key
        assert v.ravel().tolist() == rec["v"], key
        o = oracle.fa_f32_reference(q, k, v)
        np.testing.assert_allclose(o.ravel(), np.array(rec["o"], np.float32), rtol=0, atol=1e-6)


def test_fa_f32_independent_numpy(oracle):
    q, k, v = oracle.fa_f32_inputs(16, 64, 32, 21)
    qf, kf, vf = (oracle.f16_bits_to_f32(x).astype(np.float64) for x in (q, k, v))
    s = qf @ kf.T
    p = np.exp2(s - s.max(axis=1, keepdims=True))
    ref = (p @ vf) / p.sum(axis=1, keepdims=True)
    np.testing.assert_allclose(oracle.fa_f32_reference(q, k, v), ref, rtol=0, atol=1e-6)
    # zero scores -> every row is the column mean of V
    z = np.zeros_like(q)
    np.testing.assert_allclose(oracle.fa_f32_reference(z, k, v),
                               np.broadcast_to(vf.mean(axis=0), (16, 32)), atol=1e-6)


def test_fa_gfx950_matches_runner(oracle, fa):
    import hashlib
    for key, rec in fa["fa_gfx950"].items():
        b, h, s, seed, iscale = map(int, key.split(":"))
        n = b * h * s * 128
        q, k, v = oracle.fa_gfx950_inputs(n, seed, iscale)
        assert hashlib.sha256(q.tobytes()).hexdigest() == rec["sha256_q"]
        assert hashlib.sha256(k.tobytes()).hexdigest() == rec["sha256_k"]
        assert hashlib.sha256(v.tobytes()).hexdigest() == rec["sha256_v"]
        items = [tuple(map(int, kk.split(":"))) for kk in rec["rows"]]
        heads = [x[0] for x in items]
        rows = [x[1] for x in items]
        out = oracle.attention_rows(q, k, v, dtype=oracle.BF16, batch=b, q_heads=h, kv_heads=h,
                                    seq_q=s, seq_k=s, head_dim=128, causal=False,
                                    scale=1 / math.sqrt(128), heads=heads, rows=rows, threads=2)
        exp = np.array([rec["rows"][kk] for kk in rec["rows"]], np.float32)
        np.testing.assert_allclose(out, exp, rtol=0, atol=1e-6)


def test_fa_sample_rows_and_heads(oracle):
    # wave-fa-gfx950-runner.cpp:204-232
    assert oracle.fa_reference_rows(256) == list(range(256))
    assert oracle.fa_reference_rows(4096) == [0, 31, 32, 127, 2048, 3968, 4095]
    assert oracle.fa_reference_heads(3) == [0, 1, 2]
    assert oracle.fa_reference_heads(128) == [0, 64, 127]


def _np_attention(q, k, v, causal, scale, group):
    # q [Hq,S,D], k/v [Hkv,S,D] float64
    hq, s, d = q.shape
    out = np.zeros_like(q)
    for h in range(hq):
        kk = k[h // group]
        vv = v[h // group]
        sc = q[h] @ kk.T * scale
        if causal:
            sc = np.where(np.tril(np.ones((s, s), bool)), sc, -np.inf)
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        out[h] = (p @ vv) / p.sum(axis=1, keepdims=True)
    return out


@pytest.mark.parametrize("causal,hq,hkv", [(False, 4, 4), (True, 4, 4), (True, 8, 2), (False, 6, 3)])
def test_attention_rows_vs_numpy(oracle, causal, hq, hkv):
    rng = np.random.default_rng(hq * 10 + hkv + causal)
    s, d = 48, 32
    q = rng.standard_normal((hq, s, d)).astype(np.float32).astype(np.float16)
    k = rng.standard_normal((hkv, s, d)).astype(np.float32).astype(np.float16)
    v = rng.standard_normal((hkv, s, d)).astype(np.float32).astype(np.float16)
    heads = np.repeat(np.arange(hq), s)
    rows = np.tile(np.arange(s), hq)
    scale = 1 / math.sqrt(d)
    out = oracle.attention_rows(q.view(np.uint16), k.view(np.uint16), v.view(np.uint16),
                                dtype=oracle.F16, batch=1, q_heads=hq, kv_heads=hkv, seq_q=s,
                                seq_k=s, head_dim=d, causal=causal, scale=scale,
                                heads=heads, rows=rows, threads=2)
    ref = _np_attention(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                        causal, scale, hq // hkv)
    np.testing.assert_allclose(out, ref.reshape(-1, d), rtol=0, atol=2e-6)
    if causal:
        # closed form: causal row 0 attends only to key 0
        for h in range(hq):
            np.testing.assert_array_equal(out[h * s], v[h // (hq // hkv), 0].astype(np.float32))


def test_attention_zero_qk_is_mean_v(oracle):
    n = 1 * 2 * 256 * 128
    q, k, v = oracle.fa_gfx950_inputs(n, 3, 1, zero_qk=True)
    out = oracle.attention_rows(q, k, v, dtype=oracle.BF16, batch=1, q_heads=2, kv_heads=2,
                                seq_q=256, seq_k=256, head_dim=128, causal=False,
                                scale=1 / math.sqrt(128), heads=[0, 1], rows=[5, 200])
    vf = oracle.bf16_bits_to_f32(v).reshape(2, 256, 128).astype(np.float64)
    np.testing.assert_allclose(out, vf.mean(axis=1), atol=1e-6)


# ---- Stream-K partition ----------------------------------------------------------------------
def _check_partition(oracle, tile_count, k_iterations, workers):
    # test/python/dialects/wave_matmul_streamk.py:13-50
    total = tile_count * k_iterations
    covered = []
    partials = {}
    for worker in range(workers):
        begin, end = oracle.streamk_worker_interval(total, workers, worker)
        covered.extend(range(begin, end))
        segs = oracle.streamk_worker_segments(tile_count, k_iterations, workers, worker)
        assert sum(e - b for _, b, e, _ in segs) == end - begin
        assert sum(s is not None for *_, s in segs) <= 2
        for tile, b, e, slot in segs:
            if slot is None:
                assert (b, e) == (0, k_iterations)
                continue
            assert slot in (0, 1)
            partials.setdefault(tile, []).append((worker, b, e))
    assert covered == list(range(total))
    for it in range(total):
        owner = oracle.streamk_owner_for_iteration(total, workers, it)
        b, e = oracle.streamk_worker_interval(total, workers, owner)
        assert b <= it < e
    for tile, contrib in partials.items():
        first = oracle.streamk_owner_for_iteration(total, workers, tile * k_iterations)
        last = oracle.streamk_owner_for_iteration(total, workers, (tile + 1) * k_iterations - 1)
        assert [w for w, _, _ in contrib] == list(range(first, last + 1))
        cursor = 0
        for _, b, e in contrib:
            assert b == cursor
            cursor = e
        assert cursor == k_iterations


def test_streamk_partition_exhaustive(oracle):
    for tile_count in range(1, 10):
        for k_iterations in range(1, 12):
            total = tile_count * k_iterations
            for workers in range(1, total + 1):
                _check_partition(oracle, tile_count, k_iterations, workers)


def test_streamk_rejects_bad_arguments(oracle):
    with pytest.raises(ValueError):
        oracle.streamk_worker_interval(10, 11, 0)
    with pytest.raises(ValueError):
        oracle.streamk_worker_interval(10, 0, 0)
    with pytest.raises(ValueError):
        oracle.streamk_owner_for_iteration(10, 3, 10)
