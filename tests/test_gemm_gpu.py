"""GPU parity of the tiled GEMM (wave_gemm_launch) against the CPU oracle.

With the reference's bucket generator (values k/4, |k| <= 8;
wave_matmul.py:828-836) every product is a multiple of 1/16 and every
partial sum is exact in fp32 for K < 2^18, so the GPU result must be
bit-identical to the oracle whatever the summation order -- the reference's
own bar (test/Integration/wave_mfma_tiled.mlir:9, max_abs_diff=0.0).  f16 /
bf16 outputs are one RNE rounding of that exact sum and are compared
bitwise too.  For the uniform / normal inputs of the perf configs the
tolerance is BASELINE.json's 2e-3*sqrt(K) on sampled rows.
"""

import numpy as np
import pytest
import torch

from conftest import to_bits, to_dev

pytestmark = pytest.mark.gpu

TDT = {1: torch.float16, 2: torch.bfloat16}
ODT = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}


def run_gemm(wave, oracle, dev, M, N, K, in_dt, out_dt, layout="row", seed=7,
             mode=None):
    mode = oracle.MODE_RANDOM if mode is None else mode
    a = oracle.gemm_inputs(M, K, in_dt, seed, 0, mode)
    b = oracle.gemm_inputs(N, K, in_dt, seed, 1, mode)
    c = wave.gemm(to_dev(a, TDT[in_dt], dev), to_dev(b, TDT[in_dt], dev),
                  out_dtype=ODT[out_dt], layout=layout)
    torch.cuda.synchronize()
    ref = oracle.gemm_nt(a, b, in_dt)
    if layout == "col":
        c = c.t()
    return a, b, c, ref


def assert_exact(oracle, c, ref, out_dt):
    if out_dt == 0:
        got = c.cpu().numpy()
        assert np.array_equal(got, ref), f"max |diff| {np.abs(got - ref).max()}"
    else:
        exp = oracle.round_output(ref, out_dt)
        got = to_bits(c.contiguous())
        bad = np.argwhere(got != exp)
        assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[:3].tolist()}"


def test_config1_compare_cpu_bit_exact(wave, oracle, dev):
    """32x32x64 f16, seed 7, f32 row-major out
    (README.md:116-117; wave_mfma_dma_lds_f16_runtime.mlir:3)."""
    _, _, c, ref = run_gemm(wave, oracle, dev, 32, 32, 64, 1, 0, seed=7)
    assert_exact(oracle, c, ref, 0)


def test_integration_64x96x64_seed37(wave, oracle, dev):
    # test/Integration/wave_mfma_tiled.mlir:3-9: elements=6144 max_abs_diff=0.0
    _, _, c, ref = run_gemm(wave, oracle, dev, 64, 96, 64, 1, 0, seed=37)
    assert c.numel() == 6144
    assert_exact(oracle, c, ref, 0)


@pytest.mark.parametrize("in_dt", [1, 2])
@pytest.mark.parametrize("out_dt", [0, 1, 2])
@pytest.mark.parametrize("layout", ["row", "col"])
@pytest.mark.parametrize("shape", [(256, 256, 64), (512, 768, 192), (32, 32, 64),
                                   (300, 200, 100), (1, 1, 1), (257, 513, 4100),
                                   (130, 70, 63), (64, 96, 64),
                                   # whole tiles, K off the 64-deep stage (the
                                   # hybrid path's 32-element tail after 0, 1, 2
                                   # stages), and 2 and 5 whole 64-deep stages
                                   (256, 512, 32), (512, 256, 96), (256, 256, 160),
                                   (256, 256, 128), (512, 512, 320),
                                   # ragged tiles on the DMA ring: K below one
                                   # stage (tail only), K % 32 = 8 and 4, C
                                   # lines not 16-byte aligned (N, M = 300, 270)
                                   (300, 260, 20), (300, 300, 200), (270, 300, 72),
                                   (1000, 600, 36)])
def test_bucket_inputs_bit_exact(wave, oracle, dev, in_dt, out_dt, layout, shape):
    M, N, K = shape
    _, _, c, ref = run_gemm(wave, oracle, dev, M, N, K, in_dt, out_dt, layout, seed=9)
    assert_exact(oracle, c, ref, out_dt)


def test_rand_int_2x2x4_golden(wave, oracle, dev):
    # test/Integration/Inputs/wave_matmul_rand_int_test.cpp:78
    for dt in (1, 2):
        _, _, c, _ = run_gemm(wave, oracle, dev, 2, 2, 4, dt, 0, mode=oracle.MODE_RAND_INT)
        assert c.cpu().numpy().ravel().tolist() == [0, -2, 2, -2]


def test_halves_fill_gives_k_2k_4k(wave, oracle, dev):
    # test/Integration/wave_wmma_tiled.mlir:19-48: first half 1.0, second 2.0
    M = N = 64
    K = 128
    _, _, c, ref = run_gemm(wave, oracle, dev, M, N, K, 1, 0, mode=oracle.MODE_HALVES)
    got = c.cpu().numpy()
    assert set(np.unique(got).tolist()) == {K, 2 * K, 4 * K}
    assert np.array_equal(got, ref)


def test_f16_output_rounding_golden(wave, oracle, dev):
    # test/python/dialects/wave_matmul.py:922-937 (CHECK :1075): M=N=16,
    # K=512, seed 91: fp32 sum -132.5625 rounds to f16 -132.5.
    a, b, c32, ref = run_gemm(wave, oracle, dev, 16, 16, 512, 1, 0, seed=91)
    c16 = wave.gemm(to_dev(a, torch.float16, dev), to_dev(b, torch.float16, dev),
                    out_dtype=torch.float16)
    got32 = c32.cpu().numpy().ravel()
    got16 = c16.float().cpu().numpy().ravel()
    i = int(np.argwhere(got32 == -132.5625)[0][0])
    assert got16[i] == -132.5
    assert np.array_equal(got32, ref.ravel())


def _sample_rows(M, count, rng):
    rows = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, count)]))
    return rows


@pytest.mark.parametrize("dt", [1, 2])
def test_config2_8192_bucket_sampled_rows_exact(wave, oracle, dev, dt):
    """8192^3 with the bucket generator: every sampled row is bit-exact
    (sums stay exact in fp32 at K=8192), f16/bf16 output."""
    M = N = K = 8192
    a = oracle.gemm_inputs(M, K, dt, 7, 0)
    b = oracle.gemm_inputs(N, K, dt, 7, 1)
    c = wave.gemm(to_dev(a, TDT[dt], dev), to_dev(b, TDT[dt], dev), out_dtype=TDT[dt])
    torch.cuda.synchronize()
    got = to_bits(c)
    rows = _sample_rows(M, 24, np.random.default_rng(0))
    for r0 in rows:
        ref = oracle.gemm_nt_rows(a, b, int(r0), int(r0) + 1, dt)
        assert np.array_equal(got[r0], oracle.round_output(ref, dt)[0]), int(r0)


def _uniform_f16(shape, seed, dev):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.rand(shape, generator=g) * 2 - 1).to(torch.float16)


def test_config2_8192_uniform_tolerance(wave, oracle, dev):
    """f16 uniform [-1, 1), max |err| <= 2e-3*sqrt(K)."""
    M = N = K = 8192
    a = _uniform_f16((M, K), 7, dev)
    b = _uniform_f16((N, K), 8, dev)
    c = wave.gemm(a.to(dev), b.to(dev), out_dtype=torch.float16)
    torch.cuda.synchronize()
    abits = a.view(torch.int16).numpy().view(np.uint16)
    bbits = b.view(torch.int16).numpy().view(np.uint16)
    got = c.float().cpu().numpy()
    tol = 2e-3 * np.sqrt(K)
    worst = 0.0
    for r0 in _sample_rows(M, 16, np.random.default_rng(1)):
        ref = oracle.gemm_nt_rows(abits, bbits, int(r0), int(r0) + 1, 1)[0]
        worst = max(worst, float(np.abs(got[r0] - ref).max()))
    assert worst <= tol, worst


@pytest.mark.parametrize("shape", [(128, 8192, 8192), (4000, 4096, 4100), (8192, 1024, 28672)])
def test_config3_ragged_bf16_tolerance(wave, oracle, dev, shape):
    """bf16 N(0,1)/sqrt(K), bf16 out, 2e-3*sqrt(K)."""
    M, N, K = shape
    g = torch.Generator(device="cpu").manual_seed(3)
    a = (torch.randn((M, K), generator=g) / np.sqrt(K)).to(torch.bfloat16)
    b = (torch.randn((N, K), generator=g) / np.sqrt(K)).to(torch.bfloat16)
    c = wave.gemm(a.to(dev), b.to(dev), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    abits = a.view(torch.int16).numpy().view(np.uint16)
    bbits = b.view(torch.int16).numpy().view(np.uint16)
    got = c.float().cpu().numpy()
    tol = 2e-3 * np.sqrt(K)
    for r0 in _sample_rows(M, 6, np.random.default_rng(2)):
        ref = oracle.gemm_nt_rows(abits, bbits, int(r0), int(r0) + 1, 2)[0]
        err = float(np.abs(got[r0] - ref).max())
        assert err <= tol, (int(r0), err)


def test_repeat_launch_deterministic(wave, oracle, dev):
    """Same inputs, same bits, launch after launch (no order dependence)."""
    g = torch.Generator(device="cpu").manual_seed(5)
    a = torch.randn((1024, 2048), generator=g).to(torch.float16).to(dev)
    b = torch.randn((768, 2048), generator=g).to(torch.float16).to(dev)
    first = wave.gemm(a, b, out_dtype=torch.float32)
    for _ in range(5):
        again = wave.gemm(a, b, out_dtype=torch.float32)
        assert torch.equal(first, again)


@pytest.mark.parametrize("dt", [1, 2])
@pytest.mark.parametrize("out_dt", [0, 1, 2])
@pytest.mark.parametrize("layout", ["row", "col"])
@pytest.mark.parametrize("shape", [(128, 1024, 512), (1, 2048, 64), (100, 1056, 256),
                                   (77, 3000, 128), (128, 8192, 1024)])
def test_short_m_bucket_bit_exact(wave, oracle, dev, dt, out_dt, layout, shape):
    """M <= 128 with K % 64 == 0 runs the short-M kernel (one CTA per 32
    columns of N); bucket inputs make it bit-exact like the tiled path."""
    M, N, K = shape
    _, _, c, ref = run_gemm(wave, oracle, dev, M, N, K, dt, out_dt, layout, seed=13)
    assert_exact(oracle, c, ref, out_dt)


# ---- tile-packed C (wave_gemm_tile_packed_launch) ------------------------------
@pytest.mark.parametrize("case", [
    # (M, N, K, in_dt, out_dt, blocking, mode): the reference's own
    # tile-packed test (wave_matmul_rand_int_runtime.mlir:7-8), ragged shapes
    # on the bounds-checked path, whole 256x256 tiles on the DMA path, the
    # 16-wave profile's blocking and a 16-bit output.
    (32, 64, 32, 2, 0, (1, 2, 2, 1), "rand_int"),
    (48, 80, 40, 1, 0, (1, 1, 1, 1), "bucket"),
    (64, 96, 64, 1, 0, (2, 1, 2, 3), "bucket"),
    (512, 768, 192, 1, 1, (2, 2, 4, 4), "bucket"),
    (1024, 512, 256, 2, 0, (4, 4, 4, 4), "bucket"),
    (256, 256, 4100, 2, 2, (2, 2, 2, 2), "bucket"),
])
def test_tile_packed_bit_exact(wave, oracle, dev, case):
    M, N, K, in_dt, out_dt, blocking, mode = case
    m = oracle.MODE_RAND_INT if mode == "rand_int" else oracle.MODE_RANDOM
    a = oracle.gemm_inputs(M, K, in_dt, 4, 0, m)
    b = oracle.gemm_inputs(N, K, in_dt, 4, 1, m)
    bm, bn, wmt, wnt = blocking
    c = wave.gemm_tile_packed(to_dev(a, TDT[in_dt], dev), to_dev(b, TDT[in_dt], dev), bm=bm,
                              bn=bn, wave_m_tiles=wmt, wave_n_tiles=wnt, out_dtype=ODT[out_dt])
    torch.cuda.synchronize()
    ref = oracle.to_tile_packed(oracle.gemm_nt(a, b, in_dt), bm, bn, wmt, wnt)
    assert_exact(oracle, c, ref, out_dt)


def test_tile_packed_default_blocking_through_wave_gemm_launch(wave, oracle, dev):
    """c_layout = WAVE_TILE_PACKED in wave_gemm_launch: the reference's
    default blocking (bm = bn = 1, one 16x16 tile per wave)."""
    M, N, K = 80, 48, 96
    a = oracle.gemm_inputs(M, K, 1, 6, 0)
    b = oracle.gemm_inputs(N, K, 1, 6, 1)
    A, B = to_dev(a, torch.float16, dev), to_dev(b, torch.float16, dev)
    c = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    rt = wave.runtime
    rt.check(rt.lib().wave_gemm_launch(A.data_ptr(), B.data_ptr(), c.data_ptr(), M, N, K, rt.F16,
                                       rt.F32, rt.TILE_PACKED,
                                       torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), oracle.to_tile_packed(oracle.gemm_nt(a, b, 1), 1, 1,
                                                                 1, 1))


@pytest.mark.parametrize("M,N,blocking", [(48, 64, (1, 2, 2, 1)),  # 48 % 32
                                          (32, 48, (1, 2, 2, 1)),  # 48 % 64
                                          (64, 64, (0, 1, 1, 1)), (64, 64, (8, 8, 1, 1))])
def test_tile_packed_rejects_bad_blocking(wave, dev, M, N, blocking):
    a = torch.zeros((M, 32), dtype=torch.float16, device=dev)
    b = torch.zeros((N, 32), dtype=torch.float16, device=dev)
    bm, bn, wmt, wnt = blocking
    with pytest.raises(ValueError):
        wave.gemm_tile_packed(a, b, bm=bm, bn=bn, wave_m_tiles=wmt, wave_n_tiles=wnt)


def test_tile_packed_not_for_streamk(wave, dev):
    a = torch.zeros((256, 64), dtype=torch.float16, device=dev)
    rt = wave.runtime
    ws = wave.StreamKWorkspace(256, 256, 2, dev)
    c = torch.empty(256 * 256, dtype=torch.float16, device=dev)
    st = rt.lib().wave_gemm_streamk_launch(a.data_ptr(), a.data_ptr(), c.data_ptr(), 256, 256,
                                           64, rt.F16, rt.F16, rt.TILE_PACKED,
                                           ws.scratch.data_ptr(), ws.counters.data_ptr(), 2,
                                           None)
    assert st == rt.ERR_UNSUPPORTED
