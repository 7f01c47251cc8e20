"""GPU parity of the MXFP4 scaled GEMM (wave_gemm_mxfp4_launch) against the
CPU oracle.

With the reference runner's inputs (random e2m1 codes, |x| <= 6, and e8m0
scales 124..127, runner.cpp:1135-1150, :1208-1220) every product is a
multiple of 2^-8 and every partial sum stays below 2^16 for K <= 1024, so
fp32 accumulation is exact in any order: the GPU result must equal the
oracle bit for bit, and f16 / bf16 outputs are one RNE rounding of it.  The
Python builder's inputs (codes 1.0 / 2.0, scales 0x7f - group) are exact in
the same way.  Larger K is held to the runner's own limit,
1e-2 + 1e-3 * |expected| (runner.cpp:925-960 validateRowMajorOutput).
The AITER input layout (wave_gemm_mxfp4_aiter_launch) gets its operands
from the oracle's AITER shuffles, which are pinned to the reference runner's
makeAITERBBytes / makeAITERScaleBytes; it must give the canonical result
bit for bit.
"""

import numpy as np
import pytest
import torch

from conftest import to_bits

pytestmark = pytest.mark.gpu

ODT = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}


def up(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.uint8)).to(dev)


def run(wave, dev, a, b, sa, sb, out_dt=0, layout="row"):
    c = wave.gemm_mxfp4(up(a, dev), up(b, dev), up(sa, dev), up(sb, dev),
                        out_dtype=ODT[out_dt], layout=layout)
    torch.cuda.synchronize()
    return c.t() if layout == "col" else c


def assert_exact(oracle, c, ref, out_dt):
    if out_dt == 0:
        got = c.cpu().numpy()
        assert np.array_equal(got, ref), f"max |diff| {np.abs(got - ref).max()}"
    else:
        exp = oracle.round_output(ref, out_dt)
        got = to_bits(c.contiguous())
        bad = np.argwhere(got != exp)
        assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[:3].tolist()}"


@pytest.mark.parametrize("out_dt", [0, 1, 2])
@pytest.mark.parametrize("layout", ["row", "col"])
@pytest.mark.parametrize("shape", [(256, 256, 128), (512, 256, 256), (256, 768, 1024),
                                   (768, 512, 384)])
def test_runner_inputs_bit_exact(wave, oracle, dev, out_dt, layout, shape):
    M, N, K = shape
    print(f"mxfp4 runner inputs {shape} out={out_dt} {layout}", flush=True)
    a, b, sa, sb = oracle.mxfp4_operands(M, N, K, 7)
    c = run(wave, dev, a, b, sa, sb, out_dt, layout)
    assert_exact(oracle, c, oracle.gemm_mxfp4(a, b, sa, sb), out_dt)


@pytest.mark.parametrize("mode", ["halves", "py_random"])
def test_python_builder_inputs_bit_exact(wave, oracle, dev, mode):
    # The inputs of compute_wmma_f16_matmul_reference_buffer(input_type="mxfp4")
    # (wave_matmul.py:966-994, :937-950) at a whole-tile shape.
    m = oracle.MODE_HALVES if mode == "halves" else oracle.MODE_PY_RANDOM
    # K = 256: the scales fall by 2 per group, and over 8 groups every
    # partial sum still fits fp32 exactly.
    a, b, sa, sb = oracle.mxfp4_operands(256, 512, 256, 7, m)
    c = run(wave, dev, a, b, sa, sb)
    assert_exact(oracle, c, oracle.gemm_mxfp4(a, b, sa, sb), 0)


def test_all_ones_closed_form(wave, oracle, dev):
    # --all-ones: codes 0x22, scales 0x7f -> every element equals K.
    a, b, sa, sb = oracle.mxfp4_operands(512, 256, 2048, 0, oracle.MODE_ALL_ONES)
    c = run(wave, dev, a, b, sa, sb)
    assert torch.all(c == 2048).item()


def test_scales_follow_rows_and_columns(wave, oracle, dev):
    # Scales constant over groups but spread over rows / columns across a
    # wide exponent range: C[m, n] = 2^(sa_m + sb_n - 254) * (code sum),
    # exact in fp32, so a row / column mix-up in the scale path shows.
    M, N, K = 256, 512, 256
    rng = np.random.default_rng(3)
    a = oracle.mxfp4_inputs(M, K, 5, 0)
    b = oracle.mxfp4_inputs(N, K, 5, 1)
    sa = np.repeat(rng.integers(80, 171, M, dtype=np.uint8)[None], K // 32, 0)
    sb = np.repeat(rng.integers(80, 171, N, dtype=np.uint8)[None], K // 32, 0)
    c = run(wave, dev, a, b, sa, sb)
    assert_exact(oracle, c, oracle.gemm_mxfp4(a, b, sa, sb), 0)


def test_group_scales_vary_within_row(wave, oracle, dev):
    # Each 32-value group with its own scale, A from 120..123 and B from
    # 128..131 (products are multiples of 2^-8 below 36, as for the
    # runner's 124..127): exact at K = 512, and a swap of A and B scales or
    # a group off by one changes the result.
    M, N, K = 256, 256, 512
    rng = np.random.default_rng(4)
    a = oracle.mxfp4_inputs(M, K, 6, 0)
    b = oracle.mxfp4_inputs(N, K, 6, 1)
    sa = rng.integers(120, 124, (K // 32, M), dtype=np.uint8)
    sb = rng.integers(128, 132, (K // 32, N), dtype=np.uint8)
    c = run(wave, dev, a, b, sa, sb)
    assert_exact(oracle, c, oracle.gemm_mxfp4(a, b, sa, sb), 0)


@pytest.mark.parametrize("shape", [(4096, 4096, 8192), (256, 768, 16384)])
def test_large_k_runner_limit(wave, oracle, dev, shape):
    M, N, K = shape
    print(f"mxfp4 large K {shape}", flush=True)
    a, b, sa, sb = oracle.mxfp4_operands(M, N, K, 7)
    c = run(wave, dev, a, b, sa, sb).cpu().numpy()
    rng = np.random.default_rng(8)
    rows = np.concatenate([[0, M - 1], rng.integers(0, M, 254)])
    cols = np.concatenate([[0, N - 1], rng.integers(0, N, 254)])
    exp = oracle.gemm_mxfp4_elements(a, b, sa, sb, rows, cols)
    got = c[rows, cols]
    lim = 1e-2 + 1e-3 * np.abs(exp)
    assert np.all(np.abs(got - exp) <= lim), f"max |diff| {np.abs(got - exp).max()}"


def test_back_to_back_calls_and_out_argument(wave, oracle, dev):
    a, b, sa, sb = oracle.mxfp4_operands(256, 256, 256, 1)
    out = torch.full((256, 256), float("nan"), device=dev)
    A, B, SA, SB = up(a, dev), up(b, dev), up(sa, dev), up(sb, dev)
    for _ in range(3):
        wave.gemm_mxfp4(A, B, SA, SB, out=out)
    torch.cuda.synchronize()
    assert_exact(oracle, out, oracle.gemm_mxfp4(a, b, sa, sb), 0)


def test_rejects_unsupported_shapes(wave, dev):
    z = lambda *s: torch.zeros(s, dtype=torch.uint8, device=dev)  # noqa: E731
    with pytest.raises(ValueError):  # K % 128
        wave.gemm_mxfp4(z(256, 32), z(256, 32), z(2, 256), z(2, 256))
    with pytest.raises(NotImplementedError):  # M % 256
        wave.gemm_mxfp4(z(128, 64), z(256, 64), z(4, 128), z(4, 256))
    with pytest.raises(ValueError):  # scale shape
        wave.gemm_mxfp4(z(256, 64), z(256, 64), z(4, 256), z(2, 256))


def aiter_operands(oracle, b, sa, sb, N, K):
    M = sa.shape[1]
    return (oracle.mxfp4_aiter_b(b, N, K).reshape(N, K // 2),
            oracle.mxfp4_aiter_scales(sa, M, K), oracle.mxfp4_aiter_scales(sb, N, K))


@pytest.mark.parametrize("out_dt", [0, 1])
@pytest.mark.parametrize("layout", ["row", "col"])
@pytest.mark.parametrize("shape", [(256, 256, 256), (256, 512, 384), (512, 256, 1024)])
def test_aiter_layout_bit_exact(wave, oracle, dev, out_dt, layout, shape):
    """K = 384 leaves the second 8-group scale block half used (padding)."""
    M, N, K = shape
    print(f"mxfp4 aiter {shape} out={out_dt} {layout}", flush=True)
    a, b, sa, sb = oracle.mxfp4_operands(M, N, K, 9)
    ba, saa, sba = aiter_operands(oracle, b, sa, sb, N, K)
    c = wave.gemm_mxfp4(up(a, dev), up(ba, dev), up(saa, dev), up(sba, dev),
                        out_dtype=ODT[out_dt], layout=layout, input_layout="aiter")
    torch.cuda.synchronize()
    c = c.t() if layout == "col" else c
    assert_exact(oracle, c, oracle.gemm_mxfp4(a, b, sa, sb), out_dt)


def test_aiter_matches_canonical_large_k(wave, oracle, dev):
    M, N, K = 1024, 2048, 8192
    a, b, sa, sb = oracle.mxfp4_operands(M, N, K, 4)
    ba, saa, sba = aiter_operands(oracle, b, sa, sb, N, K)
    ref = wave.gemm_mxfp4(up(a, dev), up(b, dev), up(sa, dev), up(sb, dev),
                          out_dtype=torch.float16)
    got = wave.gemm_mxfp4(up(a, dev), up(ba, dev), up(saa, dev), up(sba, dev),
                          out_dtype=torch.float16, input_layout="aiter")
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
