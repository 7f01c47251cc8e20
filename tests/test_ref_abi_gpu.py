"""The reference's device-side kernel ABI: code objects built from
7_amd/csrc/ref_abi.hip, loaded with hipModuleLoad and launched with
hipModuleLaunchKernel exactly as the reference's launchers do (grid, block,
dynamic LDS and bare-pointer arguments), checked against the oracle.

* wmma_f16_matmul_tiled(A, B, C, trip): grid (M_blocks, N_blocks) and block
  64 * BM * BN of the reference's tiling (wave-matmul-calibrate-runner.cpp
  :1114-1131, :1745-1762), no dynamic LDS -- the reference's kernels declare
  their LDS statically and both of its launchers pass 0 (the runner's
  --dynamic-lds default and tools/wave-matmul-calibrate/
  wave-matmul-calibrate.py:901-902; the mlir-runner gpu.launch_func,
  python/mlir/dialects/wave_matmul.py:6976-6982).  Blocks of 64, 128, 256,
  512 and 1024 threads, as the reference's tests and profiles use them.
  Bucket and rand_int inputs make every result bit-exact
  (wave_mfma_tiled.mlir:9).
* wmma_f16_matmul_tiled(A, B, C, A_scale, B_scale, trip), mxfp4 input type
  (runner.cpp:1792-1794): block 512 or 256, no dynamic LDS; the runner's
  random codes and scales are exact at K = 512.
* gfx950_f16_streamk_gemm(A, B, C, scratch, counters, workers): grid
  (workers), block 256, no dynamic LDS; column-major C; counters back at
  zero afterwards (runner.cpp:1718-1742).
* flash_attention_bf16_gfx950(Q, K, V, O): grid (S/256, B*H), block 512,
  dynamic LDS 136192 set with hipFuncSetAttribute (wave-fa-gfx950-runner.cpp
  :396-428); 1.35e-3 beyond the bf16 rounding of O.
* flash_attention_f32(Q, K, V, O): grid 1, the runner's --threads
  (wave-fa-calibrate-runner.cpp:346-361); tolerance 3e-3 (:263).
"""

import importlib
import math

import numpy as np
import pytest
import torch

from conftest import to_bits, to_dev

pytestmark = pytest.mark.gpu

FA_LDS = 136192


@pytest.fixture(scope="module")
def co():
    return importlib.import_module("7_amd.code_object")


def bucket_gemm(oracle, dev, M, N, K, dt, seed, mode=None):
    mode = oracle.MODE_RANDOM if mode is None else mode
    a = oracle.gemm_inputs(M, K, dt, seed, 0, mode)
    b = oracle.gemm_inputs(N, K, dt, seed, 1, mode)
    tdt = {1: torch.float16, 2: torch.bfloat16}[dt]
    return a, b, to_dev(a, tdt, dev), to_dev(b, tdt, dev)


def launch_tiled(co, name, grid, A, B, C, block=256, trip=0):
    """The runner's launch: hipModuleLaunchKernel(grid, block, dynamic LDS 0)."""
    with co.CodeObject(name) as mod:
        mod.kernel("wmma_f16_matmul_tiled").launch(grid, (block,), [A, B, C, trip],
                                                   dynamic_lds=0)
        torch.cuda.synchronize()


def runner_grid(M, N, bm, bn, wmt, wnt):
    """(M_blocks, N_blocks) of the reference tiling (runner.cpp:1114-1131)."""
    assert M % (16 * bm * wmt) == 0 and N % (16 * bn * wnt) == 0
    return (M // (16 * bm * wmt), N // (16 * bn * wnt))


def test_tiled_config1_bit_exact(co, oracle, dev):
    """32x32x64 f16 -> f32 row-major, seed 7, BM=BN=2
    wave_k_tiles=2: grid (1,1), block 256, dynamic LDS 0."""
    a, b, A, B = bucket_gemm(oracle, dev, 32, 32, 64, 1, 7)
    C = torch.zeros((32, 32), dtype=torch.float32, device=dev)
    launch_tiled(co, "gemm_f16_f32_rm_32x32x64", (1, 1), A, B, C)
    assert np.array_equal(C.cpu().numpy(), oracle.gemm_nt(a, b, 1))


def test_tiled_64x96x64_block128(co, oracle, dev):
    """wave_mfma_tiled.mlir:3-9 (seed 37, max_abs_diff 0.0): bm=2 bn=1,
    wave tiles 2 x 3 -> grid (1, 2), block 128."""
    a, b, A, B = bucket_gemm(oracle, dev, 64, 96, 64, 1, 37)
    C = torch.full((64, 96), float("nan"), dtype=torch.float32, device=dev)
    launch_tiled(co, "gemm_f16_f32_rm_64x96x64_b128", runner_grid(64, 96, 2, 1, 2, 3), A, B, C,
                 block=128)
    assert np.array_equal(C.cpu().numpy(), oracle.gemm_nt(a, b, 1))


def test_tiled_64x32x64_block64(co, oracle, dev):
    """wave_mfma_dma_lds_remap_runtime.mlir:3 (seed 23, --compare-cpu):
    bm=bn=1 -> grid (4, 2), block 64 (one wave)."""
    a, b, A, B = bucket_gemm(oracle, dev, 64, 32, 64, 1, 23)
    C = torch.full((64, 32), float("nan"), dtype=torch.float32, device=dev)
    launch_tiled(co, "gemm_f16_f32_rm_64x32x64_b64", runner_grid(64, 32, 1, 1, 1, 1), A, B, C,
                 block=64)
    assert np.array_equal(C.cpu().numpy(), oracle.gemm_nt(a, b, 1))


@pytest.mark.parametrize("layout", ["rm", "cm"])
def test_tiled_rand_int_32x64x32_block128(co, oracle, dev, layout):
    """wave_matmul_rand_int_runtime.mlir:3-6 (ROW / COLUMN): 32x64x32 f16,
    rand_int inputs, f32 C, bm=1 bn=2 wave_m_tiles=2 -> grid (1, 2), block
    128; strict check."""
    a, b, A, B = bucket_gemm(oracle, dev, 32, 64, 32, 1, 0, oracle.MODE_RAND_INT)
    shape = (32, 64) if layout == "rm" else (64, 32)
    C = torch.full(shape, float("nan"), dtype=torch.float32, device=dev)
    launch_tiled(co, f"gemm_f16_f32_{layout}_32x64x32_b128", runner_grid(32, 64, 1, 2, 2, 1),
                 A, B, C, block=128)
    got = C.cpu().numpy() if layout == "rm" else C.cpu().numpy().T
    assert np.array_equal(got, oracle.gemm_nt(a, b, 1))


def test_tiled_tile_packed_32x64x32_block128(co, oracle, dev):
    """wave_matmul_rand_int_runtime.mlir:7-8 (TILE): bf16 rand_int inputs,
    f32 C in the tile-packed layout of bm=1 bn=2 wave_m_tiles=2, grid (1, 2),
    block 128; decoded as the runner's getOutputCoordinate does."""
    a, b, A, B = bucket_gemm(oracle, dev, 32, 64, 32, 2, 0, oracle.MODE_RAND_INT)
    C = torch.full((32 * 64,), float("nan"), dtype=torch.float32, device=dev)
    launch_tiled(co, "gemm_bf16_f32_pk_32x64x32_b128", runner_grid(32, 64, 1, 2, 2, 1), A, B, C,
                 block=128)
    exp = oracle.to_tile_packed(oracle.gemm_nt(a, b, 2), 1, 2, 2, 1)
    assert np.array_equal(C.cpu().numpy(), exp)


@pytest.mark.parametrize("name,K,block,blocking", [
    # test/Integration/wave_hipblaslt_f16_profiles_runtime.mlir:3-14: the
    # 4-, 8- and 16-wave gfx950 profiles at 1024x512, rand_int, f16
    # column-major C (examples/wave/wmma_matmul_tiled.py:115-146).
    ("gemm_f16_f16_cm_1024x512x256", 256, 256, (2, 2, 8, 8)),
    ("gemm_f16_f16_cm_1024x512x512_b512", 512, 512, (2, 4, 8, 4)),
    ("gemm_f16_f16_cm_1024x512x256_b1024", 256, 1024, (4, 4, 4, 4)),
])
@pytest.mark.parametrize("mode", ["rand_int", "bucket"])
def test_tiled_profiles_1024x512(co, oracle, dev, name, K, block, blocking, mode):
    M, N = 1024, 512
    m = oracle.MODE_RAND_INT if mode == "rand_int" else oracle.MODE_RANDOM
    a, b, A, B = bucket_gemm(oracle, dev, M, N, K, 1, 17, m)
    C = torch.full((N, M), float("nan"), dtype=torch.float16, device=dev)
    launch_tiled(co, name, runner_grid(M, N, *blocking), A, B, C, block=block)
    exp = oracle.round_output(oracle.gemm_nt(a, b, 1), 1)
    assert np.array_equal(to_bits(C).T, exp)


def test_tiled_tile_packed_16wave_block1024(co, oracle, dev):
    """The 16-wave profile's blocking (bm = bn = 4, 4 x 4 wave tiles) with
    tile-packed f32 C, bf16 bucket inputs, block 1024."""
    M, N, K = 1024, 512, 256
    a, b, A, B = bucket_gemm(oracle, dev, M, N, K, 2, 5)
    C = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    launch_tiled(co, "gemm_bf16_f32_pk_1024x512x256_b1024", runner_grid(M, N, 4, 4, 4, 4),
                 A, B, C, block=1024)
    exp = oracle.to_tile_packed(oracle.gemm_nt(a, b, 2), 4, 4, 4, 4)
    assert np.array_equal(C.cpu().numpy(), exp)


@pytest.mark.parametrize("grid", [(2, 2), (1, 1), (3, 1), (16, 16)])
def test_tiled_512_any_grid(co, oracle, dev, grid):
    """512^3 f16 -> f16: the runner's 256x256 grid (2,2), fewer CTAs than
    tiles (grid-stride loop) and more (the extra CTAs exit)."""
    a, b, A, B = bucket_gemm(oracle, dev, 512, 512, 512, 1, 11)
    C = torch.zeros((512, 512), dtype=torch.float16, device=dev)
    launch_tiled(co, "gemm_f16_f16_rm_512x512x512", grid, A, B, C)
    exp = oracle.round_output(oracle.gemm_nt(a, b, 1), 1)
    assert np.array_equal(to_bits(C), exp)


@pytest.mark.parametrize("name,block,grid", [("gemm_bf16_bf16_cm_300x200x100", 256, (2, 1)),
                                             ("gemm_bf16_bf16_rm_300x200x100_b1024", 1024,
                                              (1, 1))])
def test_tiled_ragged_bf16(co, oracle, dev, name, block, grid):
    """300x200x100 bf16 -> bf16 (masked load path), column-major C with 4
    waves and row-major C with 16."""
    a, b, A, B = bucket_gemm(oracle, dev, 300, 200, 100, 2, 5)
    cm = "_cm_" in name
    C = torch.zeros((200, 300) if cm else (300, 200), dtype=torch.bfloat16, device=dev)
    launch_tiled(co, name, grid, A, B, C, block=block)
    exp = oracle.round_output(oracle.gemm_nt(a, b, 2), 2)
    got = to_bits(C)
    assert np.array_equal(got.T if cm else got, exp)


def test_tiled_8192_matches_c_abi(co, wave, dev):
    """The 8192^3 code object computes what wave_gemm_launch computes, bit
    for bit (same tiles, same kernel body), on uniform [-1, 1) inputs."""
    g = torch.Generator(device="cpu").manual_seed(7)
    A = (torch.rand((8192, 8192), generator=g) * 2 - 1).to(torch.float16).to(dev)
    B = (torch.rand((8192, 8192), generator=g) * 2 - 1).to(torch.float16).to(dev)
    C = torch.empty((8192, 8192), dtype=torch.float16, device=dev)
    launch_tiled(co, "gemm_f16_f16_rm_8192x8192x8192", (32, 32), A, B, C)
    ref = wave.gemm(A, B, out_dtype=torch.float16)
    torch.cuda.synchronize()
    assert torch.equal(C, ref)


def test_tiled_8192_8wave_profile(co, wave, oracle, dev):
    """gfx950-f16-256x256-8wave at 8192^3 (block 512, bm=2 bn=4, wave tiles
    8 x 4 -> grid (32, 32), column-major f16 C) on bucket inputs: every sum
    is exact, so it equals wave_gemm_launch's column-major C bit for bit."""
    a = oracle.gemm_inputs(8192, 8192, 1, 3, 0)
    b = oracle.gemm_inputs(8192, 8192, 1, 3, 1)
    A, B = to_dev(a, torch.float16, dev), to_dev(b, torch.float16, dev)
    del a, b
    C = torch.empty((8192, 8192), dtype=torch.float16, device=dev)
    launch_tiled(co, "gemm_f16_f16_cm_8192x8192x8192_b512", runner_grid(8192, 8192, 2, 4, 8, 4),
                 A, B, C, block=512)
    ref = wave.gemm(A, B, out_dtype=torch.float16, layout="col")
    torch.cuda.synchronize()
    assert torch.equal(C, ref)


@pytest.mark.parametrize("block", [128, 64])
def test_tiled_wrong_block_writes_nothing(co, oracle, dev, block):
    """A launch with a smaller block than the code object is built for
    returns without touching C (a larger one the runtime refuses: the
    kernel's launch bounds cap its block size)."""
    _, _, A, B = bucket_gemm(oracle, dev, 32, 32, 64, 1, 7)
    C = torch.full((32, 32), 3.0, dtype=torch.float32, device=dev)
    launch_tiled(co, "gemm_f16_f32_rm_32x32x64", (1, 1), A, B, C, block=block)
    assert bool((C == 3.0).all())


def up8(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.uint8)).to(dev)


@pytest.mark.parametrize("name,block", [("mxfp4_f32_rm_256x512x512", 512),
                                        ("mxfp4_f32_rm_256x512x512_b256", 256)])
@pytest.mark.parametrize("grid", [(1, 2), (2, 1), (1, 1), (8, 8)])
def test_mxfp4_runner_launch(co, oracle, dev, grid, name, block):
    """wmma_f16_matmul_tiled(A, B, C, A_scale, B_scale, trip), mxfp4 input
    type (runner.cpp:1792-1794): block 512 (gfx950-mxfp4-256x256-8wave) or
    256, no dynamic LDS, the runner's random codes and scales (exact at
    K = 512), any grid."""
    M, N, K = 256, 512, 512
    a, b, sa, sb = oracle.mxfp4_operands(M, N, K, 7)
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    with co.CodeObject(name) as mod:
        mod.kernel("wmma_f16_matmul_tiled").launch(
            grid, (block,), [up8(a, dev), up8(b, dev), C, up8(sa, dev), up8(sb, dev), 3])
        torch.cuda.synchronize()
    assert np.array_equal(C.cpu().numpy(), oracle.gemm_mxfp4(a, b, sa, sb))


def test_mxfp4_wrong_block_writes_nothing(co, oracle, dev):
    a, b, sa, sb = oracle.mxfp4_operands(256, 512, 512, 7)
    C = torch.full((256, 512), 3.0, dtype=torch.float32, device=dev)
    with co.CodeObject("mxfp4_f32_rm_256x512x512") as mod:
        mod.kernel("wmma_f16_matmul_tiled").launch(
            (2, 1), (256,), [up8(a, dev), up8(b, dev), C, up8(sa, dev), up8(sb, dev), 0])
        torch.cuda.synchronize()
    assert bool((C == 3.0).all())


def test_mxfp4_aiter_code_object(co, oracle, dev):
    """-DWAVE_ABI_MXFP4_AITER: the same symbol and arguments, B and scales in
    the AITER layouts (--mxfp4-input-layout aiter), no dynamic LDS."""
    M, N, K = 256, 512, 384
    a, b, sa, sb = oracle.mxfp4_operands(M, N, K, 7)
    ba = oracle.mxfp4_aiter_b(b, N, K)
    saa, sba = oracle.mxfp4_aiter_scales(sa, M, K), oracle.mxfp4_aiter_scales(sb, N, K)
    C = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    with co.CodeObject("mxfp4a_f16_rm_256x512x384") as mod:
        mod.kernel("wmma_f16_matmul_tiled").launch(
            (2,), (512,), [up8(a, dev), up8(ba, dev), C, up8(saa, dev), up8(sba, dev), 0])
        torch.cuda.synchronize()
    exp = oracle.round_output(oracle.gemm_mxfp4(a, b, sa, sb), 1)
    assert np.array_equal(to_bits(C), exp)


def test_mxfp4_4096_matches_c_abi(co, wave, dev):
    """The 4096x4096x8192 f16 column-major code object (the reference's MXFP4
    profile layout) computes what wave_gemm_mxfp4_launch computes, bit for
    bit."""
    g = torch.Generator(device=dev).manual_seed(3)
    M, N, K = 4096, 4096, 8192
    A = torch.randint(0, 256, (M, K // 2), generator=g, device=dev, dtype=torch.uint8)
    B = torch.randint(0, 256, (N, K // 2), generator=g, device=dev, dtype=torch.uint8)
    SA = torch.randint(124, 128, (K // 32, M), generator=g, device=dev, dtype=torch.uint8)
    SB = torch.randint(124, 128, (K // 32, N), generator=g, device=dev, dtype=torch.uint8)
    C = torch.empty((N, M), dtype=torch.float16, device=dev)
    with co.CodeObject("mxfp4_f16_cm_4096x4096x8192") as mod:
        mod.kernel("wmma_f16_matmul_tiled").launch((256,), (512,), [A, B, C, SA, SB, 0])
    ref = wave.gemm_mxfp4(A, B, SA, SB, out_dtype=torch.float16, layout="col")
    torch.cuda.synchronize()
    assert torch.equal(C, ref)


@pytest.mark.parametrize("workers", [6, 7, 13, 64])
def test_streamk_runner_launch(co, wave, oracle, dev, workers):
    """512x768x1024 f16, column-major f16 C: 6 tiles x 16 K units; 6 workers
    is the aligned case, the others split tiles across workers."""
    M, N, K = 512, 768, 1024
    a, b, A, B = bucket_gemm(oracle, dev, M, N, K, 1, 3)
    sb, cb = wave.streamk_workspace_bytes(M, N, workers)
    scratch = torch.empty(sb // 4, dtype=torch.float32, device=dev)
    counters = torch.zeros(cb // 4, dtype=torch.int32, device=dev)
    C = torch.zeros((N, M), dtype=torch.float16, device=dev)  # column-major M x N
    with co.CodeObject("streamk_f16_512x768x1024") as mod:
        mod.kernel("gfx950_f16_streamk_gemm").launch(
            (workers,), (256,), [A, B, C, scratch, counters, workers])
        torch.cuda.synchronize()
    exp = oracle.round_output(oracle.gemm_nt(a, b, 1), 1)
    assert np.array_equal(to_bits(C).T, exp)
    assert int(counters.count_nonzero()) == 0


def test_fa_bf16_runner_launch(co, wave, oracle, dev):
    """B1 H2 S512 bf16 with the reference's bucket inputs (runner :194-202),
    grid (S/256, B*H) = (2, 2), block 512, dynamic LDS 136192: every row
    within the reference's 1.35e-3 of the double-precision softmax beyond the
    bf16 rounding of O (WaveGfx950FlashAttention.md:39-41), and bit-identical
    to wave_fa_fwd_launch."""
    Bt, H, S, D = 1, 2, 512, 128
    q, k, v = oracle.fa_gfx950_inputs(Bt * H * S * D, 3, 1)
    Q, Kt, V = (to_dev(x, torch.bfloat16, dev).view(Bt, H, S, D) for x in (q, k, v))
    O = torch.zeros_like(Q)
    with co.CodeObject("fa_bf16_b1_h2_s512") as mod:
        mod.kernel("flash_attention_bf16_gfx950").launch(
            (S // 256, Bt * H), (512,), [Q, Kt, V, O], dynamic_lds=FA_LDS)
        torch.cuda.synchronize()
    got = oracle.bits_to_f32(to_bits(O).reshape(Bt * H, S, D), 2)
    hh, rr = np.meshgrid(np.arange(H), np.arange(S), indexing="ij")
    ref = oracle.attention_rows(q, k, v, dtype=2, batch=Bt, q_heads=H, kv_heads=H, seq_q=S,
                                seq_k=S, head_dim=D, causal=False, scale=1.0 / math.sqrt(D),
                                heads=hh.ravel(), rows=rr.ravel())
    excess = np.abs(got[hh.ravel(), rr.ravel()] - ref) - 2.0 ** -8 * np.abs(ref)
    assert float(excess.max()) <= 1.35e-3
    assert torch.equal(O, wave.flash_attention(Q, Kt, V))


@pytest.mark.parametrize("lds", [68096, 102400 - 16])
def test_fa_bf16_too_little_lds_writes_nothing(co, oracle, dev, lds):
    """The runner's 4-wave default --dynamic-lds (68096) is too small for the
    8-wave kernel (102400): it returns without writing O."""
    Bt, H, S, D = 1, 2, 512, 128
    q, k, v = oracle.fa_gfx950_inputs(Bt * H * S * D, 3, 1)
    Q, Kt, V = (to_dev(x, torch.bfloat16, dev).view(Bt, H, S, D) for x in (q, k, v))
    O = torch.full_like(Q, 5.0)
    with co.CodeObject("fa_bf16_b1_h2_s512") as mod:
        mod.kernel("flash_attention_bf16_gfx950").launch(
            (S // 256, Bt * H), (512,), [Q, Kt, V, O], dynamic_lds=lds)
        torch.cuda.synchronize()
    assert bool((O == 5.0).all())


def test_fa_bf16_exact_lds_minimum(co, wave, oracle, dev):
    """102400 bytes (the kernel's K and V^T rings) is enough."""
    Bt, H, S, D = 1, 2, 512, 128
    q, k, v = oracle.fa_gfx950_inputs(Bt * H * S * D, 4, 1)
    Q, Kt, V = (to_dev(x, torch.bfloat16, dev).view(Bt, H, S, D) for x in (q, k, v))
    O = torch.zeros_like(Q)
    with co.CodeObject("fa_bf16_b1_h2_s512") as mod:
        mod.kernel("flash_attention_bf16_gfx950").launch(
            (S // 256, Bt * H), (512,), [Q, Kt, V, O], dynamic_lds=102400)
        torch.cuda.synchronize()
    assert torch.equal(O, wave.flash_attention(Q, Kt, V))


@pytest.mark.parametrize("threads", [64, 32, 256])
def test_fa_f32_runner_launch(co, oracle, dev, threads):
    """block_m 16, seq_n 256, head_dim 64, grid 1, the runner's --threads."""
    q, k, v = oracle.fa_f32_inputs(16, 256, 64, 9)
    Q, Kt, V = (to_dev(x, torch.float16, dev) for x in (q, k, v))
    O = torch.zeros((16, 64), dtype=torch.float32, device=dev)
    with co.CodeObject("fa32_m16_n256_d64") as mod:
        mod.kernel("flash_attention_f32").launch((1,), (threads,), [Q, Kt, V, O])
        torch.cuda.synchronize()
    assert float(np.abs(O.cpu().numpy() - oracle.fa_f32_reference(q, k, v)).max()) <= 3e-3


@pytest.mark.parametrize("name,qk", [("fa4_bf16_b1_h2_s512", None),
                                     ("fa4_bf16_b1_h2_s512_qk1", 1.0)])
def test_fa4_bf16_runner_default_launch(co, wave, dev, name, qk):
    """The 4-wave code objects under the FA runner's defaults (--threads 256
    --dynamic-lds 68096; wave_flash_attention.py:114-135): bit-identical to
    the C ABI's 4-wave kernel."""
    B, H, S, D = 1, 2, 512, 128
    g = torch.Generator(device="cpu").manual_seed(31)
    q, k, v = ((torch.rand((B, H, S, D), generator=g) * 2 - 1).to(torch.bfloat16).to(dev)
               for _ in range(3))
    o = torch.full_like(q, float("nan"))
    with co.CodeObject(name) as mod:
        mod.kernel("flash_attention_bf16_gfx950").launch((S // 256, B * H), (256,),
                                                         [q, k, v, o], dynamic_lds=68096)
    ref = wave.flash_attention(q, k, v, qk_max_abs=qk, waves=4)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)


@pytest.mark.parametrize("block,lds", [(128, 68096), (256, 45056 - 1024)])
def test_fa4_bf16_outside_contract_writes_nothing(co, dev, block, lds):
    """Another block size (below the 256 the object is built for; above it
    the runtime refuses the launch, its registers do not fit two waves per
    SIMD) or too little dynamic LDS: the kernel returns without writing."""
    q = torch.zeros((1, 2, 512, 128), dtype=torch.bfloat16, device=dev)
    o = torch.full_like(q, 3.0)
    with co.CodeObject("fa4_bf16_b1_h2_s512") as mod:
        mod.kernel("flash_attention_bf16_gfx950").launch((2, 2), (block,), [q, q, q, o],
                                                         dynamic_lds=lds)
        torch.cuda.synchronize()
    assert bool((o == 3.0).all())


def test_fa_bf16_fixed_max_code_object(co, wave, oracle, dev):
    """The reference's qk_max_abs=1 profile as a code object
    (-DWAVE_ABI_FA_QK_MAX_ABS=1.0): bit-identical to
    wave_fa_fwd_bounded_launch with the same bound."""
    Bt, H, S, D = 1, 2, 512, 128
    q, k, v = oracle.fa_gfx950_inputs(Bt * H * S * D, 6, 1)
    Q, Kt, V = (to_dev(x, torch.bfloat16, dev).view(Bt, H, S, D) for x in (q, k, v))
    O = torch.zeros_like(Q)
    with co.CodeObject("fa_bf16_b1_h2_s512_qk1") as mod:
        mod.kernel("flash_attention_bf16_gfx950").launch(
            (S // 256, Bt * H), (512,), [Q, Kt, V, O], dynamic_lds=FA_LDS)
        torch.cuda.synchronize()
    assert torch.equal(O, wave.flash_attention(Q, Kt, V, qk_max_abs=1.0))
