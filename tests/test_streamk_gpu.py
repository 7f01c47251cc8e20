"""GPU parity of the Stream-K GEMM (wave_gemm_streamk_launch).

Mirrors test/Integration/wave_gfx950_streamk_f16_runtime.mlir:3-80: split
(5 workers) and aligned (2 workers) partitions of 512x512x256, random and
HPL inputs, column-major f16 output, many launches reusing one workspace,
and the post-run "counters are zero" check (runner.cpp:1718-1742).  Bucket
inputs make the fp32 sums exact, so results are compared bitwise with the
oracle and with the tiled kernel; the fixed-order reduction makes repeated
launches bit-identical.
"""

import numpy as np
import pytest
import torch

from conftest import to_bits, to_dev

pytestmark = pytest.mark.gpu

TDT = {1: torch.float16, 2: torch.bfloat16}


def inputs(oracle, dev, M, N, K, dt, seed=5, mode=None):
    mode = oracle.MODE_RANDOM if mode is None else mode
    a = oracle.gemm_inputs(M, K, dt, seed, 0, mode)
    b = oracle.gemm_inputs(N, K, dt, seed, 1, mode)
    return a, b, to_dev(a, TDT[dt], dev), to_dev(b, TDT[dt], dev)


@pytest.mark.parametrize("workers", [5, 2, 1, 3, 7, 16])
@pytest.mark.parametrize("mode", ["random", "hpl"])
def test_reference_streamk_cases(wave, oracle, dev, workers, mode):
    M = N = 512
    K = 256
    m = oracle.MODE_RANDOM if mode == "random" else oracle.MODE_HPL
    a, b, da, db = inputs(oracle, dev, M, N, K, 1, mode=m)
    ws = wave.StreamKWorkspace(M, N, workers, dev)
    c = wave.gemm_streamk(da, db, workers, out_dtype=torch.float16, layout="col",
                          workspace=ws)
    torch.cuda.synchronize()
    ref = oracle.round_output(oracle.gemm_nt(a, b, 1), 1)
    got = to_bits(c.t().contiguous())
    if mode == "random":
        assert np.array_equal(got, ref)
    else:
        # HPL values are not dyadic-exact; runner tolerance 1e-2 + 1e-3|exp|
        g = oracle.f16_bits_to_f32(got)
        e = oracle.f16_bits_to_f32(ref)
        assert np.all(np.abs(g - e) <= 1e-2 + 1e-3 * np.abs(e))
    assert ws.nonzero_counters() == 0


def test_workspace_reuse_many_launches(wave, oracle, dev):
    M = N = 512
    K = 256
    a, b, da, db = inputs(oracle, dev, M, N, K, 1)
    ws = wave.StreamKWorkspace(M, N, 5, dev)
    first = wave.gemm_streamk(da, db, 5, out_dtype=torch.float16, workspace=ws)
    out = torch.empty_like(first)
    for _ in range(200):
        wave.gemm_streamk(da, db, 5, out_dtype=torch.float16, workspace=ws, out=out)
    torch.cuda.synchronize()
    assert torch.equal(first, out)
    assert ws.nonzero_counters() == 0
    ref = oracle.round_output(oracle.gemm_nt(a, b, 1), 1)
    assert np.array_equal(to_bits(first), ref)


@pytest.mark.parametrize("in_dt", [1, 2])
@pytest.mark.parametrize("out_dt", [torch.float32, torch.float16, torch.bfloat16])
# All of these have K % 4 == 0 and 8-byte aligned rows, so Stream-K and the
# tiled kernel both run the hybrid DMA path (whole 64-deep stages on the
# ring, the K remainder through registers); (512, 512, 1056) is whole tiles
# with K off the 64-deep stage.  test_masked_streamk_many_contributors covers
# the bounds-checked Stream-K path.
@pytest.mark.parametrize("shape,workers", [((128, 1024, 2048), 40), ((300, 520, 700), 9),
                                           ((257, 255, 4100), 13), ((1024, 1024, 1024), 64),
                                           ((512, 512, 1056), 7)])
def test_ragged_streamk_matches_tiled(wave, oracle, dev, in_dt, out_dt, shape, workers):
    M, N, K = shape
    a, b, da, db = inputs(oracle, dev, M, N, K, in_dt, seed=11)
    sk = wave.gemm_streamk(da, db, workers, out_dtype=out_dt)
    tiled = wave.gemm(da, db, out_dtype=out_dt)
    torch.cuda.synchronize()
    assert torch.equal(sk, tiled)


@pytest.mark.parametrize("in_dt", [1, 2])
@pytest.mark.parametrize("out_dt", [torch.float32, torch.float16])
@pytest.mark.parametrize("shape,workers", [((300, 520, 701), 30), ((257, 255, 4102), 13)])
def test_masked_streamk_many_contributors(wave, oracle, dev, in_dt, out_dt, shape, workers):
    """K % 4 != 0: Stream-K runs its bounds-checked kernel (element loads with
    zero fill, the path taken for K % 4 != 0 or unaligned A/B), here with 3
    to 6 contributors per tile, so its fold of more than two partials and
    the two-part pass both run.  Bucket inputs: bit-exact against the tiled
    kernel, and the counters are zero again after every launch."""
    M, N, K = shape
    a, b, da, db = inputs(oracle, dev, M, N, K, in_dt, seed=19)
    ws = wave.StreamKWorkspace(M, N, workers, dev)
    tiled = wave.gemm(da, db, out_dtype=out_dt)
    for _ in range(3):
        sk = wave.gemm_streamk(da, db, workers, out_dtype=out_dt, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(sk, tiled)
        assert ws.nonzero_counters() == 0
    if out_dt == torch.float32:
        assert np.array_equal(sk.cpu().numpy(), oracle.gemm_nt(a, b, in_dt))


def test_dirty_counters_are_detected_and_reset(wave, oracle, dev):
    """Failure contract: counters must start at zero (Stream-K design doc
    :98-101).  Dirty them from the host, see the check report it, reset."""
    M = N = 512
    ws = wave.StreamKWorkspace(M, N, 5, dev)
    ws.counters.fill_(3)
    assert ws.nonzero_counters() == 4
    ws.reset()
    assert ws.nonzero_counters() == 0


def test_config3_streamk_bf16(wave, oracle, dev):
    """BASELINE config 3a through Stream-K: 128x8192x8192 bf16 has only 32
    output tiles, so 256 workers split the K loop of every tile."""
    M, N, K = 128, 8192, 8192
    g = torch.Generator(device="cpu").manual_seed(3)
    a = (torch.randn((M, K), generator=g) / np.sqrt(K)).to(torch.bfloat16)
    b = (torch.randn((N, K), generator=g) / np.sqrt(K)).to(torch.bfloat16)
    c = wave.gemm_streamk(a.to(dev), b.to(dev), 256, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    abits = a.view(torch.int16).numpy().view(np.uint16)
    bbits = b.view(torch.int16).numpy().view(np.uint16)
    got = c.float().cpu().numpy()
    ref = oracle.gemm_nt_rows(abits, bbits, 0, M, 2)
    assert float(np.abs(got - ref).max()) <= 2e-3 * np.sqrt(K)


# ---- shape-driven dispatch (wave_gemm_auto_launch) ------------------------------
def auto_workers(M, N, K, cus):
    """Stream-K workers wave_gemm_auto_launch picks for (M, N, K) on a device
    with `cus` compute units (0: the tiled or short-M kernel); the rules of
    auto_workers in 7_amd/csrc/wave_runtime.cpp, restated so the expected
    choice follows the CU count the device reports."""
    t = -(-M // 256) * -(-N // 256)
    if M <= 128 or K < 4096 or t >= cus:
        return 0
    if t * 2 >= cus and K < 8192:
        return 0
    if t * 2 > cus:
        return 0
    w = min(t * 2, cus)
    if t * 4 <= cus:
        w = max(w, min(t * (K // 2048), cus // 2))
    return min(w, t * -(-K // 64))


def short_m_plan(M, N, K, cus):
    """(column block, K splits) of the split short-M kernel
    wave_gemm_auto_launch picks for (M, N, K), (0, 0) for none; the rules of
    skinny_split_plan in 7_amd/csrc/gemm_skinny.hip: 64-column blocks when
    CUs / blocks >= 2, else 128-column ones (2 splits at least when the
    unsplit kernel's N / 32 CTAs exceed the CUs); at most 4 splits, at least
    8 stages of 64 a split; none when a split keeps less than 2048 of K, or
    less than 4096 where M <= 96 or the unsplit kernel's N / 32 CTAs do not
    fill the CUs."""
    if M > 128 or N < 1024 or K % 64 or K * 2 * 128 >= 2**32 or N * K * 2 >= 2**32:
        return 0, 0
    unsplit = -(-N // 32)
    for bn in (64, 128):
        s = min(cus // -(-N // bn), 4)
        if s < 2 and bn == 128 and unsplit > cus:
            s = 2
        while s > 1 and K // 64 < 8 * s:
            s -= 1
        if s < 2:
            continue
        ks = K // s
        if ks < 2048 or (ks < 4096 and (M <= 96 or unsplit < cus)):
            return 0, 0
        return bn, s
    return 0, 0


def device_cus(dev):
    return torch.cuda.get_device_properties(dev).multi_processor_count


def expected_workspace(wave, M, N, K, dev):
    bn, s = short_m_plan(M, N, K, device_cus(dev))
    if s:  # fp32 partial slots, then two 64-bit counters a column block
        tiles = -(-N // bn)
        return 0, tiles * s * 128 * bn * 4 + tiles * 16
    w = auto_workers(M, N, K, device_cus(dev))
    if w == 0:
        return 0, 0
    sb, cb = wave.streamk_workspace_bytes(M, N, w)
    return w, sb + cb


@pytest.mark.parametrize("shape", [(2048, 512, 8192),    # 16 tiles, long K
                                   (1000, 300, 4100),    # ragged, 8 tiles
                                   # K % 4 != 0: the bounds-checked Stream-K kernel
                                   (1000, 300, 4101),
                                   # ragged, K off the stage, 16 tiles:
                                   # 128 workers, 8-9 contributors a tile
                                   (1000, 1000, 16400),
                                   (4096, 4096, 512),    # 256 tiles
                                   (3072, 3072, 8192),   # 144 tiles: uneven split
                                   (4096, 2048, 4096),   # 128 tiles, K 4096
                                   (128, 1024, 8192),    # split short-M kernel
                                   (128, 1024, 192)])    # unsplit short-M kernel
def test_auto_dispatch_matches_tiled(wave, oracle, dev, shape):
    """The workspace size names the worker count the dispatch picks (checked
    against the rules for this device's CU count).  Bucket inputs make every
    sum exact, so the auto path (Stream-K or not) equals wave_gemm_launch bit
    for bit; a too-small workspace falls back to the tiled kernel."""
    M, N, K = shape
    need = wave.gemm_auto_workspace_bytes(M, N, K)
    assert need == expected_workspace(wave, M, N, K, dev)[1]
    a = oracle.gemm_inputs(M, K, 2, 5, 0)
    b = oracle.gemm_inputs(N, K, 2, 5, 1)
    A, B = to_dev(a, torch.bfloat16, dev), to_dev(b, torch.bfloat16, dev)
    ref = wave.gemm(A, B, out_dtype=torch.bfloat16)
    ws = torch.full((max(need, 1),), 0xFF, dtype=torch.uint8, device=dev)  # dirty counters
    for _ in range(2):
        got = wave.gemm_auto(A, B, out_dtype=torch.bfloat16, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
    small = torch.empty((max(need // 2, 1),), dtype=torch.uint8, device=dev)
    assert torch.equal(wave.gemm_auto(A, B, out_dtype=torch.bfloat16, workspace=small), ref)


def test_config3c_auto_dispatch(wave, oracle, dev):
    """BASELINE config 3c (8192 x 1024 x 28672 bf16: 128 output tiles) through
    wave_gemm_auto_launch, the path bench.py reports for it (Stream-K with
    2 * tiles workers on 256 CUs: 448 K units a tile split in two).
    * N(0,1)/sqrt(K) inputs: sampled rows within 2e-3 * sqrt(K) of the
      oracle;
    * bucket inputs: bit-identical to wave_gemm_launch, on a dirty workspace,
      twice, with the counters back at zero."""
    M, N, K = 8192, 1024, 28672
    w, need = expected_workspace(wave, M, N, K, dev)
    assert wave.gemm_auto_workspace_bytes(M, N, K) == need
    if device_cus(dev) == 256:
        assert w == 256
    g = torch.Generator(device="cpu").manual_seed(31)
    a = (torch.randn((M, K), generator=g) / np.sqrt(K)).to(torch.bfloat16)
    b = (torch.randn((N, K), generator=g) / np.sqrt(K)).to(torch.bfloat16)
    ws = torch.full((max(need, 1),), 0xFF, dtype=torch.uint8, device=dev)
    c = wave.gemm_auto(a.to(dev), b.to(dev), out_dtype=torch.bfloat16, workspace=ws)
    torch.cuda.synchronize()
    abits = a.view(torch.int16).numpy().view(np.uint16)
    bbits = b.view(torch.int16).numpy().view(np.uint16)
    got = c.float().cpu().numpy()
    bt = oracle.gemm_prepare_bt(bbits, 2)
    rows = [0, 1, 255, 256, 4095, 4096, 8190, 8191] + list(range(97, M, 1021))
    worst = 0.0
    for r in rows:
        ref = oracle.gemm_nt_rows_bt(abits, bt, r, r + 1, 2)[0]
        worst = max(worst, float(np.abs(got[r] - ref).max()))
    assert worst <= 2e-3 * np.sqrt(K), worst
    del a, b, c, bt
    a = oracle.gemm_inputs(M, K, 2, 5, 0)
    b = oracle.gemm_inputs(N, K, 2, 5, 1)
    A, B = to_dev(a, torch.bfloat16, dev), to_dev(b, torch.bfloat16, dev)
    ref = wave.gemm(A, B, out_dtype=torch.bfloat16)
    ws.fill_(0xFF)
    for _ in range(2):
        got = wave.gemm_auto(A, B, out_dtype=torch.bfloat16, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
    if w:
        sb, _ = wave.streamk_workspace_bytes(M, N, w)
        assert int(ws[sb:].count_nonzero()) == 0


# ---- split short-M kernel (wave_gemm_auto_launch, M <= 128) ---------------------
def test_config3a_auto_dispatch(wave, oracle, dev):
    """BASELINE config 3a (128 x 8192 x 8192 bf16) through
    wave_gemm_auto_launch, the path bench.py reports for it: 128 column
    blocks of 64, K split in 2 on 256 CUs, partials reduced by each block's
    last arriver.
    * N(0,1)/sqrt(K) inputs: every row within 2e-3 * sqrt(K) of the oracle;
    * bucket inputs: bit-identical to wave_gemm_launch (the unsplit short-M
      kernel), on a dirty workspace, twice, with the counters back at zero."""
    M, N, K = 128, 8192, 8192
    cus = device_cus(dev)
    bn, s = short_m_plan(M, N, K, cus)
    need = wave.gemm_auto_workspace_bytes(M, N, K)
    assert need == expected_workspace(wave, M, N, K, dev)[1]
    if cus == 256:
        assert (bn, s) == (64, 2)
    g = torch.Generator(device="cpu").manual_seed(37)
    a = (torch.randn((M, K), generator=g) / np.sqrt(K)).to(torch.bfloat16)
    b = (torch.randn((N, K), generator=g) / np.sqrt(K)).to(torch.bfloat16)
    ws = torch.full((max(need, 1),), 0xFF, dtype=torch.uint8, device=dev)
    c = wave.gemm_auto(a.to(dev), b.to(dev), out_dtype=torch.bfloat16, workspace=ws)
    torch.cuda.synchronize()
    abits = a.view(torch.int16).numpy().view(np.uint16)
    bbits = b.view(torch.int16).numpy().view(np.uint16)
    ref = oracle.gemm_nt_rows_bt(abits, oracle.gemm_prepare_bt(bbits, 2), 0, M, 2)
    worst = float(np.abs(c.float().cpu().numpy() - ref).max())
    assert worst <= 2e-3 * np.sqrt(K), worst
    a = oracle.gemm_inputs(M, K, 2, 5, 0)
    b = oracle.gemm_inputs(N, K, 2, 5, 1)
    A, B = to_dev(a, torch.bfloat16, dev), to_dev(b, torch.bfloat16, dev)
    ref = wave.gemm(A, B, out_dtype=torch.bfloat16)
    ws.fill_(0xFF)
    for _ in range(2):
        got = wave.gemm_auto(A, B, out_dtype=torch.bfloat16, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
    if s:
        tiles = -(-N // bn)
        assert int(ws[tiles * s * 128 * bn * 4:].count_nonzero()) == 0


@pytest.mark.parametrize("in_dt", [1, 2])
@pytest.mark.parametrize("out_dt,layout", [(torch.float32, "row"), (torch.float16, "col"),
                                           (torch.bfloat16, "row")])
# On 256 CUs: M from 1 to 128 (waves with no rows skip their MFMAs), N
# ragged against the column block, K splits of unequal length (131 stages
# in 4 splits), 64-column blocks in 4, 3 and 2 splits (N 1500, 5000, 8192)
# and 128-column blocks in 2 (N 11000, 16384, and 24576: 384 CTAs, two
# rounds); 128 x 4096 x 4096 takes the unsplit kernel (1024 of K a split).
@pytest.mark.parametrize("shape", [(1, 1024, 8192), (33, 1500, 8384), (100, 8192, 8192),
                                   (100, 11000, 4096), (128, 16384, 4096), (128, 4096, 8192),
                                   (100, 5000, 12288), (128, 24576, 4096), (128, 4096, 4096)])
def test_split_short_m_matches_unsplit(wave, oracle, dev, in_dt, out_dt, layout, shape):
    """Bucket inputs make every fp32 sum exact, so the split short-M kernel
    equals the unsplit one (wave_gemm_launch) bit for bit, on a dirty
    workspace, twice in a row."""
    M, N, K = shape
    need = wave.gemm_auto_workspace_bytes(M, N, K)
    assert need == expected_workspace(wave, M, N, K, dev)[1]
    a = oracle.gemm_inputs(M, K, in_dt, 7, 0)
    b = oracle.gemm_inputs(N, K, in_dt, 7, 1)
    A, B = to_dev(a, TDT[in_dt], dev), to_dev(b, TDT[in_dt], dev)
    ref = wave.gemm(A, B, out_dtype=out_dt, layout=layout)
    ws = torch.full((max(need, 1),), 0xFF, dtype=torch.uint8, device=dev)
    for _ in range(2):
        got = wave.gemm_auto(A, B, out_dtype=out_dt, layout=layout, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)


@pytest.mark.parametrize("shape,workers", [((2048, 2048, 8192), 128),   # 2 contributors
                                           ((1024, 1024, 8192), 64),    # 4
                                           ((1000, 1000, 8200), 128)])  # ragged, 8-9
def test_streamk_alternating_inputs(wave, oracle, dev, shape, workers):
    """Two different B on one Stream-K workspace, alternated launch after
    launch: each output equals the tiled kernel's for its own B, so the last
    arriver of a tile never reads a contributor's partial from an earlier
    launch (partials are read with device-coherent loads)."""
    M, N, K = shape
    a = oracle.gemm_inputs(M, K, 1, 9, 0)
    b0 = oracle.gemm_inputs(N, K, 1, 9, 1)
    b1 = oracle.gemm_inputs(N, K, 1, 9, 2)
    A = to_dev(a, torch.float16, dev)
    Bs = [to_dev(b0, torch.float16, dev), to_dev(b1, torch.float16, dev)]
    refs = [wave.gemm(A, B, out_dtype=torch.float32) for B in Bs]
    assert not torch.equal(refs[0], refs[1])
    ws = wave.StreamKWorkspace(M, N, workers, dev)
    out = torch.empty_like(refs[0])
    for i in range(16):
        wave.gemm_streamk(A, Bs[i & 1], workers, out_dtype=torch.float32, workspace=ws, out=out)
        torch.cuda.synchronize()
        assert torch.equal(out, refs[i & 1]), i
    assert ws.nonzero_counters() == 0


@pytest.mark.parametrize("shape", [(128, 8192, 8192), (128, 4096, 8192), (100, 5000, 12288)])
def test_split_short_m_alternating_inputs(wave, oracle, dev, shape):
    """Two different B on one workspace, alternated launch after launch: each
    output equals wave_gemm_launch's for its own B, so the last arriver never
    reads a partial of the other input (the exchange's device-scope stores
    and loads leave no stale copy in a cache on the way)."""
    M, N, K = shape
    need = wave.gemm_auto_workspace_bytes(M, N, K)
    assert need == expected_workspace(wave, M, N, K, dev)[1]
    a = oracle.gemm_inputs(M, K, 2, 7, 0)
    b0 = oracle.gemm_inputs(N, K, 2, 7, 1)
    b1 = oracle.gemm_inputs(N, K, 2, 7, 2)
    A = to_dev(a, torch.bfloat16, dev)
    Bs = [to_dev(b0, torch.bfloat16, dev), to_dev(b1, torch.bfloat16, dev)]
    refs = [wave.gemm(A, B, out_dtype=torch.bfloat16) for B in Bs]
    assert not torch.equal(refs[0], refs[1])
    ws = torch.zeros((max(need, 1),), dtype=torch.uint8, device=dev)
    out = torch.empty_like(refs[0])
    for i in range(24):
        wave.gemm_auto(A, Bs[i & 1], out_dtype=torch.bfloat16, workspace=ws, out=out)
        torch.cuda.synchronize()
        assert torch.equal(out, refs[i & 1]), i


def test_split_short_m_graph_replays(wave, oracle, dev):
    """A captured split short-M launch replays with one fixed counter epoch:
    each replay equals wave_gemm_launch's output, with eager launches for
    another B on the same workspace between the replays (every launch leaves
    the counters at zero, and a word of another epoch counts as zero).  On
    256 CUs: 64-column blocks in 3 K splits."""
    M, N, K = 100, 5000, 12288
    bn, s = short_m_plan(M, N, K, device_cus(dev))
    if not s:
        pytest.skip("this device's CU count takes the unsplit kernel at this shape")
    need = wave.gemm_auto_workspace_bytes(M, N, K)
    a = oracle.gemm_inputs(M, K, 2, 11, 0)
    b0 = oracle.gemm_inputs(N, K, 2, 11, 1)
    b1 = oracle.gemm_inputs(N, K, 2, 11, 2)
    A = to_dev(a, torch.bfloat16, dev)
    B0, B1 = to_dev(b0, torch.bfloat16, dev), to_dev(b1, torch.bfloat16, dev)
    ref0 = wave.gemm(A, B0, out_dtype=torch.bfloat16)
    ref1 = wave.gemm(A, B1, out_dtype=torch.bfloat16)
    assert not torch.equal(ref0, ref1)
    ws = torch.full((need,), 0xFF, dtype=torch.uint8, device=dev)
    out = torch.empty_like(ref0)
    wave.gemm_auto(A, B0, out_dtype=torch.bfloat16, workspace=ws, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out, ref0)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph.capture_begin()
        wave.gemm_auto(A, B0, out_dtype=torch.bfloat16, workspace=ws, out=out)
        graph.capture_end()
    torch.cuda.current_stream().wait_stream(stream)
    other = torch.empty_like(ref1)
    for i in range(4):
        out.zero_()
        wave.gemm_auto(A, B1, out_dtype=torch.bfloat16, workspace=ws, out=other)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref0), i
        assert torch.equal(other, ref1), i
    tiles = -(-N // bn)
    assert int(ws[tiles * s * 128 * bn * 4:].count_nonzero()) == 0


def test_split_short_m_shared_workspace_two_shapes(wave, oracle, dev):
    """One workspace alternated between two split shapes whose layouts
    overlap: on 256 CUs the counters of 100 x 5000 x 12288 (3 splits) sit
    inside the fp32 partial slots of 128 x 8192 x 8192 (2 splits), so its
    launches find their counter words holding partial sums the other shape
    left there.  A word carrying another launch's epoch counts as zero, so
    every output equals wave_gemm_launch's, bit for bit (bucket inputs)."""
    cus = device_cus(dev)
    shapes = [(128, 8192, 8192), (100, 5000, 12288)]
    plans = [short_m_plan(M, N, K, cus) for M, N, K in shapes]
    if not all(s for _, s in plans):
        pytest.skip("this device's CU count takes the unsplit kernel for one of the shapes")
    need = max(wave.gemm_auto_workspace_bytes(*sh) for sh in shapes)
    ws = torch.zeros((need,), dtype=torch.uint8, device=dev)
    cases = []
    for i, (M, N, K) in enumerate(shapes):
        a = oracle.gemm_inputs(M, K, 2, 13 + i, 0)
        b = oracle.gemm_inputs(N, K, 2, 13 + i, 1)
        A, B = to_dev(a, torch.bfloat16, dev), to_dev(b, torch.bfloat16, dev)
        cases.append((A, B, wave.gemm(A, B, out_dtype=torch.bfloat16)))
    for it in range(6):
        for j, (A, B, ref) in enumerate(cases):
            got = wave.gemm_auto(A, B, out_dtype=torch.bfloat16, workspace=ws)
            torch.cuda.synchronize()
            assert torch.equal(got, ref), (it, j)


def test_split_short_m_float_inputs_same_bits(wave, oracle, dev):
    """Inexact inputs, fp32 C: the last arriver sums the partials in split
    order whichever arrives last, so every launch gives the same bits, within
    2e-3 * sqrt(K) of the oracle."""
    M, N, K = 96, 4096, 8192
    g = torch.Generator(device="cpu").manual_seed(41)
    a = (torch.randn((M, K), generator=g) / np.sqrt(K)).to(torch.float16)
    b = (torch.randn((N, K), generator=g) / np.sqrt(K)).to(torch.float16)
    A, B = a.to(dev), b.to(dev)
    ws = torch.empty((max(wave.gemm_auto_workspace_bytes(M, N, K), 1),), dtype=torch.uint8,
                     device=dev)
    first = wave.gemm_auto(A, B, out_dtype=torch.float32, workspace=ws)
    out = torch.empty_like(first)
    for _ in range(20):
        wave.gemm_auto(A, B, out_dtype=torch.float32, workspace=ws, out=out)
        torch.cuda.synchronize()
        assert torch.equal(out, first)
    abits = a.view(torch.int16).numpy().view(np.uint16)
    bbits = b.view(torch.int16).numpy().view(np.uint16)
    ref = oracle.gemm_nt_rows_bt(abits, oracle.gemm_prepare_bt(bbits, 1), 0, M, 1)
    assert float(np.abs(first.cpu().numpy() - ref).max()) <= 2e-3 * np.sqrt(K)


@pytest.mark.parametrize("shape,workers", [((1024, 1024, 8192), 64),    # 4 contributors
                                           ((1000, 1000, 8200), 128),   # ragged, 8-9
                                           ((512, 512, 4096), 12),      # 5-6
                                           ((2048, 2048, 8192), 128)])  # 2
def test_float_inputs_same_bits_every_launch(wave, dev, shape, workers):
    """Inexact (normal-distributed) inputs with fp32 C: the reduction sums
    the contributors in worker order whichever of them arrives last (and
    takes its own partial from registers or from its slot), so every launch
    gives the same bits; the result is an fp32-accumulated product of the
    bf16 inputs (float64 check on a row sample)."""
    M, N, K = shape
    g = torch.Generator(device="cpu").manual_seed(17)
    a = torch.randn((M, K), generator=g).to(torch.bfloat16)
    b = torch.randn((N, K), generator=g).to(torch.bfloat16)
    A, B = a.to(dev), b.to(dev)
    ws = wave.StreamKWorkspace(M, N, workers, dev)
    first = wave.gemm_streamk(A, B, workers, out_dtype=torch.float32, workspace=ws)
    out = torch.empty_like(first)
    for _ in range(20):
        wave.gemm_streamk(A, B, workers, out_dtype=torch.float32, workspace=ws, out=out)
        torch.cuda.synchronize()
        assert torch.equal(out, first)
    assert ws.nonzero_counters() == 0
    rows = torch.arange(0, M, 97)
    ref = a[rows].double() @ b.double().t()
    err = (first[rows].cpu().double() - ref).abs().max().item()
    assert err <= 1e-5 * K ** 0.5 * 4, err
