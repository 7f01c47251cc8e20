"""The allocation-free Stream-K entry point, wave_gemm_streamk_noalloc_launch
(workspace in the library's static device array), against
wave_gemm_streamk_launch with a caller-owned workspace: the same kernels and
partition, so C must be bit-identical.  Two calls in a row, the second on a
smaller problem, so the second runs on the array the first left behind."""

import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def w():
    m = importlib.import_module("7_amd")
    m.runtime.lib()
    return m


def noalloc(w, a, b, c, workers, layout):
    rt = w.runtime
    M, K = a.shape
    N = b.shape[0]
    odt = {torch.float32: rt.F32, torch.float16: rt.F16, torch.bfloat16: rt.BF16}[c.dtype]
    idt = rt.F16 if a.dtype == torch.float16 else rt.BF16
    return rt.lib().wave_gemm_streamk_noalloc_launch(
        a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K, idt, odt,
        rt.ROW_MAJOR if layout == "row" else rt.COL_MAJOR, workers,
        torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_noalloc_matches_caller_workspace_two_calls(w, dev, dtype):
    g = torch.Generator(device="cpu").manual_seed(21)
    # (M, N, K, workers, layout, out dtype): first a split-tile problem on the
    # DMA path with the maximum worker count, then a smaller ragged one
    # (K % 4 == 0: the hybrid DMA path with a K remainder), then a smaller
    # one with K % 4 != 0 (the bounds-checked Stream-K kernel).
    cases = [(1024, 1536, 2048, 128, "col", dtype), (300, 200, 500, 7, "row", torch.float32),
             (200, 100, 301, 5, "col", torch.float32)]
    for M, N, K, workers, layout, odt in cases:
        a = (torch.rand((M, K), generator=g) * 2 - 1).to(dtype).to(dev)
        b = (torch.rand((N, K), generator=g) * 2 - 1).to(dtype).to(dev)
        ref = w.gemm_streamk(a, b, workers, out_dtype=odt, layout=layout)
        shape = (M, N) if layout == "row" else (N, M)
        got = torch.full(shape, float("nan"), dtype=odt, device=dev)
        assert noalloc(w, a, b, got, workers, layout) == 0, w.runtime.lib().wave_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (M, N, K, workers)


def test_noalloc_repeated_calls_identical(w, dev):
    """Back-to-back calls on one stream (the array's counters reset each
    time) give identical C."""
    g = torch.Generator(device="cpu").manual_seed(5)
    a = (torch.rand((512, 768), generator=g) * 2 - 1).to(torch.float16).to(dev)
    b = (torch.rand((768, 768), generator=g) * 2 - 1).to(torch.float16).to(dev)
    outs = [torch.empty((512, 768), dtype=torch.float16, device=dev) for _ in range(3)]
    for o in outs:
        assert noalloc(w, a, b, o, 13, "row") == 0
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
    assert torch.equal(outs[0], w.gemm_streamk(a, b, 13, out_dtype=torch.float16))


@pytest.mark.parametrize("M,N,workers,layout,status,text", [
    (256, 256, 129, "row", "UNSUPPORTED", b"static workspace"),       # > 128 workers
    (256 * 65, 256 * 64, 8, "row", "UNSUPPORTED", b"static workspace"),  # > 4096 tiles
    (256, 256, 0, "row", "INVALID", b"positive"),
    (256, 256, 2, "row", "INVALID", b"workers=2"),   # more workers than 1 work unit
    (256, 256, 1, "packed", "UNSUPPORTED", b"tile-packed")])
def test_noalloc_rejects_beyond_static_workspace(w, dev, M, N, workers, layout, status, text):
    """Requests beyond the static workspace, or that wave_gemm_streamk_launch
    itself rejects (workers > tiles * K units, tile-packed C): a clear error
    before any device access (the counter reset comes after every check)."""
    rt = w.runtime
    a = torch.zeros((16, 16), dtype=torch.float16, device=dev)
    lay = rt.ROW_MAJOR if layout == "row" else rt.TILE_PACKED
    st = rt.lib().wave_gemm_streamk_noalloc_launch(a.data_ptr(), a.data_ptr(), a.data_ptr(),
                                                   M, N, 64, rt.F16, rt.F16, lay, workers,
                                                   None)
    assert st == getattr(rt, "ERR_" + status)
    assert text in rt.lib().wave_last_error()


def test_noalloc_replays_in_a_hip_graph(w, dev):
    """A noalloc launch captured into a HIP graph (the callers it exists for)
    replays correctly: the first call on the device is made eagerly (it
    resolves the static array's address), then a capture of the counter
    reset and the Stream-K kernel is replayed three times, with eager work
    and a synchronisation between replays, each checked bit for bit against
    wave_gemm_streamk_launch with a caller-owned workspace."""
    g = torch.Generator(device="cpu").manual_seed(8)
    M, N, K, workers = 768, 512, 1024, 11
    a = (torch.rand((M, K), generator=g) * 2 - 1).to(torch.float16).to(dev)
    b = (torch.rand((N, K), generator=g) * 2 - 1).to(torch.float16).to(dev)
    ref = w.gemm_streamk(a, b, workers, out_dtype=torch.float32)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    assert noalloc(w, a, b, out, workers, "row") == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph.capture_begin()
        st = noalloc(w, a, b, out, workers, "row")
        graph.capture_end()
    assert st == 0, w.runtime.lib().wave_last_error()
    torch.cuda.current_stream().wait_stream(stream)
    for i in range(3):
        out.fill_(float("nan"))
        w.gemm_streamk(b, a, 3, out_dtype=torch.float16)  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i
