"""Argument checks of the tensor front end (7_amd/ops.py): every request that
would make a kernel read or write past a buffer through its bare pointers
raises ValueError before anything is launched, and the tensors stay
untouched."""

import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def w():
    m = importlib.import_module("7_amd")
    m.runtime.lib()
    return m


def f16(*shape, dev="cuda:0"):
    return torch.zeros(shape, dtype=torch.float16, device=dev)


def test_gemm_out_checked(w, dev):
    a, b = f16(64, 32), f16(48, 32)
    for out in (f16(48, 64), torch.zeros((64, 48), dtype=torch.float32, device=dev),
                f16(64, 96)[:, ::2]):
        with pytest.raises(ValueError):
            w.gemm(a, b, out_dtype="f16", out=out)


def test_gemm_streamk_workspace_and_out_checked(w, dev):
    a, b = f16(512, 128), f16(256, 128)
    small = w.StreamKWorkspace(256, 256, 4, dev)   # made for another M
    few = w.StreamKWorkspace(512, 256, 2, dev)     # fewer workers
    sentinel = small.counters.clone()
    with pytest.raises(ValueError):
        w.gemm_streamk(a, b, 4, workspace=small)
    with pytest.raises(ValueError):
        w.gemm_streamk(a, b, 4, workspace=few)
    with pytest.raises(ValueError):
        w.gemm_streamk(a, b, 2, workspace=few, out=f16(256, 512))  # wrong shape
    with pytest.raises(ValueError):
        w.gemm_streamk(a, b, 2, workspace=few,
                       out=torch.zeros((512, 256), dtype=torch.float32, device=dev))
    torch.cuda.synchronize()
    assert torch.equal(small.counters, sentinel)
    # the matching workspace and out are accepted
    out = w.gemm_streamk(a, b, 2, workspace=few, out=f16(512, 256))
    torch.cuda.synchronize()
    assert bool((out == 0).all()) and few.nonzero_counters() == 0


def test_flash_attention_out_checked(w, dev):
    q = torch.zeros((1, 2, 64, 128), dtype=torch.bfloat16, device=dev)
    for out in (torch.zeros((1, 2, 32, 128), dtype=torch.bfloat16, device=dev),
                torch.zeros((1, 2, 64, 128), dtype=torch.float16, device=dev)):
        with pytest.raises(ValueError):
            w.flash_attention(q, q, q, out=out)


def test_flash_attention_f32_shapes_checked(w, dev):
    q = f16(16, 64)
    k = f16(256, 64)
    for kk, vv in ((f16(256, 32), f16(256, 32)),   # head_dim differs from q
                   (k, f16(128, 64)),               # v shorter than k
                   (k, f16(256, 32))):
        with pytest.raises(ValueError):
            w.flash_attention_f32(q, kk, vv)
    for out in (torch.zeros((16, 32), dtype=torch.float32, device=dev),
                torch.zeros((16, 64), dtype=torch.float16, device=dev),
                torch.zeros((64, 16), dtype=torch.float32, device=dev).t()):
        with pytest.raises(ValueError):
            w.flash_attention_f32(q, k, k, out=out)
