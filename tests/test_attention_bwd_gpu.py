"""GPU parity of the flash-attention backward (wave_fa_bwd_launch) and of
the forward's lse output (wave_fa_fwd_lse_launch) against the float64
oracle (oracle.fa_backward, itself checked against torch autograd in
tests/test_oracle_fa_bwd.py).

Inputs: N(0, 1) Q, K, V, dO rounded to f16 / bf16; the oracle runs on the
rounded values and on the kernel's own O (16-bit), as the kernels do.
Tolerance, per gradient: max |got - ref| <= TOL * max |ref| + 1e-3, with
TOL = 2e-2 (f16) and 4e-2 (bf16: P and dS are rounded to 8-bit mantissas
before the gradient products); lse within 1e-3 (f16) / 5e-3 (bf16).  The
reference has no backward.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TDT = {1: torch.float16, 2: torch.bfloat16}
TOL = {1: 2e-2, 2: 4e-2}
# lse = m + ln(sum of the 16-bit P values the forward multiplies V with):
# the bf16 rounding of P (relative 2^-9) bounds its error near 2e-3.
TOL_LSE = {1: 1e-3, 2: 5e-3}


def run_bwd(wave, oracle, dev, dt, B, Hq, Hkv, S, causal, seed=1, scale=None):
    D = 128
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn(shape, generator=g).to(TDT[dt])
                   for shape in ((B, Hq, S, D), (B, Hkv, S, D), (B, Hkv, S, D), (B, Hq, S, D)))
    qd, kd, vd, dod = (t.to(dev) for t in (q, k, v, do))
    o, lse = wave.flash_attention_lse(qd, kd, vd, causal=causal, scale=scale)
    dq, dk, dv = wave.flash_attention_bwd(qd, kd, vd, o, dod, lse, causal=causal, scale=scale)
    torch.cuda.synchronize()
    f64 = lambda t: t.float().cpu().numpy().astype(np.float64)
    # The kernels take delta = rowsum(dO o O) from their own 16-bit O.
    ref = oracle.fa_backward(f64(q), f64(k), f64(v), f64(do), scale=scale, causal=causal,
                             o_delta=f64(o))
    return (f64(o), lse.cpu().numpy(), f64(dq), f64(dk), f64(dv)), ref


def check(got, ref, dt):
    names = ("o", "lse", "dq", "dk", "dv")
    for name, x, y in zip(names, got, ref):
        err = float(np.max(np.abs(x - y)))
        bound = TOL_LSE[dt] if name == "lse" else TOL[dt] * float(np.max(np.abs(y))) + 1e-3
        assert err <= bound, f"{name}: max abs err {err:.4g} > {bound:.4g}"


@pytest.mark.parametrize("dt", [1, 2])
@pytest.mark.parametrize("causal", [False, True])
# S % 128 == 0 runs the two-group dK/dV kernel (several 128-key blocks, GQA
# and causal at 384), the other lengths the 64-key one.
@pytest.mark.parametrize("B,Hq,Hkv,S", [(1, 2, 2, 64), (1, 2, 2, 256), (2, 4, 2, 192),
                                         (1, 4, 1, 320), (2, 4, 2, 384)])
def test_fa_bwd_parity(wave, oracle, dev, dt, causal, B, Hq, Hkv, S):
    got, ref = run_bwd(wave, oracle, dev, dt, B, Hq, Hkv, S, causal)
    check(got, ref, dt)


# Relative bound at the benchmarked shape, max |got - ref| / max |ref| per
# gradient.  f16: P and dS carry 11-bit mantissas into the gradient products,
# so the error is a few 2^-11 relative; bf16 (8-bit mantissas) about 8x that.
TOL_FULL = {1: 5e-3, 2: 2e-2}


@pytest.mark.parametrize("dt", [1, 2])
def test_fa_bwd_benchmark_shape(wave, oracle, dev, dt):
    """The backward at the shape bench.py reports (B4 H32 S4096 D128,
    non-causal): the whole problem on the GPU, three (batch, head) pairs
    against the float64 oracle (each head's gradients depend on that head
    alone), at TOL_FULL relative to each gradient's largest magnitude."""
    B, H, S, D = 4, 32, 4096, 128
    g = torch.Generator().manual_seed(23)
    q, k, v, do = (torch.randn((B, H, S, D), generator=g).to(TDT[dt]) for _ in range(4))
    qd, kd, vd, dod = (t.to(dev) for t in (q, k, v, do))
    o, lse = wave.flash_attention_lse(qd, kd, vd)
    dq, dk, dv = wave.flash_attention_bwd(qd, kd, vd, o, dod, lse)
    torch.cuda.synchronize()
    f64 = lambda t: t.float().cpu().numpy().astype(np.float64)
    worst = {}
    for b, h in ((0, 0), (1, 13), (3, 31)):
        one = lambda t: f64(t[b:b + 1, h:h + 1])
        ref = oracle.fa_backward(one(q), one(k), one(v), one(do), o_delta=one(o))
        got = (one(o), lse[b:b + 1, h:h + 1].cpu().numpy(), one(dq), one(dk), one(dv))
        for name, x, y in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
            err = float(np.max(np.abs(x - y)))
            rel = err if name == "lse" else err / float(np.max(np.abs(y)))
            worst[name] = max(worst.get(name, 0.0), rel)
    msg = ", ".join(f"{n} {r:.3g}" for n, r in worst.items())
    assert worst["lse"] <= TOL_LSE[dt], msg
    for name in ("o", "dq", "dk", "dv"):
        assert worst[name] <= TOL_FULL[dt], f"{name}: {msg}"


def test_fa_bwd_explicit_scale(wave, oracle, dev):
    got, ref = run_bwd(wave, oracle, dev, 1, 1, 2, 1, 128, True, seed=4, scale=0.05)
    check(got, ref, 1)


def test_fa_bwd_deterministic(wave, oracle, dev):
    # No atomics: two runs give bit-identical gradients.
    g = torch.Generator().manual_seed(9)
    q, k, v, do = (torch.randn((1, 4, 256, 128), generator=g).to(torch.bfloat16).to(dev)
                   for _ in range(4))
    k, v = k[:, :2].contiguous(), v[:, :2].contiguous()
    o, lse = wave.flash_attention_lse(q, k, v, causal=True)
    a = wave.flash_attention_bwd(q, k, v, o, do, lse, causal=True)
    b = wave.flash_attention_bwd(q, k, v, o, do, lse, causal=True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_fa_lse_matches_forward_output(wave, dev):
    # flash_attention_lse's O is the plain forward's O, bit for bit.
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn((1, 2, 320, 128), generator=g).to(torch.float16).to(dev)
               for _ in range(3))
    o1 = wave.flash_attention(q, k, v, causal=True)
    o2, _ = wave.flash_attention_lse(q, k, v, causal=True)
    assert torch.equal(o1, o2)


def test_fa_bwd_rejects_ragged_seq(wave, dev):
    # WAVE_ERR_UNSUPPORTED, raised before any launch.
    t = torch.zeros((1, 1, 100, 128), dtype=torch.float16, device=dev)
    lse = torch.zeros((1, 1, 100), dtype=torch.float32, device=dev)
    with pytest.raises(NotImplementedError, match="multiple of 64"):
        wave.flash_attention_bwd(t, t, t, t, t, lse)
