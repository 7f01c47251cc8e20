"""GPU parity of the block-scaled FP8 flash-attention forward
(wave_fa_fwd_mxfp8_launch) against the oracle's float64 attention of the
decoded MX-FP8 inputs (oracle.mxfp8_decode + oracle.attention_forward).

No reference counterpart: the reference names a block-scaled FP8 attention
contract as its next FA step (docs/PerfReferences/WaveGfx950FlashAttention.md:
94-99), so the oracle is the math of the decoded values.  The kernel rounds
the probabilities to e4m3 before the PV product and the row sums (relative
error at most 2^-4 each, as 2^4 times the probability after the running max;
O = sum P~ V / sum P~ then lies within 2 * 2^-4 relative of the exact
weights to first order), so:
  * zero Q: every probability is exactly 2^4 in e4m3, and O is the mean of
    the decoded V rows (the unmasked ones): pinned to fp32-accumulation level
    beyond the output rounding.  This pins the V path (transpose, key order,
    V scales, lane-half swap, normalisation);
  * V rows one-hot (V[k] = e_k): O[q][k] is the probability of key k, within
    2 * 2^-4 of it relative.  This pins the QK path (Q, K and their scales);
  * general inputs: |O - O_ref| <= 2 * 2^-4 max|V| + output rounding, a bound
    the P rounding cannot exceed, and the mean error below 2e-3 max|V|; lse
    within ln(1 + 2^-4) (the row sums are of the rounded P), mean 5e-3.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ODT = {1: torch.float16, 2: torch.bfloat16}
REL = {1: 2.0 ** -11, 2: 2.0 ** -8}   # output rounding (half an ulp)


def quantized(wave, x, dim=-1):
    e, s = wave.mxfp8_quantize(x, dim=dim)
    return e, s


def decode(oracle, e, s, axis):
    return oracle.mxfp8_decode(e.cpu().numpy(), s.cpu().numpy(), axis=axis)


def run(wave, q, k, v, *, causal, out_dt, lse=False, scale=None):
    (qe, qs), (ke, ks), (ve, vs) = (quantized(wave, q), quantized(wave, k),
                                    quantized(wave, v, dim=2))
    dev = torch.device("cuda:0")
    l = torch.empty(q.shape[:3], dtype=torch.float32, device=dev) if lse else None
    o = wave.flash_attention_mxfp8(qe.to(dev), qs.to(dev), ke.to(dev), ks.to(dev),
                                   ve.to(dev), vs.to(dev), causal=causal, scale=scale,
                                   out_dtype=ODT[out_dt], lse=l)
    torch.cuda.synchronize()
    return (qe, qs, ke, ks, ve, vs), o.float().cpu().numpy(), (l.cpu().numpy() if lse else None)


@pytest.mark.parametrize("out_dt", [1, 2])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,Hq,Hkv,S", [(1, 2, 1, 256), (2, 4, 2, 320), (1, 1, 1, 1000)])
def test_zero_q_gives_the_mean_of_v(wave, oracle, dev, out_dt, causal, B, Hq, Hkv, S):
    g = torch.Generator().manual_seed(11)
    q = torch.zeros(B, Hq, S, 128)
    k = torch.randn(B, Hkv, S, 128, generator=g)
    v = torch.randn(B, Hkv, S, 128, generator=g) * torch.exp2(
        torch.randint(-6, 6, (B, Hkv, S, 1), generator=g).float())
    (_, _, _, _, ve, vs), o, _ = run(wave, q, k, v, causal=causal, out_dt=out_dt)
    vd = decode(oracle, ve, vs, axis=2)
    vv = np.repeat(vd, Hq // Hkv, axis=1)
    if causal:
        ref = np.cumsum(vv, axis=2) / np.arange(1, S + 1)[:, None]
    else:
        ref = np.broadcast_to(vv.mean(axis=2, keepdims=True), vv.shape)
    err = np.abs(o - ref)
    assert np.all(err <= REL[out_dt] * np.abs(ref) + 1e-5 * np.abs(vd).max()), err.max()


@pytest.mark.parametrize("causal", [False, True])
def test_one_hot_v_shows_the_probabilities(wave, oracle, dev, causal):
    B, Hq, Hkv, S = 1, 2, 2, 128
    g = torch.Generator().manual_seed(13)
    q = torch.randn(B, Hq, S, 128, generator=g) * torch.exp2(
        torch.randint(-3, 3, (B, Hq, S, 4), generator=g).float()).repeat_interleave(32, -1)
    k = torch.randn(B, Hkv, S, 128, generator=g) * torch.exp2(
        torch.randint(-3, 3, (B, Hkv, S, 4), generator=g).float()).repeat_interleave(32, -1)
    v = torch.eye(S, 128).expand(B, Hkv, S, 128).contiguous()
    (qe, qs, ke, ks, ve, vs), o, _ = run(wave, q, k, v, causal=causal, out_dt=1)
    qd, kd = decode(oracle, qe, qs, 3), decode(oracle, ke, ks, 3)
    vd = decode(oracle, ve, vs, 2)
    assert np.array_equal(vd, v.numpy())
    ref, _ = oracle.attention_forward(qd, kd, vd, causal=causal)
    # O[q][k] = P[q][k]: e4m3 rounding of 2^4 P in the numerator and in the
    # row sum (relative 2^-4 each, plus the smallest subnormal step 2^-13 of
    # the row max) and f16 output rounding.
    tol = 2 * 2.0 ** -4 * ref + 2.0 ** -13 + REL[1] * ref
    assert np.all(np.abs(o - ref) <= tol), np.abs(o - ref).max()


@pytest.mark.parametrize("out_dt", [1, 2])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,Hq,Hkv,S", [(1, 2, 1, 256), (2, 4, 2, 320), (1, 2, 2, 1000),
                                        (1, 8, 1, 64)])
def test_random_inputs_against_decoded_float64(wave, oracle, dev, out_dt, causal, B, Hq, Hkv, S):
    g = torch.Generator().manual_seed(17 + S)
    q = torch.randn(B, Hq, S, 128, generator=g)
    k = torch.randn(B, Hkv, S, 128, generator=g)
    v = torch.randn(B, Hkv, S, 128, generator=g)
    (qe, qs, ke, ks, ve, vs), o, lse = run(wave, q, k, v, causal=causal, out_dt=out_dt,
                                           lse=True)
    qd, kd, vd = decode(oracle, qe, qs, 3), decode(oracle, ke, ks, 3), decode(oracle, ve, vs, 2)
    ref, ref_lse = oracle.attention_forward(qd, kd, vd, causal=causal)
    vmax = np.abs(vd).max()
    err = np.abs(o - ref)
    assert err.max() <= 2 * 2.0 ** -4 * vmax + REL[out_dt] * np.abs(ref).max(), err.max()
    assert err.mean() <= 2e-3 * vmax, err.mean()
    dl = np.abs(lse - ref_lse)
    # Unbiased rounding of each term (std 2^-4 / sqrt 3 relative) over a row
    # of >= 50 effective terms: a mean of at most about 5e-3.
    assert dl.max() <= np.log1p(2.0 ** -4) and dl.mean() <= 5e-3, (dl.max(), dl.mean())


def test_benchmark_shape_sampled_rows(wave, oracle, dev):
    """B4 H32 S4096 (the f16 benchmark shape) on device-quantized inputs:
    three heads, seven rows each, against the decoded float64 attention."""
    B, H, S = 4, 32, 4096
    g = torch.Generator(device=dev).manual_seed(23)
    q = torch.randn(B, H, S, 128, generator=g, device=dev)
    k = torch.randn(B, H, S, 128, generator=g, device=dev)
    v = torch.randn(B, H, S, 128, generator=g, device=dev)
    (qe, qs), (ke, ks), (ve, vs) = (wave.mxfp8_quantize(q), wave.mxfp8_quantize(k),
                                    wave.mxfp8_quantize(v, dim=2))
    o = wave.flash_attention_mxfp8(qe, qs, ke, ks, ve, vs, out_dtype=torch.float16)
    torch.cuda.synchronize()
    rows = [0, 31, 32, 255, 2048, 4032, 4095]
    for bh in (0, 2 * H + 17, B * H - 1):
        b, h = divmod(bh, H)
        qd = decode(oracle, qe[b, h, rows], qs[b, h, rows], 1)
        kd = decode(oracle, ke[b, h], ks[b, h], 1)
        vd = decode(oracle, ve[b, h], vs[b, h], 0)
        s = qd @ kd.T / np.sqrt(128)
        p = np.exp(s - s.max(-1, keepdims=True))
        ref = (p / p.sum(-1, keepdims=True)) @ vd
        err = np.abs(o[b, h, rows].float().cpu().numpy() - ref)
        assert err.max() <= 2 * 2.0 ** -4 * np.abs(vd).max(), err.max()
        assert err.mean() <= 2e-3 * np.abs(vd).max(), err.mean()


def test_rejections(wave, dev):
    q = torch.zeros(1, 2, 64, 128, dtype=torch.uint8, device=dev)
    s = torch.full((1, 2, 64, 4), 127, dtype=torch.uint8, device=dev)
    vs = torch.full((1, 2, 2, 128), 127, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        wave.flash_attention_mxfp8(q, s, q, s, q, s)          # v_scale shape
    with pytest.raises(ValueError):
        wave.flash_attention_mxfp8(q.float(), s, q, s, q, vs)  # element dtype
    kq = torch.zeros(1, 3, 64, 128, dtype=torch.uint8, device=dev)
    ks = torch.full((1, 3, 64, 4), 127, dtype=torch.uint8, device=dev)
    kvs = torch.full((1, 3, 2, 128), 127, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError, match="multiple"):          # 2 q heads on 3 kv heads
        wave.flash_attention_mxfp8(q, s, kq, ks, kq, kvs)
