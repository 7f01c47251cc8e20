"""CPU checks of the MX-FP8 pieces: the oracle's e4m3 / e8m0 decoders and
float64 attention, and the product's quantizer (7_amd.ops.mxfp8_quantize).

The formats are OCP's (8-bit Floating Point Specification, E4M3; Microscaling
Formats v1.0, E8M0 over blocks of 32).  Pins: every e4m3 code against torch's
float8_e4m3fn conversion (an independent implementation); e8m0 against its
closed form; oracle.attention_forward against torch's float64 softmax
attention; the quantizer's scale rule and rounding against the decoder.
"""

import importlib

import numpy as np
import torch

from oracle import oracle

ops = importlib.import_module("7_amd.ops")


def test_e4m3_decoder_matches_torch_on_every_code():
    ours = oracle.e4m3_to_float(np.arange(256))
    theirs = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))
    ok = ~np.isnan(ours)
    assert np.array_equal(ours[ok], theirs[ok])
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6
    assert np.isnan(ours[0x7F]) and np.isnan(ours[0xFF])


def test_e8m0_closed_form():
    v = oracle.e8m0_to_float(np.array([0, 1, 126, 127, 128, 254, 255]))
    assert list(v[:6]) == [2.0 ** -127, 2.0 ** -126, 0.5, 1.0, 2.0, 2.0 ** 127]
    assert np.isnan(v[6])


def test_quantizer_scale_rule_rounding_and_saturation():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(6, 40, 96, generator=g, dtype=torch.float64) * torch.exp2(
        torch.randint(-20, 20, (6, 40, 1), generator=g).double())
    x[0, 0, :32] = 0.0                      # an all-zero block
    x[1, 1, :32] = 1.0
    x[1, 1, 5] = 480.0                      # amax 480: scale 2^0, saturates to 448
    for dim in (-1, 1):
        e, s = ops.mxfp8_quantize(x, dim=dim)
        assert e.dtype == torch.uint8 and s.dtype == torch.uint8
        xn = x.numpy()
        dec = oracle.mxfp8_decode(e.numpy(), s.numpy(), axis=dim % 3)
        # Scale rule: 2^(floor(log2 amax) - 8) per block of 32 along dim.
        xb = np.moveaxis(xn, dim, -1)
        nb = -(-xb.shape[-1] // 32)
        pad = np.zeros(xb.shape[:-1] + (nb * 32,))
        pad[..., :xb.shape[-1]] = xb
        amax = np.abs(pad.reshape(*xb.shape[:-1], nb, 32)).max(-1)
        want = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1))) - 8, -127)
        assert np.array_equal(np.moveaxis(s.numpy(), dim, -1).astype(int), want.astype(int) + 127)
        # Rounding: within half an e4m3 step of x / scale (saturated at 448).
        sc = oracle.mxfp8_decode(np.full(e.shape, 0x38, np.uint8), s.numpy(), axis=dim % 3)
        t = np.clip(xn / sc, -448, 448)
        step = np.exp2(np.floor(np.log2(np.maximum(np.abs(t), 2.0 ** -6))) - 3)
        assert np.all(np.abs(dec / sc - t) <= step / 2 * (1 + 1e-12))
    e, s = ops.mxfp8_quantize(x)
    assert int(s[0, 0, 0]) == 0 and int(e[0, 0, :32].sum()) == 0
    assert oracle.e4m3_to_float(e[1, 1, 5].numpy()) == 448.0 and int(s[1, 1, 0]) == 127


def test_attention_forward_matches_torch_float64():
    g = torch.Generator().manual_seed(5)
    B, Hq, Hkv, S, D = 2, 4, 2, 80, 128
    q = torch.randn(B, Hq, S, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, Hkv, S, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, Hkv, S, D, generator=g, dtype=torch.float64)
    for causal in (False, True):
        o, lse = oracle.attention_forward(q.numpy(), k.numpy(), v.numpy(), causal=causal)
        kk = k.repeat_interleave(Hq // Hkv, dim=1)
        vv = v.repeat_interleave(Hq // Hkv, dim=1)
        s = (q @ kk.transpose(-1, -2)) / D ** 0.5
        if causal:
            s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
        ref = torch.softmax(s, dim=-1) @ vv
        assert np.allclose(o, ref.numpy(), rtol=1e-12, atol=1e-12)
        assert np.allclose(lse, torch.logsumexp(s, dim=-1).numpy(), rtol=1e-12, atol=1e-12)
