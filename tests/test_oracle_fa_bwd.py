"""The flash-attention backward oracle (oracle.fa_backward) against torch
autograd in float64: an independent implementation of the same gradients.
The reference has no backward, so this is what pins the oracle."""
import numpy as np
import pytest
import torch

from oracle import oracle


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("hq,hkv", [(2, 2), (4, 2), (4, 1)])
def test_fa_backward_matches_autograd(causal, hq, hkv):
    rng = np.random.default_rng(3 + hq + 7 * hkv + int(causal))
    B, S, D = 2, 48, 32
    q = rng.standard_normal((B, hq, S, D))
    k = rng.standard_normal((B, hkv, S, D))
    v = rng.standard_normal((B, hkv, S, D))
    do = rng.standard_normal((B, hq, S, D))
    scale = 0.3
    o, lse, dq, dk, dv = oracle.fa_backward(q, k, v, do, scale=scale, causal=causal)

    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    g = hq // hkv
    kk = tk.repeat_interleave(g, dim=1)
    vv = tv.repeat_interleave(g, dim=1)
    s = scale * tq @ kk.transpose(-1, -2)
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    to = torch.softmax(s, dim=-1) @ vv
    to.backward(torch.tensor(do))
    np.testing.assert_allclose(o, to.detach().numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(lse, torch.logsumexp(s, dim=-1).detach().numpy(), rtol=1e-12)
    np.testing.assert_allclose(dq, tq.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dk, tk.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dv, tv.grad.numpy(), rtol=1e-9, atol=1e-11)


def test_fa_backward_uniform_attention_closed_form():
    # Q = 0: every row attends uniformly, so dV[k] = sum_q dO[q] / S for each
    # key k (non-causal) and dQ, dK follow from dS = (dP - delta) / S.
    rng = np.random.default_rng(5)
    B, H, S, D = 1, 1, 16, 8
    q = np.zeros((B, H, S, D))
    k = rng.standard_normal((B, H, S, D))
    v = rng.standard_normal((B, H, S, D))
    do = rng.standard_normal((B, H, S, D))
    o, lse, dq, dk, dv = oracle.fa_backward(q, k, v, do)
    np.testing.assert_allclose(lse, np.full((B, H, S), np.log(S)), rtol=1e-14)
    np.testing.assert_allclose(o[0, 0], np.tile(v[0, 0].mean(axis=0), (S, 1)), rtol=1e-12)
    np.testing.assert_allclose(dv[0, 0], np.tile(do[0, 0].sum(axis=0) / S, (S, 1)), rtol=1e-12)
    # dK = scale * dS^T Q = 0 when Q = 0.
    np.testing.assert_array_equal(dk, np.zeros_like(dk))
