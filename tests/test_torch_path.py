"""The fly actor's PyTorch paths on the CPU (row a21; flyguy/fly.py:51-72, 286-305), against the dense "blind"
computation over every neuron and connection (tests/test_fly.py:29-41), as the reference's own test does
(tests/test_fly.py:44-74):
  * the gather path (small batch x connection counts) gives the blind outputs (1e-4, float32 against float64);
  * the sparse-product path (torch.sparse.mm forward, sampled_addmm / CSC products backward) gives the gather path's
    outputs (1e-5) and gradients (1e-6 absolute, 1e-4 relative);
  * both paths' gradients match float64 autograd of the blind model (1e-4 of the largest entry), and only strengths
    in play learn.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import CASES, toy
from test_oracle import actor, blind, blind_params, rel

NAMES = ("w", "gain", "theta", "in_w", "in_b", "out.weight", "out.bias")
BLIND = {"w": "w", "gain": "gain", "theta": "theta", "in_w": "in_w", "in_b": "in_b", "out.weight": "out_w",
         "out.bias": "out_b"}


def _grads(f, obs, R):
    f.zero_grad()
    out = f(obs)
    ((out * R).sum() + 0.1 * out.pow(2).sum()).backward()
    return out.detach(), {k: p.grad.detach().clone() for k, p in f.named_parameters()}


@pytest.mark.parametrize("name,hops,fan", CASES)
def test_gather_and_sparse_paths_match_blind(name, hops, fan):
    f = actor(name, hops, fan)
    f.kernel = "torch"
    obs = torch.as_tensor(np.random.default_rng(3).standard_normal((6, 517)).astype(np.float32))
    R = torch.as_tensor(np.random.default_rng(4).standard_normal((6, 90)).astype(np.float32))
    P = blind_params(f)
    ref = blind(f, toy(name), obs.double(), P)
    ((ref * R.double()).sum() + 0.1 * ref.pow(2).sum()).backward()
    out_g, g_gather = _grads(f, obs, R)
    assert out_g.shape == (6, 90) and torch.isfinite(out_g).all()
    assert rel(out_g, ref.detach()) < 1e-4
    f.gather_limit = 0                                          # the sparse-product path
    out_s, g_sparse = _grads(f, obs, R)
    assert torch.allclose(out_g, out_s, atol=1e-5)
    for k in NAMES:
        assert torch.allclose(g_gather[k], g_sparse[k], atol=1e-6, rtol=1e-4), k
        want = P[BLIND[k]].grad.numpy()
        assert rel(g_gather[k].numpy(), want) < 1e-4, k
    assert int((g_gather["w"] != 0).sum()) <= f.in_play        # only strengths in play learn
    assert float(np.abs(P["w"].grad.numpy()).max()) > 0
