"""FlyActor.from_structure: an actor over a library structure (NET.bin's arrays) plays and learns as the actor whose
structure it is: the same buffers the export reads back, the same logits and gradients on every PyTorch path."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import CASES, lively, toy
from flyguy_amd.export import net_bytes, params_from_torch, read_net, structure
from flyguy_amd.fly import FlyActor


@pytest.mark.parametrize("name,hops,fan", CASES[:5])
def test_same_network_as_the_actor(name, hops, fan, monkeypatch):
    torch.manual_seed(0)
    f = lively(FlyActor(toy(name), 517, 90, hops=hops, fan=fan), 0)
    s = structure(f)
    P = params_from_torch(f, s)
    g = FlyActor.from_structure(read_net(net_bytes(s)), P)
    s2 = structure(g)
    assert net_bytes(s2)[: -4 * len(s["wmap"])] == net_bytes(s)[: -4 * len(s["wmap"])]     # (wmap: its own strengths)
    x = torch.randn(6, 517)
    R = torch.randn(6, 90)
    for limit in (60_000_000, 0):                      # gather path, sparse-product path
        f.gather_limit = g.gather_limit = limit
        outs = []
        for a in (f, g):
            a.zero_grad()
            out = a(x)
            (out * R).sum().backward()
            outs.append(out.detach())
        assert torch.allclose(outs[0], outs[1], atol=1e-6)
        wmap = torch.as_tensor(np.asarray(s["wmap"], np.int64))
        assert torch.allclose(f.w.grad[wmap], g.w.grad, atol=1e-6)
        for n in ("gain", "theta", "in_w", "in_b"):
            assert torch.allclose(getattr(f, n).grad, getattr(g, n).grad, atol=1e-6), n
    monkeypatch.setenv("FLYGUY_NATIVE", "0")           # playing on the CPU through sparse CSR products
    with torch.no_grad():
        assert torch.allclose(f(x), g(x), atol=1e-6)
