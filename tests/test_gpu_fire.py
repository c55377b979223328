"""FireHip (fh_fire / fh_fire_bwd), the neuron activation relu(g z - t) of FlyActor's GPU path in one pass: its
output and state gradient bit for bit against PyTorch's elementwise operations on the same device, the per-row
gradients of g and t against float64, and the whole actor's gradients through the library's products and FireHip
against the PyTorch path in float64."""
from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from conftest import lively, toy
from flyguy_amd.fly import FlyActor
from gpu_helpers import rel, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,B", [(1, 4), (37, 32), (300, 96), (2000, 4096)])
def test_fire_matches_pytorch(gpu_lib, rows, B):
    from flyguy_amd.fly_hip import FireHip
    say(f"fire {rows} x {B}")
    gen = torch.Generator().manual_seed(rows + B)
    z = (torch.randn(rows, B, generator=gen) * 3).cuda()
    z[0, 0] = float("nan")                                  # relu passes a NaN on; its gradient is 0
    if rows > 1:
        z[1, :] = 0.0                                       # a row at the threshold's edge (t = 0 below)
    g = (torch.rand(rows, generator=gen) * 2).cuda()
    g[-1] = 0.0                                             # a neuron of gain 0: g z - t = -t
    t = torch.nn.functional.softplus(torch.randn(rows, generator=gen) * 2).cuda()
    if rows > 1:
        t[1] = 0.0
    zf, gf, tf = z.clone().requires_grad_(True), g.clone().requires_grad_(True), t.clone().requires_grad_(True)
    got = FireHip.apply(zf, gf, tf)
    zr, gr, tr = z.clone().requires_grad_(True), g.clone().requires_grad_(True), t.clone().requires_grad_(True)
    want = torch.relu(gr[:, None] * zr - tr[:, None])
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    assert torch.equal(torch.nan_to_num(got), torch.nan_to_num(want))
    gh = torch.randn(rows, B, generator=gen).cuda()
    got.backward(gh)
    want.backward(gh)
    assert torch.equal(zf.grad, zr.grad)                    # gh g where g z - t is not <= 0: the same products
    for a, b in ((gf.grad, gr.grad), (tf.grad, tr.grad)):   # the same sums over the samples, in another order
        assert torch.equal(torch.isnan(a), torch.isnan(b))
        fin = ~torch.isnan(b)
        assert rel(a[fin].double().cpu().numpy(), b[fin].double().cpu().numpy()) <= 1e-5


@pytest.mark.parametrize("hops", [3, 1, 5])
def test_actor_gradients_through_the_library(gpu_lib, hops):
    """FlyActor with kernel "hip" (HopHip products, FireHip activations): logits and every parameter's gradient
    against the PyTorch path in float64 (fly.py:286-305), on toy networks of one, three and five hops (the deeper two
    with re-driven rows; at one hop the toy network has none)."""
    say(f"actor gradients through HopHip and FireHip, {hops} hops")
    torch.manual_seed(2)
    f = lively(FlyActor(toy("b"), 517, 90, hops=hops, fan=16))
    assert hops == 1 or any(len(getattr(f, f"s{k}")) for k in range(1, hops + 1))    # re-driven sensory rows
    x = torch.randn(96, 517)
    R = torch.randn(96, 90)
    g = copy.deepcopy(f).cuda()
    g.kernel = "hip"
    out = g(x.cuda())
    (out * R.cuda()).sum().backward()
    ref = copy.deepcopy(f).double()
    ref.kernel = "torch"
    ref_out = ref(x.double())
    (ref_out * R.double()).sum().backward()
    assert rel(out.detach().cpu().numpy(), ref_out.detach().numpy()) <= 1e-5
    for (name, p), (_, q) in zip(g.named_parameters(), ref.named_parameters()):
        assert p.grad is not None, name
        assert rel(p.grad.double().cpu().numpy(), q.grad.numpy()) <= 1e-4, name
