"""The oracle is pinned before it is trusted (CPU only).

  forward   against the dense "blind" computation over every neuron and connection of the reference's own test
            (tests/test_fly.py:29-41), in float64, and against the reference's compiled CPU forward
            (flyguy/native/fly_infer.cpp, built into oracle/_ref/ from the reference checkout);
  backward  against float64 autograd of the blind computation, and against central finite differences;
  loss      against torch.log_softmax (the form export.py:135-136 uses);
  Adam      against torch.optim.Adam(eps=1e-8) and the running-average recurrence.
A planted mistake (a dropped re-drive term in a copy of the dense model) must be caught by the same comparison.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import CASES, lively, toy
from flyguy_amd.export import net_bytes, params_from_torch, structure
from flyguy_amd.fly import FlyActor
from flyguy_amd.synth import scaled_3hop
from oracle import refinfer
from oracle.oracle import Oracle


def rel(a, b) -> float:
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)) if b.size else 0.0


def actor(name, hops, fan, seed=0):
    torch.manual_seed(seed)
    return lively(FlyActor(toy(name), 517, 90, hops=hops, fan=fan), seed)


def blind_params(f):
    P = {"w": f.w, "gain": f.gain, "theta": f.theta, "in_w": f.in_w, "in_b": f.in_b, "out_w": f.out.weight,
         "out_b": f.out.bias}
    return {k: v.detach().double().clone().requires_grad_(True) for k, v in P.items()}


def blind(f, g, obs, P, redrive=True):
    """Every neuron, every connection, every hop (tests/test_fly.py:29-41), differentiable, float64."""
    n = f.n_neurons
    pre, post = torch.as_tensor(g["pre"]).long(), torch.as_tensor(g["post"]).long()
    W = torch.zeros(n, n, dtype=torch.float64).index_put((post, pre), P["w"])
    drive_in = torch.zeros(obs.shape[0], f.sizes[0], dtype=torch.float64).index_add(
        1, f.in_r, obs[:, f.in_c] * P["in_w"]) + P["in_b"]
    drive = torch.zeros(obs.shape[0], n, dtype=torch.float64).index_copy(1, f.n0, drive_in)
    thr = torch.nn.functional.softplus(P["theta"])
    h = torch.relu(P["gain"] * drive - thr)
    for _ in range(f.hops):
        h = torch.relu(P["gain"] * (h @ W.t() + (drive if redrive else 0)) - thr)
    dn_ids = getattr(f, f"n{f.hops}")[f.dn_rows]
    return h[:, dn_ids] @ P["out_w"].t() + P["out_b"]


def setup(name, hops, fan, B=6, seed=0):
    f = actor(name, hops, fan, seed)
    s = structure(f)
    params = params_from_torch(f, s)
    rng = np.random.default_rng(seed)
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    return f, s, params, obs


@pytest.mark.parametrize("name,hops,fan", CASES)
def test_forward_matches_blind(name, hops, fan):
    f, s, params, obs = setup(name, hops, fan)
    ref = blind(f, toy(name), torch.as_tensor(obs).double(), blind_params(f)).detach().numpy()
    o64 = Oracle(net_bytes(s), params, "f64").forward(obs)
    o32 = Oracle(net_bytes(s), params, "f32").forward(obs)
    assert np.abs(ref).max() > 0.05                        # lively enough to mean something
    assert rel(o64, ref) < 1e-6                           # (logits are rounded to float32 on output)
    assert rel(o32, ref) < 1e-5


def test_planted_mistake_is_caught():
    """A dense model without the sensory re-drive differs from the oracle by far more than the tolerance."""
    f, s, params, obs = setup("b", 3, 16)
    wrong = blind(f, toy("b"), torch.as_tensor(obs).double(), blind_params(f), redrive=False).detach().numpy()
    assert rel(Oracle(net_bytes(s), params, "f64").forward(obs), wrong) > 1e-3


@pytest.mark.parametrize("name,hops,fan", CASES)
def test_backward_matches_blind_autograd(name, hops, fan):
    f, s, params, obs = setup(name, hops, fan)
    P = blind_params(f)
    out = blind(f, toy(name), torch.as_tensor(obs).double(), P)
    R = torch.as_tensor(np.random.default_rng(1).standard_normal(out.shape))
    ((out * R).sum() + 0.1 * out.pow(2).sum()).backward()
    dl = (R + 0.2 * out.detach()).numpy().astype(np.float32)
    o = Oracle(net_bytes(s), params, "f64")
    o.forward(obs)
    got = o.backward(dl)
    wmap = s["wmap"]
    want = [P["w"].grad.numpy()[wmap], P["gain"].grad.numpy(), P["theta"].grad.numpy(), P["in_w"].grad.numpy(),
            P["in_b"].grad.numpy(), P["out_w"].grad.numpy().reshape(-1), P["out_b"].grad.numpy()]
    out_of_play = np.ones(f.n_conn, bool)
    out_of_play[wmap] = False
    assert np.abs(P["w"].grad.numpy()[out_of_play]).max(initial=0) == 0      # only strengths in play learn
    for name_, g, w in zip(("W", "gain", "theta", "in_w", "in_b", "out_w", "out_b"), got, want):
        assert rel(g, w) < 1e-5, name_                     # dl was rounded to float32
    assert np.abs(want[0]).max() > 0


def test_backward_matches_finite_differences():
    f, s, params, obs = setup("a", 3, 5, B=4)
    net = net_bytes(s)
    rng = np.random.default_rng(3)
    R = rng.standard_normal((4, 90))

    def loss(ps):
        lg = Oracle(net, ps, "f64").forward(obs).astype(np.float64)
        return float((lg * R).sum())

    o = Oracle(net, params, "f64")
    o.forward(obs)
    grads = o.backward(R.astype(np.float32))
    for arr in range(7):
        g = grads[arr]
        for i in rng.choice(len(g), min(4, len(g)), replace=False):
            if abs(g[i]) < 1e-3:
                continue
            eps = 1e-2 * max(1.0, abs(float(params[arr][i])))
            up = [p.copy() for p in params]
            dn = [p.copy() for p in params]
            up[arr][i] += eps
            dn[arr][i] -= eps
            fd = (loss(up) - loss(dn)) / (2 * eps)
            assert abs(fd - g[i]) <= 2e-2 * abs(g[i]) + 1e-4, (arr, i, fd, g[i])


@pytest.mark.parametrize("name,hops,fan", [("a", 3, 5), ("b", 3, 16), ("c", 4, 6)])
def test_oracle_matches_reference_compiled_forward(name, hops, fan):
    if not refinfer.available():
        pytest.skip("oracle/_ref/libfly_infer.so not built (needs the reference checkout)")
    f, s, params, obs = setup(name, hops, fan)
    got = refinfer.RefInfer(s, params).forward(obs)
    assert rel(Oracle(net_bytes(s), params, "f64").forward(obs), got) < 1e-5


def test_oracle_matches_reference_compiled_forward_synthetic():
    if not refinfer.available():
        pytest.skip("oracle/_ref/libfly_infer.so not built (needs the reference checkout)")
    s, params = scaled_3hop(64)
    obs = np.random.default_rng(0).standard_normal((8, 517)).astype(np.float32)
    got = refinfer.RefInfer(s, params).forward(obs)
    want = Oracle(net_bytes(s), params, "f64").forward(obs)
    assert np.abs(want).max() > 0.01
    assert rel(want, got) < 1e-5


def test_loss_matches_log_softmax():
    rng = np.random.default_rng(0)
    lg = rng.standard_normal((64, 90)).astype(np.float32) * 3
    tl = rng.standard_normal((64, 90)).astype(np.float32) * 2
    lg[5, 7] = lg[5, 9] = 50.0                             # a tie: the first maximum wins
    tl[5, 7] = tl[5, 9] = 40.0
    for it in (1.0, 2.0):
        o = Oracle.__new__(Oracle)
        from oracle.oracle import _lib
        o.L = _lib("f64")
        dl, kl, agree = o.loss(lg, tl, it)
        lt, ls = torch.as_tensor(tl).double() * it, torch.as_tensor(lg).double()
        lpt, lps = torch.log_softmax(lt, -1), torch.log_softmax(ls, -1)
        want_kl = float((lpt.exp() * (lpt - lps)).sum())
        want_dl = ((lps.exp() - lpt.exp()) / 64).numpy()
        assert abs(kl - want_kl) < 1e-9 * max(1, abs(want_kl))
        assert rel(dl, want_dl) < 1e-6
        assert agree == float((ls.argmax(-1) == lt.argmax(-1)).sum())


def test_adam_matches_torch():
    rng = np.random.default_rng(0)
    n = 1000
    p0 = rng.standard_normal(n).astype(np.float32)
    p, m, v, ema = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32), p0.copy()
    tp = torch.nn.Parameter(torch.as_tensor(p0.copy()))
    opt = torch.optim.Adam([tp], lr=1e-3, betas=(0.9, 0.999), eps=1e-8)
    o = Oracle.__new__(Oracle)
    from oracle.oracle import _lib
    o.L = _lib("f32")
    ema_ref = p0.astype(np.float64)
    for t in range(1, 6):
        g = rng.standard_normal(n).astype(np.float32)
        o.adam(p, g, m, v, ema, 1e-3, t, 1.0, 0.99)
        tp.grad = torch.as_tensor(g.copy())
        opt.step()
        ema_ref = 0.99 * ema_ref + 0.01 * tp.detach().numpy().astype(np.float64)
        assert np.abs(p - tp.detach().numpy()).max() < 1e-6
        assert np.abs(ema - ema_ref).max() < 1e-5
