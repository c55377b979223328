"""The library core with bfloat16 states (fc_create_ex(..., FC_STATES_BF16)) against its numpy restatement
(oracle/core16.py: float64 arithmetic, bfloat16 rounding where the library stores a state).

Bars:
  * the rounding (obs -> x) bit-exact against hand-worked ties and special values;
  * networks whose values and sums are all exact (integer states, weights +-1): logits, every layer's state and all
    seven gradients bit-exact; the same with strengths and plug weights off the bfloat16 grid (1 + 2^-9, a tie
    1 + 2^-8, 1 - 2^-10), which the products must round to +-1 first;
  * general networks: logits within 1e-3 and gradients within 1e-2 of the largest entry (a float32 sum and the
    float64 oracle may round a state to neighbouring bfloat16 values, 2^-8 apart), argmax identical where the top-2
    margin exceeds 1e-2;
  * batch independence: a sample's logits are bit-identical in a batch of 4096 and of 64.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import lively, toy
from flyguy_amd.export import params_from_torch, structure
from flyguy_amd.fly import FlyActor
from flyguy_amd.synth import scaled_3hop
from gpu_helpers import NAMES, Core, argmax_agrees, rel, say
from oracle.core16 import Core16, bf16

pytestmark = pytest.mark.gpu
BF16 = 1


def toy_net(name, hops, fan, seed=0):
    torch.manual_seed(seed)
    f = lively(FlyActor(toy(name), 517, 90, hops=hops, fan=fan), seed)
    s = structure(f)
    return s, params_from_torch(f, s)


def test_rounding(gpu_lib):
    s, params = toy_net("a", 2, 5)
    core = Core(s, params, max_batch=64, flags=BF16)
    one = 1.0
    vals = [one + 2 ** -8, one + 3 * 2 ** -8, one + 2 ** -8 + 2 ** -20, -(one + 2 ** -8), 0.0, -0.0, np.inf, -np.inf,
            3.4028235e38, 65504.0, 1.17549435e-38, -2.5, 1e-3, 123456.7]
    obs = np.random.default_rng(0).standard_normal((64, 517)).astype(np.float32)
    obs[0, :len(vals)] = vals
    obs[1, :3] = [np.nan, 1e-40, -1e-40]                       # a NaN and two subnormals
    core.forward(obs)
    x = core.state(0, 2, 517, 64)                               # the stored observations, widened
    want = bf16(obs.T)
    ok = np.ones_like(x, bool)
    ok[:3, 1] = False
    assert np.array_equal(x[ok].view(np.uint32), want.astype(np.float32)[ok].view(np.uint32))
    assert np.isnan(x[0, 1])
    for i in (1, 2):                                            # a subnormal is kept (rounded) or flushed to a signed 0
        assert x[i, 1] == want[i, 1] or (x[i, 1] == 0 and np.signbit(x[i, 1]) == np.signbit(obs[1, i])), x[i, 1]
    assert x[0, 0] == 1.0 and x[1, 0] == 1 + 2 ** -6 and x[2, 0] == 1 + 2 ** -7 and x[8, 0] == np.inf


def _exact_case(name, hops, fan, seed):
    """Integer states: weights in {-1, 0, 1} (mostly 0), gain 1, softplus(theta) = 0, obs in {-1, 0, 1}."""
    s, params = toy_net(name, hops, fan, seed)
    rng = np.random.default_rng(seed)
    P = [p.copy() for p in params]
    for i in (0, 3, 5):
        P[i] = (rng.choice([-1.0, 0.0, 0.0, 0.0, 1.0], P[i].size) * (rng.random(P[i].size) < 0.3)).astype(np.float32)
    P[1][:] = 1.0
    P[2][:] = -200.0                                            # softplus(-200) = 0 in float32
    P[4][:] = rng.choice([-1.0, 0.0, 1.0], P[4].size).astype(np.float32)
    P[6][:] = rng.choice([-1.0, 0.0, 1.0], P[6].size).astype(np.float32)
    obs = rng.choice([-1.0, 0.0, 1.0], (64, 517)).astype(np.float32)
    return s, P, obs


@pytest.mark.parametrize("name,hops,fan", [("a", 3, 5), ("b", 2, 8), ("c", 3, 16)])
def test_exact_forward_backward(gpu_lib, name, hops, fan):
    s, P, obs = _exact_case(name, hops, fan, 3)
    say(f"bf16 exact {name} hops {hops} fan {fan}")
    o = Core16(s, P)
    want = o.forward(obs)
    for layer, (h, _) in enumerate(o.states):                 # the case is exact: every state is an integer < 2^8
        assert np.array_equal(bf16(h), h) and np.abs(h).max() < 256, layer
    core = Core(s, P, max_batch=64, flags=BF16)
    got = core.forward(obs)
    assert np.array_equal(got, want.astype(np.float32))
    for layer, (h, _) in enumerate(o.states):
        assert np.array_equal(core.state(layer, 0, s["sizes"][layer], 64), h.astype(np.float32)), layer
    assert np.array_equal(core.state(0, 1, s["sizes"][0], 64), o.drive.astype(np.float32))
    rng = np.random.default_rng(9)
    dl = rng.choice([-1.0, 0.0, 1.0], got.shape).astype(np.float32)
    core.zero_grad()
    core.backward(dl)
    grads = core.get(4)
    wg = o.backward(dl)
    for n, g, w in zip(NAMES, grads, wg):
        assert np.array_equal(g, w.astype(np.float32)), (n, rel(g, w))


@pytest.mark.parametrize("fan,split", [(8, "1"), (24, "3")])
def test_exact_plug_staged_in_lds(gpu_lib, monkeypatch, fan, split):
    """The plug with each tile's observation slab staged in LDS (forced with FLYGUY_PLUG_LDS = workgroups per tile),
    bit-exact at B = 192 (three tiles of 64 samples) against the oracle, logits, sensory states and all seven
    gradients, as with the plug that gathers through the vector-memory path.  With fan 24, above the least segment
    cap (16), the plug's rows are split over two segments (partial sums, the combine kernel) and its gradient takes
    a third chunk of columns.  (The bfloat16 core keeps the plug's gradients in the sensory finish: a separate
    kernel as in float32 was slower here, its float32 drive gradient at B=16384 being 1.1 GB to write and read.)"""
    s, P, obs = _exact_case("b", 3, fan, 4)
    obs = np.concatenate([obs, -obs[::-1], np.roll(obs, 5, axis=1)])
    o = Core16(s, P)
    want = o.forward(obs)
    for layer, (h, _) in enumerate(o.states):
        assert np.array_equal(bf16(h), h) and np.abs(h).max() < 256, layer
    dl = np.random.default_rng(11).choice([-1.0, 0.0, 1.0], want.shape).astype(np.float32)
    want_g = o.backward(dl)
    for mode in ("0", split):
        monkeypatch.setenv("FLYGUY_PLUG_LDS", mode)
        say(f"bf16 exact b hops 3 fan {fan}, B 192, plug staged in LDS {mode}")
        core = Core(s, P, max_batch=192, flags=BF16)
        assert np.array_equal(core.forward(obs), want.astype(np.float32))
        assert np.array_equal(core.state(0, 1, s["sizes"][0], 192), o.drive.astype(np.float32))
        assert np.array_equal(core.state(0, 0, s["sizes"][0], 192), o.states[0][0].astype(np.float32))
        core.zero_grad()
        core.backward(dl)
        for n, g, w in zip(NAMES, core.get(4), want_g):
            assert np.array_equal(g, w.astype(np.float32)), (n, rel(g, w))
        del core


@pytest.mark.parametrize("tiles", ["1", "2"])
@pytest.mark.parametrize("hops", [3, 4])
def test_exact_one_and_two_tile_backward(gpu_lib, monkeypatch, tiles, hops):
    """Both hop backward kernels (one tile per workgroup, two: chosen per layer from how unevenly the gathered rows
    are used, forced here), bit-exact at B = 192: three tiles, so the two-tile kernel also meets a lone last tile.
    With 4 hops, a source row of hop 2 sends 18 connections, more than the backward plan's segment cap (16 for a
    product this small): its row is split, so the split-row combine runs in its paired form on a hop layer."""
    monkeypatch.setenv("FLYGUY_BWD_TILES", tiles)
    s, P, obs = _exact_case("b", hops, 8, 4)
    if hops == 4:
        out = np.bincount(np.asarray(s["hop"][1]["col"]), minlength=s["sizes"][1])
        assert out.max() > 16
    rng = np.random.default_rng(50)
    for i in (0, 3):                                            # denser strengths and plug weights: most gradients move
        P[i] = (rng.choice([-1.0, 1.0, 1.0], P[i].size) * (rng.random(P[i].size) < 0.5)).astype(np.float32)
    obs = np.concatenate([obs, -obs[::-1], np.roll(obs, 7, axis=1)])
    say(f"bf16 exact b hops {hops} fan 8, B 192, {tiles} tile(s) per backward workgroup")
    o = Core16(s, P)
    want = o.forward(obs)
    for layer, (h, _) in enumerate(o.states):
        assert np.array_equal(bf16(h), h) and np.abs(h).max() < 256, layer
    core = Core(s, P, max_batch=192, flags=BF16)
    assert np.array_equal(core.forward(obs), want.astype(np.float32))
    dl = np.random.default_rng(10).choice([-1.0, 0.0, 1.0], want.shape).astype(np.float32)
    core.zero_grad()
    core.backward(dl)
    for n, g, w in zip(NAMES, core.get(4), o.backward(dl)):
        assert np.array_equal(g, w.astype(np.float32)), (n, rel(g, w))


def test_weights_are_rounded_to_bfloat16(gpu_lib):
    """The sparse products use the strengths and plug weights rounded to bfloat16 (nearest even); the masters keep
    their float32 values.  Weights 1 + 2^-9, 1 + 2^-8 (a tie, to even: 1) and 1 - 2^-10 all round to 1, so the case
    stays exact and the library must equal the rounding oracle bit for bit, while the oracle without weight rounding
    differs."""
    s, P, obs = _exact_case("a", 3, 5, 5)
    rng = np.random.default_rng(12)
    off = np.array([1 + 2.0 ** -9, 1 + 2.0 ** -8, 1 - 2.0 ** -10], np.float32)
    for i in (0, 3):
        nz = P[i] != 0
        P[i][nz] = np.sign(P[i][nz]) * off[rng.integers(0, 3, int(nz.sum()))]
    assert not np.array_equal(bf16(P[0]), P[0].astype(np.float64))
    say("bf16 weights off the bfloat16 grid")
    o = Core16(s, P)
    want = o.forward(obs)
    for layer, (h, _) in enumerate(o.states):
        assert np.array_equal(bf16(h), h) and np.abs(h).max() < 256, layer
    core = Core(s, P, max_batch=64, flags=BF16)
    got = core.forward(obs)
    assert np.array_equal(got, want.astype(np.float32))
    dl = np.random.default_rng(13).choice([-1.0, 0.0, 1.0], got.shape).astype(np.float32)
    core.zero_grad()
    core.backward(dl)
    wg = o.backward(dl)
    for n, g, w in zip(NAMES, core.get(4), wg):
        assert np.array_equal(g, w.astype(np.float32)), (n, rel(g, w))
    un = Core16(s, P, round_weights=False)                      # the check has teeth: unrounded weights differ
    un.forward(obs)
    assert any(not np.array_equal(a, b) for a, b in zip(un.backward(dl), wg))
    assert np.array_equal(core.get(0)[0], P[0])                 # the master strengths are untouched


def _general(s, params, B, seed):
    obs = np.random.default_rng(seed).standard_normal((B, 517)).astype(np.float32)
    core = Core(s, params, max_batch=B, flags=BF16)
    got = core.forward(obs)
    o = Core16(s, params)
    want = o.forward(obs)
    assert np.isfinite(got).all()
    r = rel(got, want)
    ok, ties = argmax_agrees(got, want, margin=1e-2 * np.abs(want).max())
    say(f"   logits rel {r:.2e}, near ties {ties}")
    assert r <= 1e-3 and ok
    rng = np.random.default_rng(seed + 1)
    dl = ((rng.standard_normal(got.shape) + 0.2 * got) / B).astype(np.float32)
    core.zero_grad()
    core.backward(dl)
    for n, g, w in zip(NAMES, core.get(4), o.backward(dl)):
        r = rel(g, w)
        say(f"   grad {n:6s} rel {r:.2e}")
        assert r <= 1e-2, (n, r)
    return core, got


@pytest.mark.parametrize("name,hops,fan", [("a", 3, 5), ("b", 3, 16), ("c", 4, 6)])
def test_toy_against_oracle(gpu_lib, name, hops, fan):
    say(f"bf16 toy {name} hops {hops} fan {fan}")
    s, params = toy_net(name, hops, fan)
    _general(s, params, 128, 1)


def test_scaled_synthetic_against_oracle(gpu_lib):
    """The benchmark shape at 1/16 size: split rows, re-drive rows."""
    s, params = scaled_3hop(16)
    say("bf16 scaled synthetic 1/16, B 192")
    _general(s, params, 192, 2)


def test_oracle_without_rounding_is_the_float32_path(gpu_lib):
    """With its rounding switched off the restatement is the float32 core (checked against the float32 library)."""
    s, params = toy_net("b", 3, 16)
    obs = np.random.default_rng(4).standard_normal((64, 517)).astype(np.float32)
    got = Core(s, params, max_batch=64).forward(obs)
    want = Core16(s, params, round=False).forward(obs)
    assert rel(got, want) <= 1e-5


def test_batch_independence(gpu_lib):
    s, params = scaled_3hop(8)
    core = Core(s, params, max_batch=4096, flags=BF16)
    obs = np.random.default_rng(11).standard_normal((4096, 517)).astype(np.float32)
    big = core.forward(obs)
    for start in (0, 1984, 4032):
        assert np.array_equal(core.forward(obs[start:start + 64]), big[start:start + 64]), start
    perm = np.random.default_rng(1).permutation(4096)
    assert np.array_equal(core.forward(obs[perm]), big[perm])


def test_batch_must_be_a_multiple_of_64(gpu_lib):
    from flyguy_amd._lib import LibraryError
    s, params = toy_net("a", 2, 5)
    core = Core(s, params, max_batch=128, flags=BF16)
    with pytest.raises(LibraryError, match="multiple of 64"):
        core.forward(np.zeros((96, 517), np.float32))
