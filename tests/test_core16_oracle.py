"""The bfloat16-state oracle (oracle/core16.py) pinned on the CPU: its rounding against hand-worked cases, and with
the rounding switched off, its forward and backward against the float64 C oracle (oracle/fly_oracle.c)."""
from __future__ import annotations

import numpy as np
import torch

from conftest import lively, toy
from flyguy_amd.export import net_bytes, params_from_torch, structure
from flyguy_amd.fly import FlyActor
from oracle.core16 import Core16, bf16
from oracle.oracle import Oracle


def test_bf16_rounding():
    e = 2.0 ** -8
    cases = {1 + e: 1.0,                       # a tie goes to the even neighbour
             1 + 3 * e: 1 + 4 * e,             # a tie whose even neighbour is above
             1 + e + 2 ** -20: 1 + 2 * e,      # just above a tie
             -(1 + e): -1.0, 0.0: 0.0, 255.0: 255.0, 257.0: 256.0, 259.0: 260.0,
             3.4028235e38: np.inf, np.inf: np.inf, -np.inf: -np.inf}
    for v, w in cases.items():
        assert bf16(np.array([v]))[0] == w, v
    assert np.signbit(bf16(np.array([-0.0]))[0]) and np.isnan(bf16(np.array([np.nan]))[0])


def _net(name, hops, fan):
    torch.manual_seed(0)
    f = lively(FlyActor(toy(name), 517, 90, hops=hops, fan=fan), 0)
    s = structure(f)
    return s, params_from_torch(f, s)


def test_unrounded_restatement_is_the_float64_oracle():
    for name, hops, fan in (("a", 3, 5), ("c", 4, 6)):
        s, params = _net(name, hops, fan)
        obs = np.random.default_rng(1).standard_normal((32, 517)).astype(np.float32)
        o = Oracle(net_bytes(s), params, "f64")
        want = o.forward(obs)
        c = Core16(s, params, round=False)
        got = c.forward(obs)
        assert np.abs(got - want).max() <= 1e-6 * max(1.0, np.abs(want).max())
        dl = np.random.default_rng(2).standard_normal(want.shape).astype(np.float32)
        for g, w in zip(c.backward(dl), o.backward(dl)):
            assert np.abs(g - w).max() <= 1e-5 * max(1e-30, np.abs(w).max())
