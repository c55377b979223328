"""Randomised parity: graphs drawn at random in the graph-file form (a few hundred to 1,500 neurons, skewed
in-degree, random sensory and descending sets), indexed by FlyActor with 2-4 hops (1, 5, 6, 9 in one test) and fan
4, 8 or 16, then run through the library at a random batch against the float64 oracle, with the one-/two-tile choice
and the silent-row skips set per case.  Bars as tests/test_gpu_parity.py (logits and states <= 1e-5, gradients <= 1e-4,
relative to the largest entry; argmax identical off near-ties); the teaching step is held bit for bit to its parts;
the bfloat16 core to its numpy oracle at the general-network bars of tests/test_gpu_core16.py."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import lively
from flyguy_amd._lib import call
from flyguy_amd.export import params_from_torch, structure
from flyguy_amd.fly import FlyActor
from gpu_helpers import NAMES, Core, argmax_agrees, rel, say
from oracle.core16 import Core16
from test_gpu_parity import check_backward, check_forward

pytestmark = pytest.mark.gpu

TRANSMITTERS = np.array(["glutamate", "histamine", "acetylcholine", "serotonin", "gaba"])


def random_graph(seed: int) -> tuple[dict, np.random.Generator]:
    """A graph file's arrays: neurons with ids from 1000, synapse rows (pre, post, count) with a lognormal
    popularity of targets, distinct sensory and descending sets."""
    rng = np.random.default_rng(seed)
    n = int(rng.integers(150, 1500))
    E = int(n * rng.uniform(6, 14))
    pop = rng.lognormal(0.0, rng.uniform(0.5, 1.8), n)
    post = rng.choice(n, E, p=pop / pop.sum()).astype(np.int32)
    pre = rng.integers(0, n, E).astype(np.int32)
    keep = pre != post
    pre, post = pre[keep], post[keep]
    perm = rng.permutation(n)
    n_s, n_d = max(5, n // int(rng.integers(8, 14))), max(4, n // int(rng.integers(15, 30)))
    g = {"body": np.arange(1000, 1000 + n), "nt": TRANSMITTERS[rng.integers(0, len(TRANSMITTERS), n)], "pre": pre,
         "post": post, "syn": rng.integers(1, 40, len(pre)).astype(np.int32),
         "sensory": np.sort(perm[:n_s]).astype(np.int32), "descending": np.sort(perm[n_s:n_s + n_d]).astype(np.int32)}
    return g, rng


def case(seed: int):
    g, rng = random_graph(seed)
    hops, fan = int(rng.integers(2, 5)), int(rng.choice([4, 8, 16]))
    torch.manual_seed(seed)
    f = lively(FlyActor(g, 517, 90, hops=hops, fan=fan), seed)
    s = structure(f)
    return s, params_from_torch(f, s), rng, hops, fan


@pytest.mark.parametrize("seed", range(16))
def test_random_graph_against_oracle(gpu_lib, monkeypatch, seed):
    s, params, rng, hops, fan = case(seed)
    B = int(rng.choice([32, 64, 96, 160]))
    tiles = ("", "1", "2")[seed % 3]
    if tiles:
        monkeypatch.setenv("FLYGUY_BWD_TILES", tiles)
    monkeypatch.setenv("FLYGUY_SKIP_SILENT", "0" if seed % 4 == 3 else "1")
    say(f"random graph {seed}: sizes {s['sizes']}, edges {[len(h['col']) for h in s['hop']]}, hops {hops}, fan {fan}, "
        f"B {B}, tiles {tiles or 'rule'}, skips {'off' if seed % 4 == 3 else 'on'}")
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    core, o64, got, _ = check_forward(s, params, obs)
    check_backward(core, o64, s, got, seed=seed)


@pytest.mark.parametrize("seed", range(16, 24))
def test_random_graph_teach_step_and_its_parts(gpu_lib, seed):
    s, params, rng, hops, fan = case(seed)
    B = 64
    say(f"random graph {seed}: sizes {s['sizes']}, hops {hops}, fan {fan}: teaching step against its parts")
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    x = torch.as_tensor(obs).cuda()
    t = torch.as_tensor((2 * rng.standard_normal((B, 90))).astype(np.float32)).cuda()
    a, b = Core(s, params, max_batch=B), Core(s, params, max_batch=B)
    for _ in range(2):
        call("fc_teach_step", a.h, x.data_ptr(), t.data_ptr(), B, 1.0, 1e-2, 3e-3, 1e-2, 0.0, 0.9, None)
        lg = torch.as_tensor(b.forward(obs)).cuda()
        dl = torch.empty(B, 90, device="cuda")
        st = torch.zeros(2, device="cuda")
        call("fc_kl_loss", b.h, lg.data_ptr(), t.data_ptr(), B, 1.0, dl.data_ptr(), st.data_ptr())
        b.zero_grad()
        b.backward(dl.cpu().numpy())
        call("fc_step", b.h, 1e-2, 3e-3, 1e-2, 0.0, 0.9)
    torch.cuda.synchronize()
    for which in (0, 1, 2, 3):
        for pa, pb in zip(a.get(which), b.get(which)):
            assert np.array_equal(pa.view(np.uint32), pb.view(np.uint32)), which


@pytest.mark.parametrize("seed", range(24, 32))
def test_random_graph_bfloat16_against_its_oracle(gpu_lib, seed):
    s, params, rng, hops, fan = case(seed)
    B = int(rng.choice([64, 128]))
    say(f"random graph {seed}: sizes {s['sizes']}, hops {hops}, fan {fan}, B {B}: bfloat16 core")
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    o = Core16(s, params)
    want = o.forward(obs)
    core = Core(s, params, max_batch=B, flags=1)
    got = core.forward(obs)
    assert rel(got, want) <= 1e-3, rel(got, want)
    ok, _ = argmax_agrees(got, want, 1e-2)
    assert ok
    dl = (rng.standard_normal(want.shape) + 0.2 * want).astype(np.float32)
    core.zero_grad()
    core.backward(dl)
    for name, g, w in zip(NAMES, core.get(4), o.backward(dl)):
        assert rel(g, w) <= 1e-2, (name, rel(g, w))


@pytest.mark.parametrize("seed", range(32, 40))
def test_random_graph_backward_staged_in_lds(gpu_lib, monkeypatch, seed):
    """The last hop's backward with its gathered rows staged in LDS (k_bwd_lds / k_cbwd16_lds, forced at every batch
    with FLYGUY_BWD_LDS=1; a random graph's last layer fits the LDS whole) against the one-tile kernel it replaces
    (FLYGUY_BWD_TILES=1, FLYGUY_BWD_LDS=0), on random graphs of 2-4 hops: logits and all seven gradients bit for bit,
    over float32 states (even seeds) and bfloat16 states (odd seeds), at batches of one to three tiles."""
    s, params, rng, hops, fan = case(seed)
    flags = seed % 2
    B = int(rng.choice([64, 128, 192] if flags else [32, 96, 160]))
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    dl = (rng.standard_normal((B, 90)) / B).astype(np.float32)
    monkeypatch.setenv("FLYGUY_BWD_TILES", "1")
    out = {}
    for lds in ("0", "1"):
        say(f"random graph {seed}: sizes {s['sizes']}, hops {hops}, fan {fan}, B {B}, flags {flags}: "
            f"FLYGUY_BWD_LDS={lds}")
        monkeypatch.setenv("FLYGUY_BWD_LDS", lds)
        core = Core(s, params, max_batch=B, flags=flags)
        lg = core.forward(obs)
        core.zero_grad()
        core.backward(dl)
        out[lds] = (lg, core.get(4))
        del core
    (l0, g0), (l1, g1) = out["0"], out["1"]
    assert np.array_equal(l0, l1)
    for name, a, b in zip(NAMES, g0, g1):
        assert np.isfinite(b).all(), name
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), name


@pytest.mark.parametrize("hops,seed", [(1, 40), (1, 41), (1, 42), (1, 43), (1, 44), (1, 45), (5, 50), (6, 51),
                                       (9, 50)])
def test_random_graph_one_and_many_hops(gpu_lib, hops, seed):
    """Networks of one hop (FlyActor's hops=1: the sensory layer feeds the layer the read-out reads, whose backward
    is the sensory finish and has no hop above it to stage in LDS) and of 5, 6 and 9 hops (beyond the profiler's 8
    per-hop stages): float32 against the float64 oracle at the bars of tests/test_gpu_parity.py at a batch of 32 or
    96, and the bfloat16 core against its oracle at 64."""
    g, rng = random_graph(seed)
    torch.manual_seed(seed)
    f = lively(FlyActor(g, 517, 90, hops=hops, fan=8), seed)
    s = structure(f)
    params = params_from_torch(f, s)
    B = int(rng.choice([32, 96]))
    say(f"random graph {seed}, {hops} hops: sizes {s['sizes']}, edges {[len(h['col']) for h in s['hop']]}, B {B}")
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    core, o64, got, _ = check_forward(s, params, obs)
    check_backward(core, o64, s, got, seed=seed)
    obs16 = rng.standard_normal((64, 517)).astype(np.float32)
    o = Core16(s, params)
    want = o.forward(obs16)
    c16 = Core(s, params, max_batch=64, flags=1)
    got16 = c16.forward(obs16)
    assert rel(got16, want) <= 1e-3, rel(got16, want)
    dl = (rng.standard_normal(want.shape) + 0.2 * want).astype(np.float32)
    c16.zero_grad()
    c16.backward(dl)
    for name, g16, w in zip(NAMES, c16.get(4), o.backward(dl)):
        assert rel(g16, w) <= 1e-2, (name, rel(g16, w))
