"""Parity of the MI355X library with the oracle, through the C-ABI (fc_*).

Tolerances (from the target: fp32 logits within 1e-5 relative, weight gradients within 1e-4 relative, argmax
identical), relative to the largest entry as flyguy/native/core_check.py:59 measures:
  logits and every internal state vs the float64 oracle   <= 1e-5
  logits vs the float32 oracle (the reference's arithmetic) <= 4e-6  (rows split over several waves are summed
                                                                      in pieces, the read-out on the matrix cores
                                                                      in 4 partial sums of 2-product steps rather
                                                                      than in row order; softplus may differ by an
                                                                      ulp)
  each of the seven gradient arrays vs the float64 oracle    <= 1e-4
  argmax identical wherever the top-2 margin exceeds 1e-4.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import CASES, lively, toy
from flyguy_amd.export import net_bytes, params_from_torch, structure
from flyguy_amd.fly import FlyActor
from flyguy_amd.synth import scaled_3hop, synth_3hop
from gpu_helpers import NAMES, Core, argmax_agrees, rel, say
from oracle.oracle import Oracle

pytestmark = pytest.mark.gpu


def toy_net(name, hops, fan, seed=0):
    torch.manual_seed(seed)
    f = lively(FlyActor(toy(name), 517, 90, hops=hops, fan=fan), seed)
    s = structure(f)
    return s, params_from_torch(f, s)


def check_forward(s, params, obs, core=None, states=True):
    core = core or Core(s, params, max_batch=obs.shape[0])
    got = core.forward(obs)
    o64 = Oracle(net_bytes(s), params, "f64")
    o32 = Oracle(net_bytes(s), params, "f32")
    want = o64.forward(obs)
    w32 = o32.forward(obs)
    assert np.isfinite(got).all()
    assert rel(got, want) <= 1e-5, rel(got, want)
    assert rel(got, w32) <= 4e-6, rel(got, w32)
    ok, ties = argmax_agrees(got, want)
    assert ok
    if states:
        B = obs.shape[0]
        for layer in range(s["hops"] + 1):
            rows = s["sizes"][layer]
            for what in ((0, 1) if layer == 0 else (0,)):       # hop layers keep h only (z is recomputed)
                g = core.state(layer, what, rows, B)
                w = o64.state(layer, what, rows)
                assert rel(g, w) <= 1e-5, (layer, what, rel(g, w))
    return core, o64, got, want


def check_backward(core, o64, s, logits, seed=1):
    rng = np.random.default_rng(seed)
    R = rng.standard_normal(logits.shape).astype(np.float32)
    dl = (R + 0.2 * logits).astype(np.float32)
    core.zero_grad()
    core.backward(dl)
    got = core.get(4)
    want = o64.backward(dl)
    for name, g, w in zip(NAMES, got, want):
        r = rel(g, w)
        say(f"      grad {name:6s} rel {r:.2e} (max {np.abs(w).max():.2e})")
        assert r <= 1e-4, (name, r)


@pytest.mark.parametrize("name,hops,fan", CASES)
def test_toy_forward_backward(gpu_lib, name, hops, fan):
    say(f"toy {name} hops {hops} fan {fan}")
    s, params = toy_net(name, hops, fan)
    obs = np.random.default_rng(0).standard_normal((64, 517)).astype(np.float32)
    core, o64, got, _ = check_forward(s, params, obs)
    check_backward(core, o64, s, got)


def test_zero_gain_neurons(gpu_lib):
    """Neurons of gain 0 never fire; their gain gradient is 0 (the reference sums g * z = 0), not 0 / 0."""
    say("toy a, 3 hops, fan 5, a tenth of the neurons at gain 0")
    s, params = toy_net("a", 3, 5, seed=5)
    rng = np.random.default_rng(5)
    ids = np.unique(np.concatenate([np.asarray(h["nid"]) for h in s["hop"]] + [np.asarray(s["n0"])]))
    params[1][rng.choice(ids, max(3, len(ids) // 10), replace=False)] = 0.0
    obs = rng.standard_normal((64, 517)).astype(np.float32)
    core, o64, got, _ = check_forward(s, params, obs)
    check_backward(core, o64, s, got)
    assert all(np.isfinite(g).all() for g in core.get(4))


@pytest.mark.parametrize("B", [32, 96, 256])
def test_scaled_synthetic(gpu_lib, B):
    """The 3-hop shape at 1/16 size: heavy rows split over several waves, re-drive rows, B not a multiple of 256."""
    say(f"scaled synthetic 1/16, B {B}")
    s, params = scaled_3hop(16)
    assert max(int(np.diff(h["crow"]).max()) for h in s["hop"]) > 256        # split rows are exercised
    obs = np.random.default_rng(B).standard_normal((B, 517)).astype(np.float32)
    core, o64, got, _ = check_forward(s, params, obs)
    check_backward(core, o64, s, got)


@pytest.mark.parametrize("tiles", ["1", "2"])
def test_one_and_two_tile_backward(gpu_lib, monkeypatch, tiles):
    """Both layer backward kernels (one tile per workgroup, two: chosen per layer from how unevenly the gathered
    rows are used, forced here), at B = 160: five tiles, so the two-tile kernel also meets a lone last tile."""
    monkeypatch.setenv("FLYGUY_BWD_TILES", tiles)
    say(f"scaled synthetic 1/16, B 160, {tiles} tile(s) per backward workgroup")
    s, params = scaled_3hop(16)
    obs = np.random.default_rng(160).standard_normal((160, 517)).astype(np.float32)
    core, o64, got, _ = check_forward(s, params, obs, states=False)
    check_backward(core, o64, s, got)


@pytest.mark.parametrize("case,B,split", [("toy", 96, "1"), ("toy", 96, "3"), ("scaled", 160, "2")])
def test_plug_staged_in_lds(gpu_lib, monkeypatch, case, B, split):
    """The plug with each tile's observation slab staged in LDS (launch_fwd_lds, and its gradients through
    launch_plug_bwd_lds: by default from 64 tiles up, forced here with FLYGUY_PLUG_LDS = workgroups per tile) sums the
    same terms in the same order as the plug that gathers through the vector-memory path: the sensory layer's drive
    and output, the logits and all seven gradients are bit-identical, and both match the oracle.  The toy has fan 24,
    above the least segment cap (16), so its plug rows are split over two segments (partial sums, k_fwd_combine) and
    take a third chunk of 8 columns in the gradient kernel; the 1/16 benchmark shape has 5 tiles (not a multiple of
    8)."""
    if case == "toy":
        s, params = toy_net("b", 3, 24)
        assert int(np.diff(s["in_crow"]).max()) > 16
    else:
        s, params = scaled_3hop(16)
    obs = np.random.default_rng(B + int(split)).standard_normal((B, 517)).astype(np.float32)
    out = {}
    for mode in ("0", split):
        monkeypatch.setenv("FLYGUY_PLUG_LDS", mode)
        say(f"{case}, B {B}: plug staged in LDS {mode}")
        core, o64, got, _ = check_forward(s, params, obs, states=True)
        check_backward(core, o64, s, got)
        out[mode] = (got, core.state(0, 0, s["n_s"], B), core.state(0, 1, s["n_s"], B), *core.get(4))
        del core
    for a, b in zip(out["0"], out[split]):
        assert np.array_equal(a, b)


@pytest.fixture(scope="module")
def full():
    return synth_3hop()


def test_full_size_against_oracle(gpu_lib, full):
    """The benchmark network (70k neurons in 3 hops, 2,992,734 strengths) at B = 64."""
    s, params = full
    say("full-size synthetic, B 64: forward")
    obs = np.random.default_rng(7).standard_normal((64, 517)).astype(np.float32)
    core, o64, got, _ = check_forward(s, params, obs, states=True)
    say("full-size synthetic, B 64: backward")
    check_backward(core, o64, s, got)


def test_full_size_batch_independence(gpu_lib, full):
    """At the benchmark batch (4096) every sample's logits are bit-identical to the same sample run in a batch of
    32: a sample's arithmetic does not depend on the batch around it or on the tile it lands in."""
    s, params = full
    say("full-size synthetic, B 4096 vs 32")
    core = Core(s, params, max_batch=4096)
    obs = np.random.default_rng(11).standard_normal((4096, 517)).astype(np.float32)
    big = core.forward(obs)
    for start in (0, 1024, 4064):
        small = core.forward(obs[start:start + 32])
        assert np.array_equal(small, big[start:start + 32]), start
    perm = np.random.default_rng(1).permutation(4096)
    assert np.array_equal(core.forward(obs[perm]), big[perm])


def test_gradients_add_up_over_pieces(gpu_lib, full):
    """fc_backward ADDS: two half batches give the gradient of the whole batch (to rounding)."""
    s, params = full
    core = Core(s, params, max_batch=512)
    obs = np.random.default_rng(5).standard_normal((512, 517)).astype(np.float32)
    R = np.random.default_rng(6).standard_normal((512, 90)).astype(np.float32)
    core.zero_grad()
    core.forward(obs)
    core.backward(R)
    whole = core.get(4)
    core.zero_grad()
    for i in (0, 256):
        core.forward(obs[i:i + 256])
        core.backward(R[i:i + 256])
    halves = core.get(4)
    for name, a, b in zip(NAMES, halves, whole):
        assert rel(a, b) <= 1e-5, name


@pytest.mark.parametrize("B,flags", [(96, 0), (4096, 0), (192, 1), (4096, 1)])
def test_skipping_silent_rows_changes_nothing(gpu_lib, monkeypatch, full, B, flags):
    """The forward skips the gathers of source rows that fire on no sample of a tile, the backward those of rows whose
    own output is zero on it (FLYGUY_SKIP_SILENT=0 turns both off): logits, every layer's state and all seven
    gradients are bit-identical with and without, on the benchmark network with a third of its neurons silenced
    (threshold raised) so that whole lines are zero; float32 states at B = 96 (a lone last tile of the two-tile
    backward) and 4096, bfloat16 states (flags 1, tiles of 64 samples) at B = 192 and 4096."""
    s, params = full
    P = [p.copy() for p in params]
    rng = np.random.default_rng(31)
    P[2][rng.random(P[2].size) < 1 / 3] = 6.0                  # softplus(6) ~ 6: these neurons almost never fire
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    dl = (rng.standard_normal((B, 90)) / B).astype(np.float32)
    out = {}
    monkeypatch.setenv("FLYGUY_BWD_SKIP", "1")                 # every layer's backward skips (short waves too)
    for mode in ("1", "0"):
        monkeypatch.setenv("FLYGUY_SKIP_SILENT", mode)
        core = Core(s, P, max_batch=B, flags=flags)
        lg = core.forward(obs)
        states = [core.state(layer, 0, s["sizes"][layer], B) for layer in range(s["hops"] + 1)]
        core.zero_grad()
        core.backward(dl)
        out[mode] = (lg, states, core.get(4))
        del core
    (l1, s1, g1), (l0, s0, g0) = out["1"], out["0"]
    tile = 64 if flags else 32
    silent = [float((~(st > 0).reshape(st.shape[0], -1, tile).any(2)).mean()) for st in s1[:-1]]
    say(f"   B {B} flags {flags}: silent (row, tile) lines per layer {[round(v, 3) for v in silent]}")
    assert max(silent) > 0.2
    assert np.array_equal(l1, l0)
    for a, b in zip(s1, s0):
        assert np.array_equal(a, b)
    for name, a, b in zip(NAMES, g1, g0):
        assert np.array_equal(a, b), name


@pytest.mark.parametrize("B,flags,tiles,plug", [(96, 0, "2", ""), (4096, 0, "1", ""), (4096, 0, "2", ""),
                                                 (192, 1, "2", ""), (4096, 1, "1", ""), (96, 0, "2", "fan32"),
                                                 (192, 1, "1", "fan32")])
def test_pair_storage_changes_nothing(gpu_lib, monkeypatch, full, B, flags, tiles, plug):
    """A plan's (source, weight) pairs are stored in 6 bytes (weights, then 16-bit sources, per wave step) when the
    state its product gathers has at most 65,535 rows and its waves walk 3 steps or more on average (on the benchmark
    network every product but the plug and hop 3's backward); FLYGUY_PAIR_BYTES=8 keeps the 8-byte pairs, =6 stores
    every plan whose gathered state allows it in 6 bytes (the plug and hop 3's backward too).  Logits, every layer's
    state and all seven gradients are bit-identical either way: float32 states at B = 96 and 4096, one
    and two tiles per backward workgroup, bfloat16 states (flags 1) at B = 192 and 4096, with a third of the neurons
    silenced so that the forward's silent-source drops (made after the staging with 6-byte pairs) are taken; and a
    network of the benchmark shape whose plug reads 32 inputs per sensory neuron (4 steps a wave, so its pairs take 6
    bytes too) through the plug kernels that stage the observations in LDS (FLYGUY_PLUG_LDS=4)."""
    if plug == "fan32":
        s, params = synth_3hop(fan=32)
        monkeypatch.setenv("FLYGUY_PLUG_LDS", "4")
    else:
        s, params = full
    P = [p.copy() for p in params]
    rng = np.random.default_rng(32)
    P[2][rng.random(P[2].size) < 1 / 3] = 6.0                  # softplus(6) ~ 6: these neurons almost never fire
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    dl = (rng.standard_normal((B, 90)) / B).astype(np.float32)
    monkeypatch.setenv("FLYGUY_BWD_TILES", tiles)
    out = {}
    for pb in ("8", "6"):
        monkeypatch.setenv("FLYGUY_PAIR_BYTES", pb)
        core = Core(s, P, max_batch=B, flags=flags)
        lg = core.forward(obs)
        states = [core.state(layer, 0, s["sizes"][layer], B) for layer in range(s["hops"] + 1)]
        core.zero_grad()
        core.backward(dl)
        out[pb] = (lg, states, core.get(4))
        del core
    (l8, s8, g8), (l6, s6, g6) = out["8"], out["6"]
    assert np.isfinite(l6).all()
    assert np.array_equal(l8, l6)
    for a, b in zip(s8, s6):
        assert np.array_equal(a, b)
    for name, a, b in zip(NAMES, g8, g6):
        assert np.array_equal(a, b), name


@pytest.mark.parametrize("net,B,mode,pb,skip,flags", [("full", 4096, "auto", "", "", 0), ("full", 4096, "1", "6", "1", 0),
                                                       ("full", 512, "auto", "", "", 0), ("full", 96, "1", "", "1", 0),
                                                       ("scaled", 160, "1", "6", "", 0), ("full", 4096, "auto", "", "", 1),
                                                       ("full", 192, "1", "6", "1", 1)])
def test_backward_staged_in_lds_changes_nothing(gpu_lib, monkeypatch, full, net, B, mode, pb, skip, flags):
    """The last hop's backward gathers the descending layer's gradient (1,332 rows, 170 kB a tile).  From 16 tiles up
    (FLYGUY_BWD_LDS=1: at every batch) it runs k_bwd_lds: each workgroup stages the 1,231 most gathered of those rows
    in LDS and gathers the other 101 (about 0.2% of the gathers) through the vector-memory path in the steps that
    need one.  Its sums are those of the one-tile kernel it replaces (FLYGUY_BWD_TILES=1, FLYGUY_BWD_LDS=0), term for
    term: all seven gradients are bit-identical on the benchmark network at B = 4096, 512 and 96 (three tiles: many
    workgroups per tile), with 8- and 6-byte pairs, with the backward's silent-row skip forced on (FLYGUY_BWD_SKIP=1)
    and a third of the neurons silenced so that it is taken; on the 1/16 network, whose 83 descending rows all fit
    the LDS; and over bfloat16 states (flags 1: k_cbwd16_lds against k_cbwd16) at B = 4096 and 192 (three 64-sample
    tiles)."""
    s, params = full if net == "full" else scaled_3hop(16)
    P = [p.copy() for p in params]
    rng = np.random.default_rng(B + 7)
    P[2][rng.random(P[2].size) < 1 / 3] = 6.0                  # softplus(6) ~ 6: these neurons almost never fire
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    dl = (rng.standard_normal((B, 90)) / B).astype(np.float32)
    monkeypatch.setenv("FLYGUY_BWD_TILES", "1")
    if pb:
        monkeypatch.setenv("FLYGUY_PAIR_BYTES", pb)
    if skip:
        monkeypatch.setenv("FLYGUY_BWD_SKIP", skip)
    out = {}
    for lds in ("0", mode):
        say(f"{net} B {B} flags {flags}: FLYGUY_BWD_LDS={lds} pairs {pb or 'by plan'} skip {skip or 'by plan'}")
        monkeypatch.setenv("FLYGUY_BWD_LDS", lds)
        core = Core(s, P, max_batch=B, flags=flags)
        lg = core.forward(obs)
        core.zero_grad()
        core.backward(dl)
        out[lds] = (lg, core.get(4))
        del core
    (l0, g0), (l1, g1) = out["0"], out[mode]
    assert np.array_equal(l0, l1)
    for name, a, b in zip(NAMES, g0, g1):
        assert np.isfinite(b).all(), name
        assert np.array_equal(a, b), name

