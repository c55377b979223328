"""Decisions on the host CPU (flyguy_amd/libfly_infer.so, include/fly_infer.h) and the visualizer tap.

The library against the reference's own compiled CPU forward (oracle/_ref, built from fly_infer.cpp where the
reference checkout is present): logits and firing bytes bit-identical (same float32 sums in the same order).  The
actor's CPU play through it against the float64 oracle (<= 1e-5 of the largest logit) and against the sparse-product
path it replaces.  The VizTap file's fields."""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from conftest import CASES, lively, toy
from flyguy_amd.export import net_bytes, params_from_torch, structure
from flyguy_amd.fly import FlyActor, VizTap
from oracle import refinfer
from oracle.oracle import Oracle

OURS = FlyActor.__module__ and __import__("pathlib").Path(__import__("flyguy_amd").__file__).parent / "libfly_infer.so"


def _actor(name, hops, fan, seed=0):
    torch.manual_seed(seed)
    return lively(FlyActor(toy(name), 517, 90, hops=hops, fan=fan), seed)


@pytest.mark.skipif(not refinfer.available(), reason="the reference's CPU forward is not built here")
@pytest.mark.parametrize("name,hops,fan", CASES)
def test_bit_identical_to_the_reference_cpu_forward(name, hops, fan):
    f = _actor(name, hops, fan)
    s = structure(f)
    P = params_from_torch(f, s)
    obs = np.random.default_rng(1).standard_normal((16, 517)).astype(np.float32)
    n = sum(s["sizes"])
    tap_ref, tap_ours = np.zeros(n, np.uint8), np.zeros(n, np.uint8)
    ref = refinfer.RefInfer(s, P).forward(obs, tap_ref)
    ours = refinfer.RefInfer(s, P, lib_path=OURS).forward(obs, tap_ours)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(tap_ours, tap_ref) and tap_ours.any()


@pytest.mark.parametrize("name,hops,fan", [("a", 3, 5), ("b", 3, 16), ("c", 4, 6)])
def test_actor_cpu_play(monkeypatch, name, hops, fan):
    f = _actor(name, hops, fan)
    s = structure(f)
    obs = np.random.default_rng(2).standard_normal((8, 517)).astype(np.float32)
    want = Oracle(net_bytes(s), params_from_torch(f, s), "f64").forward(obs)
    with torch.no_grad():
        got = f(torch.as_tensor(obs)).numpy()
        assert f._decider[1] is not None                        # the library played
        monkeypatch.setenv("FLYGUY_NATIVE", "0")
        f.w.mul_(1.0)                                           # (a new weight version: set-up again, now without it)
        sparse = f(torch.as_tensor(obs)).numpy()
        assert f._decider[1] is None
    scale = max(1.0, np.abs(want).max())
    assert np.abs(got - want).max() <= 1e-5 * scale
    assert np.abs(sparse - want).max() <= 1e-5 * scale
    # weights changed after set-up are picked up
    monkeypatch.setenv("FLYGUY_NATIVE", "1")
    with torch.no_grad():
        f.out.bias.add_(1.0)
        moved = f(torch.as_tensor(obs)).numpy()
    assert np.allclose(moved, got + 1.0, atol=1e-5 * scale)


def test_viz_tap(tmp_path, monkeypatch):
    f = _actor("a", 3, 5)
    path = tmp_path / "viz.bin"
    tap = VizTap(f.sizes, path)
    f.tap = tap
    obs = torch.as_tensor(np.random.default_rng(3).standard_normal((4, 517)).astype(np.float32))
    with torch.no_grad():
        f(obs)                                                 # through the CPU library: bytes as they come out
    first = np.asarray(tap.acts).copy()
    tap.publish(7, np.arange(8, dtype=np.float32), np.full(90, 1 / 90, np.float32), clock=12.5, frame=99)
    raw = path.read_bytes()
    assert raw[:4] == b"FLYV" and struct.unpack("<I", raw[4:8])[0] == 1
    seq, tick = struct.unpack("<II", raw[8:16])
    assert seq == 2 and tick == 1 and struct.unpack("<i", raw[24:28])[0] == 7
    assert np.array_equal(np.frombuffer(raw[28:60], np.float32), np.arange(8, dtype=np.float32))
    assert struct.unpack("<5I", raw[60:80]) == (len(f.sizes), *(list(f.sizes) + [0] * 4)[:4])
    assert struct.unpack("<fIi", raw[440:452]) == (12.5, 99, 0)
    body = np.frombuffer(raw[512:], np.uint8)
    assert len(body) == sum(f.sizes) and np.array_equal(body, first) and body.any()
    # the sparse-product path hands over one tensor per layer; its bytes agree with the library's within one step
    monkeypatch.setenv("FLYGUY_NATIVE", "0")
    with torch.no_grad():
        f.w.mul_(1.0)
        f(obs)
    tap.publish(3, np.zeros(8), np.zeros(90))
    body2 = np.frombuffer(path.read_bytes()[512:], np.uint8)
    assert np.abs(body2.astype(int) - first.astype(int)).max() <= 1
    tap.close()


@pytest.mark.skipif(not refinfer.available(), reason="the reference's CPU forward is not built here")
@pytest.mark.parametrize("name,hops,fan", [("a", 3, 5), ("c", 4, 6)])
def test_cpu_decisions_from_a_network_file(tmp_path, name, hops, fan):
    """flyguy_amd.cpu_decisions.CpuDecisions on NET.bin / PARAMS.bin: the reference's compiled CPU forward's logits and
    firing bytes, bit for bit, and the float64 oracle's logits within 1e-5."""
    from flyguy_amd.cpu_decisions import CpuDecisions
    from flyguy_amd.export import read_net, read_params, write_params
    f = _actor(name, hops, fan)
    s = structure(f)
    P = params_from_torch(f, s)
    (tmp_path / "net.bin").write_bytes(net_bytes(s))
    write_params(P, tmp_path / "p.bin", 7)
    s2 = read_net(tmp_path / "net.bin")
    step, P2 = read_params(tmp_path / "p.bin", s2)
    assert step == 7
    obs = np.random.default_rng(2).standard_normal((9, 517)).astype(np.float32)
    tap_ours, tap_ref = (np.zeros(int(sum(s["sizes"])), np.uint8) for _ in range(2))
    got = CpuDecisions(s2, P2).forward(obs, tap_ours)
    want = refinfer.RefInfer(s, P).forward(obs, tap_ref)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(tap_ours, tap_ref)
    o = Oracle(net_bytes(s), P, "f64").forward(obs)
    assert np.abs(got - o).max() <= 1e-5 * max(np.abs(o).max(), 1.0)


@pytest.mark.parametrize("name,hops,fan", [("a", 3, 5), ("c", 4, 6)])
@pytest.mark.parametrize("threads", [2, 3, 8])
def test_cpu_decisions_on_several_threads(name, hops, fan, threads):
    """One car decided on several threads (fly_set_threads): the logits and firing bytes of one thread, bit for bit,
    for several cars in a row and for batches (the threads wait between cars and between calls)."""
    from flyguy_amd.cpu_decisions import CpuDecisions
    f = _actor(name, hops, fan)
    s = structure(f)
    P = params_from_torch(f, s)
    obs = np.random.default_rng(3).standard_normal((7, 517)).astype(np.float32)
    one = CpuDecisions(s, P)
    many = CpuDecisions(s, P, threads=threads)
    for rep in range(3):
        tap1, tapn = (np.zeros(int(sum(s["sizes"])), np.uint8) for _ in range(2))
        want = one.forward(obs[rep:], tap1)
        got = many.forward(obs[rep:], tapn)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
        assert np.array_equal(tapn, tap1), rep
    for i in range(len(obs)):
        assert np.array_equal(many.forward(obs[i:i + 1]), one.forward(obs[i:i + 1]))


def test_actor_cpu_play_on_several_threads(monkeypatch):
    """FLYGUY_CPU_THREADS: the actor's CPU play on 4 threads gives one thread's logits bit for bit."""
    f = _actor("a", 3, 5)
    obs = torch.as_tensor(np.random.default_rng(5).standard_normal((6, 517)).astype(np.float32))
    with torch.no_grad():
        one = f(obs).numpy()
        monkeypatch.setenv("FLYGUY_CPU_THREADS", "4")
        f.w.mul_(1.0)                                           # (a new weight version: set-up again, on 4 threads)
        four = f(obs).numpy()
        assert f._decider[1] is not None
    assert np.array_equal(four.view(np.uint32), one.view(np.uint32))
