"""The converter's command line (python -m flyguy_amd.export; the reference's flyguy/native/export.py:91-147):
graph -> NET.bin + initial PARAMS, checkpoint -> PARAMS.bin -> checkpoint (strengths in play scattered through wmap,
bit-exact round trip), and the FLYB batch with the PyTorch path's answer."""
from __future__ import annotations

import re
import struct

import numpy as np
import torch

from conftest import GOLDEN, lively
from flyguy_amd.export import main, net_bytes, params_from_torch, read_params, structure, write_params
from flyguy_amd.fly import FlyActor

GRAPH = GOLDEN / "toy_b.npz"


def _actor(seed=0):
    torch.manual_seed(seed)
    return FlyActor(str(GRAPH), 517, 90, hops=3, fan=16)


def _checkpoint(tmp_path, f, steps=123):
    ck = {"model": {"actor." + k: v.detach().clone() for k, v in f.state_dict().items()},
          "config": {"model": {"fly_graph": str(GRAPH), "fly_hops": 3}}, "steps": steps}
    path = tmp_path / "ck.pt"
    torch.save(ck, path)
    return path


def test_net_writes_the_network_and_its_initial_weights(tmp_path, capsys):
    torch.manual_seed(7)
    assert main(["net", str(GRAPH), str(tmp_path / "net.bin"), "--hops", "3", "--fan", "16"]) == 0
    f = _actor(7)
    s = structure(f)
    assert (tmp_path / "net.bin").read_bytes() == net_bytes(s)
    step, P = read_params(tmp_path / "net.init.bin", s)
    assert step == 0
    for a, b in zip(P, params_from_torch(f, s)):
        assert np.array_equal(a, b)
    assert "strengths in play" in capsys.readouterr().out


def test_checkpoint_round_trip_through_params(tmp_path):
    f = lively(_actor(1), 1)
    s = structure(f)
    ck = _checkpoint(tmp_path, f)
    assert main(["params", str(ck), str(tmp_path / "p.bin")]) == 0
    step, P = read_params(tmp_path / "p.bin", s)
    assert step == 0
    for a, b in zip(P, params_from_torch(f, s)):
        assert np.array_equal(a, b)
    # trained weights (every array moved) back into the checkpoint
    rng = np.random.default_rng(2)
    P2 = [(p + rng.standard_normal(p.shape).astype(np.float32) * 0.1).astype(np.float32) for p in P]
    write_params(P2, tmp_path / "p2.bin", 777)
    assert main(["torch", str(tmp_path / "p2.bin"), str(ck), str(tmp_path / "out.pt")]) == 0
    out = torch.load(tmp_path / "out.pt", map_location="cpu", weights_only=True)
    assert out["steps"] == 777
    m = out["model"]
    wmap = np.asarray(s["wmap"], np.int64)
    w = m["actor.w"].numpy()
    assert np.array_equal(w[wmap], P2[0])
    off = np.ones(len(w), bool)
    off[wmap] = False
    assert off.any() and np.array_equal(w[off], f.w.detach().numpy()[off])      # strengths not in play untouched
    assert m["actor.out.weight"].shape == f.out.weight.shape
    for key, a in zip(("actor.gain", "actor.theta", "actor.in_w", "actor.in_b", "actor.out.weight", "actor.out.bias"),
                      P2[1:]):
        assert np.array_equal(m[key].numpy().reshape(-1), a), key
    # and once more to PARAMS: bit-exact
    assert main(["params", str(tmp_path / "out.pt"), str(tmp_path / "p3.bin")]) == 0
    _, P3 = read_params(tmp_path / "p3.bin", s)
    for a, b in zip(P3, P2):
        assert np.array_equal(a, b)


def test_batch_file_and_the_pytorch_answer(tmp_path, capsys):
    f = lively(_actor(3), 3)
    ck = _checkpoint(tmp_path, f)
    assert main(["batch", str(ck), str(tmp_path / "b.bin"), "--n", "64"]) == 0
    raw = (tmp_path / "b.bin").read_bytes()
    assert raw[:4] == b"FLYB" and struct.unpack("<i", raw[4:8])[0] == 64
    x = np.frombuffer(raw, np.float32, 64 * 517, 8).reshape(64, 517)
    t = np.frombuffer(raw, np.float32, 64 * 90, 8 + 4 * 64 * 517).reshape(64, 90)
    assert len(raw) == 8 + 4 * 64 * (517 + 90)
    torch.manual_seed(0)
    assert np.array_equal(x, (0.7 * torch.randn(64, 517)).numpy())
    out = capsys.readouterr().out
    with torch.no_grad():
        lg = f(torch.as_tensor(x.copy()))
        lt = torch.log_softmax(torch.as_tensor(t.copy()), -1)
        loss = float((lt.exp() * (lt - torch.log_softmax(lg, -1))).sum(-1).mean())
    m = re.search(r"torch: loss ([-0-9.e+]+) agree ([0-9.]+)", out)
    assert m and abs(float(m.group(1)) - loss) <= 1e-5 * max(1.0, abs(loss))
    for name in ("W", "gain", "theta", "in_w", "in_b", "out_w", "out_b"):
        assert re.search(rf"grad {name}\s+norm [-0-9.e+]+ sum [-+0-9.e]+", out), name


def test_checkpoint_fan_comes_from_its_config(tmp_path):
    """A checkpoint trained with another plug fan (config.model.fly_fan) converts without --fan."""
    torch.manual_seed(4)
    f = FlyActor(str(GRAPH), 517, 90, hops=3, fan=8)
    s = structure(f)
    ck = {"model": {"actor." + k: v.detach().clone() for k, v in f.state_dict().items()},
          "config": {"model": {"fly_graph": str(GRAPH), "fly_hops": 3, "fly_fan": 8}}, "steps": 5}
    torch.save(ck, tmp_path / "ck8.pt")
    assert main(["params", str(tmp_path / "ck8.pt"), str(tmp_path / "p8.bin")]) == 0
    step, P = read_params(tmp_path / "p8.bin", s)
    assert s["fan"] == 8 and P[3].size == 8 * s["n_s"]
    for a, b in zip(P, params_from_torch(f, s)):
        assert np.array_equal(a, b)
