"""The CPU revive tool (python -m flyguy_amd.revive, the reference's native/revive.py on NET.bin): silent neurons of a
toy network come back, the network's answers do not change, and the surgery's rules hold (signs, zeros, resets)."""
from __future__ import annotations

import numpy as np
import torch

from conftest import lively, toy
from flyguy_amd.export import net_bytes, params_from_torch, read_net, read_params, structure, write_params
from flyguy_amd.fly import FlyActor
from flyguy_amd.revive import Net, main
from oracle import trainer as ot
from oracle.oracle import Oracle


def test_revive_tool(tmp_path, capsys):
    torch.manual_seed(0)
    f = lively(FlyActor(toy("a"), 517, 90, hops=3, fan=5), 0)
    s = structure(f)
    P = params_from_torch(f, s)
    rng = np.random.default_rng(0)
    sens = set(np.asarray(s["n0"]).tolist())
    cand = sorted({int(g) for h in s["hop"] for g in h["nid"]} - sens)
    forced = rng.choice(cand, max(3, len(cand) // 8), replace=False)
    P[1][forced] = 0.0
    (tmp_path / "net.bin").write_bytes(net_bytes(s))
    write_params(P, tmp_path / "p.bin", 17)
    obs = rng.standard_normal((256, 517)).astype(np.float16)
    tl = (2 * rng.standard_normal((256, 90))).astype(np.float16)
    ot.write_chunk(tmp_path / "chunk.bin", obs, tl)
    assert main([str(tmp_path / "net.bin"), str(tmp_path / "p.bin"), str(tmp_path / "chunk.bin"), str(tmp_path / "out.bin"),
                 "--samples", "192"]) == 0
    out = capsys.readouterr().out
    assert "silent neurons" in out and ": written" in out
    s2 = read_net(tmp_path / "net.bin")
    step, Q = read_params(tmp_path / "out.bin", s2)
    assert step == 17
    net = Net(s2)
    x = torch.from_numpy(obs[:192].astype(np.float32))
    t = torch.from_numpy(tl[:192].astype(np.float32))
    fired, seen, _, _, kl0 = net.survey(P, x, t)
    dead = seen & (fired == 0)
    dead[np.asarray(s["n0"])] = False
    assert set(forced.tolist()) <= set(np.flatnonzero(dead).tolist())
    # the rules: resets, signs kept in size but not in direction, zero onto live neurons and actions
    assert (Q[1][dead] == 1).all() and (Q[2][dead] == -4).all()
    inc, outg = dead[net.post], dead[net.pre]
    assert (Q[0][outg & ~inc] == 0).all()
    untouched = ~inc & ~outg
    assert np.array_equal(Q[0][untouched], P[0][untouched])
    dn_ids = np.asarray(s["hop"][-1]["nid"])[np.asarray(s["dn_rows"])]
    assert (Q[5].reshape(90, -1)[:, dead[dn_ids]] == 0).all()
    # the revived neurons fire; the answers are the same (float64 oracle before and after)
    fired2, _, _, _, kl1 = net.survey(Q, x, t)
    assert (fired2[dead] > 0).mean() > 0.5
    assert abs(kl1 - kl0) < 1e-4
    o1 = Oracle(net_bytes(s), P, "f64").forward(obs[:64].astype(np.float32))
    o2 = Oracle(net_bytes(s), Q, "f64").forward(obs[:64].astype(np.float32))
    assert np.abs(o1 - o2).max() <= 1e-9 * max(1.0, np.abs(o1).max())
