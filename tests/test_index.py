"""Graph indexing is bit-exact with the reference (flyguy/fly.py:35-154, flyguy/native/export.py:32-65).

Golden vectors: tests/golden/idx_*.npz were written by tests/golden/make_golden.py from the reference's own
FlyActor and export.write_net on the toy graphs tests/golden/toy_*.npz; shipped_3hop.json holds SHA-256 digests of
every array of the reference's shipped 3-hop graph (checked when the reference checkout is present).
"""
from __future__ import annotations

import hashlib
import json

import numpy as np
import pytest
import torch

from conftest import CASES, GOLDEN, golden, toy
from flyguy_amd.export import net_bytes, structure
from flyguy_amd.fly import FlyActor
from oracle import index as oindex

BUFS = ["e", "r", "c", "crow", "tcrow", "tcol", "tperm", "ci", "tci", "n", "s", "d"]
PLUG = ["in_r", "in_c", "in_crow", "in_tcrow", "in_tcol", "in_tperm", "in_ci", "in_tci", "n0", "dn_rows"]


def _actor(name, hops, fan):
    torch.manual_seed(0)
    return FlyActor(toy(name), 517, 90, hops=hops, fan=fan)


@pytest.mark.parametrize("name,hops,fan", CASES)
def test_buffers_bit_exact(name, hops, fan):
    gv = golden(name, hops, fan)
    f = _actor(name, hops, fan)
    for k in range(1, hops + 1):
        for b in BUFS:
            got, want = getattr(f, f"{b}{k}").numpy(), gv[f"{b}{k}"]
            assert got.dtype == want.dtype and np.array_equal(got, want), f"{b}{k}"
    for b in PLUG:
        got, want = getattr(f, b).numpy(), gv[b]
        assert got.dtype == want.dtype and np.array_equal(got, want), b
    assert f.sizes == gv["sizes"].tolist()
    assert [f.n_neurons, f.n_conn, f.used, f.in_play] == gv["counts"].tolist()


@pytest.mark.parametrize("name,hops,fan", CASES)
def test_initial_parameters_bit_exact(name, hops, fan):
    gv = golden(name, hops, fan)
    sd = _actor(name, hops, fan).state_dict()
    for p in ("w", "gain", "theta", "in_w", "in_b", "out.weight", "out.bias"):
        assert np.array_equal(sd[p].numpy(), gv["param_" + p]), p
    assert list(sd.keys()) == ["w", "gain", "theta", "in_w", "in_b", "out.weight", "out.bias"]


@pytest.mark.parametrize("name,hops,fan", CASES)
def test_structure_and_net_bytes_bit_exact(name, hops, fan):
    gv = golden(name, hops, fan)
    s = structure(_actor(name, hops, fan))
    assert np.array_equal(s["wmap"], gv["wmap"])
    for k, h in enumerate(s["hop"], 1):
        for key in ("widx", "twidx", "drow"):
            assert np.array_equal(h[key], gv[f"st_{key}{k}"]), f"{key}{k}"
    assert net_bytes(s) == gv["net_bin"].tobytes()


@pytest.mark.parametrize("name,hops,fan", CASES)
def test_oracle_index_restatement_matches_golden(name, hops, fan):
    gv = golden(name, hops, fan)
    g = toy(name)
    ix = oindex.index(g, 517, hops, fan)
    for k in range(1, hops + 1):
        for b in BUFS:
            assert list(gv[f"{b}{k}"]) == list(ix[f"{b}{k}"]), f"{b}{k}"
    for b in PLUG:
        assert list(gv[b]) == list(ix[b]), b
    assert ix["sizes"] == gv["sizes"].tolist()
    assert [ix["used"], ix["in_play"]] == gv["counts"].tolist()[2:]
    assert np.array_equal(ix["w"], gv["param_w"])
    s = oindex.structure(ix, len(g["body"]), 517, 90, hops, fan)
    assert oindex.net_bytes(s) == gv["net_bin"].tobytes()


def test_too_many_hops_for_a_trimmed_graph_is_refused():
    with pytest.raises(AssertionError):
        FlyActor(toy("c"), 517, 90, hops=5, fan=4)          # toy c is cut for 4 hops (tests/test_fly.py:131-132)


def test_index_invariants():
    f = _actor("b", 3, 16)
    for k in range(1, 4):
        crow, tcrow = getattr(f, f"crow{k}").numpy(), getattr(f, f"tcrow{k}").numpy()
        r, c, tperm = getattr(f, f"r{k}").numpy(), getattr(f, f"c{k}").numpy(), getattr(f, f"tperm{k}").numpy()
        assert crow[0] == 0 and crow[-1] == len(r) and np.all(np.diff(crow) >= 0)
        assert tcrow[0] == 0 and tcrow[-1] == len(r) and np.all(np.diff(tcrow) >= 0)
        assert np.array_equal(np.sort(tperm), np.arange(len(r)))
        assert np.array_equal(getattr(f, f"tcol{k}").numpy(), r[tperm])
        assert np.all(np.diff(c[tperm]) >= 0)                                # CSC sorted by source
        key = r * (c.max() + 1) + c
        assert np.all(np.diff(key) > 0)                                      # CSR sorted by (target, source), unique


SHIPPED = __import__("pathlib").Path("/root/reference/flyguy/graphs/male_cns_min2_3hop.npz")


@pytest.mark.skipif(not SHIPPED.exists(), reason="the reference checkout (shipped graph) is not here")
def test_shipped_graph_digests():
    """The shipped 3-hop graph: every buffer and the NET.bin match the reference's by SHA-256, and the counts
    match the published ones (70,636 neurons in play is not a buffer; 2,992,734 connections and 3,688,058
    connection steps are: docs/HOW_IT_WORKS.md:53-59, README.md:60-66)."""
    want = json.loads((GOLDEN / "shipped_3hop.json").read_text())
    torch.manual_seed(0)
    f = FlyActor(SHIPPED, 517, 90, hops=3, fan=16)
    assert f.sizes == want["_sizes"] == [16894, 46393, 37748, 1332]
    assert f.used == 3_688_058 and f.in_play == 2_992_734
    h = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()   # noqa: E731
    for k in range(1, 4):
        for b in BUFS:
            assert h(getattr(f, f"{b}{k}").numpy()) == want[f"{b}{k}"], f"{b}{k}"
    for b in PLUG:
        assert h(getattr(f, b).numpy()) == want[b], b
    s = structure(f)
    assert h(s["wmap"]) == want["wmap"]
    assert h(np.frombuffer(net_bytes(s), np.uint8)) == want["net_bin"]
    nid = np.unique(np.concatenate([f.n0.numpy()] + [getattr(f, f"n{k}").numpy() for k in (1, 2, 3)]))
    assert len(nid) == 70_636
