"""The library's row plans equal the plain-Python restatement (oracle/plan.py) bit for bit, and obey the rules'
invariants:
  * fc_plan_rows (one product, no re-drive fields): every edge at exactly one position, each segment's edges in CSR
    order on its group's slots, segments no longer than seg_max and longest first, waves sized by their longest
    segment;
  * fc_net_plan / fc_net_marks (the plans and reduction tables a handle's kernels run, computed on the host from
    NET.bin): on the golden toy networks, the benchmark network at 1/16 and full size, and the shipped network when
    its data files are present, every product's forward and backward plan with its re-drive fields and first-write
    encodings, the backward's column neurons and first-write marks; and the invariants no restatement can share a
    mistake with: among segments of equal length, rows that read a drive line come first and each group keeps
    (row, segment) order; every re-drive field is the hop's drow (forward) or its first-write encoding (backward,
    checked against the order in which the hops write); every gradient entry is marked first exactly once, at its
    first write in the order of reductions."""
from __future__ import annotations

import numpy as np
import pytest

from pathlib import Path

from conftest import CASES
from flyguy_amd._lib import net_marks, net_plan, plan_rows, seg_cap
from flyguy_amd.export import net_bytes, read_net
from flyguy_amd.synth import scaled_3hop, synth_3hop
from oracle import plan as oracle_plan
from oracle.plan import net_plans, plan


def _check(rowptr, seg_max):
    p = plan_rows(rowptr, seg_max)
    want_wave, want_seg, want_split, want_nslot, want_pos = plan(rowptr, seg_max)
    assert [tuple(x) for x in p["wave"].tolist()] == want_wave
    assert [tuple(x) for x in p["seg"].tolist()] == want_seg
    assert [tuple(x) for x in p["split"].tolist()] == want_split
    assert p["nslot"] == want_nslot
    assert np.array_equal(p["pos"], want_pos)
    rows, E = len(rowptr) - 1, int(rowptr[-1])
    pos, seg, wave = p["pos"], p["seg"], p["wave"]
    # every edge exactly once
    used = pos[pos >= 0]
    assert np.array_equal(np.sort(used), np.arange(E))
    # each segment: its edges are a run of one row in CSR order on its group's slots; lengths fall
    seen_rows = np.zeros(rows, np.int64)
    lens = []
    for i, (r, slot, drow, _) in enumerate(seg.tolist()):
        w, g = divmod(i, 8)
        woff, longest = wave[w]
        steps = -(-int(longest) // 8)
        mine = np.array([pos[woff + 64 * j + 8 * g + s] for j in range(steps) for s in range(8)])
        mine = mine[mine >= 0]
        if len(mine):
            assert np.array_equal(mine, np.arange(mine[0], mine[0] + len(mine)))
            assert rowptr[r] <= mine[0] and mine[-1] < rowptr[r + 1]
        assert len(mine) <= seg_max and drow == -1
        # the slots a segment fills are exactly its first len(mine) slots
        flat = np.array([pos[woff + 64 * j + 8 * g + s] for j in range(steps) for s in range(8)])
        assert (flat[:len(mine)] >= 0).all() and (flat[len(mine):] < 0).all()
        lens.append(len(mine))
        seen_rows[r] += 1
    assert np.all(seen_rows >= 1)                           # empty rows still get a segment (their output is written)
    assert np.all(np.diff(lens) <= 0)
    for w, (woff, longest) in enumerate(wave.tolist()):
        assert longest == max(lens[8 * w:8 * w + 8])
        end = wave[w + 1][0] if w + 1 < len(wave) else len(pos)
        assert end - woff == 64 * (-(-longest // 8))
    slots = sorted(s for s in seg[:, 1].tolist() if s >= 0)
    assert slots == list(range(p["nslot"]))


@pytest.mark.parametrize("seed", range(5))
def test_plan_random(seed):
    rng = np.random.default_rng(seed)
    d = rng.lognormal(0, 2.0, 300).astype(np.int64)
    d[rng.choice(300, 20)] = 0
    rowptr = np.concatenate([[0], np.cumsum(d)])
    for seg_max in (1, 7, 64, 256):
        _check(rowptr, seg_max)


def test_plan_edge_cases():
    _check(np.array([0]), 256)                              # no rows
    _check(np.array([0, 0, 0]), 256)                        # rows without edges
    _check(np.array([0, 256, 257, 1000]), 256)              # exactly seg_max, seg_max+1
    _check(np.array([0, 9, 18, 27, 36, 45, 54, 63, 72, 81]), 16)   # a ninth segment starts a second wave


def test_plan_synthetic_graph():
    s, _ = scaled_3hop(16)
    for h in s["hop"]:
        E = int(h["crow"][-1])
        _check(np.asarray(h["crow"]), seg_cap(E))
        _check(np.asarray(h["tcrow"]), seg_cap(E))


def test_seg_cap():
    for E in (0, 1, 65_536, 65_537, 292_734, 1_200_000, 1_500_000, 2_569_085, 10 ** 9):
        assert seg_cap(E) == oracle_plan.seg_cap(E)
    assert seg_cap(0) == 16 and seg_cap(292_734) == 72 and seg_cap(600_000) == 147 and seg_cap(1_200_000) == 293
    assert seg_cap(1_500_000) == 367 and seg_cap(10 ** 9) == 512


def test_whole_connectome_generator_small():
    """The whole-connectome generator at a small size: the counts asked for, no repeated (pre, post) pair, disjoint
    sensory and descending sets, and a graph FlyActor indexes."""
    from flyguy_amd.fly import FlyActor
    from flyguy_amd.synth import whole_connectome
    g = whole_connectome(neurons=3000, connections=90_000, sensory=400, descending=60, seed=1)
    assert len(g["pre"]) == 90_000 and len(g["body"]) == 3000
    key = g["pre"].astype(np.int64) * 3000 + g["post"]
    assert len(np.unique(key)) == len(key)
    assert not set(g["sensory"].tolist()) & set(g["descending"].tolist())
    assert not np.all(np.diff(g["post"]) >= 0)                      # connections in random order
    f = FlyActor(g, 517, 90, hops=3, fan=16)
    assert f.sizes[0] == 400 and 0 < f.sizes[3] <= 60


# ------------------------------------------------------------------------------------------------ a network's plans
def _same_plan(got: dict, want) -> None:
    wave, seg, split, nslot, pos = want
    assert [tuple(x) for x in got["wave"].tolist()] == wave
    assert [tuple(x) for x in got["seg"].tolist()] == seg
    assert [tuple(x) for x in got["split"].tolist()] == split
    assert got["nslot"] == nslot
    assert np.array_equal(got["pos"], pos)


def _tie_break(p: dict, field_reads) -> None:
    """Among segments of equal length: the whole rows that read a drive line first, each part in (row, seg) order."""
    seg, pos = p["seg"], p["pos"]
    rows, slots, fields = seg[:, 0], seg[:, 1], seg[:, 2]
    reads = np.array([slots[i] < 0 and field_reads(int(fields[i])) for i in range(len(seg))], bool)
    # segment lengths from the positions: a wave's 8 groups take 8 consecutive positions of each 64
    length = np.zeros(len(seg), np.int64)
    for w, (woff, longest) in enumerate(p["wave"].tolist()):
        steps = -(-longest // 8)
        block = pos[woff:woff + 64 * steps].reshape(steps, 8, 8)             # [step][group][slot]
        n = (block >= 0).sum(axis=(0, 2))
        cnt = min(8, len(seg) - 8 * w)
        length[8 * w:8 * w + cnt] = n[:cnt]
    assert np.all(np.diff(length) <= 0)
    for L in np.unique(length):
        at = np.flatnonzero(length == L)
        r = reads[at]
        assert np.all(np.diff(r.astype(int)) <= 0), L                       # readers, then the others
        for part in (at[r], at[~r]):
            key = rows[part].astype(np.int64) * (1 << 20) + np.where(slots[part] < 0, 0, slots[part] + 1)
            assert np.all(np.diff(key) > 0), L


def _check_network(s: dict) -> None:
    raw = net_bytes(s)
    want = net_plans(read_net(raw))
    K = s["hops"]
    _same_plan(net_plan(raw, 0), want["plug"])
    # which hop writes each sensory row's drive gradient first, hops from the top down
    first_writer = {}
    for k in range(K - 1, -1, -1):
        for d in np.asarray(s["hop"][k]["drow"]):
            if d >= 0:
                first_writer.setdefault(int(d), k)
    for k in range(K):
        h = s["hop"][k]
        fwd, bwd = net_plan(raw, k + 1), net_plan(raw, k + 1, backward=True)
        _same_plan(fwd, want["fwd"][k])
        _same_plan(bwd, want["bwd"][k])
        drow = np.asarray(h["drow"])
        assert np.array_equal(fwd["seg"][:, 2], drow[fwd["seg"][:, 0]])
        _tie_break(fwd, lambda f: f >= 0)
        # the backward's rows are layer k: the sensory rows (k = 0), else hop k's rows with hop k's drow
        below = np.asarray(s["hop"][k - 1]["drow"]) if k >= 1 else None
        for r, f in zip(bwd["seg"][:, 0].tolist(), bwd["seg"][:, 2].tolist()):
            if k == 0:
                assert f == (-1 if r in first_writer else -2)
            else:
                d = int(below[r])
                assert f == (-1 if d < 0 else (-(d + 3) if first_writer[d] == k - 1 else d))
        _tie_break(bwd, lambda f: f >= 0)
        assert np.array_equal(net_marks(raw, k + 1, 0), want["gidx"][k])
        assert np.array_equal(net_marks(raw, k + 1, 1), want["ridx"][k])
        assert np.array_equal(net_marks(raw, k + 1, 2), want["gridx"][k])
    top = net_marks(raw, 0, 3)
    assert np.array_equal(top, want["top"])
    # every gradient entry marked first exactly once, at its first write in the order of reductions
    for marks in ([top] + [want["gridx"][k] for k in range(K - 1, -1, -1)],
                  [want["ridx"][k] for k in range(K - 1, -1, -1)]):
        flat = np.concatenate([np.asarray(m, np.int64) for m in marks])
        live = flat != -1
        entry = np.where(flat >= 0, flat, -flat - 2)[live]
        is_first = flat[live] < -1
        _, first_at = np.unique(entry, return_index=True)
        assert np.array_equal(np.sort(np.flatnonzero(is_first)), np.sort(first_at))


@pytest.mark.parametrize("name,hops,fan", CASES)
def test_net_plans_on_the_golden_toys(name, hops, fan):
    from flyguy_amd.fly import FlyActor
    from conftest import toy
    import torch
    torch.manual_seed(0)
    f = FlyActor(toy(name), 517, 90, hops=hops, fan=fan)
    from flyguy_amd.export import structure
    _check_network(structure(f))


def test_net_plans_on_the_benchmark_network_small():
    s, _ = scaled_3hop(16)
    _check_network(s)


def test_net_plans_on_the_benchmark_network():
    s, _ = synth_3hop()
    _check_network(s)


SHIPPED = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "shipped" / "male_cns_min2_3hop.npz"


@pytest.mark.skipif(not SHIPPED.exists(), reason="the shipped graph is not in oracle/_ref/shipped")
def test_net_plans_on_the_shipped_network():
    import torch
    from flyguy_amd.export import structure
    from flyguy_amd.fly import FlyActor
    torch.manual_seed(0)
    _check_network(structure(FlyActor(str(SHIPPED), 517, 90, hops=3, fan=16)))


def test_net_plan_refuses_bad_arguments():
    s, _ = scaled_3hop(16)
    raw = net_bytes(s)
    from flyguy_amd._lib import LibraryError
    for product, backward in ((0, True), (4, False), (-1, False)):
        with pytest.raises(LibraryError):
            net_plan(raw, product, backward)
    with pytest.raises(LibraryError):
        net_plan(b"FLY0" + raw[4:], 1)
    with pytest.raises(LibraryError):
        net_marks(raw, 0, 1)


def test_a_strength_joins_the_same_neurons_in_every_hop():
    """A network in which one strength stands for two different connections (other source or target neuron in another
    hop) is refused: the revive surgery and the first-write marks take a strength's neurons from any of its hops."""
    from flyguy_amd._lib import LibraryError
    s, _ = scaled_3hop(16)
    h1, h2 = s["hop"][0], s["hop"][1]
    w_new, w_old = int(h1["widx"][0]), int(h2["widx"][0])
    h2["widx"] = np.asarray(h2["widx"]).copy()
    h2["twidx"] = np.asarray(h2["twidx"]).copy()
    h2["widx"][0] = w_new
    h2["twidx"][h2["twidx"] == w_old] = w_new
    with pytest.raises(LibraryError, match="joins different neurons"):
        net_plan(net_bytes(s), 1)
