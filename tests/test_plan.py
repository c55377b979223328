"""The library's row plan (fc_plan_rows, host code) equals the plain-Python restatement bit for bit, and obeys
the rule's invariants: every edge at exactly one position, each segment's edges in CSR order on its group's slots,
segments no longer than seg_max and longest first, waves sized by their longest segment."""
from __future__ import annotations

import numpy as np
import pytest

from flyguy_amd._lib import plan_rows, seg_cap
from flyguy_amd.synth import scaled_3hop
from oracle.plan import plan


def _check(rowptr, seg_max):
    p = plan_rows(rowptr, seg_max)
    want_wave, want_seg, want_split, want_nslot, want_pos = plan(rowptr, seg_max)
    assert [tuple(x) for x in p["wave"].tolist()] == want_wave
    assert [tuple(x) for x in p["seg"].tolist()] == want_seg
    assert [tuple(x) for x in p["split"].tolist()] == want_split
    assert p["nslot"] == want_nslot
    assert p["pos"].tolist() == want_pos
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
