"""The library's row plan (fc_plan_segments, host code) equals the plain-Python restatement bit for bit, and obeys
the rule's invariants: every edge in exactly one segment, segments no longer than seg_max, longest first."""
from __future__ import annotations

import numpy as np
import pytest

from flyguy_amd._lib import plan_segments
from flyguy_amd.synth import scaled_3hop
from oracle.plan import plan


def _check(rowptr, seg_max):
    seg, split, nslot = plan_segments(rowptr, seg_max)
    want_seg, want_split, want_nslot = plan(rowptr, seg_max)
    assert [tuple(x) for x in seg.tolist()] == want_seg
    assert [tuple(x) for x in split.tolist()] == want_split
    assert nslot == want_nslot
    rows = len(rowptr) - 1
    cover = np.zeros(int(rowptr[-1]), np.int64)
    seen_rows = np.zeros(rows, np.int64)
    for r, b, e, slot in seg.tolist():
        assert rowptr[r] <= b <= e <= rowptr[r + 1] and e - b <= seg_max
        cover[b:e] += 1
        seen_rows[r] += 1
    assert np.all(cover == 1)
    assert np.all(seen_rows >= 1)                           # empty rows still get a segment (their output is written)
    lens = seg[:, 2] - seg[:, 1]
    assert np.all(np.diff(lens) <= 0)
    slots = sorted(s for s in seg[:, 3].tolist() if s >= 0)
    assert slots == list(range(nslot))


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


def test_plan_synthetic_graph():
    s, _ = scaled_3hop(16)
    for h in s["hop"]:
        _check(np.asarray(h["crow"]), 256)
        _check(np.asarray(h["tcrow"]), 256)
