"""The HopHip plan cache can never hand one structure's plan to another (CPU).

A plan is cached by (address, length, version) of its row pointer and index arrays.  If a cached tensor were freed,
a new tensor of the same length could be given the same address and receive a plan whose positions belong to another
hop; the kernels would then read and write past that hop's arrays.  The cache therefore holds the tensors themselves.
"""
from __future__ import annotations

import gc
import weakref

import numpy as np
import pytest
import torch

from flyguy_amd import fly_hip
from flyguy_amd._lib import NO_ROW, seg_cap
from oracle.plan import plan


def _rowptr(deg, rows=199):
    return torch.as_tensor(np.concatenate([[0], np.cumsum(np.full(rows, deg))]).astype(np.int64))


def test_cache_keeps_its_tensors_alive_and_plans_by_content():
    a = _rowptr(6)                                            # 200 entries, E 1194
    ca = torch.arange(1194, dtype=torch.int32) % 50
    ref = weakref.ref(a)
    pa = fly_hip._plan(a, ca, None, int(a[-1]))
    del a
    gc.collect()
    assert ref() is not None                                  # the cached tensor's memory stays taken
    b = _rowptr(1)                                            # same length, E 199
    cb = torch.arange(199, dtype=torch.int32) % 7
    pb = fly_hip._plan(b, cb, None, 199)
    want_wave, want_seg, _, _, want_pos = plan(b.numpy(), seg_cap(199))
    assert [tuple(x) for x in pb["wave"].tolist()] == want_wave            # b's own plan, not a's
    assert [tuple(x) for x in pb["seg"].tolist()] == want_seg
    pos = np.array(want_pos)
    assert pb["pidx"].tolist() == want_pos.tolist()           # weight index = the edge itself
    assert pb["pcol"].tolist() == [int(cb[e]) if e >= 0 else NO_ROW for e in pos]
    assert pa["npos"] != pb["npos"] or not torch.equal(pa["pcol"], pb["pcol"])


def test_transposed_plan_maps_positions_through_tperm():
    rp = torch.as_tensor(np.array([0, 3, 5, 5, 9], np.int64))
    tcol = torch.as_tensor(np.array([4, 1, 2, 0, 3, 1, 1, 2, 0], np.int32))
    tperm = torch.as_tensor(np.array([8, 7, 6, 5, 4, 3, 2, 1, 0], np.int64))
    d = fly_hip._plan(rp, tcol, tperm, 9)
    _, _, _, _, pos = plan(rp.numpy(), seg_cap(9))
    assert d["pidx"].tolist() == [int(tperm[e]) if e >= 0 else -1 for e in pos]
    assert d["pcol"].tolist() == [int(tcol[e]) if e >= 0 else NO_ROW for e in pos]


def test_plan_refuses_a_row_pointer_of_other_arrays():
    rp = torch.as_tensor(np.array([0, 3, 5], np.int64))
    with pytest.raises(ValueError):
        fly_hip._plan(rp, torch.zeros(7, dtype=torch.int32), None, 7)
