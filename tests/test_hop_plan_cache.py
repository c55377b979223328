"""The HopHip row-plan cache can never hand one structure tensor's plan to another (CPU).

A plan is cached by (address, length, version) of its row pointer.  If the cached tensor were freed, a new tensor of
the same length could be given the same address and receive a plan whose edge ranges belong to another hop; the
kernels would then read and write past that hop's arrays.  The cache therefore holds the tensor itself.
"""
from __future__ import annotations

import gc
import weakref

import numpy as np
import pytest
import torch

from flyguy_amd import fly_hip
from oracle.plan import plan


def test_cache_keeps_its_tensor_alive_and_plans_by_content():
    a = torch.as_tensor(np.concatenate([[0], np.cumsum(np.full(199, 6))]).astype(np.int64))    # 200 entries, E 1194
    ref = weakref.ref(a)
    pa = fly_hip._plan(a, int(a[-1]))
    del a
    gc.collect()
    assert ref() is not None                                  # the cached tensor's memory stays taken
    b = torch.as_tensor(np.concatenate([[0], np.cumsum(np.full(199, 1))]).astype(np.int64))    # same length, E 199
    pb = fly_hip._plan(b, 199)
    seg = pb[0].numpy()
    assert int(seg[:, 2].max()) == 199                        # b's own plan, not a's
    want, _, _ = plan(b.numpy())
    assert [tuple(x) for x in seg.tolist()] == want
    assert pa[0].shape != pb[0].shape or not torch.equal(pa[0], pb[0])


def test_plan_refuses_a_row_pointer_of_other_arrays():
    rp = torch.as_tensor(np.array([0, 3, 5], np.int64))
    with pytest.raises(ValueError):
        fly_hip._plan(rp, 7)
