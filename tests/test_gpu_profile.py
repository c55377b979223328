"""fc_profile / fc_profile_read: every stage bracketed by HIP events (on = 1), or one stage alone (on = 2 + s, what
bench.py uses inside its timed region so that the events do not lengthen it)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import lively, toy
from flyguy_amd._lib import LibraryError, call, profile_read
from flyguy_amd.export import params_from_torch, structure
from flyguy_amd.fly import FlyActor
from gpu_helpers import Core, say

pytestmark = pytest.mark.gpu


def test_profile_every_stage_or_one(gpu_lib):
    torch.manual_seed(0)
    f = lively(FlyActor(toy("b"), 517, 90, hops=3, fan=8))
    s = structure(f)
    core = Core(s, params_from_torch(f, s), max_batch=64)
    rng = np.random.default_rng(0)
    obs = torch.as_tensor(rng.standard_normal((64, 517)).astype(np.float32)).cuda()
    tl = torch.as_tensor(rng.standard_normal((64, 90)).astype(np.float32)).cuda()
    say("fc_profile on a toy network, B 64")

    def steps(n):
        for _ in range(n):
            call("fc_teach_step", core.h, obs.data_ptr(), tl.data_ptr(), 64, 1.0, 0.0, 0.0, 0.0, 0.0, 0.999, None)
        torch.cuda.synchronize()

    call("fc_profile", core.h, 1)
    profile_read(core.h, reset=True)
    steps(2)
    every = profile_read(core.h, reset=True)
    for name in ("plug", "hop1 fwd", "hop2 fwd", "hop3 fwd", "logits", "loss", "readout bwd", "hop1 bwd", "hop2 bwd",
                 "hop3 bwd", "adam"):
        assert every[name][1] == 2 and every[name][0] > 0, name
    call("fc_profile", core.h, 2 + 4)             # stage 4: the forward of hop 2
    steps(3)
    one = profile_read(core.h, reset=True)
    assert set(one) == {"hop2 fwd"} and one["hop2 fwd"][1] == 3 and one["hop2 fwd"][0] > 0
    call("fc_profile", core.h, 0)
    steps(1)
    assert profile_read(core.h, reset=True) == {}
    with pytest.raises(LibraryError):
        call("fc_profile", core.h, 2 + 25)       # past the last stage


def test_gather_ceiling(gpu_lib):
    """fc_gather_ceiling (bench.py's gather ceiling): a positive time per line; no smaller for a slab larger than an
    XCD's L2 than for one that fits it (misses cost), nor for two tiles' slabs than for one; rows drawn from a
    connection table (here every connection on row 0: one line, always in the cache) no slower than uniform ones over
    a large slab; bad arguments refused before any device work."""
    import ctypes
    from flyguy_amd._lib import lib

    def ns(rows, tiles=1, row_of=None):
        v = ctypes.c_double(-1.0)
        ptr, n = (row_of.data_ptr(), row_of.numel()) if row_of is not None else (None, 0)
        call("fc_gather_ceiling", rows, tiles, ptr, n, 3, None, ctypes.byref(v))
        return v.value

    small, large, two = ns(1024), ns(200000), ns(100000, 2)
    hot = ns(200000, 1, torch.zeros(4096, dtype=torch.int32, device="cuda"))
    say(f"   gather ceiling: {small:.5f} ns per line (1,024 rows), {large:.5f} (200,000 rows: 25.6 MB), "
        f"{two:.5f} (2 x 100,000), {hot:.5f} (200,000 rows, every draw row 0)")
    assert 0 < small < 1 and np.isfinite(large) and large >= small and two >= small and hot <= large
    v = ctypes.c_double(0.0)
    assert lib().fc_gather_ceiling(0, 1, None, 0, 3, None, ctypes.byref(v)) == -1
    with pytest.raises(LibraryError):
        call("fc_gather_ceiling", 1024, 3, None, 0, 3, None, ctypes.byref(v))
    with pytest.raises(LibraryError):
        call("fc_gather_ceiling", 1024, 1, None, 0, 0, None, ctypes.byref(v))
