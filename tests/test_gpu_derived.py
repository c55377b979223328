"""The tables a pass derives from the weights (packed (source, weight) pairs, per-row records, the transposed
read-out weights) are made again only when the weights they came from were written since.  Every kind of write
must show in the next pass: fc_copy into the weights or the running average, an Adam step, a change of stream, and
alternating between the two sets.  Each result is compared bit for bit with a fresh handle given the same weights."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import lively, toy
from flyguy_amd._lib import call
from flyguy_amd.export import params_from_torch, structure
from flyguy_amd.fly import FlyActor
from gpu_helpers import Core, say

pytestmark = pytest.mark.gpu


def _bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("flags", [0, 1])
def test_passes_follow_every_weight_write(gpu_lib, flags):
    torch.manual_seed(3)
    f = lively(FlyActor(toy("b"), 517, 90, hops=3, fan=8), 3)
    s = structure(f)
    p1 = params_from_torch(f, s)
    rng = np.random.default_rng(7)
    p2 = [(p * (1 + 0.25 * rng.standard_normal(p.shape))).astype(np.float32) for p in p1]
    obs = rng.standard_normal((64, 517)).astype(np.float32)
    say(f"derived tables, flags {flags}")

    def fresh(params):
        return Core(s, params, max_batch=64, flags=flags).forward(obs)

    want1, want2 = fresh(p1), fresh(p2)
    assert not np.array_equal(_bits(want1), _bits(want2))
    core = Core(s, p1, max_batch=64, flags=flags)             # weights and running average both p1
    assert np.array_equal(_bits(core.forward(obs)), _bits(want1))
    assert np.array_equal(_bits(core.forward(obs)), _bits(want1))                  # nothing written: same tables
    core.set(0, p2)                                                                # the weights only
    assert np.array_equal(_bits(core.forward(obs)), _bits(want2))
    assert np.array_equal(_bits(core.forward(obs, ema=1)), _bits(want1))           # the average is still p1
    assert np.array_equal(_bits(core.forward(obs)), _bits(want2))
    core.set(1, p2)                                                                # the average too
    assert np.array_equal(_bits(core.forward(obs, ema=1)), _bits(want2))

    # an Adam step writes both sets; the next pass is that of a fresh handle given the stepped arrays
    x = torch.as_tensor(obs).cuda()
    tl = torch.as_tensor(rng.standard_normal((64, 90)).astype(np.float32)).cuda()
    call("fc_teach_step", core.h, x.data_ptr(), tl.data_ptr(), 64, 1.0, 1e-2, 1e-2, 1e-2, 0.0, 0.9, None)
    torch.cuda.synchronize()
    stepped, average = core.get(0), core.get(1)
    assert not np.array_equal(_bits(stepped[0]), _bits(p2[0]))
    assert np.array_equal(_bits(core.forward(obs)), _bits(fresh(stepped)))
    assert np.array_equal(_bits(core.forward(obs, ema=1)), _bits(fresh(average)))

    # a step right after a forward from the running average: its backward must use tables of the weights, so its
    # result is that of a handle that saw no average forward (the same weights, average and Adam state)
    twin = Core(s, stepped, max_batch=64, flags=flags)
    for which in (1, 2, 3):
        twin.set(which, core.get(which))
    call("fc_adam_t", twin.h, call("fc_adam_t", core.h, -1))
    call("fc_teach_step", core.h, x.data_ptr(), tl.data_ptr(), 64, 1.0, 1e-2, 1e-2, 1e-2, 0.0, 0.9, None)
    call("fc_teach_step", twin.h, x.data_ptr(), tl.data_ptr(), 64, 1.0, 1e-2, 1e-2, 1e-2, 0.0, 0.9, None)
    torch.cuda.synchronize()
    for which in (0, 1, 2, 3):
        for a, b in zip(core.get(which), twin.get(which)):
            assert np.array_equal(_bits(a), _bits(b)), which
    assert np.array_equal(_bits(core.forward(obs)), _bits(fresh(core.get(0))))

    # another stream: the tables are made again there
    side = torch.cuda.Stream()
    call("fc_set_stream", core.h, ctypes.c_void_p(side.cuda_stream))
    with torch.cuda.stream(side):
        got = core.forward(obs)
    side.synchronize()
    call("fc_set_stream", core.h, None)
    assert np.array_equal(_bits(got), _bits(fresh(core.get(0))))


@pytest.mark.parametrize("flags", [0, 1])
@pytest.mark.parametrize("name,hops,fan", [("b", 4, 8), ("a", 4, 5)])
def test_teach_step_stores_first_sums_as_its_parts_add_them(gpu_lib, flags, name, hops, fan):
    """A teaching step stores the first sum into each gradient entry instead of adding it to the cleared entry.  On
    networks whose hops share strengths and neurons (an entry summed by several reductions), two steps leave the
    weights, running average and Adam moments bit-identical to zero_grad + backward (which adds) + step."""
    torch.manual_seed(5)
    f = lively(FlyActor(toy(name), 517, 90, hops=hops, fan=fan), 5)
    s = structure(f)
    used = np.concatenate([np.asarray(h["widx"]) for h in s["hop"]])
    assert len(np.unique(used)) < len(used)                    # some strengths are summed in several hops
    params = params_from_torch(f, s)
    B = 128
    rng = np.random.default_rng(11)
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    x = torch.as_tensor(obs).cuda()
    t = torch.as_tensor((2 * rng.standard_normal((B, 90))).astype(np.float32)).cuda()
    say(f"teach step vs its parts, {name} hops {hops} fan {fan}, flags {flags}")
    a = Core(s, params, max_batch=B, flags=flags)
    b = Core(s, params, max_batch=B, flags=flags)
    for _ in range(2):
        call("fc_teach_step", a.h, x.data_ptr(), t.data_ptr(), B, 1.0, 1e-2, 3e-3, 1e-2, 0.0, 0.9, None)
        lg = torch.as_tensor(b.forward(obs)).cuda()
        dl = torch.empty(B, 90, device="cuda")
        st = torch.zeros(2, device="cuda")
        call("fc_kl_loss", b.h, lg.data_ptr(), t.data_ptr(), B, 1.0, dl.data_ptr(), st.data_ptr())
        b.zero_grad()
        b.backward(dl.cpu().numpy())
        call("fc_step", b.h, 1e-2, 3e-3, 1e-2, 0.0, 0.9)
    torch.cuda.synchronize()
    for which in (0, 1, 2, 3):
        for pa, pb in zip(a.get(which), b.get(which)):
            assert np.array_equal(_bits(pa), _bits(pb)), which
