"""The data-parallel gradient hook (flyguy_amd/dist.py; the reference's stub flyguy/dist.py:1-13, called at
fly_native.py:78-81) on the CPU: two gloo ranks on 127.0.0.1, each with its own gradients, end with the mean of
both in every array, in place; without a process group the hook changes nothing."""
from __future__ import annotations

import socket

import torch
import torch.distributed as td
import torch.multiprocessing as mp

from flyguy_amd import dist


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _rank(rank: int, world: int, port: int, out) -> None:
    td.init_process_group("gloo", init_method=f"tcp://127.0.0.1:{port}", rank=rank, world_size=world)
    try:
        g = torch.Generator().manual_seed(100 + rank)
        grads = [torch.randn(7, generator=g), torch.randn(3, 5, generator=g), torch.randn(1, generator=g)]
        views = [t.view(-1) for t in grads]
        assert dist.on()
        dist.mean_(grads)
        out[rank] = [t.clone() for t in grads]
        assert all(v.data_ptr() == t.data_ptr() for v, t in zip(views, grads))      # in place
    finally:
        td.destroy_process_group()


def test_mean_over_two_gloo_ranks():
    world, port = 2, _free_port()
    with mp.Manager() as m:
        out = m.dict()
        mp.spawn(_rank, args=(world, port, out), nprocs=world, join=True)
        got = {r: out[r] for r in range(world)}
    want = []
    for i in range(3):
        parts = []
        for r in range(world):
            g = torch.Generator().manual_seed(100 + r)
            arrs = [torch.randn(7, generator=g), torch.randn(3, 5, generator=g), torch.randn(1, generator=g)]
            parts.append(arrs[i])
        want.append((parts[0] + parts[1]) / 2)
    for r in range(world):
        for a, b in zip(got[r], want):
            assert torch.allclose(a, b, atol=1e-7, rtol=0)
    for a, b in zip(got[0], got[1]):                     # every rank holds the same mean
        assert torch.equal(a, b)


def test_no_process_group_is_a_no_op():
    assert not dist.on()
    t = [torch.arange(4.0)]
    dist.mean_(t)
    assert torch.equal(t[0], torch.arange(4.0))
