"""Data-parallel hook of the trainer: the mean of every rank's gradient before each Adam step.

The reference leaves this as a stub (flyguy/dist.py:1-13, called at fly_native.py:78-81).  Here it is a real
all-reduce over torch.distributed (RCCL on ROCm GPUs, gloo on CPU tensors) when a process group with more than
one rank is initialised, and a no-op otherwise.
"""
from __future__ import annotations

import torch
import torch.distributed as td


def on() -> bool:
    return td.is_available() and td.is_initialized() and td.get_world_size() > 1


def mean_(tensors: list[torch.Tensor]) -> None:
    """In place: each tensor becomes the mean over ranks.  One flat bucket, one all-reduce."""
    if not on() or not tensors:
        return
    flat = torch.cat([t.reshape(-1) for t in tensors])
    td.all_reduce(flat, op=td.ReduceOp.SUM)
    flat /= td.get_world_size()
    at = 0
    for t in tensors:
        n = t.numel()
        t.copy_(flat[at:at + n].view_as(t))
        at += n
