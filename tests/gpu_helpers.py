"""Helpers of the GPU tests: the C-ABI driven directly with PyTorch device tensors, and comparison measures."""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from flyguy_amd._lib import call, lib
from flyguy_amd.export import net_bytes, param_sizes

NAMES = ("W", "gain", "theta", "in_w", "in_b", "out_w", "out_b")


def rel(a, b) -> float:
    """max |a - b| / max |b| (relative to the largest entry, as flyguy/native/core_check.py:59 measures)."""
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)) if b.size else 0.0


def say(*a):
    print(*a, flush=True)


class Core:
    """One library handle (fc_create_from_memory) with the seven weight arrays set from numpy."""

    def __init__(self, s: dict, params: list[np.ndarray], max_batch: int, flags: int = 0):
        raw = net_bytes(s)
        self.s = s
        self.h = lib().fc_create_ex(raw, len(raw), max_batch, flags)
        if not self.h:
            call("fc_create_ex")
        self.sizes = param_sizes(s)
        self.set(0, params)
        self.set(1, params)

    def __del__(self):
        if getattr(self, "h", None):
            lib().fc_free(self.h)

    def _ptrs(self, ts):
        return (ctypes.c_void_p * 7)(*[t.data_ptr() for t in ts])

    def set(self, which: int, arrs) -> None:
        ts = [torch.as_tensor(np.ascontiguousarray(a, np.float32).reshape(-1)).cuda() for a in arrs]
        assert [t.numel() for t in ts] == self.sizes
        call("fc_copy", self.h, which, 1, self._ptrs(ts))

    def get(self, which: int) -> list[np.ndarray]:
        ts = [torch.empty(n, device="cuda") for n in self.sizes]
        call("fc_copy", self.h, which, 0, self._ptrs(ts))
        return [t.cpu().numpy() for t in ts]

    def forward(self, obs: np.ndarray, ema: int = 0) -> np.ndarray:
        x = torch.as_tensor(np.ascontiguousarray(obs, np.float32)).cuda()
        out = torch.empty(x.shape[0], self.s["n_act"], device="cuda")
        call("fc_forward", self.h, x.data_ptr(), x.shape[0], out.data_ptr(), ema)
        return out.cpu().numpy()

    def zero_grad(self):
        call("fc_zero_grad", self.h)

    def backward(self, dl: np.ndarray) -> None:
        d = torch.as_tensor(np.ascontiguousarray(dl, np.float32)).cuda()
        call("fc_backward", self.h, d.data_ptr(), d.shape[0])
        torch.cuda.synchronize()

    def state(self, layer: int, what: int, rows: int, B: int) -> np.ndarray:
        out = torch.empty(rows, B, device="cuda")
        call("fc_export_state", self.h, layer, what, out.data_ptr(), B)
        return out.cpu().numpy()


def argmax_agrees(got: np.ndarray, want: np.ndarray, margin: float = 1e-4) -> tuple[bool, int]:
    """Argmax identical on every sample whose top-2 margin (in want) exceeds `margin`; returns (ok, near ties)."""
    top2 = np.sort(want, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > margin
    ok = bool(np.all(got.argmax(1)[clear] == want.argmax(1)[clear]))
    return ok, int((~clear).sum())
