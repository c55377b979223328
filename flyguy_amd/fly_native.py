"""The fly actor with its hops, their backward pass and Adam in the MI355X library (flyguy_amd/libflyguy_core.so).

Interface of the reference's flyguy/fly_native.py:37-226: NativeFlyActor IS a FlyActor (same weights, same
checkpoint keys), `native_adam()` returns the optimiser the learner uses, gradients are ADDED in the library
until zero_grad, and after every step the weights are copied back into the PyTorch tensors.  Batches are padded
to a multiple of 32 (the last row repeated) and cut into pieces of `max_batch`; the backward of a batch of
several pieces runs each piece's forward again, since only the last piece's states stay in the library.

Differences from the reference, all on failure paths: on a GPU a missing library is an error (the reference
quietly fell back to the PyTorch path), and the library's errors surface as exceptions instead of ending the
process.  On the CPU the actor behaves exactly as FlyActor.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import dist
from ._lib import call, lib
from .export import net_bytes, structure
from .fly import FlyActor


class _NativeLogits(torch.autograd.Function):
    @staticmethod
    def forward(ctx, obs, hook, actor):
        ctx.actor, ctx.obs = actor, obs
        out = actor._run(obs)
        ctx.gen = actor._gen                    # the states of the last piece are still in the library
        return out

    @staticmethod
    def backward(ctx, g):
        a = ctx.actor
        n, mb = ctx.obs.shape[0], a.max_batch
        for i in range(0, n, mb):
            if not (n <= mb and a._gen == ctx.gen):     # several pieces, or something ran in between: states again
                a._piece(ctx.obs[i:i + mb])
            gi = g[i:i + mb]
            pad = (-gi.shape[0]) % 32
            if pad:
                gi = torch.cat([gi, gi.new_zeros(pad, gi.shape[1])])
            gi = gi.contiguous().float()
            a._sync_stream()
            call("fc_backward", a._core, gi.data_ptr(), gi.shape[0])
        return None, None, None


class NativeAdam:
    """The actor's optimiser as the learner sees it; the work is done in the library (fly_native.py:61-102)."""

    def __init__(self, actor: "NativeFlyActor", lr: float, max_norm: float = 0.0, ema: float = 0.999):
        self.actor, self.max_norm, self.ema = actor, max_norm, ema
        self.param_groups = [{"lr": lr}]
        self.grad_norm = 0.0

    def zero_grad(self, set_to_none: bool = True) -> None:
        a = self.actor
        if a._ready():
            a._sync_stream()
            call("fc_zero_grad", a._core)

    def step(self) -> None:
        a = self.actor
        if not a._ready():
            return
        if dist.on():                            # several ranks: the mean of every rank's gradient
            g = a._fetch(4)
            dist.mean_(g)
            a._store(4, g)
        lr = float(self.param_groups[0]["lr"])
        a._sync_stream()
        self.grad_norm = float(call("fc_step", a._core, lr, lr * a.lr_neuron, lr * a.lr_plug, float(self.max_norm),
                                    float(self.ema)))
        a.pull()

    def state_dict(self) -> dict:
        a = self.actor
        if not a._ready():
            return {"native": True, "adam_t": 0}
        out = {"native": True, "adam_t": int(call("fc_adam_t", a._core, -1))}
        for name, which in (("ema", 1), ("m", 2), ("v", 3)):
            out[name] = [t.cpu() for t in a._fetch(which)]
        return out

    def load_state_dict(self, d: dict) -> None:
        a = self.actor
        if not d.get("native") or "m" not in d or not a._ready():
            return
        for name, which in (("ema", 1), ("m", 2), ("v", 3)):
            a._store(which, [t.to(a.gain.device) for t in d[name]])
        call("fc_adam_t", a._core, int(d.get("adam_t", 0)))
        a._avg_follows = False                   # its own running average came with the state


class NativeFlyActor(FlyActor):
    lr_neuron, lr_plug = 0.3, 1.0               # rates of gain / threshold and of the plugs, as shares of W's

    def __init__(self, *args, max_batch: int = 2048, **kw):
        super().__init__(*args, **kw)
        self.max_batch = int(max_batch)
        self._core = None
        self._stream = None
        self._gen, self._stale, self._hook_t = 0, True, None
        self._avg_follows = True

    def __deepcopy__(self, memo):
        """A copy is a plain FlyActor with the same weights: two objects never share one library network."""
        import copy
        new = FlyActor.__new__(FlyActor)
        memo[id(self)] = new
        for k, v in self.__dict__.items():
            if k not in ("_core", "_stream", "_hook_t", "_wmap", "_w_play", "_gen", "_stale", "_avg_follows", "max_batch"):
                new.__dict__[k] = copy.deepcopy(v, memo)
        return new

    def __del__(self):
        core = getattr(self, "_core", None)
        if core is not None:
            try:
                lib().fc_free(core)
            except Exception:
                pass

    # ---- the library
    def _ready(self) -> bool:
        if self._core is not None:
            return True
        if not self.gain.is_cuda:
            return False
        torch.cuda.synchronize()
        s = structure(self)
        raw = net_bytes(s)
        core = lib().fc_create_from_memory(raw, len(raw), self.max_batch)
        if not core:
            call("fc_create_from_memory")
            raise RuntimeError("fc_create_from_memory failed")
        sizes = (ctypes.c_longlong * 10)()
        lib().fc_sizes(core, sizes)
        dev = self.gain.device
        self._wmap = torch.as_tensor(s["wmap"], device=dev)
        self._w_play = torch.empty(len(s["wmap"]), device=dev)
        if [int(v) for v in sizes[:7]] != [t.numel() for t in self._tensors()]:
            lib().fc_free(core)
            raise RuntimeError("the library's network is not this actor's")
        self._core = core
        self._hook_t = torch.zeros(1, device=dev, requires_grad=True)
        self._sync_stream()
        self.push(also_average=True)
        return True

    def _sync_stream(self) -> None:
        """The library's work goes on PyTorch's current stream, so it is ordered with PyTorch's own."""
        s = torch.cuda.current_stream(self.gain.device).cuda_stream
        if s != self._stream:
            lib().fc_set_stream(self._core, s)
            self._stream = s

    def _tensors(self) -> list[torch.Tensor]:
        return [self._w_play, self.gain.data, self.theta.data, self.in_w.data, self.in_b.data, self.out.weight.data,
                self.out.bias.data]

    def _ptrs(self, tensors):
        assert all(t.is_cuda and t.is_contiguous() and t.dtype == torch.float32 for t in tensors)
        return (ctypes.c_void_p * 7)(*[t.data_ptr() for t in tensors])

    def push(self, also_average: bool = False) -> None:
        """PyTorch's weights -> the library (after a checkpoint was loaded)."""
        self._w_play.copy_(self.w.data[self._wmap])
        self._sync_stream()
        call("fc_copy", self._core, 0, 1, self._ptrs(self._tensors()))
        if also_average:
            call("fc_copy", self._core, 1, 1, self._ptrs(self._tensors()))
        self._stale = False

    def pull(self) -> None:
        """The library's weights -> PyTorch's (after every optimiser step)."""
        self._sync_stream()
        call("fc_copy", self._core, 0, 0, self._ptrs(self._tensors()))
        self.w.data[self._wmap] = self._w_play

    def _fetch(self, which: int) -> list[torch.Tensor]:
        out = [torch.empty_like(t) for t in self._tensors()]
        self._sync_stream()
        call("fc_copy", self._core, which, 0, self._ptrs(out))
        return out

    def _store(self, which: int, tensors: list[torch.Tensor]) -> None:
        ts = [t.contiguous().float() for t in tensors]
        self._sync_stream()
        call("fc_copy", self._core, which, 1, self._ptrs(ts))

    def _load_from_state_dict(self, *a, **k):
        super()._load_from_state_dict(*a, **k)
        self._stale = True

    def native_adam(self, lr: float, max_norm: float = 0.0) -> NativeAdam | None:
        return NativeAdam(self, lr, max_norm) if self._ready() else None

    # ---- forward
    def _piece(self, obs: torch.Tensor) -> torch.Tensor:
        b = obs.shape[0]
        pad = (-b) % 32
        x = obs if not pad else torch.cat([obs, obs[-1:].expand(pad, -1)])
        x = x.contiguous()
        out = torch.empty(x.shape[0], self.out.out_features, device=x.device)
        self._sync_stream()
        call("fc_forward", self._core, x.data_ptr(), x.shape[0], out.data_ptr(), 0)
        self._gen += 1
        return out[:b]

    def _run(self, obs: torch.Tensor) -> torch.Tensor:
        if self._stale:
            self.push(also_average=self._avg_follows)
        if obs.shape[0] <= self.max_batch:
            return self._piece(obs)
        return torch.cat([self._piece(obs[i:i + self.max_batch]) for i in range(0, obs.shape[0], self.max_batch)])

    def forward(self, obs: torch.Tensor, extra: torch.Tensor | None = None) -> torch.Tensor:
        if not obs.is_cuda:
            return super().forward(obs, extra)
        if not self._ready():
            raise RuntimeError("NativeFlyActor: observations are on the GPU but the actor's weights are not")
        obs = obs.float()
        if torch.is_grad_enabled():
            return _NativeLogits.apply(obs, self._hook_t, self)
        return self._run(obs)


def grad_arrays(actor: NativeFlyActor) -> list[np.ndarray]:
    """The gradient the library has gathered since zero_grad (for checks against PyTorch's own)."""
    return [t.cpu().numpy() for t in actor._fetch(4)]
