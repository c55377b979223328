"""NativeFlyActor: the fly actor whose forward pass, backward pass and Adam run in the MI355X library
(flyguy_amd/libflyguy_core.so, the fc_* C-ABI of include/flyguy_core.h).

The interface is that of the reference's flyguy/fly_native.py:37-226, so a learner written against it runs
unchanged:
  - NativeFlyActor IS a FlyActor: the same weights and checkpoint keys; a checkpoint loads into either class, and on
    the CPU it behaves exactly as a FlyActor;
  - on a GPU, forward() evaluates the network in the library (with gradients enabled, as an autograd node whose
    backward hands the logits' gradient to the library, which ADDS the weights' gradients to its own buffers);
  - native_adam() is the optimiser: zero_grad / step (three rates: strengths, neurons at lr_neuron of the rate, plugs
    at lr_plug), and after every step the weights are copied back into the PyTorch tensors; state_dict carries the
    library's Adam moments and running average;
  - a deep copy is a plain FlyActor, so two Python objects never share one network in the library.

How a batch meets the library: the library takes batches that are a multiple of 32 samples and at most
`max_batch`.  A batch is cut into pieces of at most max_batch; a piece whose length is not a multiple of 32 is
padded by repeating its last observation (forward) and with zero rows (backward: padded samples then add
nothing).  The library keeps the states of the last piece it evaluated only; the backward of a batch evaluated in
several pieces, or of one whose states were replaced by a later forward, evaluates each piece again first.

Differences from the reference, on failure paths only: on a GPU a missing library is an error (the reference fell
back to PyTorch quietly), and errors the library reports surface as exceptions (the reference's library ended the
process).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import dist
from ._lib import call, lib
from .export import net_bytes, structure
from .fly import FlyActor

TILE = 32                      # the library's batch granule (samples per tile)

# fc_copy's sets
WEIGHTS, AVERAGE, ADAM_M, ADAM_V, GRADIENT = 0, 1, 2, 3, 4


def _tile_up(n: int) -> int:
    return -(-n // TILE) * TILE


def _pieces(n: int, cap: int) -> list[slice]:
    """A batch of n samples as consecutive slices of at most cap samples."""
    return [slice(i, min(i + cap, n)) for i in range(0, n, cap)]


class _Session:
    """The library network of one actor: its handle, the stream its work is queued on, and where the seven weight
    arrays live on the PyTorch side (the strengths in play are a gathered copy of actor.w through wmap)."""

    def __init__(self, actor: FlyActor, max_batch: int):
        torch.cuda.synchronize()
        s = structure(actor)
        raw = net_bytes(s)
        handle = lib().fc_create_from_memory(raw, len(raw), max_batch)
        if not handle:
            call("fc_create_from_memory")
            raise RuntimeError("fc_create_from_memory failed")
        self.handle = handle
        self.stream = None
        self.evaluations = 0               # forward passes run so far (the library holds the last one's states)
        dev = actor.gain.device
        self.wmap = torch.as_tensor(np.asarray(s["wmap"], np.int64), device=dev)
        self.w_play = torch.empty(len(s["wmap"]), device=dev)
        counts = (ctypes.c_longlong * 10)()
        lib().fc_sizes(handle, counts)
        if [int(v) for v in counts[:7]] != [t.numel() for t in self.arrays(actor)]:
            self.close()
            raise RuntimeError("the library's network is not this actor's")

    def close(self) -> None:
        if self.handle is not None:
            lib().fc_free(self.handle)
            self.handle = None

    def arrays(self, actor: FlyActor) -> list[torch.Tensor]:
        """The PyTorch tensors the library exchanges with, in fc_copy's order: the gathered in-play strengths, gain,
        theta, in_w, in_b, out.weight, out.bias."""
        return [self.w_play, actor.gain.data, actor.theta.data, actor.in_w.data, actor.in_b.data, actor.out.weight.data,
                actor.out.bias.data]

    def on_current_stream(self, device) -> None:
        """Queue the library's work on PyTorch's current stream, so it is ordered with PyTorch's own."""
        s = torch.cuda.current_stream(device).cuda_stream
        if s != self.stream:
            lib().fc_set_stream(self.handle, s)
            self.stream = s

    def transfer(self, which: int, tensors: list[torch.Tensor], into_library: bool) -> None:
        for t in tensors:
            if not (t.is_cuda and t.is_contiguous() and t.dtype == torch.float32):
                raise ValueError("the library exchanges contiguous float32 device tensors")
        self.on_current_stream(tensors[0].device)
        ptrs = (ctypes.c_void_p * 7)(*[t.data_ptr() for t in tensors])
        call("fc_copy", self.handle, which, 1 if into_library else 0, ptrs)

    def evaluate(self, obs: torch.Tensor, n_act: int) -> torch.Tensor:
        """Logits of one piece (at most max_batch samples), padded to the tile granule by repeating the last row."""
        n = obs.shape[0]
        pad = _tile_up(n) - n
        x = torch.cat([obs, obs[-1:].expand(pad, obs.shape[1])]) if pad else obs
        x = x.contiguous()
        logits = torch.empty(x.shape[0], n_act, device=x.device)
        self.on_current_stream(x.device)
        call("fc_forward", self.handle, x.data_ptr(), x.shape[0], logits.data_ptr(), 0)
        self.evaluations += 1
        return logits[:n]

    def backpropagate(self, grad: torch.Tensor) -> None:
        """The logits' gradient of the last evaluated piece (zero rows pad it to the granule); adds to the gradient."""
        n = grad.shape[0]
        pad = _tile_up(n) - n
        g = grad.float()
        if pad:
            g = torch.cat([g, g.new_zeros(pad, g.shape[1])])
        g = g.contiguous()
        self.on_current_stream(g.device)
        call("fc_backward", self.handle, g.data_ptr(), g.shape[0])


class _LibraryLogits(torch.autograd.Function):
    """logits = the library's forward of obs.  `anchor` is a parameter-like leaf that requires a gradient, so the
    node is recorded even though the weights live in the library; its gradient is None."""

    @staticmethod
    def forward(ctx, obs, anchor, actor):
        logits = actor._evaluate(obs)
        ctx.actor, ctx.obs = actor, obs
        ctx.ticket = actor._session.evaluations          # which forward's states the library holds now
        return logits

    @staticmethod
    def backward(ctx, grad):
        actor, obs = ctx.actor, ctx.obs
        sess = actor._session
        pieces = _pieces(obs.shape[0], actor.max_batch)
        states_kept = len(pieces) == 1 and sess.evaluations == ctx.ticket
        for sl in pieces:
            if not states_kept:
                sess.evaluate(obs[sl], actor.out.out_features)
            sess.backpropagate(grad[sl])
        return None, None, None


class NativeAdam:
    """The actor's optimiser as a learner sees it (param_groups, zero_grad, step, state_dict); the work is the
    library's (fc_zero_grad, fc_step), the reference's NativeAdam (fly_native.py:61-102)."""

    def __init__(self, actor: "NativeFlyActor", lr: float, max_norm: float = 0.0, ema: float = 0.999):
        self.actor = actor
        self.max_norm, self.ema = float(max_norm), float(ema)
        self.param_groups = [{"lr": lr}]
        self.grad_norm = 0.0

    def zero_grad(self, set_to_none: bool = True) -> None:
        sess = self.actor._open()
        if sess is not None:
            sess.on_current_stream(self.actor.gain.device)
            call("fc_zero_grad", sess.handle)

    def step(self) -> None:
        a = self.actor
        sess = a._open()
        if sess is None:
            return
        if dist.on():                      # several ranks: every rank steps with the mean gradient
            g = a._fetch(GRADIENT)
            dist.mean_(g)
            a._store(GRADIENT, g)
        rate = float(self.param_groups[0]["lr"])
        sess.on_current_stream(a.gain.device)
        self.grad_norm = float(call("fc_step", sess.handle, rate, rate * a.lr_neuron, rate * a.lr_plug, self.max_norm,
                                    self.ema))
        a.pull()

    def state_dict(self) -> dict:
        sess = self.actor._open()
        if sess is None:
            return {"native": True, "adam_t": 0}
        state = {"native": True, "adam_t": int(call("fc_adam_t", sess.handle, -1))}
        for key, which in (("ema", AVERAGE), ("m", ADAM_M), ("v", ADAM_V)):
            state[key] = [t.cpu() for t in self.actor._fetch(which)]
        return state

    def load_state_dict(self, state: dict) -> None:
        """A state written by state_dict() above; any other (a PyTorch Adam's, say) leaves the library's own."""
        sess = self.actor._open()
        if sess is None or not state.get("native") or "m" not in state:
            return
        dev = self.actor.gain.device
        for key, which in (("ema", AVERAGE), ("m", ADAM_M), ("v", ADAM_V)):
            self.actor._store(which, [t.to(dev) for t in state[key]])
        call("fc_adam_t", sess.handle, int(state.get("adam_t", 0)))
        self.actor._average_follows = False        # the running average came with the state


class NativeFlyActor(FlyActor):
    lr_neuron, lr_plug = 0.3, 1.0      # rates of gain / threshold and of the plugs, as shares of the strengths' rate

    _LIBRARY_STATE = ("_session", "_anchor", "_stale", "_average_follows", "max_batch")

    def __init__(self, *args, max_batch: int = 2048, **kw):
        super().__init__(*args, **kw)
        self.max_batch = int(max_batch)
        self._session: _Session | None = None
        self._anchor = None
        self._stale = True                 # PyTorch's weights are newer than the library's
        self._average_follows = True       # the library's running average is (re)started from the weights

    def __deepcopy__(self, memo):
        """A plain FlyActor with copies of everything but the library state."""
        import copy
        twin = FlyActor.__new__(FlyActor)
        memo[id(self)] = twin
        for k, v in self.__dict__.items():
            if k not in self._LIBRARY_STATE:
                twin.__dict__[k] = copy.deepcopy(v, memo)
        return twin

    def __del__(self):
        sess = self.__dict__.get("_session")
        if sess is not None:
            try:
                sess.close()
            except Exception:
                pass

    # ---- the library session
    def _open(self) -> _Session | None:
        """The session, made on first use on a GPU; None while the actor is on the CPU."""
        if self._session is None and self.gain.is_cuda:
            self._session = _Session(self, self.max_batch)
            self._anchor = torch.zeros(1, device=self.gain.device, requires_grad=True)
            self.push(also_average=True)
        return self._session

    def _ready(self) -> bool:
        return self._open() is not None

    @property
    def _core(self):
        return self._session.handle if self._session is not None else None

    @property
    def _wmap(self) -> torch.Tensor:
        return self._session.wmap

    def _fetch(self, which: int) -> list[torch.Tensor]:
        out = [torch.empty_like(t) for t in self._session.arrays(self)]
        self._session.transfer(which, out, into_library=False)
        return out

    def _store(self, which: int, tensors: list[torch.Tensor]) -> None:
        self._session.transfer(which, [t.contiguous().float() for t in tensors], into_library=True)

    def push(self, also_average: bool = False) -> None:
        """Copy the actor's PyTorch parameters into the library session (needed whenever they were set from outside,
        e.g. by load_state_dict); with also_average the library's running average is restarted from them too."""
        sess = self._session
        sess.w_play.copy_(self.w.data[sess.wmap])
        arrays = sess.arrays(self)
        sess.transfer(WEIGHTS, arrays, into_library=True)
        if also_average:
            sess.transfer(AVERAGE, arrays, into_library=True)
        self._stale = False

    def pull(self) -> None:
        """Copy the library's current weights back into the actor's PyTorch parameters (NativeAdam.step does this
        after every update, so PyTorch-side readers see the trained values)."""
        sess = self._session
        sess.transfer(WEIGHTS, sess.arrays(self), into_library=False)
        self.w.data[sess.wmap] = sess.w_play

    def _load_from_state_dict(self, *args, **kw):
        super()._load_from_state_dict(*args, **kw)
        self._stale = True                 # pushed before the next forward

    def native_adam(self, lr: float, max_norm: float = 0.0) -> NativeAdam | None:
        return NativeAdam(self, lr, max_norm) if self._ready() else None

    # ---- forward
    def _evaluate(self, obs: torch.Tensor) -> torch.Tensor:
        """Logits of a batch of any size, piece by piece."""
        if self._stale:
            self.push(also_average=self._average_follows)
        n_act = self.out.out_features
        parts = [self._session.evaluate(obs[sl], n_act) for sl in _pieces(obs.shape[0], self.max_batch)]
        return parts[0] if len(parts) == 1 else torch.cat(parts)

    def forward(self, obs: torch.Tensor, extra: torch.Tensor | None = None) -> torch.Tensor:
        if not obs.is_cuda:
            return super().forward(obs, extra)
        if not self._ready():
            raise RuntimeError("NativeFlyActor: observations are on the GPU but the actor's weights are not")
        obs = obs.float()
        if torch.is_grad_enabled():
            return _LibraryLogits.apply(obs, self._anchor, self)
        return self._evaluate(obs)


def grad_arrays(actor: NativeFlyActor) -> list[np.ndarray]:
    """Host copies (numpy, fc_copy's order) of the library's seven gradient buffers as accumulated since the last
    zero_grad."""
    return [t.cpu().numpy() for t in actor._fetch(GRADIENT)]
