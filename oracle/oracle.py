"""ORACLE - test infrastructure only: ctypes wrapper of fly_oracle.c (float and double builds).

Pinned by tests/test_oracle.py: the forward against the dense "blind" computation of the reference's own test
(tests/test_fly.py:29-41 restated as dense matrix products over every neuron) and against the reference's
compiled CPU forward (fly_infer.cpp, oracle/_ref); the loss against torch.log_softmax; the backward against
autograd of the dense computation in float64 and against finite differences; Adam against torch.optim.Adam.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_libs: dict[str, ctypes.CDLL] = {}
vp, ci, cll, cf = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_float


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE), "_build/liboracle_f32.so", "_build/liboracle_f64.so"], check=True)


def _lib(precision: str) -> ctypes.CDLL:
    if precision not in _libs:
        path = HERE / "_build" / f"liboracle_{precision}.so"
        if not path.exists():
            build()
        L = ctypes.CDLL(str(path))
        L.or_create.restype, L.or_create.argtypes = vp, [ctypes.c_char_p, cll]
        L.or_free.restype, L.or_free.argtypes = None, [vp]
        L.or_sizes.restype, L.or_sizes.argtypes = None, [vp, ctypes.POINTER(cll)]
        L.or_set_params.restype, L.or_set_params.argtypes = None, [vp, ctypes.POINTER(vp)]
        L.or_forward.restype, L.or_forward.argtypes = ci, [vp, vp, ci, vp]
        L.or_state.restype, L.or_state.argtypes = ci, [vp, ci, ci, vp]
        L.or_loss.restype, L.or_loss.argtypes = ci, [vp, vp, ci, ci, cf, vp, vp]
        L.or_backward.restype, L.or_backward.argtypes = ci, [vp, vp, ci, ctypes.POINTER(vp)]
        L.or_adam.restype, L.or_adam.argtypes = None, [vp, vp, vp, vp, vp, cll, cf, cll, cf, cf]
        _libs[precision] = L
    return _libs[precision]


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class Oracle:
    """One network (NET.bin bytes) with its weights; precision "f32" (the reference's arithmetic) or "f64"."""

    def __init__(self, net: bytes, params: list[np.ndarray] | None = None, precision: str = "f64"):
        self.L = _lib(precision)
        self.h = self.L.or_create(net, len(net))
        if not self.h:
            raise ValueError("oracle: not a valid FLY1 network")
        s = (cll * 10)()
        self.L.or_sizes(self.h, s)
        self.psize = [int(v) for v in s[:7]]
        self.obs_dim, self.n_act, self.hops = int(s[7]), int(s[8]), int(s[9])
        self.B = 0
        if params is not None:
            self.set_params(params)

    def __del__(self):
        if getattr(self, "h", None):
            self.L.or_free(self.h)

    def set_params(self, params: list[np.ndarray]) -> None:
        arrs = [_f32(p).reshape(-1) for p in params]
        assert [a.size for a in arrs] == self.psize, "oracle: weight array sizes differ from the network's"
        ptrs = (vp * 7)(*[a.ctypes.data for a in arrs])
        self.L.or_set_params(self.h, ptrs)

    def forward(self, obs: np.ndarray) -> np.ndarray:
        x = _f32(obs)
        B = x.shape[0]
        out = np.zeros((B, self.n_act), np.float32)
        assert self.L.or_forward(self.h, x.ctypes.data, B, out.ctypes.data) == 0
        self.B = B
        return out

    def state(self, layer: int, what: int, rows: int) -> np.ndarray:
        out = np.zeros((rows, self.B), np.float32)
        assert self.L.or_state(self.h, layer, what, out.ctypes.data) == 0
        return out

    def backward(self, dlogits: np.ndarray) -> list[np.ndarray]:
        d = _f32(dlogits)
        grads = [np.zeros(n, np.float32) for n in self.psize]
        ptrs = (vp * 7)(*[g.ctypes.data for g in grads])
        assert self.L.or_backward(self.h, d.ctypes.data, d.shape[0], ptrs) == 0
        return grads

    def loss(self, logits: np.ndarray, teacher: np.ndarray, it: float = 1.0):
        lg, tl = _f32(logits), _f32(teacher)
        B, A = lg.shape
        dl = np.zeros((B, A), np.float32)
        stats = np.zeros(2, np.float64)
        self.L.or_loss(lg.ctypes.data, tl.ctypes.data, B, A, it, dl.ctypes.data, stats.ctypes.data)
        return dl, float(stats[0]), float(stats[1])

    def adam(self, p, g, m, v, ema, lr: float, t: int, gs: float = 1.0, decay: float = 0.999) -> None:
        """In place on float32 numpy arrays (one array group)."""
        for a in (p, g, m, v, ema):
            assert a.dtype == np.float32 and a.flags.c_contiguous
        self.L.or_adam(p.ctypes.data, g.ctypes.data, m.ctypes.data, v.ctypes.data, ema.ctypes.data, p.size, lr, t, gs,
                       decay)
