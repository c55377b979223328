"""ORACLE - test infrastructure only: the reference's compiled CPU forward (flyguy/native/fly_infer.cpp).

oracle/Makefile compiles it from the reference checkout into oracle/_ref/libfly_infer.so (never committed).  It is
driven here the way the reference's FlyActor._native() drives it (flyguy/fly.py:187-241): the plug in CSR form,
each hop in CSC form (the connections by source, strengths in that order), thresholds softplus(theta), the
read-out.  It walks only the connections of firing neurons, one sample after another.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB = Path(__file__).resolve().parent / "_ref" / "libfly_infer.so"
vp, ci = ctypes.c_void_p, ctypes.c_int


def available() -> bool:
    return LIB.exists()


def _softplus(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float64)
    return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20)))).astype(np.float32)


class RefInfer:
    """The reference's CPU forward on a library structure dict + the seven weight arrays."""

    def __init__(self, s: dict, params: list[np.ndarray], lib_path: Path | None = None):
        L = ctypes.CDLL(str(lib_path or LIB))
        L.fly_create.restype, L.fly_create.argtypes = vp, [ci, ci, ci]
        L.fly_set_plug.restype, L.fly_set_plug.argtypes = None, [vp, ci, ci] + [vp] * 6
        L.fly_set_hop.restype, L.fly_set_hop.argtypes = None, [vp, ci, ci, ci, ci] + [vp] * 6
        L.fly_set_out.restype, L.fly_set_out.argtypes = None, [vp, ci, vp, vp, vp]
        L.fly_forward.restype, L.fly_forward.argtypes = None, [vp, vp, ci, vp, vp]
        L.fly_free.restype, L.fly_free.argtypes = None, [vp]
        self.L = L
        W, gain, theta, in_w, in_b, out_w, out_b = [np.asarray(p, np.float32).reshape(-1) for p in params]
        thr = _softplus(theta)
        i32 = lambda a: np.ascontiguousarray(a, dtype=np.int32)          # noqa: E731
        f32 = lambda a: np.ascontiguousarray(a, dtype=np.float32)        # noqa: E731
        self._keep = []

        def ptr(a):
            self._keep.append(a)
            return a.ctypes.data

        self.n_act, self.obs_dim = s["n_act"], s["obs_dim"]
        self.h = L.fly_create(s["obs_dim"], s["n_act"], s["hops"])
        n0 = np.asarray(s["n0"])
        a = [i32(s["in_crow"]), i32(s["in_col"]), f32(in_w), f32(in_b), f32(gain[n0]), f32(thr[n0])]
        L.fly_set_plug(self.h, s["n_s"], len(a[1]), *map(ptr, a))
        for k, hop in enumerate(s["hop"]):
            nid = np.asarray(hop["nid"])
            a = [i32(hop["tcrow"]), i32(hop["tcol"]), f32(W[np.asarray(hop["twidx"])]), f32(gain[nid]), f32(thr[nid]),
                 i32(hop["drow"])]
            L.fly_set_hop(self.h, k, len(nid), s["sizes"][k], len(a[1]), *map(ptr, a))
        a = [i32(s["dn_rows"]), f32(out_w), f32(out_b)]
        L.fly_set_out(self.h, len(a[0]), *map(ptr, a))

    def __del__(self):
        if getattr(self, "h", None):
            self.L.fly_free(self.h)

    def forward(self, obs: np.ndarray, tap: np.ndarray | None = None) -> np.ndarray:
        """logits [B][n_act]; tap (uint8, one per neuron state): the first sample's firing bytes."""
        x = np.ascontiguousarray(obs, dtype=np.float32)
        out = np.zeros((x.shape[0], self.n_act), np.float32)
        self.L.fly_forward(self.h, x.ctypes.data, x.shape[0], out.ctypes.data, None if tap is None else tap.ctypes.data)
        return out
