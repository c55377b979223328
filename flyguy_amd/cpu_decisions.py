"""Decisions on the host CPU from a network file and its weights, without a FlyActor (flyguy/native/fly_infer.cpp's
library, as flyguy/fly.py:186-241 drives it).

    from flyguy_amd.export import read_net, read_params
    from flyguy_amd.cpu_decisions import CpuDecisions
    s = read_net(Path("NET.bin")); step, P = read_params(Path("PARAMS.bin"), s)
    logits = CpuDecisions(s, P).forward(obs)          # obs [B][obs_dim] float32 -> [B][n_act]

The library is flyguy_amd/libfly_infer.so (include/fly_infer.h): the plug in CSR form, every hop by source (a hop
pushes only the neurons that fire), thresholds softplus(theta), the read-out.  threads > 1 decides each car on that
many threads (bit-identical answers).  One handle per calling thread: a handle is not thread-safe.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB = Path(__file__).resolve().parent / "libfly_infer.so"
_vp, _ci = ctypes.c_void_p, ctypes.c_int


def _softplus32(theta: np.ndarray) -> np.ndarray:
    """softplus(theta) (threshold 20, as torch's) evaluated in float64 and rounded once to float32."""
    t = np.asarray(theta, np.float32).astype(np.float64)
    return np.where(t > 20, t, np.log1p(np.exp(np.minimum(t, 20)))).astype(np.float32)


class CpuDecisions:
    """The CPU decision library on a structure dict (flyguy_amd.export.structure / read_net) and the seven weight
    arrays (W, gain, theta, in_w, in_b, out_w, out_b)."""

    def __init__(self, s: dict, params: list[np.ndarray], lib_path: Path | None = None, threads: int = 1):
        path = Path(lib_path or LIB)
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built (python -c 'import __graft_entry__ as g; g.build()')")
        L = ctypes.CDLL(str(path))
        L.fly_create.restype, L.fly_create.argtypes = _vp, [_ci, _ci, _ci]
        L.fly_set_plug.restype, L.fly_set_plug.argtypes = None, [_vp, _ci, _ci] + [_vp] * 6
        L.fly_set_hop.restype, L.fly_set_hop.argtypes = None, [_vp, _ci, _ci, _ci, _ci] + [_vp] * 6
        L.fly_set_out.restype, L.fly_set_out.argtypes = None, [_vp, _ci, _vp, _vp, _vp]
        L.fly_forward.restype, L.fly_forward.argtypes = None, [_vp, _vp, _ci, _vp, _vp]
        L.fly_free.restype, L.fly_free.argtypes = None, [_vp]
        if threads != 1:
            L.fly_set_threads.restype, L.fly_set_threads.argtypes = None, [_vp, _ci]
        self.L = L
        W, gain, theta, in_w, in_b, out_w, out_b = [np.asarray(p, np.float32).reshape(-1) for p in params]
        thr = _softplus32(theta)
        keep = []                                   # (the library copies every array during set-up)

        def ptr(a, dt):
            a = np.ascontiguousarray(a, dtype=dt)
            keep.append(a)
            return a.ctypes.data

        self.n_act, self.obs_dim = int(s["n_act"]), int(s["obs_dim"])
        self.h = L.fly_create(self.obs_dim, self.n_act, int(s["hops"]))
        n0 = np.asarray(s["n0"])
        L.fly_set_plug(self.h, int(s["n_s"]), len(s["in_col"]), ptr(s["in_crow"], np.int32), ptr(s["in_col"], np.int32),
                       ptr(in_w, np.float32), ptr(in_b, np.float32), ptr(gain[n0], np.float32), ptr(thr[n0], np.float32))
        for k, hop in enumerate(s["hop"]):
            nid = np.asarray(hop["nid"])
            L.fly_set_hop(self.h, k, len(nid), int(s["sizes"][k]), len(hop["tcol"]), ptr(hop["tcrow"], np.int32),
                          ptr(hop["tcol"], np.int32), ptr(W[np.asarray(hop["twidx"])], np.float32),
                          ptr(gain[nid], np.float32), ptr(thr[nid], np.float32), ptr(hop["drow"], np.int32))
        L.fly_set_out(self.h, len(s["dn_rows"]), ptr(s["dn_rows"], np.int32), ptr(out_w, np.float32),
                      ptr(out_b, np.float32))
        if threads != 1:
            L.fly_set_threads(self.h, int(threads))

    def __del__(self):
        if getattr(self, "h", None):
            self.L.fly_free(self.h)
            self.h = None

    def forward(self, obs: np.ndarray, tap: np.ndarray | None = None) -> np.ndarray:
        """logits [B][n_act] of obs [B][obs_dim]; tap (uint8, one per neuron state, or None): the first sample's
        firing bytes, 255 tanh(1.5 h), layer after layer."""
        x = np.ascontiguousarray(obs, dtype=np.float32).reshape(-1, self.obs_dim)
        out = np.empty((x.shape[0], self.n_act), np.float32)
        self.L.fly_forward(self.h, x.ctypes.data, x.shape[0], out.ctypes.data, None if tap is None else tap.ctypes.data)
        return out
