"""The network's structure and weights as flat binaries (the format of flyguy/native/export.py:9-15).

NET.bin (little endian, int32 unless noted): "FLY1", obs_dim, n_act, hops, n_neurons, n_w, n_s, fan, n_dn,
sizes[hops+1], E[hops]; plug: in_crow[n_s+1], in_col[E_in], in_tcrow[obs_dim+1], in_tcol[E_in], in_tperm[E_in];
n0[n_s]; per hop: nid[N_k], crow[N_k+1], col[E_k], widx[E_k], tcrow[N_{k-1}+1], tcol[E_k], twidx[E_k], drow[N_k];
dn_rows[n_dn]; wmap[n_w].  Only the n_w connections in play are library parameters ("strengths in play").
PARAMS.bin: "FLYP", step (int64), float32 W[n_w], gain, theta, in_w, in_b, out_w (row = action), out_b.

The library reads exactly this file (fc_create); structure() is computed from an actor's own buffers, so the
two cannot disagree (export.py:32-49).
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np
import torch

_HOP_KEYS = ("nid", "crow", "col", "widx", "tcrow", "tcol", "twidx", "drow")
_PLUG_KEYS = ("in_crow", "in_col", "in_tcrow", "in_tcol", "in_tperm", "n0")


def structure(f) -> dict:
    """The index arrays of the library from a FlyActor's buffers (export.py:32-49): the in-play connections
    `wmap` (sorted), each hop's connections as indices into them (`widx`, and `twidx` in CSC order), and the
    sensory row that keeps driving a hop row (`drow`, -1 for none)."""
    K = f.hops
    used = torch.unique(torch.cat([getattr(f, f"e{k}") for k in range(1, K + 1)])).cpu().numpy()
    compact = np.full(f.n_conn, -1, np.int64)
    compact[used] = np.arange(len(used))
    s = {"obs_dim": f.obs_dim, "n_act": f.out.out_features, "hops": K, "n_neurons": f.n_neurons, "n_w": len(used),
         "n_s": f.sizes[0], "fan": f.fan, "n_dn": len(f.dn_rows), "sizes": list(f.sizes), "wmap": used,
         "in_crow": f.in_crow.cpu().numpy(), "in_col": f.in_ci.cpu().numpy(), "in_tcrow": f.in_tcrow.cpu().numpy(),
         "in_tcol": f.in_tci.cpu().numpy(), "in_tperm": f.in_tperm.cpu().numpy(), "n0": f.n0.cpu().numpy(),
         "dn_rows": f.dn_rows.cpu().numpy(), "hop": []}
    for k in range(1, K + 1):
        buf = lambda name: getattr(f, f"{name}{k}").cpu().numpy()     # noqa: E731
        widx = compact[buf("e")]
        drow = np.full(f.sizes[k], -1, np.int64)
        drow[buf("s")] = buf("d")
        s["hop"].append({"nid": buf("n"), "crow": buf("crow"), "col": buf("ci"), "widx": widx, "tcrow": buf("tcrow"),
                         "tcol": buf("tci"), "twidx": widx[buf("tperm")], "drow": drow})
    return s


def net_bytes(s: dict) -> bytes:
    """NET.bin of a structure dict (export.py:52-65 layout)."""
    i32 = lambda a: np.ascontiguousarray(a, dtype=np.int32).tobytes()        # noqa: E731
    parts = [b"FLY1", struct.pack("<8i", s["obs_dim"], s["n_act"], s["hops"], s["n_neurons"], s["n_w"], s["n_s"],
                                   s["fan"], s["n_dn"]),
             i32(s["sizes"]), i32([len(h["col"]) for h in s["hop"]])]
    parts += [i32(s[k]) for k in _PLUG_KEYS]
    for h in s["hop"]:
        parts += [i32(h[k]) for k in _HOP_KEYS]
    parts += [i32(s["dn_rows"]), i32(s["wmap"])]
    return b"".join(parts)


def read_net(src) -> dict:
    """The structure dict of a NET.bin (a path or its bytes), the inverse of net_bytes (export.py:52-65 layout)."""
    raw = src if isinstance(src, (bytes, bytearray)) else Path(src).read_bytes()
    if raw[:4] != b"FLY1":
        raise ValueError("not a FLY1 network file")
    at = [4]

    def ints(n):
        a = np.frombuffer(raw, np.int32, n, at[0]).astype(np.int64)
        at[0] += 4 * n
        return a
    od, na, K, nn, nw, ns, fan, ndn = (int(v) for v in ints(8))
    s = {"obs_dim": od, "n_act": na, "hops": K, "n_neurons": nn, "n_w": nw, "n_s": ns, "fan": fan, "n_dn": ndn}
    s["sizes"] = [int(v) for v in ints(K + 1)]
    E = [int(v) for v in ints(K)]
    E_in = ns * fan
    s["in_crow"], s["in_col"] = ints(ns + 1), ints(E_in)
    s["in_tcrow"], s["in_tcol"], s["in_tperm"] = ints(od + 1), ints(E_in), ints(E_in)
    s["n0"] = ints(ns)
    s["hop"] = []
    for k in range(K):
        rows, src = s["sizes"][k + 1], s["sizes"][k]
        h = {"nid": ints(rows), "crow": ints(rows + 1), "col": ints(E[k]), "widx": ints(E[k]), "tcrow": ints(src + 1),
             "tcol": ints(E[k]), "twidx": ints(E[k]), "drow": ints(rows)}
        s["hop"].append(h)
    s["dn_rows"], s["wmap"] = ints(ndn), ints(nw)
    if at[0] != len(raw):
        raise ValueError("network file of unexpected length")
    return s


def write_net(f, out: Path) -> dict:
    s = structure(f)
    Path(out).write_bytes(net_bytes(s))
    return s


def params_from_torch(f, s: dict) -> list[np.ndarray]:
    """The seven weight arrays in the library's order (export.py:68-70)."""
    return [f.w.detach().cpu().numpy()[s["wmap"]], f.gain.detach().cpu().numpy(), f.theta.detach().cpu().numpy(),
            f.in_w.detach().cpu().numpy(), f.in_b.detach().cpu().numpy(), f.out.weight.detach().cpu().numpy().reshape(-1),
            f.out.bias.detach().cpu().numpy()]


def param_sizes(s: dict) -> list[int]:
    return [s["n_w"], s["n_neurons"], s["n_neurons"], s["n_s"] * s["fan"], s["n_s"], s["n_act"] * s["n_dn"], s["n_act"]]


def write_params(arrs: list[np.ndarray], out: Path, step: int = 0) -> None:
    with open(out, "wb") as fh:
        fh.write(b"FLYP")
        fh.write(struct.pack("<q", step))
        for a in arrs:
            fh.write(np.ascontiguousarray(a, dtype=np.float32).tobytes())


def read_params(path: Path, s: dict) -> tuple[int, list[np.ndarray]]:
    raw = Path(path).read_bytes()
    if raw[:4] != b"FLYP":
        raise ValueError(f"{path}: not a FLYP parameter file")
    step = struct.unpack("<q", raw[4:12])[0]
    out, at = [], 12
    for n in param_sizes(s):
        if at + 4 * n > len(raw):
            raise ValueError(f"{path}: short parameter file")
        out.append(np.frombuffer(raw, np.float32, n, at).copy())
        at += 4 * n
    return step, out
