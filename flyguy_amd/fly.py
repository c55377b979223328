"""The fly actor: a network wired like a connectome, one unit per neuron and one trainable strength per connection.

Interface of the reference's FlyActor (flyguy/fly.py:75-305): same constructor, the same buffers (names, dtypes,
order: e/r/c/crow/tcrow/tcol/tperm/ci/tci/n/s/d per hop, in_* for the plug, n0, dn_rows), the same parameters and
their initial values (w, gain, theta, in_w, in_b, out.weight, out.bias; same torch random draws in the same
order), so a checkpoint of either loads into the other.

A decision: the observation drives the sensory neurons through a sparse plug (each reads `fan` fixed observation
values), the signal crosses `hops` sparse hops, each neuron firing relu(gain * z - softplus(theta)), and a linear
read-out maps the descending neurons to the action logits.  Hop k only holds the neurons that can carry the
signal after k hops AND still reach a descending neuron in the hops left (fly.py:91-100), so pruning changes
nothing in the result.

Execution paths of forward():
  - on a GPU with kernel "cuda" / "cuda16" / "hip": the hops run as the MI355X library's sparse products
    (flyguy_amd.fly_hip.HopHip, the HopCuda interface of fly_cuda.py) - the library must be built, else an error;
  - otherwise the PyTorch formulation of the reference: gather / index_add for small batches, sparse products
    with their own backward for large ones, and sparse CSR products for playing on the CPU (fly.py:252-305).
NativeFlyActor (flyguy_amd.fly_native) runs the whole network, its backward and Adam in the library.
"""
from __future__ import annotations

from collections.abc import Mapping
import struct
from pathlib import Path

import numpy as np
import torch
import torch.nn as nn

ROOT = Path(__file__).resolve().parents[1]
INHIBITORY = ("gaba", "glutamate", "histamine")        # transmitters whose connections start negative (fly.py:32)


def reach(start: np.ndarray, src: np.ndarray, dst: np.ndarray, n: int, steps: int) -> list[np.ndarray]:
    """out[k][i]: neuron i is in `start` or within k steps of it along src -> dst (fly.py:35-43)."""
    cur = np.zeros(n, bool)
    cur[start] = True
    out = [cur]
    for _ in range(steps):
        nxt = cur.copy()
        nxt[dst[cur[src]]] = True
        out.append(nxt)
        cur = nxt
    return out


def rowptr(rows: np.ndarray, n_rows: int) -> np.ndarray:
    """CSR row pointer (int64) of entries already grouped by row (fly.py:46-48)."""
    counts = np.bincount(rows, minlength=n_rows)
    return np.concatenate([np.zeros(1, np.int64), np.cumsum(counts)]).astype(np.int64)


def _load_graph(graph) -> Mapping:
    if isinstance(graph, Mapping):
        return graph
    p = Path(graph)
    return np.load(p if p.is_absolute() else ROOT / p)


class _SparseHop(torch.autograd.Function):
    """z[b, target] = sum over connections of w * h[b, source], states [B, rows]; the backward is the transposed
    product for h and the product sampled at the connections for w (fly.py:51-72)."""

    @staticmethod
    def forward(ctx, w, h, crow, col, tcrow, tcol, tperm):
        a = torch.sparse_csr_tensor(crow, col, w, size=(crow.numel() - 1, h.shape[1]))
        ctx.save_for_backward(w, h, crow, col, tcrow, tcol, tperm)
        return torch.sparse.mm(a, h.t()).t()

    @staticmethod
    def backward(ctx, gz):
        w, h, crow, col, tcrow, tcol, tperm = ctx.saved_tensors
        n_rows = crow.numel() - 1
        gw = gh = None
        if ctx.needs_input_grad[0]:
            pattern = torch.sparse_csr_tensor(crow, col, torch.zeros_like(w), size=(n_rows, h.shape[1]))
            gw = torch.sparse.sampled_addmm(pattern, gz.t().contiguous(), h, beta=0.0, alpha=1.0).values()
        if ctx.needs_input_grad[1]:
            at = torch.sparse_csr_tensor(tcrow, tcol, w[tperm], size=(h.shape[1], n_rows))
            gh = torch.sparse.mm(at, gz.t()).t()
        return gw, gh, None, None, None, None, None


class FlyActor(nn.Module):
    memory = 0

    def __init__(self, graph, obs_dim: int, n_actions: int, hops: int = 3, fan: int = 16, out_gain: float = 0.01,
                 seed: int = 0):
        super().__init__()
        g = _load_graph(graph)
        files = set(g.keys()) if isinstance(g, Mapping) else set(g.files)
        n = len(g["body"])
        pre = np.asarray(g["pre"]).astype(np.int64)
        post = np.asarray(g["post"]).astype(np.int64)
        syn = np.asarray(g["syn"]).astype(np.float32)
        sens = np.asarray(g["sensory"]).astype(np.int64)
        dn = np.asarray(g["descending"]).astype(np.int64)
        self.n_neurons, self.n_conn, self.hops, self.obs_dim, self.fan = n, len(pre), hops, obs_dim, fan
        self.whole_graph = "in_total" not in files
        self.gather_limit = 60_000_000          # batch x connection steps up to which the gather path is used
        self.kernel = "torch"                   # "cuda" / "cuda16" / "hip": the library's hop kernels on a GPU

        # the neurons of each hop: reached from the sensory side in k steps, reaching a descending neuron in the rest
        down = reach(sens, pre, post, n, hops)
        up = reach(dn, post, pre, n, hops)
        sets = [np.flatnonzero(down[k] & up[hops - k]) for k in range(hops + 1)]
        self.sizes = [int(len(s)) for s in sets]
        pos = []
        for s in sets:
            q = np.full(n, -1, np.int64)
            q[s] = np.arange(len(s))
            pos.append(q)
        sensory = np.zeros(n, bool)
        sensory[sens] = True

        def keep(name, arr):
            self.register_buffer(name, torch.as_tensor(np.ascontiguousarray(arr)), persistent=False)

        self.used = 0
        in_play = np.zeros(len(pre), bool)
        for k in range(1, hops + 1):
            m = np.flatnonzero((pos[k - 1][pre] >= 0) & (pos[k][post] >= 0))
            tgt, src = pos[k][post[m]], pos[k - 1][pre[m]]
            by_row = np.lexsort((src, tgt))                     # CSR: target, then source (stable)
            m, tgt, src = m[by_row], tgt[by_row], src[by_row]
            by_col = np.lexsort((tgt, src))                     # CSC: source, then target (stable)
            keep(f"e{k}", m)
            keep(f"r{k}", tgt)
            keep(f"c{k}", src)
            keep(f"crow{k}", rowptr(tgt, len(sets[k])))
            keep(f"tcrow{k}", rowptr(src[by_col], len(sets[k - 1])))
            keep(f"tcol{k}", tgt[by_col])
            keep(f"tperm{k}", by_col)
            keep(f"ci{k}", src.astype(np.int32))
            keep(f"tci{k}", tgt[by_col].astype(np.int32))
            keep(f"n{k}", sets[k])
            here = sensory[sets[k]]
            keep(f"s{k}", np.flatnonzero(here))                 # sensory neurons among hop k's, kept driven
            keep(f"d{k}", pos[0][sets[k][here]])                # ... and their row in the sensory layer
            self.used += len(m)
            in_play[m] = True
        self.in_play = int(in_play.sum())
        keep("n0", sets[0])
        reachable = pos[hops][dn] >= 0
        assert reachable.any(), "no descending neuron can be reached in this many hops"
        keep("dn_rows", pos[hops][dn[reachable]])

        # parameters: one strength per connection, a gain and a threshold per neuron (fly.py:128-139)
        if "in_total" in files:
            assert hops <= int(g["hops"]), f"this graph file holds the connections of a {int(g['hops'])}-hop network only"
            total = np.asarray(g["in_total"]).astype(np.float32)
        else:
            total = np.zeros(n, np.float32)
            np.add.at(total, post, syn)
        sign = np.where(np.isin(np.asarray(g["nt"])[pre], INHIBITORY), -1.0, 1.0).astype(np.float32)
        self.w = nn.Parameter(torch.as_tensor(1.5 * sign * syn / np.maximum(total[post], 1.0)))
        self.gain = nn.Parameter(torch.ones(n))
        self.theta = nn.Parameter(torch.full((n,), -4.0))

        # the plug: each sensory neuron in play reads `fan` observation values chosen at random (fly.py:140-150)
        rng = np.random.default_rng(seed)
        n_s = self.sizes[0]
        picks = np.empty((n_s, fan), np.int64)
        for i in range(n_s):
            picks[i] = np.sort(rng.choice(obs_dim, size=fan, replace=False))
        cols = picks.reshape(-1)
        rows = np.repeat(np.arange(n_s), fan)
        by_col = np.lexsort((rows, cols))
        keep("in_r", rows)
        keep("in_c", cols)
        keep("in_crow", rowptr(rows, n_s))
        keep("in_tcrow", rowptr(cols[by_col], obs_dim))
        keep("in_tcol", rows[by_col])
        keep("in_tperm", by_col)
        keep("in_ci", cols.astype(np.int32))
        keep("in_tci", rows[by_col].astype(np.int32))
        self.in_w = nn.Parameter(torch.randn(n_s * fan) / fan ** 0.5)
        self.in_b = nn.Parameter(torch.zeros(n_s))
        # the read-out: descending neurons -> action logits
        self.out = nn.Linear(len(self.dn_rows), n_actions)
        nn.init.orthogonal_(self.out.weight, out_gain)
        nn.init.zeros_(self.out.bias)

    def describe(self) -> str:
        plug = self.in_w.numel() + self.in_b.numel() + sum(p.numel() for p in self.out.parameters())
        return (f"fly actor: {self.n_neurons:,} neurons and {self.n_conn:,} connections in the graph; {self.hops} hops: "
                f"{self.in_play:,} connections and {sum(self.sizes):,} neuron states in play (per hop {self.sizes}), "
                f"{self.used:,} connection steps a decision; learned outside the fly: {plug:,} numbers (each sensory "
                f"neuron hears {self.fan} observation values; {len(self.dn_rows):,} descending neurons -> actions)")

    # ---- hop products, PyTorch formulation ([B, rows] states)
    def _hop_buffers(self, k):
        if k == "in_":
            return self.in_r, self.in_c, self.in_crow, self.in_tcrow, self.in_tcol, self.in_tperm
        return (getattr(self, f"r{k}"), getattr(self, f"c{k}"), getattr(self, f"crow{k}"), getattr(self, f"tcrow{k}"),
                getattr(self, f"tcol{k}"), getattr(self, f"tperm{k}"))

    def _product(self, k, w: torch.Tensor, h: torch.Tensor, n_rows: int, small: bool) -> torch.Tensor:
        r, c, crow, tcrow, tcol, tperm = self._hop_buffers(k)
        if small:                                               # gather / scatter: cheapest for a few samples
            return torch.zeros(h.shape[0], n_rows, dtype=h.dtype, device=h.device).index_add_(1, r, h[:, c] * w)
        return _SparseHop.apply(w, h, crow, c, tcrow, tcol, tperm)

    def _forward_hip(self, obs: torch.Tensor) -> torch.Tensor:
        """States [neurons, batch], every product on the MI355X library (fly.py:170-185 with HopHip)."""
        from .fly_hip import HopHip
        half = self.kernel == "cuda16"
        x = obs.t().contiguous()
        drive = HopHip.apply(self.in_w, x, self.in_crow, self.in_ci, self.in_tcrow, self.in_tci, self.in_tperm, False)
        drive = drive + self.in_b[:, None]
        thr = nn.functional.softplus(self.theta)
        h = torch.relu(self.gain[self.n0][:, None] * drive - thr[self.n0][:, None])
        for k in range(1, self.hops + 1):
            rows = getattr(self, f"n{k}")
            z = HopHip.apply(self.w[getattr(self, f"e{k}")], h, getattr(self, f"crow{k}"), getattr(self, f"ci{k}"),
                             getattr(self, f"tcrow{k}"), getattr(self, f"tci{k}"), getattr(self, f"tperm{k}"), half)
            s_ = getattr(self, f"s{k}")
            if len(s_):
                z = z.index_add(0, s_, drive[getattr(self, f"d{k}")])
            h = torch.relu(self.gain[rows][:, None] * z - thr[rows][:, None])
        return self.out(h[self.dn_rows].t())

    def _native(self):
        """The CPU decision library (flyguy_amd/libfly_infer.so, include/fly_infer.h: a hop pushes only the neurons
        that fire), set up from the current weights (fly.py:186-241).  None when it is not built or FLYGUY_NATIVE=0:
        then the sparse products below play.  FLYGUY_CPU_THREADS=n decides each car on n threads (0: one per hardware
        thread; unset: one, as the reference does), with bit-identical answers."""
        ver = (self.w._version, self.in_w._version, self.gain._version, self.theta._version, self.in_b._version,
               self.out.weight._version, self.out.bias._version, self.w.dtype)
        nat = getattr(self, "_nat", None)
        if nat is not None and nat["ver"] == ver:
            return nat if nat["h"] else None
        import ctypes
        import os
        if nat is not None and nat["h"]:
            nat["lib"].fly_free(nat["h"])
        nat = {"ver": ver, "h": None}
        self._nat = nat
        path = Path(__file__).resolve().parent / "libfly_infer.so"
        if os.environ.get("FLYGUY_NATIVE", "1") == "0" or not path.exists() or self.w.dtype != torch.float32:
            return None
        lib = ctypes.CDLL(str(path))
        vp, ci = ctypes.c_void_p, ctypes.c_int
        lib.fly_create.restype, lib.fly_create.argtypes = vp, [ci, ci, ci]
        lib.fly_set_plug.restype, lib.fly_set_plug.argtypes = None, [vp, ci, ci] + [vp] * 6
        lib.fly_set_hop.restype, lib.fly_set_hop.argtypes = None, [vp, ci, ci, ci, ci] + [vp] * 6
        lib.fly_set_out.restype, lib.fly_set_out.argtypes = None, [vp, ci, vp, vp, vp]
        lib.fly_forward.restype, lib.fly_forward.argtypes = None, [vp, vp, ci, vp, vp]
        lib.fly_free.restype, lib.fly_free.argtypes = None, [vp]
        keep = []                      # the arrays handed over (the library copies them; kept until set-up ends)

        def arr(t, dt):
            a = np.ascontiguousarray(t.detach().cpu().numpy() if torch.is_tensor(t) else t, dtype=dt)
            keep.append(a)
            return a.ctypes.data_as(vp)
        with torch.no_grad():
            thr = nn.functional.softplus(self.theta)
            h = lib.fly_create(self.obs_dim, self.out.out_features, self.hops)
            lib.fly_set_plug(h, self.sizes[0], int(self.in_ci.numel()), arr(self.in_crow, np.int32),
                             arr(self.in_ci, np.int32), arr(self.in_w, np.float32), arr(self.in_b, np.float32),
                             arr(self.gain[self.n0], np.float32), arr(thr[self.n0], np.float32))
            for k in range(1, self.hops + 1):
                rows = getattr(self, f"n{k}")
                drow = np.full(len(rows), -1, np.int32)
                drow[getattr(self, f"s{k}").cpu().numpy()] = getattr(self, f"d{k}").cpu().numpy()
                w_by_src = self.w[getattr(self, f"e{k}")[getattr(self, f"tperm{k}")]]
                lib.fly_set_hop(h, k - 1, len(rows), self.sizes[k - 1], int(w_by_src.numel()),
                                arr(getattr(self, f"tcrow{k}"), np.int32), arr(getattr(self, f"tci{k}"), np.int32),
                                arr(w_by_src, np.float32), arr(self.gain[rows], np.float32), arr(thr[rows], np.float32),
                                arr(drow, np.int32))
            lib.fly_set_out(h, len(self.dn_rows), arr(self.dn_rows, np.int32), arr(self.out.weight, np.float32),
                            arr(self.out.bias, np.float32))
            threads = os.environ.get("FLYGUY_CPU_THREADS")
            if threads is not None:
                lib.fly_set_threads.restype, lib.fly_set_threads.argtypes = None, [vp, ci]
                lib.fly_set_threads(h, int(threads))
        nat.update(h=h, lib=lib, shade=np.zeros(int(sum(self.sizes)), np.uint8))
        return nat

    def _forward_native(self, obs: torch.Tensor, nat: dict) -> torch.Tensor:
        import ctypes
        x = np.ascontiguousarray(obs.detach().numpy(), dtype=np.float32)
        out = np.empty((x.shape[0], self.out.out_features), np.float32)
        tap = getattr(self, "tap", None)             # the visualizer: every neuron's firing for the first car
        vp = ctypes.c_void_p
        nat["lib"].fly_forward(nat["h"], x.ctypes.data_as(vp), x.shape[0], out.ctypes.data_as(vp),
                               nat["shade"].ctypes.data_as(vp) if tap is not None else None)
        if tap is not None:
            tap(nat["shade"])
        return torch.from_numpy(out)

    @torch.no_grad()
    def _forward_cpu(self, obs: torch.Tensor) -> torch.Tensor:
        """Playing on the CPU (fly.py:252-284): the CPU decision library when it is built, else sparse CSR products
        built once from the current weights."""
        nat = self._native()
        if nat is not None:
            return self._forward_native(obs, nat)
        ver = (self.w._version, self.in_w._version, self.gain._version, self.theta._version, self.in_b._version)
        c = getattr(self, "_cpu", None)
        if c is None or c["ver"] != ver:
            thr = nn.functional.softplus(self.theta)
            c = {"ver": ver, "hop": [],
                 "a_in": torch.sparse_csr_tensor(self.in_crow, self.in_c, self.in_w.detach().clone(),
                                                 size=(self.sizes[0], self.obs_dim)),
                 "g0": self.gain[self.n0][:, None].clone(), "t0": thr[self.n0][:, None].clone()}
            for k in range(1, self.hops + 1):
                rows = getattr(self, f"n{k}")
                a = torch.sparse_csr_tensor(getattr(self, f"crow{k}"), getattr(self, f"c{k}"),
                                            self.w.detach()[getattr(self, f"e{k}")], size=(len(rows), self.sizes[k - 1]))
                c["hop"].append((a, self.gain[rows][:, None].clone(), thr[rows][:, None].clone(),
                                 getattr(self, f"s{k}"), getattr(self, f"d{k}")))
            self._cpu = c
        drive = torch.sparse.mm(c["a_in"], obs.t().contiguous()) + self.in_b[:, None]
        h = torch.relu(c["g0"] * drive - c["t0"])
        tap = getattr(self, "tap", None)             # the visualizer: every layer's firing for the first car
        acts = [h[:, 0]] if tap is not None else None
        for a, g, t, s_, d_ in c["hop"]:
            z = torch.sparse.mm(a, h)
            if len(s_):
                z[s_] += drive[d_]
            h = torch.relu(g * z - t)
            if acts is not None:
                acts.append(h[:, 0])
        if tap is not None:
            tap(acts)
        return self.out(h[self.dn_rows].t())

    def forward(self, obs: torch.Tensor, extra: torch.Tensor | None = None) -> torch.Tensor:
        obs = obs.double() if self.w.dtype == torch.float64 else obs.float()    # (float64: an actor made .double())
        if not obs.is_cuda and not torch.is_grad_enabled():
            return self._forward_cpu(obs)
        small = obs.shape[0] * self.used <= self.gather_limit
        if self.kernel != "torch" and obs.is_cuda and obs.shape[0] % 32 == 0:
            return self._forward_hip(obs)
        drive = self._product("in_", self.in_w, obs, self.sizes[0], small) + self.in_b
        thr = nn.functional.softplus(self.theta)
        h = torch.relu(self.gain[self.n0] * drive - thr[self.n0])
        for k in range(1, self.hops + 1):
            rows = getattr(self, f"n{k}")
            z = self._product(str(k), self.w[getattr(self, f"e{k}")], h, len(rows), small)
            s_ = getattr(self, f"s{k}")
            if len(s_):
                z = z.index_add(1, s_, drive[:, getattr(self, f"d{k}")])
            h = torch.relu(self.gain[rows] * z - thr[rows])
        return self.out(h[:, self.dn_rows])


class VizTap:
    """The visualizer's window into a playing actor (fly.py:308-368): after every decision the firing of every neuron
    in play, layer by layer, goes into a small shared file, one byte a neuron, with the chosen action; a reader
    (the visualizer's server) maps the file, nothing waits for it.  Set `actor.tap = VizTap(actor.sizes)`.

    File (little endian): "FLYV", version 1 (u32), seq (u32, odd while being written) at 8, tick (u32) at 12, time
    (f64) at 16, action (i32) at 24, 8 controls (f32) at 28, layer count and 4 layer sizes (u32) at 60, 90 action
    probabilities (f32) at 80, match clock (f32), frame (u32), overtime (i32) at 440; the firing bytes from 512,
    the layers one after another (sensory first), 255 * tanh(1.5 * firing)."""

    HEADER = 512

    def __init__(self, sizes, path=None):
        import mmap
        import tempfile
        self.sizes = [int(v) for v in sizes]
        self.path = Path(path) if path else Path(tempfile.gettempdir()) / "flyguy_viz.bin"
        total = self.HEADER + sum(self.sizes)
        if not (self.path.exists() and self.path.stat().st_size == total):   # a file of the right size is reused
            with open(self.path, "wb") as fh:
                fh.write(bytes(total))
        self.fh = open(self.path, "r+b")
        self.mm = mmap.mmap(self.fh.fileno(), total)
        self.mm[0:8] = b"FLYV" + struct.pack("<I", 1)
        self.mm[60:80] = struct.pack("<5I", len(self.sizes), *(self.sizes + [0] * 4)[:4])
        self.seq = 0
        self.tick = 0
        self.acts = None

    def __call__(self, acts) -> None:
        """From the actor's forward pass: the first car's firing (a uint8 array from the CPU library, or one tensor
        per layer from the sparse products)."""
        self.acts = acts

    def publish(self, action: int, controls, probs, clock: float = -1.0, frame: int = 0, overtime: bool = False) -> None:
        import time
        if self.acts is None:
            return
        self.mm[440:452] = struct.pack("<fIi", float(clock), int(frame) & 0xFFFFFFFF, int(bool(overtime)))
        self.seq += 1
        self.mm[8:12] = struct.pack("<I", self.seq)
        at = self.HEADER
        if isinstance(self.acts, np.ndarray):
            b = self.acts.astype(np.uint8).tobytes()
            self.mm[at:at + len(b)] = b
        else:
            for a in self.acts:
                b = (torch.tanh(a.float() * 1.5) * 255.0).to(torch.uint8).cpu().numpy().tobytes()
                self.mm[at:at + len(b)] = b
                at += len(b)
        self.tick += 1
        self.mm[12:28] = struct.pack("<Idi", self.tick, time.time(), int(action))
        self.mm[28:60] = np.asarray(controls, np.float32)[:8].tobytes()
        p = np.asarray(probs, np.float32)[:90]
        self.mm[80:80 + 4 * len(p)] = p.tobytes()
        self.seq += 1
        self.mm[8:12] = struct.pack("<I", self.seq)
        self.acts = None

    def close(self) -> None:
        self.mm.close()
        self.fh.close()
