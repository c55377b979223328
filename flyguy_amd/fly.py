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

One walk through the layers (_walk) serves every execution path of forward(); the paths differ in the layout of
the states and in how a layer's sparse product is formed:
  - on a GPU with kernel "cuda" / "cuda16" / "hip" and a batch that is a multiple of 32: states [neurons, batch],
    products on the MI355X library (flyguy_amd.fly_hip.HopHip, the HopCuda interface of fly_cuda.py; the library
    must be built, else an error).  The reference takes its kernels only above gather_limit; the library's products
    are the faster ones at any batch, so here they are taken at any batch;
  - with gradients, or on a GPU otherwise: states [batch, neurons], gather / index_add products for a few samples
    (batch x connection steps up to gather_limit), sparse products with a backward of their own above;
  - playing on the CPU (no gradients): the CPU decision library when it is built, else sparse CSR matrices of the
    current weights, made once per weights (fly.py:186-284).
NativeFlyActor (flyguy_amd.fly_native) runs the whole network, its backward and Adam in the library.
"""
from __future__ import annotations

from collections.abc import Mapping
from typing import NamedTuple
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

    @classmethod
    def from_structure(cls, s: dict, params: list | None = None) -> "FlyActor":
        """An actor over a network given as a library structure (flyguy_amd.export.structure / read_net: NET.bin's
        arrays) instead of a graph file, with the seven weight arrays in the library's order (params, or zeros).
        Its strengths are the network's strengths in play (w[i] is NET.bin's strength i, so e{k} = widx); buffers,
        parameters and every forward path are FlyActor's."""
        f = cls.__new__(cls)
        nn.Module.__init__(f)
        K = int(s["hops"])
        f.n_neurons, f.n_conn, f.hops = int(s["n_neurons"]), int(s["n_w"]), K
        f.obs_dim, f.fan = int(s["obs_dim"]), int(s["fan"])
        f.whole_graph, f.gather_limit, f.kernel = True, 60_000_000, "torch"
        f.sizes = [int(v) for v in s["sizes"]]

        def keep(name, arr, dtype=np.int64):
            f.register_buffer(name, torch.as_tensor(np.ascontiguousarray(arr, dtype=dtype)), persistent=False)

        f.used = 0
        for k in range(1, K + 1):
            h = s["hop"][k - 1]
            crow, col, widx = (np.asarray(h[x], np.int64) for x in ("crow", "col", "widx"))
            tcrow, tcol, twidx = (np.asarray(h[x], np.int64) for x in ("tcrow", "tcol", "twidx"))
            edge_of = np.full(f.n_conn, -1, np.int64)
            edge_of[widx] = np.arange(len(widx))
            drow = np.asarray(h["drow"], np.int64)
            keep(f"e{k}", widx)
            keep(f"r{k}", np.repeat(np.arange(len(crow) - 1), np.diff(crow)))
            keep(f"c{k}", col)
            keep(f"crow{k}", crow)
            keep(f"tcrow{k}", tcrow)
            keep(f"tcol{k}", tcol)
            keep(f"tperm{k}", edge_of[twidx])
            keep(f"ci{k}", col, np.int32)
            keep(f"tci{k}", tcol, np.int32)
            keep(f"n{k}", h["nid"])
            keep(f"s{k}", np.flatnonzero(drow >= 0))
            keep(f"d{k}", drow[drow >= 0])
            f.used += len(col)
        f.in_play = f.n_conn
        keep("n0", s["n0"])
        keep("dn_rows", s["dn_rows"])
        in_crow, in_col = np.asarray(s["in_crow"], np.int64), np.asarray(s["in_col"], np.int64)
        keep("in_r", np.repeat(np.arange(len(in_crow) - 1), np.diff(in_crow)))
        keep("in_c", in_col)
        keep("in_crow", in_crow)
        keep("in_tcrow", s["in_tcrow"])
        keep("in_tcol", s["in_tcol"])
        keep("in_tperm", s["in_tperm"])
        keep("in_ci", in_col, np.int32)
        keep("in_tci", s["in_tcol"], np.int32)
        P = params if params is not None else [np.zeros(n, np.float32) for n in (
            f.n_conn, f.n_neurons, f.n_neurons, len(in_col), f.sizes[0], int(s["n_act"]) * int(s["n_dn"]), int(s["n_act"]))]
        as_param = lambda a: nn.Parameter(torch.as_tensor(np.array(a, np.float32)))   # noqa: E731
        f.w, f.gain, f.theta, f.in_w, f.in_b = (as_param(a) for a in P[:5])
        f.out = nn.Linear(int(s["n_dn"]), int(s["n_act"]))
        with torch.no_grad():
            f.out.weight.copy_(torch.as_tensor(np.asarray(P[5], np.float32)).view(int(s["n_act"]), int(s["n_dn"])))
            f.out.bias.copy_(torch.as_tensor(np.asarray(P[6], np.float32)))
        return f

    def describe(self) -> str:
        plug = self.in_w.numel() + self.in_b.numel() + sum(p.numel() for p in self.out.parameters())
        return (f"fly actor: {self.n_neurons:,} neurons and {self.n_conn:,} connections in the graph; {self.hops} hops: "
                f"{self.in_play:,} connections and {sum(self.sizes):,} neuron states in play (per hop {self.sizes}), "
                f"{self.used:,} connection steps a decision; learned outside the fly: {plug:,} numbers (each sensory "
                f"neuron hears {self.fan} observation values; {len(self.dn_rows):,} descending neurons -> actions)")


    # ---- the layers as the forward passes walk them
    def _layers(self) -> list[_Layer]:
        """The plug (layer 0, the sensory neurons) and every hop, each with its product's index buffers."""
        def csr(pre: str, post: str, n_rows: int, n_src: int) -> _Csr:
            b = lambda name: getattr(self, f"{pre}{name}{post}")            # noqa: E731
            return _Csr(b("r"), b("c"), b("crow"), b("tcrow"), b("tcol"), b("tperm"), b("ci"), b("tci"), n_rows, n_src)
        none = self.n0.new_zeros(0)
        out = [_Layer(csr("in_", "", self.sizes[0], self.obs_dim), None, self.n0, none, none)]
        for k in range(1, self.hops + 1):
            out.append(_Layer(csr("", str(k), self.sizes[k], self.sizes[k - 1]), getattr(self, f"e{k}"),
                              getattr(self, f"n{k}"), getattr(self, f"s{k}"), getattr(self, f"d{k}")))
        return out

    def _walk(self, x: torch.Tensor, product, by_neuron: bool, watch=None, activate=None) -> torch.Tensor:
        """Logits of a batch: the plug's product plus bias gives the sensory drive, each hop's product (plus the
        drive of its re-driven sensory rows) the next layer's input, every neuron fires relu(gain z - softplus
        theta), and the read-out maps the descending rows to the actions (fly.py:286-305 / 170-185 / 252-284).
        States are [rows, B] when by_neuron, else [B, rows]; product(k, layer, weights, states) is layer k's sparse
        product (k = 0: the plug).  activate(z, gain, threshold) computes the firing of [rows, B] states from the
        rows' gains and thresholds (default: PyTorch's elementwise operations).  watch(h) sees every layer's
        firing."""
        axis = 0 if by_neuron else 1
        thr = nn.functional.softplus(self.theta)

        def per_row(v):
            return v[:, None] if by_neuron else v

        def fire(z, nid):
            if activate is not None:
                return activate(z, self.gain[nid], thr[nid])
            return torch.relu(per_row(self.gain[nid]) * z - per_row(thr[nid]))

        layers = self._layers()
        drive = product(0, layers[0], self.in_w, x) + per_row(self.in_b)
        h = fire(drive, layers[0].nid)
        if watch is not None:
            watch(h)
        for k, layer in enumerate(layers[1:], start=1):
            z = product(k, layer, self.w[layer.edges], h)
            if len(layer.redriven):
                add = drive.index_select(axis, layer.drive_rows)
                # (the library's products return a new tensor of their own, which can take the sums in place; the
                # PyTorch path's product is a view made inside its autograd function, which cannot)
                z = z.index_add_(axis, layer.redriven, add) if by_neuron else z.index_add(axis, layer.redriven, add)
            h = fire(z, layer.nid)
            if watch is not None:
                watch(h)
        top = h.index_select(axis, self.dn_rows)
        return self.out(top.t() if by_neuron else top)

    # ---- CPU play
    def _host_decider(self) -> "_HostDecider | None":
        """The CPU decision library loaded with the current weights (rebuilt when a weight changed), or None when it
        is not built, FLYGUY_NATIVE=0 or the weights are not float32."""
        import os
        stamp = _weights_stamp(self)
        held = getattr(self, "_decider", None)
        if held is not None and held[0] == stamp:
            return held[1]
        if held is not None and held[1] is not None:
            held[1].close()
        dec = None
        if os.environ.get("FLYGUY_NATIVE", "1") != "0" and self.w.dtype == torch.float32 and _HostDecider.LIB.exists():
            dec = _HostDecider(self, os.environ.get("FLYGUY_CPU_THREADS"))
        self._decider = (stamp, dec)
        return dec

    def _host_matrices(self) -> list[torch.Tensor]:
        """The products as sparse CSR matrices of the current weights ([rows, sources]), made once per weights."""
        stamp = _weights_stamp(self)[:5]
        held = getattr(self, "_host_csr", None)
        if held is None or held[0] != stamp:
            mats = []
            for layer in self._layers():
                p = layer.prod
                w = (self.in_w if layer.edges is None else self.w[layer.edges]).detach().clone()
                mats.append(torch.sparse_csr_tensor(p.crow, p.c, w, size=(p.n_rows, p.n_src)))
            held = (stamp, mats)
            self._host_csr = held
        return held[1]

    @torch.no_grad()
    def _play(self, obs: torch.Tensor) -> torch.Tensor:
        """A decision on the CPU (the bot): the CPU decision library when it is there, else sparse CSR products of
        the current weights (fly.py:186-284).  A visualizer tap (self.tap) gets the first sample's firing."""
        tap = getattr(self, "tap", None)
        dec = self._host_decider()
        if dec is not None:
            return dec.decide(obs, tap)
        mats = self._host_matrices()
        first = [] if tap is not None else None
        logits = self._walk(obs.t().contiguous(), lambda k, layer, w, h: torch.sparse.mm(mats[k], h),
                            by_neuron=True, watch=(lambda h: first.append(h[:, 0])) if first is not None else None)
        if tap is not None:
            tap(first)
        return logits

    # ---- forward
    def forward(self, obs: torch.Tensor, extra: torch.Tensor | None = None) -> torch.Tensor:
        obs = obs.double() if self.w.dtype == torch.float64 else obs.float()    # (float64: an actor made .double())
        if not obs.is_cuda and not torch.is_grad_enabled():
            return self._play(obs)
        if self.kernel != "torch" and obs.is_cuda and obs.shape[0] % 32 == 0:      # (at any batch size)
            from .fly_hip import FireHip, HopHip
            half = self.kernel == "cuda16"

            def on_library(k, layer, w, h):
                p = layer.prod
                return HopHip.apply(w, h, p.crow, p.ci, p.tcrow, p.tci, p.tperm, half and k > 0)
            activate = FireHip.apply if self.w.dtype == torch.float32 else None
            return self._walk(obs.t().contiguous(), on_library, by_neuron=True, activate=activate)

        few = obs.shape[0] * self.used <= self.gather_limit        # a few samples: gather / scatter products

        def in_torch(k, layer, w, h):
            p = layer.prod
            if few:
                return h.new_zeros(h.shape[0], p.n_rows).index_add_(1, p.r, h[:, p.c] * w)
            return _RowProduct.apply(w, h, p.crow, p.c, p.tcrow, p.tcol, p.tperm)
        return self._walk(obs, in_torch, by_neuron=False)


class _Csr(NamedTuple):
    """The index buffers of one sparse product: per connection its row (target) and column (source), CSR row
    pointer, the by-source form (row pointer over sources, rows, and the permutation into CSR order) and int32 copies
    of the columns / by-source rows."""
    r: torch.Tensor
    c: torch.Tensor
    crow: torch.Tensor
    tcrow: torch.Tensor
    tcol: torch.Tensor
    tperm: torch.Tensor
    ci: torch.Tensor
    tci: torch.Tensor
    n_rows: int
    n_src: int


class _Layer(NamedTuple):
    prod: _Csr
    edges: torch.Tensor | None     # the connections' indices into w (None: the plug, whose weights are in_w)
    nid: torch.Tensor              # the neuron of each row
    redriven: torch.Tensor         # rows that are sensory neurons, kept driven by the observation ...
    drive_rows: torch.Tensor       # ... and their rows in the sensory layer


def _weights_stamp(f: FlyActor) -> tuple:
    """Changes whenever a weight does (PyTorch bumps a tensor's version on every in-place change)."""
    return (f.w._version, f.in_w._version, f.gain._version, f.theta._version, f.in_b._version,
            f.out.weight._version, f.out.bias._version, f.w.dtype)


class _RowProduct(torch.autograd.Function):
    """z[b, i] = sum over the connections e of row i of w[e] h[b, col[e]] for states [B, sources] -> [B, rows],
    with a backward of its own (fly.py:51-72): the transposed product for h, and for w the product sampled at the
    connections only, instead of the dense rows x sources gradient PyTorch's sparse products would build."""

    @staticmethod
    def forward(ctx, w, h, crow, col, tcrow, tcol, tperm):
        n_rows, n_src = crow.numel() - 1, h.shape[1]
        ctx.save_for_backward(w, h, crow, col, tcrow, tcol, tperm)
        return torch.sparse.mm(torch.sparse_csr_tensor(crow, col, w, size=(n_rows, n_src)), h.t()).t()

    @staticmethod
    def backward(ctx, gz):
        w, h, crow, col, tcrow, tcol, tperm = ctx.saved_tensors
        n_rows, n_src = crow.numel() - 1, h.shape[1]
        want_w, want_h = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        gw = gh = None
        if want_w:               # <gz[:, row], h[:, col]> at every connection, through a sampled dense product
            mask = torch.sparse_csr_tensor(crow, col, torch.zeros_like(w), size=(n_rows, n_src))
            gw = torch.sparse.sampled_addmm(mask, gz.t().contiguous(), h, beta=0.0, alpha=1.0).values()
        if want_h:               # A^T gz through the by-source form (weights in by-source order)
            at = torch.sparse_csr_tensor(tcrow, tcol, w[tperm], size=(n_src, n_rows))
            gh = torch.sparse.mm(at, gz.t()).t()
        return gw, gh, None, None, None, None, None


class _HostDecider:
    """The CPU decision library (flyguy_amd/libfly_infer.so, include/fly_infer.h: a hop pushes the neurons that fire
    along their outgoing connections) with one version of an actor's weights (fly.py:186-250).  threads: None (one
    thread, as the reference), or a count for fly_set_threads (0: one per hardware thread), with bit-identical
    answers."""

    LIB = Path(__file__).resolve().parent / "libfly_infer.so"
    _lib = None

    @classmethod
    def library(cls):
        import ctypes
        if cls._lib is None:
            L = ctypes.CDLL(str(cls.LIB))
            vp, ci = ctypes.c_void_p, ctypes.c_int
            sig = {"fly_create": (vp, [ci, ci, ci]), "fly_set_plug": (None, [vp, ci, ci] + [vp] * 6),
                   "fly_set_hop": (None, [vp, ci, ci, ci, ci] + [vp] * 6), "fly_set_out": (None, [vp, ci, vp, vp, vp]),
                   "fly_forward": (None, [vp, vp, ci, vp, vp]), "fly_free": (None, [vp]),
                   "fly_set_threads": (None, [vp, ci])}
            for name, (res, args) in sig.items():
                fn = getattr(L, name)
                fn.restype, fn.argtypes = res, args
            cls._lib = L
        return cls._lib

    def __init__(self, f: FlyActor, threads: str | None):
        L = self.library()
        held = []                          # the arrays handed over (the library copies them during set-up)

        def ptr(t, dtype):
            a = np.ascontiguousarray(t.detach().cpu().numpy() if torch.is_tensor(t) else t, dtype=dtype)
            held.append(a)
            return a.ctypes.data

        i32, f32 = np.int32, np.float32
        self.n_act = f.out.out_features
        with torch.no_grad():
            thr = nn.functional.softplus(f.theta)
            self.h = L.fly_create(f.obs_dim, self.n_act, f.hops)
            plug = f._layers()[0]
            L.fly_set_plug(self.h, f.sizes[0], int(plug.prod.ci.numel()), ptr(plug.prod.crow, i32), ptr(plug.prod.ci, i32),
                           ptr(f.in_w, f32), ptr(f.in_b, f32), ptr(f.gain[f.n0], f32), ptr(thr[f.n0], f32))
            for k, layer in enumerate(f._layers()[1:], start=1):
                p = layer.prod
                redrive = np.full(p.n_rows, -1, i32)
                redrive[layer.redriven.cpu().numpy()] = layer.drive_rows.cpu().numpy()
                by_source = f.w[layer.edges[p.tperm]]              # strengths in the by-source order
                L.fly_set_hop(self.h, k - 1, p.n_rows, p.n_src, int(by_source.numel()), ptr(p.tcrow, i32), ptr(p.tci, i32),
                              ptr(by_source, f32), ptr(f.gain[layer.nid], f32), ptr(thr[layer.nid], f32),
                              ptr(redrive, i32))
            L.fly_set_out(self.h, len(f.dn_rows), ptr(f.dn_rows, i32), ptr(f.out.weight, f32), ptr(f.out.bias, f32))
            if threads is not None:
                L.fly_set_threads(self.h, int(threads))
        self.shade = np.zeros(int(sum(f.sizes)), np.uint8)

    def decide(self, obs: torch.Tensor, tap=None) -> torch.Tensor:
        x = np.ascontiguousarray(obs.detach().numpy(), dtype=np.float32)
        out = np.empty((x.shape[0], self.n_act), np.float32)
        self.library().fly_forward(self.h, x.ctypes.data, x.shape[0], out.ctypes.data,
                                   self.shade.ctypes.data if tap is not None else None)
        if tap is not None:
            tap(self.shade)
        return torch.from_numpy(out)

    def close(self) -> None:
        if self.h:
            self.library().fly_free(self.h)
            self.h = None


class VizTap:
    """A live window for the visualizer into a playing actor (fly.py:308-368): after every decision the firing of
    every neuron in play, layer by layer, one byte each, and the chosen action go into a small memory-mapped file;
    readers (the visualizer's server) map it, and nothing waits for them.  Set `actor.tap = VizTap(actor.sizes)`.

    The file is a fixed layout (little endian): the header fields below at their byte offsets, the firing bytes from
    byte 512 (sensory layer first), each 255 * tanh(1.5 * firing) truncated to a byte.  `seq` is odd while a
    decision is being written, so a reader that sees the same even seq before and after its read has a whole one."""

    FIRING = 512
    _FIELDS = {                            # name: (offset, struct format)
        "magic": (0, "<4sI"),              #   "FLYV", layout version 1
        "seq": (8, "<I"),
        "stamp": (12, "<Idi"),             #   decisions published, wall time, action
        "controls": (28, "<8f"),
        "layers": (60, "<5I"),             #   layer count, first 4 layer sizes
        "probs": (80, "<90f"),
        "clock": (440, "<fIi"),            #   match clock, game frame, overtime
    }

    def __init__(self, sizes, path=None):
        import mmap
        import tempfile
        self.sizes = [int(v) for v in sizes]
        self.path = Path(path) if path else Path(tempfile.gettempdir()) / "flyguy_viz.bin"
        length = self.FIRING + sum(self.sizes)
        # a file of the right length is used as it is: a reader may have it mapped, and replacing it would cut them off
        if not (self.path.exists() and self.path.stat().st_size == length):
            self.path.write_bytes(bytes(length))
        self.fh = open(self.path, "r+b")
        self.mm = mmap.mmap(self.fh.fileno(), length)
        self._put("magic", b"FLYV", 1)
        self._put("layers", len(self.sizes), *(self.sizes + [0, 0, 0, 0])[:4])
        self.seq = self.tick = 0
        self.acts = None

    def _put(self, field: str, *values) -> None:
        at, fmt = self._FIELDS[field]
        struct.pack_into(fmt, self.mm, at, *values)

    def __call__(self, acts) -> None:
        """From the actor's forward pass: the first sample's firing (bytes from the CPU library, or one tensor per
        layer from the sparse products)."""
        self.acts = acts

    def _firing_bytes(self) -> bytes:
        if isinstance(self.acts, np.ndarray):
            return self.acts.astype(np.uint8).tobytes()
        return b"".join((torch.tanh(1.5 * a.float()) * 255.0).to(torch.uint8).cpu().numpy().tobytes()
                        for a in self.acts)

    def publish(self, action: int, controls, probs, clock: float = -1.0, frame: int = 0, overtime: bool = False) -> None:
        """Write the last decision: its firing, the action, the 8 controls and the action probabilities; clock /
        frame / overtime let a recording of the page be lined up with one of the game."""
        import time
        if self.acts is None:
            return
        body = self._firing_bytes()
        self.seq += 1                                   # odd: being written
        self._put("seq", self.seq)
        self.mm[self.FIRING:self.FIRING + len(body)] = body
        self.tick += 1
        self._put("stamp", self.tick, time.time(), int(action))
        self._put_floats("controls", np.asarray(controls, np.float32)[:8])
        self._put_floats("probs", np.asarray(probs, np.float32)[:90])
        self._put("clock", float(clock), int(frame) & 0xFFFFFFFF, int(bool(overtime)))
        self.seq += 1                                   # even: whole
        self._put("seq", self.seq)
        self.acts = None

    def _put_floats(self, field: str, v: np.ndarray) -> None:
        """The first len(v) floats of a field (a caller may give fewer than the field holds)."""
        at = self._FIELDS[field][0]
        self.mm[at:at + 4 * len(v)] = v.tobytes()

    def close(self) -> None:
        self.mm.close()
        self.fh.close()
