"""ORACLE - test infrastructure only: the fly actor's graph indexing in plain Python (no numpy sorting).

Restates FlyActor.__init__ (flyguy/fly.py:35-154) and export.structure / write_net (flyguy/native/export.py:32-65)
with Python sets, dicts and sorted(); meant for toy graphs.  Pinned by tests/test_index.py against the golden
vectors that tests/golden/make_golden.py wrote from the reference's own code (every buffer, the initial strengths
and the NET.bin bytes of eight toy networks).  The plug's observation columns come from numpy's
Generator.choice, as in the reference (fly.py:141-143): that draw is part of the format of a checkpoint.
"""
from __future__ import annotations

import struct

import numpy as np

INHIBITORY = ("gaba", "glutamate", "histamine")                 # fly.py:32


def reach(start, pre, post, steps):
    """[set of neurons within k steps of `start` along pre -> post for k = 0..steps]  (fly.py:35-43)."""
    cur = set(int(s) for s in start)
    out = [set(cur)]
    for _ in range(steps):
        nxt = set(cur)
        for a, b in zip(pre, post):
            if a in cur:
                nxt.add(b)
        cur = nxt
        out.append(set(cur))
    return out


def rowptr(rows, n):
    """CSR row pointer of a row list grouped by row (fly.py:46-48)."""
    counts = [0] * n
    for r in rows:
        counts[r] += 1
    out = [0]
    for c in counts:
        out.append(out[-1] + c)
    return out


def index(graph: dict, obs_dim: int, hops: int, fan: int, seed: int = 0) -> dict:
    """Every buffer FlyActor registers, as Python lists, plus sizes / used / in_play and the initial strengths."""
    pre = [int(v) for v in graph["pre"]]
    post = [int(v) for v in graph["post"]]
    syn = [float(v) for v in graph["syn"]]
    n = len(graph["body"])
    sens, dn = [int(v) for v in graph["sensory"]], [int(v) for v in graph["descending"]]
    down = reach(sens, pre, post, hops)
    up = reach(dn, post, pre, hops)
    sets = [sorted(down[k] & up[hops - k]) for k in range(hops + 1)]
    pos = [{v: i for i, v in enumerate(s)} for s in sets]
    is_sens = set(sens)
    out: dict = {"sizes": [len(s) for s in sets]}
    used, in_play = 0, set()
    for k in range(1, hops + 1):
        edges = [(pos[k][post[m]], pos[k - 1][pre[m]], m) for m in range(len(pre))
                 if pre[m] in pos[k - 1] and post[m] in pos[k]]
        csr = sorted(edges)                                     # by target, then source (then original order)
        r = [e[0] for e in csr]
        c = [e[1] for e in csr]
        t = sorted(range(len(csr)), key=lambda i: (c[i], r[i], i))   # by source, then target: the transpose
        out[f"e{k}"] = [e[2] for e in csr]
        out[f"r{k}"], out[f"c{k}"] = r, c
        out[f"crow{k}"] = rowptr(r, len(sets[k]))
        out[f"tcrow{k}"] = rowptr([c[i] for i in t], len(sets[k - 1]))
        out[f"tcol{k}"] = [r[i] for i in t]
        out[f"tperm{k}"] = t
        out[f"ci{k}"], out[f"tci{k}"] = list(c), [r[i] for i in t]
        out[f"n{k}"] = sets[k]
        out[f"s{k}"] = [i for i, v in enumerate(sets[k]) if v in is_sens]
        out[f"d{k}"] = [pos[0][v] for v in sets[k] if v in is_sens]
        used += len(csr)
        in_play.update(e[2] for e in csr)
    out["n0"] = sets[0]
    out["dn_rows"] = [pos[hops][v] for v in dn if v in pos[hops]]
    out["used"], out["in_play"] = used, len(in_play)
    # initial strengths: 1.5 * sign(transmitter) * synapses / incoming synapses of the target, in float32
    if "in_total" in graph:
        total = [np.float32(v) for v in graph["in_total"]]
    else:
        total = [np.float32(0)] * n
        for p, s in zip(post, syn):
            total[p] = np.float32(total[p] + np.float32(s))
    nt = list(graph["nt"])
    w = []
    for p, q, s in zip(pre, post, syn):
        sign = np.float32(-1.0 if nt[p] in INHIBITORY else 1.0)
        w.append(np.float32(np.float32(np.float32(1.5) * sign) * np.float32(s)) / max(total[q], np.float32(1.0)))
    out["w"] = np.array(w, np.float32)
    # the plug (fly.py:140-148)
    rng = np.random.default_rng(seed)
    n_s = len(sets[0])
    cols, rows = [], []
    for i in range(n_s):
        cols += sorted(int(v) for v in rng.choice(obs_dim, size=fan, replace=False))
        rows += [i] * fan
    t = sorted(range(len(cols)), key=lambda i: (cols[i], rows[i], i))
    out.update(in_r=rows, in_c=cols, in_crow=rowptr(rows, n_s), in_tcrow=rowptr([cols[i] for i in t], obs_dim),
               in_tcol=[rows[i] for i in t], in_tperm=t, in_ci=list(cols), in_tci=[rows[i] for i in t])
    return out


def structure(ix: dict, graph_n: int, obs_dim: int, n_act: int, hops: int, fan: int) -> dict:
    """export.structure (export.py:32-49) from the index lists."""
    used = sorted(set(m for k in range(1, hops + 1) for m in ix[f"e{k}"]))
    comp = {m: i for i, m in enumerate(used)}
    s = {"obs_dim": obs_dim, "n_act": n_act, "hops": hops, "n_neurons": graph_n, "n_w": len(used), "n_s": ix["sizes"][0],
         "fan": fan, "n_dn": len(ix["dn_rows"]), "sizes": ix["sizes"], "wmap": used, "in_crow": ix["in_crow"],
         "in_col": ix["in_ci"], "in_tcrow": ix["in_tcrow"], "in_tcol": ix["in_tci"], "in_tperm": ix["in_tperm"],
         "n0": ix["n0"], "dn_rows": ix["dn_rows"], "hop": []}
    for k in range(1, hops + 1):
        widx = [comp[m] for m in ix[f"e{k}"]]
        drow = [-1] * ix["sizes"][k]
        for a, b in zip(ix[f"s{k}"], ix[f"d{k}"]):
            drow[a] = b
        s["hop"].append({"nid": ix[f"n{k}"], "crow": ix[f"crow{k}"], "col": ix[f"ci{k}"], "widx": widx,
                         "tcrow": ix[f"tcrow{k}"], "tcol": ix[f"tci{k}"], "twidx": [widx[i] for i in ix[f"tperm{k}"]],
                         "drow": drow})
    return s


def net_bytes(s: dict) -> bytes:
    """NET.bin, field by field (export.py:9-15,52-65)."""
    def ints(v):
        return b"".join(struct.pack("<i", int(x)) for x in v)
    b = [b"FLY1", ints([s["obs_dim"], s["n_act"], s["hops"], s["n_neurons"], s["n_w"], s["n_s"], s["fan"], s["n_dn"]]),
         ints(s["sizes"]), ints([len(h["col"]) for h in s["hop"]])]
    for key in ("in_crow", "in_col", "in_tcrow", "in_tcol", "in_tperm", "n0"):
        b.append(ints(s[key]))
    for h in s["hop"]:
        for key in ("nid", "crow", "col", "widx", "tcrow", "tcol", "twidx", "drow"):
            b.append(ints(h[key]))
    b += [ints(s["dn_rows"]), ints(s["wmap"])]
    return b"".join(b)
