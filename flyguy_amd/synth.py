"""Synthetic networks of the benchmark shapes, built directly as library structures (the dict of export.structure).

The 3-hop shape of the batched benchmarks: layers of 16,894 sensory, 46,393, 37,748 and 1,332 descending rows;
hops of 1,200,000, 1,500,000 and 292,734 connections (2,992,734 strengths); per hop the in-degree of a row is
drawn LogNormal(0, sigma) and scaled to the hop's count by largest remainder, sources are uniform without
repetition within a row.  As in the real graph some hop rows are sensory neurons that the observation keeps
driving (re-drive rows: 12,698 / 5,278 / 12 of them); they share their neuron (gain, threshold) with the
sensory layer.  Weights N(0, 1/fan_in), gain 1, theta -4, plug weights N(0, 1/fan), read-out N(0, 1/n_dn),
biases 0.  kind="er" gives the Erdos-Renyi control: uniform (multinomial) in-degrees with the same counts.
"""
from __future__ import annotations

import numpy as np

from .fly import rowptr

SHAPE_3HOP = dict(sizes=(16894, 46393, 37748, 1332), edges=(1_200_000, 1_500_000, 292_734),
                  redrive=(12698, 5278, 12), obs_dim=517, n_act=90, fan=16)


def _degrees(rng, rows: int, total: int, cap: int, sigma: float, kind: str) -> np.ndarray:
    if total > rows * cap:
        raise ValueError("more connections than distinct (source, target) pairs")
    if kind == "er":
        d = rng.multinomial(total, np.full(rows, 1.0 / rows)).astype(np.int64)
    else:
        share = rng.lognormal(0.0, sigma, rows)
        share = share / share.sum() * total
        d = np.floor(share).astype(np.int64)
        rem = total - int(d.sum())
        if rem:
            d[np.argsort(-(share - d), kind="stable")[:rem]] += 1
    while d.max() > cap:                                     # give the excess of over-full rows to the others
        over = d > cap
        excess = int((d[over] - cap).sum())
        d[over] = cap
        room = np.flatnonzero(d < cap)
        add = rng.multinomial(excess, np.full(len(room), 1.0 / len(room)))
        d[room] += add
    return d


def _unique_sources(rng, d: np.ndarray, n_src: int) -> tuple[np.ndarray, np.ndarray]:
    """Row and source of every connection, sorted by (row, source), no repeated source within a row."""
    row = np.repeat(np.arange(len(d), dtype=np.int64), d)
    col = rng.integers(0, n_src, len(row), dtype=np.int64)
    while True:
        order = np.lexsort((col, row))
        col = col[order]
        dup = np.flatnonzero((col[1:] == col[:-1]) & (row[1:] == row[:-1])) + 1
        if len(dup) == 0:
            return row, col
        col[dup] = rng.integers(0, n_src, len(dup), dtype=np.int64)


def _unique_sources_large(rng, d: np.ndarray, n_src: int) -> tuple[np.ndarray, np.ndarray]:
    """_unique_sources for large graphs: one sort of (row, source) keys, then only the rows that still hold a repeated
    source are redrawn and re-sorted."""
    row = np.repeat(np.arange(len(d), dtype=np.int64), d)
    key = row * n_src + rng.integers(0, n_src, len(row), dtype=np.int64)
    key.sort()
    while True:
        dup = np.flatnonzero(key[1:] == key[:-1]) + 1
        if len(dup) == 0:
            return row, key - row * n_src
        key[dup] = row[dup] * n_src + rng.integers(0, n_src, len(dup), dtype=np.int64)
        sel = np.flatnonzero(np.isin(row, np.unique(row[dup])))      # whole rows, contiguous and in row order
        key[sel] = np.sort(key[sel])


def synth_3hop(sizes=SHAPE_3HOP["sizes"], edges=SHAPE_3HOP["edges"], redrive=SHAPE_3HOP["redrive"],
               obs_dim: int = 517, n_act: int = 90, fan: int = 16, sigma: float = 1.5, kind: str = "lognormal",
               seed: int = 1000) -> tuple[dict, list[np.ndarray]]:
    """(structure dict, the seven initial weight arrays) of a synthetic layered network."""
    sizes, edges, redrive = list(sizes), list(edges), list(redrive)
    K = len(edges)
    assert len(sizes) == K + 1 and len(redrive) == K
    n0 = np.arange(sizes[0], dtype=np.int64)
    next_id = sizes[0]
    hops, weights = [], []
    w_base = 0
    for k in range(1, K + 1):
        rng = np.random.default_rng(seed + k)
        rows, src, E = sizes[k], sizes[k - 1], edges[k - 1]
        d = _degrees(rng, rows, E, src, sigma, kind)
        row, col = _unique_sources(rng, d, src)
        widx = w_base + np.arange(E, dtype=np.int64)
        w_base += E
        fan_in = np.maximum(d[row], 1).astype(np.float64)
        weights.append((rng.standard_normal(E) / np.sqrt(fan_in)).astype(np.float32))
        by_col = np.lexsort((row, col))
        drow = np.full(rows, -1, np.int64)
        nid = np.empty(rows, np.int64)
        dr = min(redrive[k - 1], rows, sizes[0])
        kept = np.sort(rng.choice(rows, dr, replace=False)) if dr else np.zeros(0, np.int64)
        drow[kept] = rng.choice(sizes[0], dr, replace=False) if dr else drow[kept]
        fresh = drow < 0
        nid[~fresh] = n0[drow[~fresh]]
        nid[fresh] = next_id + np.arange(int(fresh.sum()))
        next_id += int(fresh.sum())
        hops.append({"nid": nid, "crow": rowptr(row, rows), "col": col, "widx": widx, "tcrow": rowptr(col[by_col], src),
                     "tcol": row[by_col], "twidx": widx[by_col], "drow": drow})
    # the plug, as FlyActor draws it (fly.py:141-149)
    prng = np.random.default_rng(0)
    n_s = sizes[0]
    picks = np.empty((n_s, fan), np.int64)
    for i in range(n_s):
        picks[i] = np.sort(prng.choice(obs_dim, size=fan, replace=False))
    cols = picks.reshape(-1)
    prow = np.repeat(np.arange(n_s), fan)
    by_col = np.lexsort((prow, cols))
    n_w = w_base
    s = {"obs_dim": obs_dim, "n_act": n_act, "hops": K, "n_neurons": next_id, "n_w": n_w, "n_s": n_s, "fan": fan,
         "n_dn": sizes[K], "sizes": sizes, "wmap": np.arange(n_w, dtype=np.int64),
         "in_crow": rowptr(prow, n_s), "in_col": cols, "in_tcrow": rowptr(cols[by_col], obs_dim), "in_tcol": prow[by_col],
         "in_tperm": by_col, "n0": n0, "dn_rows": np.arange(sizes[K], dtype=np.int64), "hop": hops}
    rng = np.random.default_rng(seed)
    params = [np.concatenate(weights) if weights else np.zeros(0, np.float32),
              np.ones(next_id, np.float32), np.full(next_id, -4.0, np.float32),
              (rng.standard_normal(n_s * fan) / np.sqrt(fan)).astype(np.float32), np.zeros(n_s, np.float32),
              (rng.standard_normal(n_act * sizes[K]) / np.sqrt(sizes[K])).astype(np.float32),
              np.zeros(n_act, np.float32)]
    return s, params


WHOLE = dict(neurons=166_700, connections=15_283_167, sensory=16_894, descending=1_332)
TRANSMITTERS = ("acetylcholine", "gaba", "glutamate", "dopamine", "serotonin", "octopamine", "histamine")


def whole_connectome(neurons: int = WHOLE["neurons"], connections: int = WHOLE["connections"],
                     sensory: int = WHOLE["sensory"], descending: int = WHOLE["descending"], sigma: float = 1.8,
                     seed: int = 4) -> dict:
    """A synthetic graph file of the whole-connectome shape (the arrays FlyActor reads: body, pre, post, syn, nt,
    sensory, descending): in-degrees LogNormal(0, sigma) scaled to the connection count, sources uniform without
    repetition, connections in random order, synapse counts 1..20, transmitters drawn per neuron (a third
    inhibitory), disjoint random sensory and descending sets.  FlyActor then keeps, per hop, the connections that
    can carry the signal (its pruning, fly.py:91-121)."""
    rng = np.random.default_rng(seed)
    d = _degrees(rng, neurons, connections, neurons, sigma, "lognormal")
    post, pre = _unique_sources_large(rng, d, neurons)
    perm = rng.permutation(connections)
    ids = rng.permutation(neurons)
    return {"body": np.arange(neurons, dtype=np.int64), "pre": pre[perm].astype(np.int32),
            "post": post[perm].astype(np.int32), "syn": rng.integers(1, 21, connections).astype(np.int32),
            "nt": np.asarray(TRANSMITTERS)[rng.choice(len(TRANSMITTERS), neurons,
                                                      p=[0.5, 0.15, 0.12, 0.06, 0.06, 0.05, 0.06])],
            "sensory": np.sort(ids[:sensory]).astype(np.int32),
            "descending": np.sort(ids[sensory:sensory + descending]).astype(np.int32)}


def scaled_3hop(div: int, **kw) -> tuple[dict, list[np.ndarray]]:
    """The 3-hop shape with every layer, hop and re-drive count divided by `div` (test sizes)."""
    sizes = [max(8, v // div) for v in SHAPE_3HOP["sizes"]]
    edges = [max(16, v // div) for v in SHAPE_3HOP["edges"]]
    redrive = [min(v // div, sizes[k + 1] // 2) for k, v in enumerate(SHAPE_3HOP["redrive"])]
    return synth_3hop(sizes=sizes, edges=edges, redrive=redrive, **kw)
