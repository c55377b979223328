"""ORACLE - test infrastructure only: the library's row plans, restated in plain Python / numpy.

The plans have no counterpart in the reference (the reference gives every (row, sample) one thread); they fix the
order in which the MI355X kernels visit rows and where each edge's (source, weight) pair is stored.  Rule of one
product (`plan`):
- a row of d edges is one segment if d <= seg_max, else ceil(d / seg_max) segments [b + d*s//n, b + d*(s+1)//n)
  numbered with consecutive partial-sum slots;
- segments are ordered by length, longest first; among equal lengths, whole rows whose re-drive field is >= 0 (they
  read a line of the drive, or of the drive gradient written so far) come first, then (row, segment) order; they
  are dealt 8 to a wave;
- wave w starts at position woff[w] (the running total) and takes 64 positions per 8 edges of its longest segment;
  edge k of the segment of group g sits at woff[w] + 64 (k // 8) + 8 g + k % 8; other positions hold no edge.
A network's plans (`net_plans`): the plug's rows without re-drive fields; per hop its CSR rows with the hop's drow,
and its CSC rows (the layer below) with the backward's re-drive fields (`backward_drive_fields`); each cut at
`seg_cap` of the product's edge count.  The backward's reduction tables: per hop the neuron of each gain / threshold
partial column (segments, then split rows), and first-write marks in the order of reductions.
tests/test_plan.py checks the library's fc_plan_rows / fc_net_plan / fc_net_marks against this bit for bit, and
checks the rules' invariants (every edge at exactly one position, each segment's edges in CSR order, slots a
permutation, the tie-break, every gradient entry marked first exactly once and before its other writes) so that
this restatement is pinned by more than itself.
"""
from __future__ import annotations

import numpy as np


def seg_cap(n_edges: int) -> int:
    """The segment cap of a product of n_edges edges: at least 4096 segments, between 16 and 512 edges."""
    return int(min(512, max(16, -(-int(n_edges) // 4096))))


def plan(rowptr, seg_max: int = 256, drow=None):
    """(wave [(woff, longest)], seg [(row, slot, field, 0)], split [(row, first slot, n, field)], nslot,
    pos int array [edge or -1]); field = drow[row] (-1 without drow)."""
    rowptr = np.asarray(rowptr, np.int64)
    field = (lambda r: int(drow[r])) if drow is not None else (lambda r: -1)
    segs, split, nslot = [], [], 0
    for r in range(len(rowptr) - 1):
        b, e = int(rowptr[r]), int(rowptr[r + 1])
        d = e - b
        if d <= seg_max:
            segs.append((r, b, e, -1))
            continue
        n = -(-d // seg_max)
        split.append((r, nslot, n, field(r)))
        for s in range(n):
            segs.append((r, b + d * s // n, b + d * (s + 1) // n, nslot + s))
        nslot += n

    def loads(i):
        r, _, _, slot = segs[i]
        return drow is not None and slot < 0 and field(r) >= 0
    order = sorted(range(len(segs)), key=lambda i: (-(segs[i][2] - segs[i][1]), not loads(i), i))
    segs = [segs[i] for i in order]
    wave, at = [], 0
    for w in range(0, len(segs), 8):
        longest = max(e - b for _, b, e, _ in segs[w:w + 8])
        wave.append((at, longest))
        at += 64 * -(-longest // 8)
    pos = np.full(at, -1, np.int64)
    for i, (_, b, e, _) in enumerate(segs):
        k = np.arange(e - b)
        pos[wave[i // 8][0] + 8 * (i % 8) + 64 * (k // 8) + k % 8] = b + k
    return wave, [(r, slot, field(r), 0) for r, _, _, slot in segs], split, nslot, pos


def backward_drive_fields(drows: list, n_s: int):
    """The backward's re-drive fields.  Hops write the drive's gradient from the top down; a row of hop k's layer
    whose sensory row no hop above re-drives writes it first: field -(d + 3).  Returns (per hop below the top: the
    fields of its rows, or None for the top hop; the sensory rows' fields: -1 if some hop re-drives the row, else
    -2)."""
    K = len(drows)
    touched = np.zeros(n_s, bool)
    out = [None] * K
    for L in range(K, 0, -1):
        dr = np.asarray(drows[L - 1], np.int64)
        if L < K:
            out[L - 1] = np.where((dr >= 0) & ~touched[np.maximum(dr, 0)], -(dr + 3), dr)
        touched[dr[dr >= 0]] = True
    return out, np.where(touched, -1, -2)


def first_writes(idx, seen: np.ndarray) -> np.ndarray:
    """Marks of one index array in reduction order: -1 no entry, -(i + 2) the first write of entry i (not seen in
    this array before nor in an earlier array: `seen`, updated), i a later write."""
    idx = np.asarray(idx, np.int64)
    out = np.full(len(idx), -1, np.int64)
    live = np.flatnonzero(idx >= 0)
    v = idx[live]
    first = np.zeros(len(v), bool)
    first[np.unique(v, return_index=True)[1]] = True
    first &= ~seen[v]
    out[live] = np.where(first, -(v + 2), v)
    seen[v] = True
    return out


def net_plans(s: dict) -> dict:
    """The plans and reduction tables of a network given as NET.bin's arrays (flyguy_amd.export.read_net's dict):
    {"plug": plan, "fwd": [plan per hop], "bwd": [plan per hop], "gidx": [...], "ridx": [...], "gridx": [...],
    "top": marks}."""
    K = s["hops"]
    hops = s["hop"]
    E_in = s["n_s"] * s["fan"]
    out = {"plug": plan(s["in_crow"], seg_cap(E_in)), "fwd": [], "bwd": [], "gidx": [], "ridx": [], "gridx": []}
    fields, sensory = backward_drive_fields([h["drow"] for h in hops], s["n_s"])
    strengths = []
    for k, h in enumerate(hops):
        E = len(h["col"])
        out["fwd"].append(plan(h["crow"], seg_cap(E), h["drow"]))
        b = plan(h["tcrow"], seg_cap(E), fields[k - 1] if k >= 1 else sensory)
        out["bwd"].append(b)
        _, seg, split, _, pos = b
        below = np.asarray(hops[k - 1]["nid"] if k >= 1 else s["n0"], np.int64)
        gidx = [int(below[r]) if slot < 0 else -1 for r, slot, _, _ in seg] + [int(below[r]) for r, _, _, _ in split]
        out["gidx"].append(np.asarray(gidx, np.int64))
        twidx = np.asarray(h["twidx"], np.int64)
        strengths.append(np.where(pos >= 0, twidx[np.maximum(pos, 0)], -1))
    wseen = np.zeros(max(s["n_w"], 1), bool)
    nseen = np.zeros(s["n_neurons"], bool)
    out["top"] = first_writes(hops[K - 1]["nid"], nseen)
    out["ridx"], out["gridx"] = [None] * K, [None] * K
    for k in range(K - 1, -1, -1):
        out["ridx"][k] = first_writes(strengths[k], wseen)
        out["gridx"][k] = first_writes(out["gidx"][k], nseen)
    return out
