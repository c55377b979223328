"""ORACLE - test infrastructure only: the library's row plan, restated in plain Python.

The plan has no counterpart in the reference (the reference gives every (row, sample) one thread); it fixes the
order in which the MI355X kernels visit rows and where each edge's (source, weight) pair is stored.  Rule:
- a row of d edges is one segment if d <= seg_max, else ceil(d / seg_max) segments [b + d*s//n, b + d*(s+1)//n)
  numbered with consecutive partial-sum slots;
- segments are ordered by length, longest first, equal lengths in (row, segment) order, and dealt 8 to a wave;
- wave w starts at position woff[w] (the running total) and takes 64 positions per 8 edges of its longest segment;
  edge k of the segment of group g sits at woff[w] + 64 (k // 8) + 8 g + k % 8; other positions hold no edge.
tests/test_plan.py checks the library's fc_plan_rows against this bit for bit, and checks the rule's invariants
(every edge at exactly one position, each segment's edges in CSR order, slots a permutation) so that this
restatement is pinned by more than itself.
"""
from __future__ import annotations


def plan(rowptr, seg_max: int = 256):
    """(wave [(woff, longest)], seg [(row, slot, -1, 0)], split [(row, first slot, n, -1)], nslot, pos [edge or -1])"""
    segs, split, nslot = [], [], 0
    for r in range(len(rowptr) - 1):
        b, e = int(rowptr[r]), int(rowptr[r + 1])
        d = e - b
        if d <= seg_max:
            segs.append((r, b, e, -1))
            continue
        n = -(-d // seg_max)
        split.append((r, nslot, n, -1))
        for s in range(n):
            segs.append((r, b + d * s // n, b + d * (s + 1) // n, nslot + s))
        nslot += n
    order = sorted(range(len(segs)), key=lambda i: (-(segs[i][2] - segs[i][1]), i))
    segs = [segs[i] for i in order]
    wave, pos, at = [], [], 0
    for w in range(0, len(segs), 8):
        group = segs[w:w + 8]
        longest = max(e - b for _, b, e, _ in group)
        steps = -(-longest // 8)
        block = [-1] * (64 * steps)
        for g, (_, b, e, _) in enumerate(group):
            for k in range(e - b):
                block[64 * (k // 8) + 8 * g + k % 8] = b + k
        wave.append((at, longest))
        pos.extend(block)
        at += 64 * steps
    return wave, [(r, slot, -1, 0) for r, _, _, slot in segs], split, nslot, pos
