"""ORACLE - test infrastructure only: the library's row plan, restated in plain Python.

The plan has no counterpart in the reference (the reference gives every (row, sample) one thread); it fixes the
order in which the MI355X kernels visit rows.  Rule: a row of d edges is one segment if d <= seg_max, else
ceil(d / seg_max) segments [b + d*s//n, b + d*(s+1)//n) numbered with consecutive partial-sum slots; segments are
ordered by length, longest first, equal lengths in (row, segment) order.  tests/test_plan.py checks the library's
fc_plan_segments against this bit for bit, and checks the rule's invariants (every edge in exactly one segment,
slots a permutation) so that this restatement is pinned by more than itself.
"""
from __future__ import annotations


def plan(rowptr, seg_max: int = 256):
    segs, split, nslot = [], [], 0
    for r in range(len(rowptr) - 1):
        b, e = int(rowptr[r]), int(rowptr[r + 1])
        d = e - b
        if d <= seg_max:
            segs.append((r, b, e, -1))
            continue
        n = -(-d // seg_max)
        split.append((r, nslot, n, 0))
        for s in range(n):
            segs.append((r, b + d * s // n, b + d * (s + 1) // n, nslot + s))
        nslot += n
    order = sorted(range(len(segs)), key=lambda i: (-(segs[i][2] - segs[i][1]), i))
    return [segs[i] for i in order], split, nslot
