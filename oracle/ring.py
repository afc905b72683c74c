"""Oracle: the serving proposer's context ring (``_ring_write`` + ``_ring_gather``).

Test infrastructure only (the tests compare the GPU results against it).

Follows ``cf/vllm_plugin/flow_proposer.py:916-945`` (``_ring_write``: rows j < Kmax of request b
come from ``sh[start_b + srcoff_j]``, srcoff_j = j, or 0 then ``1 + path[slot][j-1]`` for a tree's
accepted path; invalid rows (j >= cnt or wmask 0) go to the trash row C; then
``rpos = (rpos + add) % C``, ``nval = min(nval + add, C)``) and ``:947-961`` (``_ring_gather``:
``t = min(max(j - (C - m), 0), max(m - 1, 0))``, ``phys = (head - m + t) mod C``).
The ring is ``[R, C + 1, H]``; rpos / nval are ``[R]``.
"""
from __future__ import annotations

import numpy as np


def ring_write(ring, rpos, nval, sh, rows, starts, cnt, wmask, path, kmax):
    """In place, as the reference's index_copy_ chain (later rows win on a collision)."""
    C = ring.shape[1] - 1
    B = len(rows)
    for b in range(B):
        slot = int(rows[b])
        head = int(rpos[slot])
        for j in range(kmax):
            valid = j < cnt[b] and bool(wmask[b])
            off = j if path is None else (0 if j == 0 else 1 + int(path[slot][j - 1]))
            src = min(max(int(starts[b]) + off, 0), sh.shape[0] - 1)
            if not valid:
                src = 0
            dst = (head + j) % C if valid else C
            ring[slot, dst] = sh[src]
        add = int(cnt[b]) if wmask[b] else 0
        rpos[slot] = (head + add) % C
        nval[slot] = min(int(nval[slot]) + add, C)


def ring_gather(ring, rpos, nval, rows):
    """[B, C, H]: each slot's window oldest first, front-padded by repeating the oldest row."""
    C = ring.shape[1] - 1
    out = []
    for slot in rows:
        m, head = int(nval[slot]), int(rpos[slot])
        idx = []
        for j in range(C):
            t = min(max(j - (C - m), 0), max(m - 1, 0))
            idx.append((head - m + t) % C)
        out.append(ring[int(slot), idx])
    return np.stack(out)
