"""Pins of the context-ring oracle (oracle/ring.py), CPU only: over random multi-step histories the
ring's gathered window equals TreeFlowDrafter._context of the true history (the last C rows,
front-padded by repeating the oldest; cf/drafters/tree_flow.py:143-148) -- the invariant the
reference states for _ring_gather (cf/vllm_plugin/flow_proposer.py:950-952) -- for chain steps,
tree steps whose accepted rows are scattered, masked writes and slot resets."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import flow as oflow
from oracle import ring as oring


def simulate(seed, R=5, C=8, H=6, steps=40, kmax=6, tree=False, check=None):
    rng = np.random.default_rng(seed)
    ring = np.zeros((R, C + 1, H))
    rpos = np.zeros(R, dtype=np.int64)
    nval = np.zeros(R, dtype=np.int64)
    hist = {s: [] for s in range(R)}
    for step in range(steps):
        B = int(rng.integers(1, R + 1))
        rows = rng.permutation(R)[:B]
        cnt = rng.integers(0, kmax + 1, size=B)
        wmask = (rng.random(B) < 0.85).astype(np.int64)
        nodes = kmax + 3                       # rows per request in sh (tree: more nodes than kept)
        starts = np.arange(B) * nodes
        sh = rng.standard_normal((B * nodes, H))
        path = None
        if tree:
            path = np.zeros((R, kmax), dtype=np.int64)
            for s in range(R):
                path[s] = rng.permutation(nodes - 1)[:kmax]
        for b, s in enumerate(rows):
            if not wmask[b]:
                continue
            for j in range(int(cnt[b])):
                off = j if path is None else (0 if j == 0 else 1 + int(path[s][j - 1]))
                hist[s].append(sh[starts[b] + off].copy())
        oring.ring_write(ring, rpos, nval, sh, rows, starts, cnt, wmask, path, kmax)
        if rng.random() < 0.1:                 # a slot recycled for a new request
            s = int(rng.integers(R))
            rpos[s] = nval[s] = 0
            hist[s] = []
        live = [s for s in range(R) if hist[s]]
        if live:
            got = oring.ring_gather(ring, rpos, nval, live)
            for i, s in enumerate(live):
                want = oflow.front_pad_context(np.stack(hist[s])[None], C)[0]
                if check is not None:
                    check(s, got[i], want)
                else:
                    assert np.array_equal(got[i], want), (seed, step, s)
            for s in live:
                assert nval[s] == min(len(hist[s]), C)
    return ring, rpos, nval


@pytest.mark.parametrize("tree", [False, True])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_ring_window_equals_context_of_history(seed, tree):
    simulate(seed, tree=tree)


def test_more_rows_than_the_window_keep_the_newest():
    simulate(7, C=4, kmax=7, steps=30)


def test_a_dropped_term_is_caught():
    """The pin bites: a gather that forgets the front padding (reads phys = (head - m + j) mod C)
    disagrees with the history on short windows."""
    bad = []

    def gather_no_pad(ring, rpos, nval, rows):
        C = ring.shape[1] - 1
        return np.stack([ring[s, [(int(rpos[s]) - int(nval[s]) + j) % C for j in range(C)]] for s in rows])

    orig = oring.ring_gather
    oring.ring_gather = gather_no_pad
    try:
        simulate(3, check=lambda s, got, want: bad.append(not np.array_equal(got, want)))
    finally:
        oring.ring_gather = orig
    assert any(bad)
