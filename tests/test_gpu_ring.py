"""GPU: the context ring (cfh_ring_step) against the oracle, bit for bit, over random multi-step
histories (chain and tree steps, masked writes, padding rows that only read a live slot)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from chain_flow_amd.ring import ContextRing
from oracle import ring as oring


@pytest.mark.gpu
@pytest.mark.parametrize("tree", [False, True])
def test_ring_step_matches_oracle(cuda, tree):
    R, C, H, kmax, steps = 6, 8, 2560, 6, 25
    rng = np.random.default_rng(17 + tree)
    ring = ContextRing(R, C, H, device=cuda)
    o_ring = np.zeros((R, C + 1, H))
    o_rpos = np.zeros(R, dtype=np.int64)
    o_nval = np.zeros(R, dtype=np.int64)
    print(f"[ring] tree={tree} R={R} C={C} H={H}", flush=True)
    for step in range(steps):
        B = int(rng.integers(1, R + 1))
        rows = rng.permutation(R)[:B]
        cnt = rng.integers(0, kmax + 1, size=B)
        wmask = (rng.random(B) < 0.85).astype(np.int64)
        nodes = kmax + 3
        starts = np.arange(B) * nodes
        sh = torch.randn(B * nodes, H, generator=torch.Generator().manual_seed(step)).half()
        path = None
        if tree:
            path = np.stack([rng.permutation(nodes - 1)[:kmax] for _ in range(R)])
        # two padding rows on a live slot that append nothing (a graph bucket's tail)
        pad = 2
        k_rows = np.concatenate([rows, np.full(pad, rows[0])])
        k_starts = np.concatenate([starts, np.zeros(pad, dtype=np.int64)])
        k_cnt = np.concatenate([cnt, np.zeros(pad, dtype=np.int64)])
        k_wm = np.concatenate([wmask, np.ones(pad, dtype=np.int64)])
        ctx = ring.step(sh.to(cuda), k_rows, k_starts, k_cnt, k_wm,
                        None if path is None else torch.as_tensor(path), kmax)
        torch.cuda.synchronize()
        oring.ring_write(o_ring, o_rpos, o_nval, sh.double().numpy(), rows, starts, cnt, wmask, path, kmax)
        want = oring.ring_gather(o_ring, o_rpos, o_nval, rows)
        got = ctx[:B].double().cpu().numpy()
        live = o_nval[rows] > 0
        assert np.array_equal(got[live], want[live]), step
        assert np.array_equal(ring.rpos.cpu().numpy(), o_rpos) and np.array_equal(ring.nval.cpu().numpy(), o_nval)
        assert np.array_equal(ring.ring[:, :C].double().cpu().numpy(), o_ring[:, :C]), step
    print("  all steps bit-exact", flush=True)
