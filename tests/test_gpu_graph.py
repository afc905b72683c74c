"""GPU: the whole-draft graph (ring step -> predict_hidden -> beam) replays bit-identically to the
same steps run eagerly, step after step as the rings evolve, with unrelated eager work between
replays and batches that pad up to a bucket; for the target-width and the latent drafter."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from chain_flow_amd.config import TreeVAEFlowConfig, flownet
from chain_flow_amd.drafter import Drafter
from chain_flow_amd.graph import DraftGraphs, bucket_ladder
from chain_flow_amd.ring import ContextRing
from chain_flow_amd.weights import make_weights


def _drafter(kind, cuda, twopass_m=0, shared=True):
    d, V, n = 512, 4096, 1024
    if kind == "latent":
        cfg = TreeVAEFlowConfig(context_size=8, draft_length=8, chunk_size=4, expert_dim=d, num_heads=8,
                                ffn_multiplier=6, num_drafter_layers=1, num_flow_steps=2, latent_size=128,
                                vae_intermediate_size=256, vae_num_layers=1, vae_num_heads=4,
                                vae_max_sequence_length=16)
    else:
        cfg = flownet(d, layers=1, flow_steps=2)
    W = make_weights(cfg, V, init="test", base_seed=5, hidden=d)
    W["lm_head.weight"] = (W["lm_head.weight"].float() * 8).half()
    sl = torch.randperm(V, generator=torch.Generator().manual_seed(3))[:n].sort().values
    return Drafter(cfg, {k: v.to(cuda) for k, v in W.items()}, sl.to(torch.int32).to(cuda), device=cuda,
                   twopass_m=twopass_m, twopass_shared=shared), d, sl


@pytest.mark.gpu
@pytest.mark.parametrize("kind,search,twopass", [
    ("target", "chain", None), ("latent", "chain", None),
    # the proposer's default head: two-pass (shared candidate image at B = 1, per-request candidate
    # rows read in place at B > 1), and per-depth candidate sets
    ("target", "chain", "shared"), ("target", "chain", "per_depth"),
    ("target", "tree", None), ("target", "tree", "shared"), ("latent", "tree", "per_depth")])
def test_draft_graph_replays_equal_eager(cuda, kind, search, twopass):
    dr, d, sl = _drafter(kind, cuda, twopass_m=256 if twopass else 0, shared=twopass != "per_depth")
    R, C, kmax = 4, 8, 6
    eager_ring = ContextRing(R, C, d, device=cuda)
    graph_ring = ContextRing(R, C, d, device=cuda)
    if search == "chain":
        draft = lambda ctx, k0: dr.beam_chains(ctx, k0, 5, 4)
    else:
        draft = lambda ctx, k0: dr.beam_tree(ctx, k0, keep=4, topb=8, depth=4)
    graphs = DraftGraphs(graph_ring, draft, kmax, bucket_ladder(R))
    assert graphs.buckets == [1, 2, 4]
    rng = np.random.default_rng(9)
    print(f"[graph] {kind} {search} twopass={twopass}", flush=True)
    for step in range(6):
        B = int(rng.integers(1, R))                      # 1..3: pads to buckets 1, 2 and 4
        rows = rng.permutation(R)[:B].tolist()
        cnt = rng.integers(1, kmax + 1, size=B).tolist()
        starts = np.concatenate([[0], np.cumsum(cnt)[:-1]]).tolist()
        sh = torch.randn(sum(cnt), d, generator=torch.Generator().manual_seed(100 + step)).half().to(cuda)
        k0 = sl[rng.integers(0, len(sl), size=B)].long().tolist()
        ctx = eager_ring.step(sh, rows, starts, cnt, kmax=kmax)
        want = draft(ctx, torch.tensor(k0, device=cuda)).clone()
        torch.cuda.synchronize()
        junk = torch.randn(256, 256, device=cuda) @ torch.randn(256, 256, device=cuda)   # eager work between
        got = graphs.run(sh, rows, starts, cnt, k0).clone()
        torch.cuda.synchronize()
        del junk
        print(f"  step {step} B={B} graph {got.tolist()} eager {want.tolist()}", flush=True)
        assert torch.equal(got, want), step
        assert torch.equal(graph_ring.ring[:, :C], eager_ring.ring[:, :C])
        assert torch.equal(graph_ring.rpos, eager_ring.rpos) and torch.equal(graph_ring.nval, eager_ring.nval)


@pytest.mark.gpu
def test_graph_of_a_smaller_bucket_survives_later_captures(cuda):
    """Capturing bucket 2 after bucket 1 must not move anything graph 1 references: the flow's
    workspace is sized for the largest request group when the drafter is built and never swapped.
    After both captures a guard tensor takes whatever memory is free; replaying graph 1 leaves it
    unchanged and still equals the eager draft."""
    dr, d, sl = _drafter("target", cuda)
    R, C, kmax = 2, 8, 4
    eager_ring = ContextRing(R, C, d, device=cuda)
    graph_ring = ContextRing(R, C, d, device=cuda)
    draft = lambda ctx, k0: dr.beam_chains(ctx, k0, 5, 4)
    graphs = DraftGraphs(graph_ring, draft, kmax, [1, 2])
    rng = np.random.default_rng(4)
    print("[graph guard] bucket 1, bucket 2, guard, bucket 1 again", flush=True)
    guard = None
    for step, B in enumerate([1, 2, 1, 1]):
        rows = rng.permutation(R)[:B].tolist()
        cnt = rng.integers(1, kmax + 1, size=B).tolist()
        starts = np.concatenate([[0], np.cumsum(cnt)[:-1]]).tolist()
        sh = torch.randn(sum(cnt), d, generator=torch.Generator().manual_seed(300 + step)).half().to(cuda)
        k0 = sl[rng.integers(0, len(sl), size=B)].long().tolist()
        ctx = eager_ring.step(sh, rows, starts, cnt, kmax=kmax)
        want = draft(ctx, torch.tensor(k0, device=cuda)).clone()
        got = graphs.run(sh, rows, starts, cnt, k0).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, want), step
        if step == 1:
            torch.cuda.empty_cache()
            guard = torch.full((64 << 20,), 7, dtype=torch.uint8, device=cuda)
    torch.cuda.synchronize()
    assert int((guard != 7).sum()) == 0, "a graph replay wrote into memory it does not own"
