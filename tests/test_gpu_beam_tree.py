"""GPU: the one-pass tree draft (``_beam_tree``, cf/vllm_plugin/flow_proposer.py:1272-1332) against the
oracle's search on the same predicted hiddens, at the proposer's defaults (keep 4, top-b 8,
depth 4: CF_TREE_KEEP / CF_TREE_TOPB / CF_TREE_DEPTH) and at the tree-verify workload's depth 5;
one and two requests.  Tokens and parents equal the oracle's unless one of its decisions was within
1e-3 of a tie."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import to64
from chain_flow_amd.config import flownet
from chain_flow_amd.drafter import Drafter
from chain_flow_amd.weights import make_weights, synthetic_context
from oracle import beam as obeam
from oracle import head as ohead


@pytest.mark.gpu
@pytest.mark.parametrize("keep,topb,depth,B", [(4, 8, 4, 1), (4, 8, 5, 1), (4, 8, 5, 2), (2, 3, 5, 1)])
def test_one_pass_tree_matches_oracle(cuda, keep, topb, depth, B):
    d, V, n = 512, 4096, 2048
    cfg = flownet(d, layers=1, flow_steps=2)
    W = make_weights(cfg, V, init="test", base_seed=21)
    W["lm_head.weight"] = (W["lm_head.weight"].float() * 8).half()
    sl = torch.randperm(V, generator=torch.Generator().manual_seed(5))[:n].sort().values.to(torch.int32)
    dr = Drafter(cfg, {k: v.to(cuda) for k, v in W.items()}, sl.to(cuda), device=cuda)
    ctx = synthetic_context(B, cfg.context_size, d, seed=8)
    known0 = sl[[300, 1700][:B]].long()
    print(f"[tree one-pass] keep={keep} topb={topb} depth={depth} B={B}", flush=True)
    pred = dr.predict_hidden(ctx.to(cuda))
    tree = dr.beam_tree(None, known0.to(cuda), keep=keep, topb=topb, depth=depth, pred=pred).cpu()
    torch.cuda.synchronize()
    W64 = {k: to64(v) for k, v in W.items()}
    s64 = sl.long().numpy()
    score = lambda h, prev: ohead.head_with_bias(h, W64["lm_head.weight"][s64], W64["markov.w1.weight"],
                                                 W64["markov.w2.weight"][s64], prev)
    resid = lambda lp, nl: ohead.path_residual(W64, W64["embed_tokens.weight"], lp, nl, cfg.path_order)
    ref, trace = obeam.beam_tree(to64(pred), known0.numpy(), s64, keep, topb, depth, cfg.path_order, score, resid,
                                 return_trace=True)
    N = ref.shape[1] // 2
    assert tree.shape == (B, 2 * N)
    sizes, fr = [], 1
    for _ in range(depth):
        sizes.append(min(keep, fr * topb))
        fr = sizes[-1]
    assert N == sum(sizes)
    for b in range(B):
        print(f"  b={b} gpu {tree[b].tolist()}\n      oracle {ref[b].tolist()}", flush=True)
        par = tree[b, N:].numpy()
        assert (par < np.arange(N)).all()                      # BFS: parents precede children
        if tree[b].tolist() != ref[b].tolist():
            near = any((ohead.margins(t["lp"], topb) <= 1e-3).any() or (ohead.margins(t["cand"], keep) <= 1e-3).any()
                       for t in trace)
            assert near, (b, tree[b].tolist(), ref[b].tolist())
