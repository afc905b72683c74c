"""GPU: the two-pass candidate head.

* pass A's selection (cfh_cand_topm) picks exactly the top-M of each column's best per-depth
  log-probability computed from the kernel's own fp16 logits and log-sum-exps (and the per-depth
  sets), ties to the lower column;
* the two-pass chain and tree drafts equal the oracle's two-pass search wherever its decisions are
  not near ties (margin > 1e-3), for shared and per-depth candidate sets and the seed-conditioned
  pass A.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import to64
from chain_flow_amd import _lib
from chain_flow_amd.config import flownet
from chain_flow_amd.drafter import Drafter
from chain_flow_amd.weights import make_weights, synthetic_context
from oracle import beam as obeam
from oracle import head as ohead


def _setup(cuda, d=512, V=4096, n=2048, seed=7):
    cfg = flownet(d, layers=1, flow_steps=2)
    W = make_weights(cfg, V, init="test", base_seed=seed)
    W["lm_head.weight"] = (W["lm_head.weight"].float() * 8).half()
    sl = torch.randperm(V, generator=torch.Generator().manual_seed(3))[:n].sort().values.to(torch.int32)
    return cfg, W, sl


@pytest.mark.gpu
@pytest.mark.parametrize("shared", [True, False])
def test_candidate_selection_is_exact(cuda, shared):
    cfg, W, sl = _setup(cuda)
    dr = Drafter(cfg, {k: v.to(cuda) for k, v in W.items()}, sl.to(cuda), device=cuda)
    g = torch.Generator().manual_seed(2)
    hm = (torch.randn(2, 5, 512, generator=g) * 2).half().to(cuda)
    M = 300
    local, glob = dr.head.candidates(hm, M, shared=shared)
    logits = torch.empty(10, dr.head.n, dtype=torch.float16, device=cuda)
    lse = torch.cat([dr.head.topk(hm[b], 1, logits=logits[5 * b:5 * b + 5])[2] for b in range(2)])   # <= 8 rows a call
    torch.cuda.synchronize()
    lg = logits.float().cpu().numpy().reshape(2, 5, -1)
    ls = lse.cpu().numpy().reshape(2, 5, 1).astype(np.float32)
    vals = (lg - ls).astype(np.float32)
    print(f"[twopass cand] shared={shared} M={M}", flush=True)
    for b in range(2):
        for dd in range(5):
            v = vals[b].max(0) if shared else vals[b, dd]
            want = np.sort(np.argsort(-v, kind="stable")[:M])
            got = (local[b] if shared else local[b, dd]).cpu().numpy()
            assert np.array_equal(got, want), (b, dd)
            gg = (glob[b] if shared else glob[b, dd]).cpu().numpy()
            assert np.array_equal(gg, sl.numpy()[want])


@pytest.mark.gpu
@pytest.mark.parametrize("B,n,Vs,M,ld,kind", [
    (3, 5, 1001, 77, 1003, "ties"),          # ragged width (not a multiple of 4), heavy ties
    (2, 1, 62642, 8192, 62642, "randn"),     # the shortlist width of the d=5120 head
    (1, 3, 70001, 70001, 70001, "randn"),    # M = every column
    (2, 2, 5, 3, 8, "equal"),                # every value equal: all M from the ties
    (1, 2, 262144, 1000, 262144, "ties"),    # the largest supported width
])
def test_candidate_select_edges(cuda, B, n, Vs, M, ld, kind):
    """cfh_cand_topm through the C-ABI against numpy's stable top-M of
    max_d(float(logit) - lse) in fp32 (ties to the lower column), output in column order."""
    g = np.random.default_rng(Vs + M)
    if kind == "ties":
        lg = (g.integers(-40, 8, size=(B * n, ld)) * 0.25).astype(np.float16)
    elif kind == "equal":
        lg = np.full((B * n, ld), -1.5, np.float16)
    else:
        lg = (g.standard_normal((B * n, ld)) * 3).astype(np.float16)
    lse = (g.integers(0, 4, size=B * n) * 0.5 + 10).astype(np.float32)
    if kind == "equal":
        lse[:] = 10
    sl = np.sort(g.choice(4 * Vs, Vs, replace=False)).astype(np.int32)
    L = _lib.lib()
    dl, dlse, dsl = torch.from_numpy(lg).to(cuda), torch.from_numpy(lse).to(cuda), torch.from_numpy(sl).to(cuda)
    local = torch.full((B, M), -1, dtype=torch.int32, device=cuda)
    glob = torch.full((B, M), -1, dtype=torch.int32, device=cuda)
    ws = torch.empty(int(L.cfh_cand_ws_bytes(B, Vs)), dtype=torch.uint8, device=cuda)
    print(f"[cand edges] B={B} n={n} Vs={Vs} M={M} ld={ld} {kind}", flush=True)
    _lib.check(L.cfh_cand_topm(dl.data_ptr(), ld, dlse.data_ptr(), B, n, Vs, M, dsl.data_ptr(), local.data_ptr(),
                               glob.data_ptr(), ws.data_ptr(), _lib.stream_handle()), "cfh_cand_topm")
    torch.cuda.synchronize()
    vals = (lg[:, :Vs].astype(np.float32) - lse[:, None]).reshape(B, n, Vs).max(1)
    for b in range(B):
        want = np.sort(np.argsort(-vals[b], kind="stable")[:M])
        assert np.array_equal(local[b].cpu().numpy(), want), b
        assert np.array_equal(glob[b].cpu().numpy(), sl[want]), b


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["shared", "per_depth", "seed"])
def test_twopass_drafts_match_oracle(cuda, mode):
    cfg, W, sl = _setup(cuda)
    shared, seed = mode != "per_depth", mode == "seed"
    M = 256
    dr = Drafter(cfg, {k: v.to(cuda) for k, v in W.items()}, sl.to(cuda), device=cuda, twopass_m=M,
                 twopass_shared=shared, twopass_seed=seed)
    ctx = synthetic_context(1, cfg.context_size, 512, seed=4)
    known0 = sl[100:101].long()
    pred = dr.predict_hidden(ctx.to(cuda))
    chain = dr.beam_chains(None, known0.to(cuda), 5, 4, pred=pred).cpu()
    tree = dr.beam_tree(None, known0.to(cuda), keep=4, topb=4, depth=4, pred=pred).cpu()
    torch.cuda.synchronize()
    W64 = {k: to64(v) for k, v in W.items()}
    s64 = sl.long().numpy()
    pr = to64(pred)

    def score(h, prev):
        if prev is None:
            return ohead.head_logits(h, W64["lm_head.weight"][s64])
        return ohead.head_with_bias(h, W64["lm_head.weight"][s64], W64["markov.w1.weight"],
                                    W64["markov.w2.weight"][s64], prev)

    resid = lambda lp, nl: ohead.path_residual(W64, W64["embed_tokens.weight"], lp, nl, cfg.path_order)
    ref, trace = obeam.beam_chains(pr, known0.numpy(), s64, 4, 5, cfg.path_order, score, resid,
                                   return_trace=True, twopass_m=M, shared=shared, seed=seed)
    print(f"[twopass {mode}] chain gpu {chain[0].tolist()} oracle {ref[0].tolist()}", flush=True)
    near = lambda tr: any((ohead.margins(t["lp"], 4) <= 1e-3).any() or (ohead.margins(t["cand"], 4) <= 1e-3).any()
                          for t in tr)
    if chain[0].tolist() != ref[0].tolist():
        assert near(trace), (chain[0].tolist(), ref[0].tolist())
    tref, ttrace = obeam.beam_tree(pr, known0.numpy(), s64, 4, 4, 4, cfg.path_order, score, resid,
                                   return_trace=True, twopass_m=M, shared=shared, seed=seed)
    print(f"[twopass {mode}] tree gpu {tree[0].tolist()} oracle {tref[0].tolist()}", flush=True)
    if tree[0].tolist() != tref[0].tolist():
        assert near(ttrace), (tree[0].tolist(), tref[0].tolist())
