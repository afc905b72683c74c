"""GPU parity at the metric's own configuration: d = 5120 fp16, batch 1, L = 8 blocks, E = 8 Euler
steps, seeded N(0, 0.02) weights ("baseline"), the 62,642-row shortlist of a 248,320-row head.

* the flow (init_latents + every Euler step of both chunk experts) against the oracle in the
  numerics the reference runs at this width (torch's fp16 modules) within 2e-3, with the oracle's
  weights read from the device block by block (float32 host copies, float32 arithmetic);
* the 5-token width-4 chain and the greedy (width-1) chain against the oracle's beam on the same
  predicted hiddens: ids equal unless one of the oracle's decisions was within 1e-3 of a tie;
* the one-pass tree draft (keep 4, top-b 8, depth 5: the tree-verify workload's drafting half);
* the path residual (``cfh_path_residual``) directly, every live-offset count.

One drafter serves every test of the module (``c3``); its weights never leave the device except
as the oracle's host copies.
"""
from __future__ import annotations

from collections.abc import Mapping

import numpy as np
import pytest
import torch

from conftest import oracle_numerics, rel_err, to64
from chain_flow_amd.config import flownet
from chain_flow_amd.drafter import Drafter
from chain_flow_amd.shortlist import synthetic
from chain_flow_amd.weights import make_weights, synthetic_context
from oracle import beam as obeam
from oracle import flow as oflow
from oracle import head as ohead

D, VOCAB, SL_ROWS = 5120, 248320, 62642
TOL_FP16 = 2e-3


class _DeviceWeights(Mapping):
    """The drafter's fp16 device tensors as the oracle's weight dict: each is copied to the host as
    float32 on first use and kept (the flow's 15 GB of fp16 weights become 30 GB of float32)."""

    def __init__(self, W, names):
        self.W, self.names, self.host = W, sorted(names), {}

    def __getitem__(self, k):
        v = self.host.get(k)
        if v is None:
            if k.endswith("blocks.0.self_norm.weight") or (k.endswith(".self_norm.weight") and len(self.host) % 200 == 0):
                print(f"  [oracle weights] {k} ({len(self.host)} on the host)", flush=True)
            v = self.host[k] = self.W[k].float().cpu().numpy()
        return v

    def __iter__(self):
        return iter(self.names)

    def __len__(self):
        return len(self.names)


def _ocfg(cfg):
    return dict(draft_length=cfg.draft_length, chunk_size=cfg.chunk_size, num_layers=cfg.num_drafter_layers,
                num_heads=cfg.num_heads, num_flow_steps=cfg.num_flow_steps, init_mode=cfg.init_mode)


@pytest.fixture(scope="module")
def c3(cuda):
    cfg = flownet(D, layers=8, flow_steps=8)
    print("[c3] drawing the d=5120 drafter's weights on the device", flush=True)
    W = make_weights(cfg, VOCAB, init="baseline", base_seed=0, device=cuda)
    sl = synthetic(VOCAB, SL_ROWS, seed=2).to(cuda)
    ctx = synthetic_context(1, cfg.context_size, D, seed=1)
    dr = Drafter(cfg, W, sl, device=cuda)
    pred = dr.predict_hidden(ctx.to(cuda))
    torch.cuda.synchronize()
    print("[c3] drafter built, hiddens predicted; host copies of the head", flush=True)
    s64 = sl.long().cpu().numpy()
    host = dict(
        s64=s64,
        lm_sl=W["lm_head.weight"][sl.long()].double().cpu().numpy(),
        w2_sl=W["markov.w2.weight"][sl.long()].double().cpu().numpy(),
        w1=W["markov.w1.weight"].cpu().numpy(),
        emb=W["embed_tokens.weight"].cpu().numpy(),
        path={k: v.double().cpu().numpy() for k, v in W.items() if k.startswith("path_head.")})
    yield dict(cfg=cfg, W=W, sl=sl, ctx=ctx, dr=dr, pred=pred, host=host)
    del dr, W
    torch.cuda.empty_cache()


def _search_fns(c3):
    h = c3["host"]
    score = lambda x, prev: ohead.head_with_bias(x, h["lm_sl"], h["w1"], h["w2_sl"], prev)
    resid = lambda lp, nl: ohead.path_residual(h["path"], h["emb"], lp, nl, c3["cfg"].path_order)
    return score, resid


def _near_tie(trace, k_lp, k_cand):
    return any((ohead.margins(t["lp"], k_lp) <= 1e-3).any() or (ohead.margins(t["cand"], k_cand) <= 1e-3).any()
               for t in trace)


@pytest.mark.gpu
def test_c3_flow_d5120_L8_E8_matches_oracle(c3):
    """The whole predict_hidden at the metric's shape against the fp16-modules oracle (float32
    arithmetic on the host, weights as the device holds them)."""
    cfg, W = c3["cfg"], c3["W"]
    num = oracle_numerics(cfg)
    assert num == "fp16_modules"
    names = [k for k in W if k.startswith(("expert.", "extra_experts."))]
    Wh = _DeviceWeights(W, names)
    ctx = c3["ctx"].float().numpy()
    print(f"[c3 flow] d=5120 L=8 E=8 baseline init vs the oracle ({num}, float32 host arithmetic)", flush=True)
    ref, trace = oflow.predict_hidden(Wh, ctx, _ocfg(cfg), numerics=num, return_trace=True)
    z = to64(c3["pred"])
    assert np.isfinite(z).all()
    e = rel_err(z, ref)
    z0 = trace[0].astype(np.float64)
    eu = rel_err(z - z0, ref - z0)
    print(f"  vs {num}: {e:.3e}; the flow's update z_E - z_0: {eu:.3e} "
          f"(|z_E - z_0| / |z_E| = {np.linalg.norm(ref - z0) / np.linalg.norm(ref):.3f})", flush=True)
    del Wh
    assert e < TOL_FP16


@pytest.mark.gpu
@pytest.mark.parametrize("width", [4, 1])
def test_c3_chain_draft_matches_oracle(c3, width):
    """The 5-token chain (width 4, and the greedy width-1 chain) over the shortlisted head with the
    markov bias and the path residual, on the predicted hiddens, against the oracle's beam on the
    same hiddens."""
    sl = c3["sl"]
    known0 = sl[1234:1235].long()
    chain = c3["dr"].beam_chains(None, known0, 5, width, pred=c3["pred"]).cpu()
    torch.cuda.synchronize()
    score, resid = _search_fns(c3)
    ref, trace = obeam.beam_chains(to64(c3["pred"]), known0.cpu().numpy(), c3["host"]["s64"], width, 5,
                                   c3["cfg"].path_order, score, resid, return_trace=True)
    print(f"[c3 chain W={width}] gpu {chain[0].tolist()} oracle {ref[0].tolist()}", flush=True)
    if chain[0].tolist() != ref[0].tolist():
        assert _near_tie(trace, width, width), (chain[0].tolist(), ref[0].tolist())


@pytest.mark.gpu
def test_c3_tree_draft_matches_oracle(c3):
    """The one-pass tree draft at keep 4, top-b 8, depth 5 (20 nodes, BFS parents) against the
    oracle's tree search on the same hiddens."""
    keep, topb, depth = 4, 8, 5
    sl = c3["sl"]
    known0 = sl[4321:4322].long()
    tree = c3["dr"].beam_tree(None, known0, keep=keep, topb=topb, depth=depth, pred=c3["pred"]).cpu()
    torch.cuda.synchronize()
    score, resid = _search_fns(c3)
    ref, trace = obeam.beam_tree(to64(c3["pred"]), known0.cpu().numpy(), c3["host"]["s64"], keep, topb, depth,
                                 c3["cfg"].path_order, score, resid, return_trace=True)
    N = ref.shape[1] // 2
    assert tree.shape == (1, 2 * N) and N == 20
    print(f"[c3 tree] gpu {tree[0].tolist()}\n          oracle {ref[0].tolist()}", flush=True)
    assert (tree[0, N:].numpy() < np.arange(N)).all()
    if tree[0].tolist() != ref[0].tolist():
        assert _near_tie(trace, topb, keep), (tree[0].tolist(), ref[0].tolist())


@pytest.mark.gpu
@pytest.mark.parametrize("nlive", [1, 2, 3, 4])
def test_c3_path_residual_matches_oracle(c3, nlive):
    """cfh_path_residual at d = 5120 (offset projections of the live ancestors, masked sum, LayerNorm,
    the 2x MLP, plus the marginal hidden) for 8 rows with absent ancestors mixed in."""
    dr, cfg = c3["dr"], c3["cfg"]
    g = torch.Generator().manual_seed(40 + nlive)
    M = 8
    lastp = c3["sl"].cpu()[torch.randint(0, SL_ROWS, (M, cfg.path_order), generator=g)].to(torch.int32)
    lastp[1, 2:] = -1
    lastp[3, 1:] = -1
    lastp[6, 3:] = -1
    pred = c3["pred"][0, 2].contiguous()
    got = to64(dr.path.hidden(lastp.to(pred.device), nlive, pred))
    torch.cuda.synchronize()
    h = c3["host"]
    res = ohead.path_residual(h["path"], h["emb"], lastp.long().numpy(), nlive, cfg.path_order)
    p64 = to64(pred)[None]
    ref = ohead.r16(p64 + res, "fp16")
    e, er = rel_err(got, ref), rel_err(got - p64, ref - p64)
    print(f"[c3 path residual] nlive={nlive}: hidden {e:.3e}, residual part {er:.3e}", flush=True)
    assert e < TOL_FP16
