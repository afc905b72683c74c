"""FlowDrafterProposer end to end on the GPU: a tiny checkpoint directory, the target's embeddings
and lm_head bound, hidden states stashed, then propose() -- compared with the oracle's chain on the
same context (ids equal wherever the oracle's decisions are not near ties)."""
from __future__ import annotations

import json
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from conftest import oracle_numerics, to64
from chain_flow_amd import shortlist as slmod
from chain_flow_amd.config import flownet
from chain_flow_amd.vllm_plugin import flow_proposer as fp
from chain_flow_amd.weights import make_weights
from oracle import beam as obeam
from oracle import flow as oflow
from oracle import head as ohead


@pytest.mark.gpu
def test_proposer_chain_draft_matches_oracle(cuda, tmp_path, monkeypatch):
    from safetensors.torch import save_file
    d, V, n = 512, 4096, 1024
    cfg = flownet(d, layers=1, flow_steps=2)
    W = make_weights(cfg, V, init="test", base_seed=7)
    W["lm_head.weight"] = (W["lm_head.weight"].float() * 8).half()
    drafter = {k: v for k, v in W.items() if k not in ("lm_head.weight", "embed_tokens.weight")}
    save_file({"drafter." + k: v.contiguous() for k, v in drafter.items()}, str(tmp_path / fp.WEIGHTS_NAME))
    (tmp_path / fp.CONFIG_NAME).write_text(json.dumps({"model_args": cfg.to_dict()}))
    sl = torch.randperm(V, generator=torch.Generator().manual_seed(3))[:n]
    slmod.save(tmp_path / "shortlist.pt", sl, vocab_size=V)
    for k in ("VLLM_SPEC_TREE", "CF_SHORTLIST", "CF_FLOW_STEPS"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("CF_DRAFTER_DIR", str(tmp_path))
    vc = SimpleNamespace(speculative_config=SimpleNamespace(num_speculative_tokens=5),
                         scheduler_config=SimpleNamespace(max_num_seqs=4))
    p = fp.FlowDrafterProposer(vc)
    p.bind_target(W["embed_tokens.weight"].to(cuda), W["lm_head.weight"].to(cuda))
    g = torch.Generator().manual_seed(11)
    hid = torch.randn(3, d, generator=g)
    hid = (hid / hid.pow(2).mean(-1, keepdim=True).sqrt()).half()
    slv = torch.unique(sl.long())
    toks = [int(slv[10]), int(slv[20]), int(slv[30])]
    p.stash_hidden_states(hid.to(cuda))
    out = p.propose([toks])
    assert len(out) == 1 and len(out[0]) == 5
    # oracle on the same context: 3 hiddens front-padded to 8, known0 = last committed token
    ctx = oflow.front_pad_context(to64(hid)[None], cfg.context_size)
    W64 = {k: to64(v) for k, v in W.items()}
    ocfg = dict(draft_length=cfg.draft_length, chunk_size=cfg.chunk_size, num_layers=1, num_heads=cfg.num_heads,
                num_flow_steps=2, init_mode="delta")
    pred = oflow.predict_hidden(W64, ctx, ocfg, numerics=oracle_numerics(cfg))
    s64 = slv.numpy()
    score = lambda h, prev: ohead.head_with_bias(h, W64["lm_head.weight"][s64], W64["markov.w1.weight"],
                                                 W64["markov.w2.weight"][s64], prev)
    resid = lambda lp, nl: ohead.path_residual(W64, W64["embed_tokens.weight"], lp, nl, cfg.path_order)
    ref, trace = obeam.beam_chains(pred, np.array([toks[-1]]), s64, 4, 5, cfg.path_order, score, resid,
                                   return_trace=True)
    print(f"[proposer] gpu {out[0]} oracle {ref[0].tolist()}", flush=True)
    if out[0] != ref[0].tolist():
        near = any((ohead.margins(t["lp"], 4) <= 1e-3).any() or (ohead.margins(t["cand"], 4) <= 1e-3).any()
                   for t in trace)
        assert near, (out[0], ref[0].tolist())


def _ckpt(tmp_path, d=512, V=4096, n=1024, seed=7):
    from safetensors.torch import save_file
    cfg = flownet(d, layers=1, flow_steps=2)
    W = make_weights(cfg, V, init="test", base_seed=seed)
    W["lm_head.weight"] = (W["lm_head.weight"].float() * 8).half()
    drafter = {k: v for k, v in W.items() if k not in ("lm_head.weight", "embed_tokens.weight")}
    save_file({"drafter." + k: v.contiguous() for k, v in drafter.items()}, str(tmp_path / fp.WEIGHTS_NAME))
    (tmp_path / fp.CONFIG_NAME).write_text(json.dumps({"model_args": cfg.to_dict()}))
    sl = torch.randperm(V, generator=torch.Generator().manual_seed(3))[:n]
    slmod.save(tmp_path / "shortlist.pt", sl, vocab_size=V)
    return cfg, W, torch.unique(sl.long())


@pytest.mark.gpu
@pytest.mark.parametrize("graph", ["1", "0"])
def test_proposer_ring_steps_and_async(cuda, tmp_path, monkeypatch, graph):
    """Several propose() steps for two requests (one recycled for a new request id half way): the
    device ring (+ the draft graph when CF_CUDAGRAPH=1) gives exactly the drafts of the eager
    Drafter on the front-padded true history, and CF_ASYNC_SPEC=1 returns the same drafts as the
    [num_reqs, K] int32 device tensor, rows by batch slot, zeros for a request with no tokens."""
    from chain_flow_amd.drafter import front_pad
    d = 512
    cfg, W, slv = _ckpt(tmp_path)
    for k in ("VLLM_SPEC_TREE", "CF_SHORTLIST", "CF_FLOW_STEPS", "CF_DRAFT_BUCKETS"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("CF_DRAFTER_DIR", str(tmp_path))
    monkeypatch.setenv("CF_CUDAGRAPH", graph)
    vc = SimpleNamespace(speculative_config=SimpleNamespace(num_speculative_tokens=5),
                         scheduler_config=SimpleNamespace(max_num_seqs=4))
    p = fp.FlowDrafterProposer(vc)
    monkeypatch.setenv("CF_ASYNC_SPEC", "1")
    pa = fp.FlowDrafterProposer(vc)
    for q in (p, pa):
        q.bind_target(W["embed_tokens.weight"].to(cuda), W["lm_head.weight"].to(cuda))
    rng = np.random.default_rng(4)
    hist = {0: [], 1: []}
    ids = ["a", "b"]
    for step in range(4):
        if step == 2:
            ids = ["a", "c"]              # slot 1 now holds a new request: its history restarts
            hist[1] = []
        toks = [[int(t) for t in slv[rng.integers(0, len(slv), size=int(rng.integers(1, 4)))]] for _ in range(2)]
        if step == 3:
            toks[1] = []                  # no tokens for slot 1 this step
        n = sum(len(t) for t in toks)
        hid = torch.randn(n, d, generator=torch.Generator().manual_seed(50 + step)).half()
        off = 0
        for i, t in enumerate(toks):
            hist[i] += [hid[off + j] for j in range(len(t))]
            off += len(t)
        out = p.propose(toks, hidden_states=hid.to(cuda), req_ids=ids)
        outa = pa.propose(toks, hidden_states=hid.to(cuda), req_ids=ids)
        torch.cuda.synchronize()
        rows = [i for i in range(2) if toks[i]]
        ctx = torch.stack([front_pad(torch.stack(hist[i])[None], cfg.context_size)[0] for i in rows]).to(cuda)
        want = p.drafter.beam_chains(ctx, torch.tensor([toks[i][-1] for i in rows], device=cuda), 5, 4).cpu()
        print(f"[proposer ring] step {step} graph={graph} {out} eager {want.tolist()}", flush=True)
        for j, i in enumerate(rows):
            assert out[i] == want[j].tolist(), (step, i)
        assert outa.dtype == torch.int32 and outa.is_cuda and outa.shape == (2, 5)
        for i in range(2):
            assert outa[i].cpu().tolist() == (out[i] if toks[i] else [0] * 5), (step, i)


@pytest.mark.gpu
def test_proposer_profiling_hooks_leave_drafts_unchanged(cuda, tmp_path, monkeypatch, capsys):
    """CF_DRAFTPROF=1 (one event timing per batch bucket, the draft graph's profiling replays append
    nothing to the ring) and CF_PROFILE=1 (host-timed sections, no graphs) give the same drafts as the
    plain proposer, step after step, and print their timings."""
    d = 512
    cfg, W, slv = _ckpt(tmp_path)
    for k in ("VLLM_SPEC_TREE", "CF_SHORTLIST", "CF_FLOW_STEPS", "CF_DRAFT_BUCKETS", "CF_ASYNC_SPEC"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("CF_DRAFTER_DIR", str(tmp_path))
    vc = SimpleNamespace(speculative_config=SimpleNamespace(num_speculative_tokens=5),
                         scheduler_config=SimpleNamespace(max_num_seqs=4))
    props = {}
    for name, env in (("plain", {}), ("draftprof", {"CF_DRAFTPROF": "1"}),
                      ("profile", {"CF_PROFILE": "1", "CF_PROFILE_EVERY": "2"})):
        for k in ("CF_DRAFTPROF", "CF_PROFILE", "CF_PROFILE_EVERY"):
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        props[name] = fp.FlowDrafterProposer(vc)
        props[name].bind_target(W["embed_tokens.weight"].to(cuda), W["lm_head.weight"].to(cuda))
    assert props["profile"].use_cg is False
    rng = np.random.default_rng(8)
    for step in range(3):
        toks = [[int(t) for t in slv[rng.integers(0, len(slv), size=int(rng.integers(1, 4)))]] for _ in range(2)]
        n = sum(len(t) for t in toks)
        hid = torch.randn(n, d, generator=torch.Generator().manual_seed(70 + step)).half().to(cuda)
        outs = {k: p.propose(toks, hidden_states=hid, req_ids=["a", "b"]) for k, p in props.items()}
        torch.cuda.synchronize()
        print(f"[proposer profiling] step {step}: {outs}", flush=True)
        assert outs["draftprof"] == outs["plain"] and outs["profile"] == outs["plain"], step
    text = capsys.readouterr().out
    assert "[cf-draftprof]" in text and "[chain-flow] profile over 2 drafts" in text
