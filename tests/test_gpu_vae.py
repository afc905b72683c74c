"""GPU parity of the hidden-state VAE (cfh_vae_encode / cfh_vae_decode) and of the latent drafter
(encode -> flow at the latent width -> decode) against the CPU oracle.

Contract: fp16 outputs within 2e-3 norm-relative of the oracle's fp16 restatement of torch's fp16
modules (oracle/vae.py) on the same seeded weights; chain ids equal to the oracle's wherever its
decisions are not near ties (margin > 1e-3).
"""
from __future__ import annotations

import json
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from conftest import oracle_numerics, rel_err, to64
from chain_flow_amd import shortlist as slmod
from chain_flow_amd.config import TreeVAEFlowConfig
from chain_flow_amd.drafter import Drafter
from chain_flow_amd.vae import HiddenVAE
from chain_flow_amd.vllm_plugin import flow_proposer as fp
from chain_flow_amd.weights import make_weights, param_specs, synthetic_context
from oracle import beam as obeam
from oracle import flow as oflow
from oracle import head as ohead
from oracle import vae as ovae

TOL_FP16 = 2e-3


def _cfg(latent, inter, heads, vlayers, layers=1, steps=2, **kw):
    return TreeVAEFlowConfig(context_size=8, draft_length=8, chunk_size=4, num_heads=8, ffn_multiplier=6,
                             num_drafter_layers=layers, num_flow_steps=steps, init_mode="delta", latent_size=latent,
                             vae_intermediate_size=inter, vae_num_layers=vlayers, vae_num_heads=heads,
                             vae_max_sequence_length=16, **kw)


def _vcfg(cfg):
    return dict(intermediate_size=cfg.vae_intermediate_size, num_layers=cfg.vae_num_layers,
                num_heads=cfg.vae_num_heads, max_sequence_length=cfg.vae_max_sequence_length)


def _fcfg(cfg):
    return dict(draft_length=cfg.draft_length, chunk_size=cfg.chunk_size, num_layers=cfg.num_drafter_layers,
                num_heads=cfg.num_heads, num_flow_steps=cfg.num_flow_steps, init_mode=cfg.init_mode)


def _vae_weights(cfg, hidden, seed):
    names = {n for n in param_specs(cfg, 16, target=False, hidden=hidden) if n.startswith("vae.")}
    return make_weights(cfg, 16, init="test", base_seed=seed, names=names, target=False, hidden=hidden)


@pytest.mark.gpu
@pytest.mark.parametrize("hidden,latent,inter,heads,vlayers", [
    (2560, 640, 1920, 8, 2),      # the shipped 4B drafter's VAE (head_dim 240: two heads per k-chunk)
    (1024, 256, 320, 8, 1),       # head_dim 40: four heads per k-chunk
    (5120, 1024, 1920, 8, 1),     # a 27B-class target width into the latent 1024
])
def test_vae_matches_oracle(cuda, hidden, latent, inter, heads, vlayers):
    cfg = _cfg(latent, inter, heads, vlayers)
    W = _vae_weights(cfg, hidden, seed=13)
    print(f"[vae parity] hidden={hidden} latent={latent} inter={inter} heads={heads} layers={vlayers}", flush=True)
    vae = HiddenVAE(cfg, hidden, {k: v.to(cuda) for k, v in W.items()}, device=cuda)
    V = ovae.vae_weights({k: to64(v) for k, v in W.items()})
    h = synthetic_context(1, 8, hidden, seed=3)
    z = (torch.randn(1, 8, latent, generator=torch.Generator().manual_seed(4)) * 0.5).half()
    for T in (8, 5):
        mu = vae.encode(h[:, :T].to(cuda))
        torch.cuda.synchronize()
        ref = ovae.encode_sequence_mu(V, to64(h[:, :T]), _vcfg(cfg), numerics="fp16")
        err = rel_err(to64(mu), ref)
        print(f"  encode T={T} rel err {err:.3e}", flush=True)
        assert np.isfinite(to64(mu)).all() and err < TOL_FP16
    for T in (8, 3):
        out = vae.decode(z[:, :T].to(cuda))
        torch.cuda.synchronize()
        ref = ovae.decode_sequence(V, to64(z[:, :T]), _vcfg(cfg), numerics="fp16")
        err = rel_err(to64(out), ref)
        print(f"  decode T={T} rel err {err:.3e}", flush=True)
        assert np.isfinite(to64(out)).all() and err < TOL_FP16


@pytest.mark.gpu
def test_vae_batch_equals_single_sequences(cuda):
    """Sequences of a batch do not see each other: a batch of two encodes/decodes bit-identically to
    the two sequences alone (width 320 is not a multiple of 128: the per-sequence launches)."""
    hidden = 1024
    cfg = _cfg(256, 320, 8, 1)
    W = {k: v.to(cuda) for k, v in _vae_weights(cfg, hidden, seed=2).items()}
    vae = HiddenVAE(cfg, hidden, W, device=cuda)
    h = synthetic_context(2, 8, hidden, seed=6).to(cuda)
    both = vae.encode(h).clone()
    one = torch.cat([vae.encode(h[:1]).clone(), vae.encode(h[1:]).clone()], 0)
    dec = vae.decode(both).clone()
    dec1 = torch.cat([vae.decode(both[:1]).clone(), vae.decode(both[1:]).clone()], 0)
    torch.cuda.synchronize()
    assert torch.equal(both, one) and torch.equal(dec, dec1)


@pytest.mark.gpu
@pytest.mark.parametrize("B", [3, 20])
def test_vae_wide_batch_matches_oracle(cuda, B):
    """A batch of sequences at the shipped VAE's shapes (hidden 2560, latent 640, width 1920, 2
    layers) runs as groups of stacked sequences through the wide kernels (B = 20: two groups of
    10): each sequence's encode / decode within 2e-3 of the oracle and of the sequence alone."""
    hidden = 2560
    cfg = _cfg(640, 1920, 8, 2)
    W = _vae_weights(cfg, hidden, seed=4)
    vae = HiddenVAE(cfg, hidden, {k: v.to(cuda) for k, v in W.items()}, device=cuda)
    h = synthetic_context(B, 8, hidden, seed=B).to(cuda)
    print(f"[vae wide batch] B={B}", flush=True)
    mu = vae.encode(h).clone()
    dec = vae.decode(mu).clone()
    mu1 = [vae.encode(h[b:b + 1]).clone() for b in range(B)]
    dec1 = [vae.decode(mu[b:b + 1]).clone() for b in range(B)]
    torch.cuda.synchronize()
    V = ovae.vae_weights({k: to64(v) for k, v in W.items()})
    for b in range(B):
        rm = ovae.encode_sequence_mu(V, to64(h[b:b + 1]), _vcfg(cfg), "fp16")
        rd = ovae.decode_sequence(V, to64(mu[b:b + 1]), _vcfg(cfg), "fp16")
        e = (rel_err(to64(mu[b:b + 1]), rm), rel_err(to64(dec[b:b + 1]), rd),
             rel_err(to64(mu[b:b + 1]), to64(mu1[b])), rel_err(to64(dec[b:b + 1]), to64(dec1[b])))
        print(f"  sequence {b}: encode {e[0]:.2e} decode {e[1]:.2e} (vs alone {e[2]:.2e} {e[3]:.2e})", flush=True)
        assert max(e) < TOL_FP16


@pytest.mark.gpu
def test_latent_drafter_predict_hidden_matches_oracle(cuda):
    """TreeVAEFlowDrafter.predict_hidden at the shipped 4B shapes (hidden 2560, latent 640: head_dim
    80 in the flow, 240 in the VAE), two blocks, two Euler steps."""
    hidden, V = 2560, 512
    cfg = _cfg(640, 1920, 8, 2, layers=2, steps=2, expert_dim=hidden)
    W = make_weights(cfg, V, init="test", base_seed=21, hidden=hidden)
    print("[latent drafter] hidden=2560 latent=640 L=2 E=2", flush=True)
    dr = Drafter(cfg, {k: v.to(cuda) for k, v in W.items()}, None, device=cuda)
    ctx = synthetic_context(1, 8, hidden, seed=8)
    pred = dr.predict_hidden(ctx.to(cuda))
    torch.cuda.synchronize()
    ref = ovae.predict_hidden({k: to64(v) for k, v in W.items()}, to64(ctx), _vcfg(cfg), _fcfg(cfg), "fp16",
                              oracle_numerics(cfg))
    err = rel_err(to64(pred), ref)
    print(f"  rel err {err:.3e}", flush=True)
    assert pred.shape == (1, 8, hidden) and np.isfinite(to64(pred)).all()
    assert err < TOL_FP16


@pytest.mark.gpu
def test_latent_proposer_chain_matches_oracle(cuda, tmp_path, monkeypatch):
    """FlowDrafterProposer on a latent checkpoint directory (VAE tensors under drafter.vae.*, as the
    reference's drafters ship): propose() against the oracle's chain on the same context."""
    from safetensors.torch import save_file
    hidden, V, n = 512, 4096, 1024
    cfg = _cfg(128, 256, 4, 1, layers=1, steps=2, expert_dim=hidden)
    W = make_weights(cfg, V, init="test", base_seed=9, hidden=hidden)
    W["lm_head.weight"] = (W["lm_head.weight"].float() * 8).half()
    drafter = {k: v for k, v in W.items() if k not in ("lm_head.weight", "embed_tokens.weight")}
    save_file({"drafter." + k: v.contiguous() for k, v in drafter.items()}, str(tmp_path / fp.WEIGHTS_NAME))
    (tmp_path / fp.CONFIG_NAME).write_text(json.dumps({"model_args": cfg.to_dict()}))
    sl = torch.randperm(V, generator=torch.Generator().manual_seed(3))[:n]
    slmod.save(tmp_path / "shortlist.pt", sl, vocab_size=V)
    for k in ("VLLM_SPEC_TREE", "CF_SHORTLIST", "CF_FLOW_STEPS", "CF_VAE_DIR"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("CF_DRAFTER_DIR", str(tmp_path))
    vc = SimpleNamespace(speculative_config=SimpleNamespace(num_speculative_tokens=5),
                         scheduler_config=SimpleNamespace(max_num_seqs=4))
    p = fp.FlowDrafterProposer(vc)
    p.bind_target(W["embed_tokens.weight"].to(cuda), W["lm_head.weight"].to(cuda))
    g = torch.Generator().manual_seed(12)
    hid = torch.randn(3, hidden, generator=g)
    hid = (hid / hid.pow(2).mean(-1, keepdim=True).sqrt()).half()
    slv = torch.unique(sl.long())
    toks = [int(slv[5]), int(slv[15]), int(slv[25])]
    p.stash_hidden_states(hid.to(cuda))
    out = p.propose([toks])
    assert isinstance(p.cfg, TreeVAEFlowConfig) and p.drafter.vae is not None
    assert len(out) == 1 and len(out[0]) == 5
    ctx = oflow.front_pad_context(to64(hid)[None], cfg.context_size)
    W64 = {k: to64(v) for k, v in W.items()}
    pred = ovae.predict_hidden(W64, ctx, _vcfg(cfg), _fcfg(cfg), "fp16", oracle_numerics(cfg))
    s64 = slv.numpy()
    score = lambda h, prev: ohead.head_with_bias(h, W64["lm_head.weight"][s64], W64["markov.w1.weight"],
                                                 W64["markov.w2.weight"][s64], prev)
    resid = lambda lp, nl: ohead.path_residual(W64, W64["embed_tokens.weight"], lp, nl, cfg.path_order)
    ref, trace = obeam.beam_chains(pred, np.array([toks[-1]]), s64, 4, 5, cfg.path_order, score, resid,
                                   return_trace=True)
    print(f"[latent proposer] gpu {out[0]} oracle {ref[0].tolist()}", flush=True)
    if out[0] != ref[0].tolist():
        near = any((ohead.margins(t["lp"], 4) <= 1e-3).any() or (ohead.margins(t["cand"], 4) <= 1e-3).any()
                   for t in trace)
        assert near, (out[0], ref[0].tolist())


@pytest.mark.gpu
def test_anchored_latent_drafter_matches_oracle(cuda):
    """An anchor_token drafter at the shipped 4B shapes (hidden 2560, latent 640 = expert_dim): the
    committed tokens' embeddings through anchor_in and each expert's anchor_mlp condition every
    flow block (cf/drafters/tree_flow.py:237-244, chunked_flow.py:256-262, 376), three requests."""
    hidden, V, B = 2560, 512, 3
    cfg = _cfg(640, 1920, 8, 2, layers=2, steps=2, expert_dim=640, anchor_token=True)
    W = make_weights(cfg, V, init="test", base_seed=23, hidden=hidden)
    print("[anchored latent drafter] hidden=2560 latent=640 L=2 E=2 B=3", flush=True)
    dr = Drafter(cfg, {k: v.to(cuda) for k, v in W.items()}, None, device=cuda)
    assert dr.anchored
    ctx = synthetic_context(B, 8, hidden, seed=31)
    tok = torch.tensor([5, 300, 0])
    pred = dr.predict_hidden(ctx.to(cuda), tok.to(cuda))
    plain = dr.predict_hidden(ctx.to(cuda))
    torch.cuda.synchronize()
    W64 = {k: to64(v) for k, v in W.items()}
    emb = W64["embed_tokens.weight"][tok.numpy()]
    ref = ovae.predict_hidden(W64, to64(ctx), _vcfg(cfg), _fcfg(cfg), "fp16", oracle_numerics(cfg, B), anchor=emb)
    err = rel_err(to64(pred), ref)
    moved = rel_err(to64(pred), to64(plain))
    print(f"  rel err {err:.3e} (anchor moves the draft by {moved:.3e})", flush=True)
    assert np.isfinite(to64(pred)).all() and err < TOL_FP16 and moved > 10 * TOL_FP16


@pytest.mark.gpu
@pytest.mark.parametrize("d,B", [(640, 1), (640, 12), (1024, 5), (1024, 24)])
def test_anchor_rows_and_anchored_flow_match_oracle(cuda, d, B):
    """cfh_flow_anchor (anchor_in + every expert's anchor_mlp, bit-for-bit in fp16 up to summation
    order) and cfh_flow_integrate_anchored against the oracle's flow with the anchor; d=1024 x 24
    requests runs two wide request groups side by side, d=640 x 12 one wide group with the unfolded
    cross attention."""
    from chain_flow_amd.flow import FusedFlow
    hidden, V = 2048, 256
    cfg = _cfg(d, 256, 4, 1, layers=2, steps=2, expert_dim=d, anchor_token=True)
    names = {n for n in param_specs(cfg, V, hidden=hidden) if not n.startswith(("vae.", "path_head.", "markov."))}
    W = make_weights(cfg, V, init="test", base_seed=29, names=names, hidden=hidden)
    print(f"[anchored flow] d={d} B={B}", flush=True)
    ff = FusedFlow(cfg, {k: v.to(cuda) for k, v in W.items()}, device=cuda)
    ctx = synthetic_context(B, 8, d, seed=B)
    tok = torch.randint(0, V, (B,), generator=torch.Generator().manual_seed(B))
    emb_w = W["embed_tokens.weight"].to(cuda, torch.float16)
    rows = ff.anchor(tok.to(cuda), emb_w)
    z = ff.predict_hidden(ctx.to(cuda), anchor=rows)
    torch.cuda.synchronize()
    W64 = {k: to64(v) for k, v in W.items()}
    emb = W64["embed_tokens.weight"][tok.numpy()]
    prefixes = ["expert."] + [f"extra_experts.{i}." for i in range(cfg.draft_length // cfg.chunk_size - 1)]
    ref_rows = oflow.anchor_rows(W64, emb, prefixes, "fp16")
    for c, r in enumerate(ref_rows):
        assert rel_err(to64(rows[c]), r) < 1e-3, c
    num = oracle_numerics(cfg, B)
    ref = oflow.predict_hidden(W64, to64(ctx), _fcfg(cfg), numerics=num, anchor=emb)
    err = rel_err(to64(z), ref)
    print(f"  rel err {err:.3e} ({num})", flush=True)
    assert np.isfinite(to64(z)).all() and err < TOL_FP16
