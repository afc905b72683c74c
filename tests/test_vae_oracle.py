"""Pins of the VAE oracle (oracle/vae.py), CPU only.

* against golden vectors written by the reference itself (tests/golden/make_golden_vae.py):
  TransformerHiddenVAE.encode_sequence(.).mu / decode_sequence at several row counts, the one-head
  fallback, and TreeVAEFlowDrafter.predict_hidden (encode -> latent flow -> decode);
* one encoder layer against torch's own nn.TransformerEncoderLayer (norm_first, GELU), the library
  module the reference instantiates, in float64;
* the anchored drafter (anchor_token): anchor_embed, each expert's anchor_mlp and
  predict_hidden(hidden, anchor_embed(tokens)) against the reference's own outputs, and that the
  anchor changes the draft (so the pin bites);
* that the fp16 restatement stays close to the fp32 one, and the row-count guard.
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import rel_err
from chain_flow_amd.config import TreeVAEFlowConfig, config_from_model_args
from chain_flow_amd.weights import make_weights, param_specs, vae_param_names
from oracle import flow as oflow
from oracle import vae as ovae

G = np.load(Path(__file__).parent / "golden" / "reference_vae_tiny.npz")
HIDDEN, LATENT, VOCAB, RANK, SEED = 64, 32, 96, 16, 5
TOL = 1e-5


def _cfg(E=2, inter=48, heads=4, anchor=False):
    return TreeVAEFlowConfig(context_size=8, draft_length=8, chunk_size=4, expert_dim=LATENT if anchor else HIDDEN,
                             num_heads=8, ffn_multiplier=6, num_drafter_layers=2, num_flow_steps=E,
                             init_mode="delta", markov_rank=RANK, path_order=4, path_ffn_multiplier=2,
                             latent_size=LATENT, vae_intermediate_size=inter, vae_num_layers=2,
                             vae_num_heads=heads, vae_max_sequence_length=16, anchor_token=anchor)


def _vcfg(cfg):
    return dict(intermediate_size=cfg.vae_intermediate_size, num_layers=cfg.vae_num_layers,
                num_heads=cfg.vae_num_heads, max_sequence_length=cfg.vae_max_sequence_length)


def _fcfg(cfg):
    return dict(draft_length=cfg.draft_length, chunk_size=cfg.chunk_size, num_layers=cfg.num_drafter_layers,
                num_heads=cfg.num_heads, num_flow_steps=cfg.num_flow_steps, init_mode=cfg.init_mode)


def _weights(cfg, sha_key=None):
    W = make_weights(cfg, VOCAB, init="test", dtype=torch.float32, base_seed=SEED, hidden=HIDDEN)
    if sha_key is not None:
        h = hashlib.sha256()
        for k in sorted(W):
            h.update(k.encode())
            h.update(W[k].float().contiguous().numpy().tobytes())
        assert h.digest() == G[sha_key].tobytes(), "weight generator drifted from the golden run"
    return {k: v.double().numpy() for k, v in W.items()}


@pytest.mark.parametrize("tag,inter,heads", [("h4", 48, 4), ("h1", 42, 4)])
def test_encode_decode_match_reference(tag, inter, heads):
    cfg = _cfg(2, inter, heads)
    V = ovae.vae_weights(_weights(cfg, f"weights_sha_{tag}"))
    hidden, z = G["hidden"].astype(np.float64), G["z"].astype(np.float64)
    for T in (8, 5):
        mu = ovae.encode_sequence_mu(V, hidden[:, :T], _vcfg(cfg), numerics="fp32")
        assert rel_err(mu, G[f"{tag}_mu_T{T}"]) < TOL
    for T in (8, 3):
        out = ovae.decode_sequence(V, z[:, :T], _vcfg(cfg), numerics="fp32")
        assert rel_err(out, G[f"{tag}_dec_T{T}"]) < TOL


def test_one_head_fallback_is_not_four_heads():
    """The 42-wide VAE must run one head: with four it would differ (so the pin above bites)."""
    cfg = _cfg(2, 42, 4)
    V = ovae.vae_weights(_weights(cfg))
    hidden = G["hidden"].astype(np.float64)
    vc = _vcfg(cfg)
    assert ovae.effective_heads(42, 4) == 1 and ovae.effective_heads(48, 4) == 4
    mu1 = ovae.encode_sequence_mu(V, hidden, vc, numerics="fp32")
    x = hidden @ V["encoder_in.weight"].T + V["encoder_in.bias"] + V["encoder_pos.weight"][:8][None]
    y1 = ovae.encoder_layer(V, "encoder.layers.0.", x, 1, "fp32")
    y2 = ovae.encoder_layer(V, "encoder.layers.0.", x, 2, "fp32")
    assert rel_err(y1, y2) > 1e-3
    assert rel_err(mu1, G["h1_mu_T8"]) < TOL


@pytest.mark.parametrize("E", [2, 3])
def test_latent_predict_hidden_matches_reference(E):
    cfg = _cfg(E)
    W = _weights(cfg)
    pred = ovae.predict_hidden(W, G["hidden"].astype(np.float64), _vcfg(cfg), _fcfg(cfg), numerics="fp32")
    assert rel_err(pred, G[f"pred_E{E}"]) < TOL


def test_anchored_predict_hidden_matches_reference():
    """anchor_embed = anchor_in(emb(token)), each expert's anchor_mlp (Linear, SiLU, Linear), and the
    anchored predict_hidden (cf/drafters/tree_flow.py:237-244, chunked_flow.py:256-262, 376)."""
    cfg = _cfg(2, anchor=True)
    W = _weights(cfg, "weights_sha_anchor")
    tok = G["anchor_tokens"]
    emb = W["embed_tokens.weight"][tok]
    t1 = oflow._lin(emb, W["anchor_in.weight"], W["anchor_in.bias"])
    assert rel_err(t1, G["anchor_in"]) < TOL
    rows = oflow.anchor_rows(W, emb, ["expert.", "extra_experts.0."], "fp32")
    for c in range(2):
        assert rel_err(rows[c], G[f"anchor_mlp_c{c}"]) < TOL
    hidden = G["anchor_hidden"].astype(np.float64)
    pred = ovae.predict_hidden(W, hidden, _vcfg(cfg), _fcfg(cfg), numerics="fp32", anchor=emb)
    assert rel_err(pred, G["pred_anchor_E2"]) < TOL
    none = ovae.predict_hidden(W, hidden, _vcfg(cfg), _fcfg(cfg), numerics="fp32")
    assert rel_err(none, G["pred_anchor_none_E2"]) < TOL
    # the anchor moves the draft well beyond the tolerance, and a per-expert mix-up would show
    assert rel_err(pred, none) > 1e-2
    assert rel_err(rows[0], rows[1]) > 1e-2


def test_anchor_names_follow_the_module_tree():
    """anchor_in then per expert anchor_mlp.{0,2}; nothing for an unanchored config."""
    from chain_flow_amd.weights import anchor_param_names
    assert anchor_param_names(_cfg()) == []
    names = anchor_param_names(_cfg(anchor=True))
    assert names[:2] == ["anchor_in.weight", "anchor_in.bias"]
    assert names[2:6] == ["expert.anchor_mlp.0.weight", "expert.anchor_mlp.0.bias",
                          "expert.anchor_mlp.2.weight", "expert.anchor_mlp.2.bias"]
    assert len(names) == 2 + 4 * 2
    specs = param_specs(_cfg(anchor=True), VOCAB, hidden=HIDDEN)
    assert specs["anchor_in.weight"][0] == (LATENT, HIDDEN)
    assert specs["extra_experts.0.anchor_mlp.2.weight"][0] == (LATENT, LATENT)


def test_encoder_layer_equals_torch_library():
    """nn.TransformerEncoderLayer(norm_first=True, activation="gelu", batch_first=True) in float64."""
    I, heads, T = 40, 5, 7
    torch.manual_seed(0)
    layer = torch.nn.TransformerEncoderLayer(d_model=I, nhead=heads, dim_feedforward=4 * I, dropout=0.0,
                                             activation="gelu", batch_first=True, norm_first=True).double().eval()
    with torch.no_grad():
        for p in layer.parameters():
            p.add_(torch.randn_like(p) * 0.1)
    W = {"l." + k: v.detach().numpy() for k, v in layer.state_dict().items()}
    x = torch.randn(2, T, I, dtype=torch.float64)
    with torch.no_grad():
        ref = layer(x).numpy()
    out = ovae.encoder_layer(W, "l.", x.numpy(), heads, "fp32")
    assert rel_err(out, ref) < 1e-12


def test_fp16_restatement_tracks_fp32():
    cfg = _cfg(2)
    V = ovae.vae_weights(_weights(cfg))
    hidden = G["hidden"].astype(np.float64)
    a = ovae.encode_sequence_mu(V, hidden, _vcfg(cfg), numerics="fp16")
    b = ovae.encode_sequence_mu(V, hidden, _vcfg(cfg), numerics="fp32")
    assert 0 < rel_err(a, b) < 5e-3
    assert np.array_equal(a, a.astype(np.float16).astype(np.float64))


def test_rows_beyond_position_table_are_refused():
    cfg = _cfg(2)
    V = ovae.vae_weights(_weights(cfg))
    vc = dict(_vcfg(cfg), max_sequence_length=4)
    with pytest.raises(ValueError, match="max_sequence_length"):
        ovae.encode_sequence_mu(V, G["hidden"].astype(np.float64), vc)


def test_config_and_names():
    """model_args parsing keeps known fields only; the pack order covers every VAE tensor but logvar."""
    cfg = config_from_model_args({"latent_size": 640, "vae_intermediate_size": 1920, "unknown_key": 1,
                                  "expert_dim": 2560, "num_flow_steps": 2})
    assert cfg.flow_dim == 640 and cfg.vae_heads == 8 and cfg.num_flow_steps == 2
    c = _cfg()
    names = vae_param_names(c)
    specs = {k for k in param_specs(c, VOCAB, hidden=HIDDEN) if k.startswith("vae.")}
    assert len(names) == 14 + 24 * c.vae_num_layers == len(set(names))
    assert specs - set(names) == {"vae.logvar.weight", "vae.logvar.bias"}


def test_anchor_weight_shapes_are_checked_before_any_device_work():
    """An anchor_in projecting to expert_dim != latent_size (the reference's module would fail at
    its first anchor_mlp) is refused with the parameter's name, before anything is packed."""
    from chain_flow_amd.config import flownet
    from chain_flow_amd.flow import FusedFlow
    cfg = TreeVAEFlowConfig(**{**flownet(640, layers=1, flow_steps=1).to_dict(), "latent_size": 640,
                               "anchor_token": True, "expert_dim": 640})
    W = {n: torch.zeros(shape[0], *(shape[1:])) for n, (shape, _, _) in param_specs(cfg, VOCAB, hidden=2560).items()
         if not n.startswith("vae.")}
    W["anchor_in.weight"] = torch.zeros(2560, 2560)
    with pytest.raises(ValueError, match="anchor_in.weight has shape"):
        FusedFlow(cfg, W, device="cpu")
