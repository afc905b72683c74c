"""The FlowDrafterProposer surface (host logic, no GPU): constructor validation, checkpoint
loading, shortlist resolution order / vocabulary guard / declared identity.

Mirrors the reference's behaviour in cf/vllm_plugin/flow_proposer.py:330-389, 579-765, 1006-1016
and cf/defaults.py:210-244 (its own tests cover the shortlist guard, tests/test_shortlist.py:69-121).
"""
from __future__ import annotations

import json
from types import SimpleNamespace

import pytest
import torch

from chain_flow_amd import shortlist as slmod
from chain_flow_amd.config import flownet
from chain_flow_amd.vllm_plugin import flow_proposer as fp
from chain_flow_amd.weights import make_weights, param_specs


def _vcfg(k=5, seqs=8):
    return SimpleNamespace(speculative_config=SimpleNamespace(num_speculative_tokens=k),
                           scheduler_config=SimpleNamespace(max_num_seqs=seqs))


@pytest.fixture
def ckpt(tmp_path):
    from safetensors.torch import save_file
    cfg = flownet(512, layers=1, flow_steps=2)
    names = {n for n in param_specs(cfg, 64, target=False)}
    W = make_weights(cfg, 64, init="test", names=names, target=False, dtype=torch.float32)
    save_file({"drafter." + k: v.contiguous() for k, v in W.items()} | {"other.x": torch.zeros(2)},
              str(tmp_path / fp.WEIGHTS_NAME))
    margs = {k: v for k, v in cfg.to_dict().items()}
    (tmp_path / fp.CONFIG_NAME).write_text(json.dumps({"model_args": margs, "data_args": {}, "loss_args": {}}))
    return tmp_path, cfg, W


def _env(monkeypatch, **kv):
    for k in ("VLLM_SPEC_TREE", "CF_TREE_KEEP", "CF_TREE_TOPB", "CF_TREE_DEPTH", "CF_TREE_BRANCH",
              "CF_DRAFTER_DIR", "CF_SHORTLIST", "CF_FLOW_STEPS", "CF_WIDTH", "CF_VAE_DIR"):
        monkeypatch.delenv(k, raising=False)
    for k, v in kv.items():
        monkeypatch.setenv(k, str(v))


def test_requires_a_drafter_dir(monkeypatch):
    _env(monkeypatch)
    with pytest.raises(ValueError, match="CF_DRAFTER_DIR"):
        fp.FlowDrafterProposer(_vcfg())


def test_chain_mode_widths(monkeypatch, ckpt):
    _env(monkeypatch, CF_DRAFTER_DIR=ckpt[0], CF_WIDTH=3)
    p = fp.FlowDrafterProposer(_vcfg(k=5))
    assert (p.K, p.draft_width, p.width, p.branching) == (5, 5, 3, False)


@pytest.mark.parametrize("env,match", [
    (dict(CF_WIDTH=9), "CF_WIDTH=9 is not supported"),
    (dict(CF_WIDTH=0), "CF_WIDTH=0 is not supported"),
    (dict(VLLM_SPEC_TREE=1, CF_TREE_KEEP=9, CF_TREE_TOPB=9, CF_TREE_DEPTH=2), "CF_TREE_KEEP=9 x CF_TREE_TOPB=9"),
])
def test_beam_limits_are_refused_with_a_message(monkeypatch, ckpt, env, match):
    """A beam wider than the kernels rank (width*width or keep*topb above 64) is refused at
    construction, not by a failing launch (or a runaway recursion) at the first draft."""
    _env(monkeypatch, CF_DRAFTER_DIR=ckpt[0], **env)
    k = 2 * int(env.get("CF_TREE_KEEP", 0)) + 1 if "VLLM_SPEC_TREE" in env else 5
    with pytest.raises(ValueError, match=match):
        fp.FlowDrafterProposer(_vcfg(k=k))


def test_drafter_refuses_unsupported_beams():
    """Drafter.beam_chains / beam_tree check the same limits before any launch."""
    from chain_flow_amd.drafter import Drafter
    dr = Drafter.__new__(Drafter)
    dr.device, dr.order = torch.device("cpu"), 4
    with pytest.raises(ValueError, match="beam width 9"):
        dr.beam_chains(None, torch.zeros(1), 5, width=9, pred=torch.zeros(1, 8, 16))
    with pytest.raises(ValueError, match="keep 16 x top-b 8"):
        dr.beam_tree(None, torch.zeros(1), keep=16, topb=8, depth=2, pred=torch.zeros(1, 8, 16))


def test_tree_mode_sizes_and_checks(monkeypatch, ckpt):
    _env(monkeypatch, CF_DRAFTER_DIR=ckpt[0], VLLM_SPEC_TREE=1, CF_TREE_KEEP=4, CF_TREE_TOPB=8, CF_TREE_DEPTH=5)
    p = fp.FlowDrafterProposer(_vcfg(k=21))
    assert (p.N, p.K, p.draft_width) == (20, 20, 20)
    with pytest.raises(AssertionError, match="num_speculative_tokens=21"):
        fp.FlowDrafterProposer(_vcfg(k=20))
    _env(monkeypatch, CF_DRAFTER_DIR=ckpt[0], VLLM_SPEC_TREE=1, CF_TREE_KEEP=8, CF_TREE_TOPB=4)
    with pytest.raises(ValueError, match="CF_TREE_KEEP=8 > CF_TREE_TOPB=4"):
        fp.FlowDrafterProposer(_vcfg(k=33))


def test_checkpoint_config_and_weights(monkeypatch, ckpt):
    d, cfg, W = ckpt
    _env(monkeypatch, CF_FLOW_STEPS=8)
    got = fp.load_drafter_config(str(d))
    assert got.expert_dim == 512 and got.num_flow_steps == 8 and got.draft_length == cfg.draft_length
    w = fp.load_drafter_weights(str(d), torch.float32)
    assert set(w) == set(W)                                   # prefix stripped, foreign keys dropped
    assert torch.equal(w["expert.out_proj.weight"], W["expert.out_proj.weight"])
    _env(monkeypatch, CF_FLOW_STEPS=0)
    with pytest.raises(ValueError, match="CF_FLOW_STEPS must be >= 1"):
        fp.load_drafter_config(str(d))


def test_vae_checkpoints_are_refused(tmp_path):
    (tmp_path / fp.CONFIG_NAME).write_text(json.dumps({"model_args": {"architecture": "tree_vae_flow"}}))
    with pytest.raises(ValueError, match="not supported"):
        fp.load_drafter_config(str(tmp_path))


def test_shortlist_resolution_order_and_guard(tmp_path):
    V = 1000
    # no candidates -> full head
    sl, why = fp.resolve_shortlist(str(tmp_path), V, None)
    assert sl is None
    # the drafter's own list wins
    slmod.save(tmp_path / "shortlist.pt", [5, 3, 900], vocab_size=V)
    sl, why = fp.resolve_shortlist(str(tmp_path), V, None)
    assert sl.tolist() == [3, 5, 900] and why.startswith("drafter checkpoint")
    # a list built for another vocabulary is refused, not clamped
    sl, why = fp.resolve_shortlist(str(tmp_path), 2000, None)
    assert sl is None and "refused" in why and "vocab_size=1000" in why
    # explicit "" = full head; explicit missing path fails loudly
    assert fp.resolve_shortlist(str(tmp_path), V, "")[0] is None
    with pytest.raises(FileNotFoundError):
        fp.resolve_shortlist(str(tmp_path), V, str(tmp_path / "nope.pt"))


def test_packaged_shortlist_is_the_last_resort(tmp_path):
    """Step 4 of the resolution order (``cf/defaults.py:205-244``): with no list beside the checkpoint,
    the packaged Qwen3.5 list is found for its own vocabulary, and the checkpoint's list still wins."""
    assert fp.PACKAGED_SHORTLIST.is_file()
    V = slmod.PACKAGED_VOCAB
    sl, why = fp.resolve_shortlist(str(tmp_path), V, None)
    assert sl is not None and sl.numel() == slmod.PACKAGED_ROWS and why == "packaged shortlist_qwen3_5.pt"
    assert slmod.ids_content_sha(sl) == "42fb98262c247aaf79c860da979b048c96408c885416161c6e83c2a93cc6dbfb"
    assert [p for _, p in fp.shortlist_candidates(str(tmp_path))] == ["packaged"]
    slmod.save(tmp_path / "shortlist.pt", [5, 3, 900], vocab_size=V)
    sl, why = fp.resolve_shortlist(str(tmp_path), V, None)
    assert sl.tolist() == [3, 5, 900] and why.startswith("drafter checkpoint")
    assert [p for _, p in fp.shortlist_candidates(str(tmp_path))] == ["drafter checkpoint", "packaged"]


def test_declared_identity_mismatch_raises(tmp_path):
    V = 1000
    slmod.save(tmp_path / "shortlist.pt", [1, 2, 3], vocab_size=V)
    good = slmod.ids_content_sha(torch.tensor([1, 2, 3]))
    (tmp_path / fp.CONFIG_NAME).write_text(json.dumps({"model_args": {}, "shortlist": {"rows": 3, "ids_sha256": good}}))
    assert fp.resolve_shortlist(str(tmp_path), V, None)[0].tolist() == [1, 2, 3]
    (tmp_path / fp.CONFIG_NAME).write_text(json.dumps({"model_args": {}, "shortlist": {"rows": 4}}))
    with pytest.raises(RuntimeError, match="does not match what this drafter declares"):
        fp.resolve_shortlist(str(tmp_path), V, None)


def _latent_cfg(**kw):
    from chain_flow_amd.config import TreeVAEFlowConfig
    base = dict(context_size=8, draft_length=8, chunk_size=4, expert_dim=1024, num_heads=8, ffn_multiplier=6,
                num_drafter_layers=1, num_flow_steps=2, latent_size=64, vae_intermediate_size=64,
                vae_num_layers=1, vae_num_heads=4, vae_max_sequence_length=16)
    base.update(kw)
    return TreeVAEFlowConfig(**base)


def test_latent_checkpoint_is_a_vae_drafter(monkeypatch, tmp_path):
    """VAE fields in model_args (or drafter.vae.* tensors) select TreeVAEFlowConfig, as every
    checkpoint the reference proposer serves is built (cf/vllm_plugin/flow_proposer.py:616-632)."""
    from safetensors.torch import save_file
    from chain_flow_amd.config import TreeVAEFlowConfig
    _env(monkeypatch)
    cfg = _latent_cfg()
    W = make_weights(cfg, 64, init="test", target=False, dtype=torch.float32, hidden=128)
    save_file({"drafter." + k: v.contiguous() for k, v in W.items()}, str(tmp_path / fp.WEIGHTS_NAME))
    (tmp_path / fp.CONFIG_NAME).write_text(json.dumps({"model_args": cfg.to_dict()}))
    got = fp.load_drafter_config(str(tmp_path))
    assert isinstance(got, TreeVAEFlowConfig) and got.flow_dim == 64 and got.latent_size == 64
    assert W["expert.out_proj.weight"].shape == (64, 64) and W["path_head.norm.weight"].shape == (128,)
    # tensors alone (model_args without VAE fields) still mean a latent drafter
    margs = {k: v for k, v in cfg.to_dict().items() if k not in fp.VAE_FIELDS}
    (tmp_path / fp.CONFIG_NAME).write_text(json.dumps({"model_args": margs}))
    assert isinstance(fp.load_drafter_config(str(tmp_path)), TreeVAEFlowConfig)


def test_vae_dir_resolution(monkeypatch, tmp_path):
    """_load_frozen_vae's lookup (cf/drafters/tree_vae_flow.py:57-87): CF_VAE_DIR over vae_dir,
    model.safetensors else the newest checkpoint-N, vae.-prefixed or bare keys, named errors."""
    from safetensors.torch import save_file
    from chain_flow_amd.vae import load_vae_dir
    _env(monkeypatch)
    assert load_vae_dir(_latent_cfg()) is None
    for n, val in ((3, 1.0), (10, 2.0)):
        (tmp_path / f"checkpoint-{n}").mkdir()
        save_file({"encoder_in.bias": torch.full((4,), val)}, str(tmp_path / f"checkpoint-{n}" / "model.safetensors"))
    got = load_vae_dir(_latent_cfg(vae_dir=str(tmp_path)))
    assert set(got) == {"vae.encoder_in.bias"} and float(got["vae.encoder_in.bias"][0]) == 2.0
    save_file({"vae.mu.bias": torch.ones(2), "other": torch.ones(1)}, str(tmp_path / "model.safetensors"))
    assert set(load_vae_dir(_latent_cfg(vae_dir=str(tmp_path)))) == {"vae.mu.bias"}
    with pytest.raises(FileNotFoundError, match="vae_dir in the checkpoint config"):
        load_vae_dir(_latent_cfg(vae_dir=str(tmp_path / "absent")))
    monkeypatch.setenv("CF_VAE_DIR", str(tmp_path / "empty"))
    (tmp_path / "empty").mkdir()
    with pytest.raises(FileNotFoundError, match="CF_VAE_DIR") as e:
        load_vae_dir(_latent_cfg(vae_dir=str(tmp_path)))
    assert "neither of the above" in str(e.value)


def test_twopass_default_and_explicit_width(monkeypatch, ckpt):
    """CF_TWOPASS_M defaults to 8192 shared (the reference's defaults table); a default wider than
    the head is dropped, an explicit one is refused (cf/vllm_plugin/flow_proposer.py:766-775)."""
    d, cfg, W = ckpt
    _env(monkeypatch, CF_DRAFTER_DIR=d)
    for k in ("CF_TWOPASS_M", "CF_TWOPASS_SHARED", "CF_TWOPASS_SEED"):
        monkeypatch.delenv(k, raising=False)
    p = fp.FlowDrafterProposer(_vcfg())
    assert (p.twopass_m, p.twopass_shared, p.twopass_seed) == (8192, True, False)
    V = 64
    emb = torch.zeros(V, 512, dtype=torch.float16)
    monkeypatch.setenv("CF_TWOPASS_M", "100")
    monkeypatch.setenv("CF_SHORTLIST", "")               # full head: 64 rows
    q = fp.FlowDrafterProposer(_vcfg())
    q.bind_target(emb, emb.clone())
    with pytest.raises(ValueError, match="CF_TWOPASS_M=100 >= head rows 64"):
        q._build()
