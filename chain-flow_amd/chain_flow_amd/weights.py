"""Seeded synthetic drafter weights, keyed by the reference's state_dict names.

Every tensor is drawn from its own generator seeded with ``param_seed(name)`` =
sha256(name) mod 2^63 (mixed with a base seed), so any subset can be regenerated bit-identically
in another process, on the CPU or the GPU generator.  Names follow the reference's
``TreeFlowDrafter`` (``cf/drafters/tree_flow.py:107-131``), ``HiddenKVFlowExpert``
(``cf/drafters/chunked_flow.py:205-262``), ``HiddenKVFlowBlock`` (``:168-183``), ``MarkovHead``
(``cf/drafters/markov_flow.py:62-70``) and ``PathHead`` (``cf/drafters/tree_flow.py:80-96``), the
latent drafter's ``vae.`` module (``TransformerHiddenVAE``, ``cf/vae/transformer_hidden.py:9-42``),
plus the target model's ``lm_head.weight`` and ``embed_tokens.weight``.

Two initialisations:
* ``"baseline"`` -- Linear/Embedding weights ~N(0, 0.02), biases 0, LayerNorm weight 1 / bias 0
  (the synthetic drafting workloads).
* ``"test"`` -- every tensor random (weights ~N(0, 1/fan_in), biases ~N(0, 0.05), LayerNorm
  weight 1+N(0, 0.1) / bias N(0, 0.1)) so that parity tests exercise every parameter.
"""
from __future__ import annotations

import hashlib

import torch

from chain_flow_amd.config import TreeFlowConfig, TreeVAEFlowConfig


def param_seed(name: str, base_seed: int = 0) -> int:
    h = int.from_bytes(hashlib.sha256(name.encode()).digest()[:8], "little")
    return (h + base_seed * 0x9E3779B97F4A7C15) % (2 ** 63)


def expert_prefixes(cfg: TreeFlowConfig):
    return ["expert."] + [f"extra_experts.{i}." for i in range(cfg.num_chunks - 1)]


def expert_param_names(cfg: TreeFlowConfig, prefix: str):
    """State-dict names of one chunk expert in the order cfh_flow_pack_expert expects."""
    names = [prefix + "position_embedding.weight", prefix + "time_mlp.0.weight",
             prefix + "time_mlp.0.bias", prefix + "time_mlp.2.weight", prefix + "time_mlp.2.bias"]
    for l in range(cfg.num_drafter_layers):
        b = f"{prefix}blocks.{l}."
        names += [b + "self_norm.weight", b + "self_norm.bias",
                  b + "self_attn.in_proj_weight", b + "self_attn.in_proj_bias",
                  b + "self_attn.out_proj.weight", b + "self_attn.out_proj.bias",
                  b + "cross_norm.weight", b + "cross_norm.bias",
                  b + "context_norm.weight", b + "context_norm.bias",
                  b + "cross_attn.in_proj_weight", b + "cross_attn.in_proj_bias",
                  b + "cross_attn.out_proj.weight", b + "cross_attn.out_proj.bias",
                  b + "ffn.0.weight", b + "ffn.0.bias", b + "ffn.1.weight", b + "ffn.1.bias",
                  b + "ffn.4.weight", b + "ffn.4.bias"]
    names += [prefix + "out_norm.weight", prefix + "out_norm.bias",
              prefix + "out_proj.weight", prefix + "out_proj.bias"]
    return names


def anchor_param_names(cfg: TreeFlowConfig):
    """The anchored latent drafter's parameters in the order cfh_flow_anchor takes them: anchor_in,
    then each chunk expert's anchor_mlp (``cf/drafters/tree_vae_flow.py:116-125``,
    ``cf/drafters/chunked_flow.py:256-262``); none unless ``anchor_token``."""
    if not getattr(cfg, "anchor_token", False):
        return []
    names = ["anchor_in.weight", "anchor_in.bias"]
    for p in expert_prefixes(cfg):
        names += [p + "anchor_mlp.0.weight", p + "anchor_mlp.0.bias", p + "anchor_mlp.2.weight",
                  p + "anchor_mlp.2.bias"]
    return names


def vae_half_names(cfg: TreeVAEFlowConfig, side: str):
    """State-dict names (``vae.`` prefix) of one VAE half, ``side`` = "encoder" or "decoder", in
    the order cfh_vae_pack expects."""
    out_name = "vae.mu" if side == "encoder" else "vae.decoder_out"
    names = [f"vae.{side}_in.weight", f"vae.{side}_in.bias", f"vae.{side}_pos.weight"]
    for l in range(cfg.vae_num_layers):
        b = f"vae.{side}.layers.{l}."
        names += [b + "self_attn.in_proj_weight", b + "self_attn.in_proj_bias",
                  b + "self_attn.out_proj.weight", b + "self_attn.out_proj.bias",
                  b + "linear1.weight", b + "linear1.bias", b + "linear2.weight", b + "linear2.bias",
                  b + "norm1.weight", b + "norm1.bias", b + "norm2.weight", b + "norm2.bias"]
    names += [f"vae.{side}_norm.weight", f"vae.{side}_norm.bias", out_name + ".weight", out_name + ".bias"]
    return names


def vae_param_names(cfg: TreeVAEFlowConfig):
    """Every VAE parameter cfh_vae_pack reads (encoder half then decoder half; logvar is unused)."""
    return vae_half_names(cfg, "encoder") + vae_half_names(cfg, "decoder")


def _vae_specs(cfg: TreeVAEFlowConfig, hidden: int):
    I, Z, T = cfg.vae_intermediate_size, cfg.latent_size, cfg.vae_max_sequence_length
    specs = {}
    for side, kin, nout, out_name in (("encoder", hidden, Z, "vae.mu"), ("decoder", Z, hidden, "vae.decoder_out")):
        specs[f"vae.{side}_in.weight"] = ((I, kin), "linear", kin)
        specs[f"vae.{side}_in.bias"] = ((I,), "bias", kin)
        specs[f"vae.{side}_pos.weight"] = ((T, I), "embedding", I)
        for l in range(cfg.vae_num_layers):
            b = f"vae.{side}.layers.{l}."
            specs[b + "self_attn.in_proj_weight"] = ((3 * I, I), "linear", I)
            specs[b + "self_attn.in_proj_bias"] = ((3 * I,), "bias", I)
            specs[b + "self_attn.out_proj.weight"] = ((I, I), "linear", I)
            specs[b + "self_attn.out_proj.bias"] = ((I,), "bias", I)
            specs[b + "linear1.weight"] = ((4 * I, I), "linear", I)
            specs[b + "linear1.bias"] = ((4 * I,), "bias", I)
            specs[b + "linear2.weight"] = ((I, 4 * I), "linear", 4 * I)
            specs[b + "linear2.bias"] = ((I,), "bias", 4 * I)
            for n in ("norm1", "norm2"):
                specs[b + n + ".weight"] = ((I,), "ln_w", I)
                specs[b + n + ".bias"] = ((I,), "ln_b", I)
        specs[f"vae.{side}_norm.weight"] = ((I,), "ln_w", I)
        specs[f"vae.{side}_norm.bias"] = ((I,), "ln_b", I)
        specs[out_name + ".weight"] = ((nout, I), "linear", I)
        specs[out_name + ".bias"] = ((nout,), "bias", I)
        if side == "encoder":
            specs["vae.logvar.weight"] = ((Z, I), "linear", I)
            specs["vae.logvar.bias"] = ((Z,), "bias", I)
    return specs


def param_specs(cfg: TreeFlowConfig, vocab: int, target: bool = True, hidden: int | None = None):
    """name -> (shape, kind, fan_in) for every drafter parameter (and the target's head/embedding).
    The chunk experts run at ``cfg.flow_dim``; the path head, markov bias, VAE ends and target
    tensors at ``hidden`` (default ``cfg.expert_dim``: the target hidden size)."""
    d, fd = cfg.flow_dim, cfg.flow_dim * cfg.ffn_multiplier
    hidden = cfg.expert_dim if hidden is None else hidden
    specs = {}
    for p in expert_prefixes(cfg):
        for n in expert_param_names(cfg, p):
            short = n[len(p):]
            if short == "position_embedding.weight":
                specs[n] = ((cfg.draft_length, d), "embedding", d)
            elif short == "time_mlp.0.weight":
                specs[n] = ((d, 1), "linear", 1)
            elif short.endswith("norm.weight") or short.endswith("ffn.0.weight"):
                specs[n] = ((d,), "ln_w", d)
            elif short.endswith("norm.bias") or short.endswith("ffn.0.bias"):
                specs[n] = ((d,), "ln_b", d)
            elif short.endswith("in_proj_weight"):
                specs[n] = ((3 * d, d), "linear", d)
            elif short.endswith("in_proj_bias"):
                specs[n] = ((3 * d,), "bias", d)
            elif short.endswith("ffn.1.weight"):
                specs[n] = ((fd, d), "linear", d)
            elif short.endswith("ffn.1.bias"):
                specs[n] = ((fd,), "bias", d)
            elif short.endswith("ffn.4.weight"):
                specs[n] = ((d, fd), "linear", fd)
            elif short.endswith(".weight"):
                specs[n] = ((d, d), "linear", d)
            elif short.endswith(".bias"):
                specs[n] = ((d,), "bias", d)
            else:
                raise AssertionError(n)
    r = cfg.markov_rank
    specs["markov.w1.weight"] = ((vocab, r), "embedding_rank", r)
    specs["markov.w2.weight"] = ((vocab, r), "linear", r)
    d = hidden
    pf = cfg.path_ffn_multiplier * d
    for j in range(cfg.path_order):
        specs[f"path_head.offset_proj.{j}.weight"] = ((d, d), "linear", d)
        specs[f"path_head.offset_proj.{j}.bias"] = ((d,), "bias", d)
    specs["path_head.norm.weight"] = ((d,), "ln_w", d)
    specs["path_head.norm.bias"] = ((d,), "ln_b", d)
    specs["path_head.mlp.0.weight"] = ((pf, d), "linear", d)
    specs["path_head.mlp.0.bias"] = ((pf,), "bias", d)
    specs["path_head.mlp.3.weight"] = ((d, pf), "linear", pf)
    specs["path_head.mlp.3.bias"] = ((d,), "bias", pf)
    if isinstance(cfg, TreeVAEFlowConfig):
        specs.update(_vae_specs(cfg, hidden))
    for n in anchor_param_names(cfg):
        dz = cfg.flow_dim
        if n == "anchor_in.weight":
            specs[n] = ((dz, d), "linear", d)
        elif n == "anchor_in.bias":
            specs[n] = ((dz,), "bias", d)
        elif n.endswith(".weight"):
            specs[n] = ((dz, dz), "linear", dz)
        else:
            specs[n] = ((dz,), "bias", dz)
    if target:
        specs["lm_head.weight"] = ((vocab, d), "linear", d)
        specs["embed_tokens.weight"] = ((vocab, d), "embedding_tok", d)
    return specs


def _draw(shape, kind, fan_in, init, gen, device):
    def randn():
        return torch.randn(shape, generator=gen, dtype=torch.float32, device=device)
    if init == "baseline":
        if kind in ("linear", "embedding", "embedding_rank", "embedding_tok"):
            return randn() * 0.02
        if kind == "ln_w":
            return torch.ones(shape, dtype=torch.float32, device=device)
        return torch.zeros(shape, dtype=torch.float32, device=device)
    if init == "test":
        if kind == "linear":
            return randn() * (1.0 / fan_in ** 0.5)
        if kind == "embedding":
            return randn() * 0.5
        if kind == "embedding_rank":
            return randn()
        if kind == "embedding_tok":
            return randn()
        if kind == "bias":
            return randn() * 0.05
        if kind == "ln_w":
            return 1.0 + randn() * 0.1
        if kind == "ln_b":
            return randn() * 0.1
    raise ValueError(f"unknown init {init!r} / kind {kind!r}")


def make_weights(cfg: TreeFlowConfig, vocab: int, *, init: str = "test", dtype=torch.float16,
                 device="cpu", base_seed: int = 0, names=None, target: bool = True, hidden: int | None = None):
    """name -> tensor (dtype, device) for every parameter (or only ``names``)."""
    specs = param_specs(cfg, vocab, target=target, hidden=hidden)
    out = {}
    for name, (shape, kind, fan_in) in specs.items():
        if names is not None and name not in names:
            continue
        gen = torch.Generator(device=device)
        gen.manual_seed(param_seed(name, base_seed))
        out[name] = _draw(shape, kind, fan_in, init, gen, device).to(dtype)
    return out


def synthetic_context(batch: int, rows: int, d: int, seed: int = 1, dtype=torch.float16,
                      device="cpu"):
    """Context hidden states ~N(0, 1), each row rescaled to RMS 1."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(batch, rows, d, generator=g, dtype=torch.float32)
    x = x / x.pow(2).mean(-1, keepdim=True).sqrt()
    return x.to(dtype).to(device)
