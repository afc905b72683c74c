"""Oracle: the hidden-state VAE of the latent drafters and the latent drafter's ``predict_hidden``.

Test infrastructure only: the tests and the smoke check compare the GPU results against it and the
benchmark's CPU leg times it; no product code imports it.

Follows, in the reference (``cf/`` = ``src/chain_flow/``):

* ``cf/vae/transformer_hidden.py:9-42``  ``TransformerHiddenVAE``: encoder_in Linear(hidden, inter)
  + encoder_pos rows, ``nn.TransformerEncoder`` of pre-LN layers (``norm_first=True``,
  ``activation="gelu"``, ``dim_feedforward=4*inter``, ``batch_first=True``, no mask),
  encoder_norm, mu Linear(inter, latent); the decoder mirrors it (decoder_in, decoder_pos,
  decoder layers, decoder_norm, decoder_out Linear(inter, hidden)).  ``num_heads`` falls back to 1
  when ``inter % num_heads != 0`` (:13).
* ``cf/vae/transformer_hidden.py:52-59`` ``encode_sequence`` (only ``mu`` is used by the drafter),
  ``:61-68`` ``decode_sequence``; position ids ``arange(rows)``, ``rows <= max_sequence_length``
  (:44-50).
* ``torch.nn.TransformerEncoderLayer`` with ``norm_first=True``:
  ``x = x + SA(norm1(x)); x = x + linear2(gelu(linear1(norm2(x))))``, SA =
  ``nn.MultiheadAttention`` (scaled dot product per head, no mask), LayerNorm eps 1e-5.
* ``cf/drafters/tree_vae_flow.py:163-175``  ``_encode`` / ``_decode`` / ``predict_hidden``:
  ``decode(integrate(encode(ctx).mu))`` -- the flow runs at the latent width.

``numerics="fp16"`` restates torch's fp16 modules: every Linear, LayerNorm, attention and GELU
output is rounded to fp16 (fp32-or-better arithmetic inside), the residual stream is fp16
(``x = fp16(x + fp16(sublayer))``) and linear1's output is rounded before the GELU.
``numerics="fp32"`` rounds nothing (float64 arithmetic).

Weights are a dict keyed by the VAE's own ``state_dict`` names (``encoder_in.weight`` ...); the
drafter-level helpers take the drafter's names (``vae.encoder_in.weight``, ``expert.`` ...).
"""
from __future__ import annotations

from oracle import flow as oflow
from oracle.flow import _lin, attention, gelu, layer_norm, r16


def effective_heads(inter, heads):
    """``num_heads if inter % num_heads == 0 else 1`` (``cf/vae/transformer_hidden.py:13``)."""
    return heads if inter % heads == 0 else 1


def encoder_layer(W, pfx, x, heads, numerics):
    """One ``nn.TransformerEncoderLayer(norm_first=True, activation="gelu")`` on x [B, T, I]."""
    I = x.shape[-1]
    a = r16(layer_norm(x, W[pfx + "norm1.weight"], W[pfx + "norm1.bias"], numerics), numerics)
    qkv = r16(_lin(a, W[pfx + "self_attn.in_proj_weight"], W[pfx + "self_attn.in_proj_bias"]), numerics)
    o = r16(attention(qkv[..., :I], qkv[..., I:2 * I], qkv[..., 2 * I:], heads, None), numerics)
    sa = r16(_lin(o, W[pfx + "self_attn.out_proj.weight"], W[pfx + "self_attn.out_proj.bias"]), numerics)
    x = r16(x + sa, numerics)
    a = r16(layer_norm(x, W[pfx + "norm2.weight"], W[pfx + "norm2.bias"], numerics), numerics)
    u = r16(_lin(a, W[pfx + "linear1.weight"], W[pfx + "linear1.bias"]), numerics)
    g = r16(gelu(u), numerics)
    ff = r16(_lin(g, W[pfx + "linear2.weight"], W[pfx + "linear2.bias"]), numerics)
    return r16(x + ff, numerics)


def _half(W, side, x_in, cfg, numerics):
    """One half: ``{side}_in`` + ``{side}_pos`` -> layers -> ``{side}_norm`` -> output Linear."""
    T = x_in.shape[1]
    if T > cfg["max_sequence_length"]:
        raise ValueError(f"sequence length {T} exceeds max_sequence_length={cfg['max_sequence_length']}")
    heads = effective_heads(cfg["intermediate_size"], cfg["num_heads"])
    side_mod = "encoder" if side == "enc" else "decoder"
    x = r16(_lin(x_in, W[f"{side_mod}_in.weight"], W[f"{side_mod}_in.bias"]), numerics)
    x = r16(x + W[f"{side_mod}_pos.weight"][:T][None], numerics)
    for l in range(cfg["num_layers"]):
        x = encoder_layer(W, f"{side_mod}.layers.{l}.", x, heads, numerics)
    a = r16(layer_norm(x, W[f"{side_mod}_norm.weight"], W[f"{side_mod}_norm.bias"], numerics), numerics)
    out = ("mu" if side == "enc" else "decoder_out")
    return r16(_lin(a, W[out + ".weight"], W[out + ".bias"]), numerics)


def encode_sequence_mu(W, hidden, cfg, numerics="fp16"):
    """``encode_sequence(hidden).mu``: hidden [B, T, hidden] -> mu [B, T, latent].
    cfg keys: intermediate_size, num_layers, num_heads, max_sequence_length."""
    return _half(W, "enc", r16(hidden, numerics), cfg, numerics)


def decode_sequence(W, z, cfg, numerics="fp16"):
    """``decode_sequence(z)``: z [B, T, latent] -> hidden [B, T, hidden]."""
    return _half(W, "dec", r16(z, numerics), cfg, numerics)


def vae_weights(W):
    """The VAE's own names from a drafter state dict (``vae.`` prefix stripped)."""
    return {k[4:]: v for k, v in W.items() if k.startswith("vae.")}


def predict_hidden(W, context, vae_cfg, flow_cfg, numerics="fp16", flow_numerics=None, anchor=None):
    """``TreeVAEFlowDrafter.predict_hidden`` (``cf/drafters/tree_vae_flow.py:172-175``):
    context [B, C, hidden] -> decode(integrate(encode(context).mu, anchor)) [B, draft_length, hidden].
    ``flow_numerics`` (default ``numerics``) is the latent flow's mode (``oracle.flow``); ``anchor``
    the committed tokens' embeddings [B, hidden] of an anchored drafter."""
    V = vae_weights(W)
    ctx_lat = encode_sequence_mu(V, context, vae_cfg, numerics)
    z = oflow.predict_hidden(W, ctx_lat, flow_cfg, numerics=numerics if flow_numerics is None else flow_numerics,
                             anchor=anchor)
    return decode_sequence(V, z, vae_cfg, numerics)
