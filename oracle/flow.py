"""Oracle: the chain-flow velocity net and Euler integrator (``TreeFlowDrafter.predict_hidden``).

Follows, in the reference (``cf/`` = ``src/chain_flow/``):

* ``cf/drafters/tree_flow.py:143-148``  ``_context`` front-padding (repeat the oldest row)
* ``cf/drafters/tree_flow.py:150-161``  ``init_latents`` (mode ``delta`` / ``repeat_last``)
* ``cf/drafters/tree_flow.py:163-174``  ``_chunk_args`` (previous rows are sliced from the step input)
* ``cf/drafters/tree_flow.py:176-190``  ``flow_velocity`` (one expert per chunk, velocities concatenated)
* ``cf/drafters/tree_flow.py:229-235``  ``integrate`` (Euler, dt = 1/E, tau = s*dt)
* ``cf/drafters/chunked_flow.py:264-275, 333-380``  ``pre_blocks`` (positions, time MLP, causal mask)
* ``cf/drafters/chunked_flow.py:185-202``  ``HiddenKVFlowBlock.forward`` (pre-LN self-MHA, cross-MHA,
  LN -> Linear(d, f*d) -> erf-GELU -> Linear(f*d, d))
* ``cf/drafters/chunked_flow.py:382-384``  ``post_blocks`` (out_norm + out_proj on the current rows)
* ``cf/drafters/tree_flow.py:237-241``, ``cf/drafters/chunked_flow.py:256-262, 376``  the anchored
  latent drafter: ``anchor_in(emb(token))`` through each expert's ``anchor_mlp`` (Linear, SiLU,
  Linear), added to every row after the position and time embeddings
* ``cf/csrc/fused_block.cu:280-325, 452-668, 674-722``  the fused-kernel numerics: fp32 residual,
  fp16-parked LayerNorm rows, fp16 q/k/v, attention output and GELU output; cross K/V from
  ``context_norm(ctx)`` computed once per draft.

Numerics (``numerics=``):

* ``"fp16"`` -- the reference's fused block kernel, which it engages only for D in {640, 1024},
  ffn x6, 8 heads, chunk rows in {4, 8}, at most 16 context rows and batch 1
  (``cf/cuda_block.py:95-102``, ``cf/drafters/chunked_flow.py:295-331``): fp32 residual stream,
  GELU of the unrounded pre-activation.
* ``"fp16_modules"`` -- torch's fp16 modules, what the reference runs for every other shape
  (``cf/drafters/chunked_flow.py:185-202`` with ``.half()`` weights): the residual stream is fp16,
  every sublayer output (out_proj, FFN down-projection) is rounded to fp16 before the add and the
  sum rounded again, and the FFN up-projection is rounded to fp16 before the GELU.
* ``"fp32"`` -- no rounding (the fp32 CPU plumbing).

Weights come in as a dict keyed by the reference's ``state_dict`` names
(``expert.blocks.{l}.self_attn.in_proj_weight`` ...), values float arrays already holding the exact
values the device path uses (fp16-representable for the fp16 path).
"""
from __future__ import annotations

import math

import numpy as np
from scipy.special import erf

LN_EPS = 1e-5


FP16_MODES = ("fp16", "fp16_modules")


def r16(x, numerics):
    """Round to fp16 when the fp16 path materialises this tensor; identity for fp32 numerics.
    The arithmetic type is kept: float32 arrays stay float32 (the fp32 CPU timing runs), anything
    else becomes float64."""
    x = np.asarray(x)
    ft = np.float32 if x.dtype == np.float32 else np.float64
    if numerics in FP16_MODES:
        return x.astype(np.float16).astype(ft)
    return x.astype(ft, copy=False)


def layer_norm(x, w, b, numerics, eps=LN_EPS):
    """``nn.LayerNorm`` over the last dim (biased variance).  The input row is first parked as fp16
    for the fp16 path, which is the dtype the reference's LayerNorm sees
    (``cf/csrc/fused_block.cu:291-304``)."""
    xx = r16(x, numerics)
    mu = xx.mean(-1, keepdims=True)
    var = ((xx - mu) ** 2).mean(-1, keepdims=True)
    return (xx - mu) / np.sqrt(var + eps) * w + b


def gelu(x):
    """``nn.GELU()`` default (approximate='none'): 0.5 x (1 + erf(x / sqrt 2))."""
    return 0.5 * x * (1.0 + erf(x * (1.0 / math.sqrt(2.0))))


def silu(x):
    return x / (1.0 + np.exp(-x))


def attention(q, k, v, heads, mask=None):
    """Scaled dot-product attention per head for ``nn.MultiheadAttention`` (batch_first).

    q [B, Sq, d], k/v [B, Sk, d] -> [B, Sq, d] (heads merged), scale 1/sqrt(d/heads), additive mask
    [Sq, Sk] (``cf/drafters/chunked_flow.py:273-275``)."""
    B, Sq, d = q.shape
    Sk = k.shape[1]
    hd = d // heads
    qh = q.reshape(B, Sq, heads, hd).transpose(0, 2, 1, 3)
    kh = k.reshape(B, Sk, heads, hd).transpose(0, 2, 1, 3)
    vh = v.reshape(B, Sk, heads, hd).transpose(0, 2, 1, 3)
    s = qh @ kh.transpose(0, 1, 3, 2) * (1.0 / math.sqrt(hd))
    if mask is not None:
        s = s + mask.astype(s.dtype)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(-1, keepdims=True)
    o = p @ vh
    return o.transpose(0, 2, 1, 3).reshape(B, Sq, d)


def causal_mask(S):
    """``torch.triu(full(-inf), diagonal=1)`` (``cf/drafters/chunked_flow.py:273-275``)."""
    m = np.zeros((S, S))
    m[np.triu_indices(S, 1)] = -np.inf
    return m


def front_pad_context(hidden, context_size):
    """``TreeFlowDrafter._context`` (``cf/drafters/tree_flow.py:143-148``): the last C rows; fewer
    than C are front-padded by repeating the OLDEST row."""
    n = hidden.shape[1]
    if n >= context_size:
        return hidden[:, -context_size:]
    pad = np.repeat(hidden[:, :1], context_size - n, axis=1)
    return np.concatenate([pad, hidden], axis=1)


def init_latents(context, draft_length, numerics, mode="delta"):
    """``TreeFlowDrafter.init_latents`` (``cf/drafters/tree_flow.py:150-161``), computed in the
    expert dtype: fp16 rounding of the delta, of ``steps * delta`` and of the sum."""
    last = context[:, -1:, :]
    if mode == "repeat_last":
        return np.repeat(last, draft_length, axis=1).copy()
    if mode != "delta":
        raise ValueError("init_mode must be 'delta' or 'repeat_last' (noise is not deterministic)")
    if context.shape[1] > 1:
        delta = r16(context[:, -1:, :] - context[:, -2:-1, :], numerics)
    else:
        delta = np.zeros_like(last)
    steps = np.arange(1, draft_length + 1, dtype=last.dtype).reshape(1, draft_length, 1)
    return r16(last + r16(steps * delta, numerics), numerics)


def _lin(x, w, b):
    y = x @ w.T
    return y + b if b is not None else y


def tau_embedding(W, pfx, tau, numerics):
    """``time_mlp(tau)`` = Linear(1, d) -> SiLU -> Linear(d, d) (``cf/drafters/chunked_flow.py:230-234,
    264-271``).  tau is a scalar shared by the batch."""
    h = r16(tau * W[pfx + "time_mlp.0.weight"][:, 0] + W[pfx + "time_mlp.0.bias"], numerics)
    h = r16(silu(h), numerics)
    return r16(_lin(h, W[pfx + "time_mlp.2.weight"], W[pfx + "time_mlp.2.bias"]), numerics)


def cross_kv(W, bp, ctx, numerics):
    """Cross-attention K/V of one block: ``context_norm(ctx)`` through in_proj rows [d:3d]
    (``cf/drafters/chunked_flow.py:194-199``; hoisted once per draft as in
    ``cf/csrc/fused_block.cu:674-722``)."""
    d = ctx.shape[-1]
    c = r16(layer_norm(ctx, W[bp + "context_norm.weight"], W[bp + "context_norm.bias"], numerics), numerics)
    w = W[bp + "cross_attn.in_proj_weight"]
    b = W[bp + "cross_attn.in_proj_bias"]
    k = r16(_lin(c, w[d:2 * d], b[d:2 * d]), numerics)
    v = r16(_lin(c, w[2 * d:], b[2 * d:]), numerics)
    return k, v


def block_forward(W, bp, res, kv, mask, heads, numerics):
    """One ``HiddenKVFlowBlock`` on the residual ``res`` [B, S, d]
    (``cf/drafters/chunked_flow.py:185-202``; stage structure of ``cf/csrc/fused_block.cu:528-662``)."""
    d = res.shape[-1]
    modules = numerics == "fp16_modules"

    def add(res, y):
        # fused kernel: fp32 residual += fp32 sublayer output; torch modules: fp16(res + fp16(y))
        return r16(res + r16(y, numerics), numerics) if modules else res + y

    # 1-2: self attention
    a = r16(layer_norm(res, W[bp + "self_norm.weight"], W[bp + "self_norm.bias"], numerics), numerics)
    w, b = W[bp + "self_attn.in_proj_weight"], W[bp + "self_attn.in_proj_bias"]
    qkv = r16(_lin(a, w, b), numerics)
    o = r16(attention(qkv[..., :d], qkv[..., d:2 * d], qkv[..., 2 * d:], heads, mask), numerics)
    res = add(res, _lin(o, W[bp + "self_attn.out_proj.weight"], W[bp + "self_attn.out_proj.bias"]))
    # 3-4: cross attention over the (hoisted) context K/V
    a = r16(layer_norm(res, W[bp + "cross_norm.weight"], W[bp + "cross_norm.bias"], numerics), numerics)
    w, b = W[bp + "cross_attn.in_proj_weight"], W[bp + "cross_attn.in_proj_bias"]
    q = r16(_lin(a, w[:d], b[:d]), numerics)
    o = r16(attention(q, kv[0], kv[1], heads, None), numerics)
    res = add(res, _lin(o, W[bp + "cross_attn.out_proj.weight"], W[bp + "cross_attn.out_proj.bias"]))
    # 5-6: feed-forward (the modules round the up-projection before the GELU)
    a = r16(layer_norm(res, W[bp + "ffn.0.weight"], W[bp + "ffn.0.bias"], numerics), numerics)
    u = _lin(a, W[bp + "ffn.1.weight"], W[bp + "ffn.1.bias"])
    g = r16(gelu(r16(u, numerics) if modules else u), numerics)
    return add(res, _lin(g, W[bp + "ffn.4.weight"], W[bp + "ffn.4.bias"]))


def fused_kernel_shape(d, ffn_mult, heads, chunk_rows, ctx_rows, batch):
    """Whether the reference runs this flow shape on its fused block kernel (``"fp16"`` numerics)
    rather than on torch's fp16 modules (``"fp16_modules"``): ``cuda_block.supported`` plus the
    batch-1 gate of ``_cf_fused_runner`` (``cf/cuda_block.py:95-102``,
    ``cf/drafters/chunked_flow.py:295-331``; ``CF_CUDA_BLOCK_BATCH`` is off by default)."""
    return (d in (640, 1024) and ffn_mult == 6 and heads == 8 and all(s in (4, 8) for s in chunk_rows)
            and 0 < ctx_rows <= 16 and batch == 1)


def anchor_rows(W, emb_rows, prefixes, numerics):
    """The anchored latent drafter's per-expert anchor vectors: ``anchor_embed`` =
    ``anchor_in(emb(token))`` (``cf/drafters/tree_flow.py:237-241``), then each chunk expert's
    ``anchor_mlp`` = Linear -> SiLU -> Linear (``cf/drafters/chunked_flow.py:256-262``), each module's
    output materialised in the expert dtype.  emb_rows [B, hidden] -> [expert][B, d]."""
    t1 = r16(_lin(r16(emb_rows, numerics), W["anchor_in.weight"], W["anchor_in.bias"]), numerics)
    out = []
    for p in prefixes:
        t2 = r16(_lin(t1, W[p + "anchor_mlp.0.weight"], W[p + "anchor_mlp.0.bias"]), numerics)
        t3 = r16(silu(t2), numerics)
        out.append(r16(_lin(t3, W[p + "anchor_mlp.2.weight"], W[p + "anchor_mlp.2.bias"]), numerics))
    return out


def expert_velocity(W, pfx, prev, cur, tau_add, chunk_start, kvs, cfg, numerics, anchor=None):
    """``HiddenKVFlowExpert.forward`` = pre_blocks -> L blocks -> post_blocks
    (``cf/drafters/chunked_flow.py:333-414``).  prev [B, P, d], cur [B, c, d] -> velocity [B, c, d].
    anchor [B, d]: the expert's anchor vector, added to every row (``:376``)."""
    x = np.concatenate([prev, cur], axis=1)
    P, c = prev.shape[1], cur.shape[1]
    pos = np.concatenate([np.arange(P), chunk_start + np.arange(c)])
    if max(P - 1, chunk_start + c - 1) >= cfg["draft_length"]:
        raise ValueError("hidden_kv_flow position exceeds configured draft length")
    x = r16(x + W[pfx + "position_embedding.weight"][pos][None], numerics)
    x[:, P:] = r16(x[:, P:] + tau_add[None, None, :], numerics)
    if anchor is not None:
        x = r16(x + anchor[:, None, :], numerics)
    mask = causal_mask(P + c)
    res = x.copy()
    for l in range(cfg["num_layers"]):
        res = block_forward(W, f"{pfx}blocks.{l}.", res, kvs[l], mask, cfg["num_heads"], numerics)
    a = r16(layer_norm(res[:, P:], W[pfx + "out_norm.weight"], W[pfx + "out_norm.bias"], numerics), numerics)
    return r16(_lin(a, W[pfx + "out_proj.weight"], W[pfx + "out_proj.bias"]), numerics)


def expert_prefixes(num_chunks):
    """State-dict prefixes of the chunk experts, in chunk order (``cf/drafters/tree_flow.py:113-131``)."""
    return ["expert."] + [f"extra_experts.{i}." for i in range(num_chunks - 1)]


def predict_hidden(W, context, cfg, numerics="fp16", return_trace=False, z0=None, anchor=None):
    """``TreeFlowDrafter.predict_hidden`` (``cf/drafters/tree_flow.py:229-244``).

    context [B, C, d] (values in the expert dtype) -> z_E [B, draft_length, d].
    cfg keys: draft_length, chunk_size, num_layers, num_heads, num_flow_steps, init_mode.
    z0: the initial latents when given (``init_mode="noise"`` draws them from torch's generator,
    ``tree_flow.py:154-155``: the caller passes the same draw).
    anchor: the committed tokens' embeddings [B, hidden] for an anchored drafter (``anchor_rows``
    turns them into each expert's vector), or None."""
    context = r16(context, numerics)
    K, cs, E = cfg["draft_length"], cfg["chunk_size"], cfg["num_flow_steps"]
    nch = K // cs
    pfxs = expert_prefixes(nch)
    kvs = [[cross_kv(W, f"{p}blocks.{l}.", context, numerics) for l in range(cfg["num_layers"])]
           for p in pfxs]
    anc = anchor_rows(W, anchor, pfxs, numerics) if anchor is not None else [None] * len(pfxs)
    z = init_latents(context, K, numerics, cfg.get("init_mode", "delta")) if z0 is None else np.array(z0, copy=True)
    trace = [z.copy()]
    dt = 1.0 / E
    for s in range(E):
        tau = float(r16(s * dt, numerics))
        vels = []
        for ci, p in enumerate(pfxs):
            start = ci * cs
            tau_add = tau_embedding(W, p, tau, numerics)
            vels.append(expert_velocity(W, p, z[:, :start], z[:, start:start + cs], tau_add, start,
                                        kvs[ci], cfg, numerics, anc[ci]))
        v = np.concatenate(vels, axis=1)
        z = r16(z + r16(dt * v, numerics), numerics)
        trace.append(z.copy())
    return (z, trace) if return_trace else z
