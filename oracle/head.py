"""Oracle: shortlisted lm_head, markov bias, fused path residual, log-softmax and top-k.

Follows, in the reference (``cf/`` = ``src/chain_flow/``):

* ``cf/vllm_plugin/flow_proposer.py:1021-1022``  ``_head``: ``h.to(fp16) @ W_sl.T`` -> fp16 logits,
  with ``W_sl = lm_w[sl]`` (``:739``)
* ``cf/vllm_plugin/flow_proposer.py:1024-1025``  ``_bias``: ``markov.w1(prev) @ w2_sl.T`` with
  ``w2_sl = markov.w2.weight[sl]`` (``:740``); ``cf/drafters/markov_flow.py:62-74``
* ``cf/vllm_plugin/flow_proposer.py:1027-1028``  ``_map``: shortlist-local -> global id
* ``cf/vllm_plugin/flow_proposer.py:1030-1037``  ``_nlive`` path trim (offsets >= depth are dead)
* ``cf/vllm_plugin/fused.py:20-37``  fused path residual: one baddbmm over the live offsets, masked sum,
  then ``path_head.mlp(path_head.norm(h))``; un-fused twin ``cf/drafters/tree_flow.py:434-450``
* ``cf/drafters/tree_flow.py:251-255``  ``_embed``: ``F.embedding(ids.clamp_min(0), embed_w)``
"""
from __future__ import annotations

import numpy as np

from oracle.flow import gelu, layer_norm, r16


def path_residual(W, embed_w, lastp, nlive, order, numerics="fp16"):
    """Fused ``_residual_from_lastp`` (``cf/vllm_plugin/fused.py:25-37``).

    lastp [N, order] int (global token ids, -1 = no ancestor); ``nlive`` = live offsets at this
    depth (``_nlive``) or None for all.  -> residual [N, d]."""
    o = order if nlive is None else min(nlive, order)
    lp = np.asarray(lastp)[:, :o]
    ft = np.float32 if W["path_head.norm.weight"].dtype == np.float32 else np.float64
    mask = (lp >= 0).astype(ft)
    emb = embed_w[np.maximum(lp, 0)]                                    # [N, o, d]
    terms = []
    for j in range(o):
        wj = W[f"path_head.offset_proj.{j}.weight"]
        bj = W[f"path_head.offset_proj.{j}.bias"]
        terms.append(r16(emb[:, j] @ wj.T + bj, numerics) * mask[:, j:j + 1])  # baddbmm, one rounding
    h = r16(np.sum(terms, axis=0), numerics)                             # masked sum over offsets
    a = r16(layer_norm(h, W["path_head.norm.weight"], W["path_head.norm.bias"], numerics), numerics)
    u = r16(a @ W["path_head.mlp.0.weight"].T + W["path_head.mlp.0.bias"], numerics)
    g = r16(gelu(u), numerics)
    return r16(g @ W["path_head.mlp.3.weight"].T + W["path_head.mlp.3.bias"], numerics)


def head_logits(h, w_sl, numerics="fp16"):
    """``_head``: [N, d] x [Vs, d]^T -> [N, Vs] (fp16 logits on the fp16 path)."""
    return r16(r16(h, numerics) @ w_sl.T, numerics)


def markov_bias(w1, w2_sl, prev, numerics="fp16"):
    """``_bias``: ``w1[prev] @ w2_sl.T`` -> [N, Vs]."""
    return r16(w1[np.asarray(prev)] @ w2_sl.T, numerics)


def head_with_bias(h, w_sl, w1, w2_sl, prev, numerics="fp16"):
    """``_head(h) + _bias(prev)`` as the beam computes it (two fp16 GEMMs, fp16 add)."""
    return r16(head_logits(h, w_sl, numerics) + markov_bias(w1, w2_sl, prev, numerics), numerics)


def log_softmax(x):
    """``torch.log_softmax(logits.float(), -1)``."""
    x = np.asarray(x, dtype=np.float64)
    m = x.max(-1, keepdims=True)
    return x - m - np.log(np.exp(x - m).sum(-1, keepdims=True))


def topk(x, k):
    """Largest-k along the last axis, descending; equal values ordered by lower index first
    (the tie rule the device kernels implement)."""
    x = np.asarray(x)
    order = np.argsort(-x, axis=-1, kind="stable")[..., :k]
    return np.take_along_axis(x, order, -1), order


def margins(x, k):
    """Gap between consecutive sorted values around each of the first k ranks: the quantity the
    parity contract conditions on (ids must match wherever the margin exceeds 1e-3).  Returns
    [..., k] with margin[i] = min(v[i-1]-v[i], v[i]-v[i+1]) (one-sided at the ends)."""
    v = np.sort(np.asarray(x, dtype=np.float64), axis=-1)[..., ::-1][..., :k + 1]
    up = np.concatenate([np.full(v.shape[:-1] + (1,), np.inf), v[..., :-2] - v[..., 1:-1]], -1)
    dn = v[..., :-1] - v[..., 1:]
    return np.minimum(up[..., :k], dn[..., :k])
