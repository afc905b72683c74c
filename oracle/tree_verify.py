"""Oracle: the rest of the tree verify -- tree causal conv1d, the draft-tree attention's suffix half
with the log-sum-exp merge, and the greedy tree descent.

Test infrastructure only (the tests compare the GPU results against it).

Follows, in the reference:
* ``cf/vllm_tree/tree_ssm.py:393-423`` ``_tree_scan_conv_kernel``: node-serial in BFS order; node n
  reads its parent's slot (the prefix slot for roots), ``acc = bias + s0*w0 + s1*w1 + s2*w2 + x*w3``
  with bf16 products accumulated in fp32, SiLU, output in bf16; the node's slot gets
  ``(s1, s2, x, s3)``.
* patch ``vllm-0.25.1-chain-flow-tree.patch`` lines 529-575, ``_tree_suffix_eager``: fp32 scores
  ``scale * q.k`` over the request's own tree nodes, ``masked_fill(not_anc, -inf)``, ``amax``,
  ``exp``, ``sum``, ``lse = max + log(sum)``, ``probs = exp / sum``, ``probs @ v`` in fp32, cast to
  the output dtype, then vLLM's ``merge_attn_states`` with the prefix half (inf lse -> -inf,
  ``p_scale = e_p / (e_p + e_s)``, ``out = p_out * p_scale + s_out * s_scale``).
* patch lines 433-507, ``tree_greedy_descent_kernel``: from the root row emit the target's argmax,
  step to the FIRST child whose draft token equals it, repeat; tokens + bonus, path, length.

``numerics``: "bf16" / "fp16" round where the reference materialises that type; "fp32" rounds
nothing (float64 math) -- the form the library identities pin.
"""
from __future__ import annotations

import numpy as np


def round_to(x, numerics):
    x = np.asarray(x, dtype=np.float64)
    if numerics == "fp16":
        return x.astype(np.float16).astype(np.float64)
    if numerics == "bf16":
        f = x.astype(np.float32)
        u = f.view(np.uint32).astype(np.uint64)
        u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        return u.astype(np.uint32).view(np.float32).astype(np.float64)
    return x


def tree_conv(x, conv_state, weight, bias, node_slots, parent, prefix_slot, silu=True, numerics="bf16"):
    """x [N, dim]; conv_state [slots, dim, 4] (updated in place); weight [dim, 4]; bias [dim] or None.
    Returns out [N, dim].  parent: node index, -1 = root (slot prefix_slot)."""
    N, dim = x.shape
    out = np.zeros((N, dim))
    # bf16: products rounded to bf16, sums and the SiLU in fp32; fp32 numerics: float64 throughout
    ft = np.float32 if numerics == "bf16" else np.float64
    rp = (lambda v: round_to(v, "bf16").astype(ft)) if numerics == "bf16" else (lambda v: v)
    for n in range(N):
        pslot = prefix_slot if parent[n] < 0 else int(node_slots[parent[n]])
        s = conv_state[pslot].copy()
        acc = np.zeros(dim, ft) if bias is None else np.asarray(bias, ft).copy()
        acc = acc + rp(s[:, 0] * weight[:, 0])
        acc = acc + rp(s[:, 1] * weight[:, 1])
        acc = acc + rp(s[:, 2] * weight[:, 2])
        acc = acc + rp(x[n] * weight[:, 3])
        if silu:
            acc = acc * (ft(1.0) / (ft(1.0) + np.exp(-acc)))
        out[n] = round_to(acc, numerics)
        ns = int(node_slots[n])
        conv_state[ns] = np.stack([s[:, 1], s[:, 2], x[n], s[:, 3]], axis=1)
    return out


def tree_suffix_merge(q, k, v, prefix_out, prefix_lse, idx, not_anc, scale, numerics="bf16"):
    """q [T, H, D], k/v [T, Hkv, D]; prefix_out [S*N, H, D]; prefix_lse [H, S*N]; idx [S, N];
    not_anc [S, N, N] bool.  Returns merged [S*N, H, D] (compact tree order)."""
    S, N = idx.shape
    T, H, D = q.shape
    rep = H // k.shape[1]
    flat = idx.reshape(-1)
    qp = q[flat].reshape(S, N, H, D)
    kp = np.repeat(k[flat].reshape(S, N, -1, D), rep, axis=2)
    vp = np.repeat(v[flat].reshape(S, N, -1, D), rep, axis=2)
    scores = np.einsum("snhd,smhd->shnm", qp, kp) * scale
    scores = np.where(not_anc[:, None], -np.inf, scores)
    smax = scores.max(-1, keepdims=True)
    e = np.exp(scores - smax)
    den = e.sum(-1, keepdims=True)
    lse_s = (smax + np.log(den))[..., 0]                          # [S, H, N]
    probs = e / den
    s_out = round_to(np.einsum("shnm,smhd->snhd", probs, vp).reshape(S * N, H, D), numerics)
    s_lse = lse_s.transpose(1, 0, 2).reshape(H, S * N)            # [H, S*N]
    return merge_attn_states(prefix_out, prefix_lse, s_out, s_lse, numerics)


def merge_attn_states(p_out, p_lse, s_out, s_lse, numerics="bf16"):
    """vLLM's merge_attn_states: rows [M, H, D], lse [H, M]."""
    pl = np.where(np.isinf(p_lse), -np.inf, p_lse)
    sl = np.where(np.isinf(s_lse), -np.inf, s_lse)
    mx = np.maximum(pl, sl)
    ep, es = np.exp(pl - mx), np.exp(sl - mx)
    tot = ep + es
    ps, ss = (ep / tot).T[..., None], (es / tot).T[..., None]    # [M, H, 1]
    return round_to(p_out * ps + s_out * ss, numerics)


def greedy_descent(row_argmax, cu_draft, cu_sampled, draft, parents, max_spec):
    """-> out_tokens [B, max_spec+1] (-1 padded), path [B, max_spec] (-1 padded), length [B]."""
    B = len(cu_draft)
    out = np.full((B, max_spec + 1), -1, dtype=np.int64)
    path = np.full((B, max_spec), -1, dtype=np.int64)
    ln = np.zeros(B, dtype=np.int64)
    for r in range(B):
        d0 = 0 if r == 0 else int(cu_draft[r - 1])
        n = int(cu_draft[r]) - d0
        s0 = int(cu_sampled[r]) - (n + 1)
        cur, pos = -1, 0
        for _ in range(max_spec + 1):
            tok = int(row_argmax[s0 + cur + 1])
            out[r, pos] = tok
            nxt = -1
            if pos < max_spec:
                for i in range(n):
                    if parents[d0 + i] == cur and draft[d0 + i] == tok:
                        nxt = i
                        break
            if nxt < 0:
                break
            path[r, pos] = nxt
            cur = nxt
            pos += 1
        ln[r] = pos
    return out, path, ln


def first_argmax(logits):
    """torch.argmax: the first index of the maximum of each row."""
    return np.argmax(logits, axis=-1)
