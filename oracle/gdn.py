"""Oracle: tree-aware gated delta-net (GDN) recurrence for tree verification.

Follows ``cf/kernels/tree_scan.py`` (``cf/`` = ``src/chain_flow/``):

* ``:23-24``  ``_l2norm``: x / (||x|| + eps), eps 1e-6
* ``:27-38``  ``_delta_step``: S <- S e^g ; delta = (v - S^T k) beta ; S <- S + k (x) delta ; o = S^T q
* ``:41-73``  ``tree_gated_delta_scan``: every node starts from its parent's state (roots from S0),
  q/k l2-normalised, q scaled by Dk^-1/2; state layout [H, Dk, Dv]
* ``:78-90``  ``sequential_path_output``: the plain recurrence along one root->node path

and the vLLM-faithful gating prologue of ``cf/vllm_tree/tree_ssm.py:63-68``
(g = -exp(A_log) softplus(a + dt_bias), threshold 20; beta = sigmoid(b) rounded through bf16) plus
its l2norm variant x / sqrt(sum x^2 + eps) (``:60-62``).
"""
from __future__ import annotations

import numpy as np


def l2norm(x, eps=1e-6, mode="norm_eps"):
    x = np.asarray(x, dtype=np.float64)
    ss = (x * x).sum(-1, keepdims=True)
    if mode == "norm_eps":
        return x / (np.sqrt(ss) + eps)
    if mode == "sqrt_eps":
        return x / np.sqrt(ss + eps)
    raise ValueError(mode)


def delta_step(S, q, k, v, g, beta):
    """One recurrence step. S [.., H, Dk, Dv], q/k [.., H, Dk], v [.., H, Dv], g/beta [.., H]."""
    S = S * np.exp(g)[..., None, None]
    kv_mem = (S * k[..., None]).sum(-2)
    delta = (v - kv_mem) * beta[..., None]
    S = S + k[..., None] * delta[..., None, :]
    o = (S * q[..., None]).sum(-2)
    return S, o


def tree_gated_delta_scan(q, k, v, g, beta, parent, S0, use_qk_l2norm=True, l2mode="norm_eps"):
    """q,k [N,H,Dk]; v [N,H,Dv]; g,beta [N,H]; parent [N] (-1 = root, parent < node); S0 [H,Dk,Dv].
    -> (out [N,H,Dv], states [N,H,Dk,Dv]) in float64."""
    q = np.asarray(q, np.float64); k = np.asarray(k, np.float64); v = np.asarray(v, np.float64)
    g = np.asarray(g, np.float64); beta = np.asarray(beta, np.float64)
    if use_qk_l2norm:
        q = l2norm(q, mode=l2mode); k = l2norm(k, mode=l2mode)
    N, H, Dk = q.shape
    q = q * Dk ** -0.5
    states = np.zeros((N, H, Dk, v.shape[-1]))
    out = np.zeros((N, H, v.shape[-1]))
    for n in range(N):
        p = int(parent[n])
        if p >= n:
            raise ValueError("tree must be in BFS/topological order (parent < node)")
        Sp = np.asarray(S0, np.float64) if p < 0 else states[p]
        states[n], out[n] = delta_step(Sp, q[n], k[n], v[n], g[n], beta[n])
    return out, states


def path_to_root(parent, n):
    path = []
    while n >= 0:
        path.append(n)
        n = int(parent[n])
    return path[::-1]


def sequential_path_output(q, k, v, g, beta, path_ids, S0, use_qk_l2norm=True, l2mode="norm_eps"):
    """The recurrence along one path (node indices root..node) -> the last node's output [H, Dv]."""
    q = np.asarray(q, np.float64); k = np.asarray(k, np.float64)
    if use_qk_l2norm:
        q = l2norm(q, mode=l2mode); k = l2norm(k, mode=l2mode)
    q = q * q.shape[-1] ** -0.5
    S = np.asarray(S0, np.float64).copy()
    o = None
    for n in path_ids:
        S, o = delta_step(S, q[n], k[n], np.asarray(v[n], np.float64), np.asarray(g[n], np.float64),
                          np.asarray(beta[n], np.float64))
    return o


def build_ancestor_chain(parent, max_depth):
    """``build_ancestor_chain`` (``cf/vllm_tree/tree_ssm.py:314-328``): chain[i, 0] = i,
    chain[i, j] = j-th ancestor clamped at the root; depth [N]."""
    N = len(parent)
    depth = np.zeros(N, dtype=np.int64)
    for i in range(N):
        depth[i] = 0 if parent[i] < 0 else depth[parent[i]] + 1
    chain = np.zeros((N, max_depth + 1), dtype=np.int64)
    for i in range(N):
        cur = i
        for j in range(max_depth + 1):
            chain[i, j] = cur
            if parent[cur] >= 0:
                cur = int(parent[cur])
    return chain, depth


def vllm_gating(a, b, A_log, dt_bias, threshold=20.0):
    """g = -exp(A_log) softplus(a + dt_bias); beta = sigmoid(b) rounded through bf16
    (``cf/vllm_tree/tree_ssm.py:63-68``).  a, b [N, H]."""
    x = np.asarray(a, np.float64) + np.asarray(dt_bias, np.float64)
    sp = np.where(x <= threshold, np.log1p(np.exp(np.minimum(x, threshold))), x)
    g = -np.exp(np.asarray(A_log, np.float64)) * sp
    beta = 1.0 / (1.0 + np.exp(-np.asarray(b, np.float64)))
    beta = _round_bf16(beta)
    return g, beta


def _round_bf16(x):
    f = np.asarray(x, np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32).astype(np.float64)
