"""Oracle: tree-aware gated delta-net (GDN) recurrence for tree verification.

Follows ``cf/kernels/tree_scan.py`` (``cf/`` = ``src/chain_flow/``):

* ``:23-24``  ``_l2norm``: x / (||x|| + eps), eps 1e-6
* ``:27-38``  ``_delta_step``: S <- S e^g ; delta = (v - S^T k) beta ; S <- S + k (x) delta ; o = S^T q
* ``:41-73``  ``tree_gated_delta_scan``: every node starts from its parent's state (roots from S0),
  q/k l2-normalised, q scaled by Dk^-1/2; state layout [H, Dk, Dv]
* ``:78-90``  ``sequential_path_output``: the plain recurrence along one root->node path

and the vLLM-faithful gating prologue of ``cf/vllm_tree/tree_ssm.py:63-68``
(g = -exp(A_log) softplus(a + dt_bias), threshold 20; beta = sigmoid(b) rounded through bf16) plus
its l2norm variant x / sqrt(sum x^2 + eps) (``:60-62``), and the serving form of the recurrence
(``tree_gdn_vllm``): the per-node slot kernel ``cf/vllm_tree/tree_ssm.py:34-77`` and its path-parallel
twin ``:256-311``, in float32 with the storage rounding of the state slots.
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


def tree_gdn_vllm(mixed_qkv, a, b, A_log, dt_bias, state, node_slots, parent, prefix_slot, H, HV, K, V,
                  scale, state_bf16=True, use_qk_l2norm=True, form="slots"):
    """The serving tree GDN in float32.  mixed_qkv [N, 2HK + HV V] (q | k | v heads, value head hv
    uses q/k head hv // (HV // H)); a, b [N, HV]; A_log, dt_bias [HV]; state [slots, HV, V, K]
    (value-major).  form "slots" follows ``cf/vllm_tree/tree_ssm.py:34-77``: node n reads its
    parent's slot (roots read prefix_slot), stores its state to node_slots[n] (rounded to bf16 when
    state_bf16).  form "path" follows ``:256-311``: every node replays its root->node path from
    the prefix slot, rounding each ancestor's state.  -> (o [N, HV, V] float32 before the bf16
    output cast, new state array)."""
    f = np.float32
    X = np.asarray(mixed_qkv, f)
    N = X.shape[0]
    st = np.array(state, dtype=f, copy=True)
    rnd = _round_bf16_f32 if state_bf16 else (lambda x: np.asarray(x, f))
    A = np.asarray(A_log, f)
    dtb = np.asarray(dt_bias, f)
    av = np.asarray(a, f)
    bv = np.asarray(b, f)
    group = HV // H

    def qkv(m, hv):
        h = hv // group
        q = X[m, h * K:(h + 1) * K]
        k = X[m, H * K + h * K:H * K + (h + 1) * K]
        v = X[m, 2 * H * K + hv * V:2 * H * K + (hv + 1) * V]
        if use_qk_l2norm:
            q = (q / np.sqrt((q * q).sum(dtype=f) + f(1e-6))).astype(f)
            k = (k / np.sqrt((k * k).sum(dtype=f) + f(1e-6))).astype(f)
        return (q * f(scale)).astype(f), k, v

    G, B = vllm_gates_f32(av, bv, A, dtb)

    def gates(m, hv):
        return G[m, hv], B[m, hv]

    def step(Hs, m, hv):
        _, k, v = qkv(m, hv)
        g, beta = gates(m, hv)
        h2 = (Hs * np.exp(g)).astype(f)                      # [V, K]
        v2 = ((v - (h2 * k[None, :]).sum(-1, dtype=f)) * beta).astype(f)
        return (h2 + v2[:, None] * k[None, :]).astype(f)

    out = np.zeros((N, HV, V), f)
    for n in range(N):
        p = int(parent[n])
        if p >= n:
            raise ValueError("tree must be in BFS/topological order (parent < node)")
        for hv in range(HV):
            if form == "slots":
                src = prefix_slot if p < 0 else int(node_slots[p])
                Hs = step(st[src, hv], n, hv)
            else:
                path = path_to_root(parent, n)
                Hs = st[prefix_slot, hv].astype(f)
                for t, m in enumerate(path):
                    Hs = step(Hs, m, hv)
                    if t < len(path) - 1:
                        Hs = rnd(Hs)
            q, _, _ = qkv(n, hv)
            out[n, hv] = (Hs * q[None, :]).sum(-1, dtype=f)
            st[int(node_slots[n]), hv] = rnd(Hs)      # the slot holds the storage type
    return out, st


def vllm_gates_f32(a, b, A_log, dt_bias, threshold=20.0):
    """``vllm_gating`` evaluated in float32, as the kernels do (``cf/vllm_tree/tree_ssm.py:63-68``):
    -> (g, beta) [N, HV] float32."""
    f = np.float32
    x = (np.asarray(a, f) + np.asarray(dt_bias, f)[None, :]).astype(f)
    with np.errstate(over="ignore"):
        sp = np.where(x <= f(threshold), np.log(f(1.0) + np.exp(x)), x).astype(f)
    g = (-np.exp(np.asarray(A_log, f))[None, :] * sp).astype(f)
    with np.errstate(over="ignore"):
        beta = _round_bf16_f32((f(1.0) / (f(1.0) + np.exp(-np.asarray(b, f)))).astype(f))
    return g, beta


def _round_bf16_f32(x):
    return _round_bf16(x).astype(np.float32)
