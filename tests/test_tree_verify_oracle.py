"""Pins of the tree-verify oracle (oracle/tree_verify.py), CPU only.

* tree conv1d: with fp32 numerics a chain-shaped tree is torch's depthwise conv1d over the prefix
  state followed by the inputs (the library routine), and every tree node equals the chain of its
  own root->node path (the reference's claim that the tree form is the per-path causal conv);
* tree attention: the suffix + log-sum-exp merge equals one softmax over the union of the prefix
  keys and the node's ancestors computed directly (the decomposition the reference's docstring
  states, patch lines 410-418), and a chain-shaped tree with no prefix is causal attention;
* greedy descent: brute force over every root->node path on random trees, and a chain-shaped tree
  gives the stock greedy rule (accept while the draft equals the target's argmax).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import tree_verify as otv


def random_tree(rng, N, max_children=3):
    parent = [-1]
    while len(parent) < N:
        p = int(rng.integers(0, len(parent)))
        if sum(1 for q in parent if q == p) < max_children:
            parent.append(p)
    return np.array(parent)


def path_to(parent, n):
    out = []
    while n >= 0:
        out.append(n)
        n = parent[n]
    return out[::-1]


# ---------------------------------------------------------------- conv
def test_chain_conv_is_library_conv1d():
    rng = np.random.default_rng(0)
    N, dim = 9, 12
    x = rng.standard_normal((N, dim))
    w = rng.standard_normal((dim, 4))
    b = rng.standard_normal(dim)
    state = rng.standard_normal((3, dim, 4))
    parent = np.arange(N) - 1
    slots = np.arange(N) % 2 + 1          # alternate slots 1, 2 (a parent's slot is read before reuse)
    st = state.copy()
    st[0] = state[0]
    out = otv.tree_conv(x, st, w, b, slots, parent, 0, silu=False, numerics="fp32")
    seq = np.concatenate([state[0][:, :3].T, x], 0)        # [3 + N, dim]
    ref = torch.nn.functional.conv1d(torch.tensor(seq.T[None]), torch.tensor(w[:, None, :]),
                                     torch.tensor(b), groups=dim)[0].T.numpy()
    assert np.allclose(out, ref, rtol=0, atol=1e-12)
    silu = otv.tree_conv(x, state.copy(), w, b, slots, parent, 0, silu=True, numerics="fp32")
    assert np.allclose(silu, ref / (1 + np.exp(-ref)), rtol=0, atol=1e-12)


@pytest.mark.parametrize("seed", [1, 2])
def test_tree_conv_node_equals_its_path_chain(seed):
    rng = np.random.default_rng(seed)
    N, dim = 14, 10
    parent = random_tree(rng, N)
    x = rng.standard_normal((N, dim))
    w = rng.standard_normal((dim, 4))
    state = rng.standard_normal((N + 1, dim, 4))
    slots = np.arange(N) + 1
    out = otv.tree_conv(x, state.copy(), w, None, slots, parent, 0, numerics="fp32")
    for n in range(N):
        p = path_to(parent, n)
        chain = otv.tree_conv(x[p], state.copy(), w, None, np.arange(len(p)) + 1, np.arange(len(p)) - 1, 0,
                              numerics="fp32")
        assert np.array_equal(out[n], chain[-1])


def test_conv_state_roll_keeps_the_fourth_column():
    rng = np.random.default_rng(3)
    dim = 5
    x = rng.standard_normal((2, dim))
    w = rng.standard_normal((dim, 4))
    st = rng.standard_normal((3, dim, 4))
    p3 = st[0, :, 3].copy()
    otv.tree_conv(x, st, w, None, np.array([1, 2]), np.array([-1, 0]), 0, numerics="fp32")
    assert np.array_equal(st[2, :, 3], p3) and np.array_equal(st[2, :, 2], x[1])
    assert np.array_equal(st[2, :, 1], x[0]) and np.array_equal(st[1, :, 2], x[0])


# ---------------------------------------------------------------- attention
def _softmax_attn(q, K, V, scale):
    s = K @ q * scale
    m = s.max()
    e = np.exp(s - m)
    return (e / e.sum()) @ V, m + np.log(e.sum())


@pytest.mark.parametrize("rep", [1, 2])
def test_suffix_merge_is_attention_over_prefix_and_ancestors(rep):
    rng = np.random.default_rng(5)
    S, N, H, D, P = 2, 7, 4, 8, 5
    Hkv = H // rep
    T = S * N + 3
    q = rng.standard_normal((T, H, D))
    k = rng.standard_normal((T, Hkv, D))
    v = rng.standard_normal((T, Hkv, D))
    idx = rng.permutation(T)[:S * N].reshape(S, N)
    parents = [random_tree(rng, N) for _ in range(S)]
    not_anc = np.ones((S, N, N), dtype=bool)
    for s in range(S):
        for n in range(N):
            not_anc[s, n, path_to(parents[s], n)] = False
    Kp = rng.standard_normal((S, P, Hkv, D))
    Vp = rng.standard_normal((S, P, Hkv, D))
    scale = D ** -0.5
    p_out = np.zeros((S * N, H, D))
    p_lse = np.zeros((H, S * N))
    for s in range(S):
        for n in range(N):
            for h in range(H):
                o, l = _softmax_attn(q[idx[s, n], h], Kp[s, :, h // rep], Vp[s, :, h // rep], scale)
                p_out[s * N + n, h], p_lse[h, s * N + n] = o, l
    got = otv.tree_suffix_merge(q, k, v, p_out, p_lse, idx, not_anc, scale, numerics="fp32")
    for s in range(S):
        for n in range(N):
            anc = idx[s, path_to(parents[s], n)]
            for h in range(H):
                K = np.concatenate([Kp[s, :, h // rep], k[anc, h // rep]])
                V = np.concatenate([Vp[s, :, h // rep], v[anc, h // rep]])
                want, _ = _softmax_attn(q[idx[s, n], h], K, V, scale)
                assert np.allclose(got[s * N + n, h], want, rtol=0, atol=1e-12)


def test_chain_tree_without_prefix_is_causal_attention():
    rng = np.random.default_rng(6)
    N, H, D = 6, 2, 16
    q, k, v = (rng.standard_normal((N, H, D)) for _ in range(3))
    idx = np.arange(N)[None]
    not_anc = ~np.tril(np.ones((N, N), dtype=bool))[None]
    p_lse = np.full((H, N), -np.inf)
    got = otv.tree_suffix_merge(q, k, v, np.zeros((N, H, D)), p_lse, idx, not_anc, D ** -0.5, numerics="fp32")
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.tensor(q).transpose(0, 1), torch.tensor(k).transpose(0, 1), torch.tensor(v).transpose(0, 1),
        is_causal=True).transpose(0, 1).numpy()
    assert np.allclose(got, ref, rtol=0, atol=1e-12)


# ---------------------------------------------------------------- greedy descent
def _brute(row_argmax, draft, parents, s0, n):
    """The longest root->node path along which every node's token equals the argmax of its parent's
    row, first children winning ties; then the bonus at the path's end."""
    best = []
    def walk(cur, path):
        nonlocal best
        tok = row_argmax[s0 + cur + 1]
        kids = [i for i in range(n) if parents[i] == cur and draft[i] == tok]
        if not kids:
            if len(path) > len(best):
                best = list(path)
            return
        walk(kids[0], path + [kids[0]])      # only the first matching child is ever taken
    walk(-1, [])
    toks = [row_argmax[s0 + (best[j - 1] if j else -1) + 1] for j in range(len(best) + 1)]
    return best, toks


@pytest.mark.parametrize("seed", range(4))
def test_greedy_descent_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    B, V = 4, 5
    ns = [int(rng.integers(0, 12)) for _ in range(B)]
    draft, parents = [], []
    for n in ns:
        if n:
            parents += list(random_tree(rng, n, max_children=4) if n > 1 else [-1])
            draft += list(rng.integers(0, V, size=n))
    cu_draft = np.cumsum(ns)
    cu_sampled = np.cumsum([n + 1 for n in ns])
    row_argmax = rng.integers(0, V, size=int(cu_sampled[-1]))
    max_spec = max(ns + [1])
    out, path, ln = otv.greedy_descent(row_argmax, cu_draft, cu_sampled, np.array(draft, dtype=np.int64),
                                       np.array(parents, dtype=np.int64), max_spec)
    for r in range(B):
        d0 = 0 if r == 0 else int(cu_draft[r - 1])
        s0 = int(cu_sampled[r]) - (ns[r] + 1)
        bp, toks = _brute(row_argmax, draft[d0:d0 + ns[r]], parents[d0:d0 + ns[r]], s0, ns[r])
        assert ln[r] == len(bp) and list(path[r, :ln[r]]) == bp and list(out[r, :ln[r] + 1]) == toks
        assert (out[r, ln[r] + 1:] == -1).all() and (path[r, ln[r]:] == -1).all()


def test_chain_tree_is_stock_greedy_rejection():
    rng = np.random.default_rng(9)
    K, V = 6, 3
    draft = rng.integers(0, V, size=K)
    argmax = rng.integers(0, V, size=K + 1)
    out, path, ln = otv.greedy_descent(argmax, np.array([K]), np.array([K + 1]), draft, np.arange(K) - 1, K)
    acc = 0
    while acc < K and draft[acc] == argmax[acc]:
        acc += 1
    assert ln[0] == acc and list(out[0, :acc + 1]) == list(argmax[:acc + 1])


def test_wrappers_refuse_out_of_range_indices_before_any_launch():
    """Host-side index arguments are range-checked before the library is called (a negative slot or
    a parent after its child would address memory outside the buffers)."""
    from chain_flow_amd.tree_verify import tree_conv, tree_greedy_accept
    x = torch.zeros(3, 8, dtype=torch.bfloat16)
    st = torch.zeros(5, 8, 4, dtype=torch.bfloat16)
    w = torch.zeros(8, 4, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="node_slots"):
        tree_conv(x, st, w, None, [1, -1, 2], [-1, 0, 1])
    with pytest.raises(ValueError, match="node_slots"):
        tree_conv(x, st, w, None, [1, 2, 5], [-1, 0, 1])
    with pytest.raises(ValueError, match="parent"):
        tree_conv(x, st, w, None, [1, 2, 3], [-1, 2, 1])
    with pytest.raises(ValueError, match="prefix_slot"):
        tree_conv(x, st, w, None, [1, 2, 3], [-1, 0, 1], prefix_slot=5)
    lg = torch.zeros(4, 16, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="inconsistent"):
        tree_greedy_accept(lg, [2, 3], [3, 6], [1, 2, 3], [-1, 0, -1], 2)   # 6 rows > 4
