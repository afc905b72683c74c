"""GPU parity of the rest of the tree verify against the oracle: the tree causal conv1d (bf16,
states bit-exact, outputs within one bf16 ulp where the SiLU's exp rounds differently), the tree
attention suffix + log-sum-exp merge (bf16 and fp16, grouped heads; within 2e-3 and two ulps), and
the greedy tree accept (bit-exact)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_err, to64
from chain_flow_amd.tree_verify import tree_attn_merge, tree_conv, tree_greedy_accept
from oracle import tree_verify as otv


def rand_tree(n, seed=0):
    """n nodes in BFS-compatible order (every parent precedes its children), bushy near the root."""
    rng = np.random.default_rng(seed)
    return np.array([-1] + [int(rng.integers(max(0, i - 4), i)) for i in range(1, n)])


def path_to(parent, n):
    out = []
    while n >= 0:
        out.append(n)
        n = parent[n]
    return out[::-1]


@pytest.mark.gpu
def test_tree_conv_matches_oracle(cuda):
    parent = rand_tree(31, seed=1)
    N, dim, slots = len(parent), 6144, len(parent) + 4
    g = torch.Generator().manual_seed(2)
    x = torch.randn(N, dim, generator=g).bfloat16()
    w = (torch.randn(dim, 4, generator=g) * 0.5).bfloat16()
    b = (torch.randn(dim, generator=g) * 0.1).bfloat16()
    state = torch.randn(slots, dim, 4, generator=g).bfloat16()
    node_slots = np.arange(N) + 2
    print(f"[tree conv] N={N} dim={dim}", flush=True)
    st_gpu = state.to(cuda)
    out = tree_conv(x.to(cuda), st_gpu, w.to(cuda), b.to(cuda), node_slots, parent, prefix_slot=1)
    torch.cuda.synchronize()
    st_ref = to64(state)
    ref = otv.tree_conv(to64(x), st_ref, to64(w), to64(b), node_slots, parent, 1, silu=True, numerics="bf16")
    got = to64(out)
    ulp = np.abs(ref) * 2.0 ** -7 + 1e-30
    bad = np.abs(got - ref) > 0
    print(f"  differing {bad.mean():.2e} of outputs, max |d|/ulp {float((np.abs(got - ref) / ulp).max()):.2f}",
          flush=True)
    assert (np.abs(got - ref) <= ulp).all() and bad.mean() < 1e-3
    assert np.array_equal(to64(st_gpu), st_ref)             # every slot, untouched ones included


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,S,N,H,Hkv,D", [(torch.bfloat16, 1, 40, 16, 4, 256), (torch.float16, 2, 21, 8, 8, 128),
                                              (torch.bfloat16, 3, 9, 4, 2, 64)])
def test_tree_attn_merge_matches_oracle(cuda, dtype, S, N, H, Hkv, D):
    rng = np.random.default_rng(3)
    T = S * N + 5
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(T, h, D, generator=g).to(dtype) for h in (H, Hkv, Hkv))
    out = torch.randn(T, H, D, generator=g).to(dtype)
    pout = torch.randn(S * N, H, D, generator=g).to(dtype)
    plse = (torch.randn(H, S * N, generator=g) + 3.0).float()
    plse[0, 0] = float("-inf")                                # a row whose prefix is empty
    idx = rng.permutation(T)[:S * N].reshape(S, N)
    not_anc = np.ones((S, N, N), dtype=bool)
    for s in range(S):
        par = rand_tree(N, seed=10 + s)
        for n in range(N):
            not_anc[s, n, path_to(par, n)] = False
    scale = D ** -0.5
    print(f"[tree attn] {dtype} S={S} N={N} H={H} Hkv={Hkv} D={D}", flush=True)
    o_gpu = out.to(cuda)
    tree_attn_merge(q.to(cuda), k.to(cuda), v.to(cuda), o_gpu, pout.to(cuda), plse.to(cuda),
                    torch.as_tensor(idx), torch.as_tensor(not_anc), scale)
    torch.cuda.synchronize()
    num = "bf16" if dtype == torch.bfloat16 else "fp16"
    ref = otv.tree_suffix_merge(to64(q), to64(k), to64(v), to64(pout), to64(plse), idx, not_anc, scale, numerics=num)
    got = to64(o_gpu)[idx.reshape(-1)]
    err = rel_err(got, ref)
    ulp = 2.0 ** (-7 if dtype == torch.bfloat16 else -10)
    worst = float((np.abs(got - ref) / (np.abs(ref) * ulp + 1e-6)).max())
    print(f"  rel err {err:.2e}, worst {worst:.2f} ulp", flush=True)
    assert err < 2e-3 and worst <= 2.0
    others = np.setdiff1d(np.arange(T), idx.reshape(-1))
    assert torch.equal(o_gpu.cpu()[others], out[others])      # only the tree rows are written


@pytest.mark.gpu
def test_tree_greedy_accept_matches_oracle(cuda):
    rng = np.random.default_rng(5)
    V = 248320
    ns = [40, 0, 12, 20]
    parents, draft = [], []
    for r, n in enumerate(ns):
        if n:
            parents.append(rand_tree(n, seed=20 + r))
            draft.append(rng.integers(0, V, size=n))
    cu_draft = np.cumsum(ns)
    cu_sampled = np.cumsum([n + 1 for n in ns])
    R = int(cu_sampled[-1])
    logits = torch.randn(R, V, generator=torch.Generator().manual_seed(6)).bfloat16()
    # plant agreement along one random path per request so the descent goes deep
    j = 0
    for r, n in enumerate(ns):
        s0 = int(cu_sampled[r]) - (n + 1)
        if n:
            par, dr = parents[j], draft[j]
            leaf = int(rng.integers(n // 2, n))
            cur = -1
            for node in path_to(par, leaf):
                logits[s0 + cur + 1, int(dr[node])] = 20.0
                cur = node
            j += 1
        logits[s0, 7] = 19.0 if n == 0 else logits[s0, 7]
    dflat = np.concatenate(draft) if draft else np.zeros(0, np.int64)
    pflat = np.concatenate(parents) if parents else np.zeros(0, np.int64)
    max_spec = max(ns)
    print(f"[tree accept] B={len(ns)} rows={R} V={V}", flush=True)
    out, path, ln = tree_greedy_accept(logits.to(cuda), cu_draft, cu_sampled, dflat, pflat, max_spec)
    torch.cuda.synchronize()
    ra = otv.first_argmax(logits.float().numpy())
    o_ref, p_ref, l_ref = otv.greedy_descent(ra, cu_draft, cu_sampled, dflat, pflat, max_spec)
    print(f"  accepted {ln.cpu().tolist()} oracle {l_ref.tolist()}", flush=True)
    assert np.array_equal(ln.cpu().numpy(), l_ref)
    assert np.array_equal(path.cpu().numpy(), p_ref) and np.array_equal(out.cpu().numpy(), o_ref)
    assert l_ref.max() >= 3
