"""GPU parity of the tree gated delta net (cfh_gdn_tree) against the float64 oracle.

Contract (fp32 state): node outputs and node states within 1e-5 norm-relative of the oracle's
tree_gated_delta_scan on the same bf16 q/k/v and fp32 g/beta/S0.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_err, to64
from chain_flow_amd.gdn import L2_NORM_EPS, L2_SQRT_EPS, tree_gated_delta_scan
from oracle import gdn as ogdn

TOL = 1e-5


def beam_tree_parents(keep=4, depth=5, topb=4):
    """Parents of a width-`keep`, depth-`depth` beam tree in BFS order (first level: min(keep, topb)
    children of the root; later levels: `keep` nodes spread over the previous level)."""
    parents, prev = [], [-1]
    base = 0
    for lvl in range(depth):
        k = min(keep, len(prev) * topb)
        lvl_par = [prev[i % len(prev)] if lvl else -1 for i in range(k)]
        parents += lvl_par
        prev = list(range(base, base + k))
        base += k
    return np.array(parents)


def _inputs(N, H, Dk, Dv, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(N, H, Dk, generator=g).to(torch.bfloat16)
    k = torch.randn(N, H, Dk, generator=g).to(torch.bfloat16)
    v = torch.randn(N, H, Dv, generator=g).to(torch.bfloat16)
    gg = torch.nn.functional.logsigmoid(torch.randn(N, H, generator=g))
    beta = torch.rand(N, H, generator=g)
    S0 = torch.randn(H, Dk, Dv, generator=g) * 0.1
    return q, k, v, gg, beta, S0


def _run(cuda, parent, H=16, Dk=128, Dv=128, seed=5, l2mode=L2_NORM_EPS, states=True):
    N = len(parent)
    q, k, v, gg, beta, S0 = _inputs(N, H, Dk, Dv, seed)
    out, st = tree_gated_delta_scan(q.to(cuda), k.to(cuda), v.to(cuda), gg, beta, torch.tensor(parent), S0,
                                    l2mode=l2mode, write_states=states)
    torch.cuda.synchronize()
    mode = "norm_eps" if l2mode == L2_NORM_EPS else "sqrt_eps"
    ro, rs = ogdn.tree_gated_delta_scan(to64(q), to64(k), to64(v), to64(gg), to64(beta), parent, to64(S0),
                                        l2mode=mode)
    return out, st, ro, rs, (q, k, v, gg, beta, S0)


@pytest.mark.gpu
def test_gdn_beam_tree_matches_oracle(cuda):
    """Tree draft verification shape: beam width 4, depth 5 (plus a bushier variant), 16 heads,
    dk = dv = 128, fp32 state."""
    for parent in (beam_tree_parents(4, 5, 4), np.array([-1] + [0] * 4 + [1, 1, 2, 2, 3, 3, 4, 4] +
                                                         list(range(5, 13)) + list(range(13, 21)) + [21, 22])):
        out, st, ro, rs, _ = _run(cuda, parent)
        print(f"[gdn] N={len(parent)} out err {rel_err(to64(out), ro):.2e} state err {rel_err(to64(st), rs):.2e}",
              flush=True)
        assert rel_err(to64(out), ro) < TOL
        assert rel_err(to64(st), rs) < TOL


@pytest.mark.gpu
def test_gdn_chain_is_the_linear_recurrence(cuda):
    parent = np.arange(-1, 11)
    out, st, ro, rs, (q, k, v, gg, beta, S0) = _run(cuda, parent, H=4, Dv=64, seed=9)
    seq = ogdn.sequential_path_output(to64(q), to64(k), to64(v), to64(gg), to64(beta), list(range(12)), to64(S0))
    assert rel_err(to64(out)[-1], seq) < TOL
    assert rel_err(to64(st), rs) < TOL


@pytest.mark.gpu
def test_gdn_strong_decay_matches_oracle(cuda):
    """Gates of -30 (decay ~1e-13) and -inf (decay 0) along a chain and a tree: the running decay
    scale falls below its floor and is folded into the state; outputs and states stay within TOL."""
    for parent in (np.arange(-1, 9), np.array([-1, 0, 0, 1, 1, 2, 2, 3, 4, 5])):
        N = len(parent)
        q, k, v, gg, beta, S0 = _inputs(N, 4, 128, 64, 21)
        gg[2] = -30.0
        gg[5, :2] = float("-inf")
        gg[6] = -12.0
        out, st = tree_gated_delta_scan(q.to(cuda), k.to(cuda), v.to(cuda), gg, beta, torch.tensor(parent), S0)
        torch.cuda.synchronize()
        ro, rs = ogdn.tree_gated_delta_scan(to64(q), to64(k), to64(v), to64(gg), to64(beta), parent, to64(S0))
        print(f"[gdn strong decay] N={N} out err {rel_err(to64(out), ro):.2e} state err {rel_err(to64(st), rs):.2e}",
              flush=True)
        assert np.isfinite(to64(out)).all() and np.isfinite(to64(st)).all()
        assert rel_err(to64(out), ro) < TOL
        assert rel_err(to64(st), rs) < TOL


@pytest.mark.gpu
def test_gdn_forest_sqrt_eps_and_outputs_only(cuda):
    parent = np.array([-1, -1, 0, 1, 2, 2, -1, 6, 3])
    out, st, ro, rs, _ = _run(cuda, parent, H=3, Dv=192, seed=11, l2mode=L2_SQRT_EPS, states=False)
    assert st is None
    assert rel_err(to64(out), ro) < TOL


@pytest.mark.gpu
def test_gdn_large_deep_tree_matches_oracle(cuda):
    """A random 100-node tree of depth 9: paths longer than one staging batch of eight steps, and
    parents anywhere before their nodes."""
    rng = np.random.default_rng(4)
    parent = np.array([-1] + [int(rng.integers(0, i)) for i in range(1, 100)])
    out, st, ro, rs, _ = _run(cuda, parent, H=4, Dv=64, seed=13)
    print(f"[gdn] N=100 out err {rel_err(to64(out), ro):.2e} state err {rel_err(to64(st), rs):.2e}", flush=True)
    assert rel_err(to64(out), ro) < TOL
    assert rel_err(to64(st), rs) < TOL


@pytest.mark.gpu
def test_gdn_refuses_non_bfs_order(cuda):
    """A parent index at or after its node breaks the BFS contract: the kernel writes NaN for that
    node instead of reading a state that does not exist yet."""
    parent = np.array([-1, 0, 3, 1])
    q, k, v, gg, beta, S0 = _inputs(4, 2, 128, 64, 3)
    out, st = tree_gated_delta_scan(q.to(cuda), k.to(cuda), v.to(cuda), gg, beta, torch.tensor(parent), S0)
    torch.cuda.synchronize()
    assert np.isnan(to64(st)[2]).all()
    o = to64(out)
    assert np.isnan(o[2]).all()
    assert np.isfinite(o[[0, 1, 3]]).all()


# ---------------------------------------------------------------- serving (vLLM) form, row a18
def _vllm_inputs(N, H, HV, K, V, seed, state_dtype):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(N, 2 * H * K + HV * V, generator=g).to(torch.bfloat16)
    a = torch.randn(N, HV, generator=g).to(torch.bfloat16)
    b = torch.randn(N, HV, generator=g).to(torch.bfloat16)
    A_log = torch.randn(HV, generator=g) * 0.5
    dt_bias = torch.randn(HV, generator=g) * 0.5
    st = torch.zeros(N + 3, HV, V, K)
    st[1] = torch.randn(HV, V, K, generator=g) * 0.1
    st[N + 2] = 7.0                                  # a slot nobody may touch
    return X, a, b, A_log, dt_bias, st.to(state_dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("H,HV,state_dtype", [(16, 16, torch.bfloat16), (16, 16, torch.float32),
                                              (4, 16, torch.bfloat16)])
def test_gdn_vllm_form_matches_oracle(cuda, H, HV, state_dtype):
    """cfh_gdn_tree_vllm on the C5 beam tree (31 nodes, 16 value heads, K = V = 128) against the
    float32 slot-form oracle: fp32 states within 1e-5 norm-relative; bf16 states within 5e-4 (a
    storage rounding can land on the other side of a tie when the sums run in another order)."""
    from chain_flow_amd.gdn import tree_gdn_vllm
    parent = beam_tree_parents()
    N, K, V = len(parent), 128, 128
    X, a, b, A_log, dt_bias, st = _vllm_inputs(N, H, HV, K, V, 11, state_dtype)
    slots = torch.arange(2, N + 2, dtype=torch.int32)
    st_d = st.to(cuda)
    o = tree_gdn_vllm(X.to(cuda), a.to(cuda), b.to(cuda), A_log, dt_bias, st_d, slots, torch.tensor(parent),
                      num_q_heads=H, prefix_slot=1)
    torch.cuda.synchronize()
    bf = state_dtype == torch.bfloat16
    ro, rs = ogdn.tree_gdn_vllm(X.float().numpy(), a.float().numpy(), b.float().numpy(), A_log.numpy(),
                                dt_bias.numpy(), st.float().numpy(), slots.numpy(), parent, 1, H, HV, K, V,
                                K ** -0.5, state_bf16=bf, form="slots")
    got_o = o.float().cpu().numpy()
    got_s = st_d.float().cpu().numpy()
    eo = rel_err(got_o, ogdn._round_bf16(ro))
    es = rel_err(got_s, rs)
    print(f"[gdn vllm H={H} HV={HV} {state_dtype}] out err {eo:.2e} state err {es:.2e}", flush=True)
    # bf16 slots: storing the states in bf16 instead of fp32 moves them by ~2e-3 on this tree, so
    # 5e-4 also catches a kernel that skipped the storage rounding of an ancestor's state
    assert es < (5e-4 if bf else 1e-5)
    assert eo < 2e-3                             # output rounded to bf16 on both sides
    assert np.array_equal(got_s[N + 2], st[N + 2].float().numpy())   # untouched slot
    assert np.array_equal(got_s[1], st[1].float().numpy())           # the prefix slot is only read


@pytest.mark.gpu
def test_gdn_vllm_fp32_states_equal_research_kernel(cuda):
    """With fp32 slots and one q/k head per value head the serving kernel is the research kernel
    (cfh_gdn_tree, l2mode sqrt-eps) fed the same gates: same per-path recurrence."""
    from chain_flow_amd.gdn import tree_gdn_vllm
    parent = beam_tree_parents()
    N, H, K, V = len(parent), 16, 128, 128
    X, a, b, A_log, dt_bias, st = _vllm_inputs(N, H, H, K, V, 12, torch.float32)
    slots = torch.arange(2, N + 2, dtype=torch.int32)
    st_d = st.to(cuda)
    o = tree_gdn_vllm(X.to(cuda), a.to(cuda), b.to(cuda), A_log, dt_bias, st_d, slots, torch.tensor(parent),
                      num_q_heads=H)
    g, beta = ogdn.vllm_gates_f32(a.float().numpy(), b.float().numpy(), A_log.numpy(), dt_bias.numpy())
    q = X[:, :H * K].reshape(N, H, K)
    k = X[:, H * K:2 * H * K].reshape(N, H, K)
    v = X[:, 2 * H * K:].reshape(N, H, V)
    S0 = st[1].transpose(1, 2).contiguous()
    out, states = tree_gated_delta_scan(q.to(cuda), k.to(cuda), v.to(cuda), torch.from_numpy(g),
                                        torch.from_numpy(beta), torch.tensor(parent), S0, l2mode=L2_SQRT_EPS)
    torch.cuda.synchronize()
    ref_o = out.to(torch.bfloat16).float()
    assert rel_err(o.float().cpu().numpy(), ref_o.cpu().numpy()) < 4e-3
    got = st_d[2:N + 2].transpose(2, 3).cpu().numpy()
    assert rel_err(got, states.cpu().numpy()) < 1e-6


@pytest.mark.gpu
def test_gdn_vllm_refuses_bad_slots_on_the_device(cuda):
    """Slot validation happens in the kernel (no host synchronisation): nodes 3 and 5 sharing a
    slot, node 7 given the prefix slot and node 9 a slot past the state buffer get NaN outputs and
    write nothing, the status word is set, and every other node equals the run with valid slots."""
    from chain_flow_amd.gdn import tree_gdn_vllm
    parent = beam_tree_parents()
    N, H, K, V = len(parent), 16, 128, 128
    X, a, b, A_log, dt_bias, st = _vllm_inputs(N, H, H, K, V, 13, torch.bfloat16)
    good = torch.arange(2, N + 2, dtype=torch.int32)
    bad = good.clone()
    bad[5] = bad[3]
    bad[7] = 1
    bad[9] = st.shape[0]
    args = (X.to(cuda), a.to(cuda), b.to(cuda), A_log, dt_bias)
    st_good, st_bad = st.to(cuda), st.to(cuda)
    s_good = torch.zeros(1, dtype=torch.int32, device=cuda)
    s_bad = torch.zeros(1, dtype=torch.int32, device=cuda)
    print("[gdn vllm refused slots] 31 nodes, slots 3 = 5, 7 = prefix, 9 past the end", flush=True)
    og = tree_gdn_vllm(*args, st_good, good, torch.tensor(parent), num_q_heads=H, status=s_good)
    ob = tree_gdn_vllm(*args, st_bad, bad, torch.tensor(parent), num_q_heads=H, status=s_bad)
    torch.cuda.synchronize()
    assert int(s_good.item()) == 0 and int(s_bad.item()) == 1
    refused = [3, 5, 7, 9]
    assert torch.isnan(ob[refused].float()).all()
    keep = [n for n in range(N) if n not in refused]
    assert torch.equal(ob[keep], og[keep])
    stb = st_bad.cpu()
    for n in keep:
        assert torch.equal(stb[int(bad[n])], st_good.cpu()[int(good[n])])
    assert torch.equal(stb[int(bad[3])], st[int(bad[3])])          # the shared slot: untouched
    assert torch.equal(stb[1], st[1])                               # the prefix slot: only read
    for n in (7, 9):                                                # their valid slots: never written
        assert torch.equal(stb[int(good[n])], st[int(good[n])])
