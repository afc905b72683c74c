"""Pins of the serving-form tree GDN oracle (oracle/gdn.py:tree_gdn_vllm, row a18).

The serving kernels (cf/vllm_tree/tree_ssm.py:34-77 per-node slots, :256-311 path-parallel) cannot
run here (vLLM and Triton-on-GPU are absent), so their restatement is pinned by:
- the reference's own claim, as an invariant: the path form is bit-identical to the slot form;
- reduction to the pinned research oracle (tree_gated_delta_scan, cf/kernels/tree_scan.py:41-73)
  when the state is stored in fp32 and one q/k head serves each value head;
- GQA = the same problem with the q/k heads repeated per value head;
- closed forms of the gating prologue (:63-68).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import gdn as ogdn

PARENTS = [-1, 0, 0, 1, 1, 2, 3, -1, 7]


def _problem(H, HV, K=128, V=64, N=len(PARENTS), seed=0, slots=None):
    rng = np.random.default_rng(seed)
    X = ogdn._round_bf16(rng.standard_normal((N, 2 * H * K + HV * V)))
    a = ogdn._round_bf16(rng.standard_normal((N, HV)))
    b = ogdn._round_bf16(rng.standard_normal((N, HV)))
    A = rng.standard_normal(HV).astype(np.float32)
    dtb = rng.standard_normal(HV).astype(np.float32)
    st = np.zeros((N + 2, HV, V, K), np.float32)
    st[1] = ogdn._round_bf16(0.1 * rng.standard_normal((HV, V, K)))
    node_slots = np.arange(2, N + 2) if slots is None else slots
    return X, a, b, A, dtb, st, node_slots


@pytest.mark.parametrize("state_bf16", [True, False])
@pytest.mark.parametrize("H,HV", [(2, 2), (2, 4)])
def test_path_form_is_bit_identical_to_slot_form(state_bf16, H, HV):
    X, a, b, A, dtb, st, sl = _problem(H, HV)
    args = (X, a, b, A, dtb, st, sl, PARENTS, 1, H, HV, 128, 64, 128 ** -0.5)
    o1, s1 = ogdn.tree_gdn_vllm(*args, state_bf16=state_bf16, form="slots")
    o2, s2 = ogdn.tree_gdn_vllm(*args, state_bf16=state_bf16, form="path")
    assert np.array_equal(o1, o2) and np.array_equal(s1, s2)


def test_fp32_state_is_the_tree_scan_with_vllm_gates():
    H = HV = 3
    K, V = 128, 64
    X, a, b, A, dtb, st, sl = _problem(H, HV, K=K, V=V)
    o, s = ogdn.tree_gdn_vllm(X, a, b, A, dtb, st, sl, PARENTS, 1, H, HV, K, V, K ** -0.5, state_bf16=False)
    g, beta = ogdn.vllm_gates_f32(a, b, A, dtb)
    N = X.shape[0]
    q = X[:, :H * K].reshape(N, H, K)
    k = X[:, H * K:2 * H * K].reshape(N, H, K)
    v = X[:, 2 * H * K:].reshape(N, HV, V)
    S0 = st[1].transpose(0, 2, 1)                       # [HV, V, K] -> [H, Dk, Dv]
    ro, rs = ogdn.tree_gated_delta_scan(q, k, v, g, beta, np.array(PARENTS), S0, l2mode="sqrt_eps")
    assert np.abs(o - ro).max() <= 1e-5 * np.abs(ro).max()
    got_states = s[sl].transpose(0, 1, 3, 2)            # slots -> [N, H, Dk, Dv]
    assert np.abs(got_states - rs).max() <= 1e-5 * np.abs(rs).max()


def test_gqa_equals_repeated_qk_heads():
    H, HV, K, V = 2, 4, 128, 64
    X, a, b, A, dtb, st, sl = _problem(H, HV, K=K, V=V)
    o, s = ogdn.tree_gdn_vllm(X, a, b, A, dtb, st, sl, PARENTS, 1, H, HV, K, V, K ** -0.5)
    N = X.shape[0]
    q = X[:, :H * K].reshape(N, H, K).repeat(HV // H, axis=1)
    k = X[:, H * K:2 * H * K].reshape(N, H, K).repeat(HV // H, axis=1)
    Xr = np.concatenate([q.reshape(N, -1), k.reshape(N, -1), X[:, 2 * H * K:]], axis=1)
    o2, s2 = ogdn.tree_gdn_vllm(Xr, a, b, A, dtb, st, sl, PARENTS, 1, HV, HV, K, V, K ** -0.5)
    assert np.array_equal(o, o2) and np.array_equal(s, s2)


def test_gating_closed_forms():
    A = np.array([0.0, np.log(2.0)], np.float32)
    dtb = np.array([0.0, 1.0], np.float32)
    a = np.array([[25.0, 30.0], [0.0, -1.0]], np.float32)     # x = a + dt_bias
    b = np.array([[0.0, 100.0], [-100.0, 3.0]], np.float32)
    g, beta = ogdn.vllm_gates_f32(a, b, A, dtb)
    assert g[0, 0] == np.float32(-25.0)                      # above the threshold: softplus(x) = x
    assert g[0, 1] == np.float32(-2.0 * 31.0)                # exp(log 2) = 2, x = 31
    assert np.isclose(g[1, 0], -np.log(2.0), rtol=1e-6)      # softplus(0) = log 2
    assert np.isclose(g[1, 1], -2.0 * np.log1p(np.exp(0.0)), rtol=1e-6)
    assert beta[0, 0] == 0.5 and beta[0, 1] == 1.0 and beta[1, 0] == 0.0
    assert ogdn._round_bf16(beta[1, 1]) == beta[1, 1]        # rounded through bf16
    assert abs(beta[1, 1] - 1.0 / (1.0 + np.exp(-3.0))) < 2 ** -8
