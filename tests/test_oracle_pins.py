"""Pins of the CPU oracle that do not come from the reference's golden vectors: closed forms,
invariants and library identities, each chosen so that a plausible mistake (a dropped term, a
wrong sign or index, a transposed operand, an off-by-one step count) fails it.

Reference anchors: init_latents closed form (cf/drafters/tree_flow.py:150-161, pinned by the
reference's own tests/test_chunked_flow.py:80-98); Euler integrate (tree_flow.py:229-235);
causal mask (cf/drafters/chunked_flow.py:273-275); context-only cross K/V (:194-199); PathHead
offset masking and _nlive trimming (cf/vllm_plugin/fused.py:25-37, flow_proposer.py:1030-1037);
tree_gated_delta_scan (cf/kernels/tree_scan.py:27-90).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import beam as obeam
from oracle import flow as oflow
from oracle import gdn as ogdn
from oracle import head as ohead

D, H, L = 64, 8, 2


def _weights(seed=0, d=D, chunks=2, layers=L, draft_length=8, ffn=6):
    """Random float64 weights under the reference's state-dict names (every tensor random)."""
    rng = np.random.default_rng(seed)
    W = {}
    for c, p in enumerate(oflow.expert_prefixes(chunks)):
        W[p + "position_embedding.weight"] = rng.normal(0, 0.5, (draft_length, d))
        W[p + "time_mlp.0.weight"] = rng.normal(0, 1, (d, 1))
        W[p + "time_mlp.0.bias"] = rng.normal(0, 0.1, d)
        W[p + "time_mlp.2.weight"] = rng.normal(0, d ** -0.5, (d, d))
        W[p + "time_mlp.2.bias"] = rng.normal(0, 0.1, d)
        for l in range(layers):
            b = f"{p}blocks.{l}."
            for n in ("self_norm", "cross_norm", "context_norm", "ffn.0"):
                W[b + n + ".weight"] = 1 + rng.normal(0, 0.1, d)
                W[b + n + ".bias"] = rng.normal(0, 0.1, d)
            for a in ("self_attn", "cross_attn"):
                W[b + a + ".in_proj_weight"] = rng.normal(0, d ** -0.5, (3 * d, d))
                W[b + a + ".in_proj_bias"] = rng.normal(0, 0.05, 3 * d)
                W[b + a + ".out_proj.weight"] = rng.normal(0, d ** -0.5, (d, d))
                W[b + a + ".out_proj.bias"] = rng.normal(0, 0.05, d)
            W[b + "ffn.1.weight"] = rng.normal(0, d ** -0.5, (ffn * d, d))
            W[b + "ffn.1.bias"] = rng.normal(0, 0.05, ffn * d)
            W[b + "ffn.4.weight"] = rng.normal(0, (ffn * d) ** -0.5, (d, ffn * d))
            W[b + "ffn.4.bias"] = rng.normal(0, 0.05, d)
        W[p + "out_norm.weight"] = 1 + rng.normal(0, 0.1, d)
        W[p + "out_norm.bias"] = rng.normal(0, 0.1, d)
        W[p + "out_proj.weight"] = rng.normal(0, d ** -0.5, (d, d))
        W[p + "out_proj.bias"] = rng.normal(0, 0.05, d)
    return W


def _cfg(E, layers=L):
    return dict(draft_length=8, chunk_size=4, num_layers=layers, num_heads=H, num_flow_steps=E, init_mode="delta")


def _ctx(seed=1, d=D, rows=8):
    return np.random.default_rng(seed).normal(size=(1, rows, d))


# ---------------------------------------------------------------- init_latents / integrate
def test_init_latents_closed_form_on_exact_integers():
    """delta: z0[k] = h[-1] + (k+1)(h[-1] - h[-2]); repeat_last: z0[k] = h[-1].  Integer-valued
    rows make every fp16 rounding exact, so the fp16 and fp32 paths must both hit the formula."""
    ctx = np.random.default_rng(3).integers(-8, 8, size=(2, 8, 16)).astype(np.float64)
    k = np.arange(1, 9).reshape(1, 8, 1)
    want = ctx[:, -1:] + k * (ctx[:, -1:] - ctx[:, -2:-1])
    for num in ("fp32", "fp16"):
        assert np.array_equal(oflow.init_latents(ctx, 8, num, "delta"), want)
    assert np.array_equal(oflow.init_latents(ctx, 8, "fp32", "repeat_last"), np.repeat(ctx[:, -1:], 8, 1))


def test_front_padding_repeats_the_oldest_row():
    h = np.arange(3 * 2).reshape(1, 3, 2).astype(float)
    got = oflow.front_pad_context(h, 5)
    assert np.array_equal(got[0], [[0, 1], [0, 1], [0, 1], [2, 3], [4, 5]])
    assert np.array_equal(oflow.front_pad_context(np.arange(16).reshape(1, 8, 2), 4)[0], np.arange(8, 16).reshape(4, 2))


@pytest.mark.parametrize("E", [1, 3, 8])
def test_zero_velocity_net_integrates_to_the_bias(E):
    """With out_proj W = 0 and bias c the velocity is c everywhere, so E Euler steps of size 1/E
    move z0 by exactly c (sum of dt = 1): pins the step count, dt and the update sign."""
    W = _weights()
    c = np.random.default_rng(5).normal(size=D)
    for p in oflow.expert_prefixes(2):
        W[p + "out_proj.weight"] = np.zeros((D, D))
        W[p + "out_proj.bias"] = c
    ctx = _ctx()
    z = oflow.predict_hidden(W, ctx, _cfg(E), numerics="fp32")
    z0 = oflow.init_latents(ctx, 8, "fp32")
    assert np.allclose(z, z0 + c, atol=1e-12)


def test_single_step_is_one_velocity_evaluation_at_tau_zero():
    W = _weights(seed=2)
    ctx = _ctx(seed=4)
    z0 = oflow.init_latents(ctx, 8, "fp32")
    z1 = oflow.predict_hidden(W, ctx, _cfg(1), numerics="fp32")
    vel = []
    for ci, p in enumerate(oflow.expert_prefixes(2)):
        kvs = [oflow.cross_kv(W, f"{p}blocks.{l}.", ctx, "fp32") for l in range(L)]
        tau = oflow.tau_embedding(W, p, 0.0, "fp32")
        vel.append(oflow.expert_velocity(W, p, z0[:, :4 * ci], z0[:, 4 * ci:4 * ci + 4], tau, 4 * ci, kvs, _cfg(1),
                                         "fp32"))
    assert np.allclose(z1, z0 + np.concatenate(vel, 1), atol=1e-12)


# ---------------------------------------------------------------- block invariants
def test_attention_matches_a_per_head_loop_and_torch():
    rng = np.random.default_rng(0)
    q, k, v = rng.normal(size=(1, 5, D)), rng.normal(size=(1, 7, D)), rng.normal(size=(1, 7, D))
    got = oflow.attention(q, k, v, H)
    hd = D // H
    want = np.zeros_like(got)
    for h in range(H):
        sl = slice(h * hd, (h + 1) * hd)
        s = q[0, :, sl] @ k[0, :, sl].T / np.sqrt(hd)
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        want[0, :, sl] = p @ v[0, :, sl]
    assert np.allclose(got, want, atol=1e-12)
    t = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).view(1, 5, H, hd).transpose(1, 2), torch.from_numpy(k).view(1, 7, H, hd).transpose(1, 2),
        torch.from_numpy(v).view(1, 7, H, hd).transpose(1, 2))
    assert np.allclose(got, t.transpose(1, 2).reshape(1, 5, D).numpy(), atol=1e-12)


def test_layer_norm_and_gelu_match_torch():
    x = np.random.default_rng(1).normal(size=(3, D)) * 3 + 1
    w, b = np.random.default_rng(2).normal(size=D), np.random.default_rng(3).normal(size=D)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x), (D,), torch.from_numpy(w), torch.from_numpy(b), 1e-5)
    assert np.allclose(oflow.layer_norm(x, w, b, "fp32"), ref.numpy(), atol=1e-12)
    assert np.allclose(oflow.gelu(x), torch.nn.functional.gelu(torch.from_numpy(x)).numpy(), atol=1e-12)


def test_self_attention_is_causal_in_the_block_stack():
    """Perturbing row j of a block's input changes no output row < j (triu(-inf, 1) mask)."""
    W = _weights(seed=6)
    bp = "extra_experts.0.blocks.0."
    ctx = _ctx(seed=7)
    kv = oflow.cross_kv(W, bp, ctx, "fp32")
    x = np.random.default_rng(8).normal(size=(1, 8, D))
    y = oflow.block_forward(W, bp, x, kv, oflow.causal_mask(8), H, "fp32")
    for j in (0, 3, 7):
        x2 = x.copy()
        x2[0, j] += 1.0
        y2 = oflow.block_forward(W, bp, x2, kv, oflow.causal_mask(8), H, "fp32")
        assert np.array_equal(y2[0, :j], y[0, :j])
        assert not np.allclose(y2[0, j], y[0, j])


def test_cross_attention_ignores_the_order_of_context_rows():
    """Context K/V carry no positional encoding: permuting context rows leaves the draft unchanged
    (the init_latents inputs, the last two rows, are kept in place)."""
    W = _weights(seed=9)
    ctx = _ctx(seed=10)
    perm = np.r_[np.random.default_rng(0).permutation(6), 6, 7]
    a = oflow.predict_hidden(W, ctx, _cfg(2), numerics="fp32")
    b = oflow.predict_hidden(W, ctx[:, perm], _cfg(2), numerics="fp32")
    assert np.allclose(a, b, atol=1e-10)


def test_chunk_zero_does_not_see_later_rows():
    """Chunk expert 0 reads only z rows 0..3: changing chunk expert 1's weights leaves them exactly."""
    W = _weights(seed=11)
    ctx = _ctx(seed=12)
    a = oflow.predict_hidden(W, ctx, _cfg(2), numerics="fp32")
    W2 = dict(W)
    W2["extra_experts.0.out_proj.bias"] = W["extra_experts.0.out_proj.bias"] + 1.0
    b = oflow.predict_hidden(W2, ctx, _cfg(2), numerics="fp32")
    assert np.array_equal(a[:, :4], b[:, :4])
    assert not np.allclose(a[:, 4:], b[:, 4:])


# ---------------------------------------------------------------- head / path residual / beam
def _path_weights(d=D, order=4, seed=0):
    rng = np.random.default_rng(seed)
    W = {}
    for j in range(order):
        W[f"path_head.offset_proj.{j}.weight"] = rng.normal(0, d ** -0.5, (d, d))
        W[f"path_head.offset_proj.{j}.bias"] = rng.normal(0, 0.1, d)
    W["path_head.norm.weight"] = 1 + rng.normal(0, 0.1, d)
    W["path_head.norm.bias"] = rng.normal(0, 0.1, d)
    W["path_head.mlp.0.weight"] = rng.normal(0, d ** -0.5, (2 * d, d))
    W["path_head.mlp.0.bias"] = rng.normal(0, 0.1, 2 * d)
    W["path_head.mlp.3.weight"] = rng.normal(0, (2 * d) ** -0.5, (d, 2 * d))
    W["path_head.mlp.3.bias"] = rng.normal(0, 0.1, d)
    return W


def test_path_trim_equals_masking_the_dead_offsets():
    """_nlive trimming is bit-exact: skipping offsets >= nlive equals feeding them as -1 (masked)."""
    W = _path_weights()
    emb = np.random.default_rng(1).normal(size=(50, D))
    lastp = np.random.default_rng(2).integers(0, 50, size=(6, 4))
    for nl in (1, 2, 3):
        masked = lastp.copy()
        masked[:, nl:] = -1
        for num in ("fp32", "fp16"):
            assert np.array_equal(ohead.path_residual(W, emb, lastp, nl, 4, num),
                                  ohead.path_residual(W, emb, masked, None, 4, num))


def test_path_residual_of_an_empty_path_is_the_mlp_of_the_norm_bias():
    """All offsets masked: h = 0, LN(0) = beta, so the residual is mlp(beta) for every row."""
    W = _path_weights(seed=3)
    emb = np.random.default_rng(4).normal(size=(10, D))
    got = ohead.path_residual(W, emb, np.full((3, 4), -1), None, 4, "fp32")
    beta = W["path_head.norm.bias"]
    u = beta @ W["path_head.mlp.0.weight"].T + W["path_head.mlp.0.bias"]
    want = oflow.gelu(u) @ W["path_head.mlp.3.weight"].T + W["path_head.mlp.3.bias"]
    assert np.allclose(got, np.broadcast_to(want, got.shape), atol=1e-12)


def test_head_identity_rows_and_shortlist_restriction():
    h = np.random.default_rng(0).normal(size=(3, 16))
    eye = np.eye(16)
    assert np.array_equal(ohead.head_logits(h, eye, "fp32"), h)
    full = np.random.default_rng(1).normal(size=(40, 16))
    sl = np.array([3, 7, 11, 39])
    assert np.array_equal(ohead.head_logits(h, full, "fp32")[:, sl], ohead.head_logits(h, full[sl], "fp32"))


def test_log_softmax_and_topk_tie_rule():
    x = np.array([[1.0, 3.0, 3.0, 2.0, -1.0]])
    assert np.allclose(np.exp(ohead.log_softmax(x)).sum(), 1.0)
    v, i = ohead.topk(x, 3)
    assert i.tolist() == [[1, 2, 3]]                       # equal values: lower index first
    assert np.allclose(ohead.margins(x, 2), [[0.0, 0.0]])


def test_width_one_beam_is_greedy():
    """W = 1: every depth takes the argmax of its own log-probs; the chain is those argmaxes."""
    rng = np.random.default_rng(5)
    V, d, K = 12, 8, 4
    Wh = rng.normal(size=(V, d))
    pred = rng.normal(size=(1, K + 1, d))
    score = lambda h, prev: h @ Wh.T + 0.1 * prev[:, None]
    resid = lambda lp, nl: np.zeros((lp.shape[0], d)) + 0.01 * lp[:, :1]
    got = obeam.beam_chains(pred, np.array([3]), np.arange(V), 1, K, 2, score, resid, numerics="fp32")
    prev, want = 3, []
    lastp = [3, -1]
    for s in range(1, K + 1):
        h = pred[0, s] + 0.01 * lastp[0]
        t = int(np.argmax(h @ Wh.T + 0.1 * prev))
        want.append(t)
        lastp = [t, lastp[0]]
        prev = t
    assert got[0].tolist() == want


# ---------------------------------------------------------------- gated delta net
def _gdn_inputs(N, Hh=2, Dk=8, Dv=6, seed=0):
    rng = np.random.default_rng(seed)
    return (rng.normal(size=(N, Hh, Dk)), rng.normal(size=(N, Hh, Dk)), rng.normal(size=(N, Hh, Dv)),
            np.log(1 / (1 + np.exp(-rng.normal(size=(N, Hh))))), rng.uniform(size=(N, Hh)),
            rng.normal(size=(Hh, Dk, Dv)) * 0.1)


def test_gdn_single_node_closed_form():
    q, k, v, g, beta, S0 = _gdn_inputs(1)
    out, st = ogdn.tree_gated_delta_scan(q, k, v, g, beta, [-1], S0)
    kn = k / (np.linalg.norm(k, axis=-1, keepdims=True) + 1e-6)
    qn = q / (np.linalg.norm(q, axis=-1, keepdims=True) + 1e-6) / np.sqrt(q.shape[-1])
    for h in range(2):
        Sd = np.exp(g[0, h]) * S0[h]
        S1 = Sd + np.outer(kn[0, h], (v[0, h] - Sd.T @ kn[0, h]) * beta[0, h])
        assert np.allclose(st[0, h], S1, atol=1e-12)
        assert np.allclose(out[0, h], S1.T @ qn[0, h], atol=1e-12)


def test_gdn_zero_beta_only_decays():
    q, k, v, g, beta, S0 = _gdn_inputs(4, seed=1)
    parent = [-1, 0, 1, 1]
    _, st = ogdn.tree_gated_delta_scan(q, k, v, g, np.zeros_like(beta), parent, S0)
    for n, path in enumerate(([0], [0, 1], [0, 1, 2], [0, 1, 3])):
        decay = np.exp(g[path].sum(0))
        assert np.allclose(st[n], decay[:, None, None] * S0, atol=1e-12)


def test_gdn_tree_equals_sequential_recurrence_on_every_path():
    q, k, v, g, beta, S0 = _gdn_inputs(9, seed=2)
    parent = [-1, 0, 0, 1, 1, 2, -1, 6, 3]
    out, _ = ogdn.tree_gated_delta_scan(q, k, v, g, beta, parent, S0)
    for n in range(9):
        seq = ogdn.sequential_path_output(q, k, v, g, beta, ogdn.path_to_root(parent, n), S0)
        assert np.allclose(out[n], seq, atol=1e-12)


def test_gdn_refuses_a_child_before_its_parent():
    q, k, v, g, beta, S0 = _gdn_inputs(3, seed=3)
    with pytest.raises(ValueError):
        ogdn.tree_gated_delta_scan(q, k, v, g, beta, [-1, 2, 0], S0)


def test_ancestor_chain():
    chain, depth = ogdn.build_ancestor_chain([-1, 0, 0, 1, 3], 3)
    assert depth.tolist() == [0, 1, 1, 2, 3]
    assert chain[4].tolist() == [4, 3, 1, 0]
    assert chain[2].tolist() == [2, 0, 0, 0]


def test_product_and_oracle_agree_on_the_reference_numerics(monkeypatch):
    """The flow's numerics switch (chain_flow_amd.flow.reference_numerics) and the oracle's copy of
    the reference's fused-kernel gate (oracle.flow.fused_kernel_shape) pick the same mode over a
    grid of shapes and batches, and follow the reference's CF_CUDA_BLOCK / CF_CUDA_BLOCK_BATCH."""
    from chain_flow_amd import _lib
    from chain_flow_amd.config import flownet
    from chain_flow_amd.flow import reference_numerics
    from conftest import oracle_numerics
    monkeypatch.delenv("CF_CUDA_BLOCK", raising=False)
    monkeypatch.delenv("CF_CUDA_BLOCK_BATCH", raising=False)
    seen = set()
    for d in (512, 640, 1024, 2560, 5120):
        for heads in (8, 16):
            for (kd, cs) in ((8, 4), (16, 8), (12, 4)):
                for batch in (1, 2):
                    cfg = flownet(d, layers=1, flow_steps=2, num_heads=heads, draft_length=kd, chunk_size=cs)
                    got = reference_numerics(cfg, batch)
                    want = oracle_numerics(cfg, batch)
                    assert (got == _lib.FLOW_FUSED) == (want == "fp16"), (d, heads, kd, cs, batch)
                    seen.add(want)
    assert seen == {"fp16", "fp16_modules"}
    cfg = flownet(640, layers=1, flow_steps=2)
    assert reference_numerics(cfg, 1) == _lib.FLOW_FUSED and reference_numerics(cfg, 2) == _lib.FLOW_MODULES
    monkeypatch.setenv("CF_CUDA_BLOCK_BATCH", "1")
    assert reference_numerics(cfg, 2) == _lib.FLOW_FUSED
    monkeypatch.setenv("CF_CUDA_BLOCK", "0")
    assert reference_numerics(cfg, 1) == _lib.FLOW_MODULES


def test_oracle_runs_in_float32_for_the_cpu_timing():
    """Given float32 weights and context, the oracle's fp32 path stays in float32 end to end (the
    arithmetic the CPU baseline times) and agrees with its float64 run to float32 precision."""
    import torch
    from chain_flow_amd.config import flownet
    from chain_flow_amd.weights import make_weights, param_specs, synthetic_context
    cfg = flownet(128, layers=2, flow_steps=3)
    names = {n for n in param_specs(cfg, 64) if not n.startswith(("lm_head", "embed_tokens", "markov"))}
    W = make_weights(cfg, 64, init="test", base_seed=2, names=names, dtype=torch.float32)
    W32 = {k: v.numpy() for k, v in W.items()}
    W64 = {k: v.double().numpy() for k, v in W.items()}
    ctx = synthetic_context(1, 8, 128, seed=3, dtype=torch.float32).numpy()
    ocfg = dict(draft_length=8, chunk_size=4, num_layers=2, num_heads=8, num_flow_steps=3, init_mode="delta")
    z32 = oflow.predict_hidden(W32, ctx, ocfg, numerics="fp32")
    z64 = oflow.predict_hidden(W64, ctx.astype(np.float64), ocfg, numerics="fp32")
    assert z32.dtype == np.float32 and z64.dtype == np.float64
    assert np.linalg.norm(z32 - z64) / np.linalg.norm(z64) < 1e-5
    lastp = np.array([[3, 5, -1, -1], [7, 1, 2, 9]])
    emb32 = np.random.default_rng(0).standard_normal((64, 128)).astype(np.float32)
    r32 = ohead.path_residual(W32, emb32, lastp, 2, 4, numerics="fp32")
    r64 = ohead.path_residual(W64, emb32.astype(np.float64), lastp, 2, 4, numerics="fp32")
    assert r32.dtype == np.float32
    assert np.linalg.norm(r32 - r64) / np.linalg.norm(r64) < 1e-5
