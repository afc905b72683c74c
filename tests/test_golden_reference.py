"""The oracle against golden vectors written by the reference implementation itself
(tests/golden/make_golden.py; float32 reference vs the oracle's float64 math with fp32 numerics).
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import rel_err
from chain_flow_amd.config import TreeFlowConfig
from chain_flow_amd.weights import make_weights
from oracle import beam as obeam
from oracle import flow as oflow
from oracle import gdn as ogdn
from oracle import head as ohead

G = np.load(Path(__file__).parent / "golden" / "reference_tiny.npz")
D, VOCAB, LAYERS, RANK, SEED = 64, 96, 2, 16, 3
TOL = 1e-5


def _cfg(E):
    return TreeFlowConfig(context_size=8, draft_length=8, chunk_size=4, expert_dim=D, num_heads=8, ffn_multiplier=6,
                          num_drafter_layers=LAYERS, num_flow_steps=E, init_mode="delta", markov_rank=RANK,
                          path_order=4, path_ffn_multiplier=2)


def _weights(E):
    W = make_weights(_cfg(E), VOCAB, init="test", dtype=torch.float32, base_seed=SEED)
    h = hashlib.sha256()
    for k in sorted(W):
        h.update(k.encode())
        h.update(W[k].float().contiguous().numpy().tobytes())
    assert h.digest() == G[f"weights_sha_E{E}"].tobytes(), "weight generator drifted from the golden run"
    return {k: v.double().numpy() for k, v in W.items()}


def _ocfg(E):
    return dict(draft_length=8, chunk_size=4, num_layers=LAYERS, num_heads=8, num_flow_steps=E, init_mode="delta")


@pytest.mark.parametrize("E", [1, 3])
def test_init_latents_and_predict_hidden(E):
    W = _weights(E)
    ctx = G["ctx"].astype(np.float64)
    z0 = oflow.init_latents(ctx, 8, "fp32")
    assert rel_err(z0, G[f"z0_E{E}"]) < 1e-6
    pred = oflow.predict_hidden(W, ctx, _ocfg(E), numerics="fp32")
    assert rel_err(pred, G[f"pred_E{E}"]) < TOL


def test_chunk_velocities():
    W = _weights(3)
    ctx = G["ctx"].astype(np.float64)
    z0 = oflow.init_latents(ctx, 8, "fp32")
    kvs = [[oflow.cross_kv(W, f"{p}blocks.{l}.", ctx, "fp32") for l in range(LAYERS)]
           for p in oflow.expert_prefixes(2)]
    vels = []
    for ci, p in enumerate(oflow.expert_prefixes(2)):
        tau_add = oflow.tau_embedding(W, p, 0.25, "fp32")
        vels.append(oflow.expert_velocity(W, p, z0[:, :4 * ci], z0[:, 4 * ci:4 * ci + 4], tau_add, 4 * ci,
                                          kvs[ci], _ocfg(3), "fp32"))
    assert rel_err(np.concatenate(vels, 1), G["vel_tau025"]) < TOL


@pytest.mark.parametrize("nl", [1, 2, 4])
@pytest.mark.parametrize("form", ["unfused", "fused"])
def test_path_residual(nl, form):
    W = _weights(3)
    res = ohead.path_residual(W, W["embed_tokens.weight"], G["lastp"], nl, 4, numerics="fp32")
    assert rel_err(res, G[f"res_{form}_n{nl}"]) < TOL


def _oracle_tree(W, pred, keep, topb, depth, known0=17):
    sl = np.arange(VOCAB)
    score = lambda h, prev: ohead.head_with_bias(h, W["lm_head.weight"], W["markov.w1.weight"],
                                                 W["markov.w2.weight"], prev, numerics="fp32")
    resid = lambda lp, nlive: ohead.path_residual(W, W["embed_tokens.weight"], lp, nlive, 4, numerics="fp32")
    return obeam.beam_tree(pred[None], np.array([known0]), sl, keep, topb, depth, 4, score, resid,
                           numerics="fp32", return_trace=True)


@pytest.mark.parametrize("keep,topb,depth", [(4, 8, 5), (4, 4, 5), (1, 1, 5), (3, 2, 4)])
def test_beam_tree_matches_reference_search(keep, topb, depth):
    """build_tree_fast with a forced root is the proposer's _beam_tree search (plus the root node)."""
    W = _weights(3)
    pred = G["tree_pred"].astype(np.float64)
    key = f"tree_k{keep}_b{topb}_d{depth}"
    tok, par, cum = G[key + "_tokens"], G[key + "_parents"], G[key + "_cum"]
    out, trace = _oracle_tree(W, pred, keep, topb, depth)
    N = out.shape[1] // 2
    assert N == len(tok) - 1
    assert np.array_equal(out[0, :N], tok[1:])
    assert np.array_equal(out[0, N:], par[1:] - 1)
    # cumulative log-probs: the reference adds the root's own log-prob to every node
    got_cum = np.concatenate([t["cum"][0] for t in trace])
    assert np.allclose(got_cum, cum[1:] - cum[0], atol=1e-4)


def test_beam_chain_is_the_best_path_of_the_width_w_search():
    """_beam_chains with width W keeps exactly the W best candidates per depth: its backtracked chain
    is the path to the best leaf of the reference's keep=W, top_b=W search."""
    W = _weights(3)
    pred = G["tree_pred"].astype(np.float64)
    tok, par, cum = G["tree_k4_b4_d5_tokens"], G["tree_k4_b4_d5_parents"], G["tree_k4_b4_d5_cum"]
    leaves = np.arange(len(tok) - 4, len(tok))
    n = int(leaves[np.argmax(cum[leaves])])
    path = []
    while par[n] != -1:
        path.append(int(tok[n]))
        n = int(par[n])
    path = path[::-1]
    score = lambda h, prev: ohead.head_with_bias(h, W["lm_head.weight"], W["markov.w1.weight"],
                                                 W["markov.w2.weight"], prev, numerics="fp32")
    resid = lambda lp, nlive: ohead.path_residual(W, W["embed_tokens.weight"], lp, nlive, 4, numerics="fp32")
    chain = obeam.beam_chains(pred[None], np.array([17]), np.arange(VOCAB), 4, 5, 4, score, resid, numerics="fp32")
    assert chain[0].tolist() == path


def test_tree_gdn_matches_reference():
    f = lambda n: G["gdn_" + n].astype(np.float64)
    out, states = ogdn.tree_gated_delta_scan(f("q"), f("k"), f("v"), f("g"), f("beta"), G["gdn_parent"], f("S0"))
    assert rel_err(out, f("out")) < TOL
    assert rel_err(states, f("states")) < TOL
    assert rel_err(out, G["gdn_seq"]) < TOL


# ---- fp16: the reference's own drafter cast to fp16 and run on the CPU (tests/golden/make_golden_fp16.py),
# i.e. torch's fp16 modules -- the numerics the reference uses at every width its fused kernel does not take.
G16 = np.load(Path(__file__).parent / "golden" / "reference_tiny_fp16.npz")


def _weights16(E):
    assert G16[f"weights_sha_E{E}"].tobytes() == G[f"weights_sha_E{E}"].tobytes()
    return {k: v.astype(np.float16).astype(np.float64) for k, v in _weights(E).items()}


@pytest.mark.parametrize("E", [1, 3])
def test_fp16_modules_numerics_pinned_by_the_reference_fp16_drafter(E):
    """The oracle's "fp16_modules" mode (fp16 residual x = fp16(x + fp16(sublayer)), GELU of the
    rounded up-projection) agrees with the reference's fp16 predict_hidden to ~1.1e-4 norm-relative:
    one-ulp flips from torch's fp16 GEMM accumulation order.  The fused-kernel mode (fp32 residual)
    and fp32 math are measurably further (1.5-2.3e-4 and 3.7-4.5e-4), so a dropped residual or
    GELU rounding fails here."""
    W = _weights16(E)
    ctx = G16["ctx16"].astype(np.float64)
    err = {num: rel_err(oflow.predict_hidden(W, ctx, _ocfg(E), numerics=num), G16[f"pred16_E{E}"])
           for num in ("fp16_modules", "fp16", "fp32")}
    assert err["fp16_modules"] < 1.3e-4, err
    assert err["fp16_modules"] < err["fp16"] and 2.5 * err["fp16_modules"] < err["fp32"], err


def test_fp16_modules_velocity_pinned_by_the_reference():
    W = _weights16(3)
    ctx = G16["ctx16"].astype(np.float64)
    err = {}
    for num in ("fp16_modules", "fp16", "fp32"):
        z0 = oflow.init_latents(ctx, 8, "fp16")
        kvs = [[oflow.cross_kv(W, f"{p}blocks.{l}.", ctx, num) for l in range(LAYERS)]
               for p in oflow.expert_prefixes(2)]
        vels = []
        for ci, p in enumerate(oflow.expert_prefixes(2)):
            tau_add = oflow.tau_embedding(W, p, 0.25, num)
            vels.append(oflow.expert_velocity(W, p, z0[:, :4 * ci], z0[:, 4 * ci:4 * ci + 4], tau_add, 4 * ci,
                                              kvs[ci], _ocfg(3), num))
        err[num] = rel_err(np.concatenate(vels, 1), G16["vel16_tau025"])
    assert err["fp16_modules"] < 6.5e-4, err
    assert err["fp16_modules"] < min(err["fp16"], err["fp32"]), err


@pytest.mark.parametrize("nl", [1, 2, 4])
def test_fp16_path_residual_pinned_by_the_reference(nl):
    """The fused path residual's fp16 rounding points (one rounding per offset projection, the
    masked sum, LayerNorm, the MLP's up-projection and GELU) reproduce the reference's fp16 output to
    2e-5 (bit for bit at 2 and 4 live offsets); fp32 math is 4.5e-4 away."""
    W = _weights16(3)
    got = ohead.path_residual(W, W["embed_tokens.weight"], G16["lastp"], nl, 4, numerics="fp16")
    assert rel_err(got, G16[f"res16_fused_n{nl}"]) < 2e-5
    got32 = ohead.path_residual(W, W["embed_tokens.weight"], G16["lastp"], nl, 4, numerics="fp32")
    assert rel_err(got32, G16[f"res16_fused_n{nl}"]) > 2e-4
