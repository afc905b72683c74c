"""Pins of the two-pass candidate head in the beam oracle (oracle/beam.py), CPU only.

* with M = every shortlist row the two-pass search IS the one-pass search (renormalising over all
  rows is the full softmax), for chains and trees, shared and per-depth candidate sets;
* the shared candidate set is the top-M of each column's best per-depth log-probability (brute
  force), the per-depth sets are the top-M of that depth's raw logits;
* with M < rows the candidates restrict the search: every drafted token is a candidate.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import beam as obeam
from oracle import head as ohead


def _setup(seed=0, Vs=60, d=16, r=8, K=5, B=2):
    rng = np.random.default_rng(seed)
    w_sl = rng.standard_normal((Vs, d)) * 0.8
    w1 = rng.standard_normal((Vs, r)) * 0.5
    w2_sl = rng.standard_normal((Vs, r)) * 0.5
    pred = rng.standard_normal((B, K + 1, d))
    sl = np.sort(rng.permutation(500)[:Vs])
    gl2loc = {int(g): i for i, g in enumerate(sl)}
    emb = rng.standard_normal((500, d)) * 0.3

    def score(h, prev):
        if prev is None:
            return ohead.head_logits(h, w_sl)
        return ohead.head_with_bias(h, w_sl, w1[[gl2loc.get(int(p), 0) for p in prev]], w2_sl,
                                    np.arange(len(prev)))

    def residual(lastp, nlive):
        x = np.where(lastp >= 0, lastp, 0)
        return ohead.r16(emb[x[:, 0]] * 0.1, "fp16")

    known0 = sl[[3, 7][:B]]
    return pred, sl, score, residual, known0, Vs


@pytest.mark.parametrize("shared", [True, False])
def test_all_rows_is_one_pass(shared):
    pred, sl, score, residual, known0, Vs = _setup()
    one = obeam.beam_chains(pred, known0, sl, 4, 5, 4, score, residual)
    two = obeam.beam_chains(pred, known0, sl, 4, 5, 4, score, residual, twopass_m=Vs, shared=shared)
    assert np.array_equal(one, two)
    t1 = obeam.beam_tree(pred, known0, sl, 4, 3, 4, 4, score, residual)
    t2 = obeam.beam_tree(pred, known0, sl, 4, 3, 4, 4, score, residual, twopass_m=Vs, shared=shared)
    assert np.array_equal(t1, t2)


def test_candidate_sets_brute_force():
    pred, sl, score, residual, known0, Vs = _setup(1)
    M, B, n = 17, pred.shape[0], 5
    got = obeam.candidates(pred, 1, 6, score, M, shared=True)
    logits = score(ohead.r16(pred[:, 1:6], "fp16").reshape(B * n, -1), None).reshape(B, n, Vs)
    for b in range(B):
        best = np.max([ohead.log_softmax(logits[b, d]) for d in range(n)], axis=0)
        want = sorted(np.argsort(-best, kind="stable")[:M])
        for d in range(n):
            assert list(got[b, d]) == want
    per = obeam.candidates(pred, 1, 6, score, M, shared=False)
    for b in range(B):
        for d in range(n):
            assert list(per[b, d]) == sorted(np.argsort(-logits[b, d], kind="stable")[:M])


@pytest.mark.parametrize("seed_cond", [False, True])
def test_small_m_drafts_only_candidates(seed_cond):
    pred, sl, score, residual, known0, Vs = _setup(2)
    M = 9
    cands = obeam.candidates(pred, 1, 6, score, M, shared=True)
    out = obeam.beam_chains(pred, known0, sl, 4, 5, 4, score, residual, twopass_m=M, seed=seed_cond)
    if not seed_cond:
        for b in range(out.shape[0]):
            assert set(out[b].tolist()) <= set(sl[cands[b, 0]].tolist())
    tree = obeam.beam_tree(pred, known0, sl, 4, 3, 4, 4, score, residual, twopass_m=M, seed=seed_cond)
    assert tree.shape[1] % 2 == 0
