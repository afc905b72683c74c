"""Oracle: the proposer's draft beam searches (chain and tree).

Follows ``cf/vllm_plugin/flow_proposer.py`` (``cf/`` = ``src/chain_flow/``):

* ``:1187-1269``  ``_beam_chains`` with CF_FEEDBACK off and the one-pass head: depth 0 is seeded with
  the committed token (one live beam, cum = [0, -inf, ...]); depths 1..K score
  ``_head(h + res) + _bias(lastp[:, :, 0])``, take ``topk(W)`` per beam, then ``topk(W)`` over the
  W*W cumulative candidates; ``lastp`` is re-gathered by parent beam and shifted; the best beam is
  walked back through the backpointers.
* ``:1272-1332``  ``_beam_tree``: frontier of at most ``keep`` nodes, ``topb`` children per node,
  BFS-ordered nodes with parent index < child index; output = tokens || parents.
* ``:1030-1037``  ``_nlive`` (CF_PATH_TRIM on by default, ``cf/defaults.py:118``).
* ``:1142-1184``  the two-pass candidate head (``CF_TWOPASS_M``, default 8192 shared,
  ``cf/defaults.py:126-127``): ``_candidates`` keeps M shortlist columns per request from ONE score of
  the marginal hiddens of every depth (shared: by the best per-depth log-prob; else per depth by
  the raw logits), and ``_rescore`` renormalises each depth's scores over those M columns only
  (``log_softmax`` over M).  Candidate columns are kept in ascending order here (the reference
  keeps ``topk``'s value order); only exact ties can tell the two apart.

``score(h16 [N, d], prev_global [N]) -> fp16 logits [N, Vs]`` and
``residual(lastp [N, order], nlive) -> [N, d]`` are injected so this file holds only the search.
"""
from __future__ import annotations

import numpy as np

from oracle.head import log_softmax, topk
from oracle.flow import r16


def candidates(pred, lo, hi, score, M, shared=True, seed_res=None, seed_prev=None, numerics="fp16"):
    """``_candidates``: [B, hi-lo, M] shortlist-LOCAL columns (ascending) of the marginal hiddens
    ``pred[:, lo:hi]`` (+ the seed path's residual and markov bias when given)."""
    B, _, d = pred.shape
    n = hi - lo
    hm = pred[:, lo:hi]
    if seed_res is not None:
        hm = hm + np.asarray(seed_res)[:, None]
    prev = None if seed_prev is None else np.repeat(np.asarray(seed_prev), n)
    logits = score(r16(hm, numerics).reshape(B * n, d), prev)               # [B*n, Vs]
    Vs = logits.shape[-1]
    if shared:
        lp = log_softmax(logits).reshape(B, n, Vs).max(axis=1)              # [B, Vs]
        _, idx = topk(lp, M)
        return np.repeat(np.sort(idx, axis=-1)[:, None], n, axis=1)
    _, idx = topk(logits, M)
    return np.sort(idx, axis=-1).reshape(B, n, M)


def _rescored_topk(logits, cd_rows, k):
    """``_rescore`` + topk: log-softmax over the candidate columns only; ids back to shortlist-local."""
    sub = np.take_along_axis(logits, cd_rows, 1)
    lp = log_softmax(sub)
    cv, ii = topk(lp, k)
    return lp, cv, np.take_along_axis(cd_rows, ii, 1)


def beam_chains(pred, known0, sl, width, K, order, score, residual, numerics="fp16",
                path_trim=True, return_trace=False, twopass_m=0, shared=True, seed=False):
    """pred [B, Kd, d] marginal hiddens, known0 [B] committed token -> [B, min(K, Kd-1)] global ids."""
    B, Kd, d = pred.shape
    W = width
    lastp = np.full((B, W, order), -1, dtype=np.int64)
    lastp[:, :, 0] = np.asarray(known0)[:, None]
    cum = np.full((B, W), -np.inf)
    cum[:, 0] = 0.0
    steps = min(K + 1, Kd)
    toks, bps, trace = [], [], []
    cands = None
    if twopass_m and steps > 1:
        sr = sp = None
        if seed:
            sr = residual(lastp.reshape(B * W, order), 1 if path_trim else None).reshape(B, W, d)[:, 0]
            sp = lastp[:, 0, 0]
        cands = candidates(pred, 1, steps, score, twopass_m, shared, sr, sp, numerics)
    for step in range(1, steps):
        nlive = step if path_trim else None
        res = residual(lastp.reshape(B * W, order), nlive)                     # [B*W, d]
        h = r16(np.repeat(pred[:, step][:, None], W, axis=1).reshape(B * W, d) + res, numerics)
        logits = score(h, lastp[:, :, 0].reshape(-1))                          # [B*W, Vs]
        if cands is None:
            lp = log_softmax(logits)
            cv, ci = topk(lp, W)                                               # [B*W, W]
        else:
            cd = np.repeat(cands[:, step - 1], W, axis=0)                      # [B*W, M]
            lp, cv, ci = _rescored_topk(logits, cd, W)
        cand = (cum.reshape(B * W, 1) + cv).reshape(B, W * W)
        cum, flat = topk(cand, W)                                              # [B, W]
        src = flat // W
        newtok = np.asarray(sl)[np.take_along_axis(ci.reshape(B, W * W), flat, 1)]
        lastp = np.take_along_axis(lastp, src[:, :, None], 1)
        lastp = np.concatenate([newtok[:, :, None], lastp[:, :, :-1]], axis=-1)
        toks.append(newtok)
        bps.append(src)
        trace.append(dict(lp=lp, cv=cv, ci=ci, cand=cand, cum=cum.copy(), src=src, newtok=newtok))
    idx = np.argmax(cum, axis=-1)                                              # first maximum
    seq = [None] * len(toks)
    for step in range(len(toks) - 1, -1, -1):
        seq[step] = np.take_along_axis(toks[step], idx[:, None], 1)[:, 0]
        idx = np.take_along_axis(bps[step], idx[:, None], 1)[:, 0]
    out = np.stack(seq, axis=1) if seq else np.zeros((B, 0), dtype=np.int64)
    return (out, trace) if return_trace else out


def beam_tree(pred, known0, sl, keep, topb, depth, order, score, residual, numerics="fp16",
              path_trim=True, return_trace=False, twopass_m=0, shared=True, seed=False):
    """``_beam_tree``: -> [B, 2N] = N BFS-ordered draft tokens || their parent node indices
    (-1 = the committed root)."""
    B, Kd, d = pred.shape
    fr = 1
    lastp = np.full((B, fr, order), -1, dtype=np.int64)
    lastp[:, :, 0] = np.asarray(known0)[:, None]
    cum = np.zeros((B, fr))
    prev_ids = np.full((B, fr), -1, dtype=np.int64)
    toks, pars, trace = [], [], []
    base = 0
    nstep = min(depth, Kd - 1)
    cands = None
    if twopass_m:
        sr = sp = None
        if seed:
            sr = residual(lastp.reshape(B * fr, order), 1 if path_trim else None)
            sp = np.asarray(known0)
        cands = candidates(pred, 1, nstep + 1, score, twopass_m, shared, sr, sp, numerics)
    for step in range(1, nstep + 1):
        nlive = step if path_trim else None
        res = residual(lastp.reshape(B * fr, order), nlive)
        h = r16(np.repeat(pred[:, step][:, None], fr, axis=1).reshape(B * fr, d) + res, numerics)
        logits = score(h, lastp[:, :, 0].reshape(-1))
        if cands is None:
            lp = log_softmax(logits)
            cv, ci = topk(lp, topb)                                            # [B*fr, TB]
        else:
            cd = np.repeat(cands[:, step - 1], fr, axis=0)
            lp, cv, ci = _rescored_topk(logits, cd, topb)
        ci = ci.reshape(B, fr * topb)
        cand = (cum.reshape(B * fr, 1) + cv).reshape(B, fr * topb)
        k = min(keep, fr * topb)
        cum, flat = topk(cand, k)
        src = flat // topb
        newtok = np.asarray(sl)[np.take_along_axis(ci, flat, 1)]
        toks.append(newtok)
        pars.append(np.take_along_axis(prev_ids, src, 1))
        lastp = np.take_along_axis(lastp, src[:, :, None], 1)
        lastp = np.concatenate([newtok[:, :, None], lastp[:, :, :-1]], axis=-1)
        prev_ids = base + np.broadcast_to(np.arange(k), (B, k))
        base += k
        fr = k
        trace.append(dict(lp=lp, cv=cv, cand=cand, cum=cum.copy(), src=src, newtok=newtok))
    out = np.concatenate(toks + pars, axis=1)
    return (out, trace) if return_trace else out
