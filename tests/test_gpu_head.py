"""GPU parity of the draft head: shortlisted lm_head + markov bias, top-k, path residual, beam steps.

Contracts: fp16 logits equal to the oracle's within one fp16 ulp; top-k ids bit-exact on identical
logits (ties to the lower index) and log-prob values within 1e-5; path residual within 2e-3
norm-relative; beam steps bit-exact on identical inputs; end-to-end draft ids equal to the oracle's
wherever the oracle's decision margin exceeds 1e-3.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_err, to64
from chain_flow_amd.config import flownet
from chain_flow_amd.head import PathHead, ShortlistHead, row_topk
from chain_flow_amd.weights import make_weights, param_specs
from oracle import beam as obeam
from oracle import head as ohead

MARGIN = 1e-3


def _head_weights(d, V, seed=0, scale=8.0):
    cfg = flownet(d, layers=1, flow_steps=1)
    names = {n for n in param_specs(cfg, V) if n.startswith(("markov.", "path_head.", "lm_head", "embed_tokens"))}
    W = make_weights(cfg, V, init="test", base_seed=seed, names=names)
    W["lm_head.weight"] = (W["lm_head.weight"].float() * scale).half()
    return cfg, W


def _shortlist(V, n, seed=2):
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(V, generator=g)[:n].sort().values.to(torch.int32)


def _ulp16(x):
    x = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(x, 2.0 ** -14)))
    return 2.0 ** (e - 10)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 4, 8])
def test_head_logits_match_oracle(cuda, M):
    d, V, n = 512, 4096, 1024
    cfg, W = _head_weights(d, V)
    sl = _shortlist(V, n)
    g = torch.Generator().manual_seed(7)
    h = torch.randn(M, d, generator=g).half()
    prev = torch.randint(0, V, (M,), generator=g, dtype=torch.int32)
    head = ShortlistHead(W["lm_head.weight"].to(cuda), sl.to(cuda), W["markov.w1.weight"].to(cuda),
                         W["markov.w2.weight"].to(cuda))
    got = to64(head.logits(h.to(cuda), prev.to(cuda)))
    sl64 = sl.long().numpy()
    ref = ohead.head_with_bias(to64(h), to64(W["lm_head.weight"])[sl64], to64(W["markov.w1.weight"]),
                               to64(W["markov.w2.weight"])[sl64], prev.long().numpy())
    diff = np.abs(got - ref)
    assert (diff <= 2 * _ulp16(ref) + 1e-12).all(), diff.max()
    assert (diff > 0).mean() < 0.02


@pytest.mark.gpu
def test_full_head_restricted_equals_shortlist_head(cuda):
    """A full head restricted to the shortlist columns is the shortlist head (same rows, same sums)."""
    d, V, n = 512, 4096, 1024
    cfg, W = _head_weights(d, V)
    sl = _shortlist(V, n)
    h = torch.randn(4, d, generator=torch.Generator().manual_seed(3)).half().to(cuda)
    full = ShortlistHead(W["lm_head.weight"].to(cuda), None).logits(h)
    short = ShortlistHead(W["lm_head.weight"].to(cuda), sl.to(cuda)).logits(h)
    assert torch.equal(full[:, sl.long().to(cuda)], short)


@pytest.mark.gpu
def test_identity_rows_give_coordinates(cuda):
    """Head rows equal to unit vectors make the logits equal to h's coordinates."""
    d = 512
    lm = torch.zeros(d, d, dtype=torch.float16)
    lm[torch.arange(d), torch.arange(d)] = 1.0
    sl = torch.arange(0, d, 3, dtype=torch.int32)
    h = torch.randn(2, d, generator=torch.Generator().manual_seed(4)).half()
    got = ShortlistHead(lm.to(cuda), sl.to(cuda)).logits(h.to(cuda)).cpu()
    assert torch.equal(got, h[:, sl.long()])


@pytest.mark.gpu
@pytest.mark.parametrize("k", [1, 4, 8, 16])
def test_row_topk_bit_exact(cuda, k):
    g = torch.Generator().manual_seed(11)
    M, n = 6, 62642
    logits = (torch.randn(M, n, generator=g) * 3).half()
    logits[:, 100:140] = logits[:, 100:101]           # plant ties: equal values, lower index first
    logits[2, :] = 1.0                                # a row made only of ties
    vals, ids, lse = row_topk(logits.to(cuda), k)
    L = to64(logits)
    ref_lp = ohead.log_softmax(L)
    rv, ri = ohead.topk(ref_lp, k)
    assert np.array_equal(ids.cpu().numpy(), ri)
    assert np.allclose(vals.cpu().numpy(), rv, atol=1e-5, rtol=0)
    m = L.max(-1)
    assert np.allclose(lse.cpu().numpy(), m + np.log(np.exp(L - m[:, None]).sum(-1)), atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("nlive,M", [(0, 4), (1, 4), (2, 4), (3, 4), (4, 4), (4, 16), (2, 13)])
def test_path_residual_matches_oracle(cuda, nlive, M):
    """Offsets of the live ancestors + masked sum, LayerNorm, the 2x MLP, plus the marginal hidden;
    nlive = 0 (no offset live) is checked against every ancestor masked, the oracle's form of an
    empty path; 16 rows fill one launch sequence, 13 leave a ragged last 16-row tile."""
    d, V = 512, 4096
    cfg, W = _head_weights(d, V)
    ph = PathHead({k: v.to(cuda) for k, v in W.items()}, W["embed_tokens.weight"].to(cuda), cfg.path_order,
                  cfg.path_ffn_multiplier, cuda)
    g = torch.Generator().manual_seed(5 + M)
    lastp = torch.randint(0, V, (M, cfg.path_order), generator=g, dtype=torch.int32)
    lastp[1, 2:] = -1
    lastp[3, 1:] = -1
    lastp[M - 1, :] = -1                                   # a row with no ancestor at all
    pred = torch.randn(d, generator=g).half()
    got = to64(ph.hidden(lastp.to(cuda), nlive, pred.to(cuda)))
    W64 = {k: to64(v) for k, v in W.items() if k.startswith("path_head.")}
    lp_ref = lastp.long().numpy() if nlive > 0 else np.full((M, cfg.path_order), -1)
    res = ohead.path_residual(W64, to64(W["embed_tokens.weight"]), lp_ref, nlive if nlive > 0 else None,
                              cfg.path_order)
    ref = ohead.r16(to64(pred)[None] + res, "fp16")
    assert rel_err(got, ref) < 2e-3


def _np_chain_step(vals, ids, cum, lastp, sl, W):
    B = cum.shape[0]
    cand = (cum.reshape(B * W, 1) + vals).reshape(B, W * W)
    ncum, flat = ohead.topk(cand, W)
    src = flat // W
    newtok = sl[np.take_along_axis(ids.reshape(B, W * W), flat, 1)]
    lp = np.take_along_axis(lastp, src[:, :, None], 1)
    lp = np.concatenate([newtok[:, :, None], lp[:, :, :-1]], -1)
    return ncum, lp, newtok, src


@pytest.mark.gpu
def test_beam_chain_step_bit_exact(cuda):
    from chain_flow_amd import _lib
    rng = np.random.default_rng(0)
    B, W, order, n = 3, 4, 4, 500
    sl = np.sort(rng.choice(10000, n, replace=False)).astype(np.int32)
    vals = np.round(rng.normal(size=(B * W, W)) * 4, 1).astype(np.float32)   # coarse -> ties
    ids = rng.integers(0, n, size=(B * W, W)).astype(np.int32)
    cum = np.round(rng.normal(size=(B, W)), 1).astype(np.float32)
    cum[1, 1:] = -np.inf
    lastp = rng.integers(-1, 10000, size=(B, W, order)).astype(np.int32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    # every device buffer stays referenced until the asynchronous kernel has run
    vals_d, ids_d, sl_d, cum_d, lastp_d = t(vals), t(ids), t(sl), t(cum), t(lastp)
    toks = torch.empty(B, W, dtype=torch.int32, device=cuda)
    bps = torch.empty_like(toks)
    _lib.check(_lib.lib().cfh_beam_chain_step(vals_d.data_ptr(), ids_d.data_ptr(), cum_d.data_ptr(),
                                              lastp_d.data_ptr(), sl_d.data_ptr(), toks.data_ptr(), bps.data_ptr(),
                                              B, W, order, _lib.stream_handle()), "step")
    torch.cuda.synchronize()
    ncum, nlp, ntok, nsrc = _np_chain_step(vals, ids, cum, lastp, sl, W)   # float32, as on the device
    assert np.array_equal(cum_d.cpu().numpy(), ncum.astype(np.float32))
    assert np.array_equal(lastp_d.cpu().numpy(), nlp)
    assert np.array_equal(toks.cpu().numpy(), ntok)
    assert np.array_equal(bps.cpu().numpy(), nsrc)


def _near_tie(trace, W):
    """True when any beam decision of the oracle (per-beam top-W of the log-probs, top-W over the
    W*W candidates, or the final best-beam arg-max) had a margin <= MARGIN: the backtracked chain
    depends on every one of them."""
    for tr in trace:
        if (ohead.margins(tr["lp"], W) <= MARGIN).any():
            return True
        if (ohead.margins(tr["cand"], W) <= MARGIN).any():
            return True
    if (ohead.margins(trace[-1]["cum"], 1) <= MARGIN).any():
        return True
    return False


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_beam_chains_match_oracle(cuda, seed):
    from chain_flow_amd.drafter import Drafter
    d, V, n, K, Wd = 512, 4096, 1024, 5, 4
    cfg = flownet(d, layers=1, flow_steps=1)
    W = make_weights(cfg, V, init="test", base_seed=seed)
    W["lm_head.weight"] = (W["lm_head.weight"].float() * 8).half()
    sl = _shortlist(V, n, seed=seed + 2)
    dr = Drafter(cfg, {k: v.to(cuda) for k, v in W.items()}, sl.to(cuda), device=cuda)
    g = torch.Generator().manual_seed(100 + seed)
    pred = torch.randn(1, cfg.draft_length, d, generator=g).half()
    known0 = torch.tensor([int(sl[7])])
    got = dr.beam_chains(None, known0.to(cuda), K, Wd, pred=pred.to(cuda)).cpu().numpy()[0]
    W64 = {k: to64(v) for k, v in W.items()}
    sl64 = sl.long().numpy()
    score = lambda h, prev: ohead.head_with_bias(h, W64["lm_head.weight"][sl64], W64["markov.w1.weight"],
                                                 W64["markov.w2.weight"][sl64], prev)
    resid = lambda lp, nl: ohead.path_residual(W64, W64["embed_tokens.weight"], lp, nl, cfg.path_order)
    ref, trace = obeam.beam_chains(to64(pred), known0.numpy(), sl64, Wd, K, cfg.path_order, score, resid,
                                   return_trace=True)
    ref = ref[0]
    print(f"[beam chains seed={seed}] gpu {got.tolist()} oracle {ref.tolist()}", flush=True)
    if not np.array_equal(got, ref):
        assert _near_tie(trace, Wd), (got, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("M,k,markov,n,V", [(1, 4, True, 5003, 9000), (4, 4, True, 5003, 9000),
                                             (4, 8, False, 5003, 9000), (8, 16, True, 5003, 9000),
                                             (2, 16, True, 65000, 70000), (4, 8, False, 80003, 90000)])
def test_fused_head_topk_equals_logits_then_topk(cuda, M, k, markov, n, V):
    """The fused head (per-block candidates + merge) returns exactly what the unfused pair
    (fp16 logits, then per-row log-softmax top-k) returns on the same inputs.  n not a multiple
    of the 128-column block; 65,000 columns at k=16 fill the wave merge's 64 KB of LDS, 80,003
    columns (626 blocks) take the block-wide merge."""
    d = 512
    cfg, W = _head_weights(d, V)
    sl = _shortlist(V, n)
    g = torch.Generator().manual_seed(17)
    h = torch.randn(M, d, generator=g).half().to(cuda)
    prev = torch.randint(0, V, (M,), generator=g, dtype=torch.int32).to(cuda)
    head = ShortlistHead(W["lm_head.weight"].to(cuda), sl.to(cuda),
                         W["markov.w1.weight"].to(cuda) if markov else None,
                         W["markov.w2.weight"].to(cuda) if markov else None)
    logits = torch.empty(M, n, dtype=torch.float16, device=cuda)
    print(f"[fused head] M={M} k={k} markov={markov} n={n}", flush=True)
    vals, ids, lse = head.topk(h, k, prev=prev if markov else None, logits=logits)
    rv, ri, rl = row_topk(logits, k)
    torch.cuda.synchronize()
    assert torch.equal(ids, ri)
    assert torch.allclose(vals, rv, atol=2e-6, rtol=0)
    assert torch.allclose(lse, rl, atol=2e-6, rtol=0)
    L = to64(logits)
    ov, oi = ohead.topk(ohead.log_softmax(L), k)
    assert np.array_equal(ids.cpu().numpy(), oi)
    assert np.allclose(vals.cpu().numpy(), ov, atol=1e-5, rtol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("M,k,markov,n", [(1, 4, True, 5003), (4, 4, True, 62642 // 8), (8, 16, False, 1000)])
def test_packed_head_equals_in_place(cuda, M, k, markov, n):
    """The packed shortlist image (rows gathered once into the fragment order) gives bit-identical
    logits and the same top-k as the in-place row gather; n not a multiple of 16 exercises the
    padded last tile."""
    d, V = 512, 9000
    cfg, W = _head_weights(d, V)
    sl = _shortlist(V, n)
    g = torch.Generator().manual_seed(29)
    h = torch.randn(M, d, generator=g).half().to(cuda)
    prev = torch.randint(0, V, (M,), generator=g, dtype=torch.int32).to(cuda)
    args = (W["lm_head.weight"].to(cuda), sl.to(cuda), W["markov.w1.weight"].to(cuda) if markov else None,
            W["markov.w2.weight"].to(cuda) if markov else None)
    packed, in_place = ShortlistHead(*args, packed=True), ShortlistHead(*args, packed=False)
    assert packed.image is not None and in_place.image is None
    out = []
    for head in (packed, in_place):
        logits = torch.empty(M, n, dtype=torch.float16, device=cuda)
        vals, ids, lse = head.topk(h, k, prev=prev if markov else None, logits=logits)
        out.append((logits, vals, ids, lse))
    torch.cuda.synchronize()
    print(f"[packed head M={M} k={k} markov={markov} n={n}]", flush=True)
    for a, b in zip(out[0], out[1]):
        assert torch.equal(a, b)


@pytest.mark.gpu
def test_packed_head_full_width_matches_oracle(cuda):
    """The benchmark's head shape: 62,642 shortlist rows x d = 5120 with the rank-256 markov bias,
    4 beam rows, top-8, through the packed image.  Logits within 2 fp16 ulp of the oracle; top-8
    ids equal to the oracle's wherever the oracle's adjacent margins exceed 1e-3."""
    d, V, n, M, k = 5120, 70000, 62642, 4, 8
    cfg = flownet(d, layers=1, flow_steps=1)
    names = {x for x in param_specs(cfg, V) if x.startswith(("markov.", "lm_head"))}
    W = make_weights(cfg, V, init="test", base_seed=3, names=names)
    W["lm_head.weight"] = (W["lm_head.weight"].float() * 8.0).half()
    sl = _shortlist(V, n, seed=5)
    g = torch.Generator().manual_seed(13)
    h = torch.randn(M, d, generator=g).half()
    prev = torch.randint(0, V, (M,), generator=g, dtype=torch.int32)
    print(f"[head parity] n={n} d={d} M={M} k={k} (full width, packed)", flush=True)
    head = ShortlistHead(W["lm_head.weight"].to(cuda), sl.to(cuda), W["markov.w1.weight"].to(cuda),
                         W["markov.w2.weight"].to(cuda))
    logits = torch.empty(M, n, dtype=torch.float16, device=cuda)
    vals, ids, lse = head.topk(h.to(cuda), k, prev=prev.to(cuda), logits=logits)
    torch.cuda.synchronize()
    got = to64(logits)
    gid = ids.cpu().numpy()
    del head, logits
    sl64 = sl.long().numpy()
    hw = ohead.head_logits(to64(h), to64(W["lm_head.weight"][sl64]))
    mb = ohead.markov_bias(to64(W["markov.w1.weight"]), to64(W["markov.w2.weight"][sl64]), prev.long().numpy())
    ref = ohead.r16(hw + mb, "fp16")
    diff = np.abs(got - ref)
    print(f"  max logit diff {diff.max():.3e}, fraction differing {(diff > 0).mean():.4f}", flush=True)
    # each fp16 rounding point (h.W, A.W2 and their sum) may land one ulp apart when the fp32
    # accumulation order differs: the bound is one ulp of each, at its own magnitude
    assert (diff <= _ulp16(hw) + _ulp16(mb) + _ulp16(ref) + 1e-12).all()
    assert (diff > 0).mean() < 0.01
    order = np.argsort(-ref, axis=1, kind="stable")[:, :k + 1]
    for m in range(M):
        rv = ref[m, order[m]]
        for r in range(k):
            lo = rv[r] - rv[r + 1]
            hi = np.inf if r == 0 else rv[r - 1] - rv[r]
            if min(lo, hi) > MARGIN:
                assert gid[m, r] == order[m, r], (m, r)


@pytest.mark.gpu
@pytest.mark.parametrize("B,W,img", [(1, 4, False), (2, 4, False), (1, 2, False), (2, 1, False), (1, 4, True),
                                     (2, 3, True)])
def test_merged_topk_and_beam_step_equal_the_two_calls(cuda, B, W, img):
    """cfh_head_topk_packed_beam_chain (the candidate merge and the chain step in one launch) against
    cfh_head_topk_packed followed by cfh_beam_chain_step, bit for bit, over four depths of evolving
    beams: vals / ids / lse, cum, lastp, toks and bps; over the head's own packed image (ids mapped
    through the shortlist) and over a packed image of 1,000 candidate rows (ids mapped through them)."""
    from chain_flow_amd import _lib
    d, V, n, order = 512, 4096, 3000, 4
    cfg, W_ = _head_weights(d, V, seed=3)
    sl = _shortlist(V, n, seed=5).to(cuda)
    head = ShortlistHead(W_["lm_head.weight"].to(cuda), sl, W_["markov.w1.weight"].to(cuda),
                         W_["markov.w2.weight"].to(cuda))
    g = torch.Generator().manual_seed(11 + B * W)
    if img:
        cand = sl[torch.randperm(n, generator=g)[:1000].sort().values.to(cuda)].contiguous()
        image, nimg, smap = head.pack_rows(cand), 1000, cand
    else:
        image, nimg, smap = None, n, sl
    L = _lib.lib()
    st = _lib.stream_handle()
    states = []
    for fused in (False, True):
        lastp = torch.full((B, W, order), -1, dtype=torch.int32, device=cuda)
        lastp[:, :, 0] = sl[torch.arange(B) * 7 % n].view(B, 1).to(torch.int32)
        cum = torch.full((B, W), float("-inf"), device=cuda)
        cum[:, 0] = 0.0
        out = []
        for depth in range(4):
            h = torch.randn(B * W, d, generator=torch.Generator().manual_seed(100 + depth)).half().to(cuda)
            toks = torch.empty(B, W, dtype=torch.int32, device=cuda)
            bps = torch.empty(B, W, dtype=torch.int32, device=cuda)
            if fused:
                vals, ids, lse = head.topk_beam_chain(h, image, nimg, lastp.view(-1), order, cum, lastp, smap,
                                                      toks, bps, B, W, order)
            else:
                if img:
                    vals, ids, lse = head.topk_image(h, W, image, nimg, prev=lastp.view(-1), prev_stride=order)
                else:
                    vals, ids, lse = head.topk(h, W, prev=lastp.view(-1), prev_stride=order)
                _lib.check(L.cfh_beam_chain_step(vals.data_ptr(), ids.data_ptr(), cum.data_ptr(), lastp.data_ptr(),
                                                 smap.data_ptr(), toks.data_ptr(), bps.data_ptr(), B, W, order, st),
                           "cfh_beam_chain_step")
            torch.cuda.synchronize()
            out.append([t.clone().cpu() for t in (vals, ids, lse, cum, lastp, toks, bps)])
        states.append(out)
    print(f"[merged beam] B={B} W={W} image={img} toks {states[1][-1][5].tolist()}", flush=True)
    for depth, (a, b) in enumerate(zip(*states)):
        for name, x, y in zip(("vals", "ids", "lse", "cum", "lastp", "toks", "bps"), a, b):
            assert torch.equal(x, y), (depth, name)
