"""The drafting hot path on MI355X: one flow pass, then the beam over the shortlisted head.

``Drafter`` holds what the proposer's ``_build`` assembles (``cf/vllm_plugin/flow_proposer.py:579-867``):
the packed flow experts, the PathHead, the shortlisted lm_head with the markov bias, the target's
input embeddings and, for the latent drafter (``TreeVAEFlowConfig``), the packed VAE the flow runs
inside (``cf/drafters/tree_vae_flow.py:163-175``).  ``beam_chains`` / ``beam_tree`` are the proposer's ``_draft_fn``
(``:1187-1332``) with no host synchronisation until the caller reads the result.
"""
from __future__ import annotations

import ctypes as C

import torch

from chain_flow_amd import _lib
from chain_flow_amd.config import TreeFlowConfig, TreeVAEFlowConfig
from chain_flow_amd.flow import FusedFlow
from chain_flow_amd.head import GEMV_ROWS, PathHead, ShortlistHead, row_topk
from chain_flow_amd.vae import HiddenVAE


def front_pad(hidden: torch.Tensor, context_size: int) -> torch.Tensor:
    """``TreeFlowDrafter._context`` (``cf/drafters/tree_flow.py:143-148``): the last C rows, front-padded
    by repeating the oldest row."""
    n = hidden.shape[1]
    if n >= context_size:
        return hidden[:, -context_size:]
    pad = hidden[:, :1].expand(-1, context_size - n, -1)
    return torch.cat([pad, hidden], dim=1)


class Drafter:
    """``twopass_m`` > 0 switches the beam searches to the two-pass candidate head
    (``cf/vllm_plugin/flow_proposer.py:1113-1184``): one head pass over the marginal hiddens of every
    depth picks M shortlist rows (``twopass_shared``: one set for all depths, else one per depth;
    ``twopass_seed``: scored with the seed path's residual and markov bias), and each depth
    rescores only those rows, renormalised over them."""

    def __init__(self, cfg: TreeFlowConfig, weights: dict, shortlist: torch.Tensor | None, device="cuda",
                 path_trim: bool = True, twopass_m: int = 0, twopass_shared: bool = True,
                 twopass_seed: bool = False):
        self.cfg = cfg
        dev = torch.device(device)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.device = dev
        self.path_trim = path_trim
        self.vae = None
        if isinstance(cfg, TreeVAEFlowConfig):
            # lag_context only changes how training builds the context (build_context,
            # cf/drafters/tree_vae_flow.py:144-160, called from training/train_tree_flow.py:233); the
            # proposer never calls it, so at inference its lag_proj weights are unused.
            hidden = weights["lm_head.weight"].shape[1]
            self.vae = HiddenVAE(cfg, hidden, weights, device=dev)
        self.flow = FusedFlow(cfg, weights, device=dev)
        self.path = PathHead(weights, weights["embed_tokens.weight"], cfg.path_order,
                             cfg.path_ffn_multiplier, dev)
        self.head = ShortlistHead(weights["lm_head.weight"].to(dev, torch.float16), shortlist,
                                  weights["markov.w1.weight"], weights["markov.w2.weight"])
        self.order = cfg.path_order
        if twopass_m and not 0 < twopass_m < self.head.n:
            raise ValueError(f"two-pass M={twopass_m} must be below the head's {self.head.n} rows")
        self.twopass_m, self.twopass_shared, self.twopass_seed = int(twopass_m), bool(twopass_shared), \
            bool(twopass_seed)

    def _pass_a(self, pred: torch.Tensor, lastp: torch.Tensor, n0: int, n1: int, width: int):
        """Candidate rows of depths n0..n1-1: global ids [B, n1-n0, M] (a shared set repeated)."""
        B = pred.shape[0]
        sr = sp = None
        if self.twopass_seed:
            res0 = torch.empty(B * width, pred.shape[-1], dtype=torch.float16, device=self.device)
            for b in range(B):
                self.path.hidden(lastp[b], self._nlive(1), torch.zeros_like(pred[b, 0]),
                                 out=res0[b * width:(b + 1) * width])
            sr = res0.view(B, width, -1)[:, 0]
            sp = lastp[:, 0, 0]
        local, glob = self.head.candidates(pred[:, n0:n1].contiguous(), self.twopass_m, self.twopass_shared, sr, sp)
        if self.twopass_shared:
            glob = glob[:, None].expand(B, n1 - n0, self.twopass_m)
            local = local[:, None].expand(B, n1 - n0, self.twopass_m)
        # (the shortlist positions of the same rows: pass B of a large batch gathers them from one
        # full-shortlist head pass)
        self._cand_local = local
        return glob

    def _candidate_image(self, cands, B):
        """One request with a shared candidate set: its rows packed once for every depth."""
        if cands is None or B != 1 or not self.twopass_shared:
            return None
        self._cimg = self.head.pack_rows(cands[0, 0].contiguous(), getattr(self, "_cimg", None))
        return self._cimg

    def _scores(self, rows: torch.Tensor, k: int, prev: torch.Tensor, order: int, cand: torch.Tensor | None, B: int,
                image: torch.Tensor | None = None, local: torch.Tensor | None = None):
        """Per-depth top-k of rows [B*F, d]: (vals [B*F, k], ids [B*F, k] int32, map) -- one-pass over the
        shortlist (ids shortlist-local, map = the shortlist), two-pass over one request's packed
        candidate image (ids local to the candidates, map = their global ids), or over every
        request's own candidate rows read in place, all requests in one launch (ids already global,
        map None)."""
        if cand is None:
            vals, ids, _ = self.head.topk(rows, k, prev=prev, prev_stride=order)
            return vals, ids, self.head.sl
        if image is not None:
            vals, ids, _ = self.head.topk_image(rows, k, image, cand.shape[-1], prev=prev, prev_stride=order)
            return vals, ids, cand[0]
        cb = cand.contiguous()                                          # [B, M]
        F = rows.shape[0] // B
        M = cb.shape[1]
        if local is not None and B * M > self.head.n and self.head.image is not None:
            # Many requests: their candidate rows (B M, with repeats) outnumber the shortlist, so one
            # head pass over the whole shortlist for every row (the GEMM head, the markov bias at the
            # same rounding points, logits kept) reads less than each request's rows in place; each
            # row's log-softmax top-k then runs over its request's candidates gathered from those
            # logits (cfh_row_topk: the head's own top-k rule, ids = positions in the candidate list).
            BF, n = rows.shape[0], self.head.n
            lg = torch.empty(BF, n, dtype=torch.float16, device=rows.device)
            scratch = (torch.empty(BF, 1, dtype=torch.float32, device=rows.device),
                       torch.empty(BF, 1, dtype=torch.int32, device=rows.device),
                       torch.empty(BF, dtype=torch.float32, device=rows.device))
            self.head.topk(rows, 1, prev=prev, prev_stride=order, logits=lg, out=scratch)
            idx = local.contiguous().long().view(B, 1, M).expand(B, F, M)
            sub = torch.gather(lg.view(B, F, n), 2, idx).view(BF, M)
            vals, ids, _ = row_topk(sub, k)
        else:
            vals, ids, _ = self.head.topk_groups(rows, k, cb, prev=prev, prev_stride=order)
        glob = torch.gather(cb, 1, ids.view(B, F * k).long()).view(B * F, k)
        return vals, glob, None

    def _nlive(self, depth: int):
        """``_nlive`` (``cf/vllm_plugin/flow_proposer.py:1030-1037``)."""
        return depth if self.path_trim else None

    @property
    def anchored(self) -> bool:
        """True for a latent drafter trained with ``anchor_token``: its flow is conditioned on the
        committed token's embedding (``cf/drafters/tree_vae_flow.py:45, 128-129``)."""
        return bool(self.flow.anchor_params)

    def predict_hidden(self, ctx: torch.Tensor, known0: torch.Tensor | None = None) -> torch.Tensor:
        """ctx [B, C, hidden] (front-padded) -> marginal hiddens [B, draft_length, hidden]
        (``TreeFlowDrafter.predict_hidden``; latent drafter: decode(integrate(encode(ctx).mu))).
        known0 [B]: the committed tokens; an anchored drafter is given their embeddings as the
        reference's proposer does (``predict_hidden(ctx, anchor_embed(known0))``,
        ``cf/vllm_plugin/flow_proposer.py:1203, 1285``); ignored by an unanchored one."""
        ctx = ctx.to(self.device, torch.float16)
        if self.vae is None:
            return self.flow.predict_hidden(ctx)
        anchor = None
        if known0 is not None and self.anchored:
            anchor = self.flow.anchor(known0, self.path.embed_w)
        return self.vae.decode(self.flow.predict_hidden(self.vae.encode(ctx), anchor=anchor))

    def beam_chains(self, ctx: torch.Tensor, known0: torch.Tensor, K: int, width: int = 4,
                    pred: torch.Tensor | None = None) -> torch.Tensor:
        """``_beam_chains`` with the one-pass head: ctx [B, C, d], known0 [B] -> [B, K'] int64 global ids,
        K' = min(K, draft_length - 1).  ``pred`` (the flow output) may be passed in to skip the flow."""
        dev = self.device
        W, order = width, self.order
        if not 1 <= W <= 8:
            raise ValueError(f"beam width {W} is not supported: the beam step keeps W*W <= 64 candidates "
                             f"per chain (width 1..8)")
        if pred is None:
            pred = self.predict_hidden(ctx, known0)
        B, Kd, d = pred.shape
        steps = min(K + 1, Kd)
        L = _lib.lib()
        st = _lib.stream_handle()
        # lastp = -1 but the committed token in every beam's position 0; cum = 0 for beam 0, -inf else
        lastp = torch.empty(B, W, order, dtype=torch.int32, device=dev)
        cum = torch.empty(B, W, dtype=torch.float32, device=dev)
        k0 = known0.to(dev, torch.int64).contiguous()
        _lib.check(L.cfh_beam_init(k0.data_ptr(), lastp.data_ptr(), cum.data_ptr(), None, B, W, order, 0, st),
                   "cfh_beam_init")
        nst = steps - 1
        toks = torch.empty(max(nst, 1), B, W, dtype=torch.int32, device=dev)
        bps = torch.empty_like(toks)
        hbuf = torch.empty(B * W, d, dtype=torch.float16, device=dev)
        cands = self._pass_a(pred, lastp, 1, steps, W) if self.twopass_m and steps > 1 else None
        image = self._candidate_image(cands, B)
        # a packed image and at most 8 beam rows: each depth's top-k merge and beam step in one launch
        fused = W <= 4 and B * W <= GEMV_ROWS and ((cands is None and self.head.image is not None)
                                                   or image is not None)
        for step in range(1, steps):
            # every request's W beams in one call, each request's rows with its own marginal hidden
            self.path.hidden(lastp.view(B * W, order), self._nlive(step), pred[:, step], out=hbuf)
            if fused:
                img, n, smap = ((None, self.head.n, self.head.sl) if cands is None
                                else (image, cands.shape[-1], cands[0, step - 1]))
                self.head.topk_beam_chain(hbuf, img, n, lastp.view(-1), order, cum, lastp, smap,
                                          toks[step - 1], bps[step - 1], B, W, order)
                continue
            vals, ids, smap = self._scores(hbuf, W, lastp.view(-1), order,
                                           None if cands is None else cands[:, step - 1], B, image,
                                           None if cands is None else self._cand_local[:, step - 1])
            _lib.check(L.cfh_beam_chain_step(vals.data_ptr(), ids.data_ptr(), cum.data_ptr(), lastp.data_ptr(),
                                             _lib.ptr(smap), toks[step - 1].data_ptr(),
                                             bps[step - 1].data_ptr(), B, W, order, st), "cfh_beam_chain_step")
        out = torch.empty(B, nst, dtype=torch.int64, device=dev)
        if nst > 0:
            _lib.check(L.cfh_beam_backtrack(cum.data_ptr(), toks.data_ptr(), bps.data_ptr(), B, W, nst,
                                            out.data_ptr(), st), "cfh_beam_backtrack")
        return out

    def beam_tree(self, ctx: torch.Tensor, known0: torch.Tensor, keep: int = 4, topb: int = 8, depth: int = 4,
                  pred: torch.Tensor | None = None) -> torch.Tensor:
        """``_beam_tree``: -> [B, 2N] int32-valued int64: N BFS-ordered tokens || parent node indices."""
        dev = self.device
        order = self.order
        if keep < 1 or topb < 1 or keep * topb > 64:
            raise ValueError(f"tree keep {keep} x top-b {topb} is not supported: a tree step ranks at most 64 "
                             f"children per request (keep * topb <= 64)")
        if pred is None:
            pred = self.predict_hidden(ctx, known0)
        B, Kd, d = pred.shape
        nstep = min(depth, Kd - 1)
        sizes, fr = [], 1
        for _ in range(nstep):
            k = min(keep, fr * topb)
            sizes.append(k)
            fr = k
        N = sum(sizes)
        out = torch.empty(B, 2 * N, dtype=torch.int32, device=dev)
        L = _lib.lib()
        st = _lib.stream_handle()
        # lastp = -1 but the committed token in slot 0's position 0; cum = 0; prev_ids = -1
        lastp = torch.empty(B, keep, order, dtype=torch.int32, device=dev)
        cum = torch.empty(B, keep, dtype=torch.float32, device=dev)
        prev_ids = torch.empty(B, keep, dtype=torch.int32, device=dev)
        k0 = known0.to(dev, torch.int64).contiguous()
        _lib.check(L.cfh_beam_init(k0.data_ptr(), lastp.data_ptr(), cum.data_ptr(), prev_ids.data_ptr(), B, keep,
                                   order, 1, st), "cfh_beam_init")
        hbuf = torch.empty(B * keep, d, dtype=torch.float16, device=dev)
        cands = self._pass_a(pred, lastp, 1, nstep + 1, keep) if self.twopass_m and nstep > 0 else None
        image = self._candidate_image(cands, B)
        fr, base = 1, 0
        for step in range(1, nstep + 1):
            rows = torch.empty(B * fr, d, dtype=torch.float16, device=dev) if fr != keep else hbuf
            lp_rows = lastp[:, :fr].reshape(B * fr, order).contiguous()
            self.path.hidden(lp_rows, self._nlive(step), pred[:, step], out=rows)
            vals, ids, smap = self._scores(rows, topb, lp_rows.view(-1), order,
                                           None if cands is None else cands[:, step - 1], B, image,
                                           None if cands is None else self._cand_local[:, step - 1])
            _lib.check(L.cfh_beam_tree_step(vals.data_ptr(), ids.data_ptr(), cum.data_ptr(), lastp.data_ptr(),
                                            prev_ids.data_ptr(), _lib.ptr(smap), out.data_ptr(), 2 * N,
                                            base, B, fr, topb, keep, order, st), "cfh_beam_tree_step")
            base += sizes[step - 1]
            fr = sizes[step - 1]
        return out.long()
