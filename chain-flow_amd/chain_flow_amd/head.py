"""Host side of the draft head: shortlisted lm_head + markov bias + top-k, and the PathHead residual.

Mirrors the proposer's ``_head`` / ``_bias`` / ``_map`` (``cf/vllm_plugin/flow_proposer.py:1021-1028``)
and the fused ``_residual_from_lastp`` (``cf/vllm_plugin/fused.py:25-37``) over libcfhip.so.
"""
from __future__ import annotations

import ctypes as C

import torch

from chain_flow_amd import _lib


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.int32).contiguous()


GEMV_ROWS = 8        # rows the GEMV head takes per launch; more go through the MFMA GEMM head
GEMM_ROWS = 256      # rows of one GEMM head launch


class ShortlistHead:
    """The target's lm_head restricted to a shortlist, plus the markov logit bias
    ``markov.w2(markov.w1[prev])`` restricted to the same rows.

    ``packed=True`` (default) gathers the shortlisted rows of lm_head and markov.w2 once into the
    MFMA fragment order (``cfh_head_pack``: n * (d + r) * 2 bytes of HBM, 673 MB for the 62,642-row
    shortlist at d=5120, r=256), so ``topk`` streams contiguous fragments; ``packed=False`` reads
    the rows in place through the shortlist on every call.  Both give the same results."""

    def __init__(self, lm_w: torch.Tensor, shortlist: torch.Tensor | None, w1: torch.Tensor | None = None,
                 w2: torch.Tensor | None = None, packed: bool = True):
        if lm_w.dtype != torch.float16 or not lm_w.is_cuda:
            raise ValueError("lm_w must be a CUDA fp16 [V, d] tensor")
        self.lm_w = lm_w.contiguous()
        self.V, self.d = self.lm_w.shape
        self.sl = None if shortlist is None else _i32(shortlist.to(lm_w.device))
        if self.sl is not None and self.sl.numel() and (int(self.sl.min()) < 0 or int(self.sl.max()) >= self.V):
            raise ValueError("shortlist ids out of range of the lm_head")
        self.n = self.V if self.sl is None else int(self.sl.numel())
        self.w1 = None if w1 is None else w1.to(lm_w.device, torch.float16).contiguous()
        self.w2 = None if w2 is None else w2.to(lm_w.device, torch.float16).contiguous()
        if (self.w1 is None) != (self.w2 is None):
            raise ValueError("markov w1 and w2 go together")
        self.r = 0 if self.w1 is None else int(self.w1.shape[1])
        self._ws = {}
        self.image = None
        if packed:
            L = _lib.lib()
            nbytes = int(L.cfh_head_packed_bytes(self.n, self.d, self.r))
            if nbytes < 0:
                raise ValueError(f"head shape unsupported for packing: n={self.n} d={self.d} r={self.r}")
            self.image = torch.empty(nbytes, dtype=torch.uint8, device=lm_w.device)
            _lib.check(L.cfh_head_pack(self.lm_w.data_ptr(), None if self.w2 is None else self.w2.data_ptr(),
                                       _lib.ptr(self.sl), self.n, self.d, self.r, self.image.data_ptr(),
                                       _lib.stream_handle()), "cfh_head_pack")

    def map(self, local: torch.Tensor) -> torch.Tensor:
        """``_map``: shortlist-local column -> global token id."""
        return local if self.sl is None else self.sl.long()[local.long()]

    def logits(self, h: torch.Tensor, prev: torch.Tensor | None = None, prev_stride: int = 1,
               out: torch.Tensor | None = None) -> torch.Tensor:
        """h [M, d] fp16, prev (global ids, int32) -> fp16 logits [M, n] (head + markov bias)."""
        M = h.shape[0]
        if out is None:
            out = torch.empty(M, self.n, dtype=torch.float16, device=h.device)
        use_m = self.w1 is not None and prev is not None
        _lib.check(_lib.lib().cfh_head_logits(
            h.data_ptr(), M, self.d, self.lm_w.data_ptr(), _lib.ptr(self.sl), self.n,
            self.w1.data_ptr() if use_m else None, prev.data_ptr() if use_m else None, prev_stride,
            self.r, self.w2.data_ptr() if use_m else None, out.data_ptr(), _lib.stream_handle()),
            "cfh_head_logits")
        return out

    def workspace(self, M: int, k: int, device) -> torch.Tensor:
        """Candidate workspace for M rows and top-k (kept per shape, reused across calls)."""
        key = (M, k)
        ws = self._ws.get(key)
        if ws is None:
            nbytes = int(_lib.lib().cfh_head_ws_bytes(M, self.n, k))
            if nbytes < 0:
                raise ValueError(f"head top-k shape unsupported: M={M} k={k}")
            ws = self._ws[key] = torch.empty(nbytes, dtype=torch.uint8, device=device)
        return ws

    def topk(self, h: torch.Tensor, k: int, prev: torch.Tensor | None = None, prev_stride: int = 1,
             logits: torch.Tensor | None = None, out=None):
        """-> (log-prob values [M, k] f32, shortlist-local ids [M, k] int32, lse [M] f32).

        The log-softmax top-k is fused into the head; ``logits`` (fp16 [M, n]) is written only when
        given.  ``out`` = preallocated (vals, ids, lse) to fill.  Up to 8 rows run on the GEMV head;
        more (the batched and tree searches, pass A over many requests) on the MFMA GEMM head over
        the packed image, 256 rows a launch, with the same rounding points."""
        M = h.shape[0]
        dev = h.device
        if out is None:
            vals = torch.empty(M, k, dtype=torch.float32, device=dev)
            ids = torch.empty(M, k, dtype=torch.int32, device=dev)
            lse = torch.empty(M, dtype=torch.float32, device=dev)
        else:
            vals, ids, lse = out
        use_m = self.w1 is not None and prev is not None
        if M > GEMV_ROWS:
            if self.image is None:
                for r0 in range(0, M, GEMV_ROWS):
                    r1 = min(M, r0 + GEMV_ROWS)
                    self.topk(h[r0:r1], k, None if not use_m else prev[r0 * prev_stride:], prev_stride,
                              None if logits is None else logits[r0:r1], (vals[r0:r1], ids[r0:r1], lse[r0:r1]))
                return vals, ids, lse
            for r0 in range(0, M, GEMM_ROWS):
                r1 = min(M, r0 + GEMM_ROWS)
                pv = prev[r0 * prev_stride:r1 * prev_stride:prev_stride] if use_m else None
                self.gemm_topk(h[r0:r1], k, pv, None if logits is None else logits[r0:r1],
                               (vals[r0:r1], ids[r0:r1], lse[r0:r1]))
            return vals, ids, lse
        ws = self.workspace(M, k, dev)
        if self.image is not None:
            _lib.check(_lib.lib().cfh_head_topk_packed(
                h.data_ptr(), M, self.d, self.image.data_ptr(), self.n,
                self.w1.data_ptr() if use_m else None, prev.data_ptr() if use_m else None, prev_stride,
                self.r if use_m else 0, k, _lib.ptr(logits), vals.data_ptr(), ids.data_ptr(), lse.data_ptr(),
                ws.data_ptr(), _lib.stream_handle()), "cfh_head_topk_packed")
            return vals, ids, lse
        _lib.check(_lib.lib().cfh_head_topk(
            h.data_ptr(), M, self.d, self.lm_w.data_ptr(), _lib.ptr(self.sl), self.n,
            self.w1.data_ptr() if use_m else None, prev.data_ptr() if use_m else None, prev_stride,
            self.r, self.w2.data_ptr() if use_m else None, k, _lib.ptr(logits), vals.data_ptr(),
            ids.data_ptr(), lse.data_ptr(), ws.data_ptr(), _lib.stream_handle()),
            "cfh_head_topk")
        return vals, ids, lse

    def gemm_topk(self, h: torch.Tensor, k: int, prev: torch.Tensor | None, logits: torch.Tensor | None, out):
        """``topk`` of up to 256 rows on the MFMA GEMM head (cfh_head_gemm16_topk) over the packed
        image; with ``prev`` (one global id per row) the markov bias fp16(w1[prev] . w2_sl) first, as
        logits of the image's markov rows, added before the head logits' last rounding."""
        M = h.shape[0]
        L = _lib.lib()
        st = _lib.stream_handle()
        h = h.contiguous()
        bias = None
        if prev is not None and self.w1 is not None:
            a = self.w1.index_select(0, prev.to(torch.long)).contiguous()          # [M, r]
            bias = torch.empty(M, self.n, dtype=torch.float16, device=h.device)
            w2img = self.image.data_ptr() + int(L.cfh_head_packed_bytes(self.n, self.d, 0))
            _lib.check(L.cfh_head_gemm16_topk(a.data_ptr(), M, self.r, w2img, self.n, None, 0, bias.data_ptr(),
                                              None, None, None, None, st), "cfh_head_gemm16_topk (markov)")
        vals, ids, lse = out
        ws = self.workspace(M, k, h.device)
        _lib.check(L.cfh_head_gemm16_topk(h.data_ptr(), M, self.d, self.image.data_ptr(), self.n, _lib.ptr(bias), k,
                                          _lib.ptr(logits), vals.data_ptr(), ids.data_ptr(), lse.data_ptr(),
                                          ws.data_ptr(), st), "cfh_head_gemm16_topk")
        return vals, ids, lse

    def candidates(self, hm: torch.Tensor, M: int, shared: bool = True, seed_res: torch.Tensor | None = None,
                   seed_prev: torch.Tensor | None = None):
        """Pass A of the two-pass head (``_candidates``, ``cf/vllm_plugin/flow_proposer.py:1142-1165``):
        hm [B, n, d] fp16 marginal hiddens of n depths -> (local [B, M] or [B, n, M] int32 ascending
        shortlist columns, global ids of the same shape).  shared: one set per request by the best
        per-depth log-prob; else one set per depth.  seed_res [B, d] / seed_prev [B] (global ids):
        the seed path's residual and markov parent added to every row."""
        B, n, d = hm.shape
        dev = hm.device
        if not 0 < M < self.n:
            raise ValueError(f"two-pass M={M} must be in (0, {self.n})")
        rows = hm if seed_res is None else (hm.float() + seed_res.float()[:, None]).to(torch.float16)
        rows = rows.reshape(B * n, d).contiguous()
        prev = None if seed_prev is None else seed_prev.to(dev, torch.int32).repeat_interleave(n).contiguous()
        logits = torch.empty(B * n, self.n, dtype=torch.float16, device=dev)
        lse = torch.empty(B * n, dtype=torch.float32, device=dev)
        # every row in one head pass (the GEMM head above 8 rows): top-1 discarded, logits and lse kept
        self.topk(rows, 1, prev=prev, logits=logits,
                  out=(torch.empty(B * n, 1, device=dev), torch.empty(B * n, 1, dtype=torch.int32, device=dev), lse))
        nreq, nrow = (B, n) if shared else (B * n, 1)
        local = torch.empty(nreq, M, dtype=torch.int32, device=dev)
        glob = torch.empty(nreq, M, dtype=torch.int32, device=dev)
        L = _lib.lib()
        ws = torch.empty(int(L.cfh_cand_ws_bytes(nreq, self.n)), dtype=torch.uint8, device=dev)
        _lib.check(L.cfh_cand_topm(logits.data_ptr(), self.n, lse.data_ptr(), nreq, nrow, self.n, M,
                                   _lib.ptr(self.sl), local.data_ptr(), glob.data_ptr(), ws.data_ptr(),
                                   _lib.stream_handle()), "cfh_cand_topm")
        if not shared:
            local, glob = local.view(B, n, M), glob.view(B, n, M)
        return local, glob

    def pack_rows(self, rows: torch.Tensor, image: torch.Tensor | None = None) -> torch.Tensor:
        """The given global rows of lm_head and markov w2 (int32 [M]) gathered once into the MFMA
        fragment order (``cfh_head_pack``): the two-pass head's shared candidate image, read by
        ``topk_image`` at every depth (``_gather_cand``, ``flow_proposer.py:1167-1172``)."""
        n = rows.numel()
        L = _lib.lib()
        nbytes = int(L.cfh_head_packed_bytes(n, self.d, self.r))
        if image is None or image.numel() < nbytes:
            image = torch.empty(nbytes, dtype=torch.uint8, device=self.lm_w.device)
        _lib.check(L.cfh_head_pack(self.lm_w.data_ptr(), None if self.w2 is None else self.w2.data_ptr(),
                                   rows.data_ptr(), n, self.d, self.r, image.data_ptr(), _lib.stream_handle()),
                   "cfh_head_pack")
        return image

    def topk_image(self, h: torch.Tensor, k: int, image: torch.Tensor, n: int, prev: torch.Tensor | None = None,
                   prev_stride: int = 1):
        """``topk`` over a ``pack_rows`` image of n rows: ids are positions in those rows."""
        Mh = h.shape[0]
        dev = h.device
        if Mh > GEMV_ROWS:                                   # the GEMV head takes 8 rows a launch
            parts = [self.topk_image(h[r0:r0 + GEMV_ROWS], k, image, n,
                                     None if prev is None else prev[r0 * prev_stride:], prev_stride)
                     for r0 in range(0, Mh, GEMV_ROWS)]
            return tuple(torch.cat([p[i] for p in parts]) for i in range(3))
        vals = torch.empty(Mh, k, dtype=torch.float32, device=dev)
        ids = torch.empty(Mh, k, dtype=torch.int32, device=dev)
        lse = torch.empty(Mh, dtype=torch.float32, device=dev)
        key = ("image", Mh, n, k)
        ws = self._ws.get(key)
        if ws is None:
            ws = self._ws[key] = torch.empty(int(_lib.lib().cfh_head_ws_bytes(Mh, n, k)), dtype=torch.uint8,
                                             device=dev)
        use_m = self.w1 is not None and prev is not None
        _lib.check(_lib.lib().cfh_head_topk_packed(
            h.data_ptr(), Mh, self.d, image.data_ptr(), n, self.w1.data_ptr() if use_m else None,
            prev.data_ptr() if use_m else None, prev_stride, self.r if use_m else 0, k, None, vals.data_ptr(),
            ids.data_ptr(), lse.data_ptr(), ws.data_ptr(), _lib.stream_handle()), "cfh_head_topk_packed")
        return vals, ids, lse

    def topk_beam_chain(self, h: torch.Tensor, image: torch.Tensor | None, n: int, prev: torch.Tensor,
                        prev_stride: int, cum: torch.Tensor, lastp: torch.Tensor, smap: torch.Tensor | None,
                        toks: torch.Tensor, bps: torch.Tensor, B: int, W: int, order: int):
        """One depth of a chain search over B chains of W beams (h [B*W, d], B*W <= 8 rows): the top-W
        of every beam row over a packed image (the head's own, ``image=None``, or a ``pack_rows``
        image of n rows) and the beam step (cum, lastp, toks, bps in place; ``smap`` maps the ids),
        the merge and the step in one launch (``cfh_head_topk_packed_beam_chain``).
        -> (vals [B*W, W], ids [B*W, W] int32, lse [B*W]) as ``topk`` / ``topk_image`` return them."""
        M = h.shape[0]
        dev = h.device
        img = self.image if image is None else image
        if img is None or M != B * W or M > GEMV_ROWS:
            raise ValueError("topk_beam_chain needs a packed image and at most 8 beam rows")
        vals = torch.empty(M, W, dtype=torch.float32, device=dev)
        ids = torch.empty(M, W, dtype=torch.int32, device=dev)
        lse = torch.empty(M, dtype=torch.float32, device=dev)
        if image is None:
            ws = self.workspace(M, W, dev)
        else:
            key = ("image", M, n, W)
            ws = self._ws.get(key)
            if ws is None:
                ws = self._ws[key] = torch.empty(int(_lib.lib().cfh_head_ws_bytes(M, n, W)), dtype=torch.uint8,
                                                 device=dev)
        use_m = self.w1 is not None and prev is not None
        _lib.check(_lib.lib().cfh_head_topk_packed_beam_chain(
            h.data_ptr(), M, self.d, img.data_ptr(), n, self.w1.data_ptr() if use_m else None,
            prev.data_ptr() if use_m else None, prev_stride, self.r if use_m else 0, vals.data_ptr(),
            ids.data_ptr(), lse.data_ptr(), ws.data_ptr(), cum.data_ptr(), lastp.data_ptr(), _lib.ptr(smap),
            toks.data_ptr(), bps.data_ptr(), B, W, order, _lib.stream_handle()), "cfh_head_topk_packed_beam_chain")
        return vals, ids, lse

    def topk_groups(self, h: torch.Tensor, k: int, rows: torch.Tensor, prev: torch.Tensor | None = None,
                    prev_stride: int = 1):
        """Pass B for a batch in one launch (``cfh_head_topk_grouped``): h [G*F, d] (F consecutive rows
        per request), rows [G, M] int32 global candidate ids of each request (read in place), the
        head and markov bias over each request's own candidates, log-softmax over them, top-k.
        -> (vals [G*F, k], ids [G*F, k] int32 positions in the request's row list, lse [G*F])."""
        G, n = rows.shape
        GF = h.shape[0]
        F = GF // G
        dev = h.device
        vals = torch.empty(GF, k, dtype=torch.float32, device=dev)
        ids = torch.empty(GF, k, dtype=torch.int32, device=dev)
        lse = torch.empty(GF, dtype=torch.float32, device=dev)
        use_m = self.w1 is not None and prev is not None
        L = _lib.lib()
        rows = rows.contiguous()
        pid = prev.reshape(-1)[::prev_stride][:GF].view(G, F) if use_m else None   # markov parent of each row
        for c0 in range(0, F, GEMV_ROWS):                    # a launch takes at most 8 rows per request
            c1 = min(F, c0 + GEMV_ROWS)
            m = c1 - c0
            hv = h.view(G, F, -1)[:, c0:c1].contiguous() if (c0, c1) != (0, F) else h.contiguous()
            pv = pid[:, c0:c1].contiguous() if use_m else None
            v = torch.empty(G * m, k, dtype=torch.float32, device=dev)
            i = torch.empty(G * m, k, dtype=torch.int32, device=dev)
            ls = torch.empty(G * m, dtype=torch.float32, device=dev)
            key = ("groups", G * m, n, k)
            ws = self._ws.get(key)
            if ws is None:
                ws = self._ws[key] = torch.empty(int(L.cfh_head_ws_bytes(G * m, n, k)), dtype=torch.uint8, device=dev)
            _lib.check(L.cfh_head_topk_grouped(
                hv.data_ptr(), G, m, self.d, self.lm_w.data_ptr(), rows.data_ptr(), n, n,
                self.w1.data_ptr() if use_m else None, pv.data_ptr() if use_m else None, 1,
                self.r if use_m else 0, self.w2.data_ptr() if use_m else None, k, v.data_ptr(), i.data_ptr(),
                ls.data_ptr(), ws.data_ptr(), _lib.stream_handle()), "cfh_head_topk_grouped")
            if (c0, c1) == (0, F):
                return v, i, ls
            vals.view(G, F, k)[:, c0:c1] = v.view(G, m, k)
            ids.view(G, F, k)[:, c0:c1] = i.view(G, m, k)
            lse.view(G, F)[:, c0:c1] = ls.view(G, m)
        return vals, ids, lse

    def topk_rows(self, h: torch.Tensor, k: int, rows: torch.Tensor, prev: torch.Tensor | None = None,
                  prev_stride: int = 1):
        """Pass B (``_rescore`` + topk): the head and markov bias over the given global rows only
        (int32 [M], read in place), log-softmax over those M columns, top-k.
        -> (vals [Mh, k] f32, ids [Mh, k] int32 positions in ``rows``, lse [Mh])."""
        Mh, n = h.shape[0], rows.numel()
        dev = h.device
        vals = torch.empty(Mh, k, dtype=torch.float32, device=dev)
        ids = torch.empty(Mh, k, dtype=torch.int32, device=dev)
        lse = torch.empty(Mh, dtype=torch.float32, device=dev)
        key = ("rows", Mh, n, k)
        ws = self._ws.get(key)
        if ws is None:
            ws = self._ws[key] = torch.empty(int(_lib.lib().cfh_head_ws_bytes(Mh, n, k)), dtype=torch.uint8,
                                             device=dev)
        use_m = self.w1 is not None and prev is not None
        _lib.check(_lib.lib().cfh_head_topk(
            h.data_ptr(), Mh, self.d, self.lm_w.data_ptr(), rows.data_ptr(), n,
            self.w1.data_ptr() if use_m else None, prev.data_ptr() if use_m else None, prev_stride,
            self.r, self.w2.data_ptr() if use_m else None, k, None, vals.data_ptr(), ids.data_ptr(),
            lse.data_ptr(), ws.data_ptr(), _lib.stream_handle()), "cfh_head_topk")
        return vals, ids, lse


class GemmHead:
    """Batched shortlisted head for many rows (M up to 256): bf16 MFMA skinny GEMM over the
    shortlist rows of the lm_head, with the per-row log-softmax top-k fused in (the two-pass
    candidate head's pass A, ``cf/vllm_plugin/flow_proposer.py:1142-1165``).  ``packed=True`` gathers
    the shortlist rows once into the MFMA fragment image (``cfh_head_pack``; d % 256 == 0) so every
    weight load is contiguous; otherwise the rows are read in place through the shortlist."""

    def __init__(self, lm_w: torch.Tensor, shortlist: torch.Tensor | None, packed: bool = False):
        if lm_w.dtype != torch.bfloat16 or not lm_w.is_cuda:
            raise ValueError("lm_w must be a CUDA bf16 [V, d] tensor")
        self.lm_w = lm_w.contiguous()
        self.V, self.d = self.lm_w.shape
        self.sl = None if shortlist is None else _i32(shortlist.to(lm_w.device))
        self.n = self.V if self.sl is None else int(self.sl.numel())
        self._ws = {}
        self.image = None
        if packed:
            nbytes = int(_lib.lib().cfh_head_packed_bytes(self.n, self.d, 0))
            if nbytes < 0:
                raise ValueError(f"packed gemm head needs d % 256 == 0 (d={self.d})")
            self.image = torch.empty(nbytes, dtype=torch.uint8, device=lm_w.device)
            _lib.check(_lib.lib().cfh_head_pack(self.lm_w.data_ptr(), None, _lib.ptr(self.sl), self.n, self.d, 0,
                                                self.image.data_ptr(), _lib.stream_handle()), "cfh_head_pack")

    def topk(self, x: torch.Tensor, k: int, logits: torch.Tensor | None = None):
        """x [M, d] bf16 -> (vals [M, k] f32 log-probs, ids [M, k] int32 local, lse [M] f32)."""
        if x.dtype != torch.bfloat16 or x.shape[1] != self.d:
            raise ValueError(f"x must be bf16 [M, {self.d}]")
        x = x.contiguous()
        M = x.shape[0]
        dev = x.device
        key = (M, k)
        if key not in self._ws:
            nbytes = int(_lib.lib().cfh_head_ws_bytes(M, self.n, k))
            if nbytes < 0:
                raise ValueError(f"gemm head shape unsupported: M={M} k={k}")
            self._ws[key] = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        vals = torch.empty(M, k, dtype=torch.float32, device=dev)
        ids = torch.empty(M, k, dtype=torch.int32, device=dev)
        lse = torch.empty(M, dtype=torch.float32, device=dev)
        if self.image is not None:
            _lib.check(_lib.lib().cfh_head_gemm_topk_packed(
                x.data_ptr(), M, self.d, self.image.data_ptr(), self.n, k, _lib.ptr(logits), vals.data_ptr(),
                ids.data_ptr(), lse.data_ptr(), self._ws[key].data_ptr(), _lib.stream_handle()),
                "cfh_head_gemm_topk_packed")
        else:
            _lib.check(_lib.lib().cfh_head_gemm_topk(
                x.data_ptr(), M, self.d, self.lm_w.data_ptr(), _lib.ptr(self.sl), self.n, k, _lib.ptr(logits),
                vals.data_ptr(), ids.data_ptr(), lse.data_ptr(), self._ws[key].data_ptr(), _lib.stream_handle()),
                "cfh_head_gemm_topk")
        return vals, ids, lse


def row_topk(logits: torch.Tensor, k: int):
    """Per-row log-softmax top-k of fp16 logits [M, n] -> (vals f32, ids int32, lse f32)."""
    M, n = logits.shape
    logits = logits.contiguous()
    vals = torch.empty(M, k, dtype=torch.float32, device=logits.device)
    ids = torch.empty(M, k, dtype=torch.int32, device=logits.device)
    lse = torch.empty(M, dtype=torch.float32, device=logits.device)
    _lib.check(_lib.lib().cfh_row_topk(logits.data_ptr(), M, n, k, vals.data_ptr(), ids.data_ptr(),
                                       lse.data_ptr(), _lib.stream_handle()), "cfh_row_topk")
    return vals, ids, lse


def pack_linear(w: torch.Tensor) -> torch.Tensor:
    """Row-major [n, k] 2-byte weight -> MFMA tile order (same shape, new storage)."""
    w = w.contiguous()
    out = torch.empty_like(w)
    n, k = w.shape
    _lib.check(_lib.lib().cfh_pack_linear(w.data_ptr(), n, k, out.data_ptr(), _lib.stream_handle()),
               "cfh_pack_linear")
    return out


class PathHead:
    """PathHead residual ``mlp(norm(sum_j mask_j (W_j emb(lastp_j) + b_j)))`` over packed weights."""

    def __init__(self, weights: dict, embed_w: torch.Tensor, order: int, ffn_mult: int, device):
        dev = torch.device(device)
        f16 = dict(dtype=torch.float16, device=dev)
        self.order, self.ffn, self.d = order, ffn_mult, int(embed_w.shape[1])
        self.embed_w = embed_w.to(**f16).contiguous()
        g = lambda n: weights[n].to(**f16).contiguous()
        self.Wj = [pack_linear(g(f"path_head.offset_proj.{j}.weight")) for j in range(order)]
        self.bj = [g(f"path_head.offset_proj.{j}.bias") for j in range(order)]
        self.norm_w, self.norm_b = g("path_head.norm.weight"), g("path_head.norm.bias")
        self.W0, self.b0 = pack_linear(g("path_head.mlp.0.weight")), g("path_head.mlp.0.bias")
        self.W3, self.b3 = pack_linear(g("path_head.mlp.3.weight")), g("path_head.mlp.3.bias")
        ptrs = [t.data_ptr() for t in self.Wj + self.bj] + [
            self.norm_w.data_ptr(), self.norm_b.data_ptr(), self.W0.data_ptr(), self.b0.data_ptr(),
            self.W3.data_ptr(), self.b3.data_ptr()]
        self._ptrs = _lib.ptr_array(ptrs)
        self._ws = {}

    def _workspace(self, M: int, dev) -> torch.Tensor:
        ws = self._ws.get(M)
        if ws is None:
            nbytes = int(_lib.lib().cfh_path_ws_bytes(M, self.d, self.ffn, self.order))
            if nbytes < 0:
                raise ValueError(f"path residual shape unsupported: M={M} d={self.d}")
            ws = self._ws[M] = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        return ws

    def hidden(self, lastp: torch.Tensor, nlive: int | None, pred: torch.Tensor,
               out: torch.Tensor | None = None) -> torch.Tensor:
        """lastp [M, order] int32 (global ids, -1 = none); pred [d] fp16 shared by the M rows, or
        [G, d] (one marginal hidden per request, M // G consecutive rows each; a strided view such as
        pred[:, step] is fine) -> fp16(pred + residual) [M, d] (the head's input at this depth)."""
        M = lastp.shape[0]
        if pred.dim() == 1:
            pld, rpp = 0, 0
        else:
            G = pred.shape[0]
            if M % G or pred.stride(1) != 1:
                raise ValueError(f"pred [G, d] needs M % G == 0 and contiguous rows (M={M}, G={G})")
            pld, rpp = pred.stride(0), M // G
        if out is None:
            out = torch.empty(M, self.d, dtype=torch.float16, device=pred.device)
        # (16 rows at a time, or wide groups of up to 128 rows: the workspace depends on min(M, 128))
        ws = self._workspace(min(M, 128), pred.device)
        _lib.check(_lib.lib().cfh_path_residual(
            self._ptrs, self.order, self.ffn, self.d, lastp.data_ptr(), M,
            -1 if nlive is None else int(nlive), self.embed_w.data_ptr(), pred.data_ptr(), pld, rpp,
            out.data_ptr(), ws.data_ptr(), _lib.stream_handle()), "cfh_path_residual")
        return out
