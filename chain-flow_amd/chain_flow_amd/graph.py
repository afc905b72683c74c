"""Whole-draft HIP graphs: the ring step (append this step's hiddens, read each window) followed by
the draft (predict_hidden and the beam or tree search), captured once per batch bucket on fixed
buffers and replayed every step.

Mirrors the reference's draft cudagraphs (``_capture_ring`` / ``_ring_cg`` / ``_bucket_ladder``,
``cf/vllm_plugin/flow_proposer.py:1342-1365, 1511-1545, 1577-1589``), which capture ring gather ->
flow -> beam per bucket and pad a batch up to the next bucket; here the ring append is inside the
graph too (``cfh_ring_step`` is one fixed-shape launch, and padding rows append nothing).  A graph
holds no memset node: every buffer the captured work clears is cleared by a kernel.
"""
from __future__ import annotations

import os

import torch


def bucket_ladder(max_reqs: int) -> list[int]:
    """``CF_DRAFT_BUCKETS="1,2,4"`` or powers of two capped at ``max_reqs``, plus ``max_reqs``
    itself (``flow_proposer.py:1511-1545``)."""
    env = (os.environ.get("CF_DRAFT_BUCKETS", "") or "").replace(",", " ").split()
    cap = max(int(max_reqs), 1)
    if env:
        b = sorted({int(x) for x in env if int(x) > 0})
        return [x for x in b if x <= cap] or [1]
    b, n = [], 1
    while n <= cap:
        b.append(n)
        n *= 2
    if b[-1] != cap:
        b.append(cap)
    return b


class DraftGraphs:
    """``draft(ctx [B, C, H], k0 [B]) -> [B, ...]`` (the proposer's ``_draft_fn``) behind the ring,
    one captured graph per bucket.  ``kmax`` bounds the rows one request appends per step."""

    def __init__(self, ring, draft, kmax: int, buckets: list[int]):
        self.ring, self.draft, self.kmax = ring, draft, kmax
        self.buckets = sorted(buckets)
        self._g: dict[int, tuple] = {}

    def bucket_for(self, B: int):
        return next((b for b in self.buckets if b >= B), None)

    def _buffers(self, bkt: int):
        dev, H = self.ring.device, self.ring.H
        i32 = lambda: torch.zeros(bkt, dtype=torch.int32, device=dev)
        return dict(rows=i32(), starts=i32(), cnt=i32(), wmask=i32(),
                    k0=torch.zeros(bkt, dtype=torch.long, device=dev),
                    sh=torch.zeros(bkt * self.kmax, H, dtype=self.ring.dtype, device=dev),
                    ctx=torch.empty(bkt, self.ring.C, H, dtype=self.ring.dtype, device=dev))

    def _body(self, b):
        self.ring.step(b["sh"], b["rows"], b["starts"], b["cnt"], b["wmask"], kmax=self.kmax, out=b["ctx"])
        return self.draft(b["ctx"], b["k0"])

    def _capture(self, bkt: int):
        b = self._buffers(bkt)
        # warm up without appending anything (cnt = 0 leaves the ring as it is)
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            for _ in range(2):
                self._body(b)
        torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        # captured in inference mode whatever the caller's mode: torch's capture updates the CUDA
        # generator's graph state in place, and that state is an inference tensor once a capture
        # has run inside inference mode (the proposer's propose() captures there)
        with torch.inference_mode(), torch.cuda.graph(g):
            out = self._body(b)
        self._g[bkt] = (g, b, out)

    def run(self, sh: torch.Tensor, rows, starts, cnt, k0, wmask=None) -> torch.Tensor:
        """One step for B requests (B <= the largest bucket): rows / starts / cnt / k0 sequences or
        tensors of length B, sh [T, H] with every request's rows.  Returns the draft's [B, ...] rows
        of the bucket's output buffer (valid until the next run on the same bucket; an inference tensor,
        so clone it before updating it in place outside inference mode)."""
        B = len(rows)
        bkt = self.bucket_for(B)
        if bkt is None:
            raise ValueError(f"batch {B} is above the largest draft bucket {self.buckets[-1]}")
        if bkt not in self._g:
            self._capture(bkt)
        g, b, out = self._g[bkt]
        T = sh.shape[0]
        if T > b["sh"].shape[0]:
            raise ValueError(f"{T} hidden rows exceed the bucket's {b['sh'].shape[0]} (kmax {self.kmax})")
        dev = self.ring.device
        put = lambda name, v, fill: (b[name][:B].copy_(torch.as_tensor(v).to(dev, b[name].dtype)),
                                     b[name][B:].fill_(fill))
        put("rows", rows, int(torch.as_tensor(rows)[0]))    # padding rows read slot rows[0], append nothing
        put("starts", starts, 0)
        put("cnt", cnt, 0)
        put("wmask", torch.ones(B, dtype=torch.int32) if wmask is None else wmask, 0)
        put("k0", k0, int(torch.as_tensor(k0)[0]))
        b["sh"][:T].copy_(sh)
        g.replay()
        return out[:B]
