"""Host side of the context ring: ``FlowDrafterProposer``'s per-slot history of target hidden states
on the device (``_init_ring`` / ``_ring_write`` / ``_ring_gather``,
``cf/vllm_plugin/flow_proposer.py:916-961``), stepped by ``cfh_ring_step``.

Slot lifecycle (``:2045-2105``): a new request in a slot starts empty (``reset``) or from prompt
hiddens (``seed``); a live request that moved slot (vLLM's batch condense) carries its history
(``migrate``).
"""
from __future__ import annotations

import torch

from chain_flow_amd import _lib


def _i32(t, dev):
    return torch.as_tensor(t, dtype=torch.int32).to(dev).contiguous()


class ContextRing:
    def __init__(self, slots: int, ctx_size: int, hidden: int, device="cuda", dtype=torch.float16):
        if hidden % 8:
            raise ValueError("hidden size must be a multiple of 8")
        self.C, self.H, self.slots = ctx_size, hidden, slots
        self.device = torch.device(device)
        self.dtype = dtype
        self.ring = torch.zeros(slots, ctx_size + 1, hidden, dtype=dtype, device=self.device)
        self.rpos = torch.zeros(slots, dtype=torch.int32, device=self.device)
        self.nval = torch.zeros(slots, dtype=torch.int32, device=self.device)

    def reset(self, slots) -> None:
        idx = _i32(slots, self.device).long()
        self.rpos.index_fill_(0, idx, 0)
        self.nval.index_fill_(0, idx, 0)

    def seed(self, slot: int, hist: torch.Tensor) -> None:
        """Start slot from the last min(n, C) rows of ``hist`` [n, H] (prompt hiddens)."""
        L = min(int(hist.shape[0]), self.C)
        self.ring[slot, :L].copy_(hist[-L:].to(self.dtype))
        self.rpos[slot] = L % self.C
        self.nval[slot] = L

    def migrate(self, moves) -> None:
        """moves: [(new_slot, old_slot)], applied from a snapshot (two requests may swap)."""
        if not moves:
            return
        snap, sp, sn = self.ring.clone(), self.rpos.clone(), self.nval.clone()
        new = torch.tensor([m[0] for m in moves], device=self.device)
        old = torch.tensor([m[1] for m in moves], device=self.device)
        self.ring.index_copy_(0, new, snap.index_select(0, old))
        self.rpos.index_copy_(0, new, sp.index_select(0, old))
        self.nval.index_copy_(0, new, sn.index_select(0, old))

    def step(self, sh, rows, starts=None, cnt=None, wmask=None, path=None, kmax=None, out=None):
        """Append this step's rows of ``sh`` [T, H] to each request's slot and return the windows
        [B, C, H] (``cnt`` None: read only).  rows / starts / cnt / wmask are int32 device tensors
        (or sequences), path [slots, >= kmax-1] int32 (tree: accepted node per depth) or None."""
        dev = self.device
        rows = _i32(rows, dev)
        B = rows.numel()
        if out is None:
            out = torch.empty(B, self.C, self.H, dtype=self.dtype, device=dev)
        if cnt is not None:
            starts, cnt = _i32(starts, dev), _i32(cnt, dev)
            if kmax is None:
                raise ValueError("kmax (the most rows one request appends) is required with cnt")
            if sh.dtype != self.dtype or sh.shape[-1] != self.H:
                raise ValueError(f"sh must be [T, {self.H}] {self.dtype}")
            sh = sh.contiguous()
        wm = None if wmask is None else _i32(wmask, dev)
        pth = None if path is None else _i32(path, dev)
        _lib.check(_lib.lib().cfh_ring_step(
            self.ring.data_ptr(), self.rpos.data_ptr(), self.nval.data_ptr(), self.C, self.H,
            _lib.ptr(sh) if cnt is not None else None, sh.shape[0] if cnt is not None else 0,
            rows.data_ptr(), _lib.ptr(starts) if cnt is not None else None,
            _lib.ptr(cnt) if cnt is not None else None, _lib.ptr(wm), _lib.ptr(pth),
            pth.shape[1] if pth is not None else 0, kmax or 0, B, out.data_ptr(), _lib.stream_handle()),
            "cfh_ring_step")
        return out
