"""Host side of the fused flow: weight packing and ``predict_hidden`` through libcfhip.

Mirrors the reference's boundary ``cuda_block.FusedExpertBlocks`` (``cf/cuda_block.py:269-431``):
the caller owns packed weights and a workspace that persist across drafts; one call runs the
whole ``TreeFlowDrafter.predict_hidden`` (``cf/drafters/tree_flow.py:229-244``) -- init_latents
and every Euler step of every chunk expert -- on the current stream.
"""
from __future__ import annotations

import ctypes as C

import torch

from chain_flow_amd import _lib
from chain_flow_amd.config import TreeFlowConfig
from chain_flow_amd.weights import expert_param_names, expert_prefixes


def flow_dims(cfg: TreeFlowConfig) -> _lib.FlowDims:
    return _lib.FlowDims(cfg.flow_dim, cfg.ffn_multiplier, cfg.num_heads, cfg.num_drafter_layers,
                         cfg.context_size, cfg.draft_length, cfg.chunk_size, cfg.num_flow_steps)


def caps(cfg: TreeFlowConfig, batch: int = 1):
    """Workspace bytes if the build supports this flow shape, else None."""
    ws = C.c_int64(0)
    dims = flow_dims(cfg)
    rc = _lib.lib().cfh_caps(C.byref(dims), batch, C.byref(ws))
    return int(ws.value) if rc == 0 else None


class FusedFlow:
    """Packed chunk experts + workspace for one drafter on one device."""

    def __init__(self, cfg: TreeFlowConfig, weights: dict, device="cuda"):
        if cfg.init_mode != "delta":
            raise ValueError("the fused flow implements init_mode='delta' (the drafter default)")
        self.cfg = cfg
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.dims = flow_dims(cfg)
        L = _lib.lib()
        ws = caps(cfg, 1)
        if ws is None:
            raise ValueError(f"flow shape not supported by libcfhip: {cfg}")
        nbytes = int(L.cfh_flow_expert_bytes(C.byref(self.dims)))
        self.packed = []
        stream = _lib.stream_handle()
        for p in expert_prefixes(cfg):
            names = expert_param_names(cfg, p)
            raw = [weights[n].to(self.device, torch.float16).contiguous() for n in names]
            buf = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            arr = _lib.ptr_array([t.data_ptr() for t in raw])
            _lib.check(L.cfh_flow_pack_expert(C.byref(self.dims), arr, len(raw), buf.data_ptr(), stream),
                       "cfh_flow_pack_expert")
            torch.cuda.current_stream().synchronize()   # raw copies may be freed after this
            self.packed.append(buf)
        self._experts = _lib.ptr_array([b.data_ptr() for b in self.packed])
        self.ws = torch.empty(ws, dtype=torch.uint8, device=self.device)

    @property
    def weight_bytes(self) -> int:
        return sum(b.numel() for b in self.packed)

    def predict_hidden(self, ctx: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """ctx [B, context_size, d] fp16 (already front-padded; d = cfg.flow_dim) -> [B, draft_length, d]
        fp16."""
        cfg = self.cfg
        d = cfg.flow_dim
        if ctx.dim() != 3 or ctx.shape[1] != cfg.context_size or ctx.shape[2] != d:
            raise ValueError(f"ctx must be [B, {cfg.context_size}, {d}], got {tuple(ctx.shape)}")
        if ctx.dtype != torch.float16 or ctx.device != self.device:
            raise ValueError("ctx must be fp16 on the flow's device")
        ctx = ctx.contiguous()
        B = ctx.shape[0]
        if out is None:
            out = torch.empty(B, cfg.draft_length, d, dtype=torch.float16, device=self.device)
        _lib.check(_lib.lib().cfh_flow_integrate(C.byref(self.dims), self._experts, ctx.data_ptr(),
                                                 out.data_ptr(), self.ws.data_ptr(), B,
                                                 _lib.stream_handle()),
                   "cfh_flow_integrate")
        return out
