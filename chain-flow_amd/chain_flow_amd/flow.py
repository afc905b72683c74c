"""Host side of the fused flow: weight packing and ``predict_hidden`` through libcfhip.

A batch is drafted in groups of requests whose rows share each weight stream (two 8-row drafts per
16-row MFMA tile where the shape allows), so a batch of B costs about B/2 single drafts.

Mirrors the reference's boundary ``cuda_block.FusedExpertBlocks`` (``cf/cuda_block.py:269-431``):
the caller owns packed weights and a workspace that persist across drafts; one call runs the
whole ``TreeFlowDrafter.predict_hidden`` (``cf/drafters/tree_flow.py:229-244``) -- init_latents
and every Euler step of every chunk expert -- on the current stream.
"""
from __future__ import annotations

import ctypes as C
import os

import torch

from chain_flow_amd import _lib
from chain_flow_amd.config import TreeFlowConfig
from chain_flow_amd.head import pack_linear
from chain_flow_amd.weights import anchor_param_names, expert_param_names, expert_prefixes


# the shapes the reference's fused block kernel is built for (cf/cuda_block.py:46-51)
_FUSED_D, _FUSED_FM, _FUSED_HEADS, _FUSED_S, _FUSED_MAX_C = (640, 1024), (6,), 8, (4, 8), 16


def reference_numerics(cfg: TreeFlowConfig, batch: int = 1) -> int:
    """The fp16 numerics the reference runs this flow in: its fused block kernel
    (``_lib.FLOW_FUSED``) when ``cuda_block.supported`` takes every chunk expert's shape and the
    batch is 1 or ``CF_CUDA_BLOCK_BATCH`` is set (``cf/cuda_block.py:95-117, 474-481``,
    ``cf/drafters/chunked_flow.py:295-331``), else torch's fp16 modules (``_lib.FLOW_MODULES``), as
    also with ``CF_CUDA_BLOCK=0``."""
    off = ("0", "", "false", "False")
    if os.environ.get("CF_CUDA_BLOCK", "1") in off:                  # the reference's kill switch
        return _lib.FLOW_MODULES
    batch_ok = batch == 1 or os.environ.get("CF_CUDA_BLOCK_BATCH", "0") not in off
    rows = [(c + 1) * cfg.chunk_size for c in range(cfg.draft_length // cfg.chunk_size)]
    fused = (cfg.flow_dim in _FUSED_D and cfg.ffn_multiplier in _FUSED_FM and cfg.num_heads == _FUSED_HEADS
             and all(s in _FUSED_S for s in rows) and 0 < cfg.context_size <= _FUSED_MAX_C and batch_ok)
    return _lib.FLOW_FUSED if fused else _lib.FLOW_MODULES


# init_latents modes (cf/drafters/tree_flow.py:150-161) -> cfh_flow_dims.init_mode; "noise" draws
# z0 here with torch's generator, as the reference does, and hands it over through z_out
_INIT = {"delta": _lib.INIT_DELTA, "repeat_last": _lib.INIT_REPEAT_LAST, "noise": _lib.INIT_GIVEN}


def flow_dims(cfg: TreeFlowConfig, numerics: int | None = None) -> _lib.FlowDims:
    """cfh_flow_dims of ``cfg``; ``numerics`` defaults to the reference's at batch 1."""
    num = reference_numerics(cfg) if numerics is None else int(numerics)
    return _lib.FlowDims(cfg.flow_dim, cfg.ffn_multiplier, cfg.num_heads, cfg.num_drafter_layers,
                         cfg.context_size, cfg.draft_length, cfg.chunk_size, cfg.num_flow_steps, num,
                         _INIT[cfg.init_mode])


def caps(cfg: TreeFlowConfig, batch: int = 1):
    """Workspace bytes if the build supports this flow shape, else None."""
    ws = C.c_int64(0)
    dims = flow_dims(cfg)
    rc = _lib.lib().cfh_caps(C.byref(dims), batch, C.byref(ws))
    return int(ws.value) if rc == 0 else None


def group_size(cfg: TreeFlowConfig, batch: int) -> int:
    """Requests per group that share every weight stream when ``batch`` requests are drafted."""
    r = C.c_int(0)
    rc = _lib.lib().cfh_flow_group_size(C.byref(flow_dims(cfg)), int(batch), C.byref(r))
    if rc != 0:
        raise ValueError(f"flow shape not supported by libcfhip at batch {batch}: {cfg}")
    return int(r.value)


def plan_flags(cfg: TreeFlowConfig, batch: int = 1) -> int:
    """The launch forms the flow uses for ``batch`` requests (``_lib.PLAN_*`` bits; cfh_flow_plan)."""
    f = C.c_int(0)
    rc = _lib.lib().cfh_flow_plan(C.byref(flow_dims(cfg)), int(batch), C.byref(f))
    if rc != 0:
        raise ValueError(f"flow shape not supported by libcfhip at batch {batch}: {cfg}")
    return int(f.value)


class FusedFlow:
    """Packed chunk experts + workspace for one drafter on one device."""

    def __init__(self, cfg: TreeFlowConfig, weights: dict, device="cuda", max_batch: int = 256):
        self.cfg = cfg
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.dims = flow_dims(cfg)
        L = _lib.lib()
        if caps(cfg, 1) is None:
            raise ValueError(f"flow shape not supported by libcfhip: {cfg}")
        dz = cfg.flow_dim
        for n in anchor_param_names(cfg):
            want = (dz,) if n.endswith(".bias") else (dz, dz) if "anchor_mlp" in n else (dz, None)
            got = tuple(weights[n].shape)
            if len(got) != len(want) or any(w is not None and w != g for w, g in zip(want, got)):
                # (the reference's anchor_in projects to expert_dim, which must equal latent_size)
                raise ValueError(f"{n} has shape {got}; the anchored latent drafter needs "
                                 f"{tuple('hidden' if w is None else w for w in want)} (latent_size {dz})")
        # One workspace for every batch up to max_batch (the largest request group's), allocated
        # once: a captured draft graph holds its address, so it is never swapped or freed.
        ws = caps(cfg, max(1, int(max_batch)))
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
        self._retired = []   # outgrown buffers, kept alive for graphs that may still use them
        # the anchored latent drafter (anchor_token): anchor_in + each expert's anchor_mlp, matrices
        # packed, in cfh_flow_anchor's order
        self.anchor_params = []
        self.anchor_hidden = 0
        names = anchor_param_names(cfg)
        if names:
            for n in names:
                t = weights[n].to(self.device, torch.float16).contiguous()
                self.anchor_params.append(pack_linear(t) if t.dim() == 2 else t)
            self.anchor_hidden = int(weights["anchor_in.weight"].shape[1])
            self._anchor_w = _lib.ptr_array([t.data_ptr() for t in self.anchor_params])
            nws = int(L.cfh_flow_anchor_ws_bytes(C.byref(self.dims), self.anchor_hidden))
            if nws < 0:
                raise ValueError(f"anchor shape not supported by libcfhip: hidden={self.anchor_hidden}")
            self.anchor_ws = torch.empty(nws, dtype=torch.uint8, device=self.device)
            # one buffer for every batch up to max_batch (a captured draft graph holds its address)
            nch = cfg.draft_length // cfg.chunk_size
            self._anchor_buf = torch.empty(nch * max(1, int(max_batch)) * cfg.flow_dim, dtype=torch.float16,
                                           device=self.device)
        self.ws = torch.empty(ws, dtype=torch.uint8, device=self.device)
        self.concurrent = self.prepare_streams()

    def prepare_streams(self, stream=None) -> bool:
        """Creates the companion streams of ``stream`` (default: the current one) and runs their
        one-time overlap check now, so that no later ``predict_hidden`` on it synchronises
        (``cfh_flow_prepare_streams``).  True if the chunk experts will run concurrently."""
        if self.device.type != "cuda" or torch.cuda.is_current_stream_capturing():
            return False
        conc = C.c_int(0)
        _lib.check(_lib.lib().cfh_flow_prepare_streams(C.byref(self.dims), _lib.stream_handle(stream),
                                                       C.byref(conc)), "cfh_flow_prepare_streams")
        return bool(conc.value)

    @property
    def weight_bytes(self) -> int:
        return sum(b.numel() for b in self.packed)

    def anchor(self, tokens: torch.Tensor, embed_w: torch.Tensor) -> torch.Tensor:
        """The anchored drafter's per-expert anchor rows [n_chunks, B, d] fp16 for the committed
        tokens [B] (``anchor_embed`` then each expert's ``anchor_mlp``, cf/drafters/tree_flow.py:237-241,
        cf/drafters/chunked_flow.py:256-262; ``cfh_flow_anchor``).  embed_w: the LM's input embedding
        table [V, hidden] fp16 on the flow's device.  A token below 0 reads row 0."""
        if not self.anchor_params:
            raise ValueError("this drafter has no anchor_token parameters")
        cfg = self.cfg
        if embed_w.dtype != torch.float16 or embed_w.device != self.device or embed_w.dim() != 2 \
                or embed_w.shape[1] != self.anchor_hidden:
            raise ValueError(f"embed_w must be [V, {self.anchor_hidden}] fp16 on the flow's device")
        tok = tokens.reshape(-1).to(self.device, torch.int32).contiguous()
        B = tok.numel()
        nch = cfg.draft_length // cfg.chunk_size
        n = nch * B * cfg.flow_dim
        if n > self._anchor_buf.numel():
            # (a batch above max_batch: the old buffer stays referenced, never freed)
            self._retired.append(self._anchor_buf)
            self._anchor_buf = torch.empty(n, dtype=torch.float16, device=self.device)
        rows = self._anchor_buf[:n].view(nch, B, cfg.flow_dim)
        _lib.check(_lib.lib().cfh_flow_anchor(C.byref(self.dims), self.anchor_hidden, self._anchor_w,
                                              embed_w.contiguous().data_ptr(), tok.data_ptr(), B,
                                              rows.data_ptr(), self.anchor_ws.data_ptr(),
                                              _lib.stream_handle()), "cfh_flow_anchor")
        return rows

    def predict_hidden(self, ctx: torch.Tensor, out: torch.Tensor | None = None,
                       numerics: int | None = None, anchor: torch.Tensor | None = None) -> torch.Tensor:
        """ctx [B, context_size, d] fp16 (already front-padded; d = cfg.flow_dim) -> [B, draft_length, d]
        fp16, in the numerics the reference uses for this shape and batch (``reference_numerics``)
        unless ``numerics`` names one.  With ``init_mode="noise"`` the initial latents are
        ``torch.randn(B, draft_length, d, fp16) * noise_scale`` from torch's current generator on
        the flow's device (``init_latents``, cf/drafters/tree_flow.py:154-155), written into ``out``
        before the call.  ``anchor``: the anchor rows of ``anchor()`` [n_chunks, B, d], added to
        every row of every block (cf/drafters/chunked_flow.py:376), or None."""
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
        # a batch runs in groups of requests packed into one tile: its workspace grows with the group
        need = caps(cfg, B)
        if need is None:
            raise ValueError(f"flow shape not supported by libcfhip at batch {B}: {cfg}")
        if need > self.ws.numel():
            # (a batch above max_batch: the old workspace stays referenced, never freed)
            self._retired.append(self.ws)
            self.ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        self.dims.numerics = reference_numerics(cfg, B) if numerics is None else int(numerics)
        if cfg.init_mode == "noise":
            out.copy_(torch.randn(B, cfg.draft_length, d, device=self.device, dtype=torch.float16) * cfg.noise_scale)
        if anchor is not None:
            nch = cfg.draft_length // cfg.chunk_size
            if tuple(anchor.shape) != (nch, B, d) or anchor.dtype != torch.float16 \
                    or anchor.device != self.device or not anchor.is_contiguous():
                raise ValueError(f"anchor must be contiguous [{nch}, {B}, {d}] fp16 on the flow's device")
            _lib.check(_lib.lib().cfh_flow_integrate_anchored(C.byref(self.dims), self._experts, ctx.data_ptr(),
                                                              anchor.data_ptr(), out.data_ptr(),
                                                              self.ws.data_ptr(), B, _lib.stream_handle()),
                       "cfh_flow_integrate_anchored")
            return out
        _lib.check(_lib.lib().cfh_flow_integrate(C.byref(self.dims), self._experts, ctx.data_ptr(),
                                                 out.data_ptr(), self.ws.data_ptr(), B,
                                                 _lib.stream_handle()),
                   "cfh_flow_integrate")
        return out
