"""Host side of the hidden-state VAE: weight packing, ``encode`` (mu) and ``decode`` through libcfhip.

Mirrors the frozen ``TransformerHiddenVAE`` inside ``TreeVAEFlowDrafter``
(``cf/drafters/tree_vae_flow.py:50-87, 163-169``; module ``cf/vae/transformer_hidden.py:9-79``):
``encode`` is ``encode_sequence(hidden).mu`` and ``decode`` is ``decode_sequence(z)``, each one call
on the current stream into caller-visible buffers.  ``load_vae_dir`` is ``_load_frozen_vae``'s
checkpoint resolution (``CF_VAE_DIR`` over the config's ``vae_dir``, ``model.safetensors`` or the
newest ``checkpoint-N/model.safetensors``) with the same error text.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch

from chain_flow_amd import _lib
from chain_flow_amd.config import TreeVAEFlowConfig
from chain_flow_amd.weights import vae_param_names


def vae_dims(cfg: TreeVAEFlowConfig, hidden_size: int) -> _lib.VaeDims:
    return _lib.VaeDims(hidden_size, cfg.latent_size, cfg.vae_intermediate_size, cfg.vae_num_layers,
                        cfg.vae_heads, cfg.vae_max_sequence_length)


def vae_caps(cfg: TreeVAEFlowConfig, hidden_size: int, rows: int):
    """Workspace bytes if the build runs this VAE on sequences of ``rows`` rows, else None."""
    ws = C.c_int64(0)
    dims = vae_dims(cfg, hidden_size)
    rc = _lib.lib().cfh_vae_caps(C.byref(dims), rows, C.byref(ws))
    return int(ws.value) if rc == 0 else None


def load_vae_dir(cfg: TreeVAEFlowConfig) -> dict | None:
    """The VAE's own checkpoint as drafter-level names (``vae.`` prefix), or None when neither
    ``CF_VAE_DIR`` nor ``cfg.vae_dir`` is set (``cf/drafters/tree_vae_flow.py:57-87``)."""
    override = os.environ.get("CF_VAE_DIR")
    if not (override or cfg.vae_dir):
        return None
    from safetensors.torch import load_file
    d = Path(override or cfg.vae_dir)
    sp = d / "model.safetensors"
    if not sp.exists():
        cks = sorted(d.glob("checkpoint-*"), key=lambda p: int(p.name.split("-")[-1])) if d.is_dir() else []
        if not cks:
            src = "CF_VAE_DIR" if override else "vae_dir in the checkpoint config"
            raise FileNotFoundError(
                f"VAE not found for the drafter.\n"
                f"  looked in : {d}   (from {src})\n"
                f"  expected  : {d / 'model.safetensors'}, or a checkpoint-N/model.safetensors under it\n"
                f"  exists    : {'yes, but neither of the above is in it' if d.is_dir() else 'no -- the directory itself is missing'}\n"
                f"  fix       : set CF_VAE_DIR to a directory holding the VAE for this drafter.")
        sp = cks[-1] / "model.safetensors"
    sd = load_file(str(sp), device="cpu")
    vsd = {k[len("vae."):]: v for k, v in sd.items() if k.startswith("vae.")} or sd
    return {"vae." + k: v for k, v in vsd.items()}


class HiddenVAE:
    """Packed VAE image + per-row-count workspaces on one device."""

    def __init__(self, cfg: TreeVAEFlowConfig, hidden_size: int, weights: dict, device="cuda"):
        if cfg.vae_type != "transformer_hidden":
            raise ValueError(f"vae_type {cfg.vae_type!r} is not built (this build runs the "
                             f"'transformer_hidden' VAE of the shipped drafters)")
        self.cfg = cfg
        self.hidden = hidden_size
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.dims = vae_dims(cfg, hidden_size)
        L = _lib.lib()
        nbytes = int(L.cfh_vae_bytes(C.byref(self.dims)))
        if nbytes < 0:
            raise ValueError(f"VAE shape not supported by libcfhip: hidden={hidden_size} "
                             f"latent={cfg.latent_size} inter={cfg.vae_intermediate_size} "
                             f"heads={cfg.vae_heads}")
        names = vae_param_names(cfg)
        missing = [n for n in names if n not in weights]
        if missing:
            raise KeyError(f"VAE weights missing: {missing[:4]}{' ...' if len(missing) > 4 else ''}")
        raw = [weights[n].to(self.device, torch.float16).contiguous() for n in names]
        self.packed = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        arr = _lib.ptr_array([t.data_ptr() for t in raw])
        _lib.check(L.cfh_vae_pack(C.byref(self.dims), arr, len(raw), self.packed.data_ptr(),
                                  _lib.stream_handle()), "cfh_vae_pack")
        torch.cuda.current_stream().synchronize()   # raw copies may be freed after this
        self._ws: dict[int, torch.Tensor] = {}

    def _workspace(self, rows: int) -> torch.Tensor:
        ws = self._ws.get(rows)
        if ws is None:
            n = vae_caps(self.cfg, self.hidden, rows)
            if n is None:
                raise ValueError(f"VAE sequences of {rows} rows are not supported "
                                 f"(max_sequence_length={self.cfg.vae_max_sequence_length}, build limit 16)")
            ws = self._ws[rows] = torch.empty(n, dtype=torch.uint8, device=self.device)
        return ws

    def _run(self, fn, x: torch.Tensor, width_in: int, width_out: int, out, what: str) -> torch.Tensor:
        if x.dim() != 3 or x.shape[2] != width_in:
            raise ValueError(f"{what} input must be [B, L, {width_in}], got {tuple(x.shape)}")
        x = x.to(self.device, torch.float16).contiguous()
        B, T = x.shape[0], x.shape[1]
        if out is None:
            out = torch.empty(B, T, width_out, dtype=torch.float16, device=self.device)
        ws = self._workspace(T)
        _lib.check(fn(C.byref(self.dims), self.packed.data_ptr(), x.data_ptr(), out.data_ptr(), B, T,
                      ws.data_ptr(), _lib.stream_handle()), what)
        return out

    def encode(self, hidden: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """``encode_sequence(hidden).mu``: [B, L, hidden] -> [B, L, latent] fp16."""
        return self._run(_lib.lib().cfh_vae_encode, hidden, self.hidden, self.cfg.latent_size, out,
                         "cfh_vae_encode")

    def decode(self, z: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """``decode_sequence(z)``: [B, L, latent] -> [B, L, hidden] fp16."""
        return self._run(_lib.lib().cfh_vae_decode, z, self.cfg.latent_size, self.hidden, out,
                         "cfh_vae_decode")
