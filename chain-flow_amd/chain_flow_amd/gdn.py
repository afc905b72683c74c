"""Host side of the tree gated delta net (GDN) state update used in tree verification.

Mirrors ``tree_gated_delta_scan`` (``cf/kernels/tree_scan.py:41-73``): every node of a BFS-ordered
draft tree (``parent[n] < n``, -1 = root) applies the gated delta rule to its parent's state (roots
to the committed prefix's state ``S0``); outputs ``o = S^T q`` per node and, optionally, every
node's state.  One launch of libcfhip's ``cfh_gdn_tree`` on the current stream.
"""
from __future__ import annotations

import torch

from chain_flow_amd import _lib

L2_NORM_EPS = 0        # x / (|x| + 1e-6), cf/kernels/tree_scan.py:23-24
L2_SQRT_EPS = 1        # x / sqrt(|x|^2 + 1e-6), cf/vllm_tree/tree_ssm.py:60-62


def tree_gated_delta_scan(q, k, v, g, beta, parent, S0, *, use_qk_l2norm: bool = True,
                          l2mode: int = L2_NORM_EPS, write_states: bool = True):
    """q, k [N, H, Dk] bf16; v [N, H, Dv] bf16; g, beta [N, H] (log decay, update rate);
    parent [N] int (BFS order, -1 = root); S0 [H, Dk, Dv] fp32.
    -> (out [N, H, Dv] fp32, states [N, H, Dk, Dv] fp32 or None)."""
    N, H, Dk = q.shape
    Dv = v.shape[-1]
    dev = q.device
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("q, k, v must be device tensors")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("q, k, v must be bf16")
    if k.shape != q.shape or v.shape[:2] != (N, H) or g.shape != (N, H) or beta.shape != (N, H):
        raise ValueError("shape mismatch among q, k, v, g, beta")
    if S0.shape != (H, Dk, Dv):
        raise ValueError(f"S0 must be [{H}, {Dk}, {Dv}]")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    g = g.to(dev, torch.float32).contiguous()
    beta = beta.to(dev, torch.float32).contiguous()
    S0 = S0.to(dev, torch.float32).contiguous()
    parent = parent.to(dev, torch.int32).contiguous()
    out = torch.empty(N, H, Dv, dtype=torch.float32, device=dev)
    states = torch.empty(N, H, Dk, Dv, dtype=torch.float32, device=dev) if write_states else None
    _lib.check(_lib.lib().cfh_gdn_tree(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
                                       S0.data_ptr(), parent.data_ptr(), N, H, Dk, Dv, int(bool(use_qk_l2norm)),
                                       int(l2mode), out.data_ptr(), _lib.ptr(states), _lib.stream_handle()),
               "cfh_gdn_tree")
    return out, states
