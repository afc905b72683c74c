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


def tree_gdn_vllm(mixed_qkv, a, b, A_log, dt_bias, ssm_state, node_slots, parent, *, num_q_heads: int,
                  prefix_slot: int = 1, scale: float | None = None, use_qk_l2norm: bool = True,
                  status: torch.Tensor | None = None):
    """The serving form of the tree GDN (``tree_scan_gdn_recurrence_path``,
    ``cf/vllm_tree/tree_ssm.py:256-351``; bit-identical by construction to the per-node slot form
    ``:34-96``): one launch of ``cfh_gdn_tree_vllm``, with no host synchronisation (a verify step
    of many layers can be captured in one graph).

    mixed_qkv [N, 2 H K + HV V] bf16 (q heads | k heads | value heads), a, b [N, HV] bf16, A_log,
    dt_bias [HV], ssm_state [slots, HV, V, K] bf16 or fp32 (updated in place: node n's state goes to
    slot node_slots[n]; every node starts from slot ``prefix_slot``), parent [N] (BFS, -1 = root).
    -> o [N, HV, V] bf16.  The node slots are checked on the device: a node whose slot lies outside
    ssm_state, equals the prefix slot or repeats another node's gets NaN outputs and writes no
    slot, and ``status`` (int32 [1] on the device, zeroed by the caller), if given, is set to 1."""
    N, conv = mixed_qkv.shape
    nslots, HV, V, K = ssm_state.shape
    H = int(num_q_heads)
    if conv != 2 * H * K + HV * V:
        raise ValueError(f"mixed_qkv width {conv} != 2*{H}*{K} + {HV}*{V}")
    if mixed_qkv.dtype != torch.bfloat16 or a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise ValueError("mixed_qkv, a, b must be bf16")
    if ssm_state.dtype not in (torch.bfloat16, torch.float32) or not ssm_state.is_contiguous():
        raise ValueError("ssm_state must be a contiguous bf16 or fp32 [slots, HV, V, K] tensor")
    if a.shape != (N, HV) or b.shape != (N, HV) or node_slots.numel() != N:
        raise ValueError("a, b must be [N, HV] and node_slots [N]")
    if not 0 <= int(prefix_slot) < nslots:
        raise ValueError(f"prefix slot {prefix_slot} is outside ssm_state's {nslots} slots")
    if status is not None and (status.dtype != torch.int32 or status.device != mixed_qkv.device):
        raise ValueError("status must be an int32 tensor on the GDN's device")
    dev = mixed_qkv.device
    slots = node_slots.to(dev, torch.int32).contiguous()
    x, a, b = mixed_qkv.contiguous(), a.contiguous(), b.contiguous()
    A_log = A_log.to(dev, torch.float32).contiguous()
    dt_bias = dt_bias.to(dev, torch.float32).contiguous()
    parent = parent.to(dev, torch.int32).contiguous()
    out = torch.empty(N, HV, V, dtype=torch.bfloat16, device=dev)
    _lib.check(_lib.lib().cfh_gdn_tree_vllm(
        x.data_ptr(), a.data_ptr(), b.data_ptr(), A_log.data_ptr(), dt_bias.data_ptr(), ssm_state.data_ptr(),
        int(ssm_state.dtype == torch.bfloat16), nslots, slots.data_ptr(), parent.data_ptr(), int(prefix_slot), N,
        H, HV, K, V, int(bool(use_qk_l2norm)), float(K ** -0.5 if scale is None else scale), out.data_ptr(),
        _lib.ptr(status), _lib.stream_handle()), "cfh_gdn_tree_vllm")
    return out
