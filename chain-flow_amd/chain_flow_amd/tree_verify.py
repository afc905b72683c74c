"""Host side of the rest of the tree verify (the forked vLLM's tree arm) on the HIP kernels:

* ``tree_conv`` -- ``tree_scan_causal_conv1d`` (``cf/vllm_tree/tree_ssm.py:393-438``): the GDN
  layers' width-4 causal conv over the draft tree (bf16);
* ``tree_attn_merge`` -- the suffix half of ``_tree_attention_fixup`` plus the merge
  (``_tree_suffix_eager`` / ``fused_suffix_merge``, patch lines 403-575, 2793-3121): the tree rows'
  ancestor-masked attention merged into ``output`` with the prefix half by log-sum-exp;
* ``tree_greedy_accept`` -- ``tree_rejection_sample`` (patch lines 510-550): row argmax + greedy
  descent.
"""
from __future__ import annotations

import torch

from chain_flow_amd import _lib


def _i32(t, dev):
    return torch.as_tensor(t).to(dev, torch.int32).contiguous()


def _host(t):
    """The values of a host-side index argument (None for a device tensor: not read back)."""
    if isinstance(t, torch.Tensor):
        return None if t.is_cuda else t.cpu().numpy()
    import numpy as np
    return np.asarray(t)


# Every device tensor handed to a launch is kept in a local until the launch is queued: a temporary
# freed after .data_ptr() returns its block to the caching allocator, and the next temporary of
# the same size would then alias it.


def tree_conv(x, conv_state, weight, bias, node_slots, parent, *, prefix_slot: int = 1, activation="silu",
              out=None):
    """x [N, dim] bf16 (rows may be strided), conv_state [slots, dim, 4] bf16 (node slots written in
    place), weight [dim, 4] bf16, bias [dim] or None; parent [N] node indices (BFS, -1 = root).
    Returns out [N, dim] bf16."""
    if x.dtype != torch.bfloat16 or conv_state.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("tree_conv runs on bf16 tensors")
    N, dim = x.shape
    if x.stride(1) != 1 or conv_state.shape[1:] != (dim, 4) or not conv_state.is_contiguous():
        raise ValueError("x rows must be contiguous; conv_state [slots, dim, 4] contiguous")
    if activation not in ("silu", None, "none"):
        raise ValueError(f"activation {activation!r}")
    dev = x.device
    slots = conv_state.shape[0]
    hs, hp = _host(node_slots), _host(parent)
    if hs is not None and (len(hs) != N or hs.min() < 0 or hs.max() >= slots):
        raise ValueError(f"node_slots must be {N} slots in [0, {slots})")
    if hp is not None and (len(hp) != N or any(not (-1 <= int(hp[i]) < i) for i in range(N))):
        raise ValueError("parent[i] must be -1 or an earlier node (BFS order)")
    if not 0 <= prefix_slot < slots:
        raise ValueError(f"prefix_slot {prefix_slot} outside [0, {slots})")
    if out is None:
        out = torch.empty(N, dim, dtype=torch.bfloat16, device=dev)
    w = weight.contiguous()
    b = None if bias is None else bias.contiguous()
    ns, par = _i32(node_slots, dev), _i32(parent, dev)
    _lib.check(_lib.lib().cfh_tree_conv(
        x.data_ptr(), x.stride(0), conv_state.data_ptr(), w.data_ptr(), _lib.ptr(b), ns.data_ptr(),
        par.data_ptr(), prefix_slot, N, dim, 1 if activation == "silu" else 0, out.data_ptr(), out.stride(0),
        _lib.stream_handle()), "cfh_tree_conv")
    return out


def tree_attn_merge(query, key, value, output, prefix_out, prefix_lse, idx_pad, not_anc, scale: float):
    """query/key/value/output [T, heads, D] (bf16 or fp16, head dims contiguous), prefix_out
    [S*N, H, D], prefix_lse [H, S*N] fp32, idx_pad [S, N] forward rows of the tree nodes, not_anc
    [S, N, N] bool.  Writes the merged tree rows into ``output`` in place."""
    S, N = idx_pad.shape
    T, H, D = query.shape
    Hkv = key.shape[1]
    dt = query.dtype
    if dt not in (torch.bfloat16, torch.float16) or any(t.dtype != dt for t in (key, value, output, prefix_out)):
        raise ValueError("q/k/v/output/prefix_out must share one 2-byte dtype")
    for t in (query, key, value, output):
        if t.stride(2) != 1 or t.stride(1) != D:
            raise ValueError("head rows must be [.][heads][D] with contiguous heads")
    dev = query.device
    if prefix_out.shape != (S * N, H, D) or prefix_lse.shape != (H, S * N) or tuple(not_anc.shape) != (S, N, N):
        raise ValueError("prefix_out [S*N, H, D], prefix_lse [H, S*N], not_anc [S, N, N]")
    hi = _host(idx_pad)
    if hi is not None and (hi.min() < 0 or hi.max() >= min(T, key.shape[0], value.shape[0], output.shape[0])):
        raise ValueError("idx_pad rows outside the q/k/v/output rows")
    pout = prefix_out.contiguous()
    plse = prefix_lse.to(torch.float32).contiguous()
    idx = _i32(idx_pad, dev)
    mask = torch.as_tensor(not_anc).to(dev, torch.uint8).contiguous()
    _lib.check(_lib.lib().cfh_tree_attn_merge(
        query.data_ptr(), query.stride(0), key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
        output.data_ptr(), output.stride(0), pout.data_ptr(), plse.data_ptr(), idx.data_ptr(), mask.data_ptr(),
        float(scale), S, N, H, Hkv, D, 1 if dt == torch.bfloat16 else 0, _lib.stream_handle()),
        "cfh_tree_attn_merge")
    return output


def tree_greedy_accept(logits, cu_num_draft_tokens, cu_num_sampled_tokens, draft_token_ids, tree_parents,
                       max_spec_len: int):
    """logits [rows, V] (bf16 / fp16); cumulative (inclusive) per-request draft and row counts;
    draft ids and local parents (-1 = root) per draft token.  Returns (output_token_ids [B,
    max_spec_len + 1] int32, -1 padded; accepted_path [B, max_spec_len]; accepted_len [B])."""
    if logits.dtype not in (torch.bfloat16, torch.float16) or logits.stride(1) != 1:
        raise ValueError("logits must be bf16 / fp16 with contiguous rows")
    dev = logits.device
    B = len(cu_num_draft_tokens)
    R, V = logits.shape
    out = torch.empty(B, max_spec_len + 1, dtype=torch.int32, device=dev)
    path = torch.empty(B, max(max_spec_len, 1), dtype=torch.int32, device=dev)
    ln = torch.empty(B, dtype=torch.int32, device=dev)
    ra = torch.empty(R, dtype=torch.int32, device=dev)
    ws = torch.empty(int(_lib.lib().cfh_tree_accept_ws_bytes(R)), dtype=torch.uint8, device=dev)
    cd, cs = _host(cu_num_draft_tokens), _host(cu_num_sampled_tokens)
    if cd is not None and cs is not None:
        import numpy as np
        nd = np.diff(np.concatenate([[0], cd]))
        if (nd < 0).any() or nd.max(initial=0) > max_spec_len or int(cs[-1]) > R or \
                not np.array_equal(np.diff(np.concatenate([[0], cs])), nd + 1) or int(cd[-1]) > len(draft_token_ids):
            raise ValueError("cumulative draft / row counts inconsistent with the logits rows and max_spec_len")
    draft = _i32(draft_token_ids, dev) if len(draft_token_ids) else torch.zeros(1, dtype=torch.int32, device=dev)
    par = _i32(tree_parents, dev) if len(tree_parents) else torch.zeros(1, dtype=torch.int32, device=dev)
    cdg, csg = _i32(cu_num_draft_tokens, dev), _i32(cu_num_sampled_tokens, dev)
    _lib.check(_lib.lib().cfh_tree_greedy_accept(
        logits.data_ptr(), logits.stride(0), V, R, 1 if logits.dtype == torch.bfloat16 else 0, cdg.data_ptr(),
        csg.data_ptr(), draft.data_ptr(), par.data_ptr(), B, max_spec_len, out.data_ptr(), path.data_ptr(),
        ln.data_ptr(), ra.data_ptr(), ws.data_ptr(), _lib.stream_handle()), "cfh_tree_greedy_accept")
    return out, path[:, :max_spec_len], ln
