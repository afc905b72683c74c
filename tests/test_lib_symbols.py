"""libcfhip.so loads and exports every entry point include/cfhip.h declares (no GPU calls)."""
from __future__ import annotations

import re
from pathlib import Path

from chain_flow_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "cfhip.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(cfh_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert set(declared()) == set(_lib.SIGNATURES), set(declared()) ^ set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    assert _lib.LIB_PATH.exists(), "build libcfhip.so first (python chain-flow_amd/csrc/build.py)"
    assert _lib.missing_symbols() == []


def test_status_strings_without_a_device():
    L = _lib.lib()
    assert L.cfh_version() >= 100
    assert L.cfh_error_string(0) == b"ok"
    assert L.cfh_error_string(2) == b"unsupported shape"


def test_candidate_select_argument_checks_without_a_device():
    """cfh_cand_topm's host-side checks return before any launch: keys rows padded to 4 columns
    plus each 1024-column block's AND/OR masks, a 16-byte aligned workspace, widths up to 262,144
    columns."""
    L = _lib.lib()
    assert L.cfh_cand_ws_bytes(2, 5) == 2 * 8 * 4 + 2 * 1 * 8            # keys + one block's AND/OR
    assert L.cfh_cand_ws_bytes(3, 62642) == 3 * 62644 * 4 + 3 * 62 * 8
    p = 4096   # stand-in addresses: never dereferenced, the checks fail first
    # (logits, ld, lse, B, n, Vs, M, sl, cand_local, cand_global, ws, stream)
    assert L.cfh_cand_topm(p, 1003, p, 3, 5, 1001, 77, None, p, None, p + 8, None) == 1      # misaligned ws
    assert L.cfh_cand_topm(p, 1003, p, 3, 5, 1001, 1002, None, p, None, p, None) == 1       # M > Vs
    assert L.cfh_cand_topm(p, 1000, p, 3, 5, 1001, 77, None, p, None, p, None) == 1         # ld < Vs
    assert L.cfh_cand_topm(p, 262145, p, 1, 1, 262145, 8, None, p, None, p, None) == 2      # too wide
    assert L.cfh_cand_topm(p, 1003, p, 0, 5, 1001, 77, None, p, None, p, None) == 0         # nothing to do


def test_merged_topk_beam_argument_checks_without_a_device():
    """cfh_head_topk_packed_beam_chain returns before any launch when the rows are not B x W beams,
    the chain's W x W candidates exceed one wave, the markov order is outside 1..8 or a search-state
    pointer is missing."""
    L = _lib.lib()
    p = 4096   # stand-in addresses: never dereferenced, the checks fail first

    def call(M=8, B=2, W=4, order=4, cum=p):
        # (h, M, d, packed, n, a, a_ids, a_ids_stride, r, vals, ids, lse, ws, cum, lastp, sl, toks, bps,
        #  B, W, order, stream)
        return L.cfh_head_topk_packed_beam_chain(p, M, 512, p, 1000, None, None, 0, 0, p, p, p, p, cum, p,
                                                  None, p, p, B, W, order, None)
    assert call(M=7) == 1            # M != B W
    assert call(M=9, B=1, W=9) == 1  # W x W > 64
    assert call(order=0) == 1
    assert call(order=9) == 1
    assert call(cum=None) == 1
    assert call(M=0, B=0) == 1


def test_noalloc_flow_rejects_a_workspace_beyond_the_scratch_without_a_device():
    """cfh_flow_integrate_noalloc refuses, before any HIP call, a shape whose flow workspace exceeds
    the 64 MiB scratch array (d = 8192 at 8 layers needs 75.8 MiB), with its own status."""
    import ctypes as C

    from chain_flow_amd.config import flownet
    from chain_flow_amd.flow import caps, flow_dims
    L = _lib.lib()
    assert L.cfh_error_string(4).startswith(b"workspace exceeds the no-allocation scratch")
    cfg = flownet(8192, layers=8, flow_steps=8)
    assert caps(cfg) > 64 << 20
    assert caps(flownet(5120, layers=8, flow_steps=8)) <= 64 << 20
    dims = flow_dims(cfg)
    p = 4096   # stand-in addresses: never dereferenced, the size check fails first
    experts = _lib.ptr_array([p, p])
    assert L.cfh_flow_integrate_noalloc(C.byref(dims), experts, p, p, 1, None) == 4
    assert L.cfh_flow_integrate_noalloc(C.byref(dims), experts, p, p, 0, None) == 1    # batch < 1


def test_flow_dims_carry_the_init_mode():
    """init_latents' three modes reach cfh_flow_dims.init_mode ("noise" as a z0 the caller draws),
    and a checkpoint's noise_scale survives the config loader (reference default 1.0,
    cf/drafters/tree_flow.py:53)."""
    import dataclasses
    from chain_flow_amd.config import config_from_model_args, flownet
    from chain_flow_amd.flow import flow_dims
    base = flownet(512, layers=1, flow_steps=1)
    assert base.noise_scale == 1.0
    for mode, want in (("delta", _lib.INIT_DELTA), ("repeat_last", _lib.INIT_REPEAT_LAST),
                       ("noise", _lib.INIT_GIVEN)):
        assert flow_dims(dataclasses.replace(base, init_mode=mode)).init_mode == want
    args = dict(context_size=8, draft_length=8, chunk_size=4, expert_dim=512, init_mode="noise",
                noise_scale=0.25, drafter_dropout=0.1)
    cfg = config_from_model_args(args)
    assert cfg.init_mode == "noise" and cfg.noise_scale == 0.25


def test_flow_caps_shape_checks_without_a_device():
    """cfh_caps decides support and the workspace size on the host: the headline and latent
    shapes are supported; at d = 4096 a batch of two shares each weight stream in one request group
    (a larger workspace), at d = 5120 it runs one request a group (a 16-row operand of 5120 columns
    would not fit the streaming kernels' LDS); each out-of-range field of cfh_flow_dims is refused
    as unsupported."""
    import ctypes as C
    import dataclasses

    from chain_flow_amd.config import flownet
    from chain_flow_amd.flow import flow_dims
    L = _lib.lib()

    def caps(dims, batch=1):
        ws = C.c_int64(-1)
        rc = L.cfh_caps(C.byref(dims), batch, C.byref(ws))
        return rc, ws.value

    head = flownet(5120, layers=8, flow_steps=8)
    rc1, ws1 = caps(flow_dims(head))
    assert rc1 == 0 and ws1 > 0 and caps(flow_dims(head), 2) == (0, ws1)
    c4 = flow_dims(flownet(4096, layers=8, flow_steps=8))
    assert caps(c4)[0] == 0 and caps(c4, 2)[1] > caps(c4)[1]
    assert caps(flow_dims(flownet(640, layers=8, flow_steps=2)))[0] == 0
    assert caps(flow_dims(head), 0)[0] == 2                                   # batch < 1
    bad = [("d", 5120 + 32), ("heads", 7), ("ffn_mult", 9), ("layers", 0), ("ctx_rows", 1),
           ("ctx_rows", 17), ("chunk_size", 3), ("draft_length", 17), ("flow_steps", 17),
           ("numerics", 7), ("init_mode", 3)]
    for field, value in bad:
        dims = flow_dims(head)
        setattr(dims, field, value)
        assert caps(dims)[0] == 2, (field, value)
    assert L.cfh_caps(None, 1, None) == 2
    # a config field the flow ignores leaves the plan alone
    assert caps(flow_dims(dataclasses.replace(head, noise_scale=0.5)))[1] == ws1


def test_flow_two_heads_fold_layout_without_a_device():
    """A head width that puts two heads in an MFMA k-chunk (640 / 8 = 80) folds the cross attention
    of single-request groups and keeps the unfolded launches for packed groups, so the expert image
    holds the query weight twice: exactly one d x d fp16 matrix per block more than the same width
    with one head a k-chunk (640 / 10 = 64).  Both batch sizes are supported."""
    import ctypes as C

    from chain_flow_amd.config import flownet
    from chain_flow_amd.flow import flow_dims
    L = _lib.lib()
    layers, d = 3, 640
    two = flow_dims(flownet(d, layers=layers, flow_steps=2, num_heads=8))
    one = flow_dims(flownet(d, layers=layers, flow_steps=2, num_heads=10))
    extra = L.cfh_flow_expert_bytes(C.byref(two)) - L.cfh_flow_expert_bytes(C.byref(one))
    assert extra == layers * d * d * 2
    for dims in (two, one):
        for batch in (1, 2, 3):
            ws = C.c_int64(-1)
            assert L.cfh_caps(C.byref(dims), batch, C.byref(ws)) == 0 and ws.value > 0


def test_flow_plan_flags_without_a_device():
    """cfh_flow_plan reports the launch forms on the host: the shipped latent width (640, 8 heads of
    80) folds its cross attention two heads a k-chunk and, for one request, runs the residual rows
    and the cross attention as one launch; a packed pair of requests keeps the unfolded launches;
    d = 512 (heads of 64) folds one head a k-chunk with the one-launch form; d = 1024 and the
    headline d = 5120 fold without it and plan concurrent chunk experts; 32 requests at d = 4096 run
    in wide groups."""
    from chain_flow_amd.config import flownet
    from chain_flow_amd.flow import plan_flags
    F, F2, X, W, CC = _lib.PLAN_FOLD, _lib.PLAN_FOLD2, _lib.PLAN_XBLK, _lib.PLAN_WIDE, _lib.PLAN_CONC
    latent = flownet(640, layers=8, flow_steps=2)
    assert plan_flags(latent) == F | F2 | X
    assert plan_flags(latent, 2) & (F | X) == 0
    assert plan_flags(flownet(512, layers=2, flow_steps=2)) == F | X
    assert plan_flags(flownet(1024, layers=2, flow_steps=2)) == F | CC
    assert plan_flags(flownet(5120, layers=8, flow_steps=8)) == F | CC
    assert plan_flags(flownet(4096, layers=8, flow_steps=8), 32) & W
    # fewer context rows, four or seven heads, short experts: still the one-launch form
    for d, h, ctx, kd, cs in [(640, 8, 4, 8, 4), (320, 4, 8, 8, 4), (512, 8, 3, 4, 4), (448, 7, 5, 8, 4)]:
        cfg = flownet(d, layers=2, flow_steps=2, num_heads=h, context_size=ctx, draft_length=kd, chunk_size=cs)
        assert plan_flags(cfg) & X, (d, h, ctx, kd, cs)
    # 16 draft rows exceed the one-launch form's 8 rows a workgroup
    assert not plan_flags(flownet(640, layers=1, flow_steps=2, draft_length=16, chunk_size=8)) & X

