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
