"""ctypes binding of libcfhip.so (the C ABI declared in include/cfhip.h).

The library is loaded from this package directory.  There is no fallback: if it is missing or a
call fails, the caller gets an exception naming the entry point and the status.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libcfhip.so"

_lib = None


class FlowDims(C.Structure):
    _fields_ = [("d", C.c_int), ("ffn_mult", C.c_int), ("heads", C.c_int), ("layers", C.c_int),
                ("ctx_rows", C.c_int), ("draft_length", C.c_int), ("chunk_size", C.c_int),
                ("flow_steps", C.c_int), ("numerics", C.c_int), ("init_mode", C.c_int)]


FLOW_FUSED, FLOW_MODULES = 0, 1      # cfh_flow_dims.numerics (CFH_FLOW_FUSED / CFH_FLOW_MODULES)
INIT_DELTA, INIT_REPEAT_LAST, INIT_GIVEN = 0, 1, 2   # cfh_flow_dims.init_mode (CFH_INIT_*)
PLAN_FOLD, PLAN_FOLD2, PLAN_XBLK, PLAN_WIDE, PLAN_CONC = 1, 2, 4, 8, 16   # cfh_flow_plan flags (CFH_PLAN_*)


class VaeDims(C.Structure):
    _fields_ = [("hidden", C.c_int), ("latent", C.c_int), ("inter", C.c_int), ("layers", C.c_int),
                ("heads", C.c_int), ("max_rows", C.c_int)]


_VP = C.c_void_p
_I = C.c_int
_I64 = C.c_int64

# name -> (restype, argtypes); mirrors include/cfhip.h
SIGNATURES = {
    "cfh_version": (_I, []),
    "cfh_error_string": (C.c_char_p, [_I]),
    "cfh_last_hip_error": (_I, []),
    "cfh_pack_linear": (_I, [_VP, _I, _I, _VP, _VP]),
    "cfh_caps": (_I, [C.POINTER(FlowDims), _I, C.POINTER(_I64)]),
    "cfh_flow_expert_bytes": (_I64, [C.POINTER(FlowDims)]),
    "cfh_flow_pack_expert": (_I, [C.POINTER(FlowDims), C.POINTER(_VP), _I, _VP, _VP]),
    "cfh_flow_integrate": (_I, [C.POINTER(FlowDims), C.POINTER(_VP), _VP, _VP, _VP, _I, _VP]),
    "cfh_flow_integrate_noalloc": (_I, [C.POINTER(FlowDims), C.POINTER(_VP), _VP, _VP, _I, _VP]),
    "cfh_flow_prepare_streams": (_I, [C.POINTER(FlowDims), _VP, C.POINTER(_I)]),
    "cfh_flow_group_size": (_I, [C.POINTER(FlowDims), _I, C.POINTER(_I)]),
    "cfh_flow_plan": (_I, [C.POINTER(FlowDims), _I, C.POINTER(_I)]),
    "cfh_flow_anchor_ws_bytes": (_I64, [C.POINTER(FlowDims), _I]),
    "cfh_flow_anchor": (_I, [C.POINTER(FlowDims), _I, C.POINTER(_VP), _VP, _VP, _I, _VP, _VP, _VP]),
    "cfh_flow_integrate_anchored": (_I, [C.POINTER(FlowDims), C.POINTER(_VP), _VP, _VP, _VP, _VP, _I, _VP]),
    "cfh_flow_query_streams": (_I, [_VP, C.POINTER(_I), C.POINTER(_I)]),
    "cfh_flow_release_streams": (_I, [_VP]),
    "cfh_vae_bytes": (_I64, [C.POINTER(VaeDims)]),
    "cfh_vae_pack": (_I, [C.POINTER(VaeDims), C.POINTER(_VP), _I, _VP, _VP]),
    "cfh_vae_caps": (_I, [C.POINTER(VaeDims), _I, C.POINTER(_I64)]),
    "cfh_vae_encode": (_I, [C.POINTER(VaeDims), _VP, _VP, _VP, _I, _I, _VP, _VP]),
    "cfh_vae_decode": (_I, [C.POINTER(VaeDims), _VP, _VP, _VP, _I, _I, _VP, _VP]),
    "cfh_ring_step": (_I, [_VP, _VP, _VP, _I, _I, _VP, _I, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _VP, _VP]),
    "cfh_tree_conv": (_I, [_VP, _I, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _VP, _I, _VP]),
    "cfh_tree_attn_merge": (_I, [_VP, _I, _VP, _I, _VP, _I, _VP, _I, _VP, _VP, _VP, _VP, C.c_float, _I, _I, _I, _I,
                                 _I, _I, _VP]),
    "cfh_tree_accept_ws_bytes": (_I64, [_I]),
    "cfh_tree_greedy_accept": (_I, [_VP, C.c_longlong, _I, _I, _I, _VP, _VP, _VP, _VP, _I, _I, _VP, _VP, _VP, _VP,
                                    _VP, _VP]),
    "cfh_cand_ws_bytes": (_I64, [_I, _I]),
    "cfh_cand_topm": (_I, [_VP, C.c_longlong, _VP, _I, _I, _I, _I, _VP, _VP, _VP, _VP, _VP]),
    "cfh_head_logits": (_I, [_VP, _I, _I, _VP, _VP, _I, _VP, _VP, _I, _I, _VP, _VP, _VP]),
    "cfh_row_topk": (_I, [_VP, _I, _I, _I, _VP, _VP, _VP, _VP]),
    "cfh_head_ws_bytes": (_I64, [_I, _I, _I]),
    "cfh_head_topk": (_I, [_VP, _I, _I, _VP, _VP, _I, _VP, _VP, _I, _I, _VP, _I, _VP, _VP, _VP, _VP, _VP, _VP]),
    "cfh_head_packed_bytes": (_I64, [_I, _I, _I]),
    "cfh_head_pack": (_I, [_VP, _VP, _VP, _I, _I, _I, _VP, _VP]),
    "cfh_head_topk_packed": (_I, [_VP, _I, _I, _VP, _I, _VP, _VP, _I, _I, _I, _VP, _VP, _VP, _VP, _VP, _VP]),
    "cfh_head_gemm_topk": (_I, [_VP, _I, _I, _VP, _VP, _I, _I, _VP, _VP, _VP, _VP, _VP, _VP]),
    "cfh_head_gemm_topk_packed": (_I, [_VP, _I, _I, _VP, _I, _I, _VP, _VP, _VP, _VP, _VP, _VP]),
    "cfh_head_topk_grouped": (_I, [_VP, _I, _I, _I, _VP, _VP, C.c_longlong, _I, _VP, _VP, _I, _I, _VP, _I, _VP, _VP,
                                   _VP, _VP, _VP]),
    "cfh_head_gemm16_topk": (_I, [_VP, _I, _I, _VP, _I, _VP, _I, _VP, _VP, _VP, _VP, _VP, _VP]),
    "cfh_path_ws_bytes": (_I64, [_I, _I, _I, _I]),
    "cfh_path_residual": (_I, [C.POINTER(_VP), _I, _I, _I, _VP, _I, _I, _VP, _VP, C.c_longlong, _I, _VP, _VP,
                               _VP]),
    "cfh_beam_init": (_I, [_VP, _VP, _VP, _VP, _I, _I, _I, _I, _VP]),
    "cfh_beam_chain_step": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _VP]),
    "cfh_head_topk_packed_beam_chain": (_I, [_VP, _I, _I, _VP, _I, _VP, _VP, _I, _I, _VP, _VP, _VP, _VP, _VP, _VP,
                                           _VP, _VP, _VP, _I, _I, _I, _VP]),
    "cfh_beam_tree_step": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I, _I, _VP]),
    "cfh_beam_backtrack": (_I, [_VP, _VP, _VP, _I, _I, _I, _VP, _VP]),
    "cfh_gdn_tree": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I, _VP, _VP, _VP]),
    "cfh_gdn_tree_vllm": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _VP, _VP, _I, _I, _I, _I, _I, _I, _I,
                               C.c_float, _VP, _VP, _VP]),
}


def lib():
    """The loaded library (raises if libcfhip.so has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with "
                               f"`python chain-flow_amd/csrc/build.py` (hipcc, gfx950)")
        h = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | getattr(os, "RTLD_GLOBAL", 0))
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(h, name)
            except AttributeError:
                continue          # reported by missing_symbols(); calling it raises
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def missing_symbols():
    """Entry points of include/cfhip.h that the loaded library does not export."""
    h = lib()
    out = []
    for name in SIGNATURES:
        try:
            getattr(h, name)
        except AttributeError:
            out.append(name)
    return out


def check(status: int, what: str) -> None:
    if status != 0:
        L = lib()
        msg = L.cfh_error_string(status).decode()
        hip = L.cfh_last_hip_error() if status == 3 else 0
        raise RuntimeError(f"{what} failed: {msg} (status {status}"
                           + (f", hipError {hip}" if hip else "") + ")")


def ptr(t) -> int | None:
    """Device (or host) address of a tensor, None for None."""
    return None if t is None else t.data_ptr()


def stream_handle(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def ptr_array(ptrs):
    arr = (C.c_void_p * len(ptrs))(*ptrs)
    return arr
