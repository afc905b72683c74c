"""cfh_flow_integrate_noalloc (the workspace is the library's per-device scratch array) against
cfh_flow_integrate with a caller workspace: the same kernels, so the same bits, on two calls in a
row, the second on a smaller shape (less of the scratch in use, stale contents of the first call
left in it)."""
from __future__ import annotations

import ctypes as C

import pytest
import torch

from chain_flow_amd import _lib
from chain_flow_amd.config import flownet
from chain_flow_amd.flow import FusedFlow
from chain_flow_amd.weights import make_weights, param_specs, synthetic_context


def _flow(cfg, dev, seed):
    names = {n for n in param_specs(cfg, 16, target=False) if n.startswith(("expert.", "extra_experts."))}
    W = make_weights(cfg, 16, init="test", base_seed=seed, names=names, target=False)
    return FusedFlow(cfg, {k: v.to(dev) for k, v in W.items()}, device=dev)


def _noalloc(ff, ctx):
    out = torch.empty(ctx.shape[0], ff.cfg.draft_length, ff.cfg.flow_dim, dtype=torch.float16, device=ctx.device)
    _lib.check(_lib.lib().cfh_flow_integrate_noalloc(C.byref(ff.dims), ff._experts, ctx.data_ptr(), out.data_ptr(),
                                                     ctx.shape[0], _lib.stream_handle()),
               "cfh_flow_integrate_noalloc")
    return out


@pytest.mark.gpu
def test_noalloc_flow_equals_workspace_flow(cuda):
    for (d, layers, steps, batch, seed) in [(1024, 2, 2, 2, 3), (512, 1, 2, 1, 5)]:
        print(f"[noalloc] d={d} L={layers} E={steps} batch={batch}", flush=True)
        cfg = flownet(d, layers=layers, flow_steps=steps)
        ff = _flow(cfg, cuda, seed)
        ctx = synthetic_context(batch, cfg.context_size, d, seed=seed).to(cuda)
        want = ff.predict_hidden(ctx).clone()
        got = _noalloc(ff, ctx)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want), f"d={d}: noalloc differs from the workspace flow"


def _companions(stream):
    made, conc = C.c_int(-1), C.c_int(-1)
    _lib.check(_lib.lib().cfh_flow_query_streams(_lib.stream_handle(stream), C.byref(made), C.byref(conc)),
               "cfh_flow_query_streams")
    return made.value, conc.value


@pytest.mark.gpu
def test_noalloc_creates_no_streams(cuda):
    """The no-allocation entry point creates no companion stream: on a caller stream the workspace
    flow has not used, the companion count (cfh_flow_query_streams) is the same after the call as
    before it -- zero unless a pooled stream handle already had companions -- and the draft is
    bit-identical to the workspace flow's (d = 1024: the workspace flow runs its chunk experts
    concurrently); a second call, smaller, still matches."""
    cfg = flownet(1024, layers=2, flow_steps=2)
    ff = _flow(cfg, cuda, 9)
    for batch in (2, 1):
        ctx = synthetic_context(batch, cfg.context_size, 1024, seed=10 + batch).to(cuda)
        want = ff.predict_hidden(ctx).clone()
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        before = _companions(side)
        with torch.cuda.stream(side):
            got = _noalloc(ff, ctx)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        after = _companions(side)
        print(f"  batch {batch}: companions of the side stream before {before}, after {after}", flush=True)
        assert after == before, "the no-allocation entry point created companion streams"
        assert torch.equal(got, want), f"batch {batch}: noalloc on a side stream differs"
