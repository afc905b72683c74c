"""GPU parity of the fused flow (cfh_flow_integrate) against the CPU oracle.

Contract: predicted hiddens within 2e-3 norm-relative of the oracle's fp16 restatement of
``TreeFlowDrafter.predict_hidden`` on the same seeded weights and context, in the numerics the
reference runs that shape in (its fused kernel's at d in {640, 1024}, torch's fp16 modules'
elsewhere).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import oracle_numerics, rel_err, to64, weights64
from chain_flow_amd.config import flownet
from chain_flow_amd import _lib
from chain_flow_amd.flow import FusedFlow, plan_flags
from chain_flow_amd.weights import make_weights, synthetic_context
from oracle import flow as oflow

TOL_FP16 = 2e-3


def _ocfg(cfg):
    return dict(draft_length=cfg.draft_length, chunk_size=cfg.chunk_size,
                num_layers=cfg.num_drafter_layers, num_heads=cfg.num_heads,
                num_flow_steps=cfg.num_flow_steps, init_mode=cfg.init_mode)


def _flow_weights(cfg, init="test", seed=0):
    from chain_flow_amd.weights import param_specs
    names = [n for n in param_specs(cfg, 16, target=False) if n.startswith(("expert.", "extra_experts."))]
    return make_weights(cfg, 16, init=init, base_seed=seed, names=set(names), target=False)


@pytest.mark.gpu
@pytest.mark.parametrize("d,layers,steps", [(512, 1, 1), (512, 2, 2), (1024, 2, 3), (2560, 1, 2)])
def test_flow_matches_oracle(cuda, d, layers, steps):
    cfg = flownet(d, layers=layers, flow_steps=steps)
    W = _flow_weights(cfg)
    ctx = synthetic_context(1, cfg.context_size, d, seed=1)
    print(f"[flow parity] d={d} L={layers} E={steps}", flush=True)
    ff = FusedFlow(cfg, {k: v.to(cuda) for k, v in W.items()}, device=cuda)
    z = ff.predict_hidden(ctx.to(cuda))
    torch.cuda.synchronize()
    ref = oflow.predict_hidden(weights64(W), to64(ctx), _ocfg(cfg), numerics=oracle_numerics(cfg))
    err = rel_err(to64(z), ref)
    print(f"  rel err {err:.3e}", flush=True)
    assert np.isfinite(to64(z)).all()
    assert err < TOL_FP16


@pytest.mark.gpu
@pytest.mark.parametrize("d,kd,cs", [(1024, 16, 8), (640, 16, 8)])
def test_flow_long_draft_matches_oracle(cuda, d, kd, cs):
    """Draft length 16 in two chunks of 8 (16 rows in the second chunk's launches)."""
    cfg = flownet(d, layers=1, flow_steps=2, draft_length=kd, chunk_size=cs)
    W = _flow_weights(cfg)
    ctx = synthetic_context(1, cfg.context_size, d, seed=3)
    print(f"[flow parity] d={d} draft_length={kd} chunk={cs}", flush=True)
    ff = FusedFlow(cfg, {k: v.to(cuda) for k, v in W.items()}, device=cuda)
    z = ff.predict_hidden(ctx.to(cuda))
    torch.cuda.synchronize()
    ref = oflow.predict_hidden(weights64(W), to64(ctx), _ocfg(cfg), numerics=oracle_numerics(cfg))
    err = rel_err(to64(z), ref)
    print(f"  rel err {err:.3e}", flush=True)
    assert np.isfinite(to64(z)).all()
    assert err < TOL_FP16


@pytest.mark.gpu
def test_flow_is_bit_reproducible(cuda):
    """Every reduction runs in a fixed order (no atomics): repeated drafts give bit-identical
    hidden states."""
    cfg = flownet(1024, layers=2, flow_steps=2)
    W = {k: v.to(cuda) for k, v in _flow_weights(cfg, seed=4).items()}
    ctx = synthetic_context(1, cfg.context_size, 1024, seed=2).to(cuda)
    ff = FusedFlow(cfg, W, device=cuda)
    a = ff.predict_hidden(ctx).clone()
    b = ff.predict_hidden(ctx).clone()
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.gpu
def test_flow_same_on_every_caller_stream(cuda):
    """From d = 1024 an eager flow runs its second chunk expert on a companion of the caller's
    stream, created (and checked for overlap with the caller's stream) on the first call per caller
    stream: the draft is bit-identical on the default stream and on a side stream, first call and
    repeated."""
    cfg = flownet(1024, layers=2, flow_steps=2)
    assert cfg.draft_length // cfg.chunk_size == 2
    W = {k: v.to(cuda) for k, v in _flow_weights(cfg, seed=5).items()}
    ctx = synthetic_context(1, cfg.context_size, 1024, seed=6).to(cuda)
    ff = FusedFlow(cfg, W, device=cuda)
    a = ff.predict_hidden(ctx).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        b = ff.predict_hidden(ctx).clone()
        c = ff.predict_hidden(ctx).clone()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(a, c)


@pytest.mark.gpu
def test_flow_graph_replays_equal_eager(cuda):
    """Under stream capture the flow keeps both chunk experts on the caller's stream (the eager call
    at d = 1024 runs the second on a companion): every replay of the captured flow, with eager
    work and synchronisations between the replays, equals the eager draft bit for bit."""
    cfg = flownet(1024, layers=2, flow_steps=2)
    W = {k: v.to(cuda) for k, v in _flow_weights(cfg, seed=8).items()}
    ctx = synthetic_context(1, cfg.context_size, 1024, seed=9).to(cuda)
    ff = FusedFlow(cfg, W, device=cuda)
    want = ff.predict_hidden(ctx).clone()
    out = torch.empty_like(want)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ff.predict_hidden(ctx, out=out)                  # warm-up off the default stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ff.predict_hidden(ctx, out=out)
    for rep in range(3):
        out.zero_()
        junk = torch.randn(256, 256, device=cuda) @ torch.randn(256, 256, device=cuda)
        g.replay()
        torch.cuda.synchronize()
        del junk
        assert torch.equal(out, want), rep
        assert torch.equal(ff.predict_hidden(ctx), want), rep


@pytest.mark.gpu
def test_flow_full_width_matches_oracle(cuda):
    """The benchmark's width (d = 5120: head_dim 640, ffn 30720, the 16-wave and one-round grids,
    the deep operand staging) against the oracle: one block, two Euler steps."""
    d = 5120
    cfg = flownet(d, layers=1, flow_steps=2)
    print(f"[flow parity] d={d} L=1 E=2 (full width)", flush=True)
    W = _flow_weights(cfg, seed=7)
    ctx = synthetic_context(1, cfg.context_size, d, seed=3)
    ff = FusedFlow(cfg, {k: v.to(cuda) for k, v in W.items()}, device=cuda)
    z = ff.predict_hidden(ctx.to(cuda))
    torch.cuda.synchronize()
    del ff
    ref = oflow.predict_hidden(weights64(W), to64(ctx), _ocfg(cfg), numerics=oracle_numerics(cfg))
    err = rel_err(to64(z), ref)
    print(f"  rel err {err:.3e}", flush=True)
    assert np.isfinite(to64(z)).all()
    assert err < TOL_FP16


@pytest.mark.gpu
@pytest.mark.parametrize("d,heads,layers,steps", [(640, 8, 2, 2), (640, 16, 1, 2), (768, 12, 1, 1), (1920, 8, 1, 1),
                                                  (128, 8, 1, 2), (64, 8, 1, 1), (192, 4, 1, 1)])
def test_flow_latent_widths_match_oracle(cuda, d, heads, layers, steps):
    """Widths whose heads do not fill an MFMA k-step (head_dim 80, 240, 16 and 48: two heads per
    attention k-chunk; 40 and 8: four), rows that do not fill whole waves of the residual kernel
    (d = 640 and 1920: 160 and 480 four-column groups) and widths too short to split K (d <= 256).
    d = 640 with 8 heads is the latent width of the shipped VAE drafters."""
    cfg = flownet(d, layers=layers, flow_steps=steps, num_heads=heads)
    W = _flow_weights(cfg, seed=11)
    ctx = synthetic_context(1, cfg.context_size, d, seed=5)
    print(f"[flow parity] d={d} H={heads} L={layers} E={steps}", flush=True)
    ff = FusedFlow(cfg, {k: v.to(cuda) for k, v in W.items()}, device=cuda)
    z = ff.predict_hidden(ctx.to(cuda))
    torch.cuda.synchronize()
    ref = oflow.predict_hidden(weights64(W), to64(ctx), _ocfg(cfg), numerics=oracle_numerics(cfg))
    err = rel_err(to64(z), ref)
    print(f"  rel err {err:.3e}", flush=True)
    assert np.isfinite(to64(z)).all()
    assert err < TOL_FP16


@pytest.mark.gpu
@pytest.mark.parametrize("d,heads,ctx,kd,cs", [(640, 8, 4, 8, 4), (640, 8, 6, 8, 4), (320, 4, 8, 8, 4),
                                               (512, 8, 3, 4, 4), (640, 8, 8, 4, 2), (448, 7, 5, 8, 4)])
def test_flow_one_launch_cross_attention_shapes(cuda, d, heads, ctx, kd, cs):
    """One-request flows of width <= 640 run the residual rows and the folded cross attention as
    one launch a block pass; its edge cases against the oracle: fewer than 8 context rows (4, 6, 3,
    5), four and seven heads (a pair of heads a score tile, the last pair half empty), two partial
    rows of the out-projection, a single expert of 4 rows, experts of 2 and 4 rows."""
    cfg = flownet(d, layers=2, flow_steps=2, num_heads=heads, context_size=ctx, draft_length=kd, chunk_size=cs)
    assert plan_flags(cfg) & _lib.PLAN_XBLK                # the form under test is the one that runs
    W = _flow_weights(cfg, seed=17)
    c = synthetic_context(1, cfg.context_size, d, seed=8)
    print(f"[flow one-launch xattn] d={d} H={heads} C={ctx} draft={kd} chunk={cs}", flush=True)
    ff = FusedFlow(cfg, {k: v.to(cuda) for k, v in W.items()}, device=cuda)
    z = ff.predict_hidden(c.to(cuda))
    torch.cuda.synchronize()
    ref = oflow.predict_hidden(weights64(W), to64(c), _ocfg(cfg), numerics=oracle_numerics(cfg))
    err = rel_err(to64(z), ref)
    print(f"  rel err {err:.3e}", flush=True)
    assert np.isfinite(to64(z)).all()
    assert err < TOL_FP16


@pytest.mark.gpu
@pytest.mark.parametrize("d,B,layers", [(512, 2, 2), (512, 5, 1), (640, 3, 1), (1024, 2, 2), (4096, 2, 1),
                                        (1024, 3, 2), (1024, 16, 1), (1024, 21, 1), (1024, 40, 1), (2048, 8, 1),
                                        (4096, 5, 1), (640, 20, 2)])
def test_packed_batch_matches_oracle_per_request(cuda, d, B, layers):
    """A batch drafts in groups whose rows share every weight stream: two requests a 16-row tile
    (attention masked to each request's own rows and context), or, above two requests, wide groups
    of up to 16 requests (rows staged in K chunks, self attention per request; the cross attention
    folded in subgroups of two where the head width is a multiple of 128, else unfolded: q
    projection, attention per request and head, out-projection); two wide groups at a time share
    every launch.  Each request's hiddens against the oracle on its own context, and against the
    same request drafted alone in the same numerics.  d = 512 (head width 64) keeps the two-request
    tiles, B = 5 ending with a group of one; d = 640 (head width 80) runs B = 3 as one unfolded wide
    group and B = 20 as two; d = 1024: B = 3 one wide group of an odd request count, B = 21 two (11
    and 10 requests), B = 40 a pair of 14-request groups then one of 12."""
    cfg = flownet(d, layers=layers, flow_steps=2)
    W = _flow_weights(cfg, seed=13)
    ctx = synthetic_context(B, cfg.context_size, d, seed=21)
    print(f"[flow packed] d={d} B={B} L={layers}", flush=True)
    ff = FusedFlow(cfg, {k: v.to(cuda) for k, v in W.items()}, device=cuda)
    z = ff.predict_hidden(ctx.to(cuda))
    num = ff.dims.numerics                               # the batch's numerics (torch's modules at B > 1)
    singles = [ff.predict_hidden(ctx[b:b + 1].to(cuda), numerics=num).clone() for b in range(B)]
    torch.cuda.synchronize()
    onum = "fp16_modules" if num == 1 else "fp16"
    W64 = weights64(W)
    for b in range(B):
        ref = oflow.predict_hidden(W64, to64(ctx[b:b + 1]), _ocfg(cfg), numerics=onum)
        e = rel_err(to64(z[b:b + 1]), ref)
        es = rel_err(to64(z[b:b + 1]), to64(singles[b]))
        print(f"  request {b}: vs oracle {e:.3e}, vs drafted alone {es:.3e}", flush=True)
        assert np.isfinite(to64(z[b:b + 1])).all()
        assert e < TOL_FP16 and es < TOL_FP16


@pytest.mark.gpu
@pytest.mark.parametrize("mode,B", [("repeat_last", 1), ("noise", 1), ("noise", 2), ("repeat_last", 6), ("noise", 6)])
def test_init_modes_match_oracle(cuda, mode, B):
    """init_latents' other modes (cf/drafters/tree_flow.py:150-161): "repeat_last" starts every
    draft row from the last context row; "noise" from randn * noise_scale drawn with torch's
    generator, which the oracle is given (the same seeded draw).  B = 6 (48 rows) runs as one wide
    request group, whose row kernels build the initial latents of every request."""
    import dataclasses
    cfg = dataclasses.replace(flownet(512, layers=2, flow_steps=2), init_mode=mode, noise_scale=0.5)
    W = _flow_weights(cfg)
    ctx = synthetic_context(B, cfg.context_size, 512, seed=5)
    print(f"[flow init] mode={mode} B={B}", flush=True)
    ff = FusedFlow(cfg, {k: v.to(cuda) for k, v in W.items()}, device=cuda)
    torch.manual_seed(11)
    z = ff.predict_hidden(ctx.to(cuda))
    torch.cuda.synchronize()
    z0 = None
    if mode == "noise":
        torch.manual_seed(11)
        z0 = to64(torch.randn(B, cfg.draft_length, 512, device=cuda, dtype=torch.float16) * cfg.noise_scale)
    ref = oflow.predict_hidden(weights64(W), to64(ctx), _ocfg(cfg), numerics=oracle_numerics(cfg, B), z0=z0)
    err = rel_err(to64(z), ref)
    print(f"  rel err {err:.3e}", flush=True)
    assert np.isfinite(to64(z)).all()
    assert err < TOL_FP16
    if mode == "noise":     # a fresh draw gives a different draft
        z2 = ff.predict_hidden(ctx.to(cuda))
        torch.cuda.synchronize()
        assert not torch.equal(z, z2)
