"""Benchmark: microseconds per 5-token chain draft step on one MI355X (d=5120, fp16, batch 1).

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--d 5120] [--layers 8] [--no-cpu]
    python bench.py --workload latent        # the shipped 4B latent drafter (see below)

A step is one whole FlowDrafterProposer chain draft over inputs already resident in HBM:
``predict_hidden`` (init_latents + 8 Euler steps of both chunk experts, every block) followed by the
5-depth width-4 beam over the shortlisted lm_head (path residual, head GEMV + markov bias, top-k,
beam update) and the backtrack.  Weights are seeded synthetic N(0, 0.02) of the reference's
TreeFlowDrafter architecture (context 8, draft_length 8 in chunks of 4, 8 heads, ffn x6, L blocks,
E=8 Euler steps, path order 4, markov rank 256) on a 248,320-row target head restricted to a seeded
62,642-id shortlist; the context is N(0, 1) rescaled to RMS 1.

``--workload latent`` times the drafter the reference ships for its 4B target instead: hidden 2560,
the flow at the VAE latent width 640 (8 blocks, 2 Euler steps) between the TransformerHiddenVAE
encoder and decoder (intermediate 1920, 2 layers each, 8 heads), same head and beam; its
``roofline`` covers the whole predict_hidden pass (encode, flow, decode).

Prints one JSON line.  ``roofline`` covers the flow pass (the dominant part, ~96% of the bytes),
timed with HIP events on the stream it runs on; ``cpu_baseline`` is the CPU oracle timed on a
bounded sample of the same workload on this host and scaled to one draft step (rank 0, N=1 only).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "chain-flow_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
SHORTLIST_ROWS = 62642
VOCAB = 248320


def flow_bytes(d, L, E, C, ffn=6):
    """Algorithmic HBM bytes of one predict_hidden: every fp16 weight byte once per time it is
    needed (block weights per Euler step per chunk expert, cross K/V projection once per draft,
    time_mlp[2] + out_norm/out_proj per step per expert) plus context in and hiddens out."""
    blk = (3 + 1 + 1 + 1 + 2 * ffn) * d * d + (3 + 1 + 1 + 1 + ffn + 1 + 6) * d   # 18d^2 + 19d at ffn=6
    per_step = L * blk + 2 * d * d + 5 * d
    per_draft_kv = L * (2 * d * d + 4 * d)
    halves = E * C * per_step + C * per_draft_kv
    return 2 * halves + 2 * (8 * d) + 2 * (8 * d)


def head_bytes(d, K, W, n_rows, rank=256, order=4, path_ffn=2):
    """One-pass head over K depths: shortlist rows of lm_head and markov w2 once per depth, the live
    PathHead offset projections (nlive = min(depth, order)) and its MLP once per depth."""
    total = 0
    for s in range(1, K + 1):
        nlive = min(s, order)
        total += n_rows * d * 2 + n_rows * rank * 2
        total += (nlive * d * d + 2 * path_ffn * d * d) * 2
    return total


def measured_traffic(d, L, E):
    """HBM bytes per flow pass from the committed counter profile of this workload (FETCH_SIZE and
    WRITE_SIZE, calibrated with a 1 GiB copy), or None for a workload without one."""
    p = ROOT / "profiles" / f"flow_d{d}_L{L}_E{E}_traffic.json"
    if not p.exists():
        return None
    return int(json.loads(p.read_text())["traffic_bytes"])


LATENT, VAE_INTER, VAE_LAYERS = 640, 1920, 2


def vae_bytes(hidden, latent=LATENT, inter=VAE_INTER, layers=VAE_LAYERS, rows=8):
    """Algorithmic HBM bytes of one encode + one decode: every fp16 VAE weight once per pass (logvar
    unused), the position rows, the rows in and out."""
    per_layer = 12 * inter * inter + 13 * inter            # qkv, out, linear1/2 (+ biases, 2 norms)
    half = lambda kin, nout: (inter * kin + inter + 16 * inter + layers * per_layer + 2 * inter
                              + nout * inter + nout)
    return 2 * (half(hidden, latent) + half(latent, hidden)) + 2 * rows * (hidden + latent) * 2


def build_workload(d, L, E, device, latent=False):
    import torch
    from chain_flow_amd.config import TreeVAEFlowConfig, flownet
    from chain_flow_amd.drafter import Drafter
    from chain_flow_amd.shortlist import synthetic
    from chain_flow_amd.weights import make_weights, synthetic_context
    if latent:
        cfg = TreeVAEFlowConfig(context_size=8, draft_length=8, chunk_size=4, expert_dim=d, num_heads=8,
                                ffn_multiplier=6, num_drafter_layers=L, num_flow_steps=E, init_mode="delta",
                                path_order=4, path_ffn_multiplier=2, markov_rank=256, latent_size=LATENT,
                                vae_intermediate_size=VAE_INTER, vae_num_layers=VAE_LAYERS, vae_num_heads=8,
                                vae_max_sequence_length=16)
    else:
        cfg = flownet(d, layers=L, flow_steps=E)
    W = make_weights(cfg, VOCAB, init="baseline", dtype=torch.float16, device=device, base_seed=0, hidden=d)
    sl = synthetic(VOCAB, SHORTLIST_ROWS, seed=2)
    dr = Drafter(cfg, W, sl.to(device), device=device)
    ctx = synthetic_context(1, cfg.context_size, d, seed=1).to(device)
    known0 = sl[1234:1235].long().to(device)
    return cfg, W, dr, ctx, known0


def cpu_baseline_latent(W, cfg, sl, d, ctx):
    """The CPU oracle on the latent workload: the whole predict_hidden (VAE encode, the latent flow,
    decode) plus one head depth scaled to K depths."""
    import numpy as np
    from oracle import head as ohead
    from oracle import vae as ovae
    try:
        from threadpoolctl import threadpool_info
        cores = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        cores = os.cpu_count() or 1
    f64 = lambda t: t.detach().float().cpu().double().numpy()
    Wf = {k: f64(v) for k, v in W.items() if k.startswith(("vae.", "expert.", "extra_experts."))}
    vc = dict(intermediate_size=cfg.vae_intermediate_size, num_layers=cfg.vae_num_layers,
              num_heads=cfg.vae_num_heads, max_sequence_length=cfg.vae_max_sequence_length)
    fc = dict(draft_length=cfg.draft_length, chunk_size=cfg.chunk_size, num_layers=cfg.num_drafter_layers,
              num_heads=cfg.num_heads, num_flow_steps=cfg.num_flow_steps, init_mode=cfg.init_mode)
    t0 = time.perf_counter()
    ovae.predict_hidden(Wf, f64(ctx), vc, fc, "fp16")
    t_pred = time.perf_counter() - t0
    del Wf
    slt = sl.long().cpu()
    Wh = {k: f64(v) for k, v in W.items() if k.startswith("path_head.")}
    emb = f64(W["embed_tokens.weight"][slt[:4096].to(W["embed_tokens.weight"].device)])
    lastp = np.arange(16).reshape(4, 4) % 4096
    w_sl = f64(W["lm_head.weight"][slt.to(W["lm_head.weight"].device)])
    w1 = f64(W["markov.w1.weight"][slt[:4096].to(W["markov.w1.weight"].device)])
    w2_sl = f64(W["markov.w2.weight"][slt.to(W["markov.w2.weight"].device)])
    pred = np.random.default_rng(0).standard_normal((d,))
    t0 = time.perf_counter()
    res = ohead.path_residual(Wh, emb, lastp, 4, cfg.path_order, "fp16")
    h = ohead.r16(pred[None] + res, "fp16")
    lp = ohead.log_softmax(ohead.head_with_bias(h, w_sl, w1, w2_sl, lastp[:, 0]))
    ohead.topk(lp, 4)
    t_head = time.perf_counter() - t0
    K = 5
    return {"value": (t_pred + K * t_head) * 1e6, "unit": "us per draft step", "cores": int(cores),
            "kind": "port",
            "sample": (f"numpy oracle (float64 math, fp16 rounding points): the whole latent predict_hidden "
                       f"({t_pred * 1e3:.0f} ms) and one 4-beam head depth over {SHORTLIST_ROWS} rows at "
                       f"d={d} ({t_head * 1e3:.0f} ms) scaled by K={K}")}


def cpu_baseline(W, cfg, sl, d):
    """The CPU oracle on a bounded sample of the same workload, scaled to one draft step.

    Sample: one HiddenKVFlowBlock pass of each chunk expert (S = 4 and 8 rows), the cross K/V of
    one block of each expert, and one head depth (4 beams: fused path residual with 4 live offsets,
    62,642-row shortlist GEMV + markov bias, log-softmax).  One draft = E*L block passes of each
    expert + L cross K/V per expert + K head depths."""
    import numpy as np
    import torch
    from oracle import flow as oflow
    from oracle import head as ohead
    try:
        from threadpoolctl import threadpool_info
        cores = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        cores = os.cpu_count() or 1
    f64 = lambda t: t.detach().float().cpu().double().numpy()
    rng = np.random.default_rng(0)
    t_blocks = 0.0
    t_kv = 0.0
    for ci, p in enumerate(oflow.expert_prefixes(cfg.num_chunks)):
        bp = f"{p}blocks.0."
        Wb = {k: f64(v) for k, v in W.items() if k.startswith(bp)}
        S = (ci + 1) * cfg.chunk_size
        ctx = rng.standard_normal((1, cfg.context_size, d))
        t0 = time.perf_counter()
        kv = oflow.cross_kv(Wb, bp, ctx, "fp16")
        t_kv += time.perf_counter() - t0
        res = rng.standard_normal((1, S, d))
        mask = oflow.causal_mask(S)
        t0 = time.perf_counter()
        oflow.block_forward(Wb, bp, res, kv, mask, cfg.num_heads, "fp16")
        t_blocks += time.perf_counter() - t0
        del Wb
    slt = sl.long().cpu()
    Wh = {k: f64(v) for k, v in W.items() if k.startswith("path_head.")}
    emb = f64(W["embed_tokens.weight"][slt[:4096].to(W["embed_tokens.weight"].device)])
    lastp = np.arange(16).reshape(4, 4) % 4096
    w_sl = f64(W["lm_head.weight"][slt.to(W["lm_head.weight"].device)])
    w1 = f64(W["markov.w1.weight"][slt[:4096].to(W["markov.w1.weight"].device)])
    w2_sl = f64(W["markov.w2.weight"][slt.to(W["markov.w2.weight"].device)])
    pred = rng.standard_normal((d,))
    t0 = time.perf_counter()
    res = ohead.path_residual(Wh, emb, lastp, 4, cfg.path_order, "fp16")
    h = ohead.r16(pred[None] + res, "fp16")
    logits = ohead.head_with_bias(h, w_sl, w1, w2_sl, lastp[:, 0])
    lp = ohead.log_softmax(logits)
    ohead.topk(lp, 4)
    t_head = time.perf_counter() - t0
    E, L, K = cfg.num_flow_steps, cfg.num_drafter_layers, 5
    us = (E * L * t_blocks + L * t_kv + K * t_head) * 1e6
    return {"value": us, "unit": "us per draft step", "cores": int(cores), "kind": "port",
            "sample": (f"numpy oracle (float64 math, fp16 rounding points) at d={d}: one block pass of "
                       f"each chunk expert ({t_blocks * 1e3:.0f} ms), one block's cross K/V per expert "
                       f"({t_kv * 1e3:.0f} ms), one 4-beam head depth over {SHORTLIST_ROWS} rows "
                       f"({t_head * 1e3:.0f} ms); scaled by E*L={E * L}, L={L}, K={K}")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=["target", "latent"], default="target",
                    help="target: the flow at the target width d (default); latent: the shipped 4B "
                         "latent drafter (hidden 2560, VAE latent 640, 8 blocks, 2 Euler steps)")
    ap.add_argument("--d", type=int, default=None, help="target hidden size (5120; latent: 2560)")
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--flow-steps", type=int, default=None, help="Euler steps (8; latent: 2)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--calib-copy", action="store_true",
                    help="after timing, copy one 1 GiB buffer (a kernel of known traffic for calibrating "
                         "the profiler's FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU: the draft step is a single-GPU, batch-1 path and this "
              f"build has no multi-GPU mode (asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    latent = args.workload == "latent"
    d = args.d or (2560 if latent else 5120)
    L = args.layers
    E = args.flow_steps or (2 if latent else 8)
    K, Wd = 5, 4
    print(f"[bench] building workload {args.workload} d={d} L={L} E={E}", file=sys.stderr, flush=True)
    cfg, W, dr, ctx, known0 = build_workload(d, L, E, dev, latent=latent)
    torch.cuda.synchronize()

    def step():
        pred = dr.predict_hidden(ctx)
        return pred, dr.beam_chains(None, known0, K, Wd, pred=pred)

    print("[bench] warmup", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    print("[bench] timed", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev[i][0].record()
        pred = dr.predict_hidden(ctx)
        ev[i][1].record()
        dr.beam_chains(None, known0, K, Wd, pred=pred)
        ev[i][2].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    flow_ms = sorted(a.elapsed_time(b) for a, b, _ in ev)
    head_ms = sorted(b.elapsed_time(c) for _, b, c in ev)
    step_ms = sorted(a.elapsed_time(c) for a, _, c in ev)
    med = lambda v: v[len(v) // 2]
    ms = wall * 1e3 / args.steps
    if latent:
        fb = flow_bytes(LATENT, L, E, cfg.num_chunks) + vae_bytes(d)
        traffic, kern = None, "predict_hidden pass (cfh_vae_encode + cfh_flow_integrate + cfh_vae_decode)"
        workload = (f"latent chain draft: hidden {d} fp16 bs1 K={K} width {Wd}; TransformerHiddenVAE latent "
                    f"{LATENT} (intermediate {VAE_INTER}, {VAE_LAYERS}+{VAE_LAYERS} layers); flow at {LATENT}, "
                    f"L={L} E={E} 2 chunk experts; shortlisted head {SHORTLIST_ROWS}x{d}")
        metric = "us per 5-token draft step (latent drafter: hidden 2560, VAE latent 640, bs1)"
    else:
        fb = flow_bytes(d, L, E, cfg.num_chunks)
        traffic, kern = measured_traffic(d, L, E), "flow pass (cfh_flow_integrate)"
        workload = (f"chain draft d={d} fp16 bs1 K={K} width {Wd}, flow L={L} E={E} "
                    f"2 chunk experts, shortlisted head {SHORTLIST_ROWS}x{d}")
        metric = "us per 5-token draft step (d=5120, bs1) + achieved HBM GB/s vs roofline"
    hb = head_bytes(d, K, Wd, SHORTLIST_ROWS)
    flow_gbs = fb / (med(flow_ms) * 1e-3) / 1e9
    out = {
        "metric": metric,
        "value": round(ms * 1e3, 1),
        "unit": "us per draft step",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) RMS-1 context)",
        "config": {"workload": workload,
                   "d": d, "layers": L, "flow_steps": E, "draft_tokens": K, "beam_width": Wd,
                   "shortlist_rows": SHORTLIST_ROWS, "vocab": VOCAB},
        "breakdown_ms": {"flow": round(med(flow_ms), 4), "head_beam": round(med(head_ms), 4),
                         "step_event": round(med(step_ms), 4)},
        "algorithmic_bytes": {"flow": fb, "head": hb, "draft_gbs": round((fb + hb) / (ms * 1e-3) / 1e9, 1)},
        "roofline": {"bound": "hbm", "achieved": round(flow_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(flow_gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": kern},
    }
    if latent:
        out["config"].update({"latent": LATENT, "vae_intermediate": VAE_INTER, "vae_layers": VAE_LAYERS})
    if args.calib_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        out["cpu_baseline"] = (cpu_baseline_latent(W, cfg, dr.head.sl, d, ctx) if latent
                               else cpu_baseline(W, cfg, dr.head.sl, d))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
