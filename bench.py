"""Benchmark: microseconds per 5-token chain draft step on one MI355X (d=5120, fp16, batch 1).

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--d 5120] [--layers 8] [--no-cpu]
    python bench.py --workload latent        # the shipped 4B latent drafter (see below)
    python bench.py --workload verify        # the tree-verify kernels at the tree-draft shapes
    python bench.py --workload gemm          # the batched head: 32 seqs x 5 depths, d=4096 bf16
    python bench.py --workload batched       # 32 whole chain drafts at d=4096 (flow, pass A, beams)

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

``--workload verify`` times the tree-verify kernels at the tree-draft shapes, each launch alone on
resident inputs: the tree GDN state update with every node's state written (16
heads, dk = dv = 128, bf16 q/k/v, fp32 states; a 31-node tree of depth 5) -- its time is ``value`` and its bytes the
``roofline`` -- and, in ``breakdown_us``, the serving GDN (bf16 slots), the width-4 tree conv
(6144 channels), the tree attention + prefix merge (40 nodes: 8 per level over 5 levels, 16 heads
over 4 kv heads, D 256, bf16) and the greedy accept on the same tree (41 rows of a 248,320-token
vocabulary).

``--workload gemm`` times the batched-drafting head: 32 sequences x 5 depths = 160 rows at d=4096
bf16 against the 62,642-row shortlist of a 248,320-row head, MFMA skinny GEMM with the per-row
log-softmax top-8 fused in, over the packed shortlist image (`cfh_head_gemm_topk_packed`; the
in-place gather `cfh_head_gemm_topk` is reported beside it); ``roofline`` is HBM (513 MB of head
rows) and the line also states the MFMA rate against the 2.5 PFLOP/s bf16 dense peak.

Prints one JSON line.  ``roofline`` covers the flow pass (the dominant part, ~96% of the bytes),
timed with HIP events on the stream it runs on.  ``cpu_baseline`` is the CPU reference plumbing run
measured whole on this host (rank 0, N=1 only): chain drafts at d=2560 in fp32 (L=8, E=8, the
width-4 beam over the 62,642-row restriction of a 248,320-row fp32 head) by the numpy oracle in
float32, 1 warm-up and the median of 3; ``cpu_baseline_d5120_extrapolated`` scales a bounded
float32 sample of the metric's own d=5120 workload to one draft.
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


def flow_bytes(d, L, E, C, ffn=6, heads=8, ctx=8, fold=True):
    """Algorithmic HBM bytes of one predict_hidden: every fp16 weight byte once per time it is
    needed plus context in and hiddens out.  Per Euler step per chunk expert: the block weights
    (QKV, O, W1, W2 and the vectors; with the cross attention folded, the per-draft factors A and B
    of H x C rows instead of the cross q / out projections) and time_mlp[2] + out_norm/out_proj;
    once per draft: the cross K/V projection (and, folded, the cross q and out projections that
    build A and B, which are written once)."""
    vec = (3 + 1 + 1 + 1 + ffn + 1 + 6) * d                                        # 19d at ffn=6
    if fold:
        blk = (3 + 1 + 2 * ffn) * d * d + vec + 2 * heads * ctx * d                # 16d^2 + A, B
        per_draft = L * (4 * d * d + 4 * d + 2 * heads * ctx * d)
    else:
        blk = (3 + 1 + 1 + 1 + 2 * ffn) * d * d + vec                              # 18d^2 + 19d
        per_draft = L * (2 * d * d + 4 * d)
    per_step = L * blk + 2 * d * d + 5 * d
    halves = E * C * per_step + C * per_draft
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


def head_bytes_twopass(d, K, M, n_rows, rank=256, order=4, path_ffn=2):
    """Two-pass head over K depths: pass A reads the shortlist rows of lm_head once (the K marginal
    hiddens together); each depth reads its M candidate rows of lm_head and markov w2 in place, plus
    the PathHead weights as in the one-pass head."""
    total = n_rows * d * 2
    for s in range(1, K + 1):
        nlive = min(s, order)
        total += M * d * 2 + M * rank * 2
        total += (nlive * d * d + 2 * path_ffn * d * d) * 2
    return total


def measured_traffic(d, L, E):
    """HBM bytes per flow pass from the committed counter profile of this workload (FETCH_SIZE and
    WRITE_SIZE, calibrated with a 1 GiB copy), or None for a workload without one."""
    p = ROOT / "profiles" / f"flow_d{d}_L{L}_E{E}_traffic.json"
    if not p.exists():
        return None
    return int(json.loads(p.read_text())["traffic_bytes"])


def measured_gemm_traffic(M, d):
    """HBM bytes per launch of the packed batched head kernel from its committed counter profile
    (FETCH_SIZE and WRITE_SIZE, calibrated with a 1 GiB copy), or None without one."""
    p = ROOT / "profiles" / f"head_gemm_M{M}_d{d}_traffic.json"
    if not p.exists():
        return None
    return int(json.loads(p.read_text())["traffic_bytes"])


def head_compare(W, sl, d, dev, rows=4, k=8, iters=50):
    """One head top-k launch (rows x d fp16 hiddens, top-k per row, no markov bias) over the packed
    shortlist image (the drafter's path), the shortlist rows read in place, and the full vocabulary
    read in place: microseconds per call and the rows' bytes."""
    import torch
    from chain_flow_amd.head import ShortlistHead
    lm_w = W["lm_head.weight"]
    h = torch.randn(rows, d, generator=torch.Generator(device=dev).manual_seed(9), device=dev).half()
    res = {"rows": rows, "k": k, "shortlist_rows": int(sl.numel()), "full_rows": int(lm_w.shape[0])}
    for name, head in (("shortlist_packed", lambda: ShortlistHead(lm_w, sl, packed=True)),
                       ("shortlist_in_place", lambda: ShortlistHead(lm_w, sl, packed=False)),
                       ("full_in_place", lambda: ShortlistHead(lm_w, None, packed=False))):
        hd = head()
        for _ in range(5):
            hd.topk(h, k)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            hd.topk(h, k)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / iters
        nb = hd.n * d * 2
        res[name] = {"us": round(us, 2), "bytes": nb, "gbs": round(nb / (us * 1e-6) / 1e9, 1)}
        del hd
    return res


def calib_copy(dev):
    """One 1 GiB device copy: a kernel of known traffic for calibrating FETCH_SIZE / WRITE_SIZE."""
    import torch
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


LATENT, VAE_INTER, VAE_LAYERS = 640, 1920, 2


def vae_bytes(hidden, latent=LATENT, inter=VAE_INTER, layers=VAE_LAYERS, rows=8):
    """Algorithmic HBM bytes of one encode + one decode: every fp16 VAE weight once per pass (logvar
    unused), the position rows, the rows in and out."""
    per_layer = 12 * inter * inter + 13 * inter            # qkv, out, linear1/2 (+ biases, 2 norms)
    half = lambda kin, nout: (inter * kin + inter + 16 * inter + layers * per_layer + 2 * inter
                              + nout * inter + nout)
    return 2 * (half(hidden, latent) + half(latent, hidden)) + 2 * rows * (hidden + latent) * 2


def build_workload(d, L, E, device, latent=False, twopass=0):
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
    dr = Drafter(cfg, W, sl.to(device), device=device, twopass_m=twopass)
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


def host_threads():
    """The CPUs this process may run on (its affinity set), capped by OMP_NUM_THREADS when set: the
    host's share that the CPU baseline's BLAS threads use."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(n, 1)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline_c1(dev, reps=3):
    """The CPU reference plumbing run (C1), measured whole: a chain draft at d = 2560 in fp32 on the
    host -- TreeFlowDrafter.predict_hidden (L = 8 blocks, E = 8 Euler steps, 2 chunk experts,
    seeded N(0, 0.02) weights, N(0, 1) RMS-1 context) and the 5-token width-4 beam over a
    248,320 x 2560 fp32 head restricted to the seeded 62,642-id shortlist (path residual, markov
    bias, log-softmax top-k), plus the greedy (width-1) chain, timed apart.  The numpy oracle in
    float32 arithmetic with BLAS on this process's CPU share; 1 warm-up, median of ``reps``.  The
    weights are drawn on the GPU with the same per-parameter seeds and copied to the host (setup,
    not timed)."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits
    from chain_flow_amd.config import flownet
    from chain_flow_amd.shortlist import synthetic
    from chain_flow_amd.weights import make_weights, synthetic_context
    from oracle import beam as obeam
    from oracle import flow as oflow
    from oracle import head as ohead
    d, K, Wd = 2560, 5, 4
    cfg = flownet(d, layers=8, flow_steps=8)
    W = make_weights(cfg, VOCAB, init="baseline", dtype=torch.float32, device=dev, base_seed=0)
    sl = synthetic(VOCAB, SHORTLIST_ROWS, seed=2)
    sld = sl.long().to(dev)
    host = lambda t: t.detach().cpu().numpy()
    Wf = {k: host(v) for k, v in W.items() if k.startswith(("expert.", "extra_experts.", "path_head."))}
    w_sl = host(W["lm_head.weight"][sld])            # lm_w[sl], built once (flow_proposer.py:739)
    w2_sl = host(W["markov.w2.weight"][sld])
    w1 = host(W["markov.w1.weight"])
    emb = host(W["embed_tokens.weight"])
    del W, sld
    torch.cuda.empty_cache()
    ctx = synthetic_context(1, cfg.context_size, d, seed=1, dtype=torch.float32).numpy()
    known0 = np.array([int(sl[1234])])
    s64 = sl.long().numpy()
    ocfg = dict(draft_length=cfg.draft_length, chunk_size=cfg.chunk_size, num_layers=cfg.num_drafter_layers,
                num_heads=cfg.num_heads, num_flow_steps=cfg.num_flow_steps, init_mode=cfg.init_mode)
    score = lambda h, prev: ohead.head_with_bias(h, w_sl, w1, w2_sl, prev, numerics="fp32")
    resid = lambda lp, nl: ohead.path_residual(Wf, emb, lp, nl, cfg.path_order, numerics="fp32")

    def chain(pred, width):
        return obeam.beam_chains(pred, known0, s64, width, K, cfg.path_order, score, resid, numerics="fp32")

    n = host_threads()
    with threadpool_limits(limits=n):
        pred = oflow.predict_hidden(Wf, ctx, ocfg, numerics="fp32")       # warm-up
        chain(pred, Wd)
        ts, tg = [], []
        for _ in range(reps):
            t0 = time.perf_counter()
            pred = oflow.predict_hidden(Wf, ctx, ocfg, numerics="fp32")
            ids = chain(pred, Wd)
            t1 = time.perf_counter()
            greedy = chain(pred, 1)
            ts.append(t1 - t0)
            tg.append(time.perf_counter() - t1)
        # (untimed) the searches' decision margins, for the same-run comparison with the GPU's ids
        near = {}
        for name, width in (("chain", Wd), ("greedy", 1)):
            _, tr = obeam.beam_chains(pred, known0, s64, width, K, cfg.path_order, score, resid, numerics="fp32",
                                      return_trace=True)
            ms = [m for t in tr for m in (ohead.margins(t["lp"], width), ohead.margins(t["cand"], width)) if m.size]
            near[name] = min(float(m.min()) for m in ms)
    assert pred.dtype == np.float32
    med = lambda v: sorted(v)[len(v) // 2]
    return {"value": round(med(ts) * 1e6, 1), "unit": "us per draft step", "cores": n, "kind": "port",
            "sample": (f"whole C1 drafts: numpy oracle in float32 at d={d}, L=8, E=8 (predict_hidden) + the "
                       f"{K}-token width-{Wd} beam over the {SHORTLIST_ROWS}-row restriction of a {VOCAB}x{d} "
                       f"fp32 head; median of {reps} after 1 warm-up; {n} BLAS threads on a "
                       f"{cpu_model()} host (os.cpu_count() {os.cpu_count()})"),
            "runs_s": [round(t, 3) for t in ts],
            "greedy_chain_us": round(med(tg) * 1e6, 1),
            "chain_ids": [int(x) for x in ids[0]], "greedy_ids": [int(x) for x in greedy[0]],
            "min_decision_margin": {k: round(v, 6) for k, v in near.items()},
            "_pred": pred}


def c1_gpu_vs_cpu(dev, c1):
    """The same C1 draft on the GPU in fp16 (the weights of the CPU run rounded to fp16, the same
    context and known token): the predicted hiddens against the CPU's fp32 ones, and the chain and
    greedy ids against the CPU's, which must be equal wherever every decision margin of the CPU's
    search exceeds 1e-3."""
    import numpy as np
    import torch
    from chain_flow_amd.config import flownet
    from chain_flow_amd.drafter import Drafter
    from chain_flow_amd.shortlist import synthetic
    from chain_flow_amd.weights import make_weights, synthetic_context
    d, K = 2560, 5
    cfg = flownet(d, layers=8, flow_steps=8)
    W = make_weights(cfg, VOCAB, init="baseline", dtype=torch.float16, device=dev, base_seed=0)
    sl = synthetic(VOCAB, SHORTLIST_ROWS, seed=2)
    dr = Drafter(cfg, W, sl.to(dev), device=dev)
    del W
    ctx = synthetic_context(1, cfg.context_size, d, seed=1).to(dev)
    known0 = sl[1234:1235].long().to(dev)
    pred = dr.predict_hidden(ctx)
    chain = dr.beam_chains(None, known0, K, 4, pred=pred)[0].tolist()
    greedy = dr.beam_chains(None, known0, K, 1, pred=pred)[0].tolist()
    torch.cuda.synchronize()
    cpu_pred = c1["_pred"].astype(np.float64)
    gp = pred.double().cpu().numpy()
    err = float(np.linalg.norm(gp - cpu_pred) / np.linalg.norm(cpu_pred))
    out = {"pred_rel_err_fp16_vs_fp32": round(err, 6), "tolerance": 2e-3}
    for name, ids in (("chain", chain), ("greedy", greedy)):
        want = c1[f"{name}_ids"]
        margin = c1["min_decision_margin"][name]
        out[name] = {"gpu_ids": ids, "cpu_ids": want, "equal": ids == want, "cpu_min_margin": margin,
                     "required": margin > 1e-3}
    out["parity"] = all(out[n]["equal"] or not out[n]["required"] for n in ("chain", "greedy")) and err < 2e-3
    del dr
    torch.cuda.empty_cache()
    return out


def graph_replay_ms(step, warmup=10, replays=200):
    """The whole draft captured once in a HIP graph, ``warmup`` replays, then ``replays`` replays
    each timed with events on the replaying stream: (median ms, 10th and 90th percentiles)."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
    for a, b in ev:
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    t = sorted(a.elapsed_time(b) for a, b in ev)
    del g
    return t[len(t) // 2], t[len(t) // 10], t[(9 * len(t)) // 10]


def cpu_baseline(W, cfg, sl, d):
    """The CPU oracle on a bounded sample of the metric's own workload (d = 5120), scaled to one
    draft step: an extrapolation, reported beside the whole C1 run.

    Sample: one HiddenKVFlowBlock pass of each chunk expert (S = 4 and 8 rows), the cross K/V of
    one block of each expert, and one head depth (4 beams: fused path residual with 4 live offsets,
    62,642-row shortlist GEMV + markov bias, log-softmax), in float32.  One draft = E*L block passes
    of each expert + L cross K/V per expert + K head depths."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import flow as oflow
    from oracle import head as ohead
    cores = host_threads()
    f64 = lambda t: t.detach().float().cpu().numpy()
    rng = np.random.default_rng(0)
    lim = threadpool_limits(limits=cores)
    t_blocks = 0.0
    t_kv = 0.0
    for ci, p in enumerate(oflow.expert_prefixes(cfg.num_chunks)):
        bp = f"{p}blocks.0."
        Wb = {k: f64(v) for k, v in W.items() if k.startswith(bp)}
        S = (ci + 1) * cfg.chunk_size
        ctx = rng.standard_normal((1, cfg.context_size, d)).astype(np.float32)
        t0 = time.perf_counter()
        kv = oflow.cross_kv(Wb, bp, ctx, "fp32")
        t_kv += time.perf_counter() - t0
        res = rng.standard_normal((1, S, d)).astype(np.float32)
        mask = oflow.causal_mask(S)
        t0 = time.perf_counter()
        oflow.block_forward(Wb, bp, res, kv, mask, cfg.num_heads, "fp32")
        t_blocks += time.perf_counter() - t0
        del Wb
    slt = sl.long().cpu()
    Wh = {k: f64(v) for k, v in W.items() if k.startswith("path_head.")}
    emb = f64(W["embed_tokens.weight"][slt[:4096].to(W["embed_tokens.weight"].device)])
    lastp = np.arange(16).reshape(4, 4) % 4096
    w_sl = f64(W["lm_head.weight"][slt.to(W["lm_head.weight"].device)])
    w1 = f64(W["markov.w1.weight"][slt[:4096].to(W["markov.w1.weight"].device)])
    w2_sl = f64(W["markov.w2.weight"][slt.to(W["markov.w2.weight"].device)])
    pred = rng.standard_normal((d,)).astype(np.float32)
    t0 = time.perf_counter()
    res = ohead.path_residual(Wh, emb, lastp, 4, cfg.path_order, "fp32")
    h = ohead.r16(pred[None] + res, "fp32")
    logits = ohead.head_with_bias(h, w_sl, w1, w2_sl, lastp[:, 0])
    lp = ohead.log_softmax(logits)
    ohead.topk(lp, 4)
    t_head = time.perf_counter() - t0
    lim.unregister()
    E, L, K = cfg.num_flow_steps, cfg.num_drafter_layers, 5
    us = (E * L * t_blocks + L * t_kv + K * t_head) * 1e6
    return {"value": us, "unit": "us per draft step", "cores": int(cores), "kind": "port",
            "sample": (f"extrapolated: numpy oracle in float32 at d={d}: one block pass of "
                       f"each chunk expert ({t_blocks * 1e3:.0f} ms), one block's cross K/V per expert "
                       f"({t_kv * 1e3:.0f} ms), one 4-beam head depth over {SHORTLIST_ROWS} rows "
                       f"({t_head * 1e3:.0f} ms); scaled by E*L={E * L}, L={L}, K={K}")}


def verify_bench(dev, iters=200, warmup=20):
    """Per-launch times (us, HIP events over `iters` back-to-back launches) of the tree-verify kernels."""
    import ctypes as C
    import numpy as np
    import torch
    from chain_flow_amd import _lib
    L = _lib.lib()
    st = _lib.stream_handle()
    g = torch.Generator(device="cpu").manual_seed(5)
    bf = lambda *sh: torch.randn(*sh, generator=g).to(torch.bfloat16).to(dev)

    parent = np.array([-1] + [(i - 1) // 2 for i in range(1, 31)])   # 31 nodes: depth 5, two children each
    N, H, Dk, Dv = len(parent), 16, 128, 128
    par_d = torch.as_tensor(parent).to(dev, torch.int32)
    q, k, v = bf(N, H, Dk), bf(N, H, Dk), bf(N, H, Dv)
    gg = torch.nn.functional.logsigmoid(torch.randn(N, H, generator=g)).to(dev)
    beta = torch.rand(N, H, generator=g).to(dev)
    S0 = (torch.randn(H, Dk, Dv, generator=g) * 0.1).to(dev)
    out = torch.empty(N, H, Dv, device=dev)
    states = torch.empty(N, H, Dk, Dv, device=dev)
    # serving form: mixed_qkv rows, bf16 value-major slots
    HV = H
    mixed = bf(N, 2 * H * Dk + HV * Dv)
    a_, b_ = bf(N, HV), bf(N, HV)
    A_log, dt_bias = torch.randn(HV, generator=g).to(dev), torch.randn(HV, generator=g).to(dev)
    slots = torch.zeros(N + 2, HV, Dv, Dk, dtype=torch.bfloat16, device=dev)
    node_slots = torch.arange(2, N + 2, dtype=torch.int32, device=dev)
    o_vllm = torch.empty(N, HV, Dv, dtype=torch.bfloat16, device=dev)
    # tree conv over the GDN input channels
    dim = 2 * H * Dk + HV * Dv
    cx, cw, cb = bf(N, dim), bf(dim, 4), bf(dim)
    cst = bf(N + 2, dim, 4)
    cout = torch.empty(N, dim, dtype=torch.bfloat16, device=dev)
    # tree attention: one request, 40 nodes, 16 q heads over 4 kv heads, D 256
    TN, TH, THk, TD = 40, 16, 4, 256
    tq, tk, tv = bf(TN, TH, TD), bf(TN, THk, TD), bf(TN, THk, TD)
    tout, tpo = bf(TN, TH, TD), bf(TN, TH, TD)
    tpl = (torch.randn(TH, TN, generator=g) + 3).to(dev)
    # the shipped tree shape: keep 8 x depth 5 in BFS order, 8 roots, each later level's parents drawn
    # from the level above (at most 5 tree columns per row)
    trng = np.random.default_rng(1)
    tpar = np.array([-1] * 8 + [int(8 * (i // 8 - 1) + trng.integers(0, 8)) for i in range(8, TN)])
    nanc = np.ones((1, TN, TN), dtype=np.uint8)
    for n in range(TN):
        m = n
        while m >= 0:
            nanc[0, n, m] = 0
            m = tpar[m]
    tidx = torch.arange(TN, dtype=torch.int32, device=dev)
    tmask = torch.as_tensor(nanc).to(dev)
    # greedy accept: 41 rows of the full vocabulary
    V = VOCAB
    logits = bf(TN + 1, V)
    cu_d = torch.tensor([TN], dtype=torch.int32, device=dev)
    cu_s = torch.tensor([TN + 1], dtype=torch.int32, device=dev)
    dids = torch.randint(0, V, (TN,), generator=g).to(dev, torch.int32)
    dpar = torch.as_tensor(tpar).to(dev, torch.int32)
    otok = torch.empty(1, TN + 1, dtype=torch.int32, device=dev)
    opath = torch.empty(1, TN, dtype=torch.int32, device=dev)
    olen = torch.empty(1, dtype=torch.int32, device=dev)
    ra = torch.empty(TN + 1, dtype=torch.int32, device=dev)
    aws = torch.empty(int(L.cfh_tree_accept_ws_bytes(TN + 1)), dtype=torch.uint8, device=dev)
    kern = {
        "gdn_tree_with_states": lambda: L.cfh_gdn_tree(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), gg.data_ptr(), beta.data_ptr(), S0.data_ptr(),
            par_d.data_ptr(), N, H, Dk, Dv, 1, 0, out.data_ptr(), states.data_ptr(), st),
        "gdn_tree_outputs_only": lambda: L.cfh_gdn_tree(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), gg.data_ptr(), beta.data_ptr(), S0.data_ptr(),
            par_d.data_ptr(), N, H, Dk, Dv, 1, 0, out.data_ptr(), None, st),
        "gdn_serving_bf16_slots": lambda: L.cfh_gdn_tree_vllm(
            mixed.data_ptr(), a_.data_ptr(), b_.data_ptr(), A_log.data_ptr(), dt_bias.data_ptr(), slots.data_ptr(), 1,
            N + 2, node_slots.data_ptr(), par_d.data_ptr(), 1, N, H, HV, Dk, Dv, 1, C.c_float(Dk ** -0.5),
            o_vllm.data_ptr(), None, st),
        "tree_conv": lambda: L.cfh_tree_conv(
            cx.data_ptr(), dim, cst.data_ptr(), cw.data_ptr(), cb.data_ptr(), node_slots.data_ptr(), par_d.data_ptr(),
            1, N, dim, 1, cout.data_ptr(), dim, st),
        "tree_attn_merge": lambda: L.cfh_tree_attn_merge(
            tq.data_ptr(), TH * TD, tk.data_ptr(), THk * TD, tv.data_ptr(), THk * TD, tout.data_ptr(), TH * TD,
            tpo.data_ptr(), tpl.data_ptr(), tidx.data_ptr(), tmask.data_ptr(), C.c_float(TD ** -0.5), 1, TN, TH, THk,
            TD, 1, st),
        "tree_greedy_accept": lambda: L.cfh_tree_greedy_accept(
            logits.data_ptr(), V, V, TN + 1, 1, cu_d.data_ptr(), cu_s.data_ptr(), dids.data_ptr(), dpar.data_ptr(), 1,
            TN, otok.data_ptr(), opath.data_ptr(), olen.data_ptr(), ra.data_ptr(), aws.data_ptr(), st),
    }
    res = {}
    for name, fn in kern.items():
        for _ in range(warmup):
            _lib.check(fn(), name)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        res[name] = e0.elapsed_time(e1) * 1e3 / iters
    gdn_bytes = (H * Dk * Dv * 4 + 3 * N * H * Dk * 2 + 2 * N * H * 4 + N * H * Dv * 4 + N * H * Dk * Dv * 4
                 + N * 4)
    return res, gdn_bytes, N


def gemm_bench(dev, iters=100, warmup=10):
    import torch
    from chain_flow_amd.head import GemmHead
    M, d, V, n, k = 160, 4096, VOCAB, SHORTLIST_ROWS, 8
    g = torch.Generator(device=dev).manual_seed(4)
    W = (torch.randn(V, d, generator=g, device=dev) * (4.0 / d ** 0.5)).to(torch.bfloat16)
    from chain_flow_amd.shortlist import synthetic
    sl = synthetic(V, n, seed=2).to(dev)
    x = torch.randn(M, d, generator=g, device=dev).to(torch.bfloat16)
    times = {}
    for packed in (False, True):
        head = GemmHead(W, sl, packed=packed)
        for _ in range(warmup):
            head.topk(x, k)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            head.topk(x, k)
        e1.record()
        torch.cuda.synchronize()
        times["packed" if packed else "in_place"] = e0.elapsed_time(e1) * 1e-3 / iters
        del head
    nbytes = n * d * 2 + M * d * 2 + M * k * 8
    flops = 2.0 * M * n * d
    return times, nbytes, flops, (M, d, n, k)


def batched_bench(dev, steps=3, warmup=1, B=32, d=4096, L=8, E=8, M=8192, latent=False):
    """The batched drafting step: B requests, each a 5-token width-4 chain at d=4096 fp16 with the
    proposer's default two-pass head (M=8192 candidates shared across depths).  The flow drafts the
    requests in groups that share every weight stream (cfh_flow_group_size: 16 requests a group at
    d=4096); pass A scores the B*5 marginal hiddens in one fp16 MFMA GEMM
    over the 62,642-row shortlist (M=160 rows at B=32); each depth's B*4 beams run through the
    batched path residual and the grouped pass-B head.  Returns timings (ms, events on the stream)
    and byte counts."""
    import torch
    from chain_flow_amd.config import flownet
    from chain_flow_amd.drafter import Drafter
    from chain_flow_amd.flow import group_size
    from chain_flow_amd.shortlist import synthetic
    from chain_flow_amd.weights import make_weights, synthetic_context
    from chain_flow_amd.config import TreeVAEFlowConfig
    K, Wd = 5, 4
    if latent:
        # the shipped latent drafter (hidden d, VAE latent 640, the flow inside it at that width)
        cfg = TreeVAEFlowConfig(context_size=8, draft_length=8, chunk_size=4, expert_dim=d, num_heads=8,
                                ffn_multiplier=6, num_drafter_layers=L, num_flow_steps=E, init_mode="delta",
                                path_order=4, path_ffn_multiplier=2, markov_rank=256, latent_size=LATENT,
                                vae_intermediate_size=VAE_INTER, vae_num_layers=VAE_LAYERS, vae_num_heads=8,
                                vae_max_sequence_length=16)
    else:
        cfg = flownet(d, layers=L, flow_steps=E)
    W = make_weights(cfg, VOCAB, init="baseline", dtype=torch.float16, device=dev, base_seed=0, hidden=d)
    sl = synthetic(VOCAB, SHORTLIST_ROWS, seed=2)
    dr = Drafter(cfg, W, sl.to(dev), device=dev, twopass_m=M, twopass_shared=True)
    del W
    ctx = synthetic_context(B, cfg.context_size, d, seed=1).to(dev)
    known0 = sl[torch.randperm(SHORTLIST_ROWS, generator=torch.Generator().manual_seed(3))[:B]].long().to(dev)

    def step():
        pred = dr.predict_hidden(ctx)
        return pred, dr.beam_chains(None, known0, K, Wd, pred=pred)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record()
        pred = dr.predict_hidden(ctx)
        ev[i][1].record()
        dr.beam_chains(None, known0, K, Wd, pred=pred)
        ev[i][2].record()
    torch.cuda.synchronize()
    med = lambda v: sorted(v)[len(v) // 2]
    flow_ms = med([a.elapsed_time(b) for a, b, _ in ev])
    head_ms = med([b.elapsed_time(c) for _, b, c in ev])
    # pass A alone: the B*5 marginal hiddens through the fp16 GEMM head (the batched head of C4)
    hm = pred[:, 1:K + 1].contiguous()
    for _ in range(3):
        dr.head.candidates(hm, M, True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n_a = 20
    e0.record()
    for _ in range(n_a):
        dr.head.candidates(hm, M, True)
    e1.record()
    torch.cuda.synchronize()
    pass_a_ms = e0.elapsed_time(e1) / n_a
    # its two parts: the GEMM head with the logits written (+ the top-k merge), then the selection
    rows = hm.reshape(B * K, d)
    lg = torch.empty(B * K, dr.head.n, dtype=torch.float16, device=dev)
    o = (torch.empty(B * K, 1, device=dev), torch.empty(B * K, 1, dtype=torch.int32, device=dev),
         torch.empty(B * K, device=dev))
    for _ in range(3):
        dr.head.topk(rows, 1, logits=lg, out=o)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(n_a):
        dr.head.topk(rows, 1, logits=lg, out=o)
    e1.record()
    torch.cuda.synchronize()
    pass_a_gemm_ms = e0.elapsed_time(e1) / n_a
    R = group_size(cfg, B)
    groups = (B + R - 1) // R
    # the algorithm's bytes: every flow weight once for the whole batch (the reference's batched
    # path runs all 8 B rows against each weight tile); the kernels issue one stream per group, two
    # groups' streams side by side in every launch
    fd = LATENT if latent else d
    fb = flow_bytes(fd, L, E, cfg.num_chunks, fold=(fd // cfg.num_heads) % 32 == 0) + (vae_bytes(d) if latent else 0)
    return dict(flow_ms=flow_ms, head_ms=head_ms, pass_a_ms=pass_a_ms, pass_a_gemm_ms=pass_a_gemm_ms,
                flow_bytes=fb, groups=groups,
                pass_a_bytes=SHORTLIST_ROWS * d * 2 + B * K * d * 2 + B * K * SHORTLIST_ROWS * 2,
                R=R, B=B, d=d, L=L, E=E, M=M, K=K, W=Wd, latent=latent)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=["target", "latent", "verify", "gemm", "batched"], default="target",
                    help="target: the flow at the target width d (default); latent: the shipped 4B "
                         "latent drafter (hidden 2560, VAE latent 640, 8 blocks, 2 Euler steps)")
    ap.add_argument("--d", type=int, default=None, help="target hidden size (5120; latent: 2560)")
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--flow-steps", type=int, default=None, help="Euler steps (8; latent: 2)")
    ap.add_argument("--twopass", type=int, default=0,
                    help="two-pass candidate head with M candidates (0: the one-pass head of the metric)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--latent", action="store_true",
                    help="--workload batched: the shipped latent drafter (hidden 2560, VAE latent 640, L=8, E=2)")
    ap.add_argument("--no-graph", action="store_true",
                    help="skip the graph-replay timing (counter-collection runs: the profiler's counter "
                         "pass does not survive graph launches)")
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
    if args.workload == "gemm":
        times, nb, fl, (M, d_, n_, k_) = gemm_bench(dev)
        t = times["packed"]
        gbs = nb / t / 1e9
        out = {
            "metric": "us per batched head step (32 seqs x 5 depths = 160 rows, d=4096 bf16, shortlist top-8)",
            "value": round(t * 1e6, 2), "unit": "us per launch", "n_gpus": 1, "steps": 100, "warmup": 10,
            "ms_per_step": round(t * 1e3, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16", "data": "synthetic (seeded)",
            "config": {"workload": f"batched shortlisted head: M={M} rows x {n_}-row shortlist of a {VOCAB}-row "
                                   f"head, d={d_} bf16, fused log-softmax top-{k_}; shortlist rows packed once "
                                   f"(cfh_head_pack) into the MFMA fragment image"},
            "in_place_us": round(times["in_place"] * 1e6, 2),
            "mfma": {"achieved_tflops": round(fl / t / 1e12, 1), "peak_tflops": 2500.0,
                     "frac": round(fl / t / 1e12 / 2500.0, 4), "gflop": round(fl / 1e9, 1)},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_gemm_traffic(M, d_),
                         "kernel": "cfh_head_gemm_topk_packed",
                         "algorithmic_bytes": nb},
        }
        if args.calib_copy:
            calib_copy(dev)
        print(json.dumps(out), flush=True)
        return
    if args.workload == "batched":
        r = batched_bench(dev, latent=True, d=2560, E=2) if args.latent else batched_bench(dev)
        ms = r["flow_ms"] + r["head_ms"]
        gbs = r["flow_bytes"] / (r["flow_ms"] * 1e-3) / 1e9
        out = {
            "metric": (f"us per batched draft step ({r['B']} seqs x {r['K']} tokens, "
                       + (f"latent drafter hidden {r['d']} latent {LATENT}" if r["latent"] else f"d={r['d']}")
                       + " fp16, two-pass head)"),
            "value": round(ms * 1e3, 1), "unit": "us per batched draft step", "n_gpus": 1, "steps": 3, "warmup": 1,
            "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp16", "data": "synthetic (seeded N(0,0.02) weights, N(0,1) RMS-1 contexts)",
            "config": {"workload": f"batched chain draft: {r['B']} requests x {r['K']} tokens, width {r['W']}, "
                                   + (f"latent drafter (hidden {r['d']}, VAE latent {LATENT} width {VAE_INTER} "
                                      f"{VAE_LAYERS}+{VAE_LAYERS} layers, the flow at the latent width) "
                                      if r["latent"] else f"d={r['d']} ")
                                   + f"fp16, flow L={r['L']} E={r['E']} (requests drafted {r['R']} to a "
                                   f"weight stream: {r['groups']} groups), two-pass head M={r['M']} shared over a "
                                   f"{SHORTLIST_ROWS}-row shortlist"},
            "breakdown_ms": {"flow": round(r["flow_ms"], 3), "head_beam": round(r["head_ms"], 3)},
            "per_request_us": round(ms * 1e3 / r["B"], 1),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": "flow pass (cfh_flow_integrate, request groups)", "algorithmic_bytes": r["flow_bytes"],
                         "note": f"algorithmic bytes: every flow weight once for the whole batch"
                                 + (" (and the VAE's, encode + decode)" if r["latent"] else "")
                                 + f"; the kernels issue {r['groups']} weight streams ({r['R']} requests a "
                                 f"group), two groups' streams side by side in each launch"},
            "pass_a": {"rows": r["B"] * r["K"], "us": round(r["pass_a_ms"] * 1e3, 2),
                       "gemm_head_us": round(r["pass_a_gemm_ms"] * 1e3, 2),
                       "gemm_head_gbs": round(r["pass_a_bytes"] / (r["pass_a_gemm_ms"] * 1e-3) / 1e9, 1),
                       "selection_us": round((r["pass_a_ms"] - r["pass_a_gemm_ms"]) * 1e3, 2),
                       "what": "ShortlistHead.candidates: the fp16 GEMM head over the packed shortlist image "
                               "(logits written, top-1 and log-sum-exp merged) then cfh_cand_topm's top-M "
                               "selection per request; gemm_head_us times the first part alone"},
        }
        print(json.dumps(out), flush=True)
        return
    if args.workload == "verify":
        res, gb, N = verify_bench(dev)
        t = res["gdn_tree_with_states"]
        out = {
            "metric": "us per tree GDN state update with states (31-node tree, 16 heads, dk=dv=128)",
            "value": round(t, 2), "unit": "us per launch", "n_gpus": 1, "steps": 200, "warmup": 20,
            "ms_per_step": round(t / 1e3, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp32 state, bf16 q/k/v", "data": "synthetic (seeded)",
            "config": {"workload": f"tree verify kernels: {N}-node tree GDN (16 heads, dk=dv=128), serving "
                                   f"GDN bf16 slots, tree conv 6144 channels, tree attention 40 nodes x 16/4 heads "
                                   f"D 256 bf16, greedy accept 41 x {VOCAB}"},
            "breakdown_us": {k: round(v, 2) for k, v in res.items()},
            "roofline": {"bound": "hbm", "achieved": round(gb / (t * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gb / (t * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": "cfh_gdn_tree (states written)", "algorithmic_bytes": gb},
        }
        print(json.dumps(out), flush=True)
        return
    latent = args.workload == "latent"
    d = args.d or (2560 if latent else 5120)
    L = args.layers
    E = args.flow_steps or (2 if latent else 8)
    K, Wd = 5, 4
    print(f"[bench] building workload {args.workload} d={d} L={L} E={E}", file=sys.stderr, flush=True)
    cfg, W, dr, ctx, known0 = build_workload(d, L, E, dev, latent=latent, twopass=args.twopass)
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
        fb = flow_bytes(LATENT, L, E, cfg.num_chunks, fold=(LATENT // cfg.num_heads) % 32 == 0) + vae_bytes(d)
        traffic, kern = None, "predict_hidden pass (cfh_vae_encode + cfh_flow_integrate + cfh_vae_decode)"
        workload = (f"latent chain draft: hidden {d} fp16 bs1 K={K} width {Wd}; TransformerHiddenVAE latent "
                    f"{LATENT} (intermediate {VAE_INTER}, {VAE_LAYERS}+{VAE_LAYERS} layers); flow at {LATENT}, "
                    f"L={L} E={E} 2 chunk experts; shortlisted head {SHORTLIST_ROWS}x{d}")
        metric = "us per 5-token draft step (latent drafter: hidden 2560, VAE latent 640, bs1)"
    else:
        fb = flow_bytes(d, L, E, cfg.num_chunks, fold=(d // cfg.num_heads) % 32 == 0)
        traffic, kern = measured_traffic(d, L, E), "flow pass (cfh_flow_integrate)"
        workload = (f"chain draft d={d} fp16 bs1 K={K} width {Wd}, flow L={L} E={E} "
                    f"2 chunk experts, shortlisted head {SHORTLIST_ROWS}x{d}")
        metric = f"us per 5-token draft step (d={d}, bs1) + achieved HBM GB/s vs roofline"
    hb = (head_bytes_twopass(d, K, args.twopass, SHORTLIST_ROWS) if args.twopass
          else head_bytes(d, K, Wd, SHORTLIST_ROWS))
    if args.twopass:
        workload += f", two-pass head M={args.twopass} shared"
    flow_gbs = fb / (med(flow_ms) * 1e-3) / 1e9
    # the flow's bytes as the reference's algorithm needs them (cross q / out projections streamed in
    # every block pass), beside the folded algorithm's that `fb` counts
    fb_unfolded = flow_bytes(LATENT if latent else d, L, E, cfg.num_chunks, fold=False) + (vae_bytes(d) if latent else 0)
    graph = None
    if not args.no_graph:
        print("[bench] graph replays", file=sys.stderr, flush=True)
        g_med, g_p10, g_p90 = graph_replay_ms(lambda: dr.beam_chains(None, known0, K, Wd, pred=dr.predict_hidden(ctx)))
        graph = {"median_ms": round(g_med, 4), "p10_ms": round(g_p10, 4), "p90_ms": round(g_p90, 4),
                 "replays": 200, "warmup": 10,
                 "draft_frac": round((fb + hb) / (g_med * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                 "draft_frac_on_unfolded_bytes": round((fb_unfolded + hb) / (g_med * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                 "what": "the whole draft (predict_hidden + beam) captured once as a HIP graph, each replay "
                         "timed with events; a captured flow keeps its chunk experts on one stream"}
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
        "algorithmic_bytes": {"flow": fb, "flow_unfolded": fb_unfolded, "head": hb,
                              "draft_gbs": round((fb + hb) / (ms * 1e-3) / 1e9, 1),
                              "draft_gbs_unfolded": round((fb_unfolded + hb) / (ms * 1e-3) / 1e9, 1)},
        "roofline": {"bound": "hbm", "achieved": round(flow_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(flow_gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": kern,
                     "algorithmic_bytes": fb,
                     "frac_on_unfolded_bytes": round(fb_unfolded / (med(flow_ms) * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "note": ("frac counts the bytes the folded cross attention needs; frac_on_unfolded_bytes the "
                              "reference algorithm's (cross q / out projections in every block pass)")},
        "graph_replay": graph,
    }
    if latent:
        out["config"].update({"latent": LATENT, "vae_intermediate": VAE_INTER, "vae_layers": VAE_LAYERS})
    else:
        print("[bench] head comparison", file=sys.stderr, flush=True)
        out["head_compare"] = head_compare(W, dr.head.sl, d, dev)
    if args.calib_copy:
        calib_copy(dev)
    if not args.no_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        if latent:
            out["cpu_baseline"] = cpu_baseline_latent(W, cfg, dr.head.sl, d, ctx)
        else:
            out[f"cpu_baseline_d{d}_extrapolated"] = cpu_baseline(W, cfg, dr.head.sl, d)
            del W, dr
            torch.cuda.empty_cache()
            c1 = cpu_baseline_c1(dev)
            print("[bench] C1 on the GPU against the CPU run", file=sys.stderr, flush=True)
            out["c1_gpu_vs_cpu"] = c1_gpu_vs_cpu(dev, c1)
            c1.pop("_pred")
            out["cpu_baseline"] = c1
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
