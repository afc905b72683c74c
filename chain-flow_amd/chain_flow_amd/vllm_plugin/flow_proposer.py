"""``FlowDrafterProposer``: the ``custom_class`` speculative proposer surface, over the MI355X kernels.

Mirrors ``chain_flow.vllm_plugin.flow_proposer.FlowDrafterProposer`` (``cf/vllm_plugin/flow_proposer.py``):

* constructor ``FlowDrafterProposer(vllm_config)`` reads ``speculative_config.num_speculative_tokens``,
  ``scheduler_config.max_num_seqs`` and the same ``CF_*`` / ``VLLM_SPEC_TREE`` environment with the
  same validation and messages (``:330-389``);
* ``_build`` loads the drafter checkpoint directory -- ``chained_flow_tree_config.json``
  (``model_args``) and ``model.safetensors`` (keys prefixed ``drafter.``), applies ``CF_FLOW_STEPS``,
  checks the chain / tree emit limits, and resolves the shortlist with the same order, vocabulary
  guard and declared-identity check (``:579-765``, ``:1006-1016``; ``cf/defaults.py:210-244``);
* ``_draft_fn(ctx [B, C, d], known0 [B])`` is ``_beam_chains`` -> ``[B, K]`` or ``_beam_tree`` ->
  ``[B, 2N]`` (``:1187-1332``), run by ``chain_flow_amd.drafter.Drafter`` on the HIP kernels;
* ``propose(sampled_token_ids, num_tokens_no_spec, token_ids_cpu, slot_mappings=None, **kw)`` returns
  ``list[list[int]]`` (``:1698``, ``:2494-2569``), or with ``CF_ASYNC_SPEC=1`` the GPU int32 tensor
  ``[num_reqs, draft_width]`` indexed by batch row with no host read (``_async_draft_tensor``,
  ``:2326-2357``);
* the head is the two-pass candidate head by default (``CF_TWOPASS_M=8192``, ``CF_TWOPASS_SHARED=1``,
  ``CF_TWOPASS_SEED=0``; ``:1113-1184``, ``cf/defaults.py:123-127``), dropped when M does not fit
  the head unless it was asked for;
* the context lives in a device ring per batch slot (``_ring_write`` / ``_ring_gather``,
  ``:916-961``; ``cfh_ring_step``), with the slot lifecycle of ``_ctx_gpu`` (``:2045-2105``: a new
  request resets or seeds its slot, a request moved by vLLM's batch condense carries its history),
  and the ring step + draft run as one captured graph per batch bucket (``CF_CUDAGRAPH``,
  ``CF_DRAFT_BUCKETS``; ``:1342-1365, 1511-1589``) wherever the draft is launch-bound; where the
  flow's chunk experts run on concurrent streams the draft runs eagerly (the reference pairs its
  chunk experts on two streams inside its graphs, ``cf/cuda_block.py:452-466``; a captured HIP
  flow keeps them on one stream, which is slower than the eager overlap).

Drafters: the reference builds every checkpoint as the latent ``TreeVAEFlowDrafter``
(``:583, 616-632``), with the VAE from ``CF_VAE_DIR`` / the config's ``vae_dir`` overlaid by the
checkpoint's own ``drafter.vae.*`` tensors; so does this proposer for any checkpoint that carries
VAE fields or tensors.  A checkpoint with neither is served as the target-width ``TreeFlowDrafter``
(``expert_dim`` = target hidden size), the form the synthetic d = 2560 / 5120 workloads use.
Profiling: ``CF_PROFILE=1`` (host-timed sections of every draft, draft graphs off) and
``CF_DRAFTPROF=1`` (a one-off event timing of the draft and its pieces per batch bucket), as the
reference's hooks of the same names (``:400-401, 1364-1424``).
What differs, by design: no Hugging Face download (``CF_DRAFTER_DIR`` must be a local directory),
no torch.compile.  An ``anchor_token`` drafter is given the committed token's embedding on every
draft (``:1199-1203``); ``lag_context`` only changes training contexts, so it loads and drafts as
the reference's proposer runs it (its ``lag_proj`` unused).
The target's final hidden states reach the proposer through :meth:`stash_hidden_states` (the
reference monkeypatches ``GPUModelRunner.propose_draft_token_ids`` to stash
``sample_hidden_states``, ``:40-59``) and the target's input embeddings and ``lm_head`` weight
through :meth:`bind_target` (the reference reads them off ``runner.model``, ``:585-590``).
"""
from __future__ import annotations

import dataclasses
import json
import os
from pathlib import Path

import torch

from chain_flow_amd import shortlist as _sl
from chain_flow_amd.config import TreeFlowConfig, TreeVAEFlowConfig
from chain_flow_amd.drafter import Drafter
from chain_flow_amd.graph import DraftGraphs, bucket_ladder
from chain_flow_amd.ring import ContextRing
from chain_flow_amd.vae import load_vae_dir

CONFIG_NAME = "chained_flow_tree_config.json"
WEIGHTS_NAME = "model.safetensors"
PACKAGED_SHORTLIST = Path(__file__).resolve().parents[1] / "data" / "shortlist_qwen3_5.pt"


def shortlist_candidates(drafter_dir: str | None) -> list[tuple[str, str]]:
    """Shortlists to try, best first, as (path, provenance) (``cf/defaults.py:210-244``): the
    drafter checkpoint's own ``shortlist.pt``, then the packaged list (if installed)."""
    out: list[tuple[str, str]] = []
    if drafter_dir and os.path.isdir(drafter_dir):
        p = Path(drafter_dir) / "shortlist.pt"
        if p.is_file():
            out.append((str(p), "drafter checkpoint"))
    if PACKAGED_SHORTLIST.is_file():
        out.append((str(PACKAGED_SHORTLIST), "packaged"))
    return out


VAE_FIELDS = {f.name for f in dataclasses.fields(TreeVAEFlowConfig)} - {
    f.name for f in dataclasses.fields(TreeFlowConfig)}


def _checkpoint_has_vae(ckd: str) -> bool:
    from safetensors import safe_open
    path = os.path.join(ckd, WEIGHTS_NAME)
    if not os.path.exists(path):
        return False
    with safe_open(path, framework="pt") as f:
        return any(k.startswith("drafter.vae.") for k in f.keys())


def load_drafter_config(ckd: str) -> TreeFlowConfig:
    """``model_args`` of ``chained_flow_tree_config.json`` -> config, with the ``CF_FLOW_STEPS``
    inference override (``flow_proposer.py:616-631``): ``TreeVAEFlowConfig`` when the checkpoint
    carries VAE fields or ``drafter.vae.*`` tensors, else the target-width ``TreeFlowConfig``."""
    with open(os.path.join(ckd, CONFIG_NAME)) as f:
        margs = json.load(f)["model_args"]
    arch = margs.get("architecture", "tree_flow")
    if arch != "tree_flow":
        raise ValueError(f"drafter architecture {arch!r} is not supported (TreeFlowConfig.architecture "
                         f"must be 'tree_flow')")
    kind = TreeVAEFlowConfig if (VAE_FIELDS & set(margs) or _checkpoint_has_vae(ckd)) else TreeFlowConfig
    fields = {f.name for f in dataclasses.fields(kind)}
    cfg = kind(**{k: v for k, v in margs.items() if k in fields})
    fs = os.environ.get("CF_FLOW_STEPS")
    if fs:
        n = int(fs)
        if n < 1:
            raise ValueError(f"CF_FLOW_STEPS must be >= 1, got {n}")
        cfg.num_flow_steps = n
    return cfg


def load_drafter_weights(ckd: str, dtype=torch.float16, device="cpu") -> dict:
    """``drafter.``-prefixed tensors of ``model.safetensors``, prefix stripped (``:638-640``)."""
    from safetensors.torch import load_file
    sd = load_file(os.path.join(ckd, WEIGHTS_NAME), device="cpu")
    return {k[len("drafter."):]: v.to(device, dtype) for k, v in sd.items() if k.startswith("drafter.")}


def declared_shortlist(ckd: str) -> dict:
    """The optional ``shortlist`` block {rows, ids_sha256} of the drafter config (``:1006-1016``)."""
    try:
        with open(os.path.join(ckd, CONFIG_NAME)) as f:
            return json.load(f).get("shortlist") or {}
    except Exception:
        return {}


def resolve_shortlist(ckd: str, vocab_size: int, explicit: str | None):
    """(ids int32 | None, provenance) -- ``_build``'s resolution (``:680-765``).

    ``explicit`` = the value of ``CF_SHORTLIST`` when it is set: a path (must exist) or "" (full
    head by request).  Candidates built for another vocabulary are refused and the next is tried;
    a list whose content differs from the drafter's declared identity raises."""
    if explicit is not None and explicit != "":
        if not os.path.exists(explicit):
            raise FileNotFoundError(f"CF_SHORTLIST={explicit} does not exist")
        cands = [(explicit, "CF_SHORTLIST")]
    elif explicit == "":
        return None, "explicit CF_SHORTLIST='' -- FULL HEAD by request"
    else:
        cands = shortlist_candidates(ckd)
    rejected = []
    for path, src in cands:
        ids, meta = _sl.load(path)
        bad = _sl.check(ids, meta, vocab_size)
        if bad:
            rejected.append(f"{src} {path}: {bad}")
            continue
        sl = _sl.resolve(ids, vocab_size)
        decl = declared_shortlist(ckd)
        if decl:
            got = _sl.ids_content_sha(sl)
            want_rows, want_sha = decl.get("rows"), decl.get("ids_sha256")
            if (want_rows and int(want_rows) != sl.numel()) or (want_sha and want_sha != got):
                raise RuntimeError(
                    "shortlist does not match what this drafter declares.\n"
                    f"  resolved : {path}  [{src}]\n"
                    f"             {sl.numel()} rows, ids-sha256 {got}\n"
                    f"  declared : {want_rows} rows, ids-sha256 {want_sha}")
        return sl, f"{src} {os.path.basename(path)}"
    why = "FULL HEAD -- every candidate refused: " + " | ".join(rejected) if rejected else "FULL HEAD"
    return None, why


class FlowDrafterProposer:
    def __init__(self, vllm_config):
        spec = vllm_config.speculative_config
        self.tree = os.environ.get("VLLM_SPEC_TREE", "0") == "1"
        self.tree_keep = int(os.environ.get("CF_TREE_KEEP", "4"))
        self.tree_topb = int(os.environ.get("CF_TREE_TOPB", "8"))
        self.tree_depth = int(os.environ.get("CF_TREE_DEPTH", "4"))
        self.branching = self.tree and os.environ.get("CF_TREE_BRANCH", "1") == "1"
        if self.branching and self.tree_keep > self.tree_topb:
            raise ValueError(
                f"CF_TREE_KEEP={self.tree_keep} > CF_TREE_TOPB={self.tree_topb}: depth 1 expands "
                f"a single node, so it can hold at most {self.tree_topb} children while "
                f"N=keep*depth assumes {self.tree_keep}. Raise CF_TREE_TOPB to >= CF_TREE_KEEP.")
        self.N = self.tree_keep * self.tree_depth
        if self.branching:
            if int(spec.num_speculative_tokens) != self.N + 1:
                raise AssertionError(
                    f"set num_speculative_tokens={self.N + 1} for "
                    f"CF_TREE_KEEP={self.tree_keep} x CF_TREE_DEPTH={self.tree_depth}")
        self.K = int(spec.num_speculative_tokens) - (1 if self.tree else 0)
        self.draft_width = self.N if self.branching else self.K
        self.width = int(os.environ.get("CF_WIDTH", "4"))
        # the beam kernels' limits: a chain step ranks W*W candidates, a tree step keep*topb children
        if not self.tree and not 1 <= self.width <= 8:
            raise ValueError(f"CF_WIDTH={self.width} is not supported by this build: the beam step ranks "
                             f"width*width <= 64 candidates per request (CF_WIDTH 1..8)")
        if self.tree and (self.tree_keep < 1 or self.tree_topb < 1 or self.tree_keep * self.tree_topb > 64):
            raise ValueError(f"CF_TREE_KEEP={self.tree_keep} x CF_TREE_TOPB={self.tree_topb} is not supported by "
                             f"this build: a tree step ranks keep*topb <= 64 children per request")
        self.ckd = os.environ.get("CF_DRAFTER_DIR")
        if not self.ckd:
            raise ValueError("set CF_DRAFTER_DIR to the drafter checkpoint dir")
        if not os.path.isdir(self.ckd):
            raise ValueError(f"CF_DRAFTER_DIR={self.ckd} is not a directory (this build loads local "
                             f"checkpoints only; download the repo first)")
        self.shortlist_path = os.environ.get("CF_SHORTLIST")
        self.max_reqs = int(vllm_config.scheduler_config.max_num_seqs)
        self.path_trim = os.environ.get("CF_PATH_TRIM", "1") != "0"
        # CF_CUDAGRAPH: "1" (default) captures the ring step + draft per batch bucket where the draft
        # is bound by launch latency, and runs it eagerly where the flow's chunk experts run on
        # concurrent streams (a captured flow keeps them on one stream and is slower: d = 5120,
        # 20.9 against 19.7 ms a draft); "force" always captures, "0" never does
        cg = os.environ.get("CF_CUDAGRAPH", "1")
        if cg not in ("0", "1", "force"):
            raise ValueError(f"CF_CUDAGRAPH={cg!r}: expected 0, 1 or force")
        # CF_PROFILE=1: host-timed sections of every draft (each section synchronises), printed every
        # CF_PROFILE_EVERY steps; it turns the draft graphs off, as in the reference (:400-401).
        # CF_DRAFTPROF=1: a one-off GPU timing of the draft and its pieces when a batch bucket is
        # first drafted (events, no per-step synchronisation; :1364-1424).
        self.prof = os.environ.get("CF_PROFILE", "0") == "1"
        self.prof_every = int(os.environ.get("CF_PROFILE_EVERY", "100") or 100)
        self.draftprof = os.environ.get("CF_DRAFTPROF", "0") == "1"
        self._t = {"ring": 0.0, "flow": 0.0, "search": 0.0, "steps": 0}
        self._draftprof_done: set = set()
        self.use_cg = cg != "0" and not self.prof
        self.force_cg = cg == "force"
        # two-pass candidate head, on by default as in the reference's defaults table
        # (cf/defaults.py:123-127): M = CF_TWOPASS_M (8192), one candidate set for all depths
        # (CF_TWOPASS_SHARED=1), pass A on the bare marginals (CF_TWOPASS_SEED=0)
        self._twopass_explicit = "CF_TWOPASS_M" in os.environ
        self.twopass_m = int(os.environ.get("CF_TWOPASS_M", "8192") or 0)
        self.twopass_shared = os.environ.get("CF_TWOPASS_SHARED", "1") == "1"
        self.twopass_seed = os.environ.get("CF_TWOPASS_SEED", "0") == "1"
        self.async_spec = os.environ.get("CF_ASYNC_SPEC", "0") == "1"
        self.drafter: Drafter | None = None
        self._target = None
        self._hidden = None
        self._slot_req: list = [None] * self.max_reqs       # request id held by each batch slot
        self._req_slot: dict = {}
        self._dtok = None

    # ---- what the reference reads off the engine ------------------------------------------
    def bind_target(self, embed_w: torch.Tensor, lm_w: torch.Tensor) -> None:
        """The target's input embeddings [V, d] and lm_head weight [V, d] (device tensors)."""
        if embed_w.shape != lm_w.shape:
            raise ValueError("embed_tokens and lm_head must both be [V, d]")
        self._target = (embed_w, lm_w)

    def stash_hidden_states(self, hidden: torch.Tensor) -> None:
        """Final hidden states of the tokens just sampled, one row per entry of the next
        ``propose`` call's flattened ``sampled_token_ids`` (the reference's stash hook)."""
        self._hidden = hidden

    # ---- build -----------------------------------------------------------------------------
    def _build(self):
        if self._target is None:
            raise RuntimeError("bind_target(embed_w, lm_w) before the first propose")
        embed_w, lm_w = self._target
        self.dev = embed_w.device
        V, H = lm_w.shape
        cfg = load_drafter_config(self.ckd)
        latent = isinstance(cfg, TreeVAEFlowConfig)
        if not latent and cfg.expert_dim != H:
            raise ValueError(f"drafter expert_dim={cfg.expert_dim} but the target hidden size is {H}")
        vae_sd = load_vae_dir(cfg) if latent else None     # raises as _load_frozen_vae does
        if self.branching:
            emit = min(self.tree_depth, cfg.draft_length - 1)
            if emit != self.tree_depth:
                raise ValueError(
                    f"CF_TREE_DEPTH={self.tree_depth} but the drafter can only emit "
                    f"{emit} levels (draft_length={cfg.draft_length}). Set CF_TREE_DEPTH<={emit} and "
                    f"num_speculative_tokens={self.tree_keep * emit + 1}.")
        else:
            emit = cfg.draft_length - 1
            if self.K > emit:
                raise ValueError(
                    f"num_speculative_tokens={self.K} but this drafter can only emit {emit} "
                    f"chain tokens (draft_length={cfg.draft_length}; depth 0 reconstructs the "
                    f"token that was already committed). Set num_speculative_tokens<={emit}.")
        weights = load_drafter_weights(self.ckd, torch.float16, self.dev)
        if vae_sd:
            # the drafter checkpoint's own vae.* tensors win (load_state_dict after the VAE load)
            for k, v in vae_sd.items():
                weights.setdefault(k, v.to(self.dev, torch.float16))
        weights["lm_head.weight"] = lm_w.to(torch.float16)
        weights["embed_tokens.weight"] = embed_w.to(torch.float16)
        explicit = self.shortlist_path if "CF_SHORTLIST" in os.environ else None
        sl, self.shortlist_source = resolve_shortlist(self.ckd, V, explicit)
        self.cfg = cfg
        rows = V if sl is None else int(sl.numel())
        if self.twopass_m >= rows:
            # a two-pass head as wide as the head it narrows buys nothing: refuse an explicit
            # request, quietly drop the default (flow_proposer.py:766-775)
            if self._twopass_explicit:
                raise ValueError(f"CF_TWOPASS_M={self.twopass_m} >= head rows {rows}")
            self.twopass_m, self.twopass_shared = 0, False
        self.drafter = Drafter(cfg, weights, None if sl is None else sl.to(self.dev), device=self.dev,
                               path_trim=self.path_trim, twopass_m=self.twopass_m,
                               twopass_shared=self.twopass_shared, twopass_seed=self.twopass_seed)
        self.ctx_size = cfg.context_size
        # rows one request can append per step: the committed token plus every accepted draft
        self.kmax = (self.tree_depth + 1) if self.branching else (self.K + 1)
        self.ring = ContextRing(self.max_reqs, self.ctx_size, H, device=self.dev)
        capture = self.use_cg and (self.force_cg or not self.drafter.flow.concurrent)
        self.graphs = (DraftGraphs(self.ring, self._draft_fn, self.kmax, bucket_ladder(self.max_reqs))
                       if capture else None)

    # ---- drafting --------------------------------------------------------------------------
    def _search(self, ctx: torch.Tensor, known0: torch.Tensor, pred: torch.Tensor | None = None) -> torch.Tensor:
        if self.branching:
            return self.drafter.beam_tree(ctx, known0, keep=self.tree_keep, topb=self.tree_topb,
                                          depth=self.tree_depth, pred=pred)
        return self.drafter.beam_chains(ctx, known0, self.K, width=self.width, pred=pred)

    def _draft_fn(self, ctx: torch.Tensor, known0: torch.Tensor) -> torch.Tensor:
        if not self.prof:
            return self._search(ctx, known0)
        import time
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        pred = self.drafter.predict_hidden(ctx, known0)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        out = self._search(ctx, known0, pred)
        torch.cuda.synchronize()
        self._t["flow"] += t1 - t0
        self._t["search"] += time.perf_counter() - t1
        return out

    def _profile_step(self, t_ring: float) -> None:
        """CF_PROFILE: accumulate this step and print the running means every prof_every steps."""
        t = self._t
        t["ring"] += t_ring
        t["steps"] += 1
        if t["steps"] % self.prof_every == 0:
            n = t["steps"]
            print(f"[chain-flow] profile over {n} drafts (ms each, host-synchronised): ring "
                  f"{t['ring'] * 1e3 / n:.3f}, predict_hidden {t['flow'] * 1e3 / n:.3f}, "
                  f"{'tree' if self.branching else 'beam'} search {t['search'] * 1e3 / n:.3f}", flush=True)

    def _draft_breakdown(self, ctx: torch.Tensor, known0: torch.Tensor, bucket: int) -> None:
        """CF_DRAFTPROF: one GPU timing (events, mean of 20 after 3 warm-ups) of the draft and its pieces
        for this batch bucket, printed once: whether a draft is launch-bound or GPU-bound."""
        d = self.drafter

        def t(fn, n=20):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(n):
                fn()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) / n

        pred = d.predict_hidden(ctx, known0)
        parts = [("predict_hidden", lambda: d.predict_hidden(ctx, known0))]
        if d.vae is not None:
            lat = d.vae.encode(ctx.to(d.device, torch.float16))
            anc = d.flow.anchor(known0, d.path.embed_w) if d.anchored else None
            z = d.flow.predict_hidden(lat, anchor=anc)
            if d.anchored:
                parts += [("  anchor rows", lambda: d.flow.anchor(known0, d.path.embed_w))]
            parts += [("  vae encode", lambda: d.vae.encode(ctx.to(d.device, torch.float16))),
                      ("  flow integrate", lambda: d.flow.predict_hidden(lat, anchor=anc)),
                      ("  vae decode", lambda: d.vae.decode(z))]
        parts += [("beam/tree search", lambda: self._search(ctx, known0, pred)),
                  ("  one shortlist head", lambda: d.head.topk(pred[:, 0].contiguous(), 8)),
                  ("eager whole draft", lambda: self._search(ctx, known0))]
        print(f"[cf-draftprof] bucket={bucket} GPU ms (mean of 20):", flush=True)
        for name, fn in parts:
            print(f"[cf-draftprof]   {name:28s} {t(fn):8.3f}", flush=True)

    def _lifecycle(self, rows, req_ids) -> list[int]:
        """Slot bookkeeping of ``_ctx_gpu`` (``:2045-2080``): returns the slots that hold a NEW request
        (reset, then seeded or started empty); a live request found in another slot is moved with
        its history.  Without request ids every slot is taken to keep its request."""
        if req_ids is None:
            return []
        fresh, migrate = [], []
        for i in rows:
            rid = req_ids[i] if i < len(req_ids) else str(i)
            if self._slot_req[i] == rid:
                continue
            old = self._req_slot.get(rid)
            if old is not None and old != i and self._slot_req[old] == rid:
                migrate.append((i, old))
            else:
                fresh.append(i)
            self._slot_req[i] = rid
            self._req_slot[rid] = i
        live = set(req_ids)
        for k in [k for k in self._req_slot if k not in live]:
            self._req_slot.pop(k, None)
        self.ring.migrate(migrate)
        if fresh:
            self.ring.reset(fresh)
        return fresh

    def _async_draft_tensor(self, ch: torch.Tensor, rows, nreq: int) -> torch.Tensor:
        """[nreq, draft_width] int32 on the device, one row per batch slot (zeros where no draft),
        in a persistent buffer (``:2326-2357``)."""
        N = self.draft_width
        if int(ch.shape[1]) < N:
            raise AssertionError(f"draft is {tuple(ch.shape)} but {N} columns were declared to vLLM")
        if self._dtok is None:
            self._dtok = torch.zeros((self.max_reqs, N), dtype=torch.int32, device=ch.device)
        v = self._dtok[:nreq]
        v.zero_()
        v.index_copy_(0, torch.tensor(rows, device=ch.device), ch[:len(rows), :N].to(v.dtype))
        return v

    @torch.inference_mode()
    def propose(self, sampled_token_ids, num_tokens_no_spec=None, token_ids_cpu=None, slot_mappings=None,
                **kw):
        """sampled_token_ids: per request (batch slot), the tokens committed this step (list of lists).
        The stashed hidden states hold one row per committed token, requests in order.  Returns the
        next draft per request: K chain tokens, or the N tree tokens (their parents are kept in
        ``self.last_parents``); with ``CF_ASYNC_SPEC=1`` the device tensor instead.
        kw: ``hidden_states`` (instead of the stash), ``req_ids`` (slot lifecycle)."""
        if self.drafter is None:
            self._build()
        hidden = kw.get("hidden_states", self._hidden)
        if hidden is None:
            raise RuntimeError("no hidden states: stash_hidden_states() before propose()")
        hidden = hidden.to(self.dev, torch.float16)
        nreq = len(sampled_token_ids)
        if nreq > self.max_reqs:
            raise ValueError(f"{nreq} requests exceed max_num_seqs={self.max_reqs}")
        rows, starts, cnt, known, wmask = [], [], [], [], []
        off = 0
        for i, toks in enumerate(sampled_token_ids):
            n = len(toks)
            if n == 0:
                continue
            rows.append(i)
            starts.append(off)
            cnt.append(n)
            wmask.append(1)
            known.append(int(toks[-1]))
            off += n
        fresh = set(self._lifecycle(rows, kw.get("req_ids")))
        for j, i in enumerate(rows):
            if cnt[j] > self.kmax:
                # more rows than one step appends (a prefill): they seed the slot, as the
                # reference's _seed_prompt_ctx does, and are not appended again
                self.ring.seed(i, hidden[starts[j]:starts[j] + cnt[j]])
                wmask[j], cnt[j] = 0, 0
            elif i in fresh:
                pass                    # reset above: this step's rows start the history
        if not rows:
            return torch.zeros(nreq, self.draft_width, dtype=torch.int32, device=self.dev) \
                if self.async_spec else [[] for _ in sampled_token_ids]
        sh = hidden[:off]
        if self.graphs is not None and self.graphs.bucket_for(len(rows)) is not None:
            draft = self.graphs.run(sh, rows, starts, cnt, known, wmask)
            bucket = self.graphs.bucket_for(len(rows))
            if self.draftprof and bucket not in self._draftprof_done:
                self._draftprof_done.add(bucket)
                g = self.graphs._g[bucket]
                # replays with zero counts append nothing to the ring: each recomputes this step's draft
                cnt = g[1]["cnt"].clone()
                g[1]["cnt"].zero_()
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                for _ in range(20):
                    g[0].replay()
                b.record()
                g[1]["cnt"].copy_(cnt)
                torch.cuda.synchronize()
                print(f"[cf-draftprof] bucket={bucket} graph replay (ring step + whole draft, mean of 20) "
                      f"{a.elapsed_time(b) / 20:8.3f} ms", flush=True)
                self._draft_breakdown(g[1]["ctx"], g[1]["k0"], bucket)
        else:
            import time
            t0 = time.perf_counter()
            if self.prof:
                torch.cuda.synchronize()
            ctx = self.ring.step(sh, rows, starts, cnt, wmask, kmax=self.kmax)
            if self.prof:
                torch.cuda.synchronize()
                t_ring = time.perf_counter() - t0
            k0 = torch.tensor(known, device=self.dev, dtype=torch.long)
            if self.draftprof and len(rows) not in self._draftprof_done:
                self._draftprof_done.add(len(rows))
                self._draft_breakdown(ctx, k0, len(rows))
            draft = self._draft_fn(ctx, k0)
            if self.prof:
                self._profile_step(t_ring)
        if self.async_spec:
            return self._async_draft_tensor(draft, rows, nreq)
        draft = draft.cpu().tolist()                 # the one device -> host sync
        out = [[] for _ in sampled_token_ids]
        self.last_parents = {}
        for j, i in enumerate(rows):
            if self.branching:
                Nn = len(draft[j]) // 2
                out[i] = draft[j][:Nn]
                self.last_parents[i] = draft[j][Nn:]
            else:
                out[i] = draft[j]
        return out
