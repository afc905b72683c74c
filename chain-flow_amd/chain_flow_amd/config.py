"""Drafter configuration: the fields of the reference's ``TreeFlowConfig``
(``cf/drafters/tree_flow.py:40-77``) that shape the drafting hot path, with its validation rules.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass


@dataclass
class TreeFlowConfig:
    context_size: int = 8
    draft_length: int = 4
    chunk_size: int = 4
    expert_dim: int = 1024          # must equal the target LM hidden size
    num_heads: int = 8
    ffn_multiplier: int = 6
    num_drafter_layers: int = 8
    num_flow_steps: int = 2
    init_mode: str = "delta"
    noise_scale: float = 1.0        # init_mode="noise": z0 = randn * noise_scale
    markov_rank: int = 256
    path_order: int = 4
    path_ffn_multiplier: int = 2
    architecture: str = "tree_flow"

    def __post_init__(self) -> None:
        # same checks and messages as the reference (cf/drafters/tree_flow.py:67-77)
        if self.draft_length % self.chunk_size != 0:
            raise ValueError("draft_length must be divisible by chunk_size")
        if self.markov_rank < 1:
            raise ValueError("markov_rank must be >= 1")
        if not 1 <= self.path_order <= self.draft_length:
            raise ValueError("path_order must be in [1, draft_length]")
        if self.init_mode not in {"noise", "repeat_last", "delta"}:
            raise ValueError("init_mode must be 'noise', 'repeat_last', or 'delta'")
        if self.architecture != "tree_flow":
            raise ValueError("TreeFlowConfig.architecture must be 'tree_flow'")
        if self.num_flow_steps < 1:
            raise ValueError("num_flow_steps must be >= 1")

    @property
    def num_chunks(self) -> int:
        return self.draft_length // self.chunk_size

    @property
    def flow_dim(self) -> int:
        """Width the chunk experts run at: the target hidden size here, the latent size in the VAE
        drafter."""
        return self.expert_dim

    def to_dict(self) -> dict:
        return asdict(self)


@dataclass
class TreeVAEFlowConfig(TreeFlowConfig):
    """The latent drafter's config (``cf/drafters/tree_vae_flow.py:32-47``): the flow runs at
    ``latent_size`` inside a frozen ``TransformerHiddenVAE``; the path head, markov bias and lm_head
    stay at the target hidden size.  The serving proposer builds every drafter with this class
    (``cf/vllm_plugin/flow_proposer.py:616-632``)."""
    vae_dir: str | None = None
    latent_size: int = 640
    vae_type: str = "transformer_hidden"
    vae_intermediate_size: int = 1920
    vae_num_layers: int = 2
    vae_num_heads: int = 8
    vae_max_sequence_length: int = 16
    train_vae: bool = False
    lambda_vae_recon: float = 0.5
    lag_context: bool = False
    lag_extend: bool = False
    anchor_token: bool = False
    sched_sampling_p: float = 0.0
    prev_token_cond: bool = True

    @property
    def flow_dim(self) -> int:
        return self.latent_size

    @property
    def vae_heads(self) -> int:
        """``num_heads if intermediate_size % num_heads == 0 else 1``
        (``cf/vae/transformer_hidden.py:13``)."""
        h = self.vae_num_heads
        return h if self.vae_intermediate_size % h == 0 else 1

    def vae_config(self, hidden_size: int) -> dict:
        """``HiddenVAEConfig`` fields (``cf/vae/base.py:9-17``) as ``_load_frozen_vae`` fills them
        (``cf/drafters/tree_vae_flow.py:50-55``)."""
        return dict(hidden_size=hidden_size, latent_size=self.latent_size,
                    intermediate_size=self.vae_intermediate_size, num_layers=self.vae_num_layers,
                    num_heads=self.vae_num_heads, max_sequence_length=self.vae_max_sequence_length)


def config_from_model_args(model_args: dict) -> TreeVAEFlowConfig:
    """``chained_flow_tree_config.json["model_args"]`` -> config, keeping only the known fields, as
    the proposer does (``cf/vllm_plugin/flow_proposer.py:616-618``)."""
    from dataclasses import fields
    known = {f.name for f in fields(TreeVAEFlowConfig)}
    return TreeVAEFlowConfig(**{k: v for k, v in model_args.items() if k in known})


def flownet(d: int, layers: int = 8, flow_steps: int = 8, **kw) -> TreeFlowConfig:
    """The synthetic flow-net used for the d=2560/4096/5120 drafting workloads: context 8,
    draft_length 8 in two chunks of 4, 8 heads, ffn x6, delta init, path order 4, markov rank 256."""
    base = dict(context_size=8, draft_length=8, chunk_size=4, expert_dim=d, num_heads=8,
                ffn_multiplier=6, num_drafter_layers=layers, num_flow_steps=flow_steps,
                init_mode="delta", path_order=4, path_ffn_multiplier=2, markov_rank=256)
    base.update(kw)
    return TreeFlowConfig(**base)
