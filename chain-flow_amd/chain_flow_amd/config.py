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

    def to_dict(self) -> dict:
        return asdict(self)


def flownet(d: int, layers: int = 8, flow_steps: int = 8, **kw) -> TreeFlowConfig:
    """The synthetic flow-net used for the d=2560/4096/5120 drafting workloads: context 8,
    draft_length 8 in two chunks of 4, 8 heads, ffn x6, delta init, path order 4, markov rank 256."""
    base = dict(context_size=8, draft_length=8, chunk_size=4, expert_dim=d, num_heads=8,
                ffn_multiplier=6, num_drafter_layers=layers, num_flow_steps=flow_steps,
                init_mode="delta", path_order=4, path_ffn_multiplier=2, markov_rank=256)
    base.update(kw)
    return TreeFlowConfig(**base)
