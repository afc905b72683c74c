"""chain-flow drafting hot path on MI355X: PyTorch-ROCm host code over libcfhip.so (HIP/gfx950).

Modules: ``config`` (TreeFlowConfig), ``weights`` (seeded synthetic state), ``shortlist`` (the
shortlist file format and vocabulary guard), ``flow`` (fused predict_hidden), ``head`` (shortlisted
lm_head + top-k, path residual), ``drafter`` (chain/tree beam drafts), ``gdn`` (tree gated
delta net), ``vllm_plugin.flow_proposer`` (the ``FlowDrafterProposer`` custom_class surface).
"""

__version__ = "0.1.0"
