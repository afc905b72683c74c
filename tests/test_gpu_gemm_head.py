"""GPU parity of the batched MFMA head (cfh_head_gemm_topk): bf16 skinny GEMM over the shortlist
rows of the lm_head with the per-row log-softmax top-k fused in.

Contract: bf16 logits within one bf16 ulp of the float64 product of the bf16 inputs; top-k ids
equal to the oracle's top-k of the float64 logits wherever the oracle's margin exceeds 1e-3, and
bit-exact against the top-k of the kernel's own logits; log-probs within 1e-5 of the log-softmax
of the kernel's logits.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import to64
from chain_flow_amd.head import GemmHead
from oracle import head as ohead

MARGIN = 1e-3


def _bf16_ulp(x):
    x = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(x, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def _case(cuda, M, d, V, n, k, seed, scale):
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(V, d, generator=g) * (scale / d ** 0.5)).to(torch.bfloat16)
    sl = torch.randperm(V, generator=g)[:n].sort().values.to(torch.int32)
    x = torch.randn(M, d, generator=g).to(torch.bfloat16)
    head = GemmHead(W.to(cuda), sl.to(cuda))
    logits = torch.empty(M, n, dtype=torch.bfloat16, device=cuda)
    vals, ids, lse = head.topk(x.to(cuda), k, logits=logits)
    torch.cuda.synchronize()
    return W, sl, x, logits, vals, ids, lse


@pytest.mark.gpu
@pytest.mark.parametrize("M,d,n,k", [(1, 256, 1000, 4), (40, 512, 3001, 8), (160, 1024, 5000, 8),
                                     (256, 512, 2000, 16)])
def test_gemm_head_matches_oracle(cuda, M, d, n, k):
    V = 2 * n + 17
    print(f"[gemm head] M={M} d={d} n={n} k={k}", flush=True)
    W, sl, x, logits, vals, ids, lse = _case(cuda, M, d, V, n, k, seed=M + d, scale=4.0)
    ref = to64(x) @ to64(W)[sl.long().numpy()].T                      # float64 of the bf16 inputs
    got = to64(logits)
    assert (np.abs(got - ref) <= _bf16_ulp(ref) + 1e-30).all()
    # top-k of the kernel's own logits: bit-exact ids, values to 1e-5
    lp = ohead.log_softmax(got)
    ov, oi = ohead.topk(lp, k)
    assert np.array_equal(ids.cpu().numpy(), oi)
    assert np.allclose(vals.cpu().numpy(), ov, atol=1e-5, rtol=0)
    # against the float64 oracle wherever the decision margin is clear
    rv, ri = ohead.topk(ohead.log_softmax(ref), k)
    mg = ohead.margins(ref, k)
    clear = mg > MARGIN
    assert np.array_equal(ids.cpu().numpy()[clear], ri[clear])


@pytest.mark.gpu
def test_gemm_head_batched_drafting_shape(cuda):
    """32 sequences x 5 depths = 160 rows, d=4096, the 62,642-row shortlist of a 248,320-row head,
    top-8 per row (checked on a sample of rows against float64)."""
    M, d, V, n, k = 160, 4096, 248320, 62642, 8
    g = torch.Generator(device=cuda).manual_seed(4)
    W = (torch.randn(V, d, generator=g, device=cuda) * (4.0 / d ** 0.5)).to(torch.bfloat16)
    sl = torch.randperm(V, generator=torch.Generator().manual_seed(2))[:n].sort().values.to(torch.int32)
    x = torch.randn(M, d, generator=g, device=cuda).to(torch.bfloat16)
    head = GemmHead(W, sl.to(cuda))
    vals, ids, lse = head.topk(x, k)
    torch.cuda.synchronize()
    rows = np.arange(0, M, 7)
    Wsl = to64(W[sl.long().to(cuda)])
    ref = to64(x)[rows] @ Wsl.T
    rv, ri = ohead.topk(ohead.log_softmax(ref), k)
    clear = ohead.margins(ref, k) > MARGIN
    assert np.array_equal(ids.cpu().numpy()[rows][clear], ri[clear])
    assert np.allclose(vals.cpu().numpy()[rows], rv, atol=2e-2, rtol=0)   # bf16 logits vs float64
