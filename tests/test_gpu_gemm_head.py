"""GPU parity of the batched MFMA head (cfh_head_gemm_topk): bf16 skinny GEMM over the shortlist
rows of the lm_head with the per-row log-softmax top-k fused in.

Contract: bf16 logits within one bf16 ulp (plus the fp32 accumulation error, which matters only
where the dot product cancels to a tiny value) of the float64 product of the bf16 inputs.  The
logits the reference ranks are bf16 themselves, so the oracle's logits are the float64 products
rounded to bf16: top-k ids must equal the oracle's wherever the oracle's (rounded) margin exceeds
1e-3, and equal the top-k of the kernel's own logits everywhere; log-probs within 1e-5 of the
log-softmax of the kernel's logits.
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


def _bf16(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).double().numpy()


def _acc_err(x, Wsl):
    """Bound of the fp32 accumulation error of each dot product: 2^-20 sum_i |x_i w_i|."""
    return 2.0 ** -20 * (np.abs(x) @ np.abs(Wsl).T)


def _case(cuda, M, d, V, n, k, seed, scale, packed=False):
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(V, d, generator=g) * (scale / d ** 0.5)).to(torch.bfloat16)
    sl = torch.randperm(V, generator=g)[:n].sort().values.to(torch.int32)
    x = torch.randn(M, d, generator=g).to(torch.bfloat16)
    head = GemmHead(W.to(cuda), sl.to(cuda), packed=packed)
    logits = torch.empty(M, n, dtype=torch.bfloat16, device=cuda)
    vals, ids, lse = head.topk(x.to(cuda), k, logits=logits)
    torch.cuda.synchronize()
    return W, sl, x, logits, vals, ids, lse


@pytest.mark.gpu
@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("M,d,n,k", [(1, 256, 1000, 4), (40, 512, 3001, 8), (160, 1024, 5000, 8),
                                     (200, 640, 3000, 8), (256, 512, 2000, 16), (97, 768, 2049, 5)])
def test_gemm_head_matches_oracle(cuda, M, d, n, k, packed):
    if packed and d % 256:
        pytest.skip("the packed image needs d % 256 == 0")
    V = 2 * n + 17
    print(f"[gemm head] M={M} d={d} n={n} k={k} packed={packed}", flush=True)
    W, sl, x, logits, vals, ids, lse = _case(cuda, M, d, V, n, k, seed=M + d, scale=4.0, packed=packed)
    Wsl = to64(W)[sl.long().numpy()]
    ref = to64(x) @ Wsl.T                                             # float64 of the bf16 inputs
    got = to64(logits)
    assert (np.abs(got - ref) <= _bf16_ulp(ref) + _acc_err(to64(x), Wsl)).all()
    # top-k of the kernel's own logits: bit-exact ids, values to 1e-5
    lp = ohead.log_softmax(got)
    ov, oi = ohead.topk(lp, k)
    assert np.array_equal(ids.cpu().numpy(), oi)
    assert np.allclose(vals.cpu().numpy(), ov, atol=1e-5, rtol=0)
    # against the float64 oracle wherever the decision margin is clear
    ref16 = _bf16(ref)
    rv, ri = ohead.topk(ohead.log_softmax(ref16), k)
    clear = ohead.margins(ref16, k) > MARGIN
    assert clear.mean() > 0.5
    assert np.array_equal(ids.cpu().numpy()[clear], ri[clear])


@pytest.mark.gpu
@pytest.mark.parametrize("packed", [False, True])
def test_gemm_head_batched_drafting_shape(cuda, packed):
    """32 sequences x 5 depths = 160 rows, d=4096, the 62,642-row shortlist of a 248,320-row head,
    top-8 per row (checked on a sample of rows against float64)."""
    M, d, V, n, k = 160, 4096, 248320, 62642, 8
    g = torch.Generator(device=cuda).manual_seed(4)
    W = (torch.randn(V, d, generator=g, device=cuda) * (4.0 / d ** 0.5)).to(torch.bfloat16)
    sl = torch.randperm(V, generator=torch.Generator().manual_seed(2))[:n].sort().values.to(torch.int32)
    x = torch.randn(M, d, generator=g, device=cuda).to(torch.bfloat16)
    head = GemmHead(W, sl.to(cuda), packed=packed)
    vals, ids, lse = head.topk(x, k)
    torch.cuda.synchronize()
    rows = np.arange(0, M, 7)
    Wsl = to64(W[sl.long().to(cuda)])
    ref16 = _bf16(to64(x)[rows] @ Wsl.T)
    rv, ri = ohead.topk(ohead.log_softmax(ref16), k)
    clear = ohead.margins(ref16, k) > MARGIN
    assert clear.mean() > 0.5
    assert np.array_equal(ids.cpu().numpy()[rows][clear], ri[clear])
    # log-probs: equal up to the rare one-ulp rounding differences of single logits
    assert np.allclose(vals.cpu().numpy()[rows][clear], rv[clear], atol=5e-2, rtol=0)
