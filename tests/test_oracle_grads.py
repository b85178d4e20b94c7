"""The row-sampled attention gradients of the oracle against torch autograd
through its own dense-mask attention (small shapes, CPU)."""

import numpy as np
import torch

from oracle.attention import attention_grads_at, masked_attention
from oracle.masks import FullTopology


def test_attention_grads_at_matches_autograd():
    rng = np.random.default_rng(3)
    P, T, L, N, KL, KG, n, W, H, D = 3, 6, 10, 2, 2, 2, 3, 4, 2, 16
    mem = rng.random((T, N, P)) < 0.5
    go = ~mem.any(1) & (rng.random((T, P)) < 0.5)
    topo = FullTopology(P, T, L, N, KL, KG, n, W, True, membership=mem, global_only=go)
    S = topo.S
    g = torch.Generator().manual_seed(1)
    q, k, v, dout = (torch.randn(S, H, D, generator=g, dtype=torch.float64) for _ in range(4))
    qf, kf, vf = (t.clone().requires_grad_(True) for t in (q, k, v))
    masked_attention(qf, kf, vf, topo).backward(dout.float())
    rows = np.arange(S)
    # a row block smaller than S exercises the accumulation over blocks
    dq, dk, dv = attention_grads_at(q, k, v, dout, topo, q_rows=rows, k_rows=rows, row_block=37)
    for got, ref in ((dq, qf.grad), (dk, kf.grad), (dv, vf.grad)):
        ref = ref.float()
        assert (got - ref).abs().max().item() <= 1e-4 * ref.abs().max().item()
    # a subset of rows, in any order, gives the same values
    sub = rng.permutation(S)[:17]
    dq2, dk2, dv2 = attention_grads_at(q, k, v, dout, topo, q_rows=sub, k_rows=sub[::-1])
    assert torch.allclose(dq2, dq[sub], atol=1e-5)
    assert torch.allclose(dk2, dk[sub[::-1].copy()], atol=1e-5)
    assert torch.allclose(dv2, dv[sub[::-1].copy()], atol=1e-5)
