"""Checks of the membership STE definition (oracle/ste.py) on the CPU.

* Its value is the plain masked attention (the surrogate bias is zero).
* Its logit gradient equals sigmoid'(logit) times the sum of dS = P (dP - delta)
  over the gated edges, computed here independently from the dense
  probabilities, and is zero for bits whose edges are all absent.
* The gate index names the bit of every player<->local-hub edge and no other.
"""

import math

import numpy as np
import torch

from oracle.attention import masked_attention
from oracle.masks import FullTopology, mask_rows, inactive_local_rows
from oracle.ste import gate_index, ste_attention


def _case(seed=0):
    rng = np.random.default_rng(seed)
    P, T, L, N, KL, KG, n, W, H, D = 3, 4, 5, 2, 2, 2, 2, 3, 2, 16
    logits = torch.from_numpy(rng.standard_normal((T, N, P))).float()
    mem = (logits > 0).numpy()
    go = ~mem.any(1)
    topo = FullTopology(P, T, L, N, KL, KG, n, W, True, membership=mem, global_only=go)
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = [torch.randn(topo.S, H, D, generator=g) for _ in range(4)]
    return topo, logits, q, k, v, do


def test_value_is_plain_attention():
    topo, logits, q, k, v, _ = _case()
    assert torch.allclose(ste_attention(q, k, v, topo, logits), masked_attention(q, k, v, topo),
                          atol=1e-6)


def test_gradient_closed_form():
    topo, logits, q, k, v, do = _case(1)
    lg = logits.clone().requires_grad_(True)
    out = ste_attention(q, k, v, topo, lg)
    (out * do).sum().backward()
    # independent: dS = P (dP - delta) from dense probabilities
    S, H, D = q.shape
    m = torch.from_numpy(mask_rows(topo))
    live = ~torch.from_numpy(inactive_local_rows(topo))
    s = torch.einsum("qhd,khd->hqk", q, k) / math.sqrt(D)
    p = torch.nan_to_num(torch.softmax(s.masked_fill(~m[None], float("-inf")), -1), nan=0.0)
    p = p * live[None, :, None]
    o = torch.einsum("hqk,khd->qhd", p, v)
    dp = torch.einsum("qhd,khd->hqk", do, v)
    delta = (do * o).sum(-1).permute(1, 0)[:, :, None]
    ds = (p * (dp - delta)).sum(0)
    gi = gate_index(topo)
    want = np.zeros(logits.numel())
    np.add.at(want, gi[gi >= 0], ds.numpy()[gi >= 0])
    sig = torch.sigmoid(logits).reshape(-1)
    want = torch.from_numpy(want).float() * sig * (1 - sig)
    assert torch.allclose(lg.grad.reshape(-1), want, atol=1e-5, rtol=1e-4)


def test_gate_index_classes():
    topo, logits, *_ = _case(2)
    gi = gate_index(topo)
    kind, t, p, g = topo.token_ids(np.arange(topo.S))
    gated = gi >= 0
    pl = (kind[:, None] == 0) & (kind[None, :] == 1)
    lp = (kind[:, None] == 1) & (kind[None, :] == 0)
    assert np.array_equal(gated, pl | lp)
    T, N, P = logits.shape
    qi, ki = np.nonzero(pl)
    assert np.array_equal(gi[qi, ki], (t[qi] * N + g[ki]) * P + p[qi])
    qi, ki = np.nonzero(lp)
    assert np.array_equal(gi[qi, ki], (t[qi] * N + g[qi]) * P + p[ki])


def test_row_sampled_gradient_equals_autograd():
    """``ste_grad_at`` (only the gated rows, per bit) equals the autograd
    logit gradient of the dense definition at every bit, including bits that
    are off (no edges: zero) and inactive hub slots."""
    from oracle.ste import ste_grad_at
    for seed in (3, 4):
        topo, logits, q, k, v, do = _case(seed)
        lg = logits.clone().requires_grad_(True)
        (ste_attention(q, k, v, topo, lg) * do).sum().backward()
        T, N, P = logits.shape
        bits = [(t, g, p) for t in range(T) for g in range(N) for p in range(P)]
        got = ste_grad_at(q, k, v, do, topo, logits, bits)
        want = lg.grad.reshape(-1).double().numpy()
        assert np.allclose(got, want, atol=1e-5, rtol=1e-4), (got, want)
        assert (np.abs(want) > 1e-4).sum() >= 4
