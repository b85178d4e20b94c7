"""fp32 definition of the membership straight-through gradient.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference has no gradient with respect to group membership: its training
forward (``SelfAttention.forward_hier_tiled_ste``, multics/models/attention.py:
367-434) takes the Tiled128 value and the FlexAttention Jacobian with respect
to Q/K/V only, on a boolean mask.  The membership gradient of the training
configuration is therefore defined by this build, and this module *is* that
definition, in fp32 torch autograd:

* the forward mask is the hard one of ``oracle.masks`` for membership
  ``logits > 0``;
* every edge whose existence depends on exactly one membership bit (t, g, p)
  -- player p's query row at frame t to a local-hub key of group g
  (hier_masks.py:593-594), group g's local-hub row at frame t to a key of
  player p (hier_masks.py:611-612) -- gets the additive bias
  ``sigmoid(logit) - sigmoid(logit).detach()`` on its scaled score (zero in
  value, derivative sigmoid'(logit));
* autograd of sum(out * dout) gives dL/dlogits.

Parity unpinned by the reference (no reference counterpart); pinned only by
this autograd definition, which ``tests/test_gpu_backward.py`` checks the HIP
implementation against, plus the closed-form checks of ``tests/test_ste_oracle.py``.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from .masks import FullTopology, inactive_local_rows, mask_rows


def gate_index(topo: FullTopology):
    """[S, S] int64 index into logits.flatten() of the gating bit, -1 if none."""
    S = topo.S
    kind, t, p, g = topo.token_ids(np.arange(S))
    N, P = topo.N, topo.P
    idx = np.full((S, S), -1, dtype=np.int64)
    a = (kind[:, None] == 0) & (kind[None, :] == 1)         # player q -> local key
    gi = (t[:, None] * N + g[None, :]) * P + p[:, None]
    idx[a] = np.broadcast_to(gi, (S, S))[a]
    b = (kind[:, None] == 1) & (kind[None, :] == 0)         # local q -> player key
    gj = (t[:, None] * N + g[:, None]) * P + p[None, :]
    idx[b] = np.broadcast_to(gj, (S, S))[b]
    return idx


def ste_attention(q, k, v, topo: FullTopology, logits: torch.Tensor, scale=None) -> torch.Tensor:
    """fp32 attention [S, H, D] with the surrogate membership bias (value 0)."""
    S, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    m = torch.from_numpy(mask_rows(topo))
    live = ~torch.from_numpy(inactive_local_rows(topo))
    sig = torch.sigmoid(logits.float()).reshape(-1)
    beta = sig - sig.detach()
    gi = torch.from_numpy(gate_index(topo))
    bias = torch.where(gi >= 0, beta[gi.clamp(min=0)], torch.zeros((), dtype=torch.float32))
    s = torch.einsum("qhd,khd->hqk", q.float(), k.float()) * scale + bias[None]
    s = s.masked_fill(~m[None], float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
    o = torch.einsum("hqk,khd->qhd", p, v.float())
    return o * live[:, None, None]


def ste_grad_at(q, k, v, dout, topo: FullTopology, logits: torch.Tensor, bits, scale=None):
    """dL/dlogit of ``sum(ste_attention(q, k, v, topo, logits) * dout)`` at the
    membership bits ``bits`` (an iterable of (t, g, p)), without the S x S
    pass: only the rows whose edges a bit gates are evaluated.

    The bias of bit (t, g, p) sits on two edge sets (see ``gate_index``):
    player p's rows at frame t to every local-hub key of group g, and group
    g's hub rows at frame t to every key of player p.  With the bias zero in
    value, dL/dbias_ij = dS_ij = P_ij (dP_ij - delta_i) (dP_ij = dO_i.v_j,
    delta_i = dO_i.O_i), summed over heads because the bias is shared by all
    heads, so dL/dlogit = sigmoid'(logit) * sum of dS over those edges.
    Inactive local-hub rows output 0 (their dO counts as 0).  Returns a float64
    numpy array, one value per bit.
    """
    S, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    P, T, L, N, KL = topo.P, topo.T, topo.L, topo.N, topo.KL
    qf, kf, vf, df = (t.float() for t in (q, k, v, dout))
    dead = inactive_local_rows(topo)
    kind, _, kp, kg = topo.token_ids(np.arange(S))
    a0 = P * T * L
    lg = logits.detach().double().reshape(T, N, P)
    out = []
    for (t, g, p) in bits:
        total = 0.0
        player_rows = p * T * L + t * L + np.arange(L)
        local_rows = a0 + (t * N + g) * KL + np.arange(KL)
        for rows, gated in ((player_rows, (kind == 1) & (kg == g)),
                            (local_rows, (kind == 0) & (kp == p))):
            rows = rows[~dead[rows]]
            if len(rows) == 0:
                continue
            rt = torch.from_numpy(rows)
            m = torch.from_numpy(mask_rows(topo, q_idx=rows))                 # [r, S]
            s = torch.einsum("qhd,khd->hqk", qf[rt], kf) * scale
            s = s.masked_fill(~m[None], float("-inf"))
            pr = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)          # [H, r, S]
            o = torch.einsum("hqk,khd->qhd", pr, vf)
            delta = (df[rt] * o).sum(-1)                                      # [r, H]
            dp = torch.einsum("qhd,khd->hqk", df[rt], vf)
            ds = pr * (dp - delta.T[:, :, None])
            total += float(ds[:, :, torch.from_numpy(gated)].double().sum())
        sig = 1.0 / (1.0 + math.exp(-float(lg[t, g, p])))
        out.append(sig * (1.0 - sig) * total)
    return np.array(out, dtype=np.float64)
