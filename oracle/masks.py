"""Dense hierarchical attention mask (the semantic spec), CPU numpy.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates ``build_stage2_hier_self_attn_mask`` (labels form,
multics/models/hier_masks.py:364-507) and
``_build_stage2_hier_self_attn_mask_membership`` (membership form,
hier_masks.py:510-641), including the no-local-hub variant
(hier_masks.py:489-494, 623-628), over the full-sequence token order
``[P*T*L agents | T*N*KL locals | T*KG global]`` (hier_masks.py:549-571).

``mask_rows`` evaluates only a subset of query rows so that C2-sized rows can be
produced block by block without an S x S matrix.

Parity pins: the reference tests' hand-asserted edges
(tests/test_hier_flexible_membership_mask.py:156-347,
tests/test_hier_no_local_hub.py:58-95), restated in tests/test_oracle_masks.py,
and edge-set equality with the reference's golden Tiled128 layouts
(as tests/test_hier_tiled_layout.py:30-95 does) and golden segmented lists.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np


@dataclass(frozen=True)
class FullTopology:
    P: int
    T: int
    L: int
    N: int
    KL: int
    KG: int
    n: int               # num_frame_per_block
    window: int          # local_attn_size, -1 = unbounded
    direct: bool
    labels: Optional[np.ndarray] = None       # [T,P] int
    active: Optional[np.ndarray] = None       # [T,N] bool (labels form: scatter default)
    membership: Optional[np.ndarray] = None   # [T,N,P] bool
    global_only: Optional[np.ndarray] = None  # [T,P] bool
    no_local: bool = False

    @property
    def S(self) -> int:
        return self.P * self.T * self.L + self.T * (self.N * self.KL + self.KG)

    def normalized(self):
        """Membership bitsets, active slots and global_only (hier_masks.py:22-71, 127-193)."""
        T, N, P = self.T, self.N, self.P
        if self.membership is not None:
            mem = np.asarray(self.membership, dtype=bool).reshape(T, N, P)
            if self.global_only is None:
                raise ValueError("hier_group_format=membership requires global_only")
            go = np.asarray(self.global_only, dtype=bool).reshape(T, P)
            act = mem.any(-1) if self.active is None else np.asarray(self.active, dtype=bool)
            labels_form = False
        else:
            lab = np.asarray(self.labels, dtype=np.int64).reshape(T, P)
            if lab.size and (lab.min() < 0 or lab.max() >= N):
                raise ValueError(f"group_labels values must be in [0,{N})")
            mem = np.zeros((T, N, P), dtype=bool)
            for t in range(T):
                mem[t, lab[t], np.arange(P)] = True
            if self.active is None:
                act = mem.any(-1)
            else:
                act = np.asarray(self.active, dtype=bool).reshape(T, N)
            go = np.zeros((T, P), dtype=bool)
            labels_form = True
        if N > 62:
            raise ValueError(f"membership bitset path supports N<=62, got N={N}")
        bits = (mem.astype(np.int64) << np.arange(N, dtype=np.int64)[None, :, None]).sum(1)
        return bits, act, go, labels_form

    def token_ids(self, idx: np.ndarray):
        """(kind, t, p, g) of token indices; kind 0=agent 1=local 2=global."""
        P, T, L, N, KL, KG = self.P, self.T, self.L, self.N, self.KL, self.KG
        idx = np.asarray(idx, dtype=np.int64)
        agent_len = P * T * L
        glob0 = agent_len + T * N * KL
        kind = np.where(idx < agent_len, 0, np.where(idx < glob0, 1, 2))
        t = np.zeros_like(idx)
        p = np.zeros_like(idx)
        g = np.zeros_like(idx)
        a = kind == 0
        p[a] = idx[a] // (T * L)
        t[a] = idx[a] % (T * L) // L
        if KL > 0:
            lo = kind == 1
            rel = idx[lo] - agent_len
            t[lo] = rel // (N * KL)
            g[lo] = rel % (N * KL) // KL
        if KG > 0:
            gl = kind == 2
            t[gl] = (idx[gl] - glob0) // KG
        return kind, t, p, g


def mask_rows(topo: FullTopology, q_idx=None, k_idx=None) -> np.ndarray:
    """Boolean mask [len(q_idx), len(k_idx)] of the hierarchical edge rule."""
    if topo.no_local and (topo.KL != 0 or topo.KG <= 0):
        raise ValueError("hier_no_local_hub requires K_L=0 and K_G>0")
    if topo.window != -1 and topo.window < topo.n:
        raise ValueError("hier_hub requires local_attn_size=-1 or >= num_frame_per_block")
    S = topo.S
    q_idx = np.arange(S) if q_idx is None else np.asarray(q_idx, dtype=np.int64)
    k_idx = np.arange(S) if k_idx is None else np.asarray(k_idx, dtype=np.int64)
    bits, act, go, labels_form = topo.normalized()
    qk, qt, qp, qg = topo.token_ids(q_idx)
    kk, kt, kp, kg = topo.token_ids(k_idx)
    QK, QT, QP, QG = qk[:, None], qt[:, None], qp[:, None], qg[:, None]
    KK, KT, KP, KG_ = kk[None, :], kt[None, :], kp[None, :], kg[None, :]
    qa, ka = QK == 0, KK == 0
    ql, kl = QK == 1, KK == 1
    qgl, kgl = QK == 2, KK == 2
    n = topo.n
    win = (KT // n) <= (QT // n)
    if topo.window != -1:
        win &= (QT - KT) < topo.window
    same_blk = (QT // n) == (KT // n)
    q_bits = bits[qt, qp][:, None]
    k_bits_at_qt = bits[QT, KP]          # key player's groups at the query frame
    act_q = act[qt, qg][:, None]
    act_k = act[kt, kg][None, :]
    m = qa & ka & (QP == KP) & win                                       # own history
    if topo.direct:
        m |= qa & ka & (QP != KP) & ((q_bits & k_bits_at_qt) != 0) & same_blk
    m |= qa & kl & act_k & (((q_bits >> KG_) & 1) != 0) & win            # player -> local
    m |= ql & act_q & ka & (((k_bits_at_qt >> QG) & 1) != 0) & win       # local -> player
    m |= ql & act_q & kgl & win                                          # local -> global
    m |= ql & act_q & kl & act_k & (QG == KG_) & win                     # local -> local
    m |= ql & ~act_q & kl & (q_idx[:, None] == k_idx[None, :])           # inactive self
    m |= qgl & kl & act_k & win                                          # global -> local
    m |= qgl & kgl & win                                                 # global -> global
    if topo.no_local:
        m |= qa & kgl & win
        m |= qgl & ka & win
    elif not labels_form:
        m |= qa & kgl & go[qt, qp][:, None] & win                        # player -> global
        m |= qgl & ka & go[kt, kp][None, :] & win                        # global -> player
    return m


def inactive_local_rows(topo: FullTopology) -> np.ndarray:
    """Bool [S]: local-hub query rows whose slot is inactive (the kernel writes 0 there).

    Same row selection as ``build_hier_query_active_mask`` (hier_tiled_attention.py:432-459).
    """
    _, act, _, _ = topo.normalized()
    kind, t, _, g = topo.token_ids(np.arange(topo.S))
    return (kind == 1) & ~act[t, g]
