"""fp32 CPU restatement of the cached (rollout) hierarchical attention.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* ``RollingCache`` / ``append`` / ``append_bool`` -- the rolling per-stream KV
  cache: append new frames, refresh a re-run range in place, evict the oldest
  frames by shifting when over capacity (multics/models/attention.py:90-228).
* ``HierCacheState`` -- one layer's caches: P agent streams, N local-hub
  streams (+ per-token active flags), one global stream, each of capacity
  (W + n) frames (wan_video_Nplayers.py:888-989).
* ``cached_block_forward`` -- one cached block: append the block's K/V, then
  per-stream masked attention over the cache windows -- players, local hubs,
  global hub -- in the block's token order [P*n*L | n*N*KL | n*KG]
  (attention.py:456-1005, the per-stream SDPA path, labels and membership).

Parity pins: with blocks appended in order and clean K/V, the cached output of
every block equals the full-sequence dense-mask attention of ``oracle.masks``
on the same rows (``tests/test_cached_oracle.py``); the cache bookkeeping is
checked against closed forms of the window (last W + n frames, refresh leaves
the window unchanged).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np
import torch


@dataclass
class RollingCache:
    k: torch.Tensor              # [cap, H, D]
    v: torch.Tensor
    global_end: int = 0          # absolute token index one past the newest cached token
    local_end: int = 0           # number of valid tokens in the buffer
    active: Optional[torch.Tensor] = None   # [cap] bool (local hubs)


def _append_rows(buf, values, cur_start, cur_end, window, state):
    """Shared bookkeeping of append / append_bool; returns the new local end."""
    cap = buf[0].shape[0]
    g_end, l_end = state.global_end, state.local_end
    progress = max(0, cur_end - g_end)
    n_new = min(values[0].shape[0], progress)
    if n_new == 0 and l_end > 0:                       # refresh a re-run range in place
        cached_start = g_end - l_end
        lo, hi = max(cur_start, cached_start), min(cur_end, g_end)
        if hi > lo:
            for b, x in zip(buf, values):
                b[lo - cached_start:hi - cached_start] = x[lo - cur_start:hi - cur_start]
    new_end = l_end + n_new
    if window != -1 and cur_end > g_end and new_end > cap:   # evict the oldest tokens
        n_ev = max(0, min(new_end - cap, new_end - 1))
        if n_ev > 0:
            keep = max(0, l_end - n_ev)
            for b in buf:
                if keep > 0:
                    b[:keep] = b[n_ev:n_ev + keep].clone()
            new_end = min(l_end + n_new - n_ev, cap)
    if n_new > 0:
        for b, x in zip(buf, values):
            b[new_end - n_new:new_end] = x[-n_new:]
    return new_end


def append(cache: RollingCache, k_new, v_new, cur_start, cur_end, window, tpf):
    """attention.py:90-167 (sink_size = 0)."""
    new_end = _append_rows((cache.k, cache.v), (k_new, v_new), cur_start, cur_end, window, cache)
    cache.global_end, cache.local_end = cur_end, new_end


def append_bool(cache: RollingCache, values, cur_start, cur_end, window, tpf):
    """attention.py:170-228, run before ``append`` on the same cache."""
    _append_rows((cache.active,), (values,), cur_start, cur_end, window, cache)


@dataclass
class HierCacheState:
    P: int
    N: int
    L: int
    KL: int
    KG: int
    H: int
    D: int
    window: int                  # local_attn_size W (-1 = unbounded)
    n: int                       # frames per block
    T_max: int = 64              # frames the unbounded cache can hold
    agent: List[RollingCache] = field(default_factory=list)
    local: List[RollingCache] = field(default_factory=list)
    glob: Optional[RollingCache] = None

    def __post_init__(self):
        R = (self.window + self.n) if self.window != -1 else self.T_max
        z = lambda w: torch.zeros(R * w, self.H, self.D)
        self.agent = [RollingCache(z(self.L), z(self.L)) for _ in range(self.P)]
        self.local = [RollingCache(z(self.KL), z(self.KL),
                                   active=torch.zeros(R * self.KL, dtype=torch.bool))
                      for _ in range(self.N)]
        self.glob = RollingCache(z(self.KG), z(self.KG))

    @property
    def retention(self):
        return self.window + self.n if self.window != -1 else -1


def _temporal(qf, kf, n_block, window):
    m = (kf[None, :] // n_block) <= (qf[:, None] // n_block)
    if window != -1:
        m &= (qf[:, None] - kf[None, :]) < window
    return m


def _frames(cache: RollingCache, tpf, end_frame):
    n_cached = cache.local_end // tpf if tpf > 0 else 0
    return end_frame - n_cached + 1 + torch.arange(cache.local_end) // max(tpf, 1)


def _sdpa(q, k, v, mask, scale):
    s = torch.einsum("qhd,khd->hqk", q.float(), k.float()) * scale
    s = s.masked_fill(~mask[None], float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
    return torch.einsum("hqk,khd->qhd", p, v.float())


def cached_block_forward(st: HierCacheState, q, k, v, start_frame, *, n_block, direct,
                         labels=None, active=None, membership=None, global_only=None):
    """One cached block.  ``q, k, v``: [P*n*L + n*(N*KL+KG), H, D] in the block
    order; ``labels`` [n, P] / ``active`` [n, N] for the block, or full-clip
    ``membership`` [T, N, P] / ``global_only`` [T, P] (``active`` then [n, N]
    defaults to membership.any(-1) at the block's frames).  Returns fp32
    output rows in the same order."""
    P, N, L, KL, KG, n, H, D = st.P, st.N, st.L, st.KL, st.KG, st.n, st.H, st.D
    scale = 1.0 / math.sqrt(D)
    window, R = st.window, st.retention
    use_mem = membership is not None
    if use_mem:
        mem = torch.as_tensor(np.asarray(membership, bool))
        go = torch.as_tensor(np.asarray(global_only, bool))
        act = mem[start_frame:start_frame + n].any(-1) if active is None else \
            torch.as_tensor(np.asarray(active, bool))
    else:
        lab = torch.as_tensor(np.asarray(labels)).long()
        act = torch.as_tensor(np.asarray(active, bool))
    aL, lL = P * n * L, n * N * KL
    end_frame = start_frame + n - 1
    # ---- append (attention.py:605-666)
    for p in range(P):
        sl = slice(p * n * L, (p + 1) * n * L)
        append(st.agent[p], k[sl], v[sl], start_frame * L, (start_frame + n) * L, R, L)
    lk = k[aL:aL + lL].reshape(n, N, KL, H, D)
    lv = v[aL:aL + lL].reshape(n, N, KL, H, D)
    for g in range(N):
        append_bool(st.local[g], act[:, g].repeat_interleave(KL), start_frame * KL,
                    (start_frame + n) * KL, R, KL)
        append(st.local[g], lk[:, g].reshape(-1, H, D), lv[:, g].reshape(-1, H, D),
               start_frame * KL, (start_frame + n) * KL, R, KL)
    if KG > 0:
        append(st.glob, k[aL + lL:], v[aL + lL:], start_frame * KG, (start_frame + n) * KG, R, KG)
    # ---- windows
    af = [_frames(c, L, end_frame) for c in st.agent]
    ak = [c.k[:c.local_end] for c in st.agent]
    av = [c.v[:c.local_end] for c in st.agent]
    lf = [_frames(c, KL, end_frame) for c in st.local]
    lk_ = [c.k[:c.local_end] for c in st.local]
    lv_ = [c.v[:c.local_end] for c in st.local]
    la = [c.active[:c.local_end] for c in st.local]
    gf = _frames(st.glob, KG, end_frame)
    gk, gv = st.glob.k[:st.glob.local_end], st.glob.v[:st.glob.local_end]
    lf_all = torch.cat(lf) if N else torch.zeros(0, dtype=torch.long)
    lk_all, lv_all = (torch.cat(lk_) if N else gk[:0]), (torch.cat(lv_) if N else gv[:0])
    la_all = torch.cat(la) if N else torch.zeros(0, dtype=torch.bool)
    lg_all = torch.cat([torch.full_like(lf[g], g) for g in range(N)]) if N else lf_all
    out = torch.zeros(q.shape[0], H, D)
    # ---- players (attention.py:797-888)
    qaf = start_frame + torch.arange(n * L) // L
    for p in range(P):
        rows = slice(p * n * L, (p + 1) * n * L)
        if use_mem:
            q_mem = mem[qaf, :, p]
            q_go = go[qaf, p]
        else:
            q_grp = lab[qaf - start_frame, p]
        keys, vals, masks = [ak[p]], [av[p]], [_temporal(qaf, af[p], n_block, window)]
        if direct:
            for o in range(P):
                if o == p:
                    continue
                ofr = start_frame + torch.arange(n * L) // L
                if use_mem:
                    om = (q_mem & mem[qaf, :, o]).any(-1)[:, None]
                else:
                    om = (lab[qaf - start_frame, o] == q_grp)[:, None]
                om = om & ((ofr[None, :] // n_block) == (qaf[:, None] // n_block))
                keys.append(k[o * n * L:(o + 1) * n * L])
                vals.append(v[o * n * L:(o + 1) * n * L])
                masks.append(om)
        lm = _temporal(qaf, lf_all, n_block, window) & la_all[None, :]
        if use_mem:
            lm &= q_mem[:, lg_all]
        else:
            lm &= lg_all[None, :] == q_grp[:, None]
        keys.append(lk_all)
        vals.append(lv_all)
        masks.append(lm)
        if use_mem and KG > 0:
            keys.append(gk)
            vals.append(gv)
            masks.append(_temporal(qaf, gf, n_block, window) & q_go[:, None])
        out[rows] = _sdpa(q[rows], torch.cat(keys), torch.cat(vals), torch.cat(masks, 1), scale)
    # ---- local hubs (attention.py:889-947)
    qlf = start_frame + torch.arange(n * KL) // KL
    ql = q[aL:aL + lL].reshape(n, N, KL, H, D)
    lo = torch.zeros(n, N, KL, H, D)
    for g in range(N):
        if not bool(act[:, g].any()):
            continue
        qa = act[qlf - start_frame, g]
        keys, vals, masks = [], [], []
        for p in range(P):
            pm = _temporal(qlf, af[p], n_block, window) & qa[:, None]
            if use_mem:
                pm &= mem[qlf, g, p][:, None]
            else:
                pm &= (lab[qlf - start_frame, p] == g)[:, None]
            keys.append(ak[p])
            vals.append(av[p])
            masks.append(pm)
        keys.append(lk_[g])
        vals.append(lv_[g])
        masks.append(_temporal(qlf, lf[g], n_block, window) & qa[:, None] & la[g][None, :])
        if KG > 0:
            keys.append(gk)
            vals.append(gv)
            masks.append(_temporal(qlf, gf, n_block, window) & qa[:, None])
        og = _sdpa(ql[:, g].reshape(-1, H, D), torch.cat(keys), torch.cat(vals),
                   torch.cat(masks, 1), scale)
        lo[:, g] = og.reshape(n, KL, H, D)
    out[aL:aL + lL] = lo.reshape(-1, H, D)
    # ---- global hub (attention.py:948-996)
    if KG > 0:
        qgf = start_frame + torch.arange(n * KG) // KG
        keys = [lk_all, gk]
        vals = [lv_all, gv]
        masks = [_temporal(qgf, lf_all, n_block, window) & la_all[None, :],
                 _temporal(qgf, gf, n_block, window)]
        if use_mem:
            for p in range(P):
                go_k = go[af[p].clamp(0, go.shape[0] - 1), p]
                keys.append(ak[p])
                vals.append(av[p])
                masks.append(_temporal(qgf, af[p], n_block, window) & go_k[None, :])
        out[aL + lL:] = _sdpa(q[aL + lL:], torch.cat(keys), torch.cat(vals), torch.cat(masks, 1),
                              scale)
    return out
