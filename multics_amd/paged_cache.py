"""Paged KV cache for the cached (chunked causal rollout) hierarchical attention.

The reference keeps one rolling buffer per stream -- P agent caches, N local
hub caches (+ per-token active flags), one global cache -- appends a block's
K/V, shifts the buffer when it overflows and concatenates every buffer into one
pool on each attention call (attention.py:90-228, 605-796;
wan_video_Nplayers.py:888-1058; hier_segmented_attention.py:458-469).

Here one layer owns a single K pool and a single V pool ``[rows, H, D]``.  Every
(stream, frame) has a fixed page of rows -- L rows for an agent frame, KL for a
local-hub frame, KG for a global frame -- in a ring of R = W + n frame slots
(W = local_attn_size, n = frames per block; R = max_frames when W = -1):

    rows [ agents p-major: P x R x L | locals g-major: N x R x KL | global: R x KG ]

Appending frame f writes slot f mod R of every stream with one HIP scatter
(``hier_kv_append``).  A re-run of the same block (a denoising step)
overwrites the same pages, which is the reference's refresh-in-place; a new
frame overwrites the page of frame f - R, which is the reference's eviction.
No row ever moves and nothing is concatenated: the attention tile list
addresses the pool rows directly.
"""

from __future__ import annotations

import ctypes as C
from typing import Optional

import numpy as np
import torch

from . import _capi


def _stream(dev) -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


class HierPagedKVCache:
    """One layer's hierarchical KV cache (pools + ring bookkeeping).

    Reads like the reference's cache dict for the keys the attention module
    inspects (``hier_hub``, ``num_players``, ``num_groups``,
    ``num_local_hub_tokens``, ``num_global_hub_tokens``, ``hier_no_local_hub``).

    ``batch`` > 1 holds that many caches of the same topology in one pool,
    interleaved per row: ``k`` / ``v`` are ``[rows, batch * H, D]``, so batch
    member b's head h is head ``b * H + h``.  The classifier-free-guidance
    pair of caches (wan_video_Nplayers.py:645-648, one model call per prompt
    at :739-776) then shares the ring bookkeeping, the tile list and one
    kernel launch per block, which sees ``batch * H`` heads.
    """

    def __init__(self, *, num_players: int, num_groups: int, num_patches: int,
                 num_local_hub_tokens: int, num_global_hub_tokens: int, num_heads: int,
                 head_dim: int, local_attn_size: int, num_frame_per_block: int, device,
                 dtype=torch.bfloat16, max_frames: Optional[int] = None,
                 hier_no_local_hub: bool = False, batch: int = 1):
        self.P, self.N, self.L = int(num_players), int(num_groups), int(num_patches)
        self.KL, self.KG = int(num_local_hub_tokens), int(num_global_hub_tokens)
        self.H, self.D = int(num_heads), int(head_dim)
        self.B = int(batch)
        if self.B < 1:
            raise ValueError(f"batch must be >= 1, got {batch}")
        self.W, self.n = int(local_attn_size), int(num_frame_per_block)
        self.no_local = bool(hier_no_local_hub)
        if self.no_local and (self.KL != 0 or self.KG <= 0):
            raise ValueError("hier_no_local_hub requires K_L=0 and K_G>0")
        if self.W == -1:
            if max_frames is None:
                raise ValueError("an unbounded window (local_attn_size=-1) needs max_frames")
            self.R = int(max_frames)
        else:
            if self.W < self.n:
                raise ValueError("hier_hub requires local_attn_size=-1 or >= num_frame_per_block")
            self.R = self.W + self.n
        self.a_rows = self.P * self.R * self.L
        self.l_rows = 0 if self.no_local else self.N * self.R * self.KL
        self.g_rows = self.R * self.KG
        rows = self.a_rows + self.l_rows + self.g_rows
        self.device = torch.device(device)
        self.k = torch.zeros((rows, self.B * self.H, self.D), dtype=dtype, device=self.device)
        self.v = torch.zeros_like(self.k)
        self.slot_frame = np.full(self.R, -1, dtype=np.int64)
        self.local_active = np.zeros((max(self.N, 1), self.R), dtype=bool)
        self._dst_cache = {}

    # ---- the reference dict contract (read-only) -------------------------------

    def _meta(self):
        return {"hier_hub": True, "num_players": self.P, "num_groups": self.N,
                "num_local_hub_tokens": self.KL, "num_global_hub_tokens": self.KG,
                "hier_no_local_hub": self.no_local}

    def __getitem__(self, key):
        return self._meta()[key]

    def get(self, key, default=None):
        return self._meta().get(key, default)

    def reset(self):
        """Forget every cached frame (wan_video_Nplayers.py:1024-1058)."""
        self.slot_frame.fill(-1)
        self.local_active.fill(False)

    # ---- addressing ----------------------------------------------------------------

    def agent_row(self, p: int, frame: int) -> int:
        return (p * self.R + frame % self.R) * self.L

    def local_row(self, g: int, frame: int) -> int:
        return self.a_rows + (g * self.R + frame % self.R) * self.KL

    def global_row(self, frame: int) -> int:
        return self.a_rows + self.l_rows + (frame % self.R) * self.KG

    def block_rows(self, start_frame: int, n: int) -> np.ndarray:
        """Pool row of every token of a block in the cached query order
        [P*n*L agents | n*N*KL locals | n*KG global]."""
        P, N, L, KL, KG = self.P, self.N, self.L, self.KL, self.KG
        fr = start_frame + np.arange(n)
        slot = fr % self.R
        agent = ((np.arange(P)[:, None, None] * self.R + slot[None, :, None]) * L +
                 np.arange(L)[None, None, :]).reshape(-1)
        local = (self.a_rows + (np.arange(N)[None, :, None] * self.R + slot[:, None, None]) * KL +
                 np.arange(KL)[None, None, :]).reshape(-1) if not self.no_local else \
            np.zeros(0, np.int64)
        glob = (self.a_rows + self.l_rows + slot[:, None] * KG + np.arange(KG)[None, :]).reshape(-1)
        return np.concatenate([agent, local, glob]).astype(np.int32)

    # ---- append ----------------------------------------------------------------------

    def append(self, k_blk: torch.Tensor, v_blk: torch.Tensor, start_frame: int, n: int,
               active_block) -> None:
        """Write a block's roped K and V ``[S_blk, batch * H, D]`` (cached
        order; batch-major heads) into the pages of frames [start_frame,
        start_frame + n); ``active_block`` [n, N] are the local-hub slot flags
        of those frames."""
        S = self.P * n * self.L + n * ((0 if self.no_local else self.N * self.KL) + self.KG)
        HB = self.B * self.H
        if k_blk.shape != (S, HB, self.D) or v_blk.shape != (S, HB, self.D):
            raise ValueError(f"block K/V must be [{S}, {HB}, {self.D}], "
                             f"got {tuple(k_blk.shape)}, {tuple(v_blk.shape)}")
        if k_blk.dtype != self.k.dtype or v_blk.dtype != self.k.dtype:
            raise ValueError("block K/V dtype must match the cache")
        if n > self.R:
            raise ValueError(f"a block of {n} frames does not fit a window of {self.R} frames")
        if self.W == -1 and (start_frame < 0 or start_frame + n > self.R):
            # an unbounded window keeps every frame: a ring slot may never be
            # reused, or the window would silently lose its oldest frames
            raise ValueError(f"frames [{start_frame}, {start_frame + n}) exceed the cache's "
                             f"max_frames={self.R} (local_attn_size=-1 keeps every frame)")
        key = (start_frame % self.R, n)
        dst = self._dst_cache.get(key)
        if dst is None:
            dst = torch.from_numpy(self.block_rows(start_frame, n)).to(self.device)
            self._dst_cache[key] = dst
        if k_blk.stride(2) != 1 or v_blk.stride(2) != 1:
            k_blk, v_blk = k_blk.contiguous(), v_blk.contiguous()
        args = _capi.HierPageArgs(
            H=HB, D=self.D, n_rows=S, pool_rows=self.k.shape[0], k_src=k_blk.data_ptr(),
            v_src=v_blk.data_ptr(), k_src_ss=k_blk.stride(0), k_src_sh=k_blk.stride(1),
            v_src_ss=v_blk.stride(0), v_src_sh=v_blk.stride(1), dst_rows=dst.data_ptr(),
            k_pool=self.k.data_ptr(), v_pool=self.v.data_ptr(), pool_ss=self.k.stride(0),
            pool_sh=self.k.stride(1))
        _capi.call("hier_kv_append", C.byref(args), _stream(self.device))
        act = np.asarray(active_block, dtype=bool).reshape(n, -1)
        for j in range(n):
            slot = (start_frame + j) % self.R
            self.slot_frame[slot] = start_frame + j
            if not self.no_local:
                self.local_active[:, slot] = act[j, :self.N]

    # ---- window ----------------------------------------------------------------------

    def window(self, end_frame: int):
        """Frames held for a block ending at ``end_frame`` (the last R written
        frames up to it), their pool bases per stream and the local-hub active
        flag of each cached local frame."""
        f = self.slot_frame
        frames = sorted(int(x) for x in f[(f >= 0) & (f <= end_frame) & (f > end_frame - self.R)])
        agent = [[self.agent_row(p, x) for x in frames] for p in range(self.P)]
        local = [] if self.no_local else [[self.local_row(g, x) for x in frames]
                                          for g in range(self.N)]
        glob = [self.global_row(x) for x in frames] if self.KG > 0 else []
        lact = [] if self.no_local else [[bool(self.local_active[g, x % self.R]) for x in frames]
                                         for g in range(self.N)]
        return frames, (agent, local, glob), lact


def init_hier_paged_kv_cache(*, num_layers: int, **kw):
    """One ``HierPagedKVCache`` per transformer layer (the reference allocates
    its per-layer stream dicts in wan_video_Nplayers.py:888-989)."""
    return [HierPagedKVCache(**kw) for _ in range(int(num_layers))]
