"""Device metadata builder: hierarchical topology -> key lists and tile lists.

Host side of ``hier_meta_count`` / ``hier_meta_build`` (``include/hierattn.h``).
The host only lays out tiny per-stream address tables (the token offset of every
cached frame); the edge rule itself -- which frames of which stream each query
segment may read -- is evaluated on the GPU, which then expands and packs:

* ``SegmentedMetadata`` -- the tuple returned by the reference's
  ``_build_metadata`` (multics/models/kernels/hier_segmented_attention.py:156-395),
  bit-exact;
* ``HierTiledBlockLayout`` -- the reference's Tiled128 layout dataclass
  (hier_tiled_attention.py:37-49, 182-655), bit-exact, with a handle to
* ``TileList`` -- this library's attention work list: per (block, stream) the
  ordered union of the per-frame key lists with a visibility bitmask per key.

Two-pass sizing: the count pass is followed by one small device-to-host copy
(the counts), exactly where the reference's own builder runs on the host, and
results are cached in bounded LRU caches keyed by the topology values, like the
reference's (hier_segmented_attention.py:22-24, 137-153;
hier_tiled_attention.py:165-179).
"""

from __future__ import annotations

import ctypes as C
import dataclasses
import os
import weakref
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

from . import _capi

TILE_KEYS = 64          # attention kernel key tile
ROWS_PER_ITEM = 128     # attention kernel query rows per work item (4 waves x 32)
SEG_ROUND = 64          # hier_segmented_attention.py:371
TILED_N = 128           # hier_tiled_attention.py:33
TILED_M = 16            # hier_tiled_attention.py:32
# temporal blocks whose hub streams share one work group in a full-sequence
# list: a hub stream has n * KL (or n * KG) rows per block against a key list
# as long as a member's.  Same-box forward times, per-block / 2 / 4 blocks:
# C2 2.409 / 2.308 / 2.317 ms, P6 3.626 / 3.514 / 3.543, C3 5.635 / 5.500 /
# 5.504, P10 7.355 / 7.260 / 7.529 (random per-block groups: the union of four
# blocks' members is mostly masked), C5 0.700 / 0.698 / 0.696
MERGE_HUB_BLOCKS = 2

# A forward's own list of at least this many items runs its longest key lists
# first.  Same-box medians of five rounds, stream-major order against
# longest-first: C2 (301 items) 2.129 / 2.093 ms, P6 (448) 3.206 / 3.169,
# P10 (757) 6.999 / 6.901, but C5 (161 items, ~7 workgroups per slot at 24
# heads) 0.650 / 0.662: a short launch keeps the stream-major order, whose
# neighbouring items share key frames in L2.
LPT_MIN_ITEMS = 256


def _ceil(a: int, b: int) -> int:
    return -(-a // b)


@dataclass
class TileList:
    """Work list consumed by ``hier_attn_fwd`` (device tensors)."""

    items: torch.Tensor          # [n_items, 8] int32
    kv_idx: torch.Tensor         # [n_keys] int32
    kv_mask: torch.Tensor        # [n_keys] int32 (uint32 bits)
    blk_and: torch.Tensor        # [n_keys / 64] int32 (uint32 bits)
    n_items: int
    item_ranges: tuple           # per block: ((first item, end item) per stream, ...)
    logical_pairs: int           # useful (q, k) pairs (FLOP accounting)
    key_extent: int = 0          # 1 + largest K/V row index any key can address
    row_extent: int = 0          # 1 + largest Q/O row index any item can address
    rows_per_item: int = ROWS_PER_ITEM
    frames_per_group: int = 0    # query frames of every (block, stream) group; 0 = unknown
    # the items' rows are every row of [0, row_extent) exactly once (recorded
    # by the builder from the groups' row descriptors; False = not known)
    rows_exact_cover: bool = False
    n_groups: int = 0            # groups (items sharing a list); 0 = count from item_ranges
    merged_blocks: int = 1       # hub streams merged over this many blocks (item_ranges empty)
    # The forward's own items (None: ``items``): the players' ragged last items
    # folded into their local hubs' groups, whose items (qstride -1) take
    # their rows from ``row_table`` ([rows, 2] int32 token, mask bit).  The
    # backward and the key-major derivation use ``items``.
    fwd_items: Optional[torch.Tensor] = None
    fwd_n_items: int = 0
    row_table: Optional[torch.Tensor] = None


@dataclass(frozen=True)
class HierTiledBlockLayout:
    """Same fields as the reference dataclass (hier_tiled_attention.py:37-49)."""

    prog_qbase: torch.Tensor
    prog_nq: torch.Tensor
    prog_seg: torch.Tensor
    kv_index: torch.Tensor
    kv_valid: torch.Tensor
    kv_count: torch.Tensor
    logical_slots: int
    physical_slots: int
    dense_slots: int
    tiles: Optional[TileList] = field(default=None, compare=False, repr=False)
    block: int = field(default=0, compare=False, repr=False)


@dataclass
class BuildResult:
    tiles: TileList
    segmented: Optional[list]     # per block: (qbase, nq, seg, kv_index, kv_count, pairs)
    tiled: Optional[list]         # per block: HierTiledBlockLayout
    seg_counts: torch.Tensor      # [B, n_seg] (cpu)


# --------------------------------------------------------------------------
# topology description
# --------------------------------------------------------------------------

@dataclass
class BlockTopology:
    """Inputs of the builder for B blocks, as host numpy arrays.

    Frame lists are per block and per stream kind (equal lengths inside a
    block, as the reference requires: hier_segmented_attention.py:185-202).
    """

    P: int
    N: int
    L: int
    KL: int
    KG: int
    n_frames: int
    n_block: int
    local_attn: int
    direct: bool
    no_local: bool
    agent_frames: list            # B x [P][fa]
    local_frames: list            # B x [N][fl]
    global_frames: list           # B x [fg]
    local_active: list            # B x [N][fl] bool
    q_frames: list                # B x [n]
    q_active: list                # B x [n][N] bool
    labels: Optional[list] = None         # B x [n][P]
    membership: Optional[np.ndarray] = None   # [T][N][P] bool
    global_only: Optional[np.ndarray] = None  # [T][P] bool
    # addressing
    ref_agent_base: list = None   # B x [P][fa]
    ref_local_base: list = None
    ref_global_base: list = None
    tile_agent_base: list = None
    tile_local_base: list = None
    tile_global_base: list = None
    ref_qbase: list = None        # B x [P+N+1]
    tile_qbase: list = None
    ref_qstride: tuple = (0, 0, 0)
    tile_qstride: tuple = (0, 0, 0)
    # set by full_sequence_topology, whose frame lists satisfy the per-row
    # checks of validate() by construction (kept = [b1 - W - n, b1) clipped
    # at 0, which holds the block's query frames since W >= n)
    frames_valid: bool = False

    @property
    def B(self) -> int:
        return len(self.agent_frames)

    @property
    def n_seg(self) -> int:
        return self.n_frames * (self.P + (0 if self.no_local else self.N) + 1)

    def validate(self) -> None:
        P, N, n = self.P, self.N, self.n_frames
        if not 1 <= n <= 32:
            raise NotImplementedError(f"n_frames must be in [1, 32], got {n}")
        if self.no_local and self.KL != 0:
            raise ValueError("hier_no_local_hub metadata requires K_L=0 and empty local caches")
        T_mem = None if self.membership is None else self.membership.shape[0]
        if self.frames_valid:
            last = max((f for qf in self.q_frames for f in qf), default=0)
            if T_mem is not None and last >= T_mem:
                raise ValueError(f"membership T={T_mem} does not cover the cached frames")
            return
        for b in range(self.B):
            af = self.agent_frames[b]
            if len(af) != P or any(len(x) != len(af[0]) for x in af):
                raise ValueError("segmented hierarchical attention requires equal agent cache lengths")
            if not self.no_local:
                lf = self.local_frames[b]
                if len(lf) != N or any(len(x) != len(lf[0]) for x in lf):
                    raise ValueError("segmented hierarchical attention requires equal local cache lengths")
            for row in list(af) + list(self.local_frames[b]) + [self.global_frames[b]]:
                r = np.asarray(row, dtype=np.int64)
                if r.size and (r.min() < 0 or np.any(np.diff(r) <= 0)):
                    raise ValueError("cached frame ids must be non-negative and strictly increasing")
            for p in range(P):
                if self.direct and any(f not in set(af[p]) for f in self.q_frames[b]):
                    raise ValueError("every agent cache must hold the current query frames")
            if T_mem is not None:
                allf = [f for row in af for f in row] + list(self.q_frames[b])
                if max(allf, default=0) >= T_mem:
                    raise ValueError(f"membership T={T_mem} does not cover the cached frames")


def _cached_pool_bases(P, N, L, KL, KG, fa, fl, fg):
    """Token offsets of the reference's concatenated cache pool (hier_segmented_attention.py:247-258)."""
    agent = [[(p * fa + fi) * L for fi in range(fa)] for p in range(P)]
    local_start = P * fa * L
    local = [[local_start + (g * fl + fi) * KL for fi in range(fl)] for g in range(N)]
    glob0 = local_start + N * fl * KL
    glob = [glob0 + fi * KG for fi in range(fg)]
    return agent, local, glob


def cached_topology(*, P, N, L, KL, KG, n_frames, n_block, local_attn, agent_frame_lists,
                    local_frame_lists, global_frame_list, local_active_frames, labels, q_active,
                    direct_player, membership=None, global_only=None, hier_no_local_hub=False,
                    tile_bases=None, tile_qbase=None, tile_qstride=None) -> BlockTopology:
    """One cached call (B = 1) in the reference's cached pool and query order."""
    no_local = bool(hier_no_local_hub)
    fa = len(agent_frame_lists[0])
    fl = 0 if no_local else len(local_frame_lists[0])
    fg = len(global_frame_list)
    n = int(n_frames)
    qf = tuple(global_frame_list[-n:]) if KG > 0 else ()
    if len(qf) != n:
        qf = tuple(agent_frame_lists[0][-n:])
    if len(qf) != n:
        raise ValueError("segmented hierarchical attention cannot identify the current query frames")
    agent, local, glob = _cached_pool_bases(P, N, L, KL, KG, fa, fl, fg)
    aq = P * n * L
    ref_qbase = [p * n * L for p in range(P)] + [aq + g * KL for g in range(N)] + [aq + n * N * KL]
    ref_qstride = (L, N * KL, KG)
    if membership is not None:
        membership = np.asarray(membership, dtype=bool)
        if global_only is None:
            raise ValueError("membership metadata requires global_only")
        global_only = np.asarray(global_only, dtype=bool)
    tb = tile_bases or (agent, local, glob)
    return BlockTopology(
        P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n, n_block=int(n_block),
        local_attn=int(local_attn), direct=bool(direct_player), no_local=no_local,
        agent_frames=[[list(x) for x in agent_frame_lists]],
        local_frames=[[list(x) for x in local_frame_lists] if not no_local else []],
        global_frames=[list(global_frame_list)],
        local_active=[[list(map(bool, x)) for x in local_active_frames] if not no_local else []],
        q_frames=[list(qf)],
        q_active=[[list(map(bool, r)) for r in q_active]],
        labels=None if labels is None else [[list(map(int, r)) for r in labels]],
        membership=membership, global_only=global_only,
        ref_agent_base=[agent], ref_local_base=[local], ref_global_base=[glob],
        tile_agent_base=[tb[0]], tile_local_base=[tb[1]], tile_global_base=[tb[2]],
        ref_qbase=[ref_qbase], tile_qbase=[tile_qbase or ref_qbase],
        ref_qstride=ref_qstride, tile_qstride=tile_qstride or ref_qstride,
    )


def full_sequence_topology(*, P, T, L, N, KL, KG, n, window, direct, labels=None, active=None,
                           membership=None, global_only=None, no_local=False) -> BlockTopology:
    """All T/n temporal blocks of a full training/inference sequence.

    Block b queries frames [b*n, b*n+n) and reads the frames a rolling cache of
    W+n frames would hold (hier_tiled_attention.py:307-333), addressed in the
    full-sequence token order [P*T*L | T*N*KL | T*KG] (hier_masks.py:549-571).
    """
    if T % n != 0:
        raise ValueError(f"Tiled128 requires T % n == 0, got T={T}, n={n}")
    if window != -1 and window < n:
        raise ValueError(f"Tiled128 requires local_attn_size=-1 or >=n, got {window}, n={n}")
    if membership is not None:
        mem = np.asarray(membership, dtype=bool).reshape(T, N, P)
        if global_only is None:
            raise ValueError("membership metadata requires global_only")
        go = np.asarray(global_only, dtype=bool).reshape(T, P)
        act = mem.any(-1) if active is None else np.asarray(active, dtype=bool).reshape(T, N)
        lab = None
    else:
        lab = np.asarray(labels, dtype=np.int64).reshape(T, P)
        if lab.size and (lab.min() < 0 or lab.max() >= N):
            raise ValueError(f"group_labels values must be in [0,{N})")
        if active is None:
            act = np.zeros((T, N), dtype=bool)
            act[np.arange(T)[:, None], lab] = True
        else:
            act = np.asarray(active, dtype=bool).reshape(T, N)
        mem = go = None
    retention = T if window == -1 else window + n
    local_start = P * T * L
    global_start = local_start + T * N * KL
    A, Lo, G, AF, LF, GF, LA, QF, QA, LB, RQ = ([] for _ in range(11))
    for b in range(T // n):
        b0, b1 = b * n, b * n + n
        kept = list(range(max(0, b1 - retention), b1))
        AF.append([kept] * P)
        LF.append([] if no_local else [kept] * N)
        GF.append(kept)
        LA.append([] if no_local else [[bool(act[f, g]) for f in kept] for g in range(N)])
        QF.append(list(range(b0, b1)))
        QA.append([[bool(act[f, g]) for g in range(N)] for f in range(b0, b1)])
        if lab is not None:
            LB.append([[int(x) for x in lab[f]] for f in range(b0, b1)])
        A.append([[(p * T + f) * L for f in kept] for p in range(P)])
        Lo.append([] if no_local else [[local_start + (f * N + g) * KL for f in kept] for g in range(N)])
        G.append([global_start + f * KG for f in kept])
        RQ.append([(p * T + b0) * L for p in range(P)]
                  + [local_start + (b0 * N + g) * KL for g in range(N)]
                  + [global_start + b0 * KG])
    stride = (L, N * KL, KG)
    return BlockTopology(
        P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n, n_block=n, local_attn=window,
        direct=bool(direct), no_local=bool(no_local), agent_frames=AF, local_frames=LF,
        global_frames=GF, local_active=LA, q_frames=QF, q_active=QA,
        labels=LB if lab is not None else None, membership=mem, global_only=go,
        ref_agent_base=A, ref_local_base=Lo, ref_global_base=G,
        tile_agent_base=A, tile_local_base=Lo, tile_global_base=G,
        ref_qbase=RQ, tile_qbase=RQ, ref_qstride=stride, tile_qstride=stride, frames_valid=True)


# --------------------------------------------------------------------------
# device build
# --------------------------------------------------------------------------

def _pad3(rows_per_block, inner, width, dtype=np.int32):
    """B x [inner][<=width] ragged lists -> dense [B, inner, width] array."""
    B = len(rows_per_block)
    out = np.zeros((B, max(inner, 1), max(width, 1)), dtype=dtype)
    for b, rows in enumerate(rows_per_block):
        for i, r in enumerate(rows):
            out[b, i, :len(r)] = r
    return out


def _pad2(rows, width, dtype=np.int32):
    out = np.zeros((len(rows), max(width, 1)), dtype=dtype)
    for b, r in enumerate(rows):
        out[b, :len(r)] = r
    return out


def _qlen(topo: BlockTopology, s: int) -> int:
    if s < topo.P:
        return topo.L
    if s < topo.P + topo.N:
        return 0 if topo.no_local else topo.KL
    return topo.KG


def _seg_qlens(topo: BlockTopology) -> np.ndarray:
    n = topo.n_frames
    q = [topo.L] * (topo.P * n)
    if not topo.no_local:
        q += [topo.KL] * (n * topo.N)
    q += [topo.KG] * n
    return np.asarray(q, dtype=np.int64)


def _progs_per_block(topo: BlockTopology, bm: int) -> int:
    return int(sum(_ceil(int(x), bm) for x in _seg_qlens(topo)))


class _Upload:
    """Small host arrays gathered into one buffer and copied to the device with
    one transfer (each host->device copy costs ~20 us of latency, and a build
    has a few dozen arrays).  ``add`` returns nothing; ``flush`` uploads and
    calls each array's setter with its device address (16-byte aligned)."""

    def __init__(self):
        self._items = []

    def add(self, arr, dtype, setter):
        self._items.append((np.ascontiguousarray(arr, dtype=dtype), setter))

    def flush(self, dev) -> torch.Tensor:
        offs, total = [], 0
        for a, _ in self._items:
            offs.append(total)
            total += -(-max(a.nbytes, 1) // 16) * 16
        host = np.zeros(max(total, 16), np.uint8)
        for (a, _), o in zip(self._items, offs):
            host[o:o + a.nbytes] = a.reshape(-1).view(np.uint8)
        buf = torch.from_numpy(host).to(dev)
        base = buf.data_ptr()
        for (_, setter), o in zip(self._items, offs):
            setter(base + o)
        self._items = []
        return buf


def group_rows_cover(topo: BlockTopology):
    """``(row_extent, exact)``: 1 + the largest query row of the tile list
    built from ``topo``, and whether its (block, stream) groups' query rows
    -- ``tile_qbase + j * qstride + i`` for frame j < n and row i < qlen --
    are every row of ``[0, row_extent)`` exactly once.  The builder splits
    each group's rows into consecutive item ranges, so its items then own
    every row once.  Host arithmetic on the topology; no device access."""
    P, N, n, NS = topo.P, topo.N, topo.n_frames, topo.P + topo.N + 1
    row_ext = 0
    group_rows = []
    for b in range(topo.B):
        for s_ in range(NS):
            ql = _qlen(topo, s_)
            if ql > 0:
                kind = 0 if s_ < P else (1 if s_ < P + N else 2)
                row_ext = max(row_ext, topo.tile_qbase[b][s_] + (n - 1) * topo.tile_qstride[kind] + ql)
                group_rows.append(topo.tile_qbase[b][s_] + topo.tile_qstride[kind] *
                                  np.arange(n, dtype=np.int64)[:, None] +
                                  np.arange(ql, dtype=np.int64)[None, :])
    all_rows = np.concatenate([g.ravel() for g in group_rows]) if group_rows else \
        np.zeros(0, np.int64)
    exact = bool(len(all_rows) == row_ext and (len(all_rows) == 0 or (
        all_rows.min() >= 0 and np.bincount(all_rows, minlength=row_ext).max() == 1)))
    return int(row_ext), exact


def _item_order(P: int, N: int, B: int):
    """(stream, block) order of the work items: local hubs, global, players,
    each over all blocks."""
    return [(s, b) for s in list(range(P, P + N)) + [P + N] + list(range(P)) for b in range(B)]


def _topo_struct(topo: BlockTopology, dev: torch.device):
    """``(HierTopo, device buffer)``: the builder's view of ``topo`` with all of
    its host arrays uploaded in one transfer (the buffer must outlive every
    launch that reads the struct)."""
    P, N, n, B = topo.P, topo.N, topo.n_frames, topo.B
    NS = P + N + 1
    fa = [len(x[0]) for x in topo.agent_frames]
    fl = [0 if topo.no_local else len(x[0]) for x in topo.local_frames]
    fg = [len(x) for x in topo.global_frames]
    fa_max, fl_max, fg_max = max(fa), max(fl + [0]), max(fg + [0])
    use_mem = topo.membership is not None
    T_mem = topo.membership.shape[0] if use_mem else 0

    host = {
        "fa": np.asarray(fa, np.int32), "fl": np.asarray(fl, np.int32), "fg": np.asarray(fg, np.int32),
        "agent_frames": _pad3(topo.agent_frames, P, fa_max),
        "local_frames": _pad3(topo.local_frames, N, fl_max),
        "global_frames": _pad2(topo.global_frames, fg_max),
        "local_active": _pad3(topo.local_active, N, fl_max, np.uint8),
        "q_frames": np.asarray(topo.q_frames, np.int32).reshape(B, n),
        "q_active": np.asarray(topo.q_active, np.uint8).reshape(B, n, N),
        "labels": (np.asarray(topo.labels, np.int32).reshape(B, n, P) if topo.labels is not None
                   else np.zeros((1,), np.int32)),
        "membership": (np.ascontiguousarray(topo.membership, dtype=np.uint8) if use_mem
                       else np.zeros((1,), np.uint8)),
        "global_only": (np.ascontiguousarray(topo.global_only, dtype=np.uint8) if use_mem
                        else np.zeros((1,), np.uint8)),
        "ref_agent_base": _pad3(topo.ref_agent_base, P, fa_max),
        "ref_local_base": _pad3(topo.ref_local_base, N, fl_max),
        "ref_global_base": _pad2(topo.ref_global_base, fg_max),
        "tile_agent_base": _pad3(topo.tile_agent_base, P, fa_max),
        "tile_local_base": _pad3(topo.tile_local_base, N, fl_max),
        "tile_global_base": _pad2(topo.tile_global_base, fg_max),
        "ref_qbase": np.asarray(topo.ref_qbase, np.int32).reshape(B, NS),
        "tile_qbase": np.asarray(topo.tile_qbase, np.int32).reshape(B, NS),
    }
    t = _capi.HierTopo(P=P, N=N, L=topo.L, KL=topo.KL, KG=topo.KG, n_frames=n,
                       n_block=topo.n_block, local_attn=topo.local_attn, direct=int(topo.direct),
                       no_local=int(topo.no_local), use_membership=int(use_mem), B=B,
                       fa_max=fa_max, fl_max=fl_max, fg_max=fg_max, T_mem=T_mem)
    up = _Upload()
    for k, v in host.items():
        up.add(v, v.dtype, lambda ptr, k=k: setattr(t, k, ptr))
    dv = up.flush(dev)
    if topo.labels is None:
        t.labels = None
    if not use_mem:
        t.membership = t.global_only = None
    t.ref_qstride = (C.c_int32 * 3)(*topo.ref_qstride)
    t.tile_qstride = (C.c_int32 * 3)(*topo.tile_qstride)
    return t, dv


def _member(topo: BlockTopology, b: int, f: int, g: int, p: int) -> bool:
    """Whether player p belongs to group slot g at query frame f of block b."""
    if topo.membership is not None:
        return bool(topo.membership[topo.q_frames[b][f], g, p])
    if topo.labels is not None:
        return int(topo.labels[b][f][p]) == g
    return False


class _HubMerge:
    """The hub-stream merge of a tile list (``hier_merge_hub_lists``): host
    plan and device arrays, replayable on new lists of the same layout.

    With ``G >= 2`` (full-sequence lists) the hub streams of G consecutive
    temporal blocks share one group, and the shared list (forward and
    backward) is those groups' items followed by the players' items.  With
    ``G == 1`` nothing is merged: the shared list is the built list.

    With ``fold_tails`` the merge also writes a forward-only list: each local
    hub group may take the ragged last item of the players that belong to its
    hub in the rows' frames (a member's keys are a subset of its hub's, so the
    group's key list does not grow), as long as the group's rows fit the
    items it has anyway and its masks have bits left.  Those rows get mask
    bits of their own above the hub's frames and are addressed through a row
    table of (token, bit) pairs.  The dQ pass and the key-major derivation
    keep the list without them; the dK / dV pass replays the fold on the
    key-major list (``key_fold``, ``folded_key_list``)."""

    def __init__(self, topo: BlockTopology, G: int, tile_h, item_start, nit, n_keys: int,
                 n_items: int, rows_per_item: int, key_rows: int, dev, fold_tails: bool = False):
        P, N, n, B = topo.P, topo.N, topo.n_frames, topo.B
        rpi = rows_per_item
        self.merge = G >= 2
        hubs = ([] if topo.no_local else list(range(P, P + N))) + [P + N]
        src_item, src_group, src_shift, src_from, src_nbits = [], [], [], [], []
        caps, desc, nits = [], [], []

        def add_source(item, group, shift, first_bit=0, nbits=32):
            src_item.append(int(item))
            src_group.append(group)
            src_shift.append(int(shift))
            src_from.append(int(first_bit))
            src_nbits.append(int(nbits))

        # hub groups: merged groups of the shared list, or (G == 1) the built
        # list's own hub items, which only the fold reads
        local_hubs = []       # (group or None, hub stream, blocks, sources, capacity, descriptor)
        for s in hubs:
            ql = _qlen(topo, s)
            if ql <= 0:
                continue
            kind = 1 if s < P + N else 2
            for b0 in range(0, B, max(G, 1)):
                blocks = list(range(b0, min(B, b0 + max(G, 1))))
                srcs = [(int(item_start[b, s]), n * (b - b0)) for b in blocks]
                cap = int(sum(int(tile_h[b, s]) for b in blocks))
                d = [int(topo.tile_qbase[b0][s]), int(topo.tile_qstride[kind]), ql, n * len(blocks)]
                g = None
                if self.merge:
                    g = len(caps)
                    for it_, sh in srcs:
                        add_source(it_, g, sh)
                    caps.append(cap)
                    desc.append(d)
                    nits.append(-(-ql * d[3] // rpi))
                if kind == 1:
                    local_hubs.append((g, s, blocks, srcs, cap, d))
        self.n_groups = len(caps)                     # groups of the shared list
        self.n_items = int(sum(nits))
        # ---- forward-only groups: local hubs with their members' last items
        rows_tab, folded, replaced, taken = [], [], [], set()
        # per forward-only group: the hub's built items, [(tail's built item,
        # first bit, bits, shift)], row-table offset, rows, shared group
        fold_groups = []
        n_it_p = r0 = 0
        if fold_tails and topo.L > 0:
            ql_p = topo.L
            rows_p = n * ql_p
            n_it_p = -(-rows_p // rpi)
            r0 = (n_it_p - 1) * rpi
            tail_rows = rows_p - r0
            f0, f1 = r0 // ql_p, (rows_p - 1) // ql_p
            nb = f1 - f0 + 1
            for g, s, blocks, srcs, cap, d in (local_hubs if tail_rows < rpi else []):
                ql, frames = d[2], d[3]
                hub_rows = ql * frames
                room = max(1, -(-hub_rows // rpi)) * rpi - hub_rows
                bits = frames
                tails = []
                for b in blocks:
                    for p in range(P):
                        if ((b, p) in taken or tail_rows > room or bits + nb > 32
                                or int(tile_h[b, p]) == 0):
                            continue
                        if all(_member(topo, b, f, s - P, p) for f in range(f0, f1 + 1)):
                            tails.append((b, p, bits))
                            taken.add((b, p))
                            room -= tail_rows
                            bits += nb
                if not tails:
                    continue
                fg = len(caps)
                for it_, sh in srcs:
                    add_source(it_, fg, sh)
                table_off = len(rows_tab)
                for r in range(hub_rows):
                    f = r // ql
                    rows_tab.append((d[0] + f * d[1] + r - f * ql, f))
                for b, p, bit in tails:
                    add_source(item_start[b, p], fg, bit, f0, nb)
                    cap += int(tile_h[b, p])
                    pb, ps = int(topo.tile_qbase[b][p]), int(topo.tile_qstride[0])
                    for r in range(r0, rows_p):
                        f = r // ql_p
                        rows_tab.append((pb + f * ps + r - f * ql_p, bit + f - f0))
                n_rows = len(rows_tab) - table_off
                caps.append(cap)
                desc.append([table_off, -1, 1, n_rows])
                nits.append(-(-n_rows // rpi))
                folded.append(g)
                fold_groups.append(([int(item_start[b, s]) + i for b in blocks
                                     for i in range(int(nit[b, s]))],
                                    [(int(item_start[b, p]) + n_it_p - 1, f0, nb, bit)
                                     for b, p, bit in tails], table_off, n_rows, g))
                if not self.merge:
                    replaced += [int(item_start[b, s]) + i for b in blocks
                                 for i in range(int(nit[b, s]))]
        self.n_all_groups = len(caps)
        item_off = np.concatenate([[0], np.cumsum(nits)]).astype(np.int64)
        self.n_out_items = int(item_off[-1])
        off = n_keys + np.concatenate([[0], np.cumsum(caps)]).astype(np.int64)
        self.capacity = int(off[-1])
        # first built item the shared list keeps (the players' with a merge)
        self.first_player = int(item_start[0, 0]) if self.merge else 0
        self.frames = n * G if self.merge else n
        self.folded_tails = len(taken)
        i32 = lambda a: torch.tensor(np.asarray(a, np.int32).reshape(-1), device=dev)
        self._dev = dict(src_item=i32(src_item), src_group=i32(src_group), src_shift=i32(src_shift),
                         src_from=i32(src_from), src_nbits=i32(src_nbits),
                         out_off=torch.tensor(off[:-1], dtype=torch.int64, device=dev),
                         out_cap=i32(caps), group_desc=i32(desc), group_item_off=i32(item_off[:-1]))
        self.acc = torch.empty((max(self.n_all_groups, 1), key_rows), dtype=torch.int32,
                               device=dev)
        self.n_src, self.rows, self.rpi = len(src_item), key_rows, rpi
        # the forward list, as indices into [all merge items | the built items
        # the shared list keeps]: the forward-only groups first, the shared
        # groups (or hub items) they do not replace, the players' items but
        # the folded last ones
        self.fwd_index = self.row_table = None
        self.fwd_n_items = 0
        # the fold in the shared list's item numbering (the key-major list's
        # items are the shared list's): per forward-only group, the shared
        # items it replaces, its sources (first item, first bit, bits,
        # shift) and its row-table range
        n_sh = lambda i: self.n_items + i - self.first_player if self.merge else i
        self.key_fold = []
        for hub_built, tails, t_off, n_rows, g in fold_groups:
            hub_items = (list(range(int(item_off[g]), int(item_off[g + 1]))) if self.merge
                         else hub_built)
            srcs_k = [(hub_items[0], 0, 32, 0)] + [(n_sh(ti), fb, nbits, sh)
                                                    for ti, fb, nbits, sh in tails]
            self.key_fold.append((hub_items + [n_sh(ti) for ti, *_ in tails], srcs_k, t_off,
                                  n_rows))
        if folded:
            idx = list(range(self.n_items, self.n_out_items))
            done = set(folded)
            for g in range(self.n_groups):
                if g not in done:
                    idx += list(range(int(item_off[g]), int(item_off[g + 1])))
            skip = {int(item_start[b, p]) + n_it_p - 1 for b, p in taken} | set(replaced)
            idx += [self.n_out_items + i - self.first_player
                    for i in range(self.first_player, n_items) if i not in skip]
            self.fwd_index = torch.tensor(idx, dtype=torch.int64, device=dev)
            self.fwd_n_items = len(idx)
            self.row_table = torch.tensor(rows_tab, dtype=torch.int32, device=dev).reshape(-1, 2)

    def run(self, items, kv_idx, kv_mask, blk_and, n_items: int, stream):
        """Merged lists into their slots; the shared list's items and the
        forward list's items (None without folded rows)."""
        out = torch.empty((max(self.n_out_items, 1), 8), dtype=torch.int32, device=items.device)
        d = self._dev
        a = _capi.HierMergeArgs(
            n_groups=self.n_all_groups, n_src=self.n_src, rows=self.rows, rows_per_item=self.rpi,
            items=items.data_ptr(), kv_idx=kv_idx.data_ptr(), kv_mask=kv_mask.data_ptr(),
            blk_and=blk_and.data_ptr(), acc=self.acc.data_ptr(),
            **{k: v.data_ptr() for k, v in d.items()}, out_items=out.data_ptr())
        _capi.call("hier_merge_hub_lists", C.byref(a), stream)
        kept = items[self.first_player:n_items]
        shared = torch.cat([out[:self.n_items], kept]) if self.merge else items[:n_items]
        if self.fwd_index is None:
            return shared, None
        return shared, torch.cat([out[:self.n_out_items], kept]).index_select(0, self.fwd_index)


def build(topo: BlockTopology, device, *, segmented_block_m: Optional[int] = None,
          tiled: bool = False, rows_per_item: int = ROWS_PER_ITEM,
          merge_hubs: Optional[int] = None, fold_tails: Optional[bool] = None) -> BuildResult:
    """Run the two device passes and return device tensors.  With
    ``merge_hubs = G >= 2`` (full-sequence topologies), the hub streams of G
    consecutive temporal blocks share one work group (``_HubMerge``).  The
    default merges ``MERGE_HUB_BLOCKS`` blocks for full-sequence topologies
    when no reference-format arrays are requested (those callers may launch
    subsets of blocks through ``item_ranges``, which a merged list does not
    keep).  ``fold_tails`` (default: with a merge; without one it takes the
    built list's hub items) also writes the forward's own list, in which the
    players' ragged last items join their local hubs' groups
    (``TileList.fwd_items``)."""
    if merge_hubs is None:
        merge_hubs = MERGE_HUB_BLOCKS if (topo.frames_valid and not tiled and
                                          segmented_block_m is None) else 0
    topo.validate()
    dev = torch.device(device)
    if dev.type != "cuda":
        raise NotImplementedError("the hierarchical metadata builder runs on the GPU (HIP)")
    P, N, n, B = topo.P, topo.N, topo.n_frames, topo.B
    NS = P + N + 1
    t, dv = _topo_struct(topo, dev)
    stream = C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    n_seg = topo.n_seg
    # the five count arrays in one buffer: one fill, one readback
    cnt = torch.zeros(4 * B * n_seg + B * NS, dtype=torch.int32, device=dev)
    seg_c, til_c, den_c, log_c = (cnt[i * B * n_seg:(i + 1) * B * n_seg] for i in range(4))
    tile_c = cnt[4 * B * n_seg:]
    counts = _capi.HierMetaCounts(seg_count=seg_c.data_ptr(), tiled_count=til_c.data_ptr(),
                                  dense_count=den_c.data_ptr(), logical_count=log_c.data_ptr(),
                                  tile_count=tile_c.data_ptr())
    _capi.call("hier_meta_count", C.byref(t), C.byref(counts), stream)
    cnt_h = cnt.cpu().numpy().astype(np.int64)
    seg_h, til_h, den_h, log_h = (cnt_h[i * B * n_seg:(i + 1) * B * n_seg].reshape(B, n_seg)
                                  for i in range(4))
    tile_h = cnt_h[4 * B * n_seg:].reshape(B, NS)

    out = _capi.HierMetaOut()
    keep = []

    # the offset arrays of the output layout, uploaded together before the build
    up = _Upload()

    def dbuf(arr, dtype, field):
        up.add(np.asarray(arr), dtype, lambda ptr: setattr(out, field, ptr))

    # ---- tile list ----------------------------------------------------------
    tile_off = np.concatenate([[0], np.cumsum(tile_h.reshape(-1))])
    n_keys = int(tile_off[-1])
    rows = np.array([[n * _qlen(topo, s) for s in range(NS)] for _ in range(B)], dtype=np.int64)
    nit = -(-rows // rows_per_item)
    # Work-item order: stream-major (local hubs, global, players), then block.
    # Consecutive items of one player cover consecutive temporal blocks, whose
    # key windows overlap in all but n frames, so the workgroups an XCD runs
    # together share most of their K/V lines in that XCD's L2; the longest
    # key lists (local hubs) start first and the short global ones do not end
    # the launch (1 % at C2).  Block-major orders, which run a block's hub
    # items beside its player items, measured 4-8 % slower at C2.
    item_start = np.zeros((B, NS), dtype=np.int64)
    cursor = 0
    for s, b in _item_order(P, N, B):
        item_start[b, s] = cursor
        cursor += int(nit[b, s])
    n_items = cursor
    key_ext = 0
    for b in range(B):
        for rows_, w in ((topo.tile_agent_base[b], topo.L), (topo.tile_local_base[b], topo.KL),
                         (topo.tile_global_base[b], topo.KG)):
            flat = [x for r in rows_ for x in (r if isinstance(r, (list, tuple)) else [r])]
            if flat and w > 0:
                key_ext = max(key_ext, max(flat) + w)
    merge = None
    G = min(int(merge_hubs), 32 // n) if merge_hubs else 0
    merging = G >= 2 and topo.frames_valid and B >= 2
    # the fold pays on long launches (C2: -5 %); on a cached block (C4
    # rollout: ~3 workgroups per slot) the folded groups' long lists end the
    # launch (+5 %), so it is on by default only with the merge
    fold = merging if fold_tails is None else bool(fold_tails)
    if merging:
        merge = _HubMerge(topo, G, tile_h, item_start, nit, n_keys, n_items, rows_per_item,
                          int(key_ext), dev, fold_tails=fold)
    elif fold and not topo.no_local:
        # no merge: the forward's own list only (the players' last rows in
        # their local hubs' items), when some fold
        merge = _HubMerge(topo, 1, tile_h, item_start, nit, n_keys, n_items, rows_per_item,
                          int(key_ext), dev, fold_tails=True)
        if merge.fwd_index is None:
            merge = None
    cap = merge.capacity if merge is not None else n_keys
    kv_idx = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
    kv_mask = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
    blk_and = torch.empty(max(cap // TILE_KEYS, 1), dtype=torch.int32, device=dev)
    items = torch.empty((max(n_items, 1), 8), dtype=torch.int32, device=dev)
    dbuf(tile_off[:-1], np.int64, "tile_kv_off")
    dbuf(item_start.reshape(-1), np.int32, "tile_item_off")
    out.rows_per_item = rows_per_item
    out.tile_kv_idx, out.tile_kv_mask = kv_idx.data_ptr(), kv_mask.data_ptr()
    out.tile_blk_and, out.tile_items = blk_and.data_ptr(), items.data_ptr()

    qlens = _seg_qlens(topo)
    pairs = (seg_h * qlens[None, :]).sum(1)

    # ---- _build_metadata arrays ---------------------------------------------
    seg_res = None
    if segmented_block_m is not None:
        bm = int(segmented_block_m)
        maxk = np.array([_ceil(max(int(seg_h[b].max(initial=0)), 1), SEG_ROUND) * SEG_ROUND
                         for b in range(B)])
        kv_off = np.concatenate([[0], np.cumsum(maxk * n_seg)])
        npb = _progs_per_block(topo, bm)
        prog_off = np.arange(B + 1, dtype=np.int64) * npb
        s_kv = torch.empty(max(int(kv_off[-1]), 1), dtype=torch.int32, device=dev)
        s_cnt = torch.empty(B * n_seg, dtype=torch.int32, device=dev)
        s_pq = torch.empty(max(B * npb, 1), dtype=torch.int32, device=dev)
        s_pn = torch.empty_like(s_pq)
        s_ps = torch.empty_like(s_pq)
        out.block_m = bm
        dbuf(prog_off[:-1], np.int64, "seg_prog_off")
        dbuf(kv_off[:-1], np.int64, "seg_kv_off")
        dbuf(maxk, np.int32, "seg_max_k")
        out.seg_prog_qbase, out.seg_prog_nq, out.seg_prog_seg = (s_pq.data_ptr(), s_pn.data_ptr(),
                                                                 s_ps.data_ptr())
        out.seg_kv_index, out.seg_kv_count = s_kv.data_ptr(), s_cnt.data_ptr()
        seg_res = [(s_pq[b * npb:(b + 1) * npb], s_pn[b * npb:(b + 1) * npb],
                    s_ps[b * npb:(b + 1) * npb],
                    s_kv[int(kv_off[b]):int(kv_off[b + 1])].view(n_seg, int(maxk[b])),
                    s_cnt[b * n_seg:(b + 1) * n_seg], int(pairs[b])) for b in range(B)]

    # ---- Tiled128 arrays ----------------------------------------------------
    tiled_res = None
    if tiled:
        if topo.membership is not None or topo.no_local:
            raise ValueError("Tiled128 layouts are defined for the labels topology with local hubs")
        maxk = np.array([_ceil(max(int(til_h[b].max(initial=0)), 1), TILED_N) * TILED_N
                         for b in range(B)])
        kv_off = np.concatenate([[0], np.cumsum(maxk * n_seg)])
        npb = _progs_per_block(topo, TILED_M)
        prog_off = np.arange(B + 1, dtype=np.int64) * npb
        t_kv = torch.empty(max(int(kv_off[-1]), 1), dtype=torch.int32, device=dev)
        t_va = torch.empty(max(int(kv_off[-1]), 1), dtype=torch.uint8, device=dev)
        t_cnt = torch.empty(B * n_seg, dtype=torch.int32, device=dev)
        t_pq = torch.empty(max(B * npb, 1), dtype=torch.int32, device=dev)
        t_pn = torch.empty_like(t_pq)
        t_ps = torch.empty_like(t_pq)
        dbuf(prog_off[:-1], np.int64, "tiled_prog_off")
        dbuf(kv_off[:-1], np.int64, "tiled_kv_off")
        dbuf(maxk, np.int32, "tiled_max_k")
        out.tiled_prog_qbase, out.tiled_prog_nq, out.tiled_prog_seg = (
            t_pq.data_ptr(), t_pn.data_ptr(), t_ps.data_ptr())
        out.tiled_kv_index, out.tiled_kv_valid = t_kv.data_ptr(), t_va.data_ptr()
        out.tiled_kv_count = t_cnt.data_ptr()
        tiled_res = []
        for b in range(B):
            tiled_res.append(dict(
                prog_qbase=t_pq[b * npb:(b + 1) * npb], prog_nq=t_pn[b * npb:(b + 1) * npb],
                prog_seg=t_ps[b * npb:(b + 1) * npb],
                kv_index=t_kv[int(kv_off[b]):int(kv_off[b + 1])].view(n_seg, int(maxk[b])),
                kv_valid=t_va[int(kv_off[b]):int(kv_off[b + 1])].view(n_seg, int(maxk[b])),
                kv_count=t_cnt[b * n_seg:(b + 1) * n_seg],
                logical_slots=int(log_h[b].sum()), physical_slots=int(til_h[b].sum()),
                dense_slots=int(den_h[b].sum())))

    keep.append(up.flush(dev))
    _capi.call("hier_meta_build", C.byref(t), C.byref(out), stream)

    ranges = tuple(tuple((int(item_start[b, s]), int(item_start[b, s] + nit[b, s]))
                         for s in range(NS) if nit[b, s] > 0) for b in range(B))
    row_ext, exact = group_rows_cover(topo)
    if merge is not None and merge.merge:
        final, fwd = merge.run(items, kv_idx, kv_mask, blk_and, n_items, stream)
        if fwd is not None and fwd.shape[0] >= LPT_MIN_ITEMS:
            # longest key lists first (stable: the items of one list stay
            # together, in stream-major order among equal lengths)
            fwd = fwd.index_select(0, torch.argsort(-fwd[:, 6], stable=True))
        n_player = n_items - merge.first_player
        tiles = TileList(items=final, kv_idx=kv_idx, kv_mask=kv_mask, blk_and=blk_and,
                         n_items=int(final.shape[0]), item_ranges=(),
                         logical_pairs=int(pairs.sum()), key_extent=int(key_ext),
                         row_extent=int(row_ext), rows_per_item=rows_per_item,
                         frames_per_group=merge.frames, rows_exact_cover=exact,
                         n_groups=merge.n_groups + P * B, merged_blocks=G,
                         fwd_items=fwd, fwd_n_items=merge.fwd_n_items, row_table=merge.row_table)
        tiles._merge = merge
        tiles._prebuild_items = n_items
        assert tiles.n_items == merge.n_items + n_player
    else:
        fwd = None
        if merge is not None:          # the forward's own list only
            _, fwd = merge.run(items, kv_idx, kv_mask, blk_and, n_items, stream)
        tiles = TileList(items=items[:n_items], kv_idx=kv_idx, kv_mask=kv_mask, blk_and=blk_and,
                         n_items=n_items, item_ranges=ranges, logical_pairs=int(pairs.sum()),
                         key_extent=int(key_ext), row_extent=int(row_ext),
                         rows_per_item=rows_per_item, frames_per_group=int(n),
                         rows_exact_cover=exact, fwd_items=fwd,
                         fwd_n_items=merge.fwd_n_items if merge is not None else 0,
                         row_table=merge.row_table if merge is not None else None)
    tiles._keepalive = (dv, keep, merge)  # device inputs must outlive the async build
    # the fold plan, which the key-major list can take too (folded_key_list)
    tiles._fold = merge if merge is not None and merge.key_fold else None
    tiles._layout = (tile_off[:-1].copy(), item_start.reshape(-1).copy())   # per (block, stream)
    launch_list(tiles)
    layouts = None
    if tiled_res is not None:
        layouts = [HierTiledBlockLayout(tiles=tiles, block=b, **d) for b, d in enumerate(tiled_res)]
    return BuildResult(tiles=tiles, segmented=seg_res, tiled=layouts,
                       seg_counts=torch.from_numpy(seg_h.astype(np.int32)))


# --------------------------------------------------------------------------
# key-major (transposed) tile list for the backward
# --------------------------------------------------------------------------

def transpose_tiles_host(tiles: TileList) -> TileList:
    """Key-major counterpart of a full-sequence tile list (dK / dV pass of
    ``hier_attn_bwd``), built on the host: the specification of the device
    builder ``hier_derive_*`` (``backward_lists``), which must equal it bit
    for bit.

    In a full-sequence topology every token is a query row of exactly one
    (block, stream) group and a key of the same group; the forward list of a
    group is its ordered key list, a concatenation of whole key frames of
    other groups, each with a bitmask over the group's query frames.  The
    transposed list of a group is the ordered list of query rows that see any
    of its key frames, each with a bitmask over the group's key frames: items
    keep the forward items' row descriptors (now key rows), the lists hold
    query rows.  Query units are ordered by (query group, query frame); lists
    are padded to 64 rows with (row 0, mask 0).
    """
    dev = tiles.items.device
    items = tiles.items[:tiles.n_items].cpu().numpy().astype(np.int64)
    kv_idx = tiles.kv_idx.cpu().numpy().astype(np.int64)
    kv_mask = tiles.kv_mask.cpu().numpy().astype(np.int64) & 0xFFFFFFFF
    first = np.nonzero(items[:, 3] == 0)[0]            # first item of each group
    n_groups = len(first)
    qbase, qstride, qlen = items[first, 0], items[first, 1], items[first, 2]
    off, cnt, nfr = items[first, 5], items[first, 6], items[first, 7]
    grp_of_item = np.repeat(np.arange(n_groups), np.diff(np.append(first, len(items))))

    # token -> (group, row inside the group)
    S = int(tiles.row_extent)
    tok_g = np.full(S, -1, np.int64)
    tok_r = np.full(S, -1, np.int64)
    for g in range(n_groups):
        rows = np.arange(int(nfr[g] * qlen[g]))
        j = rows // qlen[g]
        toks = qbase[g] + j * qstride[g] + rows - j * qlen[g]
        if (tok_g[toks] >= 0).any():
            raise AssertionError("transpose_tiles: a token is a query row of two groups")
        tok_g[toks] = g
        tok_r[toks] = rows

    # edges (query group g, key group G, key frame f) -> query-frame mask
    pos = np.concatenate([np.arange(o, o + c) for o, c in zip(off, cnt)]) if n_groups else \
        np.zeros(0, np.int64)
    qg = np.repeat(np.arange(n_groups), cnt)
    m = kv_mask[pos]
    live = m != 0
    pos, qg, m = pos[live], qg[live], m[live]
    key = kv_idx[pos]
    if len(key) and (key.max() >= S or (tok_g[key] < 0).any()):
        raise AssertionError("transpose_tiles: a key is not a query row of any group")
    kg = tok_g[key]
    kf = tok_r[key] // qlen[kg]
    code = (qg * n_groups + kg) * 32 + kf
    ucode, inv, ucount = np.unique(code, return_inverse=True, return_counts=True)
    umask = np.zeros(len(ucode), np.int64)
    np.bitwise_or.at(umask, inv, m)
    mask_and = np.full(len(ucode), 0xFFFFFFFF, np.int64)
    np.bitwise_and.at(mask_and, inv, m)
    e_qg, rest = np.divmod(ucode, n_groups * 32)
    e_kg, e_kf = np.divmod(rest, 32)
    if (ucount != qlen[e_kg]).any() or (mask_and != umask).any():
        raise AssertionError("transpose_tiles: key lists are not whole key frames")

    # per key group: query units (g, j) with a bitmask over key frames
    nq_max = int(nfr.max(initial=1))
    lists = []
    for G in range(n_groups):
        sel = np.nonzero(e_kg == G)[0]
        unit_bits = {}
        for e in sel:
            g, f, qm = int(e_qg[e]), int(e_kf[e]), int(umask[e])
            for j in range(nq_max):
                if (qm >> j) & 1:
                    unit_bits[(g, j)] = unit_bits.get((g, j), 0) | (1 << f)
        lists.append(sorted(unit_bits.items()))
    sizes = np.array([sum(int(qlen[g]) for (g, _), _ in l) for l in lists], np.int64)
    padded = -(-sizes // TILE_KEYS) * TILE_KEYS
    new_off = np.concatenate([[0], np.cumsum(padded)])
    n_q = int(new_off[-1])
    q_idx = np.zeros(max(n_q, 1), np.int64)
    q_mask = np.zeros(max(n_q, 1), np.int64)
    pairs = 0
    for G, l in enumerate(lists):
        p = int(new_off[G])
        for (g, j), bits in l:
            w = int(qlen[g])
            q_idx[p:p + w] = qbase[g] + j * qstride[g] + np.arange(w)
            q_mask[p:p + w] = bits
            pairs += w * int(qlen[G]) * bin(bits).count("1")
            p += w
    if pairs != tiles.logical_pairs:
        raise AssertionError(f"transpose_tiles: {pairs} pairs, forward list has {tiles.logical_pairs}")
    blk = q_mask[:max(n_q, TILE_KEYS)].reshape(-1, TILE_KEYS) if n_q else np.zeros((1, TILE_KEYS), np.int64)
    blk_and = np.bitwise_and.reduce(blk, axis=1) if n_q else np.zeros(1, np.int64)
    kitems = items.copy()
    kitems[:, 5] = new_off[grp_of_item]
    kitems[:, 6] = padded[grp_of_item]

    def to_dev(a):
        return torch.from_numpy((a & 0xFFFFFFFF).astype(np.uint32).view(np.int32).copy()).to(dev)

    out = TileList(items=torch.from_numpy(kitems.astype(np.int32)).to(dev),
                   kv_idx=to_dev(q_idx), kv_mask=to_dev(q_mask), blk_and=to_dev(blk_and),
                   n_items=tiles.n_items, item_ranges=tiles.item_ranges,
                   logical_pairs=pairs, key_extent=tiles.row_extent, row_extent=tiles.key_extent,
                   rows_per_item=tiles.rows_per_item, rows_exact_cover=tiles.rows_exact_cover,
                   n_groups=tiles.n_groups, frames_per_group=tiles.frames_per_group,
                   merged_blocks=tiles.merged_blocks)
    return out


def ste_tiles_host(tiles: TileList, *, P: int, T: int, L: int, N: int, KL: int):
    """Query-major list of the membership-gated edges of a full-sequence tile
    list (the membership STE pass of ``hier_attn_bwd``).

    An edge's existence depends on exactly one membership bit (t, g, p) when it
    joins player p's row at frame t to a local-hub key of group g, or group g's
    local-hub row at frame t to a key of player p (membership at the query
    frame, hier_masks.py:593-594, 611-612).  The list keeps, per player group,
    its local-hub keys and, per local-hub group, its player keys, with the
    forward masks and per key the class (g for player rows, p for hub rows);
    other groups are dropped.  Returns ``(TileList, kv_class)`` or None when no
    edge is gated.  Host specification of the device builder (``backward_lists``).
    """
    a0, g0 = P * T * L, P * T * L + T * N * KL
    dev = tiles.items.device
    items = tiles.items[:tiles.n_items].cpu().numpy().astype(np.int64)
    kv_idx = tiles.kv_idx.cpu().numpy().astype(np.int64)
    kv_mask = tiles.kv_mask.cpu().numpy().astype(np.int64) & 0xFFFFFFFF
    first = np.nonzero(items[:, 3] == 0)[0]
    ends = np.append(first[1:], len(items))
    out_items, idx_parts, mask_parts, cls_parts = [], [], [], []
    cursor = 0
    for f0, f1 in zip(first, ends):
        qb, off, cnt = int(items[f0, 0]), int(items[f0, 5]), int(items[f0, 6])
        if qb >= g0 or cnt == 0:
            continue
        k = kv_idx[off:off + cnt]
        m = kv_mask[off:off + cnt]
        if qb < a0:                      # player rows: local-hub keys, class = group
            sel = (m != 0) & (k >= a0) & (k < g0)
            cls = ((k - a0) // max(KL, 1)) % max(N, 1)
        else:                            # local-hub rows: player keys, class = player
            sel = (m != 0) & (k < a0)
            cls = k // (T * L)
        if not sel.any():
            continue
        n = int(sel.sum())
        pad = -n % TILE_KEYS
        # keys grouped by class (stable), so most 32-key blocks hold one class
        # and the pass adds one sum per lane and block
        order = np.argsort(cls[sel], kind="stable")
        idx_parts += [k[sel][order], np.zeros(pad, np.int64)]
        mask_parts += [m[sel][order], np.zeros(pad, np.int64)]
        cls_parts += [cls[sel][order], np.zeros(pad, np.int64)]
        for it in range(f0, f1):
            row = items[it].copy()
            row[5], row[6] = cursor, n + pad
            out_items.append(row)
        cursor += n + pad
    if not out_items:
        res = None
    else:
        def to_dev(a):
            return torch.from_numpy((a & 0xFFFFFFFF).astype(np.uint32).view(np.int32).copy()).to(dev)
        idx = np.concatenate(idx_parts)
        msk = np.concatenate(mask_parts)
        blk = np.bitwise_and.reduce(msk.reshape(-1, TILE_KEYS), axis=1)
        lst = TileList(items=torch.from_numpy(np.asarray(out_items, np.int32)).to(dev),
                       kv_idx=to_dev(idx), kv_mask=to_dev(msk), blk_and=to_dev(blk),
                       n_items=len(out_items), item_ranges=(), logical_pairs=0,
                       key_extent=tiles.key_extent, row_extent=tiles.row_extent,
                       rows_per_item=tiles.rows_per_item)
        res = (lst, to_dev(np.concatenate(cls_parts)))
    return res


def ste_classes_host(tiles: TileList, *, P: int, T: int, L: int, N: int, KL: int) -> np.ndarray:
    """Membership-STE class of every entry of a full-sequence forward list
    (``tile_kv_class`` of ``hier_attn_bwd``, which then sums the gated dS in
    its dQ pass): the selection of ``ste_tiles_host`` kept in forward-list
    order -- g for a local-hub key of group g in a player group's list, p for
    a key of player p in a local-hub group's list, -1 for every other entry
    and for entries with mask 0.  Host specification of the device builder
    ``hier_derive_ste_classes`` (``ste_classes``); int32 ``[len(kv_idx)]``."""
    a0, g0 = P * T * L, P * T * L + T * N * KL
    items = tiles.items[:tiles.n_items].cpu().numpy().astype(np.int64)
    kv_idx = tiles.kv_idx.cpu().numpy().astype(np.int64)
    kv_mask = tiles.kv_mask.cpu().numpy().astype(np.int64) & 0xFFFFFFFF
    cls = np.full(len(kv_idx), -1, np.int64)
    # each item's own range (the items of a group share theirs; a launch
    # list's cut items may each cover only part of it)
    for qb, off, cnt in items[:, [0, 5, 6]]:
        lo, hi = max(int(off), 0), min(int(off + cnt), len(kv_idx))
        if qb >= g0 or hi <= lo:
            continue
        k, m = kv_idx[lo:hi], kv_mask[lo:hi]
        if qb < a0:                      # player rows: local-hub keys, class = group
            sel = (m != 0) & (k >= a0) & (k < g0)
            c = ((k - a0) // max(KL, 1)) % max(N, 1)
        else:                            # local-hub rows: player keys, class = player
            sel = (m != 0) & (k >= 0) & (k < a0)
            c = k // max(T * L, 1)
        cls[lo:hi] = np.where(sel, c, -1)
    return cls.astype(np.int32)


def ste_first_tiles_host(tiles: TileList, cls: np.ndarray) -> np.ndarray:
    """Per item, the first 64-entry tile of its list holding an STE class
    (``tile_ste_first`` of ``hier_attn_bwd``; the list's tile count if none):
    the dQ pass sums the STE from that tile on.  int32 ``[n_items]``."""
    items = tiles.items[:tiles.n_items].cpu().numpy().astype(np.int64)
    out = np.empty(len(items), np.int64)
    for i, (off, cnt) in enumerate(items[:, [5, 6]]):
        hit = np.nonzero(cls[max(off, 0):max(off + cnt, 0)] >= 0)[0]
        out[i] = hit[0] // TILE_KEYS if len(hit) else -(-cnt // TILE_KEYS)
    return out.astype(np.int32)


def ste_classes(tiles: TileList, ste_geometry):
    """``(ste_classes_host, ste_first_tiles_host)`` of a device tile list as
    device tensors, built on the GPU by ``hier_derive_ste_classes`` and cached
    on ``tiles`` per geometry."""
    key = tuple(int(x) for x in ste_geometry)
    cache = tiles.__dict__.setdefault("_ste_classes", {})
    hit = cache.get(key)
    if hit is not None:
        return hit
    if not tiles.items.is_cuda:
        raise NotImplementedError("ste_classes builds on the GPU; use ste_classes_host")
    P, T, L, N, KL = key
    n = int(tiles.kv_idx.numel())
    a = _capi.HierDeriveArgs(n_items=tiles.n_items, kv_len=n, P=P, T=T, L=L, N=N, KL=KL,
                             items=tiles.items.data_ptr(), kv_idx=tiles.kv_idx.data_ptr(),
                             kv_mask=tiles.kv_mask.data_ptr())
    cls = torch.empty(max(n, 4), dtype=torch.int32, device=tiles.items.device)
    first = torch.empty(max(tiles.n_items, 1), dtype=torch.int32, device=tiles.items.device)
    _capi.call("hier_derive_ste_classes", C.byref(a), cls.data_ptr(), first.data_ptr(),
               torch.cuda.current_stream(tiles.items.device).cuda_stream)
    cache[key] = (cls, first)
    return cache[key]


_DERIVE_ERRORS = ((1, "a token is a query row of two groups"),
                  (2, "a key is not a query row of any group"),
                  (4, "key lists are not whole key frames"),
                  (8, "the work items are not grouped by key list"),
                  (16, "a list offset does not fit in 32 bits"))


def _groups_and_frames(tiles: TileList):
    if tiles.n_groups and tiles.frames_per_group:
        return int(tiles.n_groups), int(tiles.frames_per_group)
    if tiles.item_ranges and tiles.frames_per_group:
        return sum(len(b) for b in tiles.item_ranges), int(tiles.frames_per_group)
    it = tiles.items[:tiles.n_items].cpu().numpy()
    return int((it[:, 3] == 0).sum()), int(it[:, 7].max(initial=1))


def _derive_device(tiles: TileList, ste_geometry):
    """Both backward lists of a device tile list with the ``hier_derive_*``
    kernels (two passes, one read-back of the totals in between)."""
    dev = tiles.items.device
    ng, nq = _groups_and_frames(tiles)
    P, T, L, N, KL = (int(x) for x in ste_geometry) if ste_geometry is not None else (0,) * 5
    a = _capi.HierDeriveArgs(n_items=tiles.n_items, n_groups=ng, rows=int(tiles.row_extent),
                             nq_max=nq, kv_len=int(tiles.kv_idx.numel()), P=P, T=T, L=L, N=N,
                             KL=KL, items=tiles.items.data_ptr(), kv_idx=tiles.kv_idx.data_ptr(),
                             kv_mask=tiles.kv_mask.data_ptr())
    ws_bytes = int(_capi.lib().hier_derive_workspace(C.byref(a)))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    totals = torch.zeros(8, dtype=torch.int64, device=dev)
    a.ws, a.ws_bytes, a.totals = ws.data_ptr(), ws_bytes, totals.data_ptr()
    stream = torch.cuda.current_stream(dev).cuda_stream
    _capi.call("hier_derive_count", C.byref(a), stream)
    n_key, pairs, n_ste, n_ste_items, err = (int(x) for x in totals[:5].cpu())
    for bit, msg in _DERIVE_ERRORS:
        if err & bit:
            raise AssertionError(f"transpose_tiles: {msg}")
    if pairs != tiles.logical_pairs:
        raise AssertionError(f"transpose_tiles: {pairs} pairs, forward list has {tiles.logical_pairs}")
    i32 = dict(dtype=torch.int32, device=dev)
    k_items = torch.empty((tiles.n_items, 8), **i32)
    k_idx = torch.zeros(max(n_key, 1), **i32)
    k_mask = torch.zeros(max(n_key, 1), **i32)
    k_blk = torch.zeros(max(n_key // TILE_KEYS, 1), **i32)
    a.key_entries, a.ste_entries = n_key, (n_ste if n_ste_items > 0 else 0)
    a.key_items, a.key_q_idx = k_items.data_ptr(), k_idx.data_ptr()
    a.key_q_mask, a.key_blk_and = k_mask.data_ptr(), k_blk.data_ptr()
    if n_ste_items > 0:
        s_items = torch.empty((n_ste_items, 8), **i32)
        s_idx, s_mask, s_cls = (torch.empty(n_ste, **i32) for _ in range(3))
        s_blk = torch.empty(n_ste // TILE_KEYS, **i32)
        a.ste_items, a.ste_kv_idx, a.ste_kv_mask = (s_items.data_ptr(), s_idx.data_ptr(),
                                                    s_mask.data_ptr())
        a.ste_blk_and, a.ste_kv_class = s_blk.data_ptr(), s_cls.data_ptr()
    _capi.call("hier_derive_build", C.byref(a), stream)
    kt = TileList(items=k_items, kv_idx=k_idx, kv_mask=k_mask, blk_and=k_blk,
                  n_items=tiles.n_items, item_ranges=tiles.item_ranges, logical_pairs=pairs,
                  key_extent=tiles.row_extent, row_extent=tiles.key_extent,
                  rows_per_item=tiles.rows_per_item, rows_exact_cover=tiles.rows_exact_cover,
                  n_groups=tiles.n_groups, frames_per_group=tiles.frames_per_group,
                  merged_blocks=tiles.merged_blocks)
    ste = None
    if n_ste_items > 0:
        lst = TileList(items=s_items, kv_idx=s_idx, kv_mask=s_mask, blk_and=s_blk,
                       n_items=n_ste_items, item_ranges=(), logical_pairs=0,
                       key_extent=tiles.key_extent, row_extent=tiles.row_extent,
                       rows_per_item=tiles.rows_per_item)
        ste = (lst, s_cls)
    kt._keepalive = (ws, totals)
    launch_list(kt)
    return kt, ste


def folded_key_list(tiles: TileList, kt: TileList) -> TileList:
    """The key-major list the dK / dV pass runs: ``kt`` (the key-major list of
    ``tiles``) with the players' last key rows folded into their local hubs'
    key items, as the forward's own list folds their query rows: the same
    groups, the same row table (token, key-frame bit), each group's list the
    union of its sources' query lists (``hier_merge_hub_lists`` on ``kt``'s
    arrays, one read-back of its item sizes).  ``kt`` itself when ``tiles``
    has no fold.  Cached on ``kt``."""
    plan = getattr(tiles, "_fold", None)
    if plan is None or not kt.items.is_cuda:
        return kt
    hit = kt.__dict__.get("_folded")
    if hit is not None:
        return hit
    dev = kt.items.device
    sizes = kt.items[:kt.n_items, 6].cpu().numpy().astype(np.int64)
    src_item, src_group, src_from, src_nbits, src_shift, caps, desc, nits = \
        [], [], [], [], [], [], [], []
    drop = set()
    for g, (items, srcs, t_off, n_rows) in enumerate(plan.key_fold):
        drop.update(items)
        for it, fb, nb, sh in srcs:
            src_item.append(it)
            src_group.append(g)
            src_from.append(fb)
            src_nbits.append(nb)
            src_shift.append(sh)
        caps.append(int(sum(sizes[it] for it, *_ in srcs)))
        desc.append([t_off, -1, 1, n_rows])
        nits.append(-(-n_rows // kt.rows_per_item))
    n_key = int(kt.kv_idx.numel())
    off = n_key + np.concatenate([[0], np.cumsum(caps)]).astype(np.int64)
    item_off = np.concatenate([[0], np.cumsum(nits)]).astype(np.int64)
    cap = int(off[-1])
    i32 = dict(dtype=torch.int32, device=dev)
    kv_idx = torch.empty(cap, **i32)
    kv_mask = torch.empty(cap, **i32)
    blk = torch.empty(cap // TILE_KEYS, **i32)
    kv_idx[:n_key].copy_(kt.kv_idx)
    kv_mask[:n_key].copy_(kt.kv_mask)
    blk[:n_key // TILE_KEYS].copy_(kt.blk_and[:n_key // TILE_KEYS])
    out = torch.empty((max(int(item_off[-1]), 1), 8), **i32)
    arr = lambda a: torch.tensor(np.asarray(a, np.int32), device=dev)
    d = dict(src_item=arr(src_item), src_group=arr(src_group), src_shift=arr(src_shift),
             src_from=arr(src_from), src_nbits=arr(src_nbits),
             out_off=torch.tensor(off[:-1], dtype=torch.int64, device=dev), out_cap=arr(caps),
             group_desc=arr(desc).reshape(-1), group_item_off=arr(item_off[:-1]))
    rows = int(kt.key_extent)                      # query rows: the lists' entries
    acc = torch.empty((len(caps), rows), **i32)
    a = _capi.HierMergeArgs(
        n_groups=len(caps), n_src=len(src_item), rows=rows, rows_per_item=kt.rows_per_item,
        items=kt.items.data_ptr(), kv_idx=kv_idx.data_ptr(), kv_mask=kv_mask.data_ptr(),
        blk_and=blk.data_ptr(), acc=acc.data_ptr(), **{k: v.data_ptr() for k, v in d.items()},
        out_items=out.data_ptr())
    _capi.call("hier_merge_hub_lists", C.byref(a), torch.cuda.current_stream(dev).cuda_stream)
    keep = torch.tensor([i for i in range(kt.n_items) if i not in drop], dtype=torch.int64,
                        device=dev)
    items = torch.cat([out[:int(item_off[-1])], kt.items[:kt.n_items].index_select(0, keep)])
    folded = dataclasses.replace(kt, items=items, n_items=int(items.shape[0]), kv_idx=kv_idx,
                                 kv_mask=kv_mask, blk_and=blk, row_table=tiles.row_table)
    folded._keepalive = (acc, d)
    kt.__dict__["_folded"] = folded
    launch_list(folded)
    return folded


def backward_lists(tiles: TileList, ste_geometry=None):
    """``(key-major list, STE list)`` of a full-sequence tile list for the
    backward, the STE list ``(TileList, kv_class)`` or None (no geometry, or no
    gated edge).  Device lists are derived on the GPU by the ``hier_derive_*``
    kernels, bit for bit the host builders ``transpose_tiles_host`` /
    ``ste_tiles_host``, which serve host lists.  Cached on ``tiles`` per STE
    geometry."""
    key = None if ste_geometry is None else tuple(int(x) for x in ste_geometry)
    cache = tiles.__dict__.setdefault("_derived", {})
    hit = cache.get(key)
    if hit is not None:
        return hit
    if tiles.items.is_cuda:
        res = _derive_device(tiles, key)
    else:
        kt = next(iter(cache.values()))[0] if cache else transpose_tiles_host(tiles)
        ste = None if key is None else ste_tiles_host(tiles, P=key[0], T=key[1], L=key[2],
                                                      N=key[3], KL=key[4])
        res = (kt, ste)
    cache[key] = res
    return res


def _trim_items(items: torch.Tensor, n: int, kv_mask: torch.Tensor,
                row_table: Optional[torch.Tensor]) -> torch.Tensor:
    """``hier_trim_key_lists`` into a new array (asynchronous, no read-back)."""
    out = torch.empty_like(items)
    if n < items.shape[0]:
        out[n:].copy_(items[n:])
    a = _capi.HierTrimArgs(n_items=n, items=items.data_ptr(), kv_mask=kv_mask.data_ptr(),
                           row_table=None if row_table is None else row_table.data_ptr(),
                           out_items=out.data_ptr())
    _capi.call("hier_trim_key_lists", C.byref(a), torch.cuda.current_stream(items.device).cuda_stream)
    return out


def launch_list(tiles: TileList) -> TileList:
    """The list the attention launches run: ``tiles`` with every item's key
    list (``items`` and ``fwd_items``) cut to the 64-entry tiles that some of
    its rows can see (``hier_trim_key_lists``).  The tiles cut away hold only
    masked entries for every row of the item, so each pass gives the results
    of the whole list.  Item order, rows and the kv arrays are shared with
    ``tiles``; the derivations (``backward_lists``, ``folded_key_list``)
    keep reading ``tiles`` itself, the dQ pass's STE classes are built on
    the launch list (``launch_ste_first``).  Built on the current
    stream on first use and cached on ``tiles``; a host list is returned as
    it is."""
    if tiles.__dict__.get("_is_launch"):
        return tiles
    hit = tiles.__dict__.get("_launch")
    if hit is not None:
        return hit
    if not tiles.items.is_cuda:
        return tiles
    items = _trim_items(tiles.items, tiles.n_items, tiles.kv_mask, tiles.row_table)
    fwd = None
    if tiles.fwd_items is not None:
        fwd = _trim_items(tiles.fwd_items, tiles.fwd_n_items, tiles.kv_mask, tiles.row_table)
    run = dataclasses.replace(tiles, items=items, fwd_items=fwd)
    # no reference back to a strong owner: a list built every training step
    # is freed when its last user drops it, without the cycle collector
    run.__dict__["_is_launch"] = True
    run.__dict__["_source"] = weakref.ref(tiles)
    tiles.__dict__["_launch"] = run
    return run


def built_list(tiles: TileList) -> TileList:
    """The list ``tiles`` was cut from when it is a launch list (while that
    list is alive), else ``tiles``."""
    ref = tiles.__dict__.get("_source")
    src = ref() if ref is not None else None
    return src if src is not None else tiles


def launch_ste_first(tiles: TileList, ste_geometry) -> tuple:
    """``ste_classes`` of the launch list (``launch_list(tiles)``): the
    classes per entry and each cut item's first tile holding one."""
    return ste_classes(launch_list(tiles), ste_geometry)


def transpose_tiles(tiles: TileList) -> TileList:
    """Key-major list of ``tiles`` (see ``backward_lists``), cached on it."""
    for (kt, _) in getattr(tiles, "_derived", {}).values():
        return kt
    return backward_lists(tiles)[0]


def ste_tiles(tiles: TileList, *, P: int, T: int, L: int, N: int, KL: int):
    """STE list of ``tiles`` (see ``backward_lists``), cached on it."""
    return backward_lists(tiles, (P, T, L, N, KL))[1]


# --------------------------------------------------------------------------
# reference-named entry points with bounded LRU caches
# --------------------------------------------------------------------------

_META_CACHE: "OrderedDict[tuple, object]" = OrderedDict()
_LAYOUT_CACHE: "OrderedDict[tuple, object]" = OrderedDict()


def _lru_get(cache, key):
    v = cache.get(key)
    if v is not None:
        cache.move_to_end(key)
    return v


def _lru_put(cache, key, value, env, default):
    n = max(int(os.environ.get(env, default)), 0)
    if n == 0:
        return
    cache[key] = value
    cache.move_to_end(key)
    while len(cache) > n:
        cache.popitem(last=False)


def _freeze(x):
    """Hashable cache-key form of a (nested) list / array argument."""
    if x is None:
        return None
    if torch.is_tensor(x):
        x = x.detach().cpu().numpy()
    if not isinstance(x, np.ndarray):
        try:   # rectangular nested lists: one array, one bytes key
            a = np.asarray(x)
        except ValueError:   # ragged
            a = None
        if a is None or a.dtype == object:
            return tuple(_freeze(v) if isinstance(v, (list, tuple, np.ndarray)) else v for v in x)
        x = a
    return (x.shape, x.dtype.str, x.tobytes())


def _build_metadata(*, device, P, N, L, KL, KG, n_frames, n_block, local_attn, agent_frame_lists,
                    local_frame_lists, global_frame_list, local_active_frames, labels, q_active,
                    direct_player, block_m, membership=None, global_only=None,
                    hier_no_local_hub=False, return_tiles=False):
    """Same arguments and return tuple as the reference
    (hier_segmented_attention.py:156-395): ``(prog_qbase, prog_nq, prog_seg,
    kv_index, kv_count, logical_pairs)``; with ``return_tiles`` a seventh
    element holds the attention kernel's ``TileList`` for the same call.
    """
    key = ("seg", str(device), P, N, L, KL, KG, n_frames, n_block, local_attn,
           _freeze(agent_frame_lists), _freeze(local_frame_lists), _freeze(global_frame_list),
           _freeze(local_active_frames), _freeze(labels), _freeze(q_active), bool(direct_player),
           bool(hier_no_local_hub), block_m, _freeze(membership), _freeze(global_only))
    hit = _lru_get(_META_CACHE, key)
    if hit is None:
        topo = cached_topology(
            P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n_frames, n_block=n_block, local_attn=local_attn,
            agent_frame_lists=agent_frame_lists, local_frame_lists=local_frame_lists,
            global_frame_list=global_frame_list, local_active_frames=local_active_frames,
            labels=labels, q_active=q_active, direct_player=direct_player, membership=membership,
            global_only=global_only, hier_no_local_hub=hier_no_local_hub)
        res = build(topo, device, segmented_block_m=block_m)
        hit = (*res.segmented[0], res.tiles)
        _lru_put(_META_CACHE, key, hit, "WAN_HIER_SEGMENTED_META_CACHE_SIZE", "64")
    return hit if return_tiles else hit[:6]


def build_hier_tiled_full_sequence_layouts(*, device, num_players, num_frames, num_patches,
                                           num_groups, num_local_hub_tokens,
                                           num_global_hub_tokens, num_frame_per_block,
                                           local_attn_size, group_labels, active_group,
                                           direct_player):
    """Same signature and per-block layouts as the reference
    (hier_tiled_attention.py:244-429); the layouts also carry the tile list
    the HIP forward consumes (one launch for all blocks)."""
    P, T, L = int(num_players), int(num_frames), int(num_patches)
    N, KL, KG = int(num_groups), int(num_local_hub_tokens), int(num_global_hub_tokens)
    n, window = int(num_frame_per_block), int(local_attn_size)
    labels, active = tiled_full_sequence_inputs(
        num_players=P, num_frames=T, num_groups=N, num_frame_per_block=n,
        local_attn_size=window, group_labels=group_labels, active_group=active_group)
    key = ("full", str(torch.device(device)), P, T, L, N, KL, KG, n, window, labels.tobytes(),
           active.tobytes(), bool(direct_player), TILED_M, TILED_N)
    hit = _lru_get(_LAYOUT_CACHE, key)
    if hit is None:
        topo = full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=window,
                                      direct=direct_player, labels=labels, active=active)
        hit = tuple(build(topo, device, tiled=True).tiled)
        _lru_put(_LAYOUT_CACHE, key, hit, "WAN_HIER_TILED_LAYOUT_CACHE_SIZE", "2")
    return hit


def tiled_full_sequence_inputs(*, num_players, num_frames, num_groups, num_frame_per_block,
                               local_attn_size, group_labels, active_group):
    """The reference's checks of a full-sequence labels topology
    (hier_tiled_attention.py:244-285): ``(labels, active)`` as host arrays."""
    P, T, N = int(num_players), int(num_frames), int(num_groups)
    n, window = int(num_frame_per_block), int(local_attn_size)
    if T % n != 0:
        raise ValueError(f"Tiled128 requires T % n == 0, got T={T}, n={n}")
    if window != -1 and window < n:
        raise ValueError(f"Tiled128 requires local_attn_size=-1 or >=n, got {window}, n={n}")
    if tuple(group_labels.shape) != (T, P) or tuple(active_group.shape) != (T, N):
        raise ValueError(
            "Tiled128 grouping shape mismatch: "
            f"labels={tuple(group_labels.shape)} expected {(T, P)}, "
            f"active={tuple(active_group.shape)} expected {(T, N)}")
    labels = group_labels.detach().to("cpu", torch.long).numpy()
    active = active_group.detach().to("cpu", torch.bool).numpy()
    for s in range(0, T, n):
        if any(not np.array_equal(labels[t], labels[s]) for t in range(s + 1, min(s + n, T))):
            raise ValueError("Tiled128 requires group labels constant inside each temporal block")
    return labels, active


def full_sequence_tiles(*, device, P, T, L, N, KL, KG, n, window, direct, labels=None, active=None,
                        membership=None, global_only=None, no_local=False) -> TileList:
    """Tile list of a full-sequence topology (labels or membership form), kept in
    the same bounded LRU as the tiled layouts (WAN_HIER_TILED_LAYOUT_CACHE_SIZE)."""
    key = ("tiles", str(torch.device(device)), P, T, L, N, KL, KG, n, window, bool(direct),
           bool(no_local), _freeze(labels), _freeze(active), _freeze(membership),
           _freeze(global_only))
    hit = _lru_get(_LAYOUT_CACHE, key)
    if hit is None:
        topo = full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=window,
                                      direct=direct, labels=labels, active=active,
                                      membership=membership, global_only=global_only,
                                      no_local=no_local)
        hit = build(topo, device).tiles
        _lru_put(_LAYOUT_CACHE, key, hit, "WAN_HIER_TILED_LAYOUT_CACHE_SIZE", "2")
    return hit


class MembershipLogitsPlan:
    """Per-step lists of a full-sequence membership topology whose membership
    is ``logits > 0`` of soft logits on the device -- the training case, where
    the reference rebuilds its mask on every forward
    (multics/models/wan_video_dit.py:633-679) -- built without any host
    read-back.

    The geometry's superset topology (every membership bit and every
    global-only bit on) admits every edge any membership can produce: the
    edge rule is monotone in the membership bits except the global-only
    edges, which the superset holds as well.  Its lists are built once; their
    per-(block, stream) sizes bound that stream's list under any membership,
    so each stream keeps the superset's list offset as a fixed slot, and the
    key-major lists fit the superset's total.  A step then
      * derives membership, global_only, the local-slot activity and the
        query-frame activity from the logits with device ops into the
        topology's fixed buffers,
      * runs the tile-list half of ``hier_meta_build`` (each list written in
        its slot, its items carrying its true padded size),
      * runs ``hier_derive_count`` / ``hier_derive_build`` into the bounded
        key-major arrays (offsets scanned on the device),
    all asynchronous on the current stream.  ``logical_pairs`` of a step's
    list is -1 (not counted: that would need a read-back)."""

    def __init__(self, *, device, P, T, L, N, KL, KG, n, window, direct, no_local=False):
        dev = torch.device(device)
        self.geometry = (P, T, L, N, KL, KG, n, window, bool(direct), bool(no_local))
        self.P, self.T, self.N, self.n = P, T, N, n
        ones = dict(membership=np.ones((T, N, P), bool), global_only=np.ones((T, P), bool))
        sup_topo = full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=window,
                                          direct=direct, no_local=no_local, **ones)
        # no folded rows: which players' rows join which hub changes with the logits
        sup = build(sup_topo, dev, fold_tails=False).tiles
        self.t, self._static = _topo_struct(sup_topo, dev)
        B = T // n
        fl_max = int(self.t.fl_max)
        u8 = dict(dtype=torch.uint8, device=dev)
        self.mem = torch.zeros((T, N, P), **u8)
        self.go = torch.zeros((T, P), **u8)
        self.la = torch.zeros((B, max(N, 1), max(fl_max, 1)), **u8)
        self.qa = torch.zeros((B, n, max(N, 1)), **u8)
        # frame of local-slot column fi of block b (padding: valid = 0)
        kf = np.full((B, max(fl_max, 1)), -1, np.int32)
        if not no_local:
            for b in range(B):
                fr = sup_topo.local_frames[b][0]
                kf[b, :len(fr)] = fr
        self.la_frame = torch.from_numpy(kf).to(dev)
        self._margs = _capi.HierMembershipArgs(
            T=T, N=N, P=P, B=B, n=n, fl_max=fl_max, la_frame=self.la_frame.data_ptr(),
            membership=self.mem.data_ptr(), global_only=self.go.data_ptr(),
            q_active=self.qa.data_ptr(), local_active=self.la.data_ptr())
        self.t.membership, self.t.global_only = self.mem.data_ptr(), self.go.data_ptr()
        self.t.local_active, self.t.q_active = self.la.data_ptr(), self.qa.data_ptr()
        tile_off, item_start = sup._layout          # the builder reads int64 / int32
        self._kv_off = torch.from_numpy(tile_off.astype(np.int64)).to(dev)
        self._item_off = torch.from_numpy(item_start.astype(np.int32)).to(dev)
        self.sup = sup
        self.n_keys = int(sup.kv_idx.numel())
        # key-major capacity: the superset's (one read-back, here only)
        kt_sup, _ = backward_lists(sup, None)
        self.key_cap = int(kt_sup.kv_idx.numel())
        self.n_groups, self.nq = _groups_and_frames(sup)
        a = self._derive_args(sup)
        self.ws = torch.empty(max(int(_capi.lib().hier_derive_workspace(C.byref(a))), 1),
                              dtype=torch.uint8, device=dev)
        self.totals = torch.zeros(8, dtype=torch.int64, device=dev)

    def _derive_args(self, tiles: TileList):
        # no STE geometry: the key-major list only (the dQ pass takes the
        # STE classes of the forward list)
        return _capi.HierDeriveArgs(
            n_items=tiles.n_items, n_groups=self.n_groups, rows=int(tiles.row_extent),
            nq_max=self.nq, kv_len=int(tiles.kv_idx.numel()), P=0, T=0, L=0, N=0, KL=0,
            items=tiles.items.data_ptr(), kv_idx=tiles.kv_idx.data_ptr(),
            kv_mask=tiles.kv_mask.data_ptr())

    def build(self, logits: torch.Tensor) -> TileList:
        """The forward tile list of ``logits > 0`` ([T, N, P]) with its
        key-major list cached on it (``backward_lists``)."""
        P, T, N, n = self.P, self.T, self.N, self.n
        dev = self.mem.device
        if tuple(logits.shape) != (T, N, P):
            raise ValueError(f"membership logits must be [T,N,P] = {(T, N, P)}")
        lg = logits.detach().to(device=dev, dtype=torch.float32).contiguous()
        stream = torch.cuda.current_stream(dev).cuda_stream
        self._margs.logits = lg.data_ptr()
        _capi.call("hier_membership_from_logits", C.byref(self._margs), stream)
        sup = self.sup
        i32 = dict(dtype=torch.int32, device=dev)
        merge = getattr(sup, "_merge", None)
        n_pre = sup._prebuild_items if merge is not None else sup.n_items
        items = torch.empty((n_pre, 8), **i32)
        kv_idx = torch.empty(self.n_keys, **i32)
        kv_mask = torch.empty(self.n_keys, **i32)
        blk = torch.empty(max(self.n_keys // TILE_KEYS, 1), **i32)
        out = _capi.HierMetaOut(rows_per_item=sup.rows_per_item)
        out.tile_kv_off = self._kv_off.data_ptr()
        out.tile_item_off = self._item_off.data_ptr()
        out.tile_kv_idx, out.tile_kv_mask = kv_idx.data_ptr(), kv_mask.data_ptr()
        out.tile_blk_and, out.tile_items = blk.data_ptr(), items.data_ptr()
        _capi.call("hier_meta_build", C.byref(self.t), C.byref(out), stream)
        if merge is not None:
            items, _ = merge.run(items, kv_idx, kv_mask, blk, n_pre, stream)
        tiles = TileList(items=items, kv_idx=kv_idx, kv_mask=kv_mask, blk_and=blk,
                         n_items=sup.n_items, item_ranges=sup.item_ranges, logical_pairs=-1,
                         key_extent=sup.key_extent, row_extent=sup.row_extent,
                         rows_per_item=sup.rows_per_item, frames_per_group=sup.frames_per_group,
                         rows_exact_cover=sup.rows_exact_cover, n_groups=sup.n_groups,
                         merged_blocks=sup.merged_blocks)
        # key-major list, sized by the superset's
        a = self._derive_args(tiles)
        a.ws, a.ws_bytes, a.totals = self.ws.data_ptr(), int(self.ws.numel()), self.totals.data_ptr()
        k_items = torch.empty((sup.n_items, 8), **i32)
        k_idx = torch.empty(max(self.key_cap, 1), **i32)
        k_mask = torch.empty(max(self.key_cap, 1), **i32)
        k_blk = torch.empty(max(self.key_cap // TILE_KEYS, 1), **i32)
        a.key_entries, a.ste_entries = self.key_cap, 0
        a.key_items, a.key_q_idx = k_items.data_ptr(), k_idx.data_ptr()
        a.key_q_mask, a.key_blk_and = k_mask.data_ptr(), k_blk.data_ptr()
        _capi.call("hier_derive_count", C.byref(a), stream)
        _capi.call("hier_derive_build", C.byref(a), stream)
        kt = TileList(items=k_items, kv_idx=k_idx, kv_mask=k_mask, blk_and=k_blk,
                      n_items=sup.n_items, item_ranges=sup.item_ranges, logical_pairs=-1,
                      key_extent=sup.row_extent, row_extent=sup.key_extent,
                      rows_per_item=sup.rows_per_item, rows_exact_cover=sup.rows_exact_cover,
                      n_groups=sup.n_groups, frames_per_group=sup.frames_per_group,
                      merged_blocks=sup.merged_blocks)
        tiles.__dict__["_derived"] = {None: (kt, None)}
        tiles._keepalive = (self, a, lg)
        launch_list(tiles)
        launch_list(kt)
        return tiles


_PLAN_LRU: "OrderedDict[tuple, MembershipLogitsPlan]" = OrderedDict()


def membership_logits_tiles(logits: torch.Tensor, *, P, T, L, N, KL, KG, n, window, direct,
                            no_local=False) -> TileList:
    """``MembershipLogitsPlan(...).build(logits)`` with the plan of the
    geometry kept in a small LRU (WAN_HIER_TILED_LAYOUT_CACHE_SIZE)."""
    key = (str(logits.device), P, T, L, N, KL, KG, n, window, bool(direct), bool(no_local))
    plan = _lru_get(_PLAN_LRU, key)
    if plan is None:
        plan = MembershipLogitsPlan(device=logits.device, P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n,
                                    window=window, direct=direct, no_local=no_local)
        _lru_put(_PLAN_LRU, key, plan, "WAN_HIER_TILED_LAYOUT_CACHE_SIZE", "2")
    return plan.build(logits)


def cached_tiles(*, device, P, N, L, KL, KG, n_frames, n_block, local_attn, frames, tile_bases,
                 local_active_frames, labels, q_active, direct_player, membership=None,
                 global_only=None, hier_no_local_hub=False) -> TileList:
    """Tile list of one cached call whose streams all hold the cached frames
    ``frames`` (ascending, the current block's n frames last), with the K/V
    rows of frame i of each stream at ``tile_bases`` = (agent [P][i], local
    [N][i], global [i]) -- a paged pool.  Queries are the block in the cached
    order [P*n*L | n*N*KL | n*KG].  Cached in the segmented-metadata LRU
    (WAN_HIER_SEGMENTED_META_CACHE_SIZE), keyed by the topology and the pages."""
    no_local = bool(hier_no_local_hub)
    fr = tuple(int(x) for x in frames)
    key = ("paged", str(torch.device(device)), P, N, L, KL, KG, n_frames, n_block, local_attn, fr,
           _freeze(tile_bases), _freeze(local_active_frames), _freeze(labels), _freeze(q_active),
           bool(direct_player), no_local, _freeze(membership), _freeze(global_only))
    hit = _lru_get(_META_CACHE, key)
    if hit is None:
        topo = cached_topology(
            P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n_frames, n_block=n_block, local_attn=local_attn,
            agent_frame_lists=[fr] * P, local_frame_lists=[] if no_local else [fr] * N,
            global_frame_list=fr if KG > 0 else (), local_active_frames=local_active_frames,
            labels=labels, q_active=q_active, direct_player=direct_player, membership=membership,
            global_only=global_only, hier_no_local_hub=no_local, tile_bases=tile_bases)
        hit = build(topo, device).tiles
        _lru_put(_META_CACHE, key, hit, "WAN_HIER_SEGMENTED_META_CACHE_SIZE", "64")
    return hit


def cached_stream_tiles(*, device, P, N, L, KL, KG, n_frames, n_block, local_attn,
                        agent_frame_lists, local_frame_lists, global_frame_list,
                        local_active_frames, labels, q_active, direct_player, tile_bases,
                        membership=None, global_only=None, hier_no_local_hub=False) -> TileList:
    """Tile list of one cached call over per-stream frame lists (the
    ``_build_metadata`` inputs) whose K/V rows sit at ``tile_bases`` = (agent
    [P][i], local [N][i], global [i]): the first row of cached frame i of each
    stream in one K/V pool.  Cached in the segmented-metadata LRU."""
    no_local = bool(hier_no_local_hub)
    key = ("streams", str(torch.device(device)), P, N, L, KL, KG, n_frames, n_block, local_attn,
           _freeze(agent_frame_lists), _freeze(local_frame_lists), _freeze(global_frame_list),
           _freeze(tile_bases), _freeze(local_active_frames), _freeze(labels), _freeze(q_active),
           bool(direct_player), no_local, _freeze(membership), _freeze(global_only))
    hit = _lru_get(_META_CACHE, key)
    if hit is None:
        topo = cached_topology(
            P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n_frames, n_block=n_block, local_attn=local_attn,
            agent_frame_lists=agent_frame_lists, local_frame_lists=local_frame_lists,
            global_frame_list=global_frame_list, local_active_frames=local_active_frames,
            labels=labels, q_active=q_active, direct_player=direct_player, membership=membership,
            global_only=global_only, hier_no_local_hub=no_local, tile_bases=tile_bases)
        hit = build(topo, device).tiles
        _lru_put(_META_CACHE, key, hit, "WAN_HIER_SEGMENTED_META_CACHE_SIZE", "64")
    return hit


def build_hier_tiled_cached_layout(*, device, P, N, L, KL, KG, n_frames, n_block, local_attn,
                                   agent_frame_lists, local_frame_lists, global_frame_list,
                                   local_active_frames, labels, q_active, direct_player):
    """Reference signature (hier_tiled_attention.py:474-655)."""
    key = ("cached", str(torch.device(device)), P, N, L, KL, KG, n_frames, n_block, local_attn,
           _freeze(agent_frame_lists), _freeze(local_frame_lists), _freeze(global_frame_list),
           _freeze(local_active_frames), _freeze(labels), _freeze(q_active), bool(direct_player),
           TILED_M, TILED_N)
    hit = _lru_get(_LAYOUT_CACHE, key)
    if hit is None:
        topo = cached_topology(
            P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n_frames, n_block=n_block, local_attn=local_attn,
            agent_frame_lists=agent_frame_lists, local_frame_lists=local_frame_lists,
            global_frame_list=global_frame_list, local_active_frames=local_active_frames,
            labels=labels, q_active=q_active, direct_player=direct_player)
        hit = (build(topo, device, tiled=True).tiled[0],)
        _lru_put(_LAYOUT_CACHE, key, hit, "WAN_HIER_TILED_LAYOUT_CACHE_SIZE", "2")
    return hit[0]


def clear_hier_tiled_layout_cache() -> None:
    """Testing/debug helper (hier_tiled_attention.py:799-801)."""
    _LAYOUT_CACHE.clear()


def clear_metadata_cache() -> None:
    _META_CACHE.clear()


# --------------------------------------------------------------------------
# packed varlen plan
# --------------------------------------------------------------------------

_PLAN_CACHE: "OrderedDict[tuple, dict]" = OrderedDict()


def _get_varlen_plan(*, kv_index, kv_count, qbase, qlen, seg_ids, query_tokens):
    """The packed-varlen plan of ``_build_metadata`` arrays built with one
    program per segment (hier_packed_attention.py:32-102): same keys, dtypes
    and errors.  The segments must partition the query rows
    ``[0, query_tokens)`` exactly (``AssertionError`` otherwise); active
    segments (rows and keys both non-empty) are flattened into ``q_index`` /
    ``k_index`` (int64) with int32 offsets ``cu_q`` / ``cu_k``.

    Validation, flattening and the index range run where the arrays live;
    the host reads back one vector of nine integers per cache miss (the
    checks' outcome, the active-segment count, the flat sizes, the maxima and
    the key index range), which the plan's Python ints and tensor shapes
    need.  The plan is cached by the source tensors' data pointers and keeps
    references to them, so a reused allocation cannot alias a stale plan
    (WAN_HIER_PACKED_PLAN_CACHE_SIZE, default 64, as the reference)."""
    dev = kv_index.device
    key = (str(dev), kv_index.data_ptr(), kv_count.data_ptr(), qbase.data_ptr(), qlen.data_ptr(),
           seg_ids.data_ptr(), int(query_tokens))
    hit = _lru_get(_PLAN_CACHE, key)
    if hit is not None:
        return hit
    flat64 = lambda t: t.detach().reshape(-1).to(device=dev, dtype=torch.int64)
    qb, qn, si, nk = flat64(qbase), flat64(qlen), flat64(seg_ids), flat64(kv_count)
    n = si.numel()
    if qb.numel() != n or qn.numel() != n:
        raise AssertionError("packed metadata must contain exactly one program per segment")
    width = int(kv_index.shape[1]) if kv_index.dim() == 2 else 0
    kv2 = kv_index.detach().reshape(-1, max(width, 1)).to(torch.int64)
    ar = torch.arange(n, device=dev, dtype=torch.int64)
    ids_ok = (si == ar).all() & torch.tensor(nk.numel() >= n and kv2.shape[0] >= n, device=dev)
    # an exact partition in program order: every non-empty program starts
    # where the previous ones end, and together they cover query_tokens rows
    qc = qn.clamp(min=0)
    start = torch.cumsum(qc, 0) - qc
    part_ok = ((qb == start) | (qc == 0)).all() & (qc.sum() == int(query_tokens))
    nk_s = nk[:n] if nk.numel() >= n else torch.zeros(n, device=dev, dtype=torch.int64)
    act = (qn > 0) & (nk_s > 0)
    qa = torch.where(act, qn, 0)
    ka_full = torch.where(act, nk_s, 0)
    ka = ka_full.clamp(max=width)       # a count past the row width gathers the row
    rows = kv2[:n] if kv2.shape[0] >= n else torch.zeros(n, max(width, 1), device=dev,
                                                         dtype=torch.int64)
    live = torch.arange(rows.shape[1], device=dev)[None, :] < ka[:, None]
    big = torch.iinfo(torch.int64).max
    zero = torch.zeros((), device=dev, dtype=torch.int64)
    stats = torch.stack([
        ids_ok.to(torch.int64), part_ok.to(torch.int64), act.sum(), qa.sum(), ka.sum(),
        qa.max() if n else zero, ka_full.max() if n else zero,
        torch.where(live, rows, big).min() if n else zero,
        torch.where(live, rows, -1).max() if n else zero - 1]).cpu().tolist()
    if not stats[0]:
        raise AssertionError("packed metadata must contain exactly one program per segment")
    if not stats[1]:
        raise AssertionError("packed query segments must partition the query sequence exactly")
    n_act, tot_q, tot_k = stats[2], stats[3], stats[4]
    # active segments in order (a stable sort moves them to the front)
    act_idx = torch.argsort((~act).to(torch.int8), stable=True)[:n_act]
    qa_a, ka_a = qa[act_idx], ka[act_idx]
    cu_q = torch.cat([zero[None], torch.cumsum(qa_a, 0)])
    cu_k = torch.cat([zero[None], torch.cumsum(ka_full[act_idx], 0)])
    gk = torch.cat([zero[None], torch.cumsum(ka_a, 0)])
    seg_ids_a = torch.arange(n_act, device=dev)
    row_seg = torch.repeat_interleave(seg_ids_a, qa_a, output_size=tot_q)
    q_flat = qb[act_idx][row_seg] + torch.arange(tot_q, device=dev) - cu_q[row_seg]
    key_seg = torch.repeat_interleave(seg_ids_a, ka_a, output_size=tot_k)
    k_flat = rows[act_idx][key_seg, torch.arange(tot_k, device=dev) - gk[key_seg]]
    res = {
        "q_index": q_flat,
        "k_index": k_flat,
        "cu_q": cu_q.to(torch.int32),
        "cu_k": cu_k.to(torch.int32),
        "max_q": int(stats[5]),
        "max_k": int(stats[6]),
        "min_k_index": int(stats[7]) if tot_k else 0,
        "max_k_index": int(stats[8]) if tot_k else -1,
        "metadata_sources": (kv_index, kv_count, qbase, qlen, seg_ids),
    }
    _lru_put(_PLAN_CACHE, key, res, "WAN_HIER_PACKED_PLAN_CACHE_SIZE", "64")
    return res


def clear_varlen_plan_cache() -> None:
    _PLAN_CACHE.clear()
