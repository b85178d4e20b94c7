"""CPU restatement of the reference's hierarchical attention metadata builders.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates, in a run-based form of this repository's own:

* ``_build_metadata``         multics/models/kernels/hier_segmented_attention.py:156-395
* ``_pack_layout``            multics/models/kernels/hier_tiled_attention.py:182-241
* full-sequence Tiled128      multics/models/kernels/hier_tiled_attention.py:244-429
* cached Tiled128             multics/models/kernels/hier_tiled_attention.py:474-655
* ``_get_varlen_plan``        multics/models/kernels/hier_packed_attention.py:32-102

Every key list of the reference is a concatenation of whole cached frames (a
"run" of L, K_L or K_G consecutive pool tokens), so each builder below first
enumerates candidate runs in the reference's concatenation order with an
``allowed`` flag per run, then expands or packs them.

Parity pins:

* the segmented lists, MAX_K rounding, zero padding and program split are
  checked against golden vectors written by the reference's own
  ``_build_metadata`` (``tests/golden/``), and against an independent
  token-by-token restatement of the cached SDPA masks (the reference's test
  oracle rule, ``tests/test_hier_segmented_metadata.py:22-108``);
* the Tiled128 arrays are checked against golden vectors written by the
  reference's own layout builders, and their logical edges against the dense
  mask (``oracle.masks``) as in ``tests/test_hier_tiled_layout.py:30-95``;
* the varlen plan is built from the reference's own golden segmented lists
  and checked by brute force: its (query, key) pairs are exactly the lists'
  pairs, their count is the reference's ``logical_pairs``, and the refusal
  cases raise (``tests/test_varlen_plan.py``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

TILED_BLOCK_M = 16     # hier_tiled_attention.py:32
TILED_BLOCK_N = 128    # hier_tiled_attention.py:33
SEGMENTED_ROUND = 64   # hier_segmented_attention.py:371


def temporal_ok(qf: int, kf: int, n_block: int, local_attn: int) -> bool:
    """Block-causal + sliding window on frame ids (hier_segmented_attention.py:117-122)."""
    if kf // n_block > qf // n_block:
        return False
    return local_attn == -1 or (qf - kf) < local_attn


@dataclass(frozen=True)
class CachedTopology:
    """Inputs of one cached hierarchical call, as plain Python values.

    Mirrors the keyword set of ``_build_metadata``
    (hier_segmented_attention.py:156-178): frame lists per cached stream, the
    per-frame activity of local slots, per-query-frame labels or absolute-frame
    membership, and the flags.
    """

    P: int
    N: int
    L: int
    KL: int
    KG: int
    n_frames: int
    n_block: int
    local_attn: int
    agent_frames: tuple          # [P][fa] absolute frame ids
    local_frames: tuple          # [N][fl]
    global_frames: tuple         # [fg]
    local_active: tuple          # [N][fl] bool
    labels: Optional[tuple]      # [n][P] int (relative to the query block)
    q_active: tuple              # [n][N] bool
    direct: bool
    membership: Optional[tuple] = None   # [T][N][P] bool, absolute frames
    global_only: Optional[tuple] = None  # [T][P] bool, absolute frames
    no_local: bool = False

    @property
    def fa(self) -> int:
        return len(self.agent_frames[0])

    @property
    def fl(self) -> int:
        return 0 if self.no_local else len(self.local_frames[0])

    def query_frames(self) -> tuple:
        """hier_segmented_attention.py:261-267."""
        n = self.n_frames
        q = tuple(self.global_frames[-n:]) if self.KG > 0 else ()
        if len(q) != n:
            q = tuple(self.agent_frames[0][-n:])
        if len(q) != n:
            raise ValueError("cannot identify the current query frames")
        return q

    # pool layout [agents p-major | locals g-major | global]
    # (hier_segmented_attention.py:247-258)
    def agent_base(self, p: int, fi: int) -> int:
        return (p * self.fa + fi) * self.L

    def local_base(self, g: int, fi: int) -> int:
        return self.P * self.fa * self.L + (g * self.fl + fi) * self.KL

    def global_base(self, fi: int) -> int:
        return self.P * self.fa * self.L + self.N * self.fl * self.KL + fi * self.KG

    def shares_slot(self, qrel: int, qf: int, p: int, o: int) -> bool:
        if self.membership is not None:
            return any(self.membership[qf][g][p] and self.membership[qf][g][o]
                       for g in range(self.N))
        return self.labels[qrel][o] == self.labels[qrel][p]

    def owned_groups(self, qrel: int, qf: int, p: int) -> list:
        if self.membership is not None:
            return [g for g in range(self.N) if self.membership[qf][g][p]]
        return [self.labels[qrel][p]]

    def in_group(self, qrel: int, qf: int, p: int, g: int) -> bool:
        if self.membership is not None:
            return bool(self.membership[qf][g][p])
        return self.labels[qrel][p] == g


def _validate(topo: CachedTopology) -> None:
    """Shape checks of hier_segmented_attention.py:185-220."""
    if not topo.agent_frames or any(len(x) != len(topo.agent_frames[0])
                                    for x in topo.agent_frames):
        raise ValueError("segmented hierarchical attention requires equal agent cache lengths")
    if topo.no_local:
        if topo.KL != 0 or topo.local_frames or topo.local_active:
            raise ValueError("hier_no_local_hub metadata requires K_L=0 and empty local caches")
    elif not topo.local_frames or any(len(x) != len(topo.local_frames[0])
                                      for x in topo.local_frames):
        raise ValueError("segmented hierarchical attention requires equal local cache lengths")
    if topo.membership is not None and topo.global_only is None:
        raise ValueError("membership metadata requires global_only")


# --------------------------------------------------------------------------
# segmented (compact) key lists
# --------------------------------------------------------------------------

def segmented_runs(topo: CachedTopology):
    """Per query segment: (qstart, qlen, [(base, width), ...] allowed runs).

    Segment order, query starts and per-segment key order follow
    hier_segmented_attention.py:269-368.
    """
    _validate(topo)
    P, N, L, KL, KG = topo.P, topo.N, topo.L, topo.KL, topo.KG
    n, nb, W = topo.n_frames, topo.n_block, topo.local_attn
    qframes = topo.query_frames()
    no_local = topo.no_local
    use_mem = topo.membership is not None
    agent_q_len = P * n * L
    local_q_len = n * N * KL
    out = []
    for p in range(P):
        for qrel, qf in enumerate(qframes):
            runs = [(topo.agent_base(p, fi), L)
                    for fi, kf in enumerate(topo.agent_frames[p]) if temporal_ok(qf, kf, nb, W)]
            if topo.direct:
                for o in range(P):
                    if o == p or not topo.shares_slot(qrel, qf, p, o):
                        continue
                    runs += [(topo.agent_base(o, fi), L)
                             for fi, kf in enumerate(topo.agent_frames[o])
                             if kf in qframes and kf // nb == qf // nb]
            if not no_local:
                for g in topo.owned_groups(qrel, qf, p):
                    runs += [(topo.local_base(g, fi), KL)
                             for fi, kf in enumerate(topo.local_frames[g])
                             if topo.local_active[g][fi] and temporal_ok(qf, kf, nb, W)]
            if KG > 0 and (no_local or (use_mem and topo.global_only[qf][p])):
                runs += [(topo.global_base(fi), KG)
                         for fi, kf in enumerate(topo.global_frames) if temporal_ok(qf, kf, nb, W)]
            out.append((p * n * L + qrel * L, L, runs))
    if not no_local:
        for qrel, qf in enumerate(qframes):
            for g in range(N):
                runs = []
                if topo.q_active[qrel][g]:
                    for p in range(P):
                        if topo.in_group(qrel, qf, p, g):
                            runs += [(topo.agent_base(p, fi), L)
                                     for fi, kf in enumerate(topo.agent_frames[p])
                                     if temporal_ok(qf, kf, nb, W)]
                    runs += [(topo.local_base(g, fi), KL)
                             for fi, kf in enumerate(topo.local_frames[g])
                             if topo.local_active[g][fi] and temporal_ok(qf, kf, nb, W)]
                    runs += [(topo.global_base(fi), KG)
                             for fi, kf in enumerate(topo.global_frames) if temporal_ok(qf, kf, nb, W)]
                out.append((agent_q_len + qrel * N * KL + g * KL, KL, runs))
    for qrel, qf in enumerate(qframes):
        runs = []
        if not no_local:
            for g in range(N):
                runs += [(topo.local_base(g, fi), KL)
                         for fi, kf in enumerate(topo.local_frames[g])
                         if topo.local_active[g][fi] and temporal_ok(qf, kf, nb, W)]
        runs += [(topo.global_base(fi), KG)
                 for fi, kf in enumerate(topo.global_frames) if temporal_ok(qf, kf, nb, W)]
        if no_local:
            for p in range(P):
                runs += [(topo.agent_base(p, fi), L)
                         for fi, kf in enumerate(topo.agent_frames[p]) if temporal_ok(qf, kf, nb, W)]
        elif use_mem:
            for p in range(P):
                runs += [(topo.agent_base(p, fi), L)
                         for fi, kf in enumerate(topo.agent_frames[p])
                         if topo.global_only[kf][p] and temporal_ok(qf, kf, nb, W)]
        out.append((agent_q_len + local_q_len + qrel * KG, KG, runs))
    return out


def _expand(runs) -> np.ndarray:
    if not runs:
        return np.zeros(0, dtype=np.int64)
    return np.concatenate([np.arange(b, b + w, dtype=np.int64) for b, w in runs])


def _split_programs(specs, block_m: int):
    """One program per ``block_m`` query rows of each segment (hier_segmented_attention.py:381-384)."""
    qb, nq, sg = [], [], []
    for sid, (qstart, qlen) in enumerate(specs):
        for off in range(0, qlen, block_m):
            qb.append(qstart + off)
            nq.append(min(block_m, qlen - off))
            sg.append(sid)
    as32 = lambda v: np.asarray(v, dtype=np.int32)
    return as32(qb), as32(nq), as32(sg)


def segmented_metadata(topo: CachedTopology, block_m: int) -> dict:
    """Arrays returned by ``_build_metadata`` (hier_segmented_attention.py:370-393)."""
    segs = segmented_runs(topo)
    keys = [_expand(runs) for _, _, runs in segs]
    max_k = max(max((len(k) for k in keys), default=1), 1)
    max_k = math.ceil(max_k / SEGMENTED_ROUND) * SEGMENTED_ROUND
    kv_index = np.zeros((len(segs), max_k), dtype=np.int32)
    kv_count = np.zeros(len(segs), dtype=np.int32)
    logical_pairs = 0
    for sid, ((qstart, qlen, _), k) in enumerate(zip(segs, keys)):
        kv_index[sid, :len(k)] = k
        kv_count[sid] = len(k)
        logical_pairs += qlen * len(k)
    qb, nq, sg = _split_programs([(s[0], s[1]) for s in segs], block_m)
    return dict(prog_qbase=qb, prog_nq=nq, prog_seg=sg, kv_index=kv_index,
                kv_count=kv_count, logical_pairs=int(logical_pairs))


# --------------------------------------------------------------------------
# Tiled128 (layout-preserving) packing
# --------------------------------------------------------------------------

def pack_layout(dense_segments: Sequence[Sequence[tuple]], query_specs) -> dict:
    """``_pack_layout``: keep 128-slot chunks holding >=1 valid slot (hier_tiled_attention.py:182-241).

    ``dense_segments[i]`` is a sequence of ``(base, width, valid)`` runs.
    """
    if len(dense_segments) != len(query_specs):
        raise ValueError("dense segment/query-spec length mismatch")
    B = TILED_BLOCK_N
    selected = []
    logical = physical = dense_total = 0
    for runs in dense_segments:
        idx = _expand([(b, w) for b, w, _ in runs])
        val = (np.concatenate([np.full(w, bool(v)) for _, w, v in runs])
               if runs else np.zeros(0, dtype=bool))
        dense_total += len(idx)
        logical += int(val.sum())
        keep_i, keep_v = [], []
        for start in range(0, len(idx), B):
            ci, cv = idx[start:start + B], val[start:start + B]
            if not cv.any():
                continue
            pad = B - len(ci)
            keep_i.append(np.concatenate([ci, np.zeros(pad, dtype=np.int64)]))
            keep_v.append(np.concatenate([cv, np.zeros(pad, dtype=bool)]))
        si = np.concatenate(keep_i) if keep_i else np.zeros(0, dtype=np.int64)
        sv = np.concatenate(keep_v) if keep_v else np.zeros(0, dtype=bool)
        physical += len(si)
        selected.append((si, sv))
    max_k = max(max((len(s[0]) for s in selected), default=1), 1)
    max_k = math.ceil(max_k / B) * B
    kv_index = np.zeros((len(selected), max_k), dtype=np.int32)
    kv_valid = np.zeros((len(selected), max_k), dtype=np.uint8)
    kv_count = np.zeros(len(selected), dtype=np.int32)
    for sid, (si, sv) in enumerate(selected):
        kv_index[sid, :len(si)] = si
        kv_valid[sid, :len(sv)] = sv
        kv_count[sid] = len(si)
    qb, nq, sg = _split_programs(query_specs, TILED_BLOCK_M)
    return dict(prog_qbase=qb, prog_nq=nq, prog_seg=sg, kv_index=kv_index,
                kv_valid=kv_valid, kv_count=kv_count, logical_slots=int(logical),
                physical_slots=int(physical), dense_slots=int(dense_total))


def tiled_cached_dense(topo: CachedTopology):
    """Dense slot runs of ``build_hier_tiled_cached_layout`` (hier_tiled_attention.py:533-647)."""
    if topo.membership is not None:
        raise ValueError("Tiled128 layouts are defined for labels only")
    P, N, L, KL, KG = topo.P, topo.N, topo.L, topo.KL, topo.KG
    n, nb, W = topo.n_frames, topo.n_block, topo.local_attn
    qframes = (tuple(topo.global_frames[-n:]) if KG > 0 else tuple(topo.agent_frames[0][-n:]))
    if len(qframes) != n:
        raise ValueError("Tiled128 cannot identify the current cached query frames")
    cur_idx = [tuple(topo.agent_frames[o].index(f) for f in qframes) for o in range(P)]
    dense, specs = [], []
    for p in range(P):
        for qrel, qf in enumerate(qframes):
            runs = [(topo.agent_base(p, fi), L, temporal_ok(qf, kf, nb, W))
                    for fi, kf in enumerate(topo.agent_frames[p])]
            if topo.direct:
                for o in range(P):
                    if o == p:
                        continue
                    same = topo.labels[qrel][o] == topo.labels[qrel][p]
                    runs += [(topo.agent_base(o, cur_idx[o][kr]), L, same and kf // nb == qf // nb)
                             for kr, kf in enumerate(qframes)]
            qg = topo.labels[qrel][p]
            for g in range(N):
                runs += [(topo.local_base(g, fi), KL,
                          g == qg and bool(topo.local_active[g][fi]) and temporal_ok(qf, kf, nb, W))
                         for fi, kf in enumerate(topo.local_frames[g])]
            dense.append(runs)
            specs.append((p * n * L + qrel * L, L))
    agent_q_len = P * n * L
    local_q_len = n * N * KL
    for qrel, qf in enumerate(qframes):
        for g in range(N):
            qa = bool(topo.q_active[qrel][g])
            runs = []
            for p in range(P):
                ok = qa and topo.labels[qrel][p] == g
                runs += [(topo.agent_base(p, fi), L, ok and temporal_ok(qf, kf, nb, W))
                         for fi, kf in enumerate(topo.agent_frames[p])]
            runs += [(topo.local_base(g, fi), KL,
                      qa and bool(topo.local_active[g][fi]) and temporal_ok(qf, kf, nb, W))
                     for fi, kf in enumerate(topo.local_frames[g])]
            runs += [(topo.global_base(fi), KG, qa and temporal_ok(qf, kf, nb, W))
                     for fi, kf in enumerate(topo.global_frames)]
            dense.append(runs)
            specs.append((agent_q_len + qrel * N * KL + g * KL, KL))
    for qrel, qf in enumerate(qframes):
        runs = []
        for g in range(N):
            runs += [(topo.local_base(g, fi), KL,
                      bool(topo.local_active[g][fi]) and temporal_ok(qf, kf, nb, W))
                     for fi, kf in enumerate(topo.local_frames[g])]
        runs += [(topo.global_base(fi), KG, temporal_ok(qf, kf, nb, W))
                 for fi, kf in enumerate(topo.global_frames)]
        dense.append(runs)
        specs.append((agent_q_len + local_q_len + qrel * KG, KG))
    return dense, specs


def tiled_cached_layout(topo: CachedTopology) -> dict:
    dense, specs = tiled_cached_dense(topo)
    return pack_layout(dense, specs)


def tiled_full_sequence_dense(P, T, L, N, KL, KG, n, window, labels, active, direct):
    """Per temporal block: dense runs of ``build_hier_tiled_full_sequence_layouts``.

    Restates hier_tiled_attention.py:260-425 (full-sequence token order: agents
    p-major, locals time-major ``[T,N,KL]``, global ``[T,KG]``).
    """
    if T % n != 0:
        raise ValueError(f"Tiled128 requires T % n == 0, got T={T}, n={n}")
    if window != -1 and window < n:
        raise ValueError(f"Tiled128 requires local_attn_size=-1 or >=n, got {window}, n={n}")
    labels = [[int(x) for x in row] for row in np.asarray(labels)]
    active = [[bool(x) for x in row] for row in np.asarray(active)]
    for s in range(0, T, n):
        if any(labels[t] != labels[s] for t in range(s + 1, min(s + n, T))):
            raise ValueError("Tiled128 requires group labels constant inside each temporal block")
    local_start = P * T * L
    global_start = local_start + T * N * KL
    retention = T if window == -1 else window + n
    abase = lambda p, f: (p * T + f) * L
    lbase = lambda g, f: local_start + (f * N + g) * KL
    gbase = lambda f: global_start + f * KG
    blocks = []
    for b0 in range(0, T, n):
        b1 = b0 + n
        kept = range(max(0, b1 - retention), b1)
        cur = range(b0, b1)
        dense, specs = [], []
        for p in range(P):
            for qf in cur:
                runs = [(abase(p, kf), L, temporal_ok(qf, kf, n, window)) for kf in kept]
                if direct:
                    for o in range(P):
                        if o != p:
                            same = labels[qf][o] == labels[qf][p]
                            runs += [(abase(o, kf), L, same and kf // n == qf // n) for kf in cur]
                for g in range(N):
                    runs += [(lbase(g, kf), KL, g == labels[qf][p] and active[kf][g]
                              and temporal_ok(qf, kf, n, window)) for kf in kept]
                dense.append(runs)
                specs.append((abase(p, qf), L))
        for qf in cur:
            for g in range(N):
                qa = active[qf][g]
                runs = []
                for p in range(P):
                    ok = qa and labels[qf][p] == g
                    runs += [(abase(p, kf), L, ok and temporal_ok(qf, kf, n, window)) for kf in kept]
                runs += [(lbase(g, kf), KL, qa and active[kf][g] and temporal_ok(qf, kf, n, window))
                         for kf in kept]
                runs += [(gbase(kf), KG, qa and temporal_ok(qf, kf, n, window)) for kf in kept]
                dense.append(runs)
                specs.append((lbase(g, qf), KL))
        for qf in cur:
            runs = []
            for g in range(N):
                runs += [(lbase(g, kf), KL, active[kf][g] and temporal_ok(qf, kf, n, window))
                         for kf in kept]
            runs += [(gbase(kf), KG, temporal_ok(qf, kf, n, window)) for kf in kept]
            dense.append(runs)
            specs.append((gbase(qf), KG))
        blocks.append((dense, specs))
    return blocks


def tiled_full_sequence_layouts(P, T, L, N, KL, KG, n, window, labels, active, direct):
    return [pack_layout(d, s) for d, s in
            tiled_full_sequence_dense(P, T, L, N, KL, KG, n, window, labels, active, direct)]


# --------------------------------------------------------------------------
# packed varlen plan
# --------------------------------------------------------------------------

def varlen_plan(kv_index, kv_count, qbase, qlen, seg_ids, query_tokens: int) -> dict:
    """Flattened plan of ``_get_varlen_plan`` (hier_packed_attention.py:50-100)."""
    qb = [int(x) for x in qbase]
    qn = [int(x) for x in qlen]
    si = [int(x) for x in seg_ids]
    nk = [int(x) for x in kv_count]
    if si != list(range(len(si))):
        raise AssertionError("packed metadata must contain exactly one program per segment")
    cover = [r for b, n in zip(qb, qn) for r in range(b, b + n)]
    if cover != list(range(query_tokens)):
        raise AssertionError("packed query segments must partition the query sequence exactly")
    act = [s for s in si if qn[s] > 0 and nk[s] > 0]
    q_index = (np.concatenate([np.arange(qb[s], qb[s] + qn[s]) for s in act])
               if act else np.zeros(0, dtype=np.int64)).astype(np.int64)
    k_index = (np.concatenate([np.asarray(kv_index[s][:nk[s]], dtype=np.int64) for s in act])
               if act else np.zeros(0, dtype=np.int64))
    cu_q = np.cumsum([0] + [qn[s] for s in act]).astype(np.int32)
    cu_k = np.cumsum([0] + [nk[s] for s in act]).astype(np.int32)
    return dict(q_index=q_index, k_index=k_index, cu_q=cu_q, cu_k=cu_k,
                max_q=max((qn[s] for s in act), default=0),
                max_k=max((nk[s] for s in act), default=0),
                min_k_index=int(k_index.min()) if k_index.size else 0,
                max_k_index=int(k_index.max()) if k_index.size else -1)
