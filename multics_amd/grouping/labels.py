"""Per-period groups -> the 24-tensor label payload (``groups.pt``).

Group slots are matched across periods by member overlap, so a slot follows
its players rather than its position in the list; period tensors are then
mapped to the clip's latent frames (every 4th RGB frame) by the period that
contains each latent frame's first RGB frame (multics/grouping/labels.py:1-212).
The payload's fields, shapes and dtypes are the schema the data loader and the
mask builder read (labels.py:127-152).
"""

from __future__ import annotations

import numpy as np

from .budget import resolve
from .partition import cohesion, flexible_partition
from .relevance import relevance_periods, threshold_graph
from .state import GroupingState, eligible_players

LATENT_STRIDE = 4
CLIP_FRAMES = 165
THRESHOLD = 0.3


def latent_frame_count(num_frames: int, stride: int = LATENT_STRIDE) -> int:
    return (num_frames - 1) // stride + 1


def track_labels(seq, n_slots: int) -> list:
    """Slot of every group of every period.  Pairs (new group, previous slot)
    are taken greedily by larger intersection, then larger Jaccard index, then
    lower group and slot index; unmatched groups take the lowest free slot
    (or their index modulo the slot count when none is free)."""
    out, prev = [], []          # prev: (slot, member set) of the last period
    for groups in seq:
        sets = [set(g) for g in groups]
        ranked = sorted((-len(s & ps), -len(s & ps) / len(s | ps), gi, slot)
                        for gi, s in enumerate(sets) for slot, ps in prev if s & ps)
        slot_of = [-1] * len(groups)
        taken = set()
        for _, _, gi, slot in ranked:
            if slot_of[gi] < 0 and slot not in taken:
                slot_of[gi] = slot
                taken.add(slot)
        free = [s for s in range(n_slots) if s not in taken]
        for gi in range(len(groups)):
            if slot_of[gi] < 0:
                slot_of[gi] = free.pop(0) if free else gi % n_slots
                taken.add(slot_of[gi])
        out.append(slot_of)
        prev = list(zip(slot_of, sets))
    return out


def flex_label_arrays(groupings, periods, keep, *, n_players: int, max_groups: int,
                      start_frame: int, num_frames: int, threshold: float, budget,
                      stride: int = LATENT_STRIDE) -> dict:
    """The 24 arrays from per-period groupings (indices into ``keep``)."""
    P, G, K = n_players, max_groups, len(groupings)
    if K == 0:
        raise ValueError("no grouping period: nothing to label")
    keep = np.asarray(keep, int)
    slots = track_labels([g.groups for g in groupings], n_slots=max(G, 1))
    mem = np.zeros((K, G, P), bool)
    go = np.zeros((K, P), bool)
    anchor = np.zeros((K, P), bool)
    score = np.full((K, G), -1.0, np.float32)
    size = np.zeros((K, G), np.int8)
    coh = np.full((K, G), -1.0, np.float32)
    for k, (gr, per, sl) in enumerate(zip(groupings, periods, slots)):
        graph = threshold_graph(per.smooth, threshold)
        for gi, g in enumerate(gr.groups):
            s = int(sl[gi]) % G
            size[k, s] = len(g)
            score[k, s] = gr.scores[gi] if gi < len(gr.scores) else 0.0
            coh[k, s] = cohesion(graph, g) if len(g) > 1 else 0.0
            mem[k, s, keep[list(g)]] = True
        go[k, keep[list(gr.global_only)]] = True
        anchor[k, keep[list(gr.shared)]] = True
    p_start = np.array([int(p.start_frame - start_frame) for p in periods], np.int32)
    p_frames = np.array([int(p.num_frames) for p in periods], np.int32)
    p_pair = np.array([gr.pair_used for gr in groupings], np.int32)
    # cost of each period's topology over the eligible players only: a player
    # outside ``keep`` is neither a member nor global-only
    p_cost = np.array([budget.topology_cost(gr.groups, n_players=len(keep)) for gr in groupings],
                      np.float32)
    has = mem.any(axis=1)
    p_lab = np.where(has, mem.argmax(axis=1), -1).astype(np.int8)

    first_rgb = np.minimum(np.arange(latent_frame_count(num_frames, stride)) * stride,
                           max(num_frames - 1, 0))
    period = np.clip(np.searchsorted(p_start, first_rgb, side="right") - 1, 0, K - 1)
    membership, global_only = mem[period], go[period]
    clip_cost = budget.topology_cost_timeline(membership, global_only)
    if clip_cost > budget.cost_limit:
        raise RuntimeError(f"dynamic membership over the communication budget: "
                           f"{clip_cost:,.0f} > {budget.cost_limit:,.0f}")
    eligible = np.zeros(P, bool)
    eligible[keep] = True
    denom = np.float32(max(P, 1))
    return {
        "membership": membership,
        "global_only": global_only,
        "eligible": eligible,
        "labels": p_lab[period],
        "latent_period": period.astype(np.int16),
        "period_membership": mem,
        "period_global_only": go,
        "period_anchor": anchor,
        "period_labels": p_lab,
        "period_start": p_start,
        "period_frames": p_frames,
        "period_scores": score,
        "period_sizes": size,
        "period_cohesion": coh,
        "period_pair_used": p_pair,
        "period_total_cost": p_cost,
        "clip_total_cost": np.array(clip_cost, dtype=np.float64),
        "cost_limit": np.array(budget.cost_limit, dtype=np.float64),
        "coverage": has.sum(axis=1).astype(np.float32) / denom,
        "orphan_ratio": go.sum(axis=1).astype(np.float32) / denom,
        "anchor_ratio": anchor.sum(axis=1).astype(np.float32) / denom,
        "pair_budget": np.array(budget.pair_budget, dtype=np.int32),
        "max_groups": np.array(G, dtype=np.int32),
        "max_size": np.array(budget.max_size, dtype=np.int32),
    }


def generate_labels(state: GroupingState) -> dict:
    """Labels of one 165-frame clip from its poses alone (deterministic, no
    random draws; labels.py:182-212)."""
    state.validate()
    if state.clip_num_frames != CLIP_FRAMES:
        raise ValueError("Automatic grouping currently requires 165 RGB frames per CSV row")
    budget = resolve(state.num_players)
    span = state.frame_window(state.clip_start_frame, state.clip_num_frames)
    keep = np.flatnonzero(eligible_players(state, span))
    if len(keep) < 2:
        raise ValueError("Fewer than two eligible players in grouping clip")
    periods = relevance_periods(state, span, state.clip_start_frame, keep)
    groupings = [flexible_partition(p.smooth, budget=budget) for p in periods]
    return flex_label_arrays(groupings, periods, keep, n_players=state.num_players,
                             max_groups=budget.groups, start_frame=state.clip_start_frame,
                             num_frames=state.clip_num_frames, threshold=THRESHOLD, budget=budget)


def membership_inputs(payload) -> tuple:
    """``(membership [T, N, P], global_only [T, P])`` bool numpy arrays of a
    label payload (the 24-field schema or its core fields), ready for
    ``metadata.full_sequence_topology`` / ``hier_masks`` builders."""
    mem = np.asarray(payload["membership"], dtype=bool)
    go = np.asarray(payload["global_only"], dtype=bool)
    if mem.ndim != 3 or go.shape != (mem.shape[0], mem.shape[2]):
        raise ValueError(f"membership [T,N,P] / global_only [T,P] expected, got "
                         f"{mem.shape} / {go.shape}")
    return mem, go
