"""Bounded clique cover of the relevance graph: local groups of one period.

1. Candidates: every maximal clique of the thresholded graph up to the size
   cap (at most 32 kept, by mass, while every covered player keeps one), then
   every thresholded edge as a pair.
2. A beam search (width 300) over sets of at most N candidates that satisfy
   the structural and budget constraints, each step adding a candidate later
   in the pool that brings a new direct pair; the best state by (players
   covered, pair mass minus 0.15 per extra membership, pair mass, fewer extra
   memberships, lower cost) wins.
3. Idle slots are filled with the uncovered players, ranked by their raw
   pair relevance (no score floor), re-using a covered player as an anchor
   when only one is left.
(multics/grouping/partition.py:1-386.)

Enumeration orders, sort keys and the order in which pair scores are summed
are those of the reference: equal-score ties (common in symmetric scenes) are
resolved by them, and the labels must come out identical.
"""

from __future__ import annotations

import itertools
from collections.abc import Sequence
from dataclasses import dataclass, field

import numpy as np

from .budget import Budget
from .relevance import threshold_graph

MAX_MEMBERSHIPS = 2
MAX_PAIRWISE_GROUP_OVERLAP = 1
OVERLAP_PENALTY = 0.15
BEAM_SIZE = 300
MAX_MAXIMAL_CLIQUES = 32
THRESHOLD = 0.30


def pairs_of(groups: Sequence[Sequence[int]]) -> set:
    """Direct (undirected) player pairs of a topology."""
    return {pair for g in groups for pair in itertools.combinations(sorted(g), 2)}


@dataclass
class FlexGrouping:
    """Local groups (indices into the period's players) and the global-only rest."""

    groups: list = field(default_factory=list)
    global_only: list = field(default_factory=list)
    scores: list = field(default_factory=list)

    @property
    def pair_used(self) -> int:
        return 2 * len(pairs_of(self.groups))

    @property
    def shared(self) -> list:
        """Anchors: players in more than one group."""
        seen, twice = set(), set()
        for g in self.groups:
            for p in g:
                (twice if p in seen else seen).add(p)
        return sorted(twice)


def _pair_sum(scores: np.ndarray, pairs) -> float:
    total = 0
    for i, j in pairs:
        total = total + scores[i, j]
    return float(total)


def group_mass(scores: np.ndarray, group: Sequence[int]) -> float:
    return _pair_sum(scores, itertools.combinations(sorted(group), 2))


def group_score(scores: np.ndarray, group: Sequence[int]) -> float:
    return group_mass(scores, group) / len(group) if len(group) >= 2 else 0.0


def cohesion(scores: np.ndarray, group: Sequence[int]) -> float:
    pairs = list(itertools.combinations(sorted(group), 2))
    return float(_pair_sum(scores, pairs) / len(pairs)) if pairs else 0.0


def _is_clique(graph: np.ndarray, members) -> bool:
    return all(graph[i, j] > 0 for i, j in itertools.combinations(members, 2))


def clique_candidates(graph: np.ndarray, max_size: int,
                      max_maximal: int = MAX_MAXIMAL_CLIQUES) -> list:
    """Maximal cliques of at most ``max_size`` players (a clique of exactly
    ``max_size`` counts as maximal), then every edge of the graph."""
    n = len(graph)
    maximal, edges = [], []
    for size in range(2, min(max_size, n) + 1):
        for group in itertools.combinations(range(n), size):
            if not _is_clique(graph, group):
                continue
            if size == 2:
                edges.append(group)
            grows = size < max_size and any(
                p not in group and all(graph[p, m] > 0 for m in group) for p in range(n))
            if not grows:
                maximal.append(group)
    if len(maximal) > max_maximal:
        ranked = sorted(maximal, reverse=True,
                        key=lambda g: (group_mass(graph, g), len(g), tuple(-x for x in g)))
        kept = ranked[:max_maximal]
        for p in range(n):
            if any(p in g for g in maximal) and not any(p in g for g in kept):
                kept.append(next(g for g in ranked if p in g))
        maximal = kept
    out = []
    for g in maximal + edges:
        g = list(g)
        if g not in out:
            out.append(g)
    return out


def _membership_counts(groups: Sequence[Sequence[int]], n: int) -> tuple:
    return tuple(sum(p in g for g in groups) for p in range(n))


def topology_constraints_hold(groups: Sequence[Sequence[int]], *, player_count: int,
                              max_groups: int, max_size: int, pair_budget: int,
                              max_memberships: int = MAX_MEMBERSHIPS,
                              max_pairwise_overlap: int = MAX_PAIRWISE_GROUP_OVERLAP,
                              budget: Budget | None = None) -> bool:
    """At most N groups of 2..K players, a player in at most two groups, two
    groups sharing at most one player, the pair budget, and (with a budget)
    the clip cost under the central design's."""
    if len(groups) > max_groups or any(not 2 <= len(g) <= max_size for g in groups):
        return False
    if max(_membership_counts(groups, player_count), default=0) > max_memberships:
        return False
    if any(len(set(a) & set(b)) > max_pairwise_overlap for a, b in itertools.combinations(groups, 2)):
        return False
    if 2 * len(pairs_of(groups)) > pair_budget:
        return False
    return budget is None or budget.affordable_groups(groups, n_players=player_count)


def _selection_key(scores, groups, *, budget, player_count) -> tuple:
    edges = pairs_of(groups)
    covered = {p for g in groups for p in g}
    mass = _pair_sum(scores, edges)
    extra = sum(len(g) for g in groups) - len(covered)
    cost = (budget.topology_cost(groups, n_players=player_count) if budget is not None
            else 2 * len(edges))
    return (len(covered), mass - OVERLAP_PENALTY * extra, mass, -extra, -cost)


def select_semantic_groups(graph: np.ndarray, candidates, *, max_groups: int, max_size: int,
                           pair_budget: int, budget: Budget | None,
                           beam_size: int = BEAM_SIZE) -> list:
    """Best feasible set of candidates (see the module docstring, step 2)."""
    n = len(graph)
    pool = sorted((sorted(g) for g in candidates), reverse=True,
                  key=lambda g: (len(g), group_mass(graph, g), tuple(-x for x in g)))
    pool_pairs = [pairs_of([g]) for g in pool]
    key = lambda state: _selection_key(graph, state[1], budget=budget, player_count=n)
    beam = [((), [], frozenset())]
    feasible = []
    for _ in range(max_groups):
        grown = []
        for chosen, groups, edges in beam:
            for idx in range(chosen[-1] + 1 if chosen else 0, len(pool)):
                if pool_pairs[idx] <= edges:
                    continue   # a hub that opens no new direct pair is wasted
                trial = groups + [pool[idx]]
                if topology_constraints_hold(trial, player_count=n, max_groups=max_groups,
                                             max_size=max_size, pair_budget=pair_budget,
                                             budget=budget):
                    grown.append((chosen + (idx,), trial, edges | pool_pairs[idx]))
        if not grown:
            break
        grown.sort(key=key, reverse=True)
        beam = grown[:beam_size]
        feasible.extend(beam)
    return max(feasible, key=key)[1] if feasible else []


def recover_new_style(scores: np.ndarray, groups, *, max_groups: int, max_size: int,
                      pair_budget: int, budget: Budget | None):
    """Fill idle slots with uncovered players (module docstring, step 3);
    returns (all groups, the groups added)."""
    result = [sorted(g) for g in groups]
    added = []
    n = len(scores)
    if max_size < 2:
        return result, added
    while len(result) < max_groups:
        counts = _membership_counts(result, n)
        loose = [p for p, c in enumerate(counts) if c == 0]
        if not loose:
            break
        take = min(max_size, max(1, -(-len(loose) // (max_groups - len(result)))), len(loose))
        cands = []
        for subset in itertools.combinations(loose, take):
            if take == 1:
                anchors = [p for p, c in enumerate(counts) if 0 < c < MAX_MEMBERSHIPS]
                cands.extend(sorted([subset[0], a]) for a in anchors)
            else:
                cands.append(sorted(subset))

        def rank(g):
            e = [float(scores[a, b]) for a, b in itertools.combinations(g, 2)]
            return (sum(e), min(e) if e else 0.0, tuple(-p for p in g))

        cands.sort(key=rank, reverse=True)
        pick = next((c for c in cands if topology_constraints_hold(
            result + [c], player_count=n, max_groups=max_groups, max_size=max_size,
            pair_budget=pair_budget, budget=budget)), None)
        if pick is None:
            break
        result.append(pick)
        added.append(pick)
    return result, added


def flexible_partition(scores: np.ndarray, *, budget: Budget) -> FlexGrouping:
    """Groups of one period from its smoothed ``[P, P]`` relevance."""
    n = len(scores)
    if scores.shape != (n, n):
        raise ValueError(f"scores must be square, got {scores.shape}")
    if budget.max_size < 2 or budget.pair_budget < 2:
        return FlexGrouping(global_only=list(range(n)))
    limits = dict(max_groups=budget.groups, max_size=budget.max_size,
                  pair_budget=budget.pair_budget, budget=budget)
    graph = threshold_graph(scores, THRESHOLD)
    semantic = select_semantic_groups(graph, clique_candidates(graph, budget.max_size), **limits)
    groups, added = recover_new_style(scores, semantic, **limits)
    covered = {p for g in groups for p in g}
    result = FlexGrouping(groups=groups, global_only=sorted(set(range(n)) - covered),
                          scores=[(-1.0 if g in added else 1.0) * group_score(scores, g)
                                  for g in groups])
    if not topology_constraints_hold(result.groups, player_count=n, **limits):
        raise RuntimeError(f"Internal error: infeasible grouping {result.groups}")
    return result
