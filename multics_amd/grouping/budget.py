"""Communication budget of the label-generation profile.

The cost of a grouping topology is the number of logical mask edges it adds
over one 42-frame latent clip (the membership mask's hub, attachment and
direct player-player edges; same-player history is common to every design and
left out).  The budget is the cost of the centralised single-hub design, so a
grouping may never exceed it (multics/grouping/budget.py:1-344).

Every cost is a sum of integer edge counts, exact in float64, so the
vectorised timeline below returns the same number as an edge-by-edge count.
"""

from __future__ import annotations

import itertools
import math
from collections.abc import Sequence
from dataclasses import dataclass

import numpy as np

TOKENS_PER_PLAYER = 220
LATENT_FRAMES = 42
FRAMES_PER_BLOCK = 3
LOCAL_ATTN_SIZE = 7          # the budget window of the generation protocol, not the model's
LOCAL_HUB_TOKENS = 5
GLOBAL_HUB_TOKENS = 6
DIRECT_FRAC = 1.0
# central hub tokens of the baseline the budget is measured against, per player count
CENTRAL_HUB_TOKENS = {4: 109, 6: 111, 8: 111, 10: 195}


def _window_mask(num_frames: int, frames_per_block: int, local_attn_size: int) -> np.ndarray:
    """``[q, k]``: key frame k is in query frame q's block-causal window."""
    q = np.arange(num_frames)[:, None]
    k = np.arange(num_frames)[None, :]
    ok = (k // frames_per_block) <= (q // frames_per_block)
    if local_attn_size != -1:
        ok = ok & ((q - k) < local_attn_size)
    return ok


def _check_frames(num_frames: int, frames_per_block: int) -> None:
    if num_frames <= 0 or frames_per_block <= 0:
        raise ValueError("num_frames and frames_per_block must be positive integers")


def temporal_window_pairs(num_frames: int, frames_per_block: int, local_attn_size: int) -> int:
    """Directed (query frame, key frame) pairs of the window (budget.py:17-30)."""
    _check_frames(num_frames, frames_per_block)
    if local_attn_size != -1 and local_attn_size < frames_per_block:
        raise ValueError("local_attn_size must be -1 or >= frames_per_block")
    return int(_window_mask(num_frames, frames_per_block, local_attn_size).sum())


def same_block_pairs(num_frames: int, frames_per_block: int) -> int:
    """Directed frame pairs inside one temporal block (budget.py:33-40)."""
    _check_frames(num_frames, frames_per_block)
    sizes = np.minimum(frames_per_block, num_frames - np.arange(0, num_frames, frames_per_block))
    return int((sizes * sizes).sum())


def _max_size_for(pair_budget: int) -> int:
    """Largest p with p (p - 1) <= pair_budget, in integers:
    p (p - 1) <= B  <=>  (2p - 1)^2 <= 4B + 1."""
    return (math.isqrt(4 * max(pair_budget, 0) + 1) + 1) // 2


def _unique_pairs(groups: Sequence[Sequence[int]]) -> set:
    pairs = set()
    for g in groups:
        pairs.update(itertools.combinations(sorted({int(i) for i in g}), 2))
    return pairs


@dataclass(frozen=True)
class Budget:
    """Budget of one (players, group slots) profile; costs cover the whole clip."""

    players: int
    groups: int
    tokens: int = TOKENS_PER_PLAYER
    num_frames: int = LATENT_FRAMES
    frames_per_block: int = FRAMES_PER_BLOCK
    local_attn_size: int = LOCAL_ATTN_SIZE
    local_hub: int = LOCAL_HUB_TOKENS
    global_hub: int = GLOBAL_HUB_TOKENS
    central_hub: int = 0
    direct_frac: float = DIRECT_FRAC

    def __post_init__(self) -> None:
        for name in ("players", "groups", "tokens", "num_frames", "frames_per_block",
                     "local_hub", "global_hub", "central_hub"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive, got {getattr(self, name)!r}")
        temporal_window_pairs(self.num_frames, self.frames_per_block, self.local_attn_size)
        if not 0.0 <= float(self.direct_frac) <= 1.0:
            raise ValueError(f"direct_frac must lie in [0, 1], got {self.direct_frac}")

    # ---- window sizes and the budget ----------------------------------------

    @property
    def a_w(self) -> int:
        """Directed frame pairs of hub / history edges."""
        return temporal_window_pairs(self.num_frames, self.frames_per_block, self.local_attn_size)

    @property
    def b_w(self) -> int:
        """Directed frame pairs of same-block direct player edges."""
        return same_block_pairs(self.num_frames, self.frames_per_block)

    @property
    def c_central(self) -> float:
        h = self.central_hub
        return self.a_w * (2.0 * self.players * self.tokens * h + h ** 2)

    @property
    def c_hier_base(self) -> float:
        """Cost of the hierarchy with every slot active and no direct edge."""
        lh, gh = self.local_hub, self.global_hub
        return self.a_w * (2.0 * self.players * self.tokens * lh + self.groups * lh ** 2
                           + 2.0 * self.groups * lh * gh + gh ** 2)

    @property
    def delta_c(self) -> float:
        return self.c_central - self.c_hier_base

    @property
    def budget_cost(self) -> float:
        """What direct player-player edges may spend: the central design's surplus."""
        return self.delta_c

    @property
    def cost_limit(self) -> float:
        """The total a grouping may cost: the central design's."""
        return self.c_central

    def _pair_units_budget(self) -> int:
        return int(math.floor(self.budget_cost / (self.direct_frac * self.b_w * self.tokens ** 2)))

    @property
    def pair_budget(self) -> int:
        """Directed pair units available to direct edges (one shared pool)."""
        if self.budget_cost <= 0 or self.direct_frac <= 0:
            return 0
        return self._pair_units_budget()

    @property
    def sum_max_size(self) -> int:
        if self.budget_cost <= 0 or self.direct_frac <= 0:
            return 1
        return max(1, min(_max_size_for(self._pair_units_budget()), self.players))

    @property
    def max_size(self) -> int:
        """Largest group the pair budget admits."""
        return self.sum_max_size

    # ---- costs ----------------------------------------------------------------

    @staticmethod
    def direct_pair_units(groups: Sequence[Sequence[int]]) -> int:
        """Directed player-player units; a pair shared by two groups counts once."""
        return 2 * len(_unique_pairs(groups))

    def direct_cost_groups(self, groups: Sequence[Sequence[int]]) -> float:
        return self.direct_frac * self.b_w * self.tokens ** 2 * self.direct_pair_units(groups)

    def hub_cost(self, active_groups: int) -> float:
        """Hub-hub edges.  An active local slot adds lh^2 + 2 lh gh per window
        pair; an inactive one only each hub token's self edge per frame."""
        active = max(0, min(int(active_groups), self.groups))
        inactive = self.groups - active
        lh, gh = self.local_hub, self.global_hub
        return (self.a_w * (active * lh ** 2 + 2.0 * active * lh * gh + gh ** 2)
                + self.num_frames * inactive * lh)

    def topology_cost(self, groups: Sequence[Sequence[int]], n_players: int | None = None) -> float:
        """Cost of holding one topology for the whole clip.  Players in no
        group are global-only; a player in two groups attaches to both."""
        gs = [tuple(sorted({int(i) for i in g})) for g in groups if len(set(g)) >= 2]
        n = self.players if n_players is None else int(n_players)
        covered = {i for g in gs for i in g}
        if any(i < 0 or i >= n for i in covered):
            raise ValueError(f"group member out of range: n_players={n}, groups={groups}")
        attach = self.a_w * (2.0 * self.tokens * self.local_hub * sum(len(g) for g in gs)
                             + 2.0 * self.tokens * self.global_hub * (n - len(covered)))
        return attach + self.hub_cost(len(gs)) + self.direct_cost_groups(gs)

    def topology_cost_timeline(self, membership, global_only) -> float:
        """Edges of a per-frame membership ``[T, N, P]`` / global-only ``[T, P]``
        timeline under the membership mask: player->local edges use query-time
        membership and key-time activity, local->player edges query-time
        membership and activity, global-only edges the query (player rows) or
        key (global rows) time, direct edges same-block pairs sharing a group
        at query time (budget.py:231-314)."""
        mem = np.asarray(membership, dtype=bool)
        go = np.asarray(global_only, dtype=bool)
        T = self.num_frames
        if len(mem) != T or len(go) != T:
            raise ValueError(f"timeline length must equal the budget's T={T}; got "
                             f"membership={len(mem)}, global_only={len(go)}")
        if mem.ndim != 3 or mem.shape[1] != self.groups:
            raise ValueError(f"membership must be [T, {self.groups}, P], got {mem.shape}")
        if go.ndim != 2 or go.shape[1] != mem.shape[2]:
            raise ValueError("global_only must be [T, P] with the membership's P")
        n, lh, gh, tok = self.frames_per_block, self.local_hub, self.global_hub, self.tokens
        win = _window_mask(T, n, self.local_attn_size).astype(np.int64)     # [q, k]
        same = win * (np.arange(T)[:, None] // n == np.arange(T)[None, :] // n)
        act = mem.any(2).astype(np.int64)            # [T, N]
        size = mem.sum(2).astype(np.int64)           # members per slot
        keys = win.sum(1)                            # window keys per query frame
        act_k = win @ act                            # active key frames per (q, slot)
        n_go = go.sum(1).astype(np.int64)
        m = mem.astype(np.int64)
        share = np.einsum("tgi,tgj->tij", m, m) > 0   # pairs sharing a slot at frame t
        pair_units = share.sum((1, 2)) - np.diagonal(share, axis1=1, axis2=2).sum(1)
        ints = (lh * int((1 - act).sum())                        # inactive self edges
                + gh * gh * int(win.sum())
                + lh * lh * int((act * act_k).sum())
                + lh * gh * int((act * keys[:, None]).sum())
                + gh * lh * int(act_k.sum())
                + tok * lh * int((size * act_k).sum())
                + lh * tok * int((size * act * keys[:, None]).sum())
                + tok * gh * int((n_go * keys).sum())
                + gh * tok * int((win @ n_go).sum()))
        direct = 0.0
        if self.direct_frac > 0:
            direct = self.direct_frac * tok ** 2 * int((pair_units * same.sum(1)).sum())
        return float(ints) + direct

    # ---- feasibility --------------------------------------------------------------

    def feasible_groups(self, groups: Sequence[Sequence[int]]) -> bool:
        gs = [tuple(sorted({int(i) for i in g})) for g in groups]
        if len(gs) > self.groups or any(len(g) > self.max_size or len(g) < 2 for g in gs):
            return False
        return self.direct_pair_units(gs) <= self.pair_budget

    def affordable_groups(self, groups: Sequence[Sequence[int]], n_players: int | None = None) -> bool:
        return (self.feasible_groups(groups)
                and self.topology_cost(groups, n_players=n_players) <= self.cost_limit)


def resolve(players: int) -> Budget:
    """The profile of a supported player count; slots = ceil(log2(P))."""
    if type(players) is not int or players not in CENTRAL_HUB_TOKENS:
        raise ValueError(f"Automatic grouping supports 4/6/8/10 players, got {players}")
    return Budget(players=players, groups=(players - 1).bit_length(),
                  central_hub=CENTRAL_HUB_TOKENS[players])
