"""Membership producer (multics_amd.grouping) against the reference's golden
labels and the properties its own tests fix (tests/test_dynamic_grouping.py).

* All 24 label fields, exactly (values and dtypes), for the five bundled
  4-player clips and the P4 / P6 / P10 synthetic fixtures
  (``tests/golden/grouping``, collected by ``make_grouping_golden.py``).
* The budget profiles of every supported player count.
* The clip cost of a membership timeline against an edge count of the dense
  membership mask (``oracle.masks``) on small profiles: every mask edge but a
  player's own history is one unit of cost.
* Causality of the relevance (poses after a period's first frame do not
  change it), the pose-only interaction validity gate, eligibility, slot
  tracking, and the refusals of the state and payload validators.
"""

from dataclasses import replace
from pathlib import Path

import numpy as np
import pytest
import torch

from multics_amd.grouping import (Budget, GroupingState, eligible_players, generate_labels,
                                  history_components, load_group_labels, membership_inputs,
                                  relevance_periods, resolve, save_group_labels, track_labels,
                                  validate_existing_labels, validate_generated_labels)
from oracle.masks import FullTopology, mask_rows

GOLD = Path(__file__).parent / "golden" / "grouping"
CASES = sorted(p.name[: -len(".state.npz")] for p in GOLD.glob("*.state.npz"))


def _expected(name):
    with np.load(GOLD / f"{name}.labels.npz", allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


@pytest.fixture(scope="module")
def example():
    state = GroupingState.load(GOLD / "example_4_01.state.npz")
    return state, generate_labels(state)


def test_golden_cases_present():
    assert len(CASES) == 8
    assert {"p4_round_start", "p6_moving_pairs", "p10_moving_pairs"} <= set(CASES)


@pytest.mark.parametrize("name", CASES)
def test_labels_all_24_fields_exact(name):
    state = GroupingState.load(GOLD / f"{name}.state.npz")
    got = generate_labels(state)
    want = _expected(name)
    assert set(got) == set(want) and len(got) == 24
    for key in want:
        assert got[key].dtype == want[key].dtype, key
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)
    validate_generated_labels({k: torch.from_numpy(v) for k, v in got.items()}, state.num_players)
    if "moving" in name:   # the groups change between periods
        pm = got["period_membership"]
        assert any(not np.array_equal(pm[0], f) for f in pm[1:])


@pytest.mark.parametrize("players,groups,pairs,size",
                         [(4, 2, 10, 3), (6, 3, 15, 4), (8, 3, 19, 4), (10, 4, 45, 7)])
def test_budget_profiles(players, groups, pairs, size):
    b = resolve(players)
    assert (b.groups, b.pair_budget, b.max_size) == (groups, pairs, size)
    assert (b.local_attn_size, b.a_w, b.b_w) == (7, 315, 126)
    assert b.cost_limit == b.a_w * (2.0 * players * 220 * b.central_hub + b.central_hub ** 2)


def test_budget_refuses_other_player_counts():
    with pytest.raises(ValueError, match="4/6/8/10"):
        resolve(5)


def _random_timeline(rng, T, N, P, n):
    """Per-block membership (a player in at most one slot, some in none)."""
    mem = np.zeros((T, N, P), bool)
    for b0 in range(0, T, n):
        slot = rng.integers(-1, N, size=P)
        for p in range(P):
            if slot[p] >= 0:
                mem[b0:b0 + n, slot[p], p] = True
    return mem, ~mem.any(1)


@pytest.mark.parametrize("seed,window", [(0, 4), (1, 6), (2, -1)])
def test_timeline_cost_counts_mask_edges(seed, window):
    rng = np.random.default_rng(seed)
    P, T, L, N, KL, KG, n = 4, 6, 3, 2, 2, 2, 3
    mem, go = _random_timeline(rng, T, N, P, n)
    b = Budget(players=P, groups=N, tokens=L, num_frames=T, frames_per_block=n,
               local_attn_size=window, local_hub=KL, global_hub=KG, central_hub=7)
    topo = FullTopology(P, T, L, N, KL, KG, n, window, True, membership=mem, global_only=go)
    m = mask_rows(topo)
    own = P * L * L * b.a_w     # a player's own history is not part of the cost
    assert b.topology_cost_timeline(mem, go) == float(m.sum() - own)


def test_constant_topology_cost_equals_its_timeline():
    b = resolve(6)
    groups = [[0, 1, 2], [2, 3], [4, 5]]
    mem = np.zeros((b.num_frames, b.groups, 6), bool)
    for g, members in enumerate(groups):
        mem[:, g, members] = True
    go = ~mem.any(1)
    assert b.topology_cost(groups) == b.topology_cost_timeline(mem, go)


def test_track_labels_follow_members_not_positions():
    assert track_labels([[[0, 1], [2, 3]], [[2, 3], [0, 1]]], 2) == [[0, 1], [1, 0]]


def test_eligibility_ignores_empty_ticks_but_not_a_missing_player(example):
    state, _ = example
    state = replace(state, present=np.ones_like(state.present))
    span = state.frame_window(state.clip_start_frame, 165)
    state.present[span.start] = False
    assert eligible_players(state, span).all()
    state.present[span.start + 1, 0] = False
    assert not eligible_players(state, span)[0]


def test_future_pose_does_not_change_current_period(example):
    state, _ = example
    other = replace(state, pos=state.pos.copy())
    t = state.clip_start_frame
    cut = np.searchsorted(state.ticks, state.frame_to_tick(t))
    other.pos[cut + 1:, 0, 0] += 10000
    span = state.frame_window(t, 165)
    left = relevance_periods(state, span, t, np.arange(4))[0]
    right = relevance_periods(other, span, t, np.arange(4))[0]
    np.testing.assert_array_equal(left.smooth, right.smooth)
    other.pos[cut, 0, 0] += 10000
    moved = relevance_periods(other, span, t, np.arange(4))[0]
    assert not np.array_equal(left.smooth, moved.smooth)


def test_interaction_validity_gate_survives_pose_only(example):
    state, _ = example
    s = replace(state, pos=np.zeros_like(state.pos), yaw=np.zeros_like(state.yaw),
                pitch=np.zeros_like(state.pitch), alive=np.ones_like(state.alive),
                present=np.ones_like(state.present))
    s.pos[:, 1, 0] = 1300       # beyond the mutual gate, inside the action gate
    s.yaw[:, 1] = 180
    parts = history_components(s, s.clip_start_frame - 12, 13)
    assert parts["mutual"][0, 1] == 0
    assert parts["interaction_valid"][0, 1] == 1


def test_state_validation_refusals_and_round_trip(example, tmp_path):
    state, _ = example
    short = replace(state, **{k: getattr(state, k)[2:]
                              for k in ("ticks", "pos", "yaw", "pitch", "alive", "present")})
    with pytest.raises(ValueError, match="history"):
        short.validate()
    with pytest.raises(ValueError, match="yaw"):
        replace(state, yaw=state.yaw.astype(np.float64)).validate()
    state.save(tmp_path / "s.npz")
    back = GroupingState.load(tmp_path / "s.npz")
    for k in ("ticks", "pos", "yaw", "pitch", "alive", "present", "player_slots"):
        np.testing.assert_array_equal(getattr(back, k), getattr(state, k))
    assert (back.map_name, back.clip_start_frame) == (state.map_name, state.clip_start_frame)


def test_payload_refusals(example, tmp_path):
    _, got = example
    base = {k: torch.from_numpy(v.copy()) for k, v in got.items()}
    validate_existing_labels(base)
    bad = {k: v.clone() for k, v in base.items()}
    bad["period_pair_used"][0] += 2
    with pytest.raises(ValueError, match="pair accounting"):
        validate_generated_labels(bad, 4)
    bad = {k: v.clone() for k, v in base.items()}
    bad["labels"][0, 0] = 1 - bad["labels"][0, 0] if bad["labels"][0, 0] >= 0 else 1
    with pytest.raises(ValueError, match="disagree"):
        validate_existing_labels(bad)
    bad = {k: v.clone() for k, v in base.items()}
    del bad["period_membership"], bad["clip_total_cost"]
    with pytest.raises(ValueError, match="all 24 fields"):
        validate_existing_labels(bad)
    other = {"membership": torch.ones(42, 3, 5, dtype=torch.bool),
             "global_only": torch.zeros(42, 5, dtype=torch.bool),
             "eligible": torch.ones(5, dtype=torch.bool)}
    other["membership"][:, 1:] = False
    validate_existing_labels(other)     # other player counts stay readable


def test_label_file_round_trip_and_topology_inputs(example, tmp_path):
    _, got = example
    path = save_group_labels(got, tmp_path / "groups.pt", num_players=4)
    back = load_group_labels(path)
    assert set(back) == set(got)
    for k, v in got.items():
        assert torch.equal(back[k], torch.from_numpy(v)), k
    assert not list(tmp_path.glob("*.tmp"))
    mem, go = membership_inputs(back)
    assert mem.shape == (42, 2, 4) and go.shape == (42, 4)
    # what the mask builders read: every player is a member or global-only
    assert ((mem.any(1) ^ go) | ~got["eligible"][None]).all()


def test_eight_player_labels_satisfy_the_generated_schema(example):
    """No golden labels exist at P8: a state of two copies of the bundled
    4-player clip (the copy moved 3000 units away, so the halves never see
    each other) must give labels that pass every generated-schema check, with
    each semantic group (positive score) inside one half; groups made by the
    idle-slot recovery (negative score) have no score floor and may span."""
    state, four = example
    pos = np.concatenate([state.pos, state.pos + np.float32(3000.0)], axis=1)
    eight = replace(state, pos=pos, yaw=np.concatenate([state.yaw] * 2, axis=1),
                    pitch=np.concatenate([state.pitch] * 2, axis=1),
                    alive=np.concatenate([state.alive] * 2, axis=1),
                    present=np.concatenate([state.present] * 2, axis=1),
                    player_slots=np.arange(8, dtype=np.int64))
    got = generate_labels(eight)
    validate_generated_labels({k: torch.from_numpy(v) for k, v in got.items()}, 8)
    assert got["period_membership"].shape == (4, 3, 8)
    for frame, scores in zip(got["period_membership"], got["period_scores"]):
        for slot, score in zip(frame, scores):
            members = np.nonzero(slot)[0]
            if score > 0:
                assert (members < 4).all() or (members >= 4).all()
    # each half alone is the 4-player clip: its best semantic group scores the same
    np.testing.assert_array_equal(got["period_scores"].max(1), four["period_scores"].max(1))
