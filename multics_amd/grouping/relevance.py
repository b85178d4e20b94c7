"""Pose-only pair relevance with fast / slow history and EMA hysteresis.

For every 48-frame grouping period the relevance of two players is read from
their poses up to and including the period's first frame (never later): a
*scene* term (eye proximity and agreement of the points 1200 units along the
view rays) and an *interaction* term (each player inside the other's view
frustum, weighted by centring and apparent size, gated by distance), each a
recency-weighted mean over the history frames (multics/grouping/relevance.py).

The float operations follow the reference's order and dtypes (view vectors in
float32 from the float32 angles, positions lifted to float64 after the eye
offset): the generated labels must equal the reference's bit for bit,
including the scores, and the symmetric test trajectories produce exact ties
whose resolution depends on the last bit.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .state import GroupingState, TICKS_PER_FRAME, update_slices

HALF_LIFE = 4.0
DEFAULT_ALPHA = 0.6
VFOV = 73.74
REFERENCE_DEPTH = 900.0
MUTUAL_FULL_DISTANCE = 900.0
MUTUAL_ZERO_DISTANCE = 1200.0
ACTION_FULL_DISTANCE = 1000.0
ACTION_ZERO_DISTANCE = 1400.0
FAST_HISTORY_FRAMES = 12
SLOW_HISTORY_FRAMES = 48
UPDATE_FRAMES = 48
FAST_HALF_LIFE = 4.0
SLOW_HALF_LIFE = 12.0
FAST_SCENE_WEIGHT = 0.75
SLOW_SCENE_WEIGHT = 0.25

_COMPONENTS = ("prox", "aim", "scene", "mutual", "interaction", "raw", "co_alive",
               "interaction_valid")


def view_dirs(yaw: np.ndarray, pitch: np.ndarray) -> np.ndarray:
    """Unit view vectors ``[..., 3]`` from yaw / pitch in degrees (positive
    pitch looks down)."""
    y, p = np.radians(yaw), np.radians(pitch)
    cp = np.cos(p)
    return np.stack([cp * np.cos(y), cp * np.sin(y), -np.sin(p)], -1)


@dataclass
class Period:
    """Relevance of one grouping period and what it was made of."""

    start_frame: int
    num_frames: int
    span: slice
    raw: np.ndarray
    smooth: np.ndarray
    co_alive: np.ndarray
    stride: int = 1
    parts: dict = field(default_factory=dict)


def recent_weights(n: int, half_life: float = HALF_LIFE) -> np.ndarray:
    """Normalised weights halving every ``half_life`` frames into the past."""
    if n <= 0:
        return np.zeros(0, np.float64)
    if half_life <= 0:
        raise ValueError(f"half_life must be positive, got {half_life}")
    w = 2.0 ** ((np.arange(n, dtype=np.float64) - (n - 1)) / half_life)
    return w / w.sum()


def cosine_distance_gate(distance, full: float, zero: float) -> np.ndarray:
    """1 up to ``full``, a half-cosine down to exactly 0 at ``zero`` and beyond."""
    if not 0 <= full < zero:
        raise ValueError(f"distance gate requires 0 <= full < zero, got {full}, {zero}")
    x = np.clip((np.asarray(distance, dtype=np.float64) - full) / (zero - full), 0.0, 1.0)
    return 0.5 * (1.0 + np.cos(np.pi * x))


def _pairwise(x: np.ndarray) -> np.ndarray:
    """``[t, i, j, :] = x[t, j] - x[t, i]``."""
    return x[:, None, :, :] - x[:, :, None, :]


def camera_quality(eye, dirs, active, *, vfov: float = VFOV,
                   reference_depth: float = REFERENCE_DEPTH) -> np.ndarray:
    """``[t, observer, target]``: how well the target sits in the observer's
    16:9 frustum (centring times apparent size; 0 outside, behind or for an
    inactive player; a pose-only candidate, no line of sight)."""
    right = np.cross(dirs, np.array([0.0, 0.0, 1.0]))
    right /= np.maximum(np.linalg.norm(right, axis=-1, keepdims=True), 1e-9)
    up = np.cross(right, dirs)
    rel = _pairwise(eye)
    depth = np.einsum("tijc,tic->tij", rel, dirs)
    side = np.einsum("tijc,tic->tij", rel, right)
    vert = np.einsum("tijc,tic->tij", rel, up)
    safe = np.maximum(depth, 1.0)
    tan_v = np.tan(np.radians(vfov / 2.0))
    tan_h = tan_v * 16.0 / 9.0
    nx = side / (safe * tan_h)
    ny = vert / (safe * tan_v)
    inside = ((depth > 1.0) & (np.abs(nx) <= 1.0) & (np.abs(ny) <= 1.0)
              & active[:, :, None] & active[:, None, :])
    centre = np.clip(1.0 - np.hypot(nx, ny) / np.sqrt(2.0), 0.0, 1.0)
    size = np.clip(reference_depth / safe, 0.0, 1.0)
    q = np.where(inside, centre * size, 0.0)
    d = np.arange(q.shape[1])
    q[:, d, d] = 0.0
    return q


def frame_rows(world: GroupingState, start_frame: int, num_frames: int) -> np.ndarray:
    """Tick row of each frame (the first record at or after its tick)."""
    ticks = [world.frame_to_tick(f) for f in range(start_frame, start_frame + num_frames)]
    rows = np.searchsorted(world.ticks, np.asarray(ticks, dtype=world.ticks.dtype))
    return np.minimum(rows, len(world.ticks) - 1).astype(np.int64)


def history_components(world: GroupingState, start_frame: int, num_frames: int, *,
                       prox_len: float = 700.0, aim_range: float = 1200.0, aim_len: float = 900.0,
                       mutual_full_distance: float = MUTUAL_FULL_DISTANCE,
                       mutual_zero_distance: float = MUTUAL_ZERO_DISTANCE,
                       action_full_distance: float = ACTION_FULL_DISTANCE,
                       action_zero_distance: float = ACTION_ZERO_DISTANCE,
                       half_life: float = HALF_LIFE) -> dict:
    """``[P, P]`` relevance components over frames [start, start + num_frames)
    (relevance.py:121-220).  Diagonals are 0; ``raw`` is symmetrised."""
    P = world.num_players
    if num_frames <= 0 or len(world.ticks) == 0:
        return {name: np.zeros((P, P), np.float64) for name in _COMPONENTS}
    if prox_len <= 0 or aim_len <= 0 or aim_range <= 0:
        raise ValueError("prox_len, aim_range and aim_len must be positive")
    rows = frame_rows(world, start_frame, num_frames)
    eye = world.eye_pos()[rows].astype(np.float64)
    active = world.alive[rows] & world.present[rows]
    both = active[:, :, None] & active[:, None, :]
    dirs = view_dirs(world.yaw[rows], world.pitch[rows])
    weights = recent_weights(len(rows), half_life=half_life)

    def recent(frames):
        return np.tensordot(weights, frames, axes=(0, 0))

    distance = np.linalg.norm(_pairwise(eye), axis=-1)
    prox = recent(np.where(both, np.exp(-distance / prox_len), 0.0))
    aim_end = eye + aim_range * dirs
    aim = recent(np.where(both, np.exp(-np.linalg.norm(_pairwise(aim_end), axis=-1) / aim_len), 0.0))
    scene = np.sqrt(np.clip(prox, 0.0, 1.0) * np.clip(aim, 0.0, 1.0))

    quality = camera_quality(eye, dirs, active)
    mutual_gate = cosine_distance_gate(distance, mutual_full_distance, mutual_zero_distance) * both
    action_gate = cosine_distance_gate(distance, action_full_distance, action_zero_distance) * both
    mutual = recent(np.sqrt(quality * quality.transpose(0, 2, 1)) * mutual_gate)
    # pose-only: no firing term, so the interaction is the mutual view term,
    # but its validity still uses the wider action gate
    valid = recent(np.maximum(mutual_gate, action_gate)) > 1e-8
    raw = np.maximum(scene, mutual)
    out = {"prox": prox, "aim": aim, "scene": scene, "mutual": mutual, "interaction": mutual,
           "raw": raw, "co_alive": both.mean(axis=0), "interaction_valid": valid.astype(np.float64)}
    for value in out.values():
        np.fill_diagonal(value, 0.0)
    out["raw"] = np.clip((raw + raw.T) / 2.0, 0.0, 1.0)
    return out


def threshold_graph(scores: np.ndarray, threshold: float) -> np.ndarray:
    """Pair scores below ``threshold`` dropped, symmetric, zero diagonal."""
    graph = np.where(scores >= threshold, scores, 0.0)
    graph = np.maximum(graph, graph.T)
    np.fill_diagonal(graph, 0.0)
    return graph


def _symmetric(x: np.ndarray) -> np.ndarray:
    return np.clip((x + x.T) / 2.0, 0.0, 1.0)


def relevance_periods(world: GroupingState, span: slice, start_frame: int,
                      keep: np.ndarray) -> list:
    """One ``Period`` per 48-frame interval of ``span``, over the players in
    ``keep`` (relevance.py:233-326).  Each period reads the fast window
    [t-12, t] and the slow window [t-48, t] of its first frame t.  The scene
    and interaction terms are smoothed separately (alpha 0.6) once an earlier
    period had any co-alive pair; the interaction only carries over where the
    current fast window's distance gate is open; pairs never co-alive in the
    fast window score 0."""
    alpha = DEFAULT_ALPHA
    sub = np.ix_(keep, keep)
    periods = []
    prev_scene = prev_inter = None
    prev_informative = False
    for t, t_span in update_slices(world, span, start_frame, UPDATE_FRAMES):
        t = int(t)
        f0 = max(0, t - FAST_HISTORY_FRAMES)
        s0 = max(0, t - SLOW_HISTORY_FRAMES)
        fast = {k: v[sub] for k, v in history_components(world, f0, t - f0 + 1,
                                                          half_life=FAST_HALF_LIFE).items()}
        slow = {k: v[sub] for k, v in history_components(world, s0, t - s0 + 1,
                                                          half_life=SLOW_HALF_LIFE).items()}
        scene_fast, scene_slow = fast["scene"], slow["scene"]
        scene = FAST_SCENE_WEIGHT * scene_fast + SLOW_SCENE_WEIGHT * scene_slow
        inter = fast["interaction"]
        carry = prev_scene is not None and prev_informative
        scene_s = alpha * scene + (1.0 - alpha) * prev_scene if carry else scene
        carry = prev_inter is not None and prev_informative
        inter_s = alpha * inter + (1.0 - alpha) * prev_inter if carry else inter
        inter_s = np.where(fast["interaction_valid"] > 0, inter_s, 0.0)
        smooth = np.where(fast["co_alive"] > 0, np.maximum(scene_s, inter_s), 0.0)
        raw = np.maximum(scene, inter)
        for value in (raw, smooth, scene, scene_fast, scene_slow, inter, scene_s, inter_s):
            np.fill_diagonal(value, 0.0)
        parts = {**fast, "scene_fast": scene_fast, "scene_slow": scene_slow, "scene": scene,
                 "interaction_fast": inter, "interaction": inter, "raw": raw,
                 "scene_smooth": scene_s, "interaction_smooth": inter_s,
                 "slow_prox": slow["prox"], "slow_aim": slow["aim"]}
        periods.append(Period(start_frame=t,
                              num_frames=int(round((t_span.stop - t_span.start) / TICKS_PER_FRAME)),
                              span=t_span, raw=_symmetric(raw), smooth=_symmetric(smooth),
                              co_alive=fast["co_alive"], stride=1, parts=parts))
        prev_scene, prev_inter = scene_s, inter_s
        prev_informative = bool(np.any(fast["co_alive"] > 0))
    return periods
