"""Per-tick player states, the input of the label generator.

``grouping_state.npz`` holds non-object arrays only and loads with
``allow_pickle=False`` (multics/grouping/state.py:12-143; the format in
docs/DYNAMIC_GROUPING.md:36-48).  Ticks run at 64 Hz on a continuous grid
(missing records kept, flagged by ``present``); the video runs at 32 fps, so
frame f of the round starts at tick ``round_tick_start + 2 f``.  A state
covers the clip and up to 48 frames of history before it.
"""

from __future__ import annotations

from dataclasses import dataclass, fields

import numpy as np

FORMAT_VERSION = 1
TICKS_PER_FRAME = 64.0 / 32.0
HISTORY_FRAMES = 48
EYE_HEIGHT = 64.0

_ARRAYS = {   # name: (shape in terms of T ticks / P players, dtype)
    "ticks": (("T",), np.int64),
    "pos": (("T", "P", 3), np.float32),
    "yaw": (("T", "P"), np.float32),
    "pitch": (("T", "P"), np.float32),
    "alive": (("T", "P"), np.bool_),
    "present": (("T", "P"), np.bool_),
    "player_slots": (("P",), np.int64),
}
_INT_SCALARS = ("round_tick_start", "round_tick_end", "match_id", "round_no",
                "clip_start_frame", "clip_num_frames")


@dataclass
class GroupingState:
    """Field names and meaning of the reference's state (state.py:12-27)."""

    ticks: np.ndarray
    pos: np.ndarray
    yaw: np.ndarray
    pitch: np.ndarray
    alive: np.ndarray
    present: np.ndarray
    player_slots: np.ndarray
    round_tick_start: int
    round_tick_end: int      # inclusive, before cropping
    match_id: int
    map_name: str
    round_no: int
    clip_start_frame: int
    clip_num_frames: int

    @property
    def num_players(self) -> int:
        return len(self.player_slots)

    def frame_to_tick(self, frame) -> int:
        return int(self.round_tick_start + round(frame * TICKS_PER_FRAME))

    def frame_window(self, start_frame, num_frames) -> slice:
        """Tick rows of frames [start_frame, start_frame + num_frames)."""
        lo, hi = np.searchsorted(self.ticks, [self.frame_to_tick(start_frame),
                                              self.frame_to_tick(start_frame + num_frames)])
        return slice(int(lo), int(hi))

    def eye_pos(self) -> np.ndarray:
        """Eye positions: the feet plus 64 units, added in float32."""
        eye = self.pos.copy()
        eye[..., 2] += EYE_HEIGHT
        return eye

    def validate(self) -> None:
        t, p = len(self.ticks), self.num_players
        if not t or p < 2 or p > 10:
            raise ValueError("Grouping state requires ticks and 2–10 players")
        dims = {"T": t, "P": p}
        for name, (shape, dtype) in _ARRAYS.items():
            want = tuple(dims.get(s, s) for s in shape)
            value = getattr(self, name)
            if value.shape != want or value.dtype != dtype:
                raise ValueError(f"Invalid {name}: expected {want}/{np.dtype(dtype)}")
        if not np.all(np.diff(self.ticks) == 1):
            raise ValueError("Grouping tick grid must be continuous (retain missing ticks)")
        slots = self.player_slots
        if len(np.unique(slots)) != p or np.any((slots < 0) | (slots >= 10)):
            raise ValueError("Grouping player_slots must be distinct physical slots in [0,9]")
        if self.clip_start_frame < 0 or self.clip_num_frames <= 0:
            raise ValueError("Invalid grouping clip range")
        first = self.frame_to_tick(max(0, self.clip_start_frame - HISTORY_FRAMES))
        last = self.frame_to_tick(self.clip_start_frame + self.clip_num_frames) - 1
        if (self.ticks[0] > first or self.ticks[-1] < last
                or self.round_tick_start > self.ticks[0] or self.round_tick_end < self.ticks[-1]):
            raise ValueError("Grouping state does not cover the clip and its 48-frame history")
        active = self.alive & self.present
        for name in ("pos", "yaw", "pitch"):
            if not np.isfinite(getattr(self, name)[active]).all():
                raise ValueError(f"Non-finite {name} for an active player")

    def save(self, path) -> None:
        self.validate()
        np.savez_compressed(path, format_version=np.int32(FORMAT_VERSION),
                            **{f.name: getattr(self, f.name) for f in fields(self)})

    @classmethod
    def load(cls, path) -> "GroupingState":
        names = {f.name for f in fields(cls)}
        with np.load(path, allow_pickle=False) as data:
            if set(data.files) != names | {"format_version"}:
                raise ValueError(f"Invalid grouping state fields: {path}")
            version = data["format_version"]
            if version.shape != () or version.item() != FORMAT_VERSION:
                raise ValueError(f"Unsupported grouping state version: {path}")
            values = {name: data[name].copy() for name in names}
        for name in _INT_SCALARS:
            v = values[name]
            if v.shape != () or v.dtype.kind not in "iu":
                raise ValueError(f"{name} must be an integer scalar: {path}")
            values[name] = int(v)
        if values["map_name"].shape != () or values["map_name"].dtype.kind != "U":
            raise ValueError(f"map_name must be a string scalar: {path}")
        values["map_name"] = str(values["map_name"].item())
        state = cls(**values)
        state.validate()
        return state


def eligible_players(world: GroupingState, span: slice) -> np.ndarray:
    """Players with a record on every tick of ``span`` that has any record
    (ticks where nobody has a record are ignored; state.py:260-265)."""
    present = world.present[span]
    rows = present.any(1) if len(present) else np.zeros(0, bool)
    if not rows.any():
        return np.zeros(world.num_players, bool)
    return present[rows].all(0)


def update_slices(world: GroupingState, span: slice, first_frame: int, every: int):
    """``(frame, tick slice)`` of each grouping period of ``every`` frames
    covering ``span`` (the last one shorter; state.py:268-278)."""
    n = int(round((span.stop - span.start) / TICKS_PER_FRAME))
    if every <= 0 or every >= n:
        return [(first_frame, span)]
    out = []
    for k in range(0, n, every):
        sub = world.frame_window(first_frame + k, min(every, n - k))
        if sub.stop > sub.start:
            out.append((first_frame + k, sub))
    return out
