"""Reading and writing label payloads (``groups.pt``: a dict of tensors).

Loads go through ``torch.load(weights_only=True)``, which executes nothing
from the file, and are validated before use; writes are atomic (a temporary
file in the target directory, flushed, then renamed), so a failed write never
leaves a file that looks valid (multics/grouping/prepare.py:41-53, 63-71).
"""

from __future__ import annotations

import os
import tempfile
from pathlib import Path

import numpy as np
import torch

from .validation import validate_existing_labels, validate_generated_labels


def load_group_labels(path) -> dict:
    """A validated label payload from ``path``."""
    path = Path(path)
    if not path.is_file():
        raise ValueError(f"Grouping path is not a file: {path}")
    payload = torch.load(path, map_location="cpu", weights_only=True)
    validate_existing_labels(payload)
    return payload


def save_group_labels(payload, path, *, num_players: int | None = None) -> Path:
    """Write a payload (numpy arrays or tensors) atomically; with
    ``num_players`` it must pass the generated-schema checks first."""
    tensors = {k: (torch.from_numpy(v.copy()) if isinstance(v, np.ndarray) else v)
               for k, v in payload.items()}
    if num_players is not None:
        validate_generated_labels(tensors, num_players)
    path = Path(path)
    fd, tmp = tempfile.mkstemp(prefix=path.name + ".", suffix=".tmp", dir=path.parent)
    try:
        with os.fdopen(fd, "wb") as fh:
            torch.save(tensors, fh)
            fh.flush()
            os.fsync(fh.fileno())
        os.replace(tmp, path)
    finally:
        if os.path.exists(tmp):
            os.unlink(tmp)
    return path
