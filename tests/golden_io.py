"""Load the golden metadata vectors written by ``tests/golden/make_golden.py``."""

from __future__ import annotations

import hashlib
import json
from functools import lru_cache
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden" / "metadata_golden.npz"


@lru_cache(maxsize=1)
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def cases(kind: str):
    g = golden()
    return [name for k, name in json.loads(str(g["index"])) if k == kind]


def inputs(kind: str, name: str) -> dict:
    return json.loads(str(golden()[f"{kind}/{name}/inputs"]))


def digest(arr) -> str:
    a = np.ascontiguousarray(arr)
    h = hashlib.sha256()
    h.update(str(a.dtype).encode())
    h.update(str(tuple(a.shape)).encode())
    h.update(a.tobytes())
    return "sha256:" + h.hexdigest()


def assert_same(key: str, actual) -> None:
    """Exact equality (dtype, shape, bytes) against a stored array or its digest."""
    exp = golden()[key]
    actual = np.asarray(actual)
    if exp.dtype.kind == "U":
        assert digest(actual) == str(exp), key
        return
    assert actual.dtype == exp.dtype, (key, actual.dtype, exp.dtype)
    assert actual.shape == exp.shape, (key, actual.shape, exp.shape)
    assert np.array_equal(actual, exp), key


def scalar(key: str) -> int:
    return int(golden()[key])
