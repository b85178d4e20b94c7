"""Helpers for the GPU parity tests."""

from __future__ import annotations

import sys

import numpy as np
import torch


def need_gpu():
    import pytest
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def say(*a):
    """Print and flush before a GPU step so a failure names its case."""
    print(*a, flush=True)
    sys.stdout.flush()


def expand_tiles(tiles):
    """TileList -> {query row: set of key indices} on the host."""
    items = tiles.items.cpu().numpy()
    idx = tiles.kv_idx.cpu().numpy()
    msk = tiles.kv_mask.cpu().numpy().view(np.uint32)
    rows = {}
    for qbase, qstride, qlen, r0, rc, off, cnt, n in items:
        kidx = idx[off:off + cnt]
        kmask = msk[off:off + cnt]
        for r in range(r0, r0 + rc):
            j, i = divmod(r, qlen)
            q = qbase + j * qstride + i
            assert q not in rows
            rows[q] = set(kidx[((kmask >> j) & 1) == 1].tolist())
    return rows


def err_stats(actual: torch.Tensor, expected: torch.Tensor):
    d = (actual.detach().float().cpu() - expected.detach().float().cpu()).abs()
    return float(d.max()), float(d.mean())
