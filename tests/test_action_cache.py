"""The action branches' rolling cache append against the oracle's restatement
of the same reference function (attention.py:90-163, sink_size = 0), on CPU."""

import numpy as np
import torch

from multics_amd.action import ensure_action_cache, rolling_cache_append
from oracle.cached import RollingCache, append


def _run(local_attn, tpf, seed):
    rng = np.random.default_rng(seed)
    B, nh, hd, n = 3, 2, 8, 3
    retention = local_attn + n if local_attn != -1 else None
    frames_total = 15
    parent = {}
    cap = (retention if retention is not None else frames_total) * tpf
    ref = RollingCache(k=torch.zeros(cap, B * nh, hd), v=torch.zeros(cap, B * nh, hd))
    g = torch.Generator().manual_seed(seed)
    for blk in range(frames_total // n):
        start = blk * n
        for _ in range(int(rng.integers(1, 3))):       # a block is re-run with new values
            k = torch.randn(B, n * tpf, nh, hd, generator=g)
            v = torch.randn(B, n * tpf, nh, hd, generator=g)
            c = ensure_action_cache(parent, "action_temporal", B, nh, hd, tpf,
                                    retention if retention is not None else frames_total,
                                    "cpu", torch.float32)
            a0, end = rolling_cache_append(c, k, v, start * tpf, (start + n) * tpf,
                                           retention if retention is not None else -1, 0, tpf)
            fold = lambda t: t.permute(1, 0, 2, 3).reshape(t.shape[1], B * nh, hd)
            append(ref, fold(k), fold(v), start * tpf, (start + n) * tpf,
                   retention if retention is not None else -1, tpf)
            assert end == ref.local_end
            assert int(c["global_end_index"]) == ref.global_end == (start + n) * tpf
            assert torch.equal(fold(c["k"])[:end], ref.k[:end])
            assert torch.equal(fold(c["v"])[:end], ref.v[:end])
            # the window: everything cached, at most retention frames
            assert a0 == 0 and end == min(start + n, retention or 10 ** 9) * tpf


def test_rolling_append_matches_oracle_windowed():
    _run(local_attn=6, tpf=1, seed=1)
    _run(local_attn=4, tpf=3, seed=2)


def test_rolling_append_matches_oracle_unbounded():
    _run(local_attn=-1, tpf=2, seed=3)


def test_ensure_action_cache_reallocates_on_shape_change():
    parent = {}
    c1 = ensure_action_cache(parent, "x", 2, 4, 8, 1, 5, "cpu", torch.float32)
    assert ensure_action_cache(parent, "x", 2, 4, 8, 1, 5, "cpu", torch.float32) is c1
    c2 = ensure_action_cache(parent, "x", 3, 4, 8, 1, 5, "cpu", torch.float32)
    assert c2 is not c1 and c2["k"].shape == (3, 5, 4, 8)
