"""The reference-format cache dicts of multics_amd/kv_cache.py on the CPU:
the keys, shapes, dtypes and zero state of wan_video_Nplayers.py:888-989,
every stream buffer a slice of one pool, the reset / detach of :991-1058, and
the rolling-buffer appends (oracle: the reference's semantics restated in
oracle/cached.py) keeping the buffers inside the pool."""

import numpy as np
import pytest
import torch

from multics_amd.kv_cache import (detach_hier_kv_cache, initialize_hier_kv_cache,
                                  reset_hier_kv_cache, stream_pool)
from multics_amd.rolling import rolling_bool_cache_append, rolling_cache_append


def _layers(**kw):
    base = dict(num_layers=2, batch_size=1, dtype=torch.bfloat16, device="cpu", num_players=3,
                num_groups=2, num_local_hub_tokens=2, num_global_hub_tokens=3,
                frame_seq_length=5, local_attn_size=4, num_frame_per_block=2, num_heads=2,
                head_dim=8)
    base.update(kw)
    return initialize_hier_kv_cache(**base)


def test_reference_format():
    layers = _layers()
    assert len(layers) == 2 and layers[0]["agent_caches"][0]["k"].data_ptr() != \
        layers[1]["agent_caches"][0]["k"].data_ptr()
    e = layers[0]
    for key, val in (("sparse_hub", True), ("hier_hub", True), ("num_players", 3),
                     ("num_hub_tokens", 2 * 2 + 3), ("num_groups", 2),
                     ("num_local_hub_tokens", 2), ("num_global_hub_tokens", 3),
                     ("hier_no_local_hub", False), ("frame_seq_length", 5)):
        assert e[key] == val, key
    retention = 4 + 2
    assert len(e["agent_caches"]) == 3 and len(e["local_hubs"]) == 2
    for c in e["agent_caches"]:
        assert c["k"].shape == (1, retention * 5, 2, 8) and c["k"].dtype == torch.bfloat16
    for c in e["local_hubs"]:
        assert c["k"].shape == (1, retention * 2, 2, 8)
        assert c["active"].shape == (retention * 2,) and c["active"].dtype == torch.bool
    assert e["global_hub"]["k"].shape == (1, retention * 3, 2, 8)
    for c in list(e["agent_caches"]) + list(e["local_hubs"]) + [e["global_hub"]]:
        assert c["global_end_index"].dtype == torch.long and c["global_end_index"].item() == 0
        assert c["local_end_index"].item() == 0 and not c["k"].any() and not c["v"].any()
    pk, pv, offs = stream_pool(e)
    assert pk.shape == (1, 3 * 30 + 2 * 12 + 18, 2, 8)
    assert list(offs) == [0, 30, 60, 90, 102, 114]
    # an unbounded window keeps 64 + n frames per stream, as the reference
    u = _layers(local_attn_size=-1, num_layers=1)[0]
    assert u["agent_caches"][0]["k"].shape[1] == (64 + 2) * 5
    nl = _layers(num_layers=1, hier_no_local_hub=True, num_local_hub_tokens=0)[0]
    assert nl["local_hubs"] == [] and stream_pool(nl) is not None


def test_appends_stay_in_the_pool_and_reset():
    e = _layers(num_layers=1)[0]
    pk, pv, offs = stream_pool(e)
    L, H, D, W, n = 5, 2, 8, 4, 2
    g = torch.Generator().manual_seed(0)
    for b in range(5):                       # overflows the 6-frame buffers: eviction shifts
        k = torch.randn(1, n * L, H, D, generator=g).to(torch.bfloat16)
        for p, c in enumerate(e["agent_caches"]):
            rolling_cache_append(c, k, k, b * n * L, (b + 1) * n * L, W + n, 0, L)
        act = torch.tensor([True, False] * 2)
        rolling_bool_cache_append(e["local_hubs"][0], "active", act, b * n * 2, (b + 1) * n * 2,
                                  W + n, 0, 2)
        rolling_cache_append(e["local_hubs"][0], k[:, :n * 2], k[:, :n * 2], b * n * 2,
                             (b + 1) * n * 2, W + n, 0, 2)
        last = k
    assert stream_pool(e) is not None
    c0 = e["agent_caches"][0]
    assert c0["local_end_index"].item() == 30 and c0["global_end_index"].item() == 50
    # the newest block sits at the end of the buffer, inside the pool rows of stream 0
    assert torch.equal(pk[0, offs[0] + 20:offs[0] + 30], last[0])
    assert e["local_hubs"][0]["active"].tolist() == [True, False] * 6
    # the reference's detach step and reset leave the pool in place
    detach_hier_kv_cache([e])
    assert stream_pool(e) is not None
    reset_hier_kv_cache([e], "cpu")
    assert c0["local_end_index"].item() == 0 and not e["local_hubs"][0]["active"].any()
    # a buffer replaced by its own tensor takes the dict out of pooled reads
    c0["k"] = torch.zeros_like(c0["k"])
    assert stream_pool(e) is None


def test_rolling_bool_cache_follows_the_kv_cache():
    """The bool cache and the K/V cache of one stream evict and refresh
    together (attention.py:170-228 against :90-163)."""
    size, tpf = 6, 2
    c = {"k": torch.zeros(1, size, 1, 1), "v": torch.zeros(1, size, 1, 1),
         "active": torch.zeros(size, dtype=torch.bool),
         "global_end_index": torch.tensor([0]), "local_end_index": torch.tensor([0])}
    marks = []
    for step, (s0, s1) in enumerate([(0, 2), (2, 4), (2, 4), (4, 6), (6, 8)]):
        flag = torch.tensor([step % 2 == 0] * (s1 - s0))
        val = torch.full((1, s1 - s0, 1, 1), float(s0) + 0.5 * (step % 2))
        rolling_bool_cache_append(c, "active", flag, s0, s1, 3, 0, 1)
        rolling_cache_append(c, val, val, s0, s1, 3, 0, 1)
        marks.append((c["active"].clone(), c["k"][0, :, 0, 0].clone(),
                      int(c["local_end_index"].item())))
    # step 2 re-runs [2,4): refreshed in place (flag False -> True, value 2.0)
    assert marks[2][0][:4].tolist() == [True, True, True, True]
    assert marks[2][1][:4].tolist() == [0.0, 0.0, 2.0, 2.0]
    # the last step evicts: both caches hold tokens [2, 8) in order
    act, k, end = marks[-1]
    assert end == 6
    assert k.tolist() == [2.0, 2.0, 4.5, 4.5, 6.0, 6.0]
    assert act.tolist() == [True, True, False, False, True, True]
    # a dict without the key is left alone
    d = {"global_end_index": torch.tensor([0]), "local_end_index": torch.tensor([0])}
    rolling_bool_cache_append(d, "active", torch.ones(2, dtype=torch.bool), 0, 2, 3, 0, 1)
    assert "active" not in d
