"""Rolling per-stream KV caches of the reference's cached attention.

``rolling_cache_append`` (attention.py:90-163) and ``rolling_bool_cache_append``
(attention.py:170-228) keep the reference's cache dict format -- ``k`` / ``v``
``[B, size, heads, head_dim]`` plus ``global_end_index`` / ``local_end_index``
(and a 1D bool ``active`` for the local hubs) -- and its semantics, which the
cached rollout's outputs depend on: tokens of a re-run block are refreshed in
place, new tokens are appended, and when a windowed buffer overflows the
oldest non-sink tokens are dropped by moving the rest towards the front.  All
writes are slice assignments on the device tensors, so a buffer that is a
view into a larger pool (``kv_cache.initialize_hier_kv_cache``) stays inside
that pool.
"""

from __future__ import annotations

import torch


def rolling_cache_append(kv_cache: dict, roped_key: torch.Tensor, value: torch.Tensor,
                         current_start: int, current_end: int, local_attn_size: int,
                         sink_size: int, tokens_per_frame: int):
    """attention.py:90-163: write tokens [current_start, current_end) into a
    rolling cache.  Tokens already cached are refreshed in place; new ones
    are appended, and when the buffer overflows (windowed caches) the oldest
    non-sink tokens are dropped by moving the rest towards the front.
    Returns ``(attn_start, local_end)``, the buffer range the new tokens
    attend to."""
    sink = sink_size * tokens_per_frame
    size = kv_cache["k"].shape[1]
    g_end = int(kv_cache["global_end_index"].item())
    l_end = int(kv_cache["local_end_index"].item())
    n_new = min(roped_key.shape[1], max(0, current_end - g_end))
    if n_new == 0 and l_end > 0:           # a re-run block: refresh what is cached
        g_start = g_end - l_end
        r0, r1 = max(current_start, g_start), min(current_end, g_end)
        if r1 > r0:
            src, dst = r0 - current_start, r0 - g_start
            kv_cache["k"][:, dst:dst + r1 - r0] = roped_key[:, src:src + r1 - r0]
            kv_cache["v"][:, dst:dst + r1 - r0] = value[:, src:src + r1 - r0]
    new_end = l_end + n_new
    if local_attn_size != -1 and current_end > g_end and new_end > size:
        evict = max(0, min(new_end - size, new_end - sink - 1))
        if evict > 0:
            keep = max(0, l_end - evict - sink)
            if keep > 0:
                for name in ("k", "v"):
                    kv_cache[name][:, sink:sink + keep] = \
                        kv_cache[name][:, sink + evict:sink + evict + keep].clone()
            new_end = min(l_end + n_new - evict, size)
    if n_new > 0:
        kv_cache["k"][:, new_end - n_new:new_end] = roped_key[:, -n_new:]
        kv_cache["v"][:, new_end - n_new:new_end] = value[:, -n_new:]
    max_attn = size if local_attn_size == -1 else min(local_attn_size * tokens_per_frame, size)
    attn_start = max(0, new_end - max_attn)
    if sink_size > 0 and sink > attn_start:
        attn_start = 0
    kv_cache["global_end_index"].fill_(current_end)
    kv_cache["local_end_index"].fill_(new_end)
    return attn_start, new_end


def rolling_bool_cache_append(kv_cache: dict, key: str, values: torch.Tensor, current_start: int,
                              current_end: int, local_attn_size: int, sink_size: int,
                              tokens_per_frame: int) -> None:
    """attention.py:170-228: the 1D bool cache ``kv_cache[key]`` (the local
    hubs' per-token ``active`` flags) in lockstep with the K/V append of the
    same tokens -- call it before ``rolling_cache_append``, which advances
    the end indices both read.  A missing key is left alone."""
    if key not in kv_cache:
        return
    sink = sink_size * tokens_per_frame
    cache = kv_cache[key]
    size = cache.shape[0]
    g_end = int(kv_cache["global_end_index"].item())
    l_end = int(kv_cache["local_end_index"].item())
    n_new = min(values.shape[0], max(0, current_end - g_end))
    if n_new == 0 and l_end > 0:           # a re-run block: refresh what is cached
        g_start = g_end - l_end
        r0, r1 = max(current_start, g_start), min(current_end, g_end)
        if r1 > r0:
            src, dst = r0 - current_start, r0 - g_start
            cache[dst:dst + r1 - r0] = values[src:src + r1 - r0]
    new_end = l_end + n_new
    if local_attn_size != -1 and current_end > g_end and new_end > size:
        evict = max(0, min(new_end - size, new_end - sink - 1))
        if evict > 0:
            keep = max(0, l_end - evict - sink)
            if keep > 0:
                cache[sink:sink + keep] = cache[sink + evict:sink + evict + keep].clone()
            new_end = min(l_end + n_new - evict, size)
    if n_new > 0:
        cache[new_end - n_new:new_end] = values[-n_new:]
