"""CPU checks of the paged KV cache addressing (multics_amd/paged_cache.py)."""

import numpy as np
import pytest
import torch

from multics_amd.paged_cache import HierPagedKVCache


def _cache(W=4, n=2, no_local=False):
    return HierPagedKVCache(num_players=3, num_groups=0 if no_local else 2, num_patches=5,
                            num_local_hub_tokens=0 if no_local else 2, num_global_hub_tokens=3,
                            num_heads=2, head_dim=8, local_attn_size=W, num_frame_per_block=n,
                            device="cpu", hier_no_local_hub=no_local)


def test_pages_partition_the_pool():
    c = _cache()
    R = c.R
    assert R == 6
    rows = np.concatenate([c.block_rows(f0, 1) for f0 in range(R)])
    assert np.array_equal(np.sort(rows), np.arange(c.k.shape[0]))   # every row once per R frames
    r = c.block_rows(7, 2)
    assert len(r) == 3 * 2 * 5 + 2 * (2 * 2 + 3)
    # agents p-major, then locals (frame, group), then global, each page contiguous
    assert r[0] == c.agent_row(0, 7) and r[5] == c.agent_row(0, 8)
    assert r[10] == c.agent_row(1, 7)
    assert r[30] == c.local_row(0, 7) and r[32] == c.local_row(1, 7) and r[34] == c.local_row(0, 8)
    assert r[38] == c.global_row(7) and r[41] == c.global_row(8)


def test_window_is_the_last_R_frames():
    c = _cache()
    for f in range(9):                      # what append() records
        c.slot_frame[f % c.R] = f
    frames, (agent, local, glob), lact = c.window(8)
    assert frames == [3, 4, 5, 6, 7, 8]
    assert agent[1] == [c.agent_row(1, f) for f in frames]
    assert glob == [c.global_row(f) for f in frames]
    assert len(local) == 2 and len(lact) == 2
    frames, *_ = c.window(4)                # an older end frame sees only frames <= 4
    assert frames == [3, 4]


def test_no_local_layout_and_errors():
    c = _cache(no_local=True)
    assert c.l_rows == 0 and c.get("hier_no_local_hub") and c["hier_hub"]
    with pytest.raises(ValueError):
        HierPagedKVCache(num_players=2, num_groups=2, num_patches=4, num_local_hub_tokens=2,
                         num_global_hub_tokens=2, num_heads=1, head_dim=8, local_attn_size=1,
                         num_frame_per_block=3, device="cpu")
    with pytest.raises(ValueError):
        HierPagedKVCache(num_players=2, num_groups=2, num_patches=4, num_local_hub_tokens=2,
                         num_global_hub_tokens=2, num_heads=1, head_dim=8, local_attn_size=-1,
                         num_frame_per_block=3, device="cpu")


def test_unbounded_window_refuses_to_wrap():
    """local_attn_size=-1 keeps every frame: appending past max_frames must
    fail instead of overwriting the oldest pages (the reference's buffer
    has no wrap either)."""
    c = HierPagedKVCache(num_players=2, num_groups=1, num_patches=4, num_local_hub_tokens=2,
                         num_global_hub_tokens=2, num_heads=1, head_dim=8, local_attn_size=-1,
                         num_frame_per_block=2, device="cpu", max_frames=4)
    S = 2 * 2 * 4 + 2 * (1 * 2 + 2)
    k = torch.zeros(S, 1, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="max_frames"):
        c.append(k, k, 3, 2, np.ones((2, 1), bool))
    with pytest.raises(ValueError, match="max_frames"):
        c.append(k, k, 4, 2, np.ones((2, 1), bool))


def test_cached_paths_refuse_autograd():
    """The cached attention (paged pool) and the action branches' frame-window
    attention are inference-only, like the reference's cached backends
    (hier_paged_attention.py:123-124): with autograd on and parameters that
    require grad they raise instead of silently detaching q/k/v."""
    from multics_amd.action import frame_attention
    from multics_amd.module import SelfAttention
    attn = SelfAttention(64, 1)
    attn.num_frame_per_block, attn.local_attn_size = 2, 4
    c = HierPagedKVCache(num_players=2, num_groups=1, num_patches=4, num_local_hub_tokens=2,
                         num_global_hub_tokens=2, num_heads=1, head_dim=64, local_attn_size=4,
                         num_frame_per_block=2, device="cpu")
    S = 2 * 2 * 4 + 2 * (2 + 2)
    x = torch.zeros(1, S, 64)
    freqs = torch.ones(S, 1, 32, dtype=torch.complex128)
    with pytest.raises(RuntimeError, match="inference-only"):
        attn.causal_forward(x, freqs, kv_cache=c, num_frames=2, num_players=2,
                            group_labels=torch.zeros(2, 2, dtype=torch.long))
    q = torch.zeros(1, 3, 1, 64, requires_grad=True)
    with pytest.raises(RuntimeError, match="inference-only"):
        frame_attention(q, q, q, torch.arange(3), torch.arange(3), 3, -1)
