"""Drop-in hierarchical "block mask" builders for the FlexAttention call path.

The reference builds a FlexAttention ``BlockMask`` over the padded full
sequence once per forward (``build_stage2_hier_flex_block_mask``,
hier_masks.py:722-1149, called from WanModel.forward, wan_video_dit.py:633-658)
and passes it to ``SelfAttention.forward(x, freqs, mask)`` of every block
(blocks.py:203, attention.py:436-442), whose FlexAttention forward and
autograd backward run over it (attention.py:322-353).

``build_stage2_hier_flex_block_mask`` here takes the same arguments and
returns the same ``(mask, S, S_pad)`` triple; the mask is a
``HierBlockMask``: the HIP tile list of the topology (which only lists the
mask's permitted keys) plus the rows of the one edge class the tile list
leaves out -- the self edge of an inactive local-hub row, which makes that
row's output its own value.  ``multics_amd.module.SelfAttention.forward``
runs the HIP forward / backward over it.  Same cache policy as the
reference: an LRU keyed by the full topology (WAN_HIER_BLOCKMASK_CACHE_SIZE,
default 2).
"""

from __future__ import annotations

import math
import os
from collections import OrderedDict
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import metadata as M
from .metadata import TileList, _freeze
from .topology import (_prepare_hier_group_tensors, _prepare_hier_membership_tensors,
                       _validate_hier_no_local_topology)


@dataclass(frozen=True)
class HierBlockMask:
    """The hierarchical attention mask of one full-sequence topology.

    ``shape`` is ``(1, 1, S_pad, S_pad)`` as a BlockMask's; ``tiles`` the HIP
    tile list; ``self_rows`` (int64, device) the inactive local-hub rows, whose
    only key is themselves."""
    tiles: TileList
    self_rows: torch.Tensor
    S: int
    S_pad: int
    num_players: int
    num_frames: int
    num_patches: int
    num_groups: int
    num_local_hub_tokens: int
    num_global_hub_tokens: int

    @property
    def shape(self):
        return (1, 1, self.S_pad, self.S_pad)


_MASK_CACHE: "OrderedDict[tuple, tuple]" = OrderedDict()


def _cache_put(key, value):
    n = int(os.environ.get("WAN_HIER_BLOCKMASK_CACHE_SIZE", "2"))
    if n < 0:
        _MASK_CACHE[key] = value
        return value
    if n == 0:
        return value
    _MASK_CACHE[key] = value
    _MASK_CACHE.move_to_end(key)
    while len(_MASK_CACHE) > n:
        _MASK_CACHE.popitem(last=False)
    return value


def clear_hier_block_mask_cache() -> None:
    _MASK_CACHE.clear()


def build_stage2_hier_flex_block_mask(num_players: int, num_frames: int, num_patches: int,
                                      num_groups: int, num_local_hub_tokens: int,
                                      num_global_hub_tokens: int, num_frame_per_block: int,
                                      local_attn_size: int, group_labels: Optional[torch.Tensor],
                                      active_group: Optional[torch.Tensor], direct_player: bool,
                                      device, membership: Optional[torch.Tensor] = None,
                                      global_only: Optional[torch.Tensor] = None,
                                      hier_no_local_hub: bool = False):
    """Same arguments, checks and return triple ``(mask, S, S_pad)`` as the
    reference (labels form hier_masks.py:722-934, membership form :937-1149)."""
    P, T, L = int(num_players), int(num_frames), int(num_patches)
    N, KL, KG = int(num_groups), int(num_local_hub_tokens), int(num_global_hub_tokens)
    _validate_hier_no_local_topology(hier_no_local_hub, KL, KG)
    if local_attn_size != -1 and local_attn_size < num_frame_per_block:
        raise ValueError(
            f"hier_hub requires local_attn_size=-1 or >= num_frame_per_block; got "
            f"local_attn_size={local_attn_size}, n={num_frame_per_block}")
    if P > 62:
        raise ValueError(f"hier_hub flex bitset path supports P<=62, got P={P}")
    if membership is not None:
        if N > 62:
            raise ValueError(f"hier_hub flex bitset path supports N<=62, got N={N}")
        mem, go, act = _prepare_hier_membership_tensors(membership, global_only, active_group, P,
                                                        T, N, "cpu")
        mem_np, go_np, act_np = mem.numpy(), go.numpy(), act.numpy()
        labels_np = None
    else:
        labels, act = _prepare_hier_group_tensors(group_labels, active_group, P, T, N, "cpu")
        labels_np, act_np = labels.numpy(), act.numpy()
        mem_np = go_np = None
    S = P * T * L + T * (N * KL + KG)
    S_pad = math.ceil(S / 128) * 128
    key = ("hier", P, T, L, N, KL, KG, int(num_frame_per_block), int(local_attn_size),
           bool(direct_player), bool(hier_no_local_hub), _freeze(labels_np), _freeze(mem_np),
           _freeze(go_np), _freeze(act_np), S_pad, str(torch.device(device)))
    hit = _MASK_CACHE.get(key)
    if hit is not None:
        _MASK_CACHE.move_to_end(key)
        return hit
    tiles = M.full_sequence_tiles(
        device=device, P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=int(num_frame_per_block),
        window=int(local_attn_size), direct=bool(direct_player), labels=labels_np, active=act_np,
        membership=mem_np, global_only=go_np, no_local=bool(hier_no_local_hub))
    # inactive local-hub rows: the time-major local token order of hier_masks.py:549-571
    if KL > 0 and not hier_no_local_hub:
        t_idx, g_idx = np.nonzero(~act_np.astype(bool))
        rows = (P * T * L + (t_idx[:, None] * N + g_idx[:, None]) * KL +
                np.arange(KL)[None, :]).reshape(-1)
    else:
        rows = np.zeros(0, dtype=np.int64)
    mask = HierBlockMask(tiles=tiles, self_rows=torch.from_numpy(rows.astype(np.int64)).to(device),
                         S=S, S_pad=S_pad, num_players=P, num_frames=T, num_patches=L,
                         num_groups=N, num_local_hub_tokens=KL, num_global_hub_tokens=KG)
    return _cache_put(key, (mask, S, S_pad))
