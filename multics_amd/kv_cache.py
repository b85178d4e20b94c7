"""The reference's per-layer hierarchical KV cache dicts, backed by one pool.

The pipeline keeps, per DiT layer, a dict with P agent caches, N local-hub
caches (plus per-token ``active`` flags) and one global cache, each ``{k, v:
[B, cap, H, D], global_end_index, local_end_index}``
(wan_video_Nplayers.py:888-989), appended through the rolling-buffer rules of
attention.py:90-228 and reset / detached by the pipeline's own code
(wan_video_Nplayers.py:991-1058).  ``initialize_hier_kv_cache`` returns dicts
of exactly that format, so that code runs unchanged on them, with one
difference in storage: every stream buffer of a layer is a slice of one K pool
and one V pool ``[B, rows, H, D]`` (rows in stream order: agents, local hubs,
global), so the attention reads the cached windows in place instead of
concatenating every stream per call (hier_segmented_attention.py:458-469).

``stream_pool(entry)`` recovers, for a dict of this format, the pool and the
first pool row of each stream -- or None when a buffer was replaced by a
tensor outside the pool (or the dict came from elsewhere), in which case the
attention concatenates the windows as the reference's backends do.

``HierKVCachePipelineMixin`` holds drop-in versions of the pipeline's
``_initialize_hier_kv_cache``, ``init_kv_cache_for_training`` and
``_reset_kv_cache`` built on it.
"""

from __future__ import annotations

from typing import Optional

import torch

_POOL_KEY = "_hier_pool"


def _zeros_index(device):
    return torch.tensor([0], dtype=torch.long, device=device)


def initialize_hier_kv_cache(*, num_layers: int, batch_size: int, dtype, device, num_players: int,
                             num_groups: int, num_local_hub_tokens: int,
                             num_global_hub_tokens: int, frame_seq_length: int,
                             local_attn_size: int, num_frame_per_block: int, num_heads: int,
                             head_dim: int, hier_no_local_hub: bool = False) -> list:
    """Per-layer cache dicts of wan_video_Nplayers.py:888-989 (same keys,
    shapes, dtypes and zero initial state).  Retention is W + n frames per
    stream, with W = 64 for an unbounded window as in the reference."""
    P, N = int(num_players), int(num_groups)
    KL, KG, L = int(num_local_hub_tokens), int(num_global_hub_tokens), int(frame_seq_length)
    no_local = bool(hier_no_local_hub)
    attn_frames = int(local_attn_size) if int(local_attn_size) != -1 else 64
    retention = attn_frames + int(num_frame_per_block)
    caps = [retention * L] * P
    if not no_local:
        caps += [retention * max(KL, 1)] * N
    caps += [retention * max(KG, 1)]
    offs = [0]
    for c in caps:
        offs.append(offs[-1] + c)
    B, H, D = int(batch_size), int(num_heads), int(head_dim)
    layers = []
    for _ in range(int(num_layers)):
        pk = torch.zeros([B, offs[-1], H, D], dtype=dtype, device=device)
        pv = torch.zeros_like(pk)

        def stream(i):
            return {"k": pk[:, offs[i]:offs[i + 1]], "v": pv[:, offs[i]:offs[i + 1]],
                    "global_end_index": _zeros_index(device),
                    "local_end_index": _zeros_index(device)}

        agents = [stream(p) for p in range(P)]
        locals_ = []
        if not no_local:
            for g in range(N):
                d = stream(P + g)
                d["active"] = torch.zeros([caps[P + g]], dtype=torch.bool, device=device)
                locals_.append(d)
        layers.append({
            "sparse_hub": True, "hier_hub": True, "num_players": P,
            "num_hub_tokens": N * KL + KG, "num_groups": N, "num_local_hub_tokens": KL,
            "num_global_hub_tokens": KG, "hier_no_local_hub": no_local, "frame_seq_length": L,
            "agent_caches": agents, "local_hubs": locals_, "global_hub": stream(len(caps) - 1),
            _POOL_KEY: (pk, pv, tuple(offs[:-1])),
        })
    return layers


def stream_pool(entry: dict) -> Optional[tuple]:
    """``(pool_k, pool_v, first pool row of each stream)`` of a layer dict
    whose stream buffers are all still slices of its pools (stream order:
    agents, local hubs, global), else None."""
    held = entry.get(_POOL_KEY)
    if held is None:
        return None
    pk, pv, offs = held
    streams = list(entry["agent_caches"]) + list(entry["local_hubs"]) + [entry["global_hub"]]
    if len(streams) != len(offs):
        return None
    row_k = pk.stride(1) * pk.element_size()
    row_v = pv.stride(1) * pv.element_size()
    for s, off in zip(streams, offs):
        k, v = s["k"], s["v"]
        if k.dtype != pk.dtype or v.dtype != pv.dtype or k.stride() != pk.stride() or \
                v.stride() != pv.stride():
            return None
        if k.data_ptr() != pk.data_ptr() + off * row_k or v.data_ptr() != pv.data_ptr() + off * row_v:
            return None
    return pk, pv, offs


def reset_hier_kv_cache(kv_cache: list, device) -> None:
    """wan_video_Nplayers.py:1024-1058: every stream's end indices back to 0,
    the local hubs' ``active`` flags cleared, the action caches' end indices
    reset (their buffers are kept)."""
    for entry in kv_cache:
        for c in list(entry["agent_caches"]) + [entry["global_hub"]]:
            c["global_end_index"] = _zeros_index(device)
            c["local_end_index"] = _zeros_index(device)
        for c in entry["local_hubs"]:
            c["active"].zero_()
            c["global_end_index"] = _zeros_index(device)
            c["local_end_index"] = _zeros_index(device)
        for name in ("action_temporal", "action_keyboard"):
            c = entry.get(name)
            if c is not None:
                c["global_end_index"] = _zeros_index(device)
                c["local_end_index"] = _zeros_index(device)


def detach_hier_kv_cache(kv_cache: list) -> None:
    """The detach step of wan_video_Nplayers.py:1009-1018 (the detached
    tensors are views of the same storage, so the pools stay valid)."""
    for entry in kv_cache:
        for c in entry["agent_caches"]:
            c["k"], c["v"] = c["k"].detach(), c["v"].detach()
        for c in entry["local_hubs"]:
            c["k"], c["v"], c["active"] = c["k"].detach(), c["v"].detach(), c["active"].detach()
        g = entry["global_hub"]
        g["k"], g["v"] = g["k"].detach(), g["v"].detach()


class HierKVCachePipelineMixin:
    """The pipeline's cache methods (wan_video_Nplayers.py:888-1058) on pooled
    cache dicts.  Reads the pipeline attributes the reference reads:
    ``num_players``, ``dit`` (``num_groups``, ``num_local_hub_tokens``,
    ``num_global_hub_tokens``, ``hier_no_local_hub``, ``blocks[0].self_attn``),
    ``frame_seq_length``, ``local_attn_size``, ``num_frame_per_block``,
    ``num_transformer_blocks``, ``torch_dtype``, ``kv_cache1`` and the
    cross-attention cache methods."""

    def _initialize_hier_kv_cache(self, batch_size, dtype, device):
        attn = self.dit.blocks[0].self_attn
        self.kv_cache1 = initialize_hier_kv_cache(
            num_layers=self.num_transformer_blocks, batch_size=batch_size, dtype=dtype,
            device=device, num_players=self.num_players, num_groups=int(self.dit.num_groups),
            num_local_hub_tokens=int(self.dit.num_local_hub_tokens),
            num_global_hub_tokens=int(self.dit.num_global_hub_tokens),
            frame_seq_length=self.frame_seq_length, local_attn_size=self.local_attn_size,
            num_frame_per_block=self.num_frame_per_block, num_heads=attn.num_heads,
            head_dim=attn.head_dim,
            hier_no_local_hub=bool(getattr(self.dit, "hier_no_local_hub", False)))

    def init_kv_cache_for_training(self, batch_size: int, device: torch.device):
        kv_batch = batch_size // self.num_players
        if self.kv_cache1 is None:
            self._initialize_hier_kv_cache(batch_size=kv_batch, dtype=self.torch_dtype,
                                           device=device)
            self._initialize_crossattn_cache(batch_size=batch_size, dtype=self.torch_dtype,
                                             device=device)
        else:
            detach_hier_kv_cache(self.kv_cache1)
            for block_index in range(self.num_transformer_blocks):
                self.crossattn_cache[block_index]["is_init"] = False
            self._reset_kv_cache(device)

    def _reset_kv_cache(self, device):
        if self.kv_cache1 is None:
            return
        reset_hier_kv_cache(self.kv_cache1, device)
