"""Simplex 4D RoPE frequency tables and their fp32 cos/sin form.

The complex128 tables keep the reference's layout and values
(multics/models/rope.py:103-237; WanModel.build_self_attn_freqs_with_hub,
multics/models/wan_video_dit.py:338-389): per token 64 rotations in four bands
-- temporal (6, the lowest frequencies of Wan's 44-channel temporal band), agent
(16, constant per player: angles of a regular-simplex vertex x gamma), height
(21) and width (21); hub tokens carry only the temporal phase.

``freqs_to_cos_sin`` turns any such ``[S,1,D/2]`` complex table into the fp32
``[S,D/2]`` cos / sin pair that the fused Q/K prologue reads.
"""

from __future__ import annotations

import os
from collections import OrderedDict
from typing import Tuple

import torch

WAN_REROPE_SPLITS = (12, 32, 42, 42)   # rope.py:5


def precompute_freqs_cis(dim: int, end: int = 1024, theta: float = 10000.0) -> torch.Tensor:
    """``exp(i * t * theta^(-2j/dim))`` for t < end, j < dim/2, complex128 (rope.py:103-107)."""
    inv = 1.0 / theta ** (torch.arange(0, dim, 2)[: dim // 2].double() / dim)
    ang = torch.outer(torch.arange(end, dtype=torch.float64), inv)
    return torch.polar(torch.ones_like(ang), ang)


def build_simplex_vertices(pool_size: int, d_agent: int) -> torch.Tensor:
    """Unit vertices of a regular (m-1)-simplex, float32 ``[m, d_agent//2]`` (rope.py:110-126)."""
    m, half = int(pool_size), d_agent // 2
    if m < 2:
        raise ValueError("pool_size must be >= 2")
    if m > half + 1:
        raise ValueError(f"pool_size {m} exceeds limit d_agent//2+1={half + 1} for d_agent={d_agent}")
    centered = torch.eye(m, dtype=torch.float64) - 1.0 / m
    unit = centered / centered.norm(dim=1, keepdim=True).clamp(min=1e-12)
    out = torch.zeros(m, half, dtype=torch.float32)
    out[:, :m] = unit.to(torch.float32)
    return out


def precompute_freqs_cis_4d_wan_rerope(head_dim: int = 128, end: int = 1024,
                                       theta: float = 10000.0,
                                       splits: Tuple[int, int, int, int] = WAN_REROPE_SPLITS):
    """Band tables of the 4D "ReRoPE" (rope.py:129-144)."""
    d_t, d_a, d_h, d_w = splits
    if d_t + d_a + d_h + d_w != head_dim:
        raise AssertionError(splits)
    wan_t = precompute_freqs_cis(head_dim - 2 * (head_dim // 3), end, theta)
    return {"t": wan_t[:, -(d_t // 2):], "h": precompute_freqs_cis(d_h, end, theta),
            "w": precompute_freqs_cis(d_w, end, theta), "splits": splits, "d_a": d_a}


def _agent_freqs_cis_from_vertex(simplex_vertices, vertex_id: int, gamma: float = 1.0):
    ang = simplex_vertices[vertex_id].to(torch.float64) * float(gamma)
    return torch.polar(torch.ones_like(ang), ang)


def build_spatial_freqs_4d_single_player(freqs_bands, f, h, w, simplex_vertices, vertex_id,
                                         gamma=1.0, device=None, start_frame=0):
    """``[f*h*w, 1, D/2]`` for one player, band order (t | a | h | w) (rope.py:155-188)."""
    d_t, d_a, d_h, d_w = freqs_bands["splits"]
    nt, nh, nw = d_t // 2, d_h // 2, d_w // 2
    ft = freqs_bands["t"][start_frame:start_frame + f].to(device)
    fh = freqs_bands["h"][:h].to(device)
    fw = freqs_bands["w"][:w].to(device)
    grid = torch.cat([ft.view(f, 1, 1, nt).expand(f, h, w, nt),
                      fh.view(1, h, 1, nh).expand(f, h, w, nh),
                      fw.view(1, 1, w, nw).expand(f, h, w, nw)], dim=-1).reshape(f * h * w, -1)
    agent = _agent_freqs_cis_from_vertex(simplex_vertices, vertex_id, gamma).to(device)
    agent = agent.view(1, -1).expand(f * h * w, -1)
    return torch.cat([grid[:, :nt], agent, grid[:, nt:]], dim=-1).unsqueeze(1)


def build_multiplayer_freqs_4d(freqs_bands, f, h, w, agent_vertex_ids, simplex_vertices,
                               gamma=1.0, device=None, start_frame=0):
    """Player-major concatenation (rope.py:191-220)."""
    if device is None:
        device = simplex_vertices.device
    return torch.cat([build_spatial_freqs_4d_single_player(
        freqs_bands, f, h, w, simplex_vertices, int(v), gamma, device, start_frame=start_frame)
        for v in agent_vertex_ids], dim=0)


def build_hub_freqs_4d(freqs_bands, f, num_hub_tokens, start_frame=0, device=None):
    """Hub tokens: frame-slot temporal phase, identity elsewhere (rope.py:223-237)."""
    d_t, d_a, d_h, d_w = freqs_bands["splits"]
    if device is None:
        device = freqs_bands["t"].device
    ft = freqs_bands["t"][start_frame:start_frame + f].to(device)
    t_grid = ft.repeat_interleave(num_hub_tokens, dim=0)
    ident = torch.ones(f * num_hub_tokens, (d_a + d_h + d_w) // 2, device=device,
                       dtype=torch.complex64)
    return torch.cat([t_grid, ident], dim=-1).unsqueeze(1)


def rope_split_sizes_4d(head_dim: int, splits=WAN_REROPE_SPLITS):
    d_t, d_a, d_h, d_w = splits
    return [d_t // 2, d_a // 2, d_h // 2, d_w // 2]


def build_self_attn_freqs_with_hub(freqs_bands, simplex_vertices, f, h, w, device,
                                   agent_vertex_ids, num_hub_tokens, gamma=1.0, start_frame=0):
    """``[P*f*h*w + f*K, 1, D/2]``: players then hub tokens
    (WanModel.build_self_attn_freqs_with_hub, wan_video_dit.py:338-359,
    honouring STAGE2_ROPE_AGENT_GLOBAL for the agent temporal offset)."""
    agent_start = start_frame if os.environ.get("STAGE2_ROPE_AGENT_GLOBAL", "1") != "0" else 0
    if isinstance(agent_vertex_ids, torch.Tensor):
        agent_vertex_ids = agent_vertex_ids.detach().cpu().tolist()
    agent = build_multiplayer_freqs_4d(freqs_bands, f, h, w, agent_vertex_ids, simplex_vertices,
                                       gamma=gamma, device=device, start_frame=agent_start)
    hub = build_hub_freqs_4d(freqs_bands, f, num_hub_tokens, start_frame=start_frame, device=device)
    return torch.cat([agent, hub], dim=0)


# The last tables converted: every layer of a model step receives the same
# complex table, so the conversion runs once per step, not once per layer.
# An entry holds its table (its storage cannot be reused while the entry
# lives) and the table's version counter (an in-place change is a miss).
_COS_SIN_CACHE: "OrderedDict[tuple, tuple]" = OrderedDict()
_COS_SIN_CACHE_SIZE = 2


def freqs_to_cos_sin(freqs: torch.Tensor, device=None):
    """``[S,1,D/2]`` (or ``[S,D/2]``) complex table -> fp32 (cos, sin) ``[S,D/2]`` on ``device``.
    The result of the last tables is cached (keyed by the table object, its
    version counter and the device)."""
    dev = torch.device(device) if device is not None else freqs.device
    key = (id(freqs), freqs._version, str(dev))
    hit = _COS_SIN_CACHE.get(key)
    if hit is not None and hit[0] is freqs:
        _COS_SIN_CACHE.move_to_end(key)
        return hit[1], hit[2]
    f = freqs.reshape(freqs.shape[0], -1)
    if device is not None:
        f = f.to(device)
    cs, sn = f.real.to(torch.float32).contiguous(), f.imag.to(torch.float32).contiguous()
    if not freqs.requires_grad:
        _COS_SIN_CACHE[key] = (freqs, cs, sn)
        while len(_COS_SIN_CACHE) > _COS_SIN_CACHE_SIZE:
            _COS_SIN_CACHE.popitem(last=False)
    return cs, sn
