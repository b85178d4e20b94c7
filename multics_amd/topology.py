"""Hierarchical topology normalisation (labels / membership / active slots).

Same names, argument meaning and errors as the reference's normalisers
(multics/models/hier_masks.py:22-214).  These run once per call on tiny
``[T,P]`` / ``[T,N,P]`` tensors; the per-token work happens in the HIP
metadata builder.
"""

from __future__ import annotations

from typing import Optional

import torch


def _prepare_hier_group_tensors(group_labels, active_group, num_players, num_frames, num_groups,
                                device):
    """labels [T,P] (or [1,T,P]) in [0,N), active [T,N] (default: scatter of labels).

    hier_masks.py:22-71.
    """
    if group_labels is None:
        raise ValueError("hier_hub requires group_labels [T,P] or [1,T,P]")
    labels = group_labels
    if labels.dim() == 3:
        if labels.shape[0] != 1:
            raise ValueError(f"hier_hub expects group_labels batch B=1, got {tuple(labels.shape)}")
        labels = labels[0]
    if labels.shape != (num_frames, num_players):
        raise ValueError(
            f"group_labels must be [T={num_frames},P={num_players}], got {tuple(labels.shape)}")
    labels = labels.to(device=device, dtype=torch.long).contiguous()
    if labels.numel():
        lo, hi = int(labels.min().item()), int(labels.max().item())
        if lo < 0 or hi >= num_groups:
            raise ValueError(
                f"group_labels values must be in [0,{num_groups}), got min={lo} max={hi}")
    if active_group is None:
        active = torch.zeros(num_frames, num_groups, device=device, dtype=torch.bool)
        active.scatter_(1, labels, True)
    else:
        active = active_group
        if active.dim() == 3:
            if active.shape[0] != 1:
                raise ValueError(
                    f"hier_hub expects active_group batch B=1, got {tuple(active.shape)}")
            active = active[0]
        if active.shape != (num_frames, num_groups):
            raise ValueError(
                f"active_group must be [T={num_frames},N={num_groups}], got {tuple(active.shape)}")
        active = active.to(device=device, dtype=torch.bool).contiguous()
    return labels, active


def _squeeze_hier_batch(tensor, expected_tail_ndim: int, name: str):
    """Drop an optional leading B=1 dim (hier_masks.py:74-91)."""
    if tensor.dim() == expected_tail_ndim + 1:
        if tensor.shape[0] != 1:
            raise ValueError(f"{name} batch B must be 1, got {tuple(tensor.shape)}")
        tensor = tensor[0]
    if tensor.dim() != expected_tail_ndim:
        raise ValueError(
            f"{name} must have rank {expected_tail_ndim} or {expected_tail_ndim + 1} with B=1, "
            f"got {tuple(tensor.shape)}")
    return tensor


def _debug_labels_from_membership(membership):
    """Argmax slot per player, -1 when in no slot (hier_masks.py:94-98)."""
    any_g = membership.any(dim=1)
    labels = membership.to(dtype=torch.long).argmax(dim=1)
    return torch.where(any_g, labels, torch.full_like(labels, -1))


def _slice_hier_active_group_for_cached_mask(active_group, start_frame: int, num_frames: int):
    """Current-block slice of a full-clip active tensor (hier_masks.py:101-124)."""
    if active_group is None:
        return None
    active = _squeeze_hier_batch(active_group, 2, "active_group")
    start, n = int(start_frame), int(num_frames)
    if start < 0 or n <= 0:
        raise ValueError(f"invalid cached active_group slice: start={start}, n={n}")
    if active.shape[0] == n:
        return active.contiguous()
    if start + n > active.shape[0]:
        raise ValueError(
            f"active_group T={active.shape[0]} does not cover cached block [{start},{start + n})")
    return active[start:start + n].contiguous()


def _prepare_hier_membership_tensors(membership, global_only, active_group, num_players,
                                     num_frames, num_groups, device, *, allow_full_t=False):
    """membership [T,N,P], global_only [T,P], active [T,N] (hier_masks.py:127-193)."""
    if membership is None:
        raise ValueError("hier_group_format=membership requires membership [T,N,P] or [1,T,N,P]")
    mem = _squeeze_hier_batch(membership, 3, "membership")
    T, N, P = (int(x) for x in mem.shape)
    if P != num_players:
        raise ValueError(
            f"membership P={P} must equal num_players={num_players}, got {tuple(mem.shape)}")
    if N != num_groups:
        raise ValueError(
            f"membership N={N} must equal num_groups={num_groups}, got {tuple(mem.shape)}")
    if num_frames is not None:
        if allow_full_t:
            if T < int(num_frames):
                raise ValueError(f"membership T={T} shorter than current block n={int(num_frames)}")
        elif T != int(num_frames):
            raise ValueError(
                f"membership must be [T={int(num_frames)},N={num_groups},P={num_players}], "
                f"got {tuple(mem.shape)}")
    mem = mem.to(device=device, dtype=torch.bool).contiguous()
    if global_only is None:
        raise ValueError("hier_group_format=membership requires global_only [T,P] or [1,T,P]")
    go = _squeeze_hier_batch(global_only, 2, "global_only")
    if go.shape != (T, P):
        raise ValueError(f"global_only must be [T={T},P={P}], got {tuple(go.shape)}")
    go = go.to(device=device, dtype=torch.bool).contiguous()
    if active_group is None:
        active = mem.any(dim=-1)
    else:
        active = _squeeze_hier_batch(active_group, 2, "active_group")
        if allow_full_t and active.shape != (T, N):
            active = mem.any(dim=-1).contiguous()
        elif active.shape != (T, N):
            raise ValueError(f"active_group must be [T={T},N={N}], got {tuple(active.shape)}")
        else:
            active = active.to(device=device, dtype=torch.bool).contiguous()
    return mem, go, active


def _refuse_membership_on_scalar_kernel(*, attn_impl: Optional[str] = None,
                                        infer_kernel: Optional[str] = None):
    """The reference's scalar-label kernels refuse membership (hier_masks.py:196-207).

    This package's kernels all accept membership; the guard is kept for callers
    that select the reference's scalar backends by name.
    """
    if attn_impl == "hier_tiled_ste":
        raise ValueError(
            "hier_group_format=membership is not supported with attn_impl=hier_tiled_ste; use "
            "--attn_impl hier_amd (membership-capable)")
    if infer_kernel in ("segmented", "tiled128"):
        raise ValueError(
            f"hier_group_format=membership is not supported with WAN_HIER_INFER_KERNEL={infer_kernel}; "
            "use hier_amd or paged_kv")


def _validate_hier_no_local_topology(no_local: bool, KL: int, KG: int) -> None:
    """hier_masks.py:210-214."""
    if bool(no_local) and (int(KL) != 0 or int(KG) <= 0):
        raise ValueError(f"hier_no_local_hub requires K_L=0 and K_G>0; got K_L={KL}, K_G={KG}")


def build_hier_query_active_mask(*, active_group, num_players, num_frames, num_patches, num_groups,
                                 num_local_hub_tokens, num_global_hub_tokens, device, dtype):
    """[1,S,1] row mask, zero only on inactive local-hub query rows
    (hier_tiled_attention.py:432-459)."""
    P, T, L = int(num_players), int(num_frames), int(num_patches)
    N, KL, KG = int(num_groups), int(num_local_hub_tokens), int(num_global_hub_tokens)
    if tuple(active_group.shape) != (T, N):
        raise ValueError(f"active_group must have shape {(T, N)}, got {tuple(active_group.shape)}")
    agent = torch.ones(P * T * L, device=device, dtype=dtype)
    local = active_group.to(device=device, dtype=dtype).reshape(T, N, 1).expand(T, N, KL).reshape(-1)
    glob = torch.ones(T * KG, device=device, dtype=dtype)
    return torch.cat((agent, local, glob), dim=0).view(1, -1, 1)
