"""Checks of label payloads: the generated 24-field schema (shapes, dtypes,
the generation profile's constants, the period / latent mapping, every derived
field against ``period_membership``, each period's topology, pair accounting
and costs), and the looser rules for existing membership files
(multics/grouping/validation.py:1-174).  The error messages are the
reference's, for drop-in error handling."""

from __future__ import annotations

import torch

from .budget import resolve
from .partition import topology_constraints_hold

LABEL_FIELDS = frozenset("""
membership global_only eligible labels latent_period period_membership
period_global_only period_anchor period_labels period_start period_frames
period_scores period_sizes period_cohesion period_pair_used period_total_cost
clip_total_cost cost_limit coverage orphan_ratio anchor_ratio pair_budget
max_groups max_size
""".split())
CORE_FIELDS = frozenset(("membership", "global_only", "eligible", "labels"))

LATENT_FRAMES = 42
PERIODS = 4
PERIOD_START = [0, 48, 96, 144]
PERIOD_FRAMES = [48, 48, 48, 21]
LATENTS_PER_PERIOD = 12


def _schema(t: int, g: int, p: int, k: int) -> dict:
    b, i8, i16, i32, f32, f64 = (torch.bool, torch.int8, torch.int16, torch.int32,
                                  torch.float32, torch.float64)
    return {
        "membership": ((t, g, p), b), "global_only": ((t, p), b), "eligible": ((p,), b),
        "labels": ((t, p), i8), "latent_period": ((t,), i16),
        "period_membership": ((k, g, p), b), "period_global_only": ((k, p), b),
        "period_anchor": ((k, p), b), "period_labels": ((k, p), i8),
        "period_start": ((k,), i32), "period_frames": ((k,), i32),
        "period_scores": ((k, g), f32), "period_sizes": ((k, g), i8),
        "period_cohesion": ((k, g), f32), "period_pair_used": ((k,), i32),
        "period_total_cost": ((k,), f32), "clip_total_cost": ((), f64), "cost_limit": ((), f64),
        "coverage": ((k,), f32), "orphan_ratio": ((k,), f32), "anchor_ratio": ((k,), f32),
        "pair_budget": ((), i32), "max_groups": ((), i32), "max_size": ((), i32),
    }


def _argmax_labels(mem: torch.Tensor) -> torch.Tensor:
    """Slot of each player (the lowest of its slots) or -1: ``[..., G, P] -> [..., P]``."""
    return torch.where(mem.any(-2), mem.long().argmax(-2), -1)


def validate_generated_labels(payload, num_players: int) -> None:
    budget = resolve(num_players)
    t, g, p, k = LATENT_FRAMES, budget.groups, num_players, PERIODS
    schema = _schema(t, g, p, k)
    if not isinstance(payload, dict) or set(payload) != set(schema):
        raise ValueError("Generated grouping must contain exactly the 24 expected tensor fields")
    for name, (shape, dtype) in schema.items():
        v = payload[name]
        if not torch.is_tensor(v) or tuple(v.shape) != shape or v.dtype != dtype:
            raise ValueError(f"Invalid generated grouping field {name}: expected {shape}/{dtype}")
        if not torch.isfinite(v).all():
            raise ValueError(f"Non-finite generated grouping field {name}")
    for name, want in (("max_groups", g), ("max_size", budget.max_size),
                       ("pair_budget", budget.pair_budget), ("cost_limit", budget.cost_limit)):
        if payload[name].item() != want:
            raise ValueError(f"Generated grouping {name} disagrees with the label-generation profile")
    if not payload["eligible"].all():
        raise ValueError("All selected players must be eligible for the training/inference clip")
    if (payload["period_start"].tolist() != PERIOD_START
            or payload["period_frames"].tolist() != PERIOD_FRAMES):
        raise ValueError("Invalid generated grouping periods")
    idx = torch.arange(t) // LATENTS_PER_PERIOD
    if not torch.equal(payload["latent_period"].long(), idx):
        raise ValueError("Invalid latent-to-period mapping")
    mem = payload["period_membership"]
    has = mem.any(1)
    counts = mem.sum(1)
    labels = _argmax_labels(mem).to(torch.int8)
    derived = {
        "membership": mem[idx], "global_only": (~has)[idx], "period_global_only": ~has,
        "labels": labels[idx], "period_labels": labels, "period_anchor": counts > 1,
        "period_sizes": mem.sum(2).to(torch.int8),
        "coverage": has.sum(1).float() / p, "orphan_ratio": (~has).sum(1).float() / p,
        "anchor_ratio": (counts > 1).sum(1).float() / p,
    }
    for name, want in derived.items():
        if not torch.equal(payload[name], want):
            raise ValueError(f"Inconsistent generated grouping field {name}")
    for i, frame in enumerate(mem):
        groups = [torch.nonzero(row).flatten().tolist() for row in frame if row.any()]
        if not topology_constraints_hold(groups, player_count=p, max_groups=g,
                                         max_size=budget.max_size, pair_budget=budget.pair_budget,
                                         budget=budget):
            raise ValueError(f"Invalid grouping topology at period {i}")
        if payload["period_pair_used"][i] != budget.direct_pair_units(groups):
            raise ValueError("Incorrect grouping pair accounting")
        cost = torch.tensor(budget.topology_cost(groups), dtype=torch.float32)
        if not torch.equal(payload["period_total_cost"][i], cost):
            raise ValueError("Incorrect grouping period cost")
    cost = budget.topology_cost_timeline(payload["membership"].numpy(), payload["global_only"].numpy())
    if payload["clip_total_cost"].item() != cost or cost > budget.cost_limit:
        raise ValueError("Incorrect or over-budget grouping timeline cost")


def validate_existing_labels(payload) -> None:
    """Membership files made elsewhere: consistent core tensors; a full
    payload of a supported profile is checked as generated, other profiles
    only for finiteness and their own budget."""
    if not isinstance(payload, dict):
        raise ValueError("Grouping labels must be a tensor dictionary")
    if "membership" not in payload:
        return      # labels-only files are checked by their loader
    for name in ("membership", "global_only", "eligible"):
        v = payload.get(name)
        if not torch.is_tensor(v) or v.dtype != torch.bool:
            raise ValueError(f"Membership grouping requires a boolean tensor {name}")
    mem, go, eligible = payload["membership"], payload["global_only"], payload["eligible"]
    if mem.ndim != 3 or go.shape != (mem.shape[0], mem.shape[2]) or eligible.shape != (mem.shape[2],):
        raise ValueError("Inconsistent membership/global_only/eligible shapes")
    has = mem.any(1)
    if not torch.equal(go, eligible.unsqueeze(0) & ~has) or (has & ~eligible).any():
        raise ValueError("Contradictory membership/global_only/eligible tensors")
    if "labels" in payload:
        lab = payload["labels"]
        if (not torch.is_tensor(lab)
                or lab.dtype not in (torch.int8, torch.int16, torch.int32, torch.int64)
                or not torch.equal(lab, _argmax_labels(mem))):
            raise ValueError("Grouping labels disagree with membership")
    if set(payload) & (LABEL_FIELDS - CORE_FIELDS):
        if set(payload) != LABEL_FIELDS:
            raise ValueError("Partial grouping payload: all 24 fields are required")
        if mem.shape[2] in (4, 6, 8, 10) and mem.shape[0] == LATENT_FRAMES:
            validate_generated_labels(payload, int(mem.shape[2]))
            return
        for name, v in payload.items():
            if not torch.is_tensor(v) or not torch.isfinite(v).all():
                raise ValueError(f"Invalid existing grouping field {name}")
        if payload["clip_total_cost"].numel() != 1 or payload["cost_limit"].numel() != 1:
            raise ValueError("Existing label costs must be scalar")
        if payload["clip_total_cost"].item() > payload["cost_limit"].item():
            raise ValueError("Existing grouping exceeds its communication budget")
