"""Write golden metadata vectors with the reference's own builders.

Run once in the build container (where the reference is mounted read-only at
/root/reference); the GPU box never runs this script and never reads the
reference.  Output: ``tests/golden/metadata_golden.npz`` -- per case a JSON
record of the inputs plus the exact arrays returned by

* ``_build_metadata``                      hier_segmented_attention.py:156-395
* ``build_hier_tiled_cached_layout``       hier_tiled_attention.py:474-655
* ``build_hier_tiled_full_sequence_layouts`` hier_tiled_attention.py:244-429

These functions' byte-level outputs (ordering, zero padding, MAX_K rounding,
program split, chunk selection) are pinned by nothing else, which is why they
are imported here.  Only the two kernel modules are loaded, by file path; they
need torch and the ``triton`` package for their decorators, not a GPU.

Usage: python tests/golden/make_golden.py [--ref /root/reference]
"""

from __future__ import annotations

import argparse
import hashlib
import importlib.util
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from tests.golden.cases import (  # noqa: E402
    full_sequence_cases,
    segmented_cases,
    tiled_cached_cases,
)


def _load(ref: Path, rel: str, name: str):
    spec = importlib.util.spec_from_file_location(name, ref / rel)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def _np(t):
    return t.detach().cpu().numpy() if torch.is_tensor(t) else np.asarray(t)


BIG = 50_000


def digest(arr) -> str:
    """sha256 over dtype, shape and C-order bytes (used for arrays too large to commit)."""
    a = np.ascontiguousarray(arr)
    h = hashlib.sha256()
    h.update(str(a.dtype).encode())
    h.update(str(tuple(a.shape)).encode())
    h.update(a.tobytes())
    return "sha256:" + h.hexdigest()


def _store(arrays, key, arr):
    arr = _np(arr)
    if arr.size > BIG:
        arrays[key] = np.asarray(digest(arr))
    else:
        arrays[key] = arr


def write_fixture_membership(ref: Path):
    """Copy membership/global_only rows of the reference grouping fixtures (data only)."""
    out = {}
    for name in ("p4_round_start", "p6_moving_pairs", "p10_moving_pairs"):
        d = np.load(ref / "tests/fixtures/grouping" / f"{name}.labels.npz", allow_pickle=False)
        out[f"{name}/membership"] = d["membership"].astype(bool)
        out[f"{name}/global_only"] = d["global_only"].astype(bool)
        out[f"{name}/labels"] = d["labels"].astype(np.int8)
    np.savez_compressed(HERE / "fixture_membership.npz", **out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--out", default=str(HERE / "metadata_golden.npz"))
    args = ap.parse_args()
    ref = Path(args.ref)
    write_fixture_membership(ref)
    seg = _load(ref, "multics/models/kernels/hier_segmented_attention.py", "_ref_seg")
    til = _load(ref, "multics/models/kernels/hier_tiled_attention.py", "_ref_tiled")

    arrays = {}
    index = []
    for name, case in segmented_cases():
        kw = dict(case)
        block_m = kw.pop("block_m")
        out = seg._build_metadata(
            device="cpu",
            P=kw["P"], N=kw["N"], L=kw["L"], KL=kw["KL"], KG=kw["KG"],
            n_frames=kw["n_frames"], n_block=kw["n_block"], local_attn=kw["local_attn"],
            agent_frame_lists=tuple(tuple(x) for x in kw["agent_frames"]),
            local_frame_lists=tuple(tuple(x) for x in kw["local_frames"]),
            global_frame_list=tuple(kw["global_frames"]),
            local_active_frames=tuple(tuple(bool(v) for v in x) for x in kw["local_active"]),
            labels=None if kw["labels"] is None else tuple(tuple(x) for x in kw["labels"]),
            q_active=tuple(tuple(bool(v) for v in x) for x in kw["q_active"]),
            direct_player=kw["direct"], block_m=block_m,
            membership=kw["membership"], global_only=kw["global_only"],
            hier_no_local_hub=kw["no_local"],
        )
        seg._META_CACHE.clear()
        for field, val in zip(("prog_qbase", "prog_nq", "prog_seg", "kv_index", "kv_count"), out[:5]):
            _store(arrays, f"seg/{name}/{field}", val)
        arrays[f"seg/{name}/logical_pairs"] = np.asarray(out[5], dtype=np.int64)
        arrays[f"seg/{name}/inputs"] = np.asarray(json.dumps(case))
        index.append(("seg", name))

    fields = ("prog_qbase", "prog_nq", "prog_seg", "kv_index", "kv_valid", "kv_count")
    scal = ("logical_slots", "physical_slots", "dense_slots")
    for name, case in tiled_cached_cases():
        kw = case
        lay = til.build_hier_tiled_cached_layout(
            device="cpu", P=kw["P"], N=kw["N"], L=kw["L"], KL=kw["KL"], KG=kw["KG"],
            n_frames=kw["n_frames"], n_block=kw["n_block"], local_attn=kw["local_attn"],
            agent_frame_lists=kw["agent_frames"], local_frame_lists=kw["local_frames"],
            global_frame_list=kw["global_frames"], local_active_frames=kw["local_active"],
            labels=kw["labels"], q_active=kw["q_active"], direct_player=kw["direct"],
        )
        til.clear_hier_tiled_layout_cache()
        for f in fields:
            _store(arrays, f"tc/{name}/{f}", getattr(lay, f))
        for f in scal:
            arrays[f"tc/{name}/{f}"] = np.asarray(getattr(lay, f), dtype=np.int64)
        arrays[f"tc/{name}/inputs"] = np.asarray(json.dumps(case))
        index.append(("tc", name))

    for name, case in full_sequence_cases():
        kw = case
        lays = til.build_hier_tiled_full_sequence_layouts(
            device="cpu", num_players=kw["P"], num_frames=kw["T"], num_patches=kw["L"],
            num_groups=kw["N"], num_local_hub_tokens=kw["KL"], num_global_hub_tokens=kw["KG"],
            num_frame_per_block=kw["n"], local_attn_size=kw["window"],
            group_labels=torch.tensor(kw["labels"], dtype=torch.long),
            active_group=torch.tensor(kw["active"], dtype=torch.bool),
            direct_player=kw["direct"],
        )
        til.clear_hier_tiled_layout_cache()
        arrays[f"tf/{name}/num_blocks"] = np.asarray(len(lays), dtype=np.int64)
        for b, lay in enumerate(lays):
            for f in fields:
                _store(arrays, f"tf/{name}/{b}/{f}", getattr(lay, f))
            for f in scal:
                arrays[f"tf/{name}/{b}/{f}"] = np.asarray(getattr(lay, f), dtype=np.int64)
        arrays[f"tf/{name}/inputs"] = np.asarray(json.dumps(case))
        index.append(("tf", name))

    arrays["index"] = np.asarray(json.dumps(index))
    np.savez_compressed(args.out, **arrays)
    print(f"wrote {len(index)} cases, {len(arrays)} arrays -> {args.out}")


if __name__ == "__main__":
    main()
