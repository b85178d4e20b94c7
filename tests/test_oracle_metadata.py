"""The CPU oracle's metadata restatement against the reference's golden vectors."""

import pytest

from oracle.metadata import (
    CachedTopology,
    segmented_metadata,
    tiled_cached_layout,
    tiled_full_sequence_layouts,
)
from tests import golden_io as G


def topo_from(inp: dict) -> CachedTopology:
    tup = lambda x: None if x is None else tuple(tuple(r) if isinstance(r, list) else r for r in x)
    mem = inp.get("membership")
    return CachedTopology(
        P=inp["P"], N=inp["N"], L=inp["L"], KL=inp["KL"], KG=inp["KG"],
        n_frames=inp["n_frames"], n_block=inp["n_block"], local_attn=inp["local_attn"],
        agent_frames=tup(inp["agent_frames"]), local_frames=tup(inp["local_frames"]),
        global_frames=tuple(inp["global_frames"]), local_active=tup(inp["local_active"]),
        labels=tup(inp["labels"]), q_active=tup(inp["q_active"]), direct=bool(inp["direct"]),
        membership=None if mem is None else tuple(tuple(tuple(g) for g in t) for t in mem),
        global_only=tup(inp.get("global_only")), no_local=bool(inp.get("no_local", False)),
    )


@pytest.mark.parametrize("name", G.cases("seg"))
def test_segmented_matches_reference_golden(name):
    inp = G.inputs("seg", name)
    out = segmented_metadata(topo_from(inp), inp["block_m"])
    for f in ("prog_qbase", "prog_nq", "prog_seg", "kv_index", "kv_count"):
        G.assert_same(f"seg/{name}/{f}", out[f])
    assert out["logical_pairs"] == G.scalar(f"seg/{name}/logical_pairs")


@pytest.mark.parametrize("name", G.cases("tc"))
def test_tiled_cached_matches_reference_golden(name):
    inp = G.inputs("tc", name)
    out = tiled_cached_layout(topo_from(inp))
    for f in ("prog_qbase", "prog_nq", "prog_seg", "kv_index", "kv_valid", "kv_count"):
        G.assert_same(f"tc/{name}/{f}", out[f])
    for f in ("logical_slots", "physical_slots", "dense_slots"):
        assert out[f] == G.scalar(f"tc/{name}/{f}")


@pytest.mark.parametrize("name", G.cases("tf"))
def test_tiled_full_sequence_matches_reference_golden(name):
    inp = G.inputs("tf", name)
    lays = tiled_full_sequence_layouts(inp["P"], inp["T"], inp["L"], inp["N"], inp["KL"],
                                       inp["KG"], inp["n"], inp["window"], inp["labels"],
                                       inp["active"], inp["direct"])
    assert len(lays) == G.scalar(f"tf/{name}/num_blocks")
    for b, out in enumerate(lays):
        for f in ("prog_qbase", "prog_nq", "prog_seg", "kv_index", "kv_valid", "kv_count"):
            G.assert_same(f"tf/{name}/{b}/{f}", out[f])
        for f in ("logical_slots", "physical_slots", "dense_slots"):
            assert out[f] == G.scalar(f"tf/{name}/{b}/{f}")
