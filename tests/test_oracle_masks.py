"""The dense-mask oracle: hand-asserted edges and edge equality with golden metadata.

The single-edge assertions restate the cases of the reference tests
tests/test_hier_flexible_membership_mask.py:156-347 and
tests/test_hier_no_local_hub.py:58-95 (inputs and expected booleans); the
set-equality tests repeat tests/test_hier_tiled_layout.py:30-95 against the
reference's golden Tiled128 layouts and extend it to the golden membership
segmented lists.
"""

import numpy as np
import pytest

from oracle.masks import FullTopology, inactive_local_rows, mask_rows
from tests import golden_io as G


def tok(P, T, L, N, KL, KG, kind, p=0, g=0, t=0, k=0):
    agent = P * T * L
    if kind == "player":
        return p * T * L + t * L + k
    if kind == "local":
        return agent + t * N * KL + g * KL + k
    return agent + T * N * KL + t * KG + k


def dense(P, T, L, N, KL, KG, n, w, labels=None, mem=None, go=None, direct=True, active=None,
          no_local=False):
    if mem is not None and go is None:
        go = np.zeros((T, P), dtype=bool)
    if labels is None and mem is None:
        labels = np.zeros((T, P), dtype=np.int64)
    topo = FullTopology(P, T, L, N, KL, KG, n, w, direct, labels=labels, active=active,
                        membership=mem, global_only=go, no_local=no_local)
    return mask_rows(topo)


def test_labels_partition_equals_membership_onehot():
    P, T, L, N, KL, KG, n = 4, 3, 2, 2, 1, 1, 3
    labels = np.array([[0, 0, 1, 1]] * T)
    mem = np.zeros((T, N, P), dtype=bool)
    mem[np.arange(T)[:, None], labels, np.arange(P)[None, :]] = True
    m_lab = dense(P, T, L, N, KL, KG, n, 7, labels=labels)
    m_mem = dense(P, T, L, N, KL, KG, n, 7, mem=mem)
    assert np.array_equal(m_lab, m_mem)
    t = lambda *a, **k: tok(P, T, L, N, KL, KG, *a, **k)
    assert not m_mem[t("player", p=0), t("global")]
    assert not m_mem[t("global"), t("player", p=0)]


def test_p4_mixed_global_only_and_empty_slot():
    P, T, L, N, KL, KG, n = 4, 3, 2, 2, 1, 1, 3
    mem = np.zeros((T, N, P), dtype=bool)
    mem[:, 0, 1] = mem[:, 0, 2] = True
    go = np.zeros((T, P), dtype=bool)
    go[:, 0] = go[:, 3] = True
    m = dense(P, T, L, N, KL, KG, n, 7, mem=mem, go=go)
    t = lambda *a, **k: tok(P, T, L, N, KL, KG, *a, **k)
    assert m[t("player", p=1), t("local", g=0)]
    assert not m[t("player", p=1), t("local", g=1)]
    assert m[t("local", g=0), t("player", p=2)]
    assert m[t("player", p=0), t("global")] and m[t("global"), t("player", p=0)]
    assert m[t("player", p=3), t("global")]
    assert not m[t("player", p=0), t("local", g=0)] and not m[t("player", p=0), t("local", g=1)]
    assert not m[t("player", p=1), t("global")] and not m[t("global"), t("player", p=1)]
    assert not m[t("player", p=0), t("player", p=1)]
    assert m[t("player", p=1), t("player", p=2)]
    assert not m[t("local", g=1), t("global")] and not m[t("global"), t("local", g=1)]
    assert m[t("local", g=1), t("local", g=1)]
    assert not m[t("local", g=1), t("player", p=1)]


def test_p4_all_global_only_both_slots_inactive():
    P, T, L, N, KL, KG, n = 4, 3, 2, 2, 1, 1, 3
    mem = np.zeros((T, N, P), dtype=bool)
    go = np.ones((T, P), dtype=bool)
    m = dense(P, T, L, N, KL, KG, n, 7, mem=mem, go=go)
    t = lambda *a, **k: tok(P, T, L, N, KL, KG, *a, **k)
    for p in range(P):
        assert m[t("player", p=p), t("global")] and m[t("global"), t("player", p=p)]
        assert not m[t("player", p=p), t("local", g=0)] and not m[t("player", p=p), t("local", g=1)]
    for g in range(N):
        assert not m[t("local", g=g), t("global")] and not m[t("global"), t("local", g=g)]
        assert m[t("local", g=g), t("local", g=g)]


def test_p10_anchor_shares_two_locals_no_cross_member_direct():
    P, T, L, N, KL, KG, n = 10, 3, 2, 4, 1, 1, 3
    mem = np.zeros((T, N, P), dtype=bool)
    mem[:, 0, 0] = mem[:, 1, 0] = mem[:, 0, 1] = mem[:, 1, 2] = True
    go = np.zeros((T, P), dtype=bool)
    go[:, 3] = True
    m = dense(P, T, L, N, KL, KG, n, 7, mem=mem, go=go)
    t = lambda *a, **k: tok(P, T, L, N, KL, KG, *a, **k)
    assert m[t("player", p=0), t("local", g=0)] and m[t("player", p=0), t("local", g=1)]
    assert not m[t("player", p=0), t("local", g=2)]
    assert m[t("player", p=0), t("player", p=1)] and m[t("player", p=0), t("player", p=2)]
    assert not m[t("player", p=1), t("player", p=2)]
    assert not m[t("player", p=0), t("global")]
    assert m[t("player", p=3), t("global")] and m[t("global"), t("player", p=3)]
    labels = mem.astype(np.int64).argmax(1)
    m_lab = dense(P, T, L, N, KL, KG, n, 7, labels=labels)
    assert not m_lab[t("player", p=0), t("local", g=1)]


def test_labels_mode_rejects_negative_ids():
    with pytest.raises(ValueError, match=r"must be in \[0,2\)"):
        dense(4, 3, 2, 2, 1, 1, 3, 7, labels=np.array([[-1, 0, 0, 1]] * 3))


def test_own_history_always_on():
    P, T, L, N = 4, 3, 2, 2
    m = dense(P, T, L, N, 1, 1, 3, 7, mem=np.zeros((T, N, P), bool), go=np.ones((T, P), bool))
    t0 = tok(P, T, L, N, 1, 1, "player", p=2, t=0)
    t1 = tok(P, T, L, N, 1, 1, "player", p=2, t=1)
    assert m[t1, t0] and m[t0, t0]


def test_no_local_topology_edges_and_global_only_invariance():
    """K_L=0: every player <-> global within the window; global_only is ignored."""
    P, T, L, N, KL, KG, n, w = 3, 4, 2, 2, 0, 2, 2, 4
    labels = np.array([[0, 0, 1]] * T)
    m = dense(P, T, L, N, KL, KG, n, w, labels=labels, no_local=True)
    t = lambda *a, **k: tok(P, T, L, N, KL, KG, *a, **k)
    for p in range(P):
        assert m[t("player", p=p, t=1), t("global", t=0)]
        assert m[t("global", t=1), t("player", p=p, t=0)]
        assert not m[t("player", p=p, t=0), t("global", t=2)]      # future block
    mem = np.zeros((T, N, P), dtype=bool)
    mem[np.arange(T)[:, None], labels, np.arange(P)[None, :]] = True
    a = dense(P, T, L, N, KL, KG, n, w, mem=mem, go=np.zeros((T, P), bool), no_local=True)
    b = dense(P, T, L, N, KL, KG, n, w, mem=mem, go=np.ones((T, P), bool), no_local=True)
    assert np.array_equal(a, b)
    with pytest.raises(ValueError):
        dense(P, T, L, N, 1, KG, n, w, labels=labels, no_local=True)


def _golden_edges(prefix):
    kv_index = G.golden()[f"{prefix}/kv_index"]
    if kv_index.dtype.kind == "U":
        return None
    kv_valid = G.golden()[f"{prefix}/kv_valid"].astype(bool)
    kv_count = G.golden()[f"{prefix}/kv_count"]
    rows = {}
    for base, nq, seg in zip(G.golden()[f"{prefix}/prog_qbase"], G.golden()[f"{prefix}/prog_nq"],
                             G.golden()[f"{prefix}/prog_seg"]):
        c = int(kv_count[seg])
        keys = set(kv_index[seg, :c][kv_valid[seg, :c]].tolist())
        for q in range(int(base), int(base) + int(nq)):
            rows[q] = keys
    return rows


@pytest.mark.parametrize("name", [n for n in G.cases("tf") if not n.startswith("c2")])
def test_dense_mask_equals_golden_tiled_full_sequence_edges(name):
    inp = G.inputs("tf", name)
    topo = FullTopology(inp["P"], inp["T"], inp["L"], inp["N"], inp["KL"], inp["KG"], inp["n"],
                        inp["window"], inp["direct"], labels=np.array(inp["labels"]),
                        active=np.array(inp["active"]))
    m = mask_rows(topo)
    inactive = inactive_local_rows(topo)
    rows = {}
    for b in range(G.scalar(f"tf/{name}/num_blocks")):
        rows.update(_golden_edges(f"tf/{name}/{b}"))
    assert len(rows) == topo.S
    for q in range(topo.S):
        if inactive[q]:
            assert rows[q] == set()
        else:
            assert rows[q] == set(np.nonzero(m[q])[0].tolist()), q


def _cached_to_full(inp, T):
    P, N, L, KL, KG = inp["P"], inp["N"], inp["L"], inp["KL"], inp["KG"]
    frames = inp["agent_frames"][0]
    fa = len(frames)
    agent_pool, local_pool = P * fa * L, N * fa * KL
    local_start = P * T * L
    global_start = local_start + T * N * KL

    def f(i):
        if i < agent_pool:
            p, r = divmod(i, fa * L)
            fi, k = divmod(r, L)
            return (p * T + frames[fi]) * L + k
        if i < agent_pool + local_pool:
            g, r = divmod(i - agent_pool, fa * KL)
            fi, k = divmod(r, KL)
            return local_start + (frames[fi] * N + g) * KL + k
        fi, k = divmod(i - agent_pool - local_pool, KG)
        return global_start + frames[fi] * KG + k
    return f


@pytest.mark.parametrize("name", [n for n in G.cases("seg")
                                  if n.startswith("mem_") or n.startswith("fx_")])
def test_dense_membership_mask_equals_golden_segmented_edges(name):
    """Cached membership key sets == the dense membership mask rows of the block."""
    inp = G.inputs("seg", name)
    P, N, L, KL, KG, n = inp["P"], inp["N"], inp["L"], inp["KL"], inp["KG"], inp["n_frames"]
    mem = np.array(inp["membership"], dtype=bool)
    go = np.array(inp["global_only"], dtype=bool)
    T = mem.shape[0]
    frames = inp["agent_frames"][0]
    assert all(x == frames for x in inp["agent_frames"]) and inp["global_frames"] == frames
    qframes = frames[-n:]
    topo = FullTopology(P, T, L, N, KL, KG, inp["n_block"], inp["local_attn"], inp["direct"],
                        membership=mem, global_only=go)
    to_full = _cached_to_full(inp, T)
    kv_index = G.golden()[f"seg/{name}/kv_index"]
    kv_count = G.golden()[f"seg/{name}/kv_count"]
    local_start = P * T * L
    global_start = local_start + T * N * KL
    seg = 0
    specs = []
    for p in range(P):
        for qf in qframes:
            specs.append([(p * T + qf) * L + i for i in range(L)])
    for qf in qframes:
        for g in range(N):
            specs.append([local_start + (qf * N + g) * KL + i for i in range(KL)])
    for qf in qframes:
        specs.append([global_start + qf * KG + i for i in range(KG)])
    inactive = inactive_local_rows(topo)
    for seg, rows in enumerate(specs):
        keys = {to_full(int(i)) for i in kv_index[seg, :int(kv_count[seg])]}
        if not rows:
            continue
        m = mask_rows(topo, q_idx=np.array(rows))
        for r, q in enumerate(rows):
            expected = set() if inactive[q] else set(np.nonzero(m[r])[0].tolist())
            assert keys == expected, (name, seg, q)
