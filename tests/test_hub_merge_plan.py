"""Host plan of the hub merge and the tail fold (``metadata._HubMerge``), on
the CPU: the item lists it describes own every query row exactly once, the
folded rows carry mask bits of their own above their hub's frames, and only
members' last items are folded.

The device kernels' output items are restated from the plan (each group's
rows split into items of up to 128 rows, as ``merge_compact_kernel`` writes
them) and the built list's items from the topology (each (block, stream)
group's rows split the same way, as ``meta_build_kernel`` writes them).
"""

import numpy as np
import pytest
import torch

from multics_amd import metadata as M

RPI = 128


def _built(topo):
    """Per (block, stream): items [qbase, qstride, qlen, r0, rc, group, 0, n]
    in the builder's order, item_start, nit, and a nonzero list size."""
    P, N, n, B = topo.P, topo.N, topo.n_frames, topo.B
    NS = P + N + 1
    nit = np.zeros((B, NS), np.int64)
    for b in range(B):
        for s in range(NS):
            nit[b, s] = -(-n * M._qlen(topo, s) // RPI)
    item_start = np.zeros((B, NS), np.int64)
    items, cur = [], 0
    for s, b in M._item_order(P, N, B):
        item_start[b, s] = cur
        ql = M._qlen(topo, s)
        kind = 0 if s < P else (1 if s < P + N else 2)
        rows = n * ql
        for i in range(int(nit[b, s])):
            items.append([topo.tile_qbase[b][s], topo.tile_qstride[kind], ql, i * RPI,
                          min(RPI, rows - i * RPI), b * NS + s, 0, n])
        cur += int(nit[b, s])
    tile_h = np.where(nit > 0, 64, 0)
    return np.asarray(items, np.int64).reshape(-1, 8), item_start, nit, tile_h


def _merge_items(plan):
    """The items ``merge_compact_kernel`` writes for the plan's groups."""
    desc = plan._dev["group_desc"].numpy().reshape(-1, 4)
    out = []
    for g, (qb, qs, ql, fr) in enumerate(desc):
        rows = ql * fr
        for i in range(-(-rows // RPI)):
            out.append([qb, qs, ql, i * RPI, min(RPI, rows - i * RPI), -1 - g, 0, fr])
    return np.asarray(out, np.int64).reshape(-1, 8)


def _owners(items, table):
    own = {}
    for qb, qs, ql, r0, rc, src, _, nf in items:
        for r in range(r0, r0 + rc):
            if qs < 0:
                tok, bit = (int(x) for x in table[qb + r])
            else:
                bit, i = divmod(r, ql)
                tok = qb + bit * qs + i
            assert tok not in own, f"row {tok} owned twice"
            own[tok] = (int(src), bit)
    return own


def _topo(kind):
    P, T, L, N, KL, KG, n, W = 4, 12, 50, 2, 5, 6, 3, 6
    rng = np.random.default_rng(5)
    if kind == "labels":
        labels = np.array([[p // 2 for p in range(P)]] * T)
        return M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                        direct=True, labels=labels)
    mem = np.repeat(rng.random((T // n, N, P)) < 0.5, n, axis=0)
    return M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W, direct=True,
                                    membership=mem, global_only=~mem.any(1))


@pytest.mark.parametrize("G", [1, 2])
@pytest.mark.parametrize("kind", ["labels", "membership"])
def test_fold_plan_owns_every_row_once(kind, G):
    topo = _topo(kind)
    P, N, n, L = topo.P, topo.N, topo.n_frames, topo.L
    S = M.group_rows_cover(topo)[0]
    built, item_start, nit, tile_h = _built(topo)
    n_items = len(built)
    plan = M._HubMerge(topo, G, tile_h, item_start, nit, int(tile_h.sum()), n_items, RPI, S,
                       torch.device("cpu"), fold_tails=True)
    out = _merge_items(plan)
    assert len(out) == plan.n_out_items
    kept = built[plan.first_player:]
    shared = np.concatenate([out[:plan.n_items], kept]) if plan.merge else built
    assert sorted(_owners(shared, None)) == list(range(S))
    assert plan.fwd_index is not None and plan.folded_tails > 0
    table = plan.row_table.numpy()
    fwd = np.concatenate([out, kept])[plan.fwd_index.numpy()]
    assert len(fwd) == plan.fwd_n_items
    own = _owners(fwd, table)
    assert sorted(own) == list(range(S))
    # the folded rows: a player's last item (n * L mod 128 rows) under bits
    # of its own above its hub's frames, in a group whose hub it belongs to
    tail_rows = n * L % RPI
    src_group = plan._dev["src_group"].numpy()
    src_from = plan._dev["src_from"].numpy()
    src_nbits = plan._dev["src_nbits"].numpy()
    src_shift = plan._dev["src_shift"].numpy()
    src_item = plan._dev["src_item"].numpy()
    desc = plan._dev["group_desc"].numpy().reshape(-1, 4)
    T = topo.B * n
    folded = 0
    for g in range(plan.n_groups, plan.n_all_groups):
        qb, qs, one, rows = desc[g]
        assert qs == -1 and one == 1
        hub_tok = int(table[qb, 0])
        slot = (hub_tok - P * T * L) // topo.KL % N          # the local hub's group slot
        srcs = np.nonzero(src_group == g)[0]
        hub_frames = n * int((src_nbits[srcs] == 32).sum())
        assert (table[qb:qb + hub_frames * topo.KL, 1] < hub_frames).all()
        for i in srcs:
            it = built[src_item[i]]
            if src_nbits[i] == 32:                                  # a hub block's list
                assert src_from[i] == 0 and it[1] == topo.tile_qstride[1]
                continue
            folded += 1
            qb_p = it[0]
            p = qb_p // (T * L)
            b = (qb_p - p * T * L) // (n * L)
            assert src_from[i] == (n * L - tail_rows) // L
            assert hub_frames <= src_shift[i] and src_shift[i] + src_nbits[i] <= 32
            for f in range(src_from[i], src_from[i] + src_nbits[i]):
                assert M._member(topo, b, f, slot, p)
            # its rows sit in the table under bits shift + (frame - from)
            base = qb_p + (n * L - tail_rows)
            for r in range(tail_rows):
                tok = base + r
                fr = (n * L - tail_rows + r) // L
                assert own[tok][1] == src_shift[i] + fr - src_from[i]
    assert folded == plan.folded_tails


def test_fold_plan_respects_the_item_capacity():
    """A group takes a tail only while its rows fit the items it already
    has: 30 hub rows + 4 x 20 = 110 <= 128 at the C2 geometry, a fifth
    member's tail stays where it was."""
    P, T, L, N, KL, KG, n, W = 6, 6, 220, 1, 5, 6, 3, 6
    topo = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                    direct=True, labels=np.zeros((T, P), int))
    built, item_start, nit, tile_h = _built(topo)
    S = M.group_rows_cover(topo)[0]
    plan = M._HubMerge(topo, 2, tile_h, item_start, nit, int(tile_h.sum()), len(built), RPI, S,
                       torch.device("cpu"), fold_tails=True)
    desc = plan._dev["group_desc"].numpy().reshape(-1, 4)
    for g in range(plan.n_groups, plan.n_all_groups):
        assert desc[g][3] <= RPI                        # no group grows an item
    # one local hub group (two blocks), 12 member tails, room for 4
    assert plan.folded_tails == 4
