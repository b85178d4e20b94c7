"""STE classes of the forward tile list (``metadata.ste_classes_host``), on
the CPU: the input of the backward's dQ pass when it sums the membership
straight-through gradient.

On forward lists written from the dense oracle mask (``synth_forward_tiles``),
an entry (key k of a group's list) carries a class exactly when its edges to
the group's query rows are gated by a membership bit in ``oracle.ste``'s
definition (``gate_index``), and the class names that bit: the group g of
a player row's bit (t, g, p), the player p of a local-hub row's bit; t is the
query row's frame.  Every gated edge of the dense mask is covered once, and
the selection is the STE list's (``ste_tiles_host``) in forward-list order.
"""

import numpy as np
import pytest

from multics_amd import metadata as M
from oracle.masks import FullTopology, inactive_local_rows, mask_rows
from oracle.ste import gate_index
from tests.test_transpose_tiles import synth_forward_tiles


def _topology(kind):
    rng = np.random.default_rng(11)
    P, T, L, N, KL, KG, n, W = 4, 6, 3, 3, 2, 2, 3, 4
    if kind == "labels":
        labels = rng.integers(0, N, size=(T, P))
        return FullTopology(P, T, L, N, KL, KG, n, W, True, labels=labels)
    mem = rng.random((T, N, P)) < (0.35 if kind == "membership" else 0.7)
    go = ~mem.any(1)
    if kind == "membership":
        go[0, 0] = False            # an orphan: no group, not global-only
    return FullTopology(P, T, L, N, KL, KG, n, W if kind == "membership" else -1, True,
                        membership=mem, global_only=go)


@pytest.mark.parametrize("kind", ["membership", "dense_unbounded", "labels"])
def test_classes_name_the_oracle_gating_bit(kind):
    topo = _topology(kind)
    P, T, L, N, KL = topo.P, topo.T, topo.L, topo.N, topo.KL
    tiles = synth_forward_tiles(topo)
    cls = M.ste_classes_host(tiles, P=P, T=T, L=L, N=N, KL=KL)
    gi = gate_index(topo)
    m = mask_rows(topo)
    dead = inactive_local_rows(topo)
    kind_, t_, p_, g_ = topo.token_ids(np.arange(topo.S))
    items = tiles.items.numpy().astype(np.int64)
    kv_idx = tiles.kv_idx.numpy().astype(np.int64)
    kv_mask = tiles.kv_mask.numpy().astype(np.int64) & 0xFFFFFFFF
    assert cls.dtype == np.int32 and cls.shape == kv_idx.shape
    covered = 0
    for qb, qs, ql, r0, rc, off, cnt, nf in items:
        if r0 != 0:
            continue
        for e in range(off, off + cnt):
            k, bits, c = kv_idx[e], kv_mask[e], int(cls[e])
            if bits == 0:
                assert c == -1
                continue
            for j in range(nf):
                if not (bits >> j) & 1:
                    continue
                for q in range(qb + j * qs, qb + j * qs + ql):
                    assert m[q, k] and not dead[q]
                    bit = gi[q, k]
                    if c < 0:
                        assert bit < 0, (q, k)
                        continue
                    t, g, p = np.unravel_index(bit, (T, N, P))
                    assert t == t_[q]
                    assert c == (g if kind_[q] == 0 else p), (q, k, c, t, g, p)
                    covered += 1
    gated = (gi >= 0) & m & ~dead[:, None]
    assert covered == int(gated.sum()) and covered > 0


@pytest.mark.parametrize("kind", ["membership", "dense_unbounded", "labels"])
def test_classes_select_the_ste_list(kind):
    topo = _topology(kind)
    geo = dict(P=topo.P, T=topo.T, L=topo.L, N=topo.N, KL=topo.KL)
    tiles = synth_forward_tiles(topo)
    cls = M.ste_classes_host(tiles, **geo)
    lst, lcls = M.ste_tiles_host(tiles, **geo)
    items = tiles.items.numpy().astype(np.int64)
    kv_idx = tiles.kv_idx.numpy()
    kv_mask = tiles.kv_mask.numpy()
    sit = lst.items.numpy().astype(np.int64)
    sidx, smask, scls = lst.kv_idx.numpy(), lst.kv_mask.numpy(), lcls.numpy()
    firsts = items[items[:, 3] == 0]
    sfirsts = sit[sit[:, 3] == 0]
    got = [(qb, o) for qb, o in zip(firsts[:, 0], firsts[:, 5])
           if (cls[o:o + firsts[firsts[:, 5] == o][0, 6]] >= 0).any()]
    assert [g[0] for g in got] == list(sfirsts[:, 0])
    for (qb, off), srow in zip(got, sfirsts):
        cnt = int(firsts[firsts[:, 5] == off][0, 6])
        sel = np.nonzero(cls[off:off + cnt] >= 0)[0] + off
        order = np.argsort(cls[sel], kind="stable")
        so, sn = int(srow[5]), len(sel)
        np.testing.assert_array_equal(kv_idx[sel][order], sidx[so:so + sn])
        np.testing.assert_array_equal(kv_mask[sel][order], smask[so:so + sn])
        np.testing.assert_array_equal(cls[sel][order], scls[so:so + sn])
        assert (smask[so + sn:so + int(srow[6])] == 0).all()       # the rest is padding


@pytest.mark.parametrize("kind", ["membership", "dense_unbounded", "labels"])
def test_first_tile_with_a_class(kind):
    topo = _topology(kind)
    tiles = synth_forward_tiles(topo)
    cls = M.ste_classes_host(tiles, P=topo.P, T=topo.T, L=topo.L, N=topo.N, KL=topo.KL)
    first = M.ste_first_tiles_host(tiles, cls)
    items = tiles.items.numpy().astype(np.int64)
    assert first.dtype == np.int32 and len(first) == len(items)
    for f, (off, cnt) in zip(first, items[:, [5, 6]]):
        tiles_cls = cls[off:off + cnt].reshape(-1, 64)
        has = (tiles_cls >= 0).any(1)
        assert not has[:f].any()
        assert f == len(has) or has[f]
    assert (first < items[:, 6] // 64).any() and (first == items[:, 6] // 64).any()

