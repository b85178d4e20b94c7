"""Key-major tile list of the backward (``metadata.transpose_tiles``), on the CPU.

A forward tile list in the device builder's format is written here from the
dense oracle mask (whole key frames per query group, bitmask over the group's
query frames, 64-row padding); its transposition must list, for every key row,
exactly the query rows the dense mask lets see it (inactive local-hub query
rows excluded: their output is 0), and nothing else.
"""

import numpy as np
import pytest
import torch

from multics_amd import metadata as M
from oracle.masks import FullTopology, inactive_local_rows, mask_rows


def _groups(topo: FullTopology):
    P, T, L, N, KL, KG, n = topo.P, topo.T, topo.L, topo.N, topo.KL, topo.KG, topo.n
    a0, g0 = P * T * L, P * T * L + T * N * KL
    out = []
    for b in range(T // n):
        for p in range(P):
            out.append((p * T * L + b * n * L, L, L, n))
        for g in range(N):
            if KL:
                out.append((a0 + (b * n * N + g) * KL, N * KL, KL, n))
        if KG:
            out.append((g0 + b * n * KG, KG, KG, n))
    return out


def synth_forward_tiles(topo: FullTopology) -> M.TileList:
    m = mask_rows(topo)
    dead = inactive_local_rows(topo)
    groups = _groups(topo)
    units = [(qb + j * qs, ql) for qb, qs, ql, nf in groups for j in range(nf)]
    items, kv_idx, kv_mask, pairs = [], [], [], 0
    for qb, qs, ql, nf in groups:
        off = len(kv_idx)
        for kb, kl in units:
            bits = 0
            for j in range(nf):
                q0 = qb + j * qs
                if not dead[q0] and m[q0, kb]:
                    bits |= 1 << j
                    pairs += ql * kl
            if bits:
                kv_idx += list(range(kb, kb + kl))
                kv_mask += [bits] * kl
        pad = -len(kv_idx) % 64
        kv_idx += [0] * pad
        kv_mask += [0] * pad
        rows = nf * ql
        for r0 in range(0, rows, 128):
            items.append([qb, qs, ql, r0, min(128, rows - r0), off, len(kv_idx) - off, nf])
    idx = np.asarray(kv_idx, np.int64)
    msk = np.asarray(kv_mask, np.int64)
    blk = np.bitwise_and.reduce(msk.reshape(-1, 64), axis=1)
    as32 = lambda a: torch.from_numpy((a & 0xFFFFFFFF).astype(np.uint32).view(np.int32).copy())
    return M.TileList(items=torch.tensor(items, dtype=torch.int32), kv_idx=as32(idx),
                      kv_mask=as32(msk), blk_and=as32(blk), n_items=len(items), item_ranges=(),
                      logical_pairs=pairs, key_extent=topo.S, row_extent=topo.S,
                      rows_exact_cover=True)


def expand_key_major(kt: M.TileList, S: int) -> np.ndarray:
    seen = np.zeros((S, S), dtype=bool)      # [query, key]
    items = kt.items.numpy()
    idx = kt.kv_idx.numpy()
    msk = kt.kv_mask.numpy().view(np.uint32).astype(np.int64)
    for kb, ks, kl, r0, rc, off, cnt, nf in items:
        if r0 != 0:            # later items of a group share its list
            continue
        for r in range(nf * kl):
            f, i = divmod(r, kl)
            key = kb + f * ks + i
            sel = ((msk[off:off + cnt] >> f) & 1) == 1
            qs = idx[off:off + cnt][sel]
            assert not seen[qs, key].any(), "a (query, key) pair is listed twice"
            seen[qs, key] = True
    return seen


CASES = [
    # P, T, L, N, KL, KG, n, W, direct, kind
    (4, 6, 20, 2, 5, 6, 3, 4, True, "labels"),
    (4, 6, 20, 2, 5, 6, 3, -1, False, "labels"),
    (3, 4, 9, 2, 2, 3, 2, 3, True, "labels_inactive"),
    (6, 6, 7, 3, 2, 3, 3, 4, True, "membership"),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[-1]}_{i}" for i, c in enumerate(CASES)])
def test_transpose_matches_dense_mask(case):
    P, T, L, N, KL, KG, n, W, direct, kind = case
    rng = np.random.default_rng(3)
    if kind == "membership":
        mem = rng.random((T, N, P)) < 0.4
        go = ~mem.any(1) & (rng.random((T, P)) < 0.6)
        topo = FullTopology(P, T, L, N, KL, KG, n, W, direct, membership=mem, global_only=go)
    else:
        labels = rng.integers(0, N, size=(T, P))
        for b in range(T // n):
            labels[b * n:(b + 1) * n] = labels[b * n]
        active = np.zeros((T, N), dtype=bool)
        active[np.arange(T)[:, None], labels] = True
        if kind == "labels_inactive":
            active[:, -1] = False
        topo = FullTopology(P, T, L, N, KL, KG, n, W, direct, labels=labels, active=active)
    fwd = synth_forward_tiles(topo)
    kt = M.transpose_tiles(fwd)
    assert M.transpose_tiles(fwd) is kt                      # cached on the forward list
    assert kt.logical_pairs == fwd.logical_pairs
    assert kt.n_items == fwd.n_items
    assert (kt.kv_idx.numel() % 64) == 0
    want = mask_rows(topo) & ~inactive_local_rows(topo)[:, None]
    got = expand_key_major(kt, topo.S)
    assert np.array_equal(got, want)
    # blk_and is the AND of the masks of each 64 rows
    msk = kt.kv_mask.numpy().view(np.uint32)
    assert np.array_equal(np.bitwise_and.reduce(msk.reshape(-1, 64), axis=1),
                          kt.blk_and.numpy().view(np.uint32))


def test_transpose_rejects_partial_frames():
    topo = FullTopology(2, 3, 8, 2, 1, 1, 3, -1, True,
                        labels=np.zeros((3, 2), int), active=np.ones((3, 2), bool))
    fwd = synth_forward_tiles(topo)
    m = fwd.kv_mask.clone()
    first_live = int(np.nonzero(m.numpy())[0][0])
    m[first_live] = 0                                        # drop one key of a frame
    bad = M.TileList(items=fwd.items, kv_idx=fwd.kv_idx, kv_mask=m, blk_and=fwd.blk_and,
                     n_items=fwd.n_items, item_ranges=(), logical_pairs=fwd.logical_pairs,
                     key_extent=fwd.key_extent, row_extent=fwd.row_extent)
    with pytest.raises(AssertionError):
        M.transpose_tiles(bad)


def test_row_coverage_decides_whether_gradients_are_cleared():
    """The kernels leave their outputs uncleared only when the list's items
    own every row once (``kernels._covers_all_rows``), a fact the builder
    records from the groups' row descriptors (``metadata.group_rows_cover``)
    and derived key-major lists inherit."""
    import dataclasses
    from multics_amd.kernels import _covers_all_rows
    rng = np.random.default_rng(3)
    mem = rng.random((6, 2, 4)) < 0.4
    tiles = synth_forward_tiles(FullTopology(4, 6, 3, 2, 2, 2, 3, 4, True, membership=mem,
                                             global_only=~mem.any(1)))
    assert _covers_all_rows(tiles)
    assert _covers_all_rows(M.transpose_tiles_host(tiles))
    assert not _covers_all_rows(dataclasses.replace(tiles, rows_exact_cover=False))
    assert not _covers_all_rows(dataclasses.replace(tiles, key_extent=tiles.key_extent + 1))


@pytest.mark.parametrize("kind", ["labels", "membership", "nodirect_w_all"])
def test_group_rows_cover_full_sequence(kind):
    """Full-sequence topologies: the groups' rows are every token once; a
    group moved onto its neighbour's rows, or one dropped, is not a cover."""
    import copy
    rng = np.random.default_rng(4)
    P, T, L, N, KL, KG, n = 4, 6, 5, 2, 2, 3, 3
    if kind == "membership":
        mem = rng.random((T, N, P)) < 0.5
        topo = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=4,
                                        direct=True, membership=mem, global_only=~mem.any(1))
    else:
        labels = np.array([[p % N for p in range(P)]] * T)
        topo = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n,
                                        window=-1 if kind != "labels" else 4,
                                        direct=kind == "labels", labels=labels)
    S = P * T * L + T * (N * KL + KG)
    assert M.group_rows_cover(topo) == (S, True)
    moved = copy.deepcopy(topo)
    moved.tile_qbase[1][0] = moved.tile_qbase[0][0]
    assert not M.group_rows_cover(moved)[1]
    short = copy.deepcopy(topo)
    short.tile_qbase = [list(r) for r in short.tile_qbase]
    short.KL = 0                        # the local-hub rows (mid-sequence) uncovered
    assert not M.group_rows_cover(short)[1]


def test_host_lists_launch_as_built():
    """``launch_list`` cuts device lists only (the cut is a device pass); a
    host list is its own launch list and its own built list."""
    tiles = synth_forward_tiles(FullTopology(2, 6, 4, 1, 1, 1, 3, 4, True, labels=np.zeros((6, 2), np.int64)))
    assert not tiles.items.is_cuda
    assert M.launch_list(tiles) is tiles and M.built_list(tiles) is tiles
