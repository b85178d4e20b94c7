"""HIP metadata builder: bit-exact against the reference's golden vectors.

Segmented lists (``_build_metadata``), cached and full-sequence Tiled128
layouts, plus the attention tile list's per-row key sets against the golden
segmented lists and the dense-mask oracle.
"""

import dataclasses

import numpy as np
import pytest
import torch

from multics_amd import metadata as M
from oracle.masks import FullTopology, inactive_local_rows, mask_rows
from tests import golden_io as G
from tests.gpu_util import expand_tiles, need_gpu, say

pytestmark = pytest.mark.gpu
SEG_FIELDS = ("prog_qbase", "prog_nq", "prog_seg", "kv_index", "kv_count")
TILED_FIELDS = ("prog_qbase", "prog_nq", "prog_seg", "kv_index", "kv_valid", "kv_count")


def _seg_call(inp, return_tiles=False):
    return M._build_metadata(
        device="cuda", P=inp["P"], N=inp["N"], L=inp["L"], KL=inp["KL"], KG=inp["KG"],
        n_frames=inp["n_frames"], n_block=inp["n_block"], local_attn=inp["local_attn"],
        agent_frame_lists=inp["agent_frames"], local_frame_lists=inp["local_frames"],
        global_frame_list=inp["global_frames"], local_active_frames=inp["local_active"],
        labels=inp["labels"], q_active=inp["q_active"], direct_player=inp["direct"],
        block_m=inp["block_m"], membership=inp["membership"], global_only=inp["global_only"],
        hier_no_local_hub=inp["no_local"], return_tiles=return_tiles)


@pytest.mark.parametrize("name", G.cases("seg"))
def test_segmented_metadata_bit_exact(name):
    need_gpu()
    say("segmented metadata", name)
    inp = G.inputs("seg", name)
    M.clear_metadata_cache()
    out = _seg_call(inp, return_tiles=True)
    torch.cuda.synchronize()
    for f, val in zip(SEG_FIELDS, out[:5]):
        G.assert_same(f"seg/{name}/{f}", val.cpu().numpy())
    assert out[5] == G.scalar(f"seg/{name}/logical_pairs")
    # the attention tile list holds exactly the same key set per query row
    kv_index, kv_count = out[3].cpu().numpy(), out[4].cpu().numpy()
    qb, nq, sg = (x.cpu().numpy() for x in out[:3])
    rows = expand_tiles(out[6])
    for base, n, s in zip(qb, nq, sg):
        keys = set(kv_index[s, :kv_count[s]].tolist())
        for q in range(base, base + n):
            assert rows[q] == keys, (name, q)


@pytest.mark.parametrize("name", G.cases("tc"))
def test_tiled_cached_layout_bit_exact(name):
    need_gpu()
    say("tiled cached layout", name)
    inp = G.inputs("tc", name)
    M.clear_hier_tiled_layout_cache()
    lay = M.build_hier_tiled_cached_layout(
        device="cuda", P=inp["P"], N=inp["N"], L=inp["L"], KL=inp["KL"], KG=inp["KG"],
        n_frames=inp["n_frames"], n_block=inp["n_block"], local_attn=inp["local_attn"],
        agent_frame_lists=inp["agent_frames"], local_frame_lists=inp["local_frames"],
        global_frame_list=inp["global_frames"], local_active_frames=inp["local_active"],
        labels=inp["labels"], q_active=inp["q_active"], direct_player=inp["direct"])
    torch.cuda.synchronize()
    for f in TILED_FIELDS:
        G.assert_same(f"tc/{name}/{f}", getattr(lay, f).cpu().numpy())
    for f in ("logical_slots", "physical_slots", "dense_slots"):
        assert getattr(lay, f) == G.scalar(f"tc/{name}/{f}"), f


@pytest.mark.parametrize("name", G.cases("tf"))
def test_tiled_full_sequence_layouts_bit_exact(name):
    need_gpu()
    say("tiled full-sequence layouts", name)
    inp = G.inputs("tf", name)
    M.clear_hier_tiled_layout_cache()
    lays = M.build_hier_tiled_full_sequence_layouts(
        device="cuda", num_players=inp["P"], num_frames=inp["T"], num_patches=inp["L"],
        num_groups=inp["N"], num_local_hub_tokens=inp["KL"], num_global_hub_tokens=inp["KG"],
        num_frame_per_block=inp["n"], local_attn_size=inp["window"],
        group_labels=torch.tensor(inp["labels"]), active_group=torch.tensor(inp["active"]),
        direct_player=inp["direct"])
    torch.cuda.synchronize()
    assert len(lays) == G.scalar(f"tf/{name}/num_blocks")
    for b, lay in enumerate(lays):
        for f in TILED_FIELDS:
            G.assert_same(f"tf/{name}/{b}/{f}", getattr(lay, f).cpu().numpy())
        for f in ("logical_slots", "physical_slots", "dense_slots"):
            assert getattr(lay, f) == G.scalar(f"tf/{name}/{b}/{f}"), f
    if inp["T"] * inp["L"] * inp["P"] <= 4096:
        topo = FullTopology(inp["P"], inp["T"], inp["L"], inp["N"], inp["KL"], inp["KG"], inp["n"],
                            inp["window"], inp["direct"], labels=np.array(inp["labels"]),
                            active=np.array(inp["active"]))
        m = mask_rows(topo)
        dead = inactive_local_rows(topo)
        rows = expand_tiles(lays[0].tiles)
        assert len(rows) == topo.S
        for q in range(topo.S):
            exp = set() if dead[q] else set(np.nonzero(m[q])[0].tolist())
            assert rows[q] == exp, (name, q)


def test_dynamic_membership_tile_list_matches_dense_mask():
    """Per-frame membership (groups change inside a block), full sequence."""
    need_gpu()
    rng = np.random.default_rng(3)
    P, T, L, N, KL, KG, n, W = 5, 6, 3, 3, 2, 2, 3, 4
    mem = rng.random((T, N, P)) < 0.4
    go = ~mem.any(1) & (rng.random((T, P)) < 0.7)
    for direct in (False, True):
        say("dynamic membership tile list, direct", direct)
        topo = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                        direct=direct, membership=mem, global_only=go)
        tiles = M.build(topo, "cuda").tiles
        torch.cuda.synchronize()
        ft = FullTopology(P, T, L, N, KL, KG, n, W, direct, membership=mem, global_only=go)
        m = mask_rows(ft)
        dead = inactive_local_rows(ft)
        rows = expand_tiles(tiles)
        assert len(rows) == ft.S
        for q in range(ft.S):
            exp = set() if dead[q] else set(np.nonzero(m[q])[0].tolist())
            assert rows[q] == exp, q


def _packed_cases():
    from tests.test_varlen_plan import _packed_cases as cases
    return cases()


@pytest.mark.parametrize("name", _packed_cases())
def test_varlen_plan_on_device_arrays(name):
    """``_get_varlen_plan`` (hier_packed_attention.py:32-102) on the device
    arrays the HIP builder returns for a one-program-per-segment call, equal
    to the oracle's plan of the reference's golden arrays; a second call hits
    the plan cache."""
    need_gpu()
    from oracle.metadata import varlen_plan
    from tests.test_varlen_plan import _arrays
    say("varlen plan on device", name)
    inp = G.inputs("seg", name)
    ref = _arrays(name)
    qt = int(np.asarray(ref["prog_nq"]).sum())
    want = varlen_plan(ref["kv_index"], ref["kv_count"], ref["prog_qbase"], ref["prog_nq"],
                       ref["prog_seg"], qt)
    M.clear_metadata_cache()
    M.clear_varlen_plan_cache()
    qb, nq, sg, kv, kc, _ = _seg_call(inp)
    assert kv.is_cuda
    got = M._get_varlen_plan(kv_index=kv, kv_count=kc, qbase=qb, qlen=nq, seg_ids=sg,
                             query_tokens=qt)
    torch.cuda.synchronize()
    for k in ("q_index", "k_index", "cu_q", "cu_k"):
        assert got[k].is_cuda and got[k].dtype == (torch.int64 if k.endswith("index") else torch.int32)
        assert np.array_equal(got[k].cpu().numpy(), want[k]), k
    for k in ("max_q", "max_k", "min_k_index", "max_k_index"):
        assert got[k] == want[k], k
    assert M._get_varlen_plan(kv_index=kv, kv_count=kc, qbase=qb, qlen=nq, seg_ids=sg,
                              query_tokens=qt) is got


def _row_owner(tiles):
    """{token: (item row index r, item)} over every item, and the token list."""
    it = tiles.items[:tiles.n_items].cpu().numpy()
    owner = {}
    for k, (qb, qs, ql, r0, rc, off, cnt, nf) in enumerate(it):
        for r in range(r0, r0 + rc):
            j, i = divmod(r, ql)
            tok = qb + j * qs + i
            assert tok not in owner, tok
            owner[tok] = (j, k)
    return owner, it


def _keys_of(tiles, it, idx, msk, owner, tok):
    j, k = owner[tok]
    off, cnt = it[k, 5], it[k, 6]
    sel = ((msk[off:off + cnt] >> j) & 1) == 1
    return set(idx[off:off + cnt][sel].tolist())


@pytest.mark.parametrize("cfg", ["c2", "c3", "p10", "c5"])
def test_merged_hub_groups_keep_every_key_set(cfg):
    """Hub streams merged across temporal blocks (two by default for
    full-sequence lists; four here, the widest masks) against the per-block
    list of the same topology:
    every row owned once, every sampled row's key set equal (players, local
    hubs and global rows of the first, middle and last blocks, random rows),
    the same pair count; hub groups span up to 12 query frames, their lists
    in key-row order."""
    need_gpu()
    from tests.test_gpu_fullsize import _case, _rows
    say("merged hub groups", cfg)
    meta, topo, _ = _case(cfg)
    assert M.build(meta, "cuda").tiles.merged_blocks == M.MERGE_HUB_BLOCKS
    merged = M.build(meta, "cuda", merge_hubs=4).tiles
    plain = M.build(meta, "cuda", merge_hubs=0).tiles
    assert merged.merged_blocks == 4 and plain.merged_blocks == 1
    assert merged.n_items < plain.n_items
    assert merged.logical_pairs == plain.logical_pairs and merged.rows_exact_cover
    own_m, it_m = _row_owner(merged)
    own_p, it_p = _row_owner(plain)
    assert sorted(own_m) == list(range(topo.S)) and own_m.keys() == own_p.keys()
    idx_m, msk_m = merged.kv_idx.cpu().numpy(), merged.kv_mask.cpu().numpy().view(np.uint32)
    idx_p, msk_p = plain.kv_idx.cpu().numpy(), plain.kv_mask.cpu().numpy().view(np.uint32)
    for r in _rows(topo, np.random.default_rng(1), n_random=256):
        assert _keys_of(merged, it_m, idx_m, msk_m, own_m, int(r)) == \
            _keys_of(plain, it_p, idx_p, msk_p, own_p, int(r)), (cfg, r)
    a0 = topo.P * topo.T * topo.L
    hub = it_m[it_m[:, 0] >= a0]
    assert (hub[:, 7] <= 12).all() and (hub[:, 7] == 12).any()
    for qb, qs, ql, r0, rc, off, cnt, nf in hub:
        live = idx_m[off:off + cnt][msk_m[off:off + cnt] != 0]
        assert (np.diff(live) > 0).all()


def _fwd_row_owner(tiles):
    """{token: (mask bit, item)} over the forward's own items, row-table
    items (qstride -1) included."""
    it = tiles.fwd_items[:tiles.fwd_n_items].cpu().numpy()
    tab = tiles.row_table.cpu().numpy()
    owner = {}
    for k, (qb, qs, ql, r0, rc, off, cnt, nf) in enumerate(it):
        for r in range(r0, r0 + rc):
            if qs < 0:
                tok, j = (int(x) for x in tab[qb + r])
            else:
                j, i = divmod(r, ql)
                tok = qb + j * qs + i
            assert tok not in owner, tok
            owner[tok] = (j, k)
    return owner, it


@pytest.mark.parametrize("cfg", ["c2", "p6", "c3", "p10"])
def test_folded_forward_list_keeps_every_key_set(cfg):
    """The forward's own list, in which each player's ragged last item
    (n * L mod 128 rows) joins its local hub's group under mask bits of its
    own: every row owned once, every folded row's key set and every sampled
    row's key set equal to the per-block list's; the hubs' key lists do not
    grow (a member's keys are a subset of its hub's); fewer items of <= 32
    rows; the backward's list unchanged."""
    need_gpu()
    import dataclasses
    from tests.test_gpu_fullsize import _case, _rows
    say("folded forward list", cfg)
    meta, topo, _ = _case(cfg)
    tiles = M.build(meta, "cuda").tiles
    unfolded = M.build(meta, "cuda", fold_tails=False).tiles
    plain = M.build(meta, "cuda", merge_hubs=0).tiles
    assert tiles.fwd_items is not None and unfolded.fwd_items is None
    assert torch.equal(tiles.items[:tiles.n_items], unfolded.items[:unfolded.n_items])
    own_f, it_f = _fwd_row_owner(tiles)
    own_p, it_p = _row_owner(plain)
    assert sorted(own_f) == list(range(topo.S))
    idx_f, msk_f = tiles.kv_idx.cpu().numpy(), tiles.kv_mask.cpu().numpy().view(np.uint32)
    idx_p, msk_p = plain.kv_idx.cpu().numpy(), plain.kv_mask.cpu().numpy().view(np.uint32)
    table_tokens = set(tiles.row_table[:, 0].cpu().tolist())
    folded = sorted(t for t in table_tokens if t < topo.P * topo.T * topo.L)
    assert folded, "no player rows folded"
    sample = set(_rows(topo, np.random.default_rng(2), n_random=128).tolist()) | set(folded)
    for r in sorted(sample):
        assert _keys_of(tiles, it_f, idx_f, msk_f, own_f, int(r)) == \
            _keys_of(plain, it_p, idx_p, msk_p, own_p, int(r)), (cfg, r)
    # folded groups walk lists no longer than the hub group they replace
    own_u, it_u = _row_owner(unfolded)
    hub0 = topo.P * topo.T * topo.L
    for qb, qs, ql, r0, rc, off, cnt, nf in it_f[it_f[:, 1] < 0]:
        hub_tok = int(tiles.row_table[qb, 0])
        assert hub0 <= hub_tok < hub0 + topo.T * topo.N * topo.KL
        assert cnt <= it_u[own_u[hub_tok][1], 6]
    small = lambda it: int((it[:, 4] <= 32).sum())
    assert small(it_f) < small(it_u)
    players = lambda it: int(((it[:, 0] < hub0) & (it[:, 1] >= 0)).sum())
    assert players(it_f) == players(it_u) - len(folded) // (topo.n * topo.L % 128)
    # the forward through both lists: the same rows, bf16 rounding apart
    S, H, D = topo.S, 2, 128
    g = torch.Generator(device="cuda").manual_seed(5)
    q, k, v = ((torch.randn(S, H, D, generator=g, device="cuda") * 0.5).to(torch.bfloat16)
               for _ in range(3))
    from multics_amd.kernels import hier_attention_forward
    outs, lses = [], []
    for t in (tiles, unfolded):
        o = torch.full((S, H, D), float("nan"), dtype=torch.bfloat16, device="cuda")
        l = torch.full((H, S), float("nan"), dtype=torch.float32, device="cuda")
        hier_attention_forward(q, k, v, t, o, lse=l)
        outs.append(o.float())
        lses.append(l)
    assert not outs[0].isnan().any() and not lses[0].isnan().any()
    assert (outs[0] - outs[1]).abs().max().item() <= 2e-3
    fin = torch.isfinite(lses[1])
    assert torch.equal(fin, torch.isfinite(lses[0]))
    assert (lses[0][fin] - lses[1][fin]).abs().max().item() <= 1e-3


def test_folded_forward_list_cached_block():
    """A cached rollout block (C4: ten players in random per-block groups,
    the window in the paged pool): with no hub merge, ``fold_tails=True``
    folds the players' last rows into the block's local hub items (off by
    default there: on a short launch the folded groups' long lists end it).  Every
    query row owned once; the key sets of every folded row and of sampled
    rows equal the unfolded list's; the forward over both lists agrees to
    bf16 rounding (the rollout tests run the folded list against the cached
    oracle)."""
    need_gpu()
    import bench
    from multics_amd.kernels import hier_attention_forward
    from multics_amd.paged_cache import HierPagedKVCache
    say("folded forward list, cached block")
    P, T, L, N, KL, KG, n, W, _, D, grp = bench.CONFIGS["c4"]
    H = 2
    _, mem, go = bench.grouping(grp, P, T, N, np.random.default_rng(bench.SEED))
    act = mem.any(-1)
    cache = HierPagedKVCache(num_players=P, num_groups=N, num_patches=L, num_local_hub_tokens=KL,
                             num_global_hub_tokens=KG, num_heads=H, head_dim=D, local_attn_size=W,
                             num_frame_per_block=n, device="cuda")
    S = P * n * L + n * (N * KL + KG)
    g = torch.Generator(device="cuda").manual_seed(7)
    q, k, v = ((torch.randn(S, H, D, generator=g, device="cuda") * 0.5).to(torch.bfloat16)
               for _ in range(3))
    b = (W + n) // n
    for bb in range(b + 1):
        cache.append(k, v, bb * n, n, act[bb * n:bb * n + n])
    frames, bases, lact = cache.window(b * n + n - 1)
    topo = M.cached_topology(
        P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n, n_block=n, local_attn=W,
        agent_frame_lists=[tuple(frames)] * P, local_frame_lists=[tuple(frames)] * N,
        global_frame_list=tuple(frames), local_active_frames=lact, labels=None,
        q_active=act[b * n:b * n + n].tolist(), direct_player=True, membership=mem,
        global_only=go, tile_bases=bases)
    tiles = M.build(topo, "cuda", fold_tails=True).tiles
    plain = M.build(topo, "cuda").tiles
    assert tiles.merged_blocks == 1 and tiles.item_ranges == plain.item_ranges
    assert tiles.fwd_items is not None and plain.fwd_items is None
    assert torch.equal(tiles.items[:tiles.n_items], plain.items[:plain.n_items])
    own_f, it_f = _fwd_row_owner(tiles)
    own_p, it_p = _row_owner(plain)
    assert sorted(own_f) == sorted(own_p) == list(range(S))
    idx_f, msk_f = tiles.kv_idx.cpu().numpy(), tiles.kv_mask.cpu().numpy().view(np.uint32)
    idx_p, msk_p = plain.kv_idx.cpu().numpy(), plain.kv_mask.cpu().numpy().view(np.uint32)
    folded = sorted(t for t in set(tiles.row_table[:, 0].cpu().tolist()) if t < P * n * L)
    assert len(folded) >= 5 * (n * L % 128)
    rng = np.random.default_rng(3)
    sample = set(folded) | set(range(P * n * L, S)) | set(rng.choice(S, 256, replace=False).tolist())
    for r in sorted(sample):
        assert _keys_of(tiles, it_f, idx_f, msk_f, own_f, int(r)) == \
            _keys_of(plain, it_p, idx_p, msk_p, own_p, int(r)), r
    outs = []
    for t in (tiles, plain):
        o = torch.full((S, H, D), float("nan"), dtype=torch.bfloat16, device="cuda")
        hier_attention_forward(q, cache.k, cache.v, t, o)
        outs.append(o.float())
    assert not outs[0].isnan().any()
    assert (outs[0] - outs[1]).abs().max().item() <= 2e-3


@pytest.mark.parametrize("cfg", ["c2", "c5"])
def test_folded_key_major_list_keeps_every_query_set(cfg):
    """The key-major list the dK / dV pass runs (``folded_key_list``): the
    players' last key rows folded into their local hubs' key items under the
    forward fold's row table.  Every key row owned once; the query set of
    every folded key row and of sampled key rows equal to the derived
    key-major list's; fewer items of <= 32 rows."""
    need_gpu()
    from tests.test_gpu_fullsize import _case, _rows
    say("folded key-major list", cfg)
    meta, topo, _ = _case(cfg)
    tiles = M.build(meta, "cuda").tiles
    kt, _ = M.backward_lists(tiles)
    ktf = M.folded_key_list(tiles, kt)
    assert ktf is not kt and M.folded_key_list(tiles, kt) is ktf
    from multics_amd.kernels import _covers_all_rows
    assert ktf.row_table is tiles.row_table and _covers_all_rows(ktf) and _covers_all_rows(kt)
    t = dataclasses.replace(ktf, fwd_items=ktf.items, fwd_n_items=ktf.n_items)
    own_f, it_f = _fwd_row_owner(t)
    own_p, it_p = _row_owner(kt)
    assert sorted(own_f) == sorted(own_p) == list(range(topo.S))
    idx_f, msk_f = ktf.kv_idx.cpu().numpy(), ktf.kv_mask.cpu().numpy().view(np.uint32)
    idx_p, msk_p = kt.kv_idx.cpu().numpy(), kt.kv_mask.cpu().numpy().view(np.uint32)
    folded = sorted(x for x in set(tiles.row_table[:, 0].cpu().tolist())
                    if x < topo.P * topo.T * topo.L)
    assert folded
    sample = set(_rows(topo, np.random.default_rng(4), n_random=128).tolist()) | set(folded)
    for r in sorted(sample):
        assert _keys_of(ktf, it_f, idx_f, msk_f, own_f, int(r)) == \
            _keys_of(kt, it_p, idx_p, msk_p, own_p, int(r)), (cfg, r)
    assert (it_f[:, 4] <= 32).sum() < (it_p[:, 4] <= 32).sum()


def _check_cut(built, run, n, mask, table):
    """Every item of ``run`` (``launch_list(built)``): same rows; its list a
    whole-tile sub-range of the built one, starting and ending on a tile
    with an entry some of its rows see, holding every such entry (items that
    see none keep their range).  Returns the entries cut."""
    b = built[:n].cpu().numpy().astype(np.int64)
    r = run[:n].cpu().numpy().astype(np.int64)
    assert np.array_equal(np.delete(b, [5, 6], 1), np.delete(r, [5, 6], 1))
    m = mask.cpu().numpy().view(np.uint32)
    rt = None if table is None else table.cpu().numpy().reshape(-1, 2)
    cut = 0
    for (qb, qs, ql, r0, rc, off, cnt, _), (*_, off2, cnt2, _) in zip(b, r):
        rows = np.arange(r0, r0 + rc)
        bits = rt[qb + rows, 1] if qs < 0 else rows // ql
        want = np.bitwise_or.reduce(np.left_shift(np.uint32(1), bits.astype(np.uint32)))
        seen = np.flatnonzero(m[off:off + cnt] & want)
        if seen.size == 0:
            assert (off2, cnt2) == (off, cnt)
            continue
        assert (off2 - off) % 64 == 0 and off <= off2 and off2 + cnt2 <= off + cnt
        first, last = off2 - off, off2 - off + cnt2 - 1
        assert first <= seen[0] and seen[-1] <= last
        assert seen[0] // 64 == first // 64 and seen[-1] // 64 == last // 64
        assert cnt2 == min(cnt - first, (last // 64 - first // 64 + 1) * 64)
        cut += cnt - cnt2
    return cut


def _as_built(tl):
    """``tl`` launched with its lists as built (no cut)."""
    r = dataclasses.replace(tl)
    r.__dict__["_is_launch"] = True
    return r


@pytest.mark.parametrize("cfg", ["c5", "c2"])
def test_launch_lists_cut_to_visible_tiles(cfg):
    """``launch_list``: the forward's own list, the shared list (dQ pass) and
    the folded key-major list (dK / dV pass) cut to the tiles their rows see;
    the forward and the backward over the cut lists equal those over the
    built lists bit for bit (the tiles cut hold only masked entries)."""
    need_gpu()
    from tests.test_gpu_fullsize import _case, _inputs
    from multics_amd.kernels import hier_attention_backward, hier_attention_forward
    say("launch lists cut to visible tiles", cfg)
    meta, topo, D = _case(cfg)
    tiles = M.build(meta, "cuda").tiles
    kt = M.folded_key_list(tiles, M.backward_lists(tiles)[0])
    run, krun = M.launch_list(tiles), M.launch_list(kt)
    assert M.launch_list(run) is run and M.launch_list(tiles) is run
    assert M.built_list(run) is tiles and M.built_list(tiles) is tiles
    cut = [_check_cut(tiles.items, run.items, tiles.n_items, tiles.kv_mask, None),
           _check_cut(tiles.fwd_items, run.fwd_items, tiles.fwd_n_items, tiles.kv_mask,
                      tiles.row_table),
           _check_cut(kt.items, krun.items, kt.n_items, kt.kv_mask, kt.row_table)]
    say("  entries cut (shared, forward, key-major)", cut)
    assert min(cut) > 0
    geom = None
    if topo.membership is not None:       # the membership-STE classes of the cut list
        geom = (topo.P, topo.T, topo.L, topo.N, topo.KL)
        cls, first = M.launch_ste_first(tiles, geom)
        host = M.ste_classes_host(run, P=geom[0], T=geom[1], L=geom[2], N=geom[3], KL=geom[4])
        sel = np.zeros(len(host), bool)
        for off, cnt in run.items[:run.n_items, 5:7].cpu().numpy().astype(np.int64):
            sel[off:off + cnt] = True
        assert np.array_equal(cls.cpu().numpy()[sel], host[sel])
        assert np.array_equal(first[:run.n_items].cpu().numpy(), M.ste_first_tiles_host(run, host))
    H = 2
    q, k, v = (t.cuda() for t in _inputs(topo.S, H, D, seed=41))
    dout = torch.randn(topo.S, H, D, generator=torch.Generator().manual_seed(42))
    dout = dout.to(torch.bfloat16).cuda()
    res = []
    for t, kl in ((tiles, kt), (_as_built(tiles), _as_built(kt))):
        o = torch.empty_like(q)
        lse = torch.empty(H, topo.S, dtype=torch.float32, device="cuda")
        hier_attention_forward(q, k, v, t, o, lse=lse)
        grads = hier_attention_backward(q, k, v, o, dout, lse, t, key_tiles=kl, ste_geometry=geom)
        res.append((o, lse) + tuple(grads))
    for name, a, b in zip(("out", "lse", "dq", "dk", "dv", "ste"), *res):
        assert torch.equal(a, b), name


def _cut_host(items, mask, table):
    """Expected cut of every item: the first and last 64-entry tile holding an
    entry that one of its rows sees (rows' bits: frame (r0 + r) // qlen, or
    the row table's bit); unchanged when no row sees any entry."""
    out = items.copy()
    for i, (qb, qs, ql, r0, rc, off, cnt, _) in enumerate(items.astype(np.int64)):
        rows = np.arange(r0, r0 + rc)
        bits = table[qb + rows, 1] if qs < 0 else rows // max(ql, 1)
        want = np.uint32(0)
        for b in np.unique(bits):
            if 0 <= b < 32:
                want |= np.uint32(1) << np.uint32(b)
        seen = np.flatnonzero(mask[off:off + cnt] & want)
        if seen.size:
            f, l = seen[0] // 64, seen[-1] // 64
            out[i, 5] = off + 64 * f
            out[i, 6] = min(cnt - 64 * f, 64 * (l - f + 1))
    return out


def test_trim_kernel_random_lists():
    """``hier_trim_key_lists`` on random items: ragged and empty ranges,
    visible entries only at either end or nowhere, row-table items, ranges
    not a multiple of four long or four-aligned."""
    need_gpu()
    rng = np.random.default_rng(11)
    n_items, n_keys, n_rows = 400, 1 << 16, 4096
    mask = np.zeros(n_keys, np.uint32)
    table = np.stack([rng.integers(0, 1 << 20, n_rows), rng.integers(0, 8, n_rows)], 1).astype(np.int32)
    items = np.zeros((n_items, 8), np.int32)
    for i in range(n_items):
        off = int(rng.integers(0, n_keys // 64 - 40)) * 64 + (int(rng.integers(1, 4)) if i % 7 == 0 else 0)
        cnt = int(rng.integers(0, 40 * 64)) if i % 5 else int(rng.integers(0, 4)) * 64
        cnt = min(cnt, n_keys - off)
        rc = int(rng.integers(1, 129))
        if i % 3 == 0:           # rows from the row table
            qb = int(rng.integers(0, n_rows - 128))
            items[i] = (qb, -1, 1, 0, rc, off, cnt, 1)
        else:
            ql = int(rng.integers(1, 300))
            items[i] = (0, ql, ql, int(rng.integers(0, 200)), rc, off, cnt, 8)
        kind = i % 4
        seg = np.arange(off, off + cnt)
        if cnt and kind == 0:      # sparse random bits
            mask[seg] |= (rng.random(cnt) < 0.02).astype(np.uint32) << rng.integers(0, 8, cnt).astype(np.uint32)
        elif cnt and kind == 1:    # one visible entry near the end
            mask[off + cnt - 1 - int(rng.integers(0, min(cnt, 70)))] |= np.uint32(0xff)
    dev = torch.device("cuda")
    t_items = torch.from_numpy(items).to(dev)
    t_mask = torch.from_numpy(mask.view(np.int32)).to(dev)
    t_table = torch.from_numpy(table).to(dev)
    got = M._trim_items(t_items, n_items, t_mask, t_table).cpu().numpy()
    want = _cut_host(items, mask, table)
    assert np.array_equal(got, want)
    assert (got[:, 6] < items[:, 6]).sum() > 50
    # in place (the output array is the input)
    a = M._capi.HierTrimArgs(n_items=n_items, items=t_items.data_ptr(), kv_mask=t_mask.data_ptr(),
                             row_table=t_table.data_ptr(), out_items=t_items.data_ptr())
    M._capi.call("hier_trim_key_lists", M.C.byref(a), torch.cuda.current_stream().cuda_stream)
    assert np.array_equal(t_items.cpu().numpy(), want)
