"""The backward's key-major and membership-STE lists built on the GPU
(``hier_derive_count`` / ``hier_derive_build`` in csrc/hier_meta.hip) equal
the host builders ``metadata.transpose_tiles_host`` / ``ste_tiles_host`` bit
for bit: items, row / key indices, masks, per-64 ANDs, classes, pair count;
the STE classes of the forward list (``hier_derive_ste_classes``) equal
``metadata.ste_classes_host``.

Cases: every bench topology that has a full-sequence tile list (C2 fixed
groups, P6 pairs, C3 per-frame dynamic groups, P10 random blocks, C5 soft
membership logits), a membership form with orphans, a no-local-hub form and a
small labels form with an inactive group; plus a list with one key of a frame
dropped, which both builders refuse (the device kernels flag it and the host
side raises).
"""

import numpy as np
import pytest
import torch

import bench
from multics_amd import metadata as M
from tests.gpu_util import need_gpu, say

pytestmark = pytest.mark.gpu


def _same(a: torch.Tensor, b: torch.Tensor, what: str):
    a, b = a.detach().cpu(), b.detach().cpu()
    assert a.dtype == b.dtype and a.shape == b.shape, (what, a.dtype, b.dtype, a.shape, b.shape)
    assert torch.equal(a, b), what


def _check_lists(tiles, geom):
    dev_kt, dev_ste = M._derive_device(tiles, geom)
    torch.cuda.synchronize()
    host_kt = M.transpose_tiles_host(tiles)
    for f in ("items", "kv_idx", "kv_mask", "blk_and"):
        _same(getattr(dev_kt, f), getattr(host_kt, f), f"key-major {f}")
    for f in ("n_items", "logical_pairs", "key_extent", "row_extent", "rows_per_item"):
        assert getattr(dev_kt, f) == getattr(host_kt, f), f
    if geom is None:
        assert dev_ste is None
        return
    host_cls = M.ste_classes_host(tiles, P=geom[0], T=geom[1], L=geom[2], N=geom[3], KL=geom[4])
    dev_cls, dev_first = M.ste_classes(tiles, geom)
    _same(dev_cls[:len(host_cls)], torch.from_numpy(host_cls), "forward-list STE classes")
    _same(dev_first[:tiles.n_items], torch.from_numpy(M.ste_first_tiles_host(tiles, host_cls)),
          "first tile with a class")
    assert M.ste_classes(tiles, geom)[0] is dev_cls               # cached on the list
    host_ste = M.ste_tiles_host(tiles, P=geom[0], T=geom[1], L=geom[2], N=geom[3], KL=geom[4])
    assert (dev_ste is None) == (host_ste is None)
    if host_ste is None:
        return
    (dl, dc), (hl, hc) = dev_ste, host_ste
    for f in ("items", "kv_idx", "kv_mask", "blk_and"):
        _same(getattr(dl, f), getattr(hl, f), f"STE {f}")
    _same(dc, hc, "STE classes")
    assert dl.n_items == hl.n_items


@pytest.mark.parametrize("cfg", ["c2", "p6", "c3", "p10", "c5"])
def test_device_lists_match_host_at_bench_sizes(cfg):
    need_gpu()
    dev = torch.device("cuda", 0)
    say(f"derive {cfg}")
    P, T, L, N, KL, KG, n, W, H, D, grp = bench.CONFIGS[cfg]
    _, tiles, _, _ = bench.build_case(cfg, dev)
    _check_lists(tiles, (P, T, L, N, KL))
    # backward_lists routes device lists through the device builder and caches
    kt, ste = M.backward_lists(tiles, (P, T, L, N, KL))
    assert M.backward_lists(tiles, (P, T, L, N, KL))[0] is kt
    assert M.transpose_tiles(tiles) is kt


@pytest.mark.parametrize("kind", ["membership", "no_local", "labels_inactive"])
def test_device_lists_match_host_small(kind):
    need_gpu()
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(7)
    P, T, L, N, KL, KG, n, W = 4, 6, 24, 3, 2, 3, 3, 4
    labels = active = mem = go = None
    no_local = False
    if kind == "membership":
        mem = rng.random((T, N, P)) < 0.35
        go = ~mem.any(1)
        go[0, 0] = False                               # an orphan: no group, not global-only
    elif kind == "no_local":
        mem = rng.random((T, N, P)) < 0.5
        go = ~mem.any(1)
        KL, no_local = 0, True
    else:
        labels = rng.integers(0, N, size=(T, P))
        active = np.zeros((T, N), dtype=bool)
        active[np.arange(T)[:, None], labels] = True
        active[:, -1] = False
    say(f"derive small {kind}")
    tiles = M.full_sequence_tiles(device=dev, P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                  direct=True, labels=labels, active=active, membership=mem,
                                  global_only=go, no_local=no_local)
    _check_lists(tiles, (P, T, L, N, KL))
    _check_lists(tiles, None)


def test_device_builder_refuses_partial_frames():
    need_gpu()
    dev = torch.device("cuda", 0)
    P, T, L, N, KL, KG, n, W = 2, 3, 8, 2, 1, 1, 3, -1
    tiles = M.full_sequence_tiles(device=dev, P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                  direct=True, labels=np.zeros((T, P), int),
                                  active=np.ones((T, N), bool))
    m = tiles.kv_mask.clone()
    live = torch.nonzero(m.cpu()).flatten()
    m[int(live[1])] = 0                                  # drop the second key of a frame
    bad = M.TileList(items=tiles.items, kv_idx=tiles.kv_idx, kv_mask=m, blk_and=tiles.blk_and,
                     n_items=tiles.n_items, item_ranges=tiles.item_ranges,
                     logical_pairs=tiles.logical_pairs, key_extent=tiles.key_extent,
                     row_extent=tiles.row_extent, frames_per_group=tiles.frames_per_group)
    say("derive refuses a partial frame")
    with pytest.raises(AssertionError, match="whole key frames"):
        M._derive_device(bad, None)
    with pytest.raises(AssertionError):
        M.transpose_tiles_host(bad)


def _group_lists(tiles, what):
    """{(qbase, qstride, qlen, row_start, row_count, n): (kv_idx, kv_mask)} of
    every item (lists by content; offsets may differ between builders)."""
    it = tiles.items[:tiles.n_items].cpu().numpy()
    idx = tiles.kv_idx.cpu().numpy()
    msk = tiles.kv_mask.cpu().numpy()
    out = {}
    for qb, qs, ql, r0, rc, off, cnt, nf in it:
        key = (qb, qs, ql, r0, rc, nf)
        assert key not in out, (what, key)
        out[key] = (idx[off:off + cnt].copy(), msk[off:off + cnt].copy())
    return out


def _same_groups(a, b, what):
    ga, gb = _group_lists(a, what), _group_lists(b, what)
    assert ga.keys() == gb.keys(), what
    for k in ga:
        assert np.array_equal(ga[k][0], gb[k][0]) and np.array_equal(ga[k][1], gb[k][1]), (what, k)


@pytest.mark.parametrize("case", ["c5", "small"])
def test_logits_plan_equals_host_topology(case):
    """``MembershipLogitsPlan`` (lists of logits > 0 rebuilt on the device
    with no read-back, in slots sized by the all-bits-on superset) against
    the host-topology build of the same membership: every item's
    descriptor, key list and masks, and every key-major list, equal; a
    training step with the membership STE gives bit-identical outputs and
    gradients.  Two builds in a row with different logits (the plan's
    buffers reused)."""
    need_gpu()
    from multics_amd.kernels import hier_attention
    dev = torch.device("cuda")
    if case == "c5":
        P, T, L, N, KL, KG, n, W, H, D, grp = bench.CONFIGS["c5"]
        H = 2
    else:
        P, T, L, N, KL, KG, n, W, H, D = 5, 9, 24, 3, 2, 3, 3, 4, 2, 128
    say("logits plan", case)
    plan = M.MembershipLogitsPlan(device=dev, P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                  direct=True)
    S = P * T * L + T * (N * KL + KG)
    g = torch.Generator(device=dev).manual_seed(4)
    q, k, v = ((torch.randn(S, H, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
               for _ in range(3))
    dout = torch.randn(S, H, D, generator=g, device=dev).to(torch.bfloat16)
    geo = (P, T, L, N, KL)
    for seed in (0, 1):
        lg = torch.randn(T, N, P, generator=torch.Generator().manual_seed(seed)).to(dev)
        mem = (lg > 0).cpu().numpy()
        # the plan folds no player rows into hub groups (fold_tails=False)
        ref = M.build(M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                               direct=True, membership=mem,
                                               global_only=~mem.any(1)), dev,
                      fold_tails=False).tiles
        got = plan.build(lg)
        torch.cuda.synchronize()
        _same_groups(got, ref, f"forward lists seed {seed}")
        _same_groups(M.backward_lists(got)[0], M.backward_lists(ref)[0],
                     f"key-major lists seed {seed}")
        res = []
        for tl in (got, ref):
            qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
            ld = lg.clone().requires_grad_(True)
            out = hier_attention(qd, kd, vd, tl, membership_logits=ld, ste_geometry=geo)
            out.backward(dout)
            res.append((out.detach(), qd.grad, kd.grad, vd.grad, ld.grad))
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "dq", "dk", "dv", "dlogits"), *res):
            assert torch.equal(a, b), (seed, name)
