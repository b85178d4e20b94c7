"""Parity at the full sizes of the bench configurations, on sampled rows.

An output row depends only on its query, the keys and values it sees and its
mask row, so a sample of rows is checked exactly against the oracle at sizes
where an S x S oracle pass per head would not fit a test.  The sample holds
every stream kind (players, local hubs, global hubs) of the first, middle and
last temporal blocks, the first and last rows of each player block (a block's
last 128-row work item holds its 20 remaining rows) and random rows.  The
backward at C5 takes dQ at the sampled rows and dK / dV at the same key rows
from ``oracle.attention.attention_grads_at``; the C4 rollout (paged KV cache,
window full) compares sampled rows of its last blocks with the full-sequence
oracle, which an in-order rollout equals.  Tolerances as in the small
cases: forward max-abs 2e-2 / mean-abs 2e-3, log-sum-exp within 2^-8;
gradients max-abs 2e-2 / mean-abs 2e-3 and within 2 % of the reference's
max and 1 % of its mean.
"""

import math

import numpy as np
import pytest
import torch

import bench
from multics_amd import metadata as M
from multics_amd.kernels import hier_attention, hier_attention_forward
from multics_amd.paged_cache import HierPagedKVCache
from oracle.attention import attention_grads_at, masked_attention
from oracle.masks import FullTopology, inactive_local_rows, mask_rows
from tests.gpu_util import err_stats, need_gpu, say
from tests.test_gpu_backward import _check

pytestmark = pytest.mark.gpu
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _case(cfg):
    """The bench's topology of ``cfg`` for the HIP builder and the oracle."""
    P, T, L, N, KL, KG, n, W, _, D, grp = bench.CONFIGS[cfg]
    first, mem, go = bench.grouping(grp, P, T, N, np.random.default_rng(bench.SEED))
    labels = None if grp == "logits" else first
    meta = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W, direct=True,
                                    labels=labels, membership=mem, global_only=go)
    if mem is None:
        topo = FullTopology(P, T, L, N, KL, KG, n, W, True, labels=labels)
    else:
        topo = FullTopology(P, T, L, N, KL, KG, n, W, True, membership=mem, global_only=go)
    return meta, topo, D


def _rows(topo, rng, n_random=64):
    P, T, L, N, KL, KG, n = topo.P, topo.T, topo.L, topo.N, topo.KL, topo.KG, topo.n
    a0, g0 = P * T * L, P * T * L + T * N * KL
    nb = -(-T // n)
    rows = set(rng.choice(topo.S, n_random, replace=False).tolist())
    for b in sorted({0, nb // 2, nb - 1}):
        f0, f1 = b * n, min(T, b * n + n)
        for p in range(P):
            base, cnt = p * T * L + f0 * L, (f1 - f0) * L
            rows |= {base, base + 127, base + 128, base + cnt - 21, base + cnt - 1}
        rows |= set(range(a0 + f0 * N * KL, a0 + f1 * N * KL))
        rows |= set(range(g0 + f0 * KG, g0 + f1 * KG))
    return np.array(sorted(r for r in rows if 0 <= r < topo.S), dtype=np.int64)


def _inputs(S, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(S, H, D, generator=g) * 0.5).to(torch.bfloat16) for _ in range(3)]


@pytest.mark.parametrize("cfg", ["c2", "c2_w7", "c3", "p10"])
def test_forward_full_size_sampled_rows(cfg):
    need_gpu()
    meta, topo, D = _case(cfg)
    H = 4
    say("full-size forward", cfg, "S", topo.S)
    tiles = M.build(meta, "cuda").tiles
    q, k, v = _inputs(topo.S, H, D, seed=21)
    out = torch.zeros(topo.S, H, D, dtype=torch.bfloat16, device="cuda")
    lse = torch.full((H, topo.S), float("nan"), dtype=torch.float32, device="cuda")
    hier_attention_forward(q.cuda(), k.cuda(), v.cuda(), tiles, out, lse=lse)
    torch.cuda.synchronize()
    rows = _rows(topo, np.random.default_rng(5))
    rt = torch.from_numpy(rows)
    say(f"  {len(rows)} sampled rows")
    ref = masked_attention(q, k, v, topo, rows=rows)
    got = out.cpu()[rt]
    mx, mn = err_stats(got, ref)
    say(f"  max-abs {mx:.3e} mean-abs {mn:.3e}")
    assert torch.isfinite(got.float()).all()
    assert mx <= MAX_ABS and mn <= MEAN_ABS
    m = torch.from_numpy(mask_rows(topo, q_idx=rows))
    s = torch.einsum("qhd,khd->hqk", q[rt].float(), k.float()) / math.sqrt(D)
    ref_lse = torch.logsumexp(s.masked_fill(~m[None], float("-inf")), dim=-1)
    live = torch.from_numpy(~inactive_local_rows(topo)[rows])
    got_lse = lse.cpu()[:, rt]
    assert torch.isneginf(got_lse[:, ~live]).all()
    assert (got_lse[:, live] - ref_lse[:, live]).abs().max() < 2.0 ** -8
    # the tile list's key set of every sampled row equals its mask row, exactly
    _check_key_sets(tiles, rows, m.numpy(), ~live.numpy())


def test_forward_c2_as_benchmarked():
    """The headline configuration exactly as ``bench.py`` times it: C2 with
    all 24 heads, Q/K head-major (``[H, S, D]`` storage presented as
    ``[S, H, D]`` views, as the prologue writes them on the module's no-grad
    path) and V token-major (the v projection read in place).  Sampled rows
    against the oracle at the north-star bounds; the whole output
    bit-identical to the same forward on token-major copies of all three (the
    layout changes only the addresses the kernel reads)."""
    need_gpu()
    meta, topo, D = _case("c2")
    H = bench.CONFIGS["c2"][8]
    assert H == 24
    say("c2 as benchmarked: S", topo.S, "H", H)
    tiles = M.build(meta, "cuda").tiles
    g = torch.Generator().manual_seed(31)
    qh, kh, vh = ((torch.randn(H, topo.S, D, generator=g) * 0.5).to(torch.bfloat16)
                  for _ in range(3))
    qd, kd = (t.cuda().permute(1, 0, 2) for t in (qh, kh))
    vd = vh.cuda().permute(1, 0, 2).contiguous()
    assert qd.stride() == (D, topo.S * D, 1) and vd.stride() == (H * D, D, 1)
    out = torch.zeros(topo.S, H, D, dtype=torch.bfloat16, device="cuda")
    hier_attention_forward(qd, kd, vd, tiles, out)
    torch.cuda.synchronize()
    say("  benchmarked layout done; token-major copies")
    out_shd = torch.zeros_like(out)
    hier_attention_forward(qd.contiguous(), kd.contiguous(), vd.contiguous(), tiles, out_shd)
    torch.cuda.synchronize()
    assert torch.equal(out, out_shd)
    rows = _rows(topo, np.random.default_rng(8), n_random=96)
    rt = torch.from_numpy(rows)
    say(f"  {len(rows)} sampled rows x {H} heads against the oracle")
    q, k, v = (t.permute(1, 0, 2) for t in (qh, kh, vh))
    ref = masked_attention(q, k, v, topo, rows=rows)
    mx, mn = err_stats(out.cpu()[rt], ref)
    say(f"  max-abs {mx:.3e} mean-abs {mn:.3e}")
    assert mx <= MAX_ABS and mn <= MEAN_ABS


def _check_key_sets(tiles, rows, m, dead):
    """The key set of every sampled row equals its mask row, in the shared
    list and in the forward's own list (rows of row-table items included)."""
    idx = tiles.kv_idx.cpu().numpy()
    msk = tiles.kv_mask.cpu().numpy().view(np.uint32)
    pos = {int(r): i for i, r in enumerate(rows)}
    lists = [(tiles.items[:tiles.n_items].cpu().numpy(), None)]
    if tiles.fwd_items is not None:
        lists.append((tiles.fwd_items[:tiles.fwd_n_items].cpu().numpy(),
                      tiles.row_table.cpu().numpy()))
    for items, table in lists:
        seen = np.zeros(len(rows), dtype=np.int64)
        for qbase, qstride, qlen, r0, rc, off, cnt, _ in items:
            if qstride < 0:
                qs, j = table[qbase + r0:qbase + r0 + rc].T
            else:
                j, i = np.divmod(np.arange(r0, r0 + rc), qlen)
                qs = qbase + j * qstride + i
            for jj, qq in zip(j[np.isin(qs, rows)], qs[np.isin(qs, rows)]):
                k = pos[int(qq)]
                seen[k] += 1
                got = set(idx[off:off + cnt][((msk[off:off + cnt] >> jj) & 1) == 1].tolist())
                exp = set() if dead[k] else set(np.nonzero(m[k])[0].tolist())
                assert got == exp, int(qq)
        assert (seen == 1).all()


def test_backward_full_size_sampled_rows():
    need_gpu()
    meta, topo, D = _case("c5")
    H = 2
    say("full-size backward c5 S", topo.S)
    tiles = M.build(meta, "cuda").tiles
    # items of <= 32 rows with at least two tiles: the dQ and dK/dV passes
    # split them over two waves / wave pairs (player blocks' ragged last rows
    # and keys, hub streams), and the sampled rows hold such rows
    it = tiles.items[:tiles.n_items].cpu().numpy()
    split = (it[:, 4] <= 32) & (it[:, 6] >= 128)
    assert split.sum() >= 20
    q, k, v = _inputs(topo.S, H, D, seed=23)
    dout = torch.randn(topo.S, H, D, generator=torch.Generator().manual_seed(24)).to(torch.bfloat16)
    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    hier_attention(qd, kd, vd, tiles).backward(dout.cuda())
    torch.cuda.synchronize()
    rows = _rows(topo, np.random.default_rng(6))
    rt = torch.from_numpy(rows)
    say(f"  {len(rows)} sampled rows")
    dq, dk, dv = attention_grads_at(q, k, v, dout, topo, q_rows=rows, k_rows=rows)
    _check("dq", qd.grad.cpu()[rt], dq)
    _check("dk", kd.grad.cpu()[rt], dk)
    _check("dv", vd.grad.cpu()[rt], dv)


def test_membership_gradient_full_size_sampled_bits():
    """C5 with soft membership logits ~ N(0, 1): the logit gradient of the HIP
    STE pass at sampled membership bits (on and off) against the row-sampled
    fp32 oracle ``oracle.ste.ste_grad_at`` (pinned to the autograd
    definition), plus dQ / dK / dV at sampled rows; north-star bounds."""
    need_gpu()
    from oracle.ste import ste_grad_at
    P, T, L, N, KL, KG, n, W, _, D, grp = bench.CONFIGS["c5"]
    logits, mem, go = bench.grouping(grp, P, T, N, np.random.default_rng(bench.SEED))
    topo = FullTopology(P, T, L, N, KL, KG, n, W, True, membership=mem, global_only=go)
    meta = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W, direct=True,
                                    membership=mem, global_only=go)
    H = 4
    say("full-size membership gradient c5 S", topo.S, "H", H)
    tiles = M.build(meta, "cuda").tiles
    q, k, v = _inputs(topo.S, H, D, seed=41)
    dout = torch.randn(topo.S, H, D, generator=torch.Generator().manual_seed(42)).to(torch.bfloat16)
    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    lg = torch.from_numpy(logits).float().cuda().requires_grad_(True)
    out = hier_attention(qd, kd, vd, tiles, membership_logits=lg, ste_geometry=(P, T, L, N, KL))
    out.backward(dout.cuda())
    torch.cuda.synchronize()
    rng = np.random.default_rng(9)
    on = np.argwhere(mem)
    off = np.argwhere(~mem)
    bits = [tuple(int(x) for x in b) for b in on[rng.choice(len(on), 10, replace=False)]]
    bits += [tuple(int(x) for x in b) for b in off[rng.choice(len(off), 3, replace=False)]]
    say(f"  {len(bits)} sampled bits")
    want = ste_grad_at(q, k, v, dout, topo, torch.from_numpy(logits).float(), bits)
    got = lg.grad.cpu().double().numpy()[tuple(np.array(bits).T)]
    err = np.abs(got - want)
    say(f"  dlogits max-abs {err.max():.3e} mean-abs {err.mean():.3e} (ref max "
        f"{np.abs(want).max():.3e})")
    assert np.isfinite(got).all() and np.abs(want[:10]).max() > 0
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS
    assert (got[10:] == 0).all()      # bits that are off gate no edge
    rows = _rows(topo, np.random.default_rng(10), n_random=32)
    rt = torch.from_numpy(rows)
    dq, dk, dv = attention_grads_at(q, k, v, dout, topo, q_rows=rows, k_rows=rows)
    _check("dq", qd.grad.cpu()[rt], dq)
    _check("dk", kd.grad.cpu()[rt], dk)
    _check("dv", vd.grad.cpu()[rt], dv)


def _block_rows(topo, b):
    """Full-sequence rows of temporal block b in the block's own token order
    (players, then local hubs, then global hubs, each frame-major)."""
    P, T, L, N, KL, KG, n = topo.P, topo.T, topo.L, topo.N, topo.KL, topo.KG, topo.n
    f = np.arange(b * n, min(T, b * n + n))
    a0, g0 = P * T * L, P * T * L + T * N * KL
    players = [p * T * L + (f[:, None] * L + np.arange(L)[None]).ravel() for p in range(P)]
    local = (a0 + f[:, None] * N * KL + np.arange(N * KL)[None]).ravel()
    glob = (g0 + f[:, None] * KG + np.arange(KG)[None]).ravel()
    return np.concatenate(players + [local, glob]).astype(np.int64)


def test_rollout_full_size_sampled_rows():
    need_gpu()
    P, T, L, N, KL, KG, n, W, _, D, grp = bench.CONFIGS["c4"]
    H = 2
    _, mem, go = bench.grouping(grp, P, T, N, np.random.default_rng(bench.SEED))
    topo = FullTopology(P, T, L, N, KL, KG, n, W, True, membership=mem, global_only=go)
    act = mem.any(-1)
    say("full-size rollout c4 S", topo.S)
    q, k, v = _inputs(topo.S, H, D, seed=25)
    cache = HierPagedKVCache(num_players=P, num_groups=N, num_patches=L, num_local_hub_tokens=KL,
                             num_global_hub_tokens=KG, num_heads=H, head_dim=D, local_attn_size=W,
                             num_frame_per_block=n, device="cuda")
    rng = np.random.default_rng(7)
    nb = T // n
    for b in range(nb):
        rows = _block_rows(topo, b)
        rt = torch.from_numpy(rows)
        cache.append(k[rt].cuda(), v[rt].cuda(), b * n, n, act[b * n:b * n + n])
        if b < nb - 2:
            continue
        frames, bases, lact = cache.window(b * n + n - 1)
        tiles = M.cached_tiles(device="cuda", P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n, n_block=n,
                               local_attn=W, frames=frames, tile_bases=bases,
                               local_active_frames=lact, labels=None,
                               q_active=act[b * n:b * n + n].tolist(), direct_player=True,
                               membership=mem, global_only=go)
        out = torch.zeros(len(rows), H, D, dtype=torch.bfloat16, device="cuda")
        hier_attention_forward(q[rt].cuda(), cache.k, cache.v, tiles, out)
        torch.cuda.synchronize()
        loc = np.unique(np.concatenate([rng.choice(len(rows), 96, replace=False),
                                        np.arange(P) * n * L, np.arange(P) * n * L + n * L - 1,
                                        np.arange(P * n * L, len(rows))]))
        ref = masked_attention(q, k, v, topo, rows=rows[loc])
        mx, mn = err_stats(out.cpu()[torch.from_numpy(loc)], ref)
        say(f"  block {b}: {len(loc)} sampled rows, max-abs {mx:.3e} mean-abs {mn:.3e}")
        assert mx <= MAX_ABS and mn <= MEAN_ABS
