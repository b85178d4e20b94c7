"""The membership producer feeding the attention path end to end.

Labels generated from a bundled tick state (the P6 and P10 synthetic
fixtures, whose groups change between periods, and a real 4-player clip) give the
``membership`` / ``global_only`` topology; the HIP metadata builder turns it
into a tile list, the forward runs on it at the C2 / C3 geometry (220 tokens
per player-frame, 42 latent frames, window 21), and sampled rows are compared
with the dense-mask oracle of the same topology (forward max-abs 2e-2 /
mean-abs 2e-3; the tile list's key set of every sampled row equal to its mask
row); the drop-in block-mask builder fed the same payload builds the same
tile list.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from multics_amd import metadata as M
from multics_amd.grouping import GroupingState, generate_labels, membership_inputs
from multics_amd.hier_masks import build_stage2_hier_flex_block_mask
from multics_amd.kernels import hier_attention_forward
from oracle.attention import masked_attention
from oracle.masks import FullTopology, inactive_local_rows, mask_rows
from tests.gpu_util import err_stats, need_gpu, say
from tests.test_gpu_fullsize import _check_key_sets, _inputs, _rows

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).parent / "golden" / "grouping"
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


@pytest.mark.parametrize("case", ["p6_moving_pairs", "p10_moving_pairs", "example_4_01"])
def test_generated_membership_drives_the_forward(case):
    need_gpu()
    state = GroupingState.load(GOLD / f"{case}.state.npz")
    mem, go = membership_inputs(generate_labels(state))
    T, N, P = mem.shape
    L, KL, KG, n, W, H, D = 220, 5, 6, 3, 21, 2, 128
    meta = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W, direct=True,
                                    membership=mem, global_only=go)
    topo = FullTopology(P, T, L, N, KL, KG, n, W, True, membership=mem, global_only=go)
    say("generated membership", case, "P", P, "S", topo.S)
    tiles = M.build(meta, "cuda").tiles
    q, k, v = _inputs(topo.S, H, D, seed=41)
    out = torch.zeros(topo.S, H, D, dtype=torch.bfloat16, device="cuda")
    hier_attention_forward(q.cuda(), k.cuda(), v.cuda(), tiles, out)
    torch.cuda.synchronize()
    rows = _rows(topo, np.random.default_rng(7))
    ref = masked_attention(q, k, v, topo, rows=rows)
    got = out.cpu()[torch.from_numpy(rows)]
    mx, mn = err_stats(got, ref)
    say(f"  {len(rows)} rows: max-abs {mx:.3e} mean-abs {mn:.3e}")
    assert mx <= MAX_ABS and mn <= MEAN_ABS
    m = mask_rows(topo, q_idx=rows)
    _check_key_sets(tiles, rows, m, inactive_local_rows(topo)[rows])
    # the drop-in block-mask builder takes the same payload as torch tensors
    bm, S, _ = build_stage2_hier_flex_block_mask(P, T, L, N, KL, KG, n, W, None, None, True, "cuda",
                                                 membership=torch.from_numpy(mem),
                                                 global_only=torch.from_numpy(go))
    assert S == topo.S and bm.tiles.n_items == tiles.n_items
    assert torch.equal(bm.tiles.items[:tiles.n_items].cpu(), tiles.items[:tiles.n_items].cpu())
    # the lists the items reference (merged hub slots keep unreferenced slack)
    it = tiles.items[:tiles.n_items].cpu().numpy()
    for name in ("kv_idx", "kv_mask"):
        a_, b_ = getattr(bm.tiles, name).cpu().numpy(), getattr(tiles, name).cpu().numpy()
        for off, cnt in {(int(o), int(c)) for o, c in it[:, 5:7]}:
            assert np.array_equal(a_[off:off + cnt], b_[off:off + cnt]), name
