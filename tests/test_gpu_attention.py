"""HIP forward attention against the fp32 dense-mask oracle.

Tolerance (the parity bar of this path): max-abs <= 2e-2 and mean-abs <= 2e-3 on the
bf16 outputs against an fp32 reference computed from the same bf16 inputs.
"""

import math

import numpy as np
import pytest
import torch

from multics_amd import metadata as M
from multics_amd.kernels import (
    hier_attention_forward,
    hierarchical_tiled_full_sequence_attention,
)
from oracle.attention import masked_attention
from oracle.masks import FullTopology
from tests.gpu_util import err_stats, need_gpu, say

pytestmark = pytest.mark.gpu
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _inputs(S, H, D, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(S, H, D, generator=g) * scale).to(torch.bfloat16) for _ in range(3)]


CASES = [
    # name, P, T, L, N, KL, KG, n, W, H, D, direct
    ("c1_n1", 4, 3, 64, 2, 1, 1, 1, -1, 4, 64, True),
    ("c1_n3_w21", 4, 3, 64, 2, 1, 1, 3, 21, 4, 64, True),
    ("c2_shrunk_w4", 4, 9, 20, 2, 5, 6, 3, 4, 2, 128, True),
    ("c2_shrunk_nodirect", 4, 9, 20, 2, 5, 6, 3, -1, 2, 128, False),
    ("ragged_rows", 3, 6, 37, 3, 2, 3, 2, 4, 2, 128, True),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_forward_matches_oracle_labels(case):
    need_gpu()
    name, P, T, L, N, KL, KG, n, W, H, D, direct = case
    say("forward labels", name)
    labels = np.array([[p % N for p in range(P)]] * T)
    if T >= 2 * n:  # regroup between blocks
        labels[n:2 * n] = [(p + 1) % N for p in range(P)]
    active = np.zeros((T, N), dtype=bool)
    active[np.arange(T)[:, None], labels] = True
    topo = FullTopology(P, T, L, N, KL, KG, n, W, direct, labels=labels, active=active)
    q, k, v = _inputs(topo.S, H, D, seed=0)
    tiles = M.build(M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                             direct=direct, labels=labels, active=active),
                    "cuda").tiles
    out = torch.zeros(topo.S, H, D, dtype=torch.bfloat16, device="cuda")
    lse = torch.full((H, topo.S), float("nan"), dtype=torch.float32, device="cuda")
    hier_attention_forward(q.cuda(), k.cuda(), v.cuda(), tiles, out, lse=lse)
    torch.cuda.synchronize()
    ref = masked_attention(q, k, v, topo)
    mx, mn = err_stats(out, ref)
    say(f"  max-abs {mx:.3e} mean-abs {mn:.3e}")
    assert mx <= MAX_ABS and mn <= MEAN_ABS
    assert torch.isfinite(out.float()).all()
    # log-sum-exp of the visible scores
    from oracle.masks import inactive_local_rows, mask_rows
    m = torch.from_numpy(mask_rows(topo))
    s = torch.einsum("qhd,khd->hqk", q.float(), k.float()) / math.sqrt(D)
    ref_lse = torch.logsumexp(s.masked_fill(~m[None], float("-inf")), dim=-1)
    dead = torch.from_numpy(inactive_local_rows(topo))
    got = lse.cpu()
    assert torch.isneginf(got[:, dead]).all()
    # the kernel's row sum adds the bf16-rounded weights that multiply V, so
    # its normaliser differs from an fp32 sum by at most 2^-9 relative
    assert (got[:, ~dead] - ref_lse[:, ~dead]).abs().max() < 2.0 ** -8


def test_forward_dynamic_membership_matches_oracle():
    need_gpu()
    rng = np.random.default_rng(7)
    P, T, L, N, KL, KG, n, W, H, D = 6, 6, 24, 3, 2, 3, 3, 4, 2, 128
    mem = rng.random((T, N, P)) < 0.35
    go = ~mem.any(1) & (rng.random((T, P)) < 0.6)
    for direct in (False, True):
        say("forward membership direct", direct)
        topo = FullTopology(P, T, L, N, KL, KG, n, W, direct, membership=mem, global_only=go)
        q, k, v = _inputs(topo.S, H, D, seed=1)
        tiles = M.build(M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                                 direct=direct, membership=mem, global_only=go),
                        "cuda").tiles
        out = torch.zeros(topo.S, H, D, dtype=torch.bfloat16, device="cuda")
        hier_attention_forward(q.cuda(), k.cuda(), v.cuda(), tiles, out)
        torch.cuda.synchronize()
        ref = masked_attention(q, k, v, topo)
        mx, mn = err_stats(out, ref)
        say(f"  max-abs {mx:.3e} mean-abs {mn:.3e}")
        assert mx <= MAX_ABS and mn <= MEAN_ABS


def test_reference_api_tiled_full_sequence_attention():
    """Drop-in call shape: layouts from build_hier_tiled_full_sequence_layouts."""
    need_gpu()
    P, T, L, N, KL, KG, n, W, H, D = 2, 3, 17, 3, 2, 2, 3, 7, 1, 128
    labels = torch.tensor([[0, 1]] * T)
    active = torch.tensor([[True, True, False]] * T)
    say("reference API tiled full-sequence")
    lays = M.build_hier_tiled_full_sequence_layouts(
        device="cuda", num_players=P, num_frames=T, num_patches=L, num_groups=N,
        num_local_hub_tokens=KL, num_global_hub_tokens=KG, num_frame_per_block=n,
        local_attn_size=W, group_labels=labels, active_group=active, direct_player=True)
    topo = FullTopology(P, T, L, N, KL, KG, n, W, True, labels=labels.numpy(), active=active.numpy())
    q, k, v = _inputs(topo.S, H, D, seed=2)
    y = hierarchical_tiled_full_sequence_attention(
        roped_q=q[None].cuda(), roped_k=k[None].cuda(), value=v[None].cuda(), layouts=lays)
    torch.cuda.synchronize()
    ref = masked_attention(q, k, v, topo).reshape(1, topo.S, H * D)
    mx, mn = err_stats(y, ref)
    assert mx <= MAX_ABS and mn <= MEAN_ABS
    with pytest.raises(NotImplementedError):
        hierarchical_tiled_full_sequence_attention(
            roped_q=q[None].float().cuda(), roped_k=k[None].float().cuda(),
            value=v[None].float().cuda(), layouts=lays)
    with pytest.raises(ValueError):
        hierarchical_tiled_full_sequence_attention(
            roped_q=q[None].cuda(), roped_k=k[None, :-1].cuda(), value=v[None].cuda(), layouts=lays)
