"""The allocation-free backward entry point ``hier_attn_bwd_noalloc``.

Called through the C ABI (via ``hier_attention_backward(...,
no_alloc_workspace=True)``, which passes NULL delta / lse2 and lets the
library use its own device array) and compared with ``hier_attn_bwd`` on the
same inputs: the kernels are the same and deterministic, so dQ / dK / dV and
the membership-STE sums must be bit-identical.  Two calls in a row, the second
on a smaller input, so that the second also shows that the array's leftovers
from the first call do not leak into it; then a workspace request beyond the
array's size is refused.
"""

import numpy as np
import pytest
import torch

from multics_amd import metadata as M
from multics_amd.kernels import hier_attention_backward, hier_attention_forward
from tests.gpu_util import need_gpu, say

pytestmark = pytest.mark.gpu


def _case(P, T, L, N, KL, KG, n, W, H, D, seed):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((T, N, P))
    mem = logits > 0
    go = ~mem.any(1)
    full = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W, direct=True,
                                    membership=mem, global_only=go)
    tiles = M.build(full, "cuda").tiles
    S = P * T * L + T * (N * KL + KG)
    g = torch.Generator().manual_seed(seed)
    q, k, v = ((torch.randn(S, H, D, generator=g) * 0.5).to(torch.bfloat16).cuda()
               for _ in range(3))
    dout = torch.randn(S, H, D, generator=g).to(torch.bfloat16).cuda()
    out = torch.zeros(S, H, D, dtype=torch.bfloat16, device="cuda")
    lse = torch.full((H, S), float("-inf"), dtype=torch.float32, device="cuda")
    hier_attention_forward(q, k, v, tiles, out, lse=lse)
    return q, k, v, out, dout, lse, tiles, (P, T, L, N, KL)


CASES = [
    # P, T, L, N, KL, KG, n, W, H, D, seed   (the second is smaller)
    (4, 6, 40, 2, 5, 6, 3, 4, 4, 128, 1),
    (3, 3, 16, 2, 2, 3, 3, -1, 2, 64, 2),
]


def test_noalloc_backward_matches_hier_attn_bwd():
    need_gpu()
    for case in CASES:
        say("noalloc backward", case)
        q, k, v, out, dout, lse, tiles, geo = _case(*case)
        want = hier_attention_backward(q, k, v, out, dout, lse, tiles, ste_geometry=geo)
        got = hier_attention_backward(q, k, v, out, dout, lse, tiles, ste_geometry=geo,
                                      no_alloc_workspace=True)
        torch.cuda.synchronize()
        for name, a, b in zip(("dq", "dk", "dv", "ste"), got, want):
            assert torch.equal(a, b), name
        assert want[0].abs().sum() > 0 and want[3].abs().sum() > 0


def test_noalloc_backward_refuses_oversize_workspace():
    need_gpu()
    q, k, v, out, dout, lse, tiles, _ = _case(*CASES[1])
    H = q.shape[1]
    big = torch.full((H, 2_100_000), float("-inf"), dtype=torch.float32, device="cuda")
    big[:, :lse.shape[1]] = lse
    say("noalloc backward, oversize workspace")
    with pytest.raises(NotImplementedError, match="workspace"):
        hier_attention_backward(q, k, v, out, dout, big, tiles, no_alloc_workspace=True)
    # the ordinary entry point takes the same request with a caller workspace
    hier_attention_backward(q, k, v, out, dout, big, tiles)
    torch.cuda.synchronize()
