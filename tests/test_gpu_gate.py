"""Gated residual after self-attention (``hier_gated_residual``) against the
reference expression ``x + gate * residual`` (multics/models/blocks.py:31-35)
evaluated by torch in bf16 on the same GPU: bit-identical, for the compact
per-frame gate and for the materialised one, in place and out of place."""

import pytest
import torch

from multics_amd.kernels import gated_residual
from multics_amd.module import GateModule
from tests.gpu_util import need_gpu, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(4, 42, 220, 3072), (2, 3, 5, 64), (1, 7, 1, 1024),
                                   (3, 2, 33, 136)])
def test_gated_residual_bit_identical_to_torch(shape):
    need_gpu()
    B, F, L, dim = shape
    say("gated residual", shape)
    g = torch.Generator(device="cuda").manual_seed(3)
    rnd = lambda *s: torch.randn(*s, generator=g, device="cuda").to(torch.bfloat16)
    x, res = rnd(B, F * L, dim), rnd(B, F * L, dim)
    gate = rnd(B, F, dim)
    full = gate.unsqueeze(2).expand(-1, -1, L, -1).reshape(B, F * L, dim)
    want = x + full * res
    assert torch.equal(gated_residual(x, gate, res), want)
    assert torch.equal(GateModule()(x, full, res), want)
    y = x.clone()
    gated_residual(y, gate, res, out=y)
    torch.cuda.synchronize()
    assert torch.equal(y, want)


def test_gated_residual_argument_errors():
    need_gpu()
    x = torch.zeros(2, 10, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        gated_residual(x, torch.zeros(2, 3, 64, dtype=torch.bfloat16, device="cuda"), x)
    with pytest.raises(NotImplementedError):
        gated_residual(x.float(), x.float(), x.float())
    with pytest.raises(ValueError):
        gated_residual(x, x, x[:, :5])
