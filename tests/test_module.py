"""CPU checks of the drop-in SelfAttention (multics/models/attention.py:231-442)."""

import numpy as np
import pytest
import torch

from multics_amd.module import CompatibleLinear, RMSNorm, SelfAttention, rope_apply
from oracle.attention import bf16, rms_norm
from oracle.attention import rope_apply as oracle_rope


def test_state_dict_keys_match_reference():
    m = SelfAttention(64, 4)
    keys = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert keys == {"q.weight": (64, 64), "q.bias": (64,), "k.weight": (64, 64), "k.bias": (64,),
                    "v.weight": (64, 64), "v.bias": (64,), "o.weight": (64, 64), "o.bias": (64,),
                    "norm_q.weight": (64,), "norm_k.weight": (64,)}
    m.enable_camera_pose_qk(12, dropout_p=0.0)
    keys = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert keys["cam_q.weight"] == (64, 12) and keys["cam_k.weight"] == (64, 12)
    assert "cam_q.bias" not in keys and torch.count_nonzero(m.cam_q.weight) == 0
    assert (m.sink_size, m.local_attn_size, m.num_frame_per_block, m.attn_impl) == (0, 6, 7, "sdpa")


def test_rmsnorm_matches_oracle():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 32, generator=g).to(torch.bfloat16)
    n = RMSNorm(32, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        n.weight.copy_(torch.rand(32, generator=g) + 0.5)
    assert torch.equal(n(x).float(), rms_norm(x, n.weight, 1e-6))


def test_rope_matches_oracle():
    g = torch.Generator().manual_seed(1)
    S, H, D = 7, 2, 16
    x = torch.randn(1, S, H * D, generator=g).to(torch.bfloat16)
    ang = torch.rand(S, 1, D // 2, generator=g, dtype=torch.float64) * 6.28
    freqs = torch.polar(torch.ones_like(ang), ang)
    assert torch.equal(rope_apply(x, freqs, H)[0].float(), oracle_rope(x[0], freqs, H))


def test_errors_match_reference_behaviour():
    m = SelfAttention(32, 2)
    x = torch.randn(1, 5, 32)
    freqs = torch.ones(5, 1, 8, dtype=torch.complex128)
    with pytest.raises(RuntimeError):
        m.forward(x, freqs, cam_tokens=torch.zeros(1, 5, 12))
    m.enable_camera_pose_qk(12, dropout_p=0.0)
    with pytest.raises(ValueError):
        m.forward(x, freqs, cam_tokens=torch.zeros(1, 4, 12))
    with pytest.raises(ValueError):
        m.enable_camera_pose_qk(12, dropout_p=1.5)
    with pytest.raises(NotImplementedError):
        m.forward(x, freqs, mask=object())
    with pytest.raises(ValueError):
        CompatibleLinear(4, 4, input_alignment=0)


def test_dense_mask_forward_is_sdpa():
    torch.manual_seed(0)
    m = SelfAttention(32, 2)
    x = torch.randn(1, 6, 32)
    freqs = torch.ones(6, 1, 8, dtype=torch.complex128)
    mask = torch.tril(torch.ones(6, 6, dtype=torch.bool))
    y = m.forward(x, freqs, mask=mask)
    q, k, v = m._project_self_attn_qkv(x, freqs)
    split = lambda t: t.view(1, 6, 2, 16).transpose(1, 2)
    s = split(q) @ split(k).transpose(-1, -2) / 4.0
    p = torch.softmax(s.masked_fill(~mask, float("-inf")), -1)
    ref = m.o((p @ split(v)).transpose(1, 2).reshape(1, 6, 32))
    assert torch.allclose(y, ref, atol=1e-5)
