"""Action branches' cached attention on the GPU: the frame-window attention
kernel against the oracle's masked SDPA, and the mouse temporal /
keyboard cached attention over a rollout (every block run twice) against the
full-sequence computation with the same mask, which an in-order rollout
equals.  Bound: max-abs 2e-2, mean-abs 2e-3 against fp32."""

import copy
import math

import pytest
import torch
from torch import nn

from multics_amd.action import (
    action_keyboard_cached_attention,
    action_temporal_cached_attention,
    frame_attention,
)
from multics_amd.rope import precompute_freqs_cis
from oracle.cached import _sdpa, _temporal
from tests.gpu_util import err_stats, need_gpu, say

pytestmark = pytest.mark.gpu
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("local_attn", [-1, 5])
def test_frame_attention_matches_oracle(D, local_attn):
    need_gpu()
    say("frame attention", D, local_attn)
    g = torch.Generator().manual_seed(D + local_attn)
    B, H, n_block = 5, 3, 3
    for Lq, Lk, q0 in ((3, 24, 21), (7 * 4, 9 * 2, 6), (1, 1, 0)):
        qf = q0 + torch.arange(Lq) * 3 // max(Lq, 1)        # a few frames, in order
        kf = torch.arange(Lk) * (q0 + 3) // max(Lk, 1)
        q, k, v = ((torch.randn(B, L, H, D, generator=g)).to(torch.bfloat16) for L in (Lq, Lk, Lk))
        got = frame_attention(q.cuda(), k.cuda(), v.cuda(), qf, kf, n_block, local_attn)
        torch.cuda.synchronize()
        m = _temporal(qf, kf, n_block, local_attn)
        ref = torch.stack([_sdpa(q[b], k[b], v[b], m, 1 / math.sqrt(D)) for b in range(B)])
        mx, mn = err_stats(got, ref)
        say(f"  Lq {Lq} Lk {Lk}: max-abs {mx:.3e} mean-abs {mn:.3e}")
        assert mx <= MAX_ABS and mn <= MEAN_ABS


class _Attn(nn.Module):
    """The attributes the reference's cached action attention reads."""

    def __init__(self, dim, nh, seed):
        super().__init__()
        torch.manual_seed(seed)
        self.num_heads = nh
        self.q, self.k, self.v, self.o = (nn.Linear(dim, dim) for _ in range(4))
        self.norm_q, self.norm_k = nn.RMSNorm(dim, eps=1e-6), nn.RMSNorm(dim, eps=1e-6)
        for lin in (self.q, self.k, self.v, self.o):
            nn.init.normal_(lin.weight, std=0.05)


def _roped(x, freqs, nh):
    b, s, dim = x.shape
    xc = torch.view_as_complex(x.double().reshape(b, s, nh, -1, 2))
    return torch.view_as_real(xc * freqs).flatten(2).float()


def test_temporal_cached_rollout_matches_full_sequence():
    need_gpu()
    B, T, n, W, nh, hd = 6, 12, 3, 4, 2, 128
    dim = nh * hd
    gpu = _Attn(dim, nh, seed=2).to("cuda", torch.bfloat16)
    ref_attn = copy.deepcopy(gpu).float().cpu()       # the same bf16 weights, in fp32
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, T, dim, generator=g).to(torch.bfloat16).float()
    freqs = precompute_freqs_cis(hd, end=T).unsqueeze(1)          # [T, 1, hd/2]
    with torch.no_grad():
        qf = _roped(ref_attn.norm_q(ref_attn.q(x)), freqs, nh).view(B, T, nh, hd)
        kf = _roped(ref_attn.norm_k(ref_attn.k(x)), freqs, nh).view(B, T, nh, hd)
        vf = ref_attn.v(x).view(B, T, nh, hd)
    cache = {}
    for b0 in range(0, T, n):
        xb = x[:, b0:b0 + n].to("cuda", torch.bfloat16)
        for rep in range(2):
            say(f"temporal block {b0 // n} pass {rep}")
            with torch.no_grad():
                y = action_temporal_cached_attention(gpu, xb, freqs[b0:b0 + n].cuda(), cache,
                                                     b0, n, W)
            torch.cuda.synchronize()
        m = _temporal(torch.arange(b0, b0 + n), torch.arange(0, b0 + n), n, W)
        att = torch.stack([_sdpa(qf[i, b0:b0 + n], kf[i, :b0 + n], vf[i, :b0 + n], m,
                                 1 / math.sqrt(hd)) for i in range(B)])
        with torch.no_grad():
            ref = ref_attn.o(att.reshape(B, n, dim))
        mx, mn = err_stats(y, ref)
        say(f"  max-abs {mx:.3e} mean-abs {mn:.3e}")
        assert mx <= MAX_ABS and mn <= MEAN_ABS


def test_keyboard_cached_rollout_matches_full_sequence():
    need_gpu()
    B, T, n, W, nh, hd, patches, tpf = 2, 9, 3, 4, 2, 64, 10, 2
    dim = nh * hd
    gpu = _Attn(dim, nh, seed=5).to("cuda", torch.bfloat16)
    ref_attn = copy.deepcopy(gpu).float().cpu()
    g = torch.Generator().manual_seed(6)
    # video tokens and keyboard tokens, frame-major
    xv = torch.randn(B, T * patches, dim, generator=g).to(torch.bfloat16).float()
    kbd = torch.randn(B, T * tpf, dim, generator=g).to(torch.bfloat16).float()
    with torch.no_grad():
        qf = ref_attn.norm_q(ref_attn.q(xv)).view(B, T * patches, nh, hd)
        kf = ref_attn.norm_k(ref_attn.k(kbd)).view(B, T * tpf, nh, hd)
        vf = ref_attn.v(kbd).view(B, T * tpf, nh, hd)
    cache = {}
    for b0 in range(0, T, n):
        xb = xv[:, b0 * patches:(b0 + n) * patches].to("cuda", torch.bfloat16)
        kb = kbd[:, b0 * tpf:(b0 + n) * tpf].to("cuda", torch.bfloat16)
        for rep in range(2):
            say(f"keyboard block {b0 // n} pass {rep}")
            with torch.no_grad():
                y = action_keyboard_cached_attention(gpu, xb, kb, cache, b0, n, W, patches, tpf)
            torch.cuda.synchronize()
        qfr = torch.arange(b0, b0 + n).repeat_interleave(patches)
        kfr = torch.arange(0, (b0 + n) * tpf) // tpf
        m = _temporal(qfr, kfr, n, W)
        att = torch.stack([_sdpa(qf[i, b0 * patches:(b0 + n) * patches], kf[i, :(b0 + n) * tpf],
                                 vf[i, :(b0 + n) * tpf], m, 1 / math.sqrt(hd)) for i in range(B)])
        with torch.no_grad():
            ref = ref_attn.o(att.reshape(B, -1, dim))
        mx, mn = err_stats(y, ref)
        say(f"  max-abs {mx:.3e} mean-abs {mn:.3e}")
        assert mx <= MAX_ABS and mn <= MEAN_ABS
