"""Drop-in SelfAttention on the GPU: the hierarchical training path (torch
projections + HIP attention forward/backward), the no-grad fused path (HIP
prologue + HIP forward) and the membership STE entry point, against the fp32
dense-mask oracle of the same projected Q/K/V."""

import math

import numpy as np
import pytest
import torch

from multics_amd import metadata as M
from multics_amd.module import SelfAttention
from oracle.attention import masked_attention
from oracle.masks import FullTopology
from oracle.ste import ste_attention
from tests.gpu_util import err_stats, need_gpu, say

pytestmark = pytest.mark.gpu


def _module(dim, H, seed, cam=True):
    torch.manual_seed(seed)
    m = SelfAttention(dim, H, eps=1e-6)
    for lin in (m.q, m.k, m.v, m.o):
        torch.nn.init.normal_(lin.weight, std=0.02)
        torch.nn.init.normal_(lin.bias, std=0.02)
    with torch.no_grad():
        m.norm_q.weight.uniform_(0.5, 1.5)
        m.norm_k.weight.uniform_(0.5, 1.5)
    if cam:
        m.enable_camera_pose_qk(12, dropout_p=0.0)
        torch.nn.init.normal_(m.cam_q.weight, std=0.05)
        torch.nn.init.normal_(m.cam_k.weight, std=0.05)
    return m.to("cuda", torch.bfloat16)


def _freqs(S, D, seed):
    g = torch.Generator().manual_seed(seed)
    ang = torch.rand(S, 1, D // 2, generator=g, dtype=torch.float64) * 6.283
    return torch.polar(torch.ones_like(ang), ang)


def _rel(a, b):
    return ((a.float() - b.float()).abs().max() / b.float().abs().max().clamp_min(1e-12)).item()


def _rel_mean(a, b):
    return ((a.float() - b.float()).abs().mean() / b.float().abs().mean().clamp_min(1e-12)).item()


def test_forward_hier_tiled_ste_training_and_inference():
    need_gpu()
    P, T, L, N, KL, KG, n, W, H, D = 4, 6, 20, 2, 5, 6, 3, 4, 2, 128
    dim = H * D
    m = _module(dim, H, seed=0)
    m.num_frame_per_block, m.local_attn_size = n, W
    labels = torch.tensor([[p // 2 for p in range(P)]] * T)
    active = torch.ones(T, N, dtype=torch.bool)
    topo = FullTopology(P, T, L, N, KL, KG, n, W, True, labels=labels.numpy(), active=active.numpy())
    S = topo.S
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, S, dim, generator=g).to("cuda", torch.bfloat16)
    cam = torch.randn(1, S, 12, generator=g).to("cuda", torch.bfloat16)
    freqs = _freqs(S, D, 2)
    kw = dict(group_labels=labels, active_group=active, num_players=P, num_frames=T, num_patches=L,
              num_groups=N, num_local_hub_tokens=KL, num_global_hub_tokens=KG, direct_player=True,
              cam_tokens=cam)
    say("module training path", S)
    xg = x.clone().requires_grad_(True)
    y = m.forward_hier_tiled_ste(xg, freqs, None, **kw)
    dy = torch.randn(1, S, dim, generator=g).to("cuda", torch.bfloat16)
    y.backward(dy)
    torch.cuda.synchronize()
    # oracle: same projections, fp32 dense-mask attention, same output projection
    with torch.no_grad():
        q, k, v = m._project_self_attn_qkv(x, freqs, cam)
        att = masked_attention(*(t.view(S, H, D).cpu() for t in (q, k, v)), topo)
        ref = torch.nn.functional.linear(att.reshape(1, S, dim), m.o.weight.float().cpu(),
                                         m.o.bias.float().cpu())
    mx, mn = err_stats(y.detach(), ref)
    say(f"  training output max-abs {mx:.3e} mean-abs {mn:.3e}")
    assert mx <= 2e-2 and mn <= 2e-3
    assert torch.isfinite(xg.grad.float()).all() and xg.grad.abs().sum() > 0
    for p_ in (m.q.weight, m.k.weight, m.v.weight, m.norm_q.weight, m.cam_q.weight):
        assert p_.grad is not None and torch.isfinite(p_.grad.float()).all()

    say("module no-grad fused path")
    with torch.no_grad():
        y2 = m.forward_hier_tiled_ste(x, freqs, None, **kw)
    torch.cuda.synchronize()
    mx, mn = err_stats(y2, ref)
    say(f"  fused output max-abs {mx:.3e} mean-abs {mn:.3e}")
    assert mx <= 2e-2 and mn <= 2e-3


def test_module_gradients_match_fp32_autograd():
    """dL/dx and dL/dW_v through the HIP backward against fp32 autograd of the
    same module math with the oracle attention: max error <= 2e-2 x the
    largest entry, mean error <= 1e-2 x the mean magnitude (bf16 projections
    and bf16 weight gradients on one side, fp32 on the other)."""
    need_gpu()
    P, T, L, N, KL, KG, n, W, H, D = 2, 3, 16, 2, 2, 2, 3, -1, 2, 64
    dim = H * D
    m = _module(dim, H, seed=3, cam=False)
    m.num_frame_per_block, m.local_attn_size = n, W
    labels = torch.tensor([[0, 1]] * T)
    active = torch.ones(T, N, dtype=torch.bool)
    topo = FullTopology(P, T, L, N, KL, KG, n, W, True, labels=labels.numpy(), active=active.numpy())
    S = topo.S
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, S, dim, generator=g).to(torch.bfloat16)
    dy = torch.randn(1, S, dim, generator=g).to(torch.bfloat16)
    freqs = _freqs(S, D, 6)
    say("module gradients", S)
    xg = x.cuda().requires_grad_(True)
    y = m.forward_hier_tiled_ste(xg, freqs, None, group_labels=labels, active_group=active,
                                 num_players=P, num_frames=T, num_patches=L, num_groups=N,
                                 num_local_hub_tokens=KL, num_global_hub_tokens=KG,
                                 direct_player=True)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    mf = SelfAttention(dim, H, eps=1e-6)
    mf.load_state_dict({k_: v_.float().cpu() for k_, v_ in m.state_dict().items()})
    mf.num_frame_per_block, mf.local_attn_size = n, W
    xf = x.float().requires_grad_(True)
    q, k, v = mf._project_self_attn_qkv(xf, freqs)
    att = masked_attention(q.view(S, H, D), k.view(S, H, D), v.view(S, H, D), topo)
    yf = mf.o(att.reshape(1, S, dim))
    yf.backward(dy.float())
    say(f"  dx rel {_rel(xg.grad.cpu(), xf.grad):.3e}  dWv rel "
        f"{_rel(m.v.weight.grad.cpu(), mf.v.weight.grad):.3e}  dWq rel "
        f"{_rel(m.q.weight.grad.cpu(), mf.q.weight.grad):.3e}")
    for got, want in ((xg.grad.cpu(), xf.grad), (m.v.weight.grad.cpu(), mf.v.weight.grad),
                      (m.q.weight.grad.cpu(), mf.q.weight.grad)):
        assert _rel(got, want) < 2e-2 and _rel_mean(got, want) < 1e-2


def test_forward_hier_membership_logits():
    need_gpu()
    P, T, L, N, KL, KG, n, W, H, D = 4, 6, 16, 2, 5, 6, 3, 4, 2, 128
    dim = H * D
    m = _module(dim, H, seed=7, cam=False)
    m.num_frame_per_block, m.local_attn_size = n, W
    rng = np.random.default_rng(8)
    logits = torch.from_numpy(rng.standard_normal((T, N, P))).float()
    mem = (logits > 0).numpy()
    topo = FullTopology(P, T, L, N, KL, KG, n, W, True, membership=mem, global_only=~mem.any(1))
    S = topo.S
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, S, dim, generator=g).to("cuda", torch.bfloat16)
    freqs = _freqs(S, D, 10)
    say("module membership logits", S)
    lg = logits.cuda().requires_grad_(True)
    y = m.forward_hier_membership(x, freqs, num_players=P, num_frames=T, num_patches=L,
                                  num_groups=N, num_local_hub_tokens=KL, num_global_hub_tokens=KG,
                                  direct_player=True, membership_logits=lg)
    dy = torch.randn(1, S, dim, generator=g).to("cuda", torch.bfloat16)
    y.backward(dy)
    torch.cuda.synchronize()
    with torch.no_grad():
        q, k, v = m._project_self_attn_qkv(x, freqs)
    q4, k4, v4 = (t.view(S, H, D).float().cpu().requires_grad_(True) for t in (q, k, v))
    lf = logits.clone().requires_grad_(True)
    att = ste_attention(q4, k4, v4, topo, lf)
    yo = torch.nn.functional.linear(att.reshape(1, S, dim), m.o.weight.float().cpu(),
                                    m.o.bias.float().cpu())
    yo.backward(dy.float().cpu())
    mx, _ = err_stats(y.detach(), yo.detach())
    say(f"  output max-abs {mx:.3e}  dlogits rel {_rel(lg.grad.cpu(), lf.grad):.3e}")
    assert mx <= 2e-2
    err = (lg.grad.cpu() - lf.grad).abs()
    assert err.max() <= 2e-2 and err.mean() <= 2e-3
    assert _rel(lg.grad.cpu(), lf.grad) < 2e-2


FLEX_CASES = [
    # name, P, T, L, N, KL, KG, n, W, H, D, kind
    ("labels_inactive", 4, 6, 20, 3, 5, 6, 3, 4, 2, 128, "labels"),
    ("membership", 4, 6, 16, 2, 5, 6, 3, -1, 2, 64, "membership"),
]


@pytest.mark.parametrize("case", FLEX_CASES, ids=[c[0] for c in FLEX_CASES])
def test_flex_block_mask_path(case):
    """The production call path: ``build_stage2_hier_flex_block_mask`` as
    WanModel.forward calls it (positional arguments, wan_video_dit.py:639-655),
    then ``SelfAttention.forward(x, freqs, mask, cam_tokens=...)`` as
    blocks.py:203 calls it.  Against the dense-mask SDPA of the same projected
    Q/K/V (the mask the Flex BlockMask encodes, including an inactive hub
    row's self edge) in fp32, for the output and, under autograd, for dL/dx
    and the weight gradients; the no-grad (fused prologue) path too."""
    need_gpu()
    from multics_amd.hier_masks import HierBlockMask, build_stage2_hier_flex_block_mask
    from oracle.masks import inactive_local_rows, mask_rows
    name, P, T, L, N, KL, KG, n, W, H, D, kind = case
    dim = H * D
    m = _module(dim, H, seed=11)
    m.num_frame_per_block, m.local_attn_size = n, W
    rng = np.random.default_rng(12)
    if kind == "labels":
        labels = torch.tensor([[p % 2 for p in range(P)]] * T)        # slot 2 never used
        topo = FullTopology(P, T, L, N, KL, KG, n, W, True, labels=labels.numpy())
        mask, S, S_pad = build_stage2_hier_flex_block_mask(P, T, L, N, KL, KG, n, W, labels,
                                                           None, True, "cuda")
    else:
        mem = np.repeat(rng.random((T // n, N, P)) < 0.5, n, axis=0)
        go = ~mem.any(1)
        topo = FullTopology(P, T, L, N, KL, KG, n, W, True, membership=mem, global_only=go)
        mask, S, S_pad = build_stage2_hier_flex_block_mask(
            P, T, L, N, KL, KG, n, W, None, None, True, "cuda",
            membership=torch.from_numpy(mem), global_only=torch.from_numpy(go))
    assert isinstance(mask, HierBlockMask) and S == topo.S and S_pad % 128 == 0
    assert mask.shape[-1] == S_pad
    dead = inactive_local_rows(topo)
    assert len(mask.self_rows) == dead.sum() and (kind != "labels" or dead.any())
    g = torch.Generator().manual_seed(13)
    x = torch.randn(1, S, dim, generator=g).to("cuda", torch.bfloat16)
    cam = torch.randn(1, S, 12, generator=g).to("cuda", torch.bfloat16)
    dy = torch.randn(1, S, dim, generator=g).to("cuda", torch.bfloat16)
    freqs = _freqs(S, D, 14)
    say("flex block-mask path", name, S)
    xg = x.clone().requires_grad_(True)
    y = m(xg, freqs, mask, cam_tokens=cam)
    y.backward(dy)
    with torch.no_grad():
        y_ng = m(x, freqs, mask, cam_tokens=cam)
    torch.cuda.synchronize()
    # fp32 reference: the module's math with dense-mask SDPA
    mf = SelfAttention(dim, H, eps=1e-6)
    mf.enable_camera_pose_qk(12, dropout_p=0.0)
    mf.load_state_dict({k_: v_.float().cpu() for k_, v_ in m.state_dict().items()})
    xf = x.float().cpu().requires_grad_(True)
    q, k, v = mf._project_self_attn_qkv(xf, freqs, cam.float().cpu())
    dm = torch.from_numpy(mask_rows(topo))
    sp = lambda t: t.view(1, S, H, D).transpose(1, 2)
    att = torch.nn.functional.scaled_dot_product_attention(sp(q), sp(k), sp(v), attn_mask=dm)
    yf = mf.o(att.transpose(1, 2).reshape(1, S, dim))
    yf.backward(dy.float().cpu())
    mx, mn = err_stats(y.detach(), yf.detach())
    mx2, mn2 = err_stats(y_ng, yf.detach())
    say(f"  out max-abs {mx:.3e} mean-abs {mn:.3e}; no-grad {mx2:.3e} / {mn2:.3e}")
    assert mx <= 2e-2 and mn <= 2e-3 and mx2 <= 2e-2 and mn2 <= 2e-3
    for nm, got, want in (("dx", xg.grad.cpu(), xf.grad), ("dWv", m.v.weight.grad.cpu(),
                                                          mf.v.weight.grad),
                          ("dWq", m.q.weight.grad.cpu(), mf.q.weight.grad),
                          ("dWcamk", m.cam_k.weight.grad.cpu(), mf.cam_k.weight.grad)):
        say(f"  {nm} rel {_rel(got, want):.3e} rel-mean {_rel_mean(got, want):.3e}")
        assert _rel(got, want) < 2e-2 and _rel_mean(got, want) < 1e-2, nm
    # a second call with the same topology returns the cached mask
    again = build_stage2_hier_flex_block_mask(P, T, L, N, KL, KG, n, W,
                                              labels if kind == "labels" else None, None, True,
                                              "cuda", **({} if kind == "labels" else dict(
                                                  membership=torch.from_numpy(mem),
                                                  global_only=torch.from_numpy(go))))
    assert again[0] is mask


def test_module_training_step_hip_prologue():
    """A training step of the module at a model dim the HIP prologue backward
    takes (512: 4 heads x 128), with the camera adapter and soft membership
    logits: ``forward_hier_membership`` runs the GEMMs, the HIP q / k tail
    forward and backward, the HIP attention forward and backward with the
    membership STE and the o-projection.  Every gradient -- x, the four
    projections (weights and biases), the RMSNorm gains, the camera adapters
    and the logits -- against fp32 autograd of the reference module math (the
    torch projection tail of attention.py:355-365) with the oracle attention
    and STE.  Every gradient within 2 % of its largest entry (max error) and
    1 % of its mean magnitude (mean error); dx and dlogits, per-token and
    per-bit quantities, also within the north-star max-abs 2e-2 / mean-abs
    2e-3 (per unit of the largest entry above 1).  The parameter gradients
    are sums over all tokens of bf16 products, whose rounding noise grows
    with the token count, so they are held to the relative bounds only."""
    need_gpu()
    from oracle.ste import ste_attention
    from tests.test_gpu_prologue import _grad_check
    P, T, L, N, KL, KG, n, W, H, D = 4, 6, 16, 2, 5, 6, 3, 4, 4, 128
    dim = H * D
    m = _module(dim, H, seed=21, cam=True)
    m.num_frame_per_block, m.local_attn_size = n, W
    rng = np.random.default_rng(22)
    logits = torch.from_numpy(rng.standard_normal((T, N, P))).float()
    mem = (logits > 0).numpy()
    topo = FullTopology(P, T, L, N, KL, KG, n, W, True, membership=mem, global_only=~mem.any(1))
    S = topo.S
    g = torch.Generator().manual_seed(23)
    x = (torch.randn(1, S, dim, generator=g) * 0.5).to(torch.bfloat16)
    dy = torch.randn(1, S, dim, generator=g).to(torch.bfloat16)
    cam = torch.zeros(1, S, 12)
    cam[0, :P * T * L] = torch.randn(P * T * L, 12, generator=g)
    cam = cam.to(torch.bfloat16)
    freqs = _freqs(S, D, 24)
    say("module training step, HIP prologue", S, dim)
    xg = x.cuda().requires_grad_(True)
    lg = logits.cuda().requires_grad_(True)
    y = m.forward_hier_membership(xg, freqs, num_players=P, num_frames=T, num_patches=L,
                                  num_groups=N, num_local_hub_tokens=KL, num_global_hub_tokens=KG,
                                  direct_player=True, membership_logits=lg, cam_tokens=cam.cuda())
    y.backward(dy.cuda())
    torch.cuda.synchronize()

    mf = SelfAttention(dim, H, eps=1e-6)
    mf.enable_camera_pose_qk(12, dropout_p=0.0)
    mf.load_state_dict({k_: v_.float().cpu() for k_, v_ in m.state_dict().items()})
    mf.num_frame_per_block, mf.local_attn_size = n, W
    xf = x.float().requires_grad_(True)
    lf = logits.clone().requires_grad_(True)
    q, k, v = mf._project_self_attn_qkv(xf, freqs, cam.float())
    att = ste_attention(q.view(S, H, D), k.view(S, H, D), v.view(S, H, D), topo, lf)
    yf = mf.o(att.reshape(1, S, dim))
    yf.backward(dy.float())
    mx, mn = err_stats(y.detach(), yf.detach())
    say(f"  output max-abs {mx:.3e} mean-abs {mn:.3e}")
    assert mx <= 2e-2 and mn <= 2e-3
    _grad_check("dx", xg.grad, xf.grad)
    _grad_check("dlogits", lg.grad, lf.grad)
    params = dict(m.named_parameters())
    for name, p_ in mf.named_parameters():
        _grad_check(f"d{name}", params[name].grad, p_.grad, absolute=False)
