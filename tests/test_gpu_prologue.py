"""Fused camera + RMSNorm + RoPE prologue against the fp32/f64 oracle."""

import numpy as np
import pytest
import torch

from multics_amd.kernels import qkv_prologue
from oracle import attention as OA
from tests.gpu_util import err_stats, need_gpu, say

pytestmark = pytest.mark.gpu


def _freqs(P, T, h, w, KG_total):
    bands = OA.rerope_bands(128)
    verts = OA.simplex_vertices(10, 32)
    agent = torch.cat([OA.player_freqs(bands, T, h, w, verts, p) for p in range(P)], 0)
    return torch.cat([agent, OA.hub_freqs(bands, T, KG_total)], 0)


@pytest.mark.parametrize("camera", [False, True])
@pytest.mark.parametrize("layout", ["shd", "hsd"])
@pytest.mark.parametrize("shape", ["small", "odd_tokens", "dim4096", "dim3072", "dim768", "d64"])
def test_prologue_matches_oracle(camera, layout, shape):
    """Model dims that are multiples of 512 run one wave per token run
    (row_prologue_kernel), others the workgroup-per-token kernel.  small: 168
    tokens, dim 512; odd_tokens: 141 tokens, so a wave's run ends on a token
    paired with itself; dim4096: 32 heads (eight chunks per lane); dim3072:
    the C2 model dim (six chunks), with camera rows changing inside a wave's
    run; dim768: 6 heads, the workgroup kernel; d64: head dim 64, 8 heads
    (dim 512, the wave kernel's D = 64 pair indexing)."""
    need_gpu()
    say("prologue camera", camera, layout, shape)
    P, T, h, w, H, D = 2, 3, 4, 5, 4, 128
    if shape == "d64":
        H, D = 8, 64
    K_total = 2 * 5 + 6
    if shape == "odd_tokens":
        h, w, K_total = 3, 5, 2 * 5 + 7
    elif shape == "dim4096":
        T, H = 2, 32
    elif shape == "dim3072":
        T, H = 2, 24
    elif shape == "dim768":
        H = 6
    S = P * T * h * w + T * K_total
    assert shape != "odd_tokens" or S % 2 == 1
    dim = H * D
    g = torch.Generator().manual_seed(5)
    qx = (torch.randn(S, dim, generator=g) * 0.7).to(torch.bfloat16)
    kx = (torch.randn(S, dim, generator=g) * 0.7).to(torch.bfloat16)
    vx = torch.randn(S, dim, generator=g).to(torch.bfloat16)
    wq = (1 + 0.1 * torch.randn(dim, generator=g)).to(torch.bfloat16)
    wk = (1 + 0.1 * torch.randn(dim, generator=g)).to(torch.bfloat16)
    freqs = _freqs(P, T, h, w, K_total)
    if D == 64:
        freqs = freqs[..., :32].contiguous()   # any unit rotations serve the comparison
    cam = wcq = wck = None
    if camera:
        cam = torch.zeros(S, 12)
        cam[:P * T * h * w] = torch.randn(P * T * h * w, 12, generator=g)
        cam = cam.to(torch.bfloat16)
        wcq = (0.05 * torch.randn(dim, 12, generator=g)).to(torch.bfloat16)
        wck = (0.05 * torch.randn(dim, 12, generator=g)).to(torch.bfloat16)
    dev = "cuda"
    q, k, v = qkv_prologue(
        qx.to(dev), kx.to(dev), vx.to(dev), norm_q_w=wq.to(dev), norm_k_w=wk.to(dev),
        rope_cos=freqs[:, 0].real.float().to(dev), rope_sin=freqs[:, 0].imag.float().to(dev),
        num_heads=H, eps=1e-6, cam=None if cam is None else cam.to(dev),
        w_cam_q=None if wcq is None else wcq.to(dev), w_cam_k=None if wck is None else wck.to(dev),
        out_layout=layout)
    torch.cuda.synchronize()
    rq, rk = OA.project_qk(qx, kx, norm_q_w=wq, norm_k_w=wk, freqs=freqs, num_heads=H, eps=1e-6,
                           cam=cam, w_cam_q=wcq, w_cam_k=wck)
    for got, ref in ((q, rq), (k, rk)):
        got = got.reshape(S, dim)
        mx, mn = err_stats(got, ref)
        same = (got.float().cpu() == ref).float().mean().item()
        say(f"  max-abs {mx:.3e} mean-abs {mn:.3e} identical {same:.5f}")
        assert mx <= 2e-2 and mn <= 2e-4 and same > 0.99
    assert torch.equal(v.reshape(S, dim).cpu(), vx)


def test_prologue_c2_full_size():
    """The prologue exactly as ``bench.py`` times it: C2 (37,632 tokens x
    3,072 channels, 24 heads), camera12 of the bench's seeded poses, the
    bench's fp32 simplex RoPE table, head-major output.  Each output token
    depends only on its own row, so sampled tokens are compared with
    ``project_qk`` over an f64 RoPE table built by the oracle: the first and
    last token of every (player, frame) camera run, every hub row of the
    first, middle and last frames, and random tokens."""
    need_gpu()
    import bench
    P, T, L, N, KL, KG, n, W, H, D, _ = bench.CONFIGS["c2"]
    K = N * KL + KG
    S, dim = P * T * L + T * K, H * D
    dev = "cuda"
    say("prologue c2 full size", S, dim)
    g = torch.Generator(device=dev).manual_seed(bench.SEED + 7)
    qx = (torch.randn(S, dim, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    kx = (torch.randn(S, dim, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    wq = (1 + 0.1 * torch.randn(dim, generator=g, device=dev)).to(torch.bfloat16)
    wk = (1 + 0.1 * torch.randn(dim, generator=g, device=dev)).to(torch.bfloat16)
    wcq = (0.02 * torch.randn(dim, 12, generator=g, device=dev)).to(torch.bfloat16)
    wck = (0.02 * torch.randn(dim, 12, generator=g, device=dev)).to(torch.bfloat16)
    cam = bench.camera_tokens(P, T, L, K, dev)
    cos, sin = bench.rope_tables(P, T, L, K, D, dev)
    q, k, _ = qkv_prologue(qx, kx, None, norm_q_w=wq, norm_k_w=wk, rope_cos=cos, rope_sin=sin,
                           num_heads=H, eps=1e-6, cam=cam, w_cam_q=wcq, w_cam_k=wck,
                           out_layout="hsd")
    torch.cuda.synchronize()
    rng = np.random.default_rng(3)
    rows = set(rng.choice(S, 1500, replace=False).tolist())
    for p in range(P):
        for t in range(T):
            base = p * T * L + t * L
            rows |= {base, base + L - 1}
    for t in (0, T // 2, T - 1):
        rows |= {P * T * L + t * N * KL + i for i in range(N * KL)}
        rows |= {P * T * L + T * N * KL + t * KG + i for i in range(KG)}
    rows = torch.tensor(sorted(rows))
    bands = OA.rerope_bands(D)
    verts = OA.simplex_vertices(10, 32)
    h, w = 11, 20
    freqs = torch.cat([OA.player_freqs(bands, T, h, w, verts, p) for p in range(P)]
                      + [OA.hub_freqs(bands, T, K)], 0)
    assert freqs.shape[0] == S
    cpu = lambda t: t.cpu()
    rq, rk = OA.project_qk(cpu(qx)[rows], cpu(kx)[rows], norm_q_w=cpu(wq), norm_k_w=cpu(wk),
                           freqs=freqs[rows], num_heads=H, eps=1e-6, cam=cpu(cam)[rows],
                           w_cam_q=cpu(wcq), w_cam_k=cpu(wck))
    for got, ref in ((q, rq), (k, rk)):
        got = got[rows.to(dev)].reshape(len(rows), dim)
        mx, mn = err_stats(got, ref)
        same = (got.float().cpu() == ref).float().mean().item()
        say(f"  {len(rows)} tokens: max-abs {mx:.3e} mean-abs {mn:.3e} identical {same:.5f}")
        assert mx <= 2e-2 and mn <= 2e-3 and same > 0.99


def _grad_check(name, got, ref, rel_max=2e-2, rel_mean=1e-2, absolute=True):
    """Relative bounds (max error within 2 % of max|ref|, mean error within
    1 % of mean|ref|) and, with ``absolute``, the north-star absolute bounds
    scaled to the gradient's size (max-abs <= 2e-2 and mean-abs <= 2e-3 per
    unit of max|ref| above 1)."""
    got = got.detach().float().cpu()
    ref = ref.detach().float()
    err = (got - ref).abs()
    scale = max(1.0, ref.abs().max().item())
    say(f"  {name}: max-abs {err.max().item():.3e} mean-abs {err.mean().item():.3e} "
        f"(ref max {ref.abs().max().item():.3e} mean {ref.abs().mean().item():.3e})")
    assert torch.isfinite(got).all(), name
    if absolute:
        assert err.max().item() <= 2e-2 * scale and err.mean().item() <= 2e-3 * scale, name
    assert err.max().item() <= rel_max * ref.abs().max().item() + 1e-6, name
    assert err.mean().item() <= rel_mean * ref.abs().mean().item() + 1e-7, name


@pytest.mark.parametrize("camera", [False, True])
@pytest.mark.parametrize("shape", ["dim512", "dim3072", "d64"])
def test_prologue_backward_matches_fp32_autograd(camera, shape):
    """``QKPrologueFunction`` (HIP forward and backward of the camera add,
    RMSNorm, gain and RoPE) against torch autograd through ``project_qk`` in
    fp32 / f64 on the CPU (the roundings of the forward pass the gradient
    through unchanged in both): gradients of the q / k projections, the
    RMSNorm gains and the camera-adapter weights."""
    need_gpu()
    from multics_amd.kernels import qk_prologue_train
    say("prologue backward", shape, "camera", camera)
    P, T, h, w, H, D = 2, 3, 4, 5, 4, 128
    if shape == "dim3072":
        T, H = 2, 24
    elif shape == "d64":
        H, D = 8, 64
    K_total = 2 * 5 + 6
    S = P * T * h * w + T * K_total
    dim = H * D
    g = torch.Generator().manual_seed(8)
    qx = (torch.randn(S, dim, generator=g) * 0.5).to(torch.bfloat16)
    kx = (torch.randn(S, dim, generator=g) * 0.5).to(torch.bfloat16)
    wq = (1 + 0.1 * torch.randn(dim, generator=g)).to(torch.bfloat16)
    wk = (1 + 0.1 * torch.randn(dim, generator=g)).to(torch.bfloat16)
    freqs = _freqs(P, T, h, w, K_total)
    if D == 64:
        freqs = freqs[..., :32].contiguous()
    cam = wcq = wck = None
    if camera:
        cam = torch.zeros(S, 12)
        cam[:P * T * h * w] = torch.randn(P * T * h * w, 12, generator=g)
        cam = cam.to(torch.bfloat16)
        wcq = (0.05 * torch.randn(dim, 12, generator=g)).to(torch.bfloat16)
        wck = (0.05 * torch.randn(dim, 12, generator=g)).to(torch.bfloat16)
    dq = (torch.randn(S, H, D, generator=g) * 0.5).to(torch.bfloat16)
    dk = (torch.randn(S, H, D, generator=g) * 0.5).to(torch.bfloat16)

    dev = "cuda"
    leaf = lambda t: None if t is None else t.to(dev).requires_grad_(True)
    hq, hk, hwq, hwk, hwcq, hwck = (leaf(t) for t in (qx, kx, wq, wk, wcq, wck))
    q, k = qk_prologue_train(hq, hk, norm_q_w=hwq, norm_k_w=hwk,
                             rope_cos=freqs[:, 0].real.float().to(dev),
                             rope_sin=freqs[:, 0].imag.float().to(dev), num_heads=H, eps=1e-6,
                             cam=None if cam is None else cam.to(dev), w_cam_q=hwcq, w_cam_k=hwck)
    torch.autograd.backward([q, k], [dq.to(dev), dk.to(dev)])
    torch.cuda.synchronize()

    f32 = lambda t: None if t is None else t.float().requires_grad_(True)
    rq, rk, rwq, rwk, rwcq, rwck = (f32(t) for t in (qx, kx, wq, wk, wcq, wck))
    oq, ok = OA.project_qk(rq, rk, norm_q_w=rwq, norm_k_w=rwk, freqs=freqs, num_heads=H, eps=1e-6,
                           cam=None if cam is None else cam.float(), w_cam_q=rwcq, w_cam_k=rwck)
    torch.autograd.backward([oq, ok], [dq.float().reshape(S, dim), dk.float().reshape(S, dim)])
    for name, a, b in (("dqx", hq.grad, rq.grad), ("dkx", hk.grad, rk.grad),
                       ("dnorm_q", hwq.grad, rwq.grad), ("dnorm_k", hwk.grad, rwk.grad)):
        _grad_check(name, a, b)
    if camera:
        _grad_check("dcam_q", hwcq.grad, rwcq.grad)
        _grad_check("dcam_k", hwck.grad, rwck.grad)
