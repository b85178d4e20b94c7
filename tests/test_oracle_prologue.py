"""Pins of the Q/K prologue part of the oracle (CPU): ``rms_norm``,
``camera_qk``, ``rope_apply`` and ``project_qk`` (multics/models/attention.py:
231-242, 307-320, 355-365; multics/models/rope.py:248-254).

Each function is checked against an implementation that shares no code with
it, and each plausible mistake is planted in a copy of the oracle to show that
the same check rejects it:

* ``rms_norm`` -- ``torch.nn.functional.rms_norm`` over the whole model dim
  (eps inside the square root), cast to bf16, then times the bf16 gain in a
  bf16 product.  Planted: the RMS of one head instead of all channels, eps
  added after the reciprocal square root, the gain applied before the bf16
  cast.
* ``camera_qk`` -- the reference's modules themselves in bf16:
  ``torch.nn.Linear(12, dim, bias=False)`` on bf16 camera rows, added to the
  bf16 projection by a bf16 add.  Planted: the camera term left unrounded
  before the add.
* ``rope_apply`` -- an explicit real rotation of adjacent channel pairs
  (2j, 2j+1) of each head, (x0 cos - x1 sin, x0 sin + x1 cos), in float64;
  two invariants: per-pair norm preservation and the relative-position
  identity <R(t1) q, R(t2) k> = <R(t1 - t2) q, k>.  Planted: rotating the
  half-split pairs (j, j + D/2).
* ``project_qk`` -- the composition in the reference's order, camera add ->
  RMSNorm -> RoPE, assembled from the independent pieces above.  Planted: the
  camera term added after the norm.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A

EPS = 1e-6
BF16_ULP = 2.0 ** -7     # relative spacing of bf16 values


def _bf16_close(got: torch.Tensor, ref: torch.Tensor, min_identical: float):
    """Fraction of bit-identical values >= min_identical, the rest within one
    bf16 ulp of the reference."""
    got, ref = got.float(), ref.float()
    same = (got == ref).float().mean().item()
    tol = BF16_ULP * ref.abs().clamp(min=1e-30) + 1e-30
    within = bool(((got - ref).abs() <= tol).all())
    return same >= min_identical and within, same


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _gain(dim, seed):
    g = torch.Generator().manual_seed(seed)
    return (1.0 + 0.3 * torch.randn(dim, generator=g)).to(torch.bfloat16)


# ---- rms_norm -----------------------------------------------------------------

def _rms_independent(x, w, eps=EPS):
    y = F.rms_norm(x.float(), (x.shape[-1],), eps=eps).to(torch.bfloat16)
    return (y * w).float()                         # bf16 x bf16 product, rounded once


def _rms_per_head(x, w, eps=EPS, head=128):
    xf = x.float().reshape(x.shape[0], -1, head)
    y = A.bf16(xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).reshape(x.shape)
    return A.bf16(y * w.float())


def _rms_eps_outside(x, w, eps=EPS):
    xf = x.float()
    y = A.bf16(xf * (torch.rsqrt(xf.pow(2).mean(-1, keepdim=True)) + eps))
    return A.bf16(y * w.float())


def _rms_gain_before_cast(x, w, eps=EPS):
    xf = x.float()
    return A.bf16(xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float())


def _rms_inputs():
    """Rows at three scales, so eps matters for some (mean square ~1e-8 to
    1e-5) and not for others; heads of different scales, so a per-head RMS
    differs from the row RMS."""
    x = _rand((48, 3072), 0).float()
    x[:16] *= 1e-4
    x[16:32] *= 3e-3
    x = x * torch.linspace(0.25, 4.0, 24).repeat_interleave(128)
    return x.to(torch.bfloat16), _gain(3072, 1)


def test_rms_norm_equals_torch_rms_norm():
    x, w = _rms_inputs()
    ok, same = _bf16_close(A.rms_norm(x, w, EPS), _rms_independent(x, w), 0.999)
    assert ok, f"identical {same}"


@pytest.mark.parametrize("mistake", [_rms_per_head, _rms_eps_outside, _rms_gain_before_cast])
def test_rms_norm_pin_rejects_planted_mistakes(mistake):
    x, w = _rms_inputs()
    ok, _ = _bf16_close(mistake(x, w), _rms_independent(x, w), 0.999)
    assert not ok


# ---- camera_qk ----------------------------------------------------------------

def _camera_inputs(dim=512, S=64):
    qx, kx = _rand((S, dim), 2), _rand((S, dim), 3)
    cam = _rand((S, 12), 4)
    w_q, w_k = _rand((dim, 12), 5, 0.05), _rand((dim, 12), 6, 0.05)
    return qx, kx, cam, w_q, w_k


def _camera_modules(qx, kx, cam, w_q, w_k):
    """qx + cam_q(cam) with the reference's bf16 modules (attention.py:307-320)."""
    out = []
    for x, w in ((qx, w_q), (kx, w_k)):
        lin = torch.nn.Linear(12, x.shape[1], bias=False, dtype=torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_(w)
            out.append((x + lin(cam)).float())
    return out


def test_camera_qk_equals_bf16_linear_modules():
    args = _camera_inputs()
    for got, ref in zip(A.camera_qk(*args), _camera_modules(*args)):
        ok, same = _bf16_close(got, ref, 0.999)
        assert ok, f"identical {same}"


def test_camera_qk_pin_rejects_unrounded_camera_term():
    qx, kx, cam, w_q, w_k = _camera_inputs()
    wrong = A.bf16(qx.float() + cam.float() @ w_q.float().t())
    ok, _ = _bf16_close(wrong, _camera_modules(qx, kx, cam, w_q, w_k)[0], 0.999)
    assert not ok


# ---- rope_apply ---------------------------------------------------------------

def _rotation_adjacent(x, freqs, H):
    """Explicit rotation of channel pairs (2j, 2j+1) of every head, float64."""
    S, dim = x.shape
    xd = x.double().reshape(S, H, dim // H // 2, 2)
    ang = torch.angle(freqs.reshape(S, 1, -1))
    c, s = torch.cos(ang), torch.sin(ang)
    y0 = xd[..., 0] * c - xd[..., 1] * s
    y1 = xd[..., 0] * s + xd[..., 1] * c
    return A.bf16(torch.stack([y0, y1], -1).reshape(S, dim).float())


def _rotation_half_split(x, freqs, H):
    S, dim = x.shape
    D = dim // H
    xd = x.double().reshape(S, H, D)
    a, b = xd[..., :D // 2], xd[..., D // 2:]
    ang = torch.angle(freqs.reshape(S, 1, -1))
    c, s = torch.cos(ang), torch.sin(ang)
    return A.bf16(torch.cat([a * c - b * s, a * s + b * c], -1).reshape(S, dim).float())


def _rope_inputs(S=40, H=4, D=128, seed=7):
    x = _rand((S, H * D), seed)
    g = torch.Generator().manual_seed(seed + 1)
    ang = torch.rand(S, 1, D // 2, generator=g, dtype=torch.float64) * 2 * math.pi
    return x, torch.polar(torch.ones_like(ang), ang), H


def test_rope_apply_equals_explicit_rotation():
    x, freqs, H = _rope_inputs()
    ok, same = _bf16_close(A.rope_apply(x, freqs, H), _rotation_adjacent(x, freqs, H), 0.999)
    assert ok, f"identical {same}"


def test_rope_pin_rejects_half_split_pairs():
    x, freqs, H = _rope_inputs()
    ok, _ = _bf16_close(_rotation_half_split(x, freqs, H), _rotation_adjacent(x, freqs, H), 0.999)
    assert not ok


def test_rope_apply_preserves_pair_norms():
    x, freqs, H = _rope_inputs()
    y = A.rope_apply(x, freqs, H)
    nx = x.float().reshape(x.shape[0], -1, 2).norm(dim=-1)
    ny = y.reshape(x.shape[0], -1, 2).norm(dim=-1)
    assert torch.allclose(ny, nx, rtol=2 * BF16_ULP, atol=1e-6)


def test_rope_apply_relative_position():
    """<R(t1) q, R(t2) k> = <R(t1 - t2) q, k> over a band of the table of
    precompute_freqs_cis (per pair: Re(q conj(k) e^{i(t1-t2)w}))."""
    H, D = 1, 128
    tab = A.precompute_freqs_cis(D, end=64)
    q, k = _rand((1, D), 11), _rand((1, D), 12)
    for t1, t2 in ((5, 2), (40, 17), (63, 0), (9, 9)):
        lhs = (A.rope_apply(q, tab[t1][None, None], H) * A.rope_apply(k, tab[t2][None, None], H)).sum()
        rhs = (A.rope_apply(q, tab[t1 - t2][None, None], H) * k.float()).sum()
        scale = (q.float().norm() * k.float().norm()).item()
        assert abs(lhs.item() - rhs.item()) <= 4 * BF16_ULP * scale, (t1, t2)


# ---- project_qk ---------------------------------------------------------------

def _project_independent(qx, kx, wq, wk, freqs, H, cam, w_cam_q, w_cam_k, *, cam_after_norm=False):
    if cam is not None and not cam_after_norm:
        qx, kx = (t.to(torch.bfloat16) for t in _camera_modules(qx, kx, cam, w_cam_q, w_cam_k))
    q = _rms_independent(qx, wq).to(torch.bfloat16)
    k = _rms_independent(kx, wk).to(torch.bfloat16)
    if cam is not None and cam_after_norm:
        q, k = (t.to(torch.bfloat16) for t in _camera_modules(q, k, cam, w_cam_q, w_cam_k))
    return _rotation_adjacent(q, freqs, H), _rotation_adjacent(k, freqs, H)


def _project_inputs(S=40, H=24, D=128):
    dim = H * D
    qx, kx = _rand((S, dim), 20, 0.5), _rand((S, dim), 21, 0.5)
    wq, wk = _gain(dim, 22), _gain(dim, 23)
    cam = _rand((S, 12), 24)
    w_cam_q, w_cam_k = _rand((dim, 12), 25, 0.3), _rand((dim, 12), 26, 0.3)
    g = torch.Generator().manual_seed(27)
    ang = torch.rand(S, 1, D // 2, generator=g, dtype=torch.float64) * 2 * math.pi
    return qx, kx, wq, wk, torch.polar(torch.ones_like(ang), ang), H, cam, w_cam_q, w_cam_k


@pytest.mark.parametrize("camera", [False, True])
def test_project_qk_equals_reference_order(camera):
    qx, kx, wq, wk, freqs, H, cam, wcq, wck = _project_inputs()
    if not camera:
        cam = wcq = wck = None
    got = A.project_qk(qx, kx, norm_q_w=wq, norm_k_w=wk, freqs=freqs, num_heads=H, eps=EPS,
                       cam=cam, w_cam_q=wcq, w_cam_k=wck)
    ref = _project_independent(qx, kx, wq, wk, freqs, H, cam, wcq, wck)
    for g_, r_ in zip(got, ref):
        ok, same = _bf16_close(g_, r_, 0.999)
        assert ok, f"identical {same}"


def test_project_qk_pin_rejects_camera_after_norm():
    qx, kx, wq, wk, freqs, H, cam, wcq, wck = _project_inputs()
    got = A.project_qk(qx, kx, norm_q_w=wq, norm_k_w=wk, freqs=freqs, num_heads=H, eps=EPS,
                       cam=cam, w_cam_q=wcq, w_cam_k=wck)
    wrong = _project_independent(qx, kx, wq, wk, freqs, H, cam, wcq, wck, cam_after_norm=True)
    ok, _ = _bf16_close(got[0], wrong[0], 0.999)
    assert not ok
