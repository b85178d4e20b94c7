"""Pins of the RoPE-table, camera12 and masked-attention parts of the oracle,
and the product twins checked against them (CPU).

What fixes each function without running the reference:
* ``simplex_vertices`` -- the reference test's invariants
  (tests/test_simplex_rope.py:21-32: unit norm, pairwise squared distance
  2m/(m-1)), plus centring (the vertices sum to 0), zero padding past m
  columns and the m = 2 closed form +-1/sqrt(2).
* ``precompute_freqs_cis`` -- unit modulus, angle t * theta^(-2j/dim) at
  spot values, the group law f(t1 + t2) = f(t1) f(t2).
* ``rerope_bands`` -- band widths (12, 32, 42, 42)/2 summing to D/2, the
  temporal band being the *lowest* six frequencies of Wan's 44-channel
  temporal band (rope.py:129-144), closed-form angles.
* ``player_freqs`` / ``hub_freqs`` -- the reference test's agent-band
  constancy and per-player difference (tests/test_simplex_rope.py:35-54),
  token order (t, y, x) with each band indexed independently, hub rows
  carrying only the temporal phase of their frame slot.
* ``camera_to_world`` / ``camera12`` -- rigid-transform identities: proper
  orthonormal rotations, forward axis from yaw / pitch, translation = the
  position; camera12's anchor (player 0, frame 0) maps to [I | 0], the
  result is invariant under a global rigid motion of every camera, the
  translation scales with 1 / pos_scale, and the relative transforms compose.
* ``masked_attention`` -- ``torch.nn.functional.scaled_dot_product_attention``
  with the dense boolean mask (attention.py:47-54), an independent
  implementation, on every live row; inactive local-hub rows are 0.
"""

import math

import numpy as np
import pytest
import torch

from multics_amd import camera as PC
from multics_amd import rope as PR
from oracle import attention as A
from oracle.masks import FullTopology, inactive_local_rows, mask_rows


# ---- simplex vertices --------------------------------------------------------

@pytest.mark.parametrize("m", [2, 3, 4, 7, 10, 16])
def test_simplex_vertices_invariants(m):
    d_a = 32
    v = A.simplex_vertices(m, d_a).double()
    assert v.shape == (m, d_a // 2)
    assert torch.allclose(v.norm(dim=1), torch.ones(m, dtype=torch.float64), atol=1e-6)
    d2 = ((v[:, None] - v[None]) ** 2).sum(-1)
    off = ~torch.eye(m, dtype=torch.bool)
    assert torch.allclose(d2[off], torch.full_like(d2[off], 2 * m / (m - 1)), atol=1e-5)
    assert torch.allclose(v.sum(0), torch.zeros(d_a // 2, dtype=torch.float64), atol=1e-6)
    assert (v[:, m:] == 0).all()
    # vertex i points most along axis i
    assert (v[:, :m].argmax(dim=1) == torch.arange(m)).all()
    assert torch.equal(PR.build_simplex_vertices(m, d_a), A.simplex_vertices(m, d_a))


def test_simplex_vertices_closed_form_and_limits():
    v = A.simplex_vertices(2, 32)
    r = 1 / math.sqrt(2)
    assert torch.allclose(v[:, :2], torch.tensor([[r, -r], [-r, r]]), atol=1e-7)
    with pytest.raises(ValueError):
        A.simplex_vertices(1, 32)
    with pytest.raises(ValueError):
        A.simplex_vertices(18, 32)           # more than d_agent/2 + 1 vertices
    with pytest.raises(ValueError):
        PR.build_simplex_vertices(18, 32)
    # m = d_agent/2 + 1 passes the reference's range check but its vertices
    # need m columns: the reference's assignment fails there (rope.py:116-126)
    with pytest.raises(RuntimeError):
        PR.build_simplex_vertices(17, 32)


# ---- frequency tables ----------------------------------------------------------

def test_precompute_freqs_cis_closed_form():
    dim, theta = 44, 10000.0
    f = A.precompute_freqs_cis(dim, end=64, theta=theta)
    assert f.shape == (64, dim // 2) and f.dtype == torch.complex128
    assert torch.allclose(f.abs(), torch.ones_like(f.abs()), atol=1e-12)
    assert torch.allclose(f[0], torch.ones(dim // 2, dtype=torch.complex128))
    for t, j in ((1, 0), (1, 21), (5, 3), (63, 10)):
        want = t * theta ** (-2.0 * j / dim)
        got = torch.angle(f[t, j]).item()
        assert abs(math.remainder(got - want, 2 * math.pi)) < 1e-9
    assert torch.allclose(f[7] * f[11], f[18], atol=1e-12)
    assert torch.equal(PR.precompute_freqs_cis(dim, 64, theta), f)


def test_rerope_bands_are_the_lowest_temporal_frequencies():
    b = A.rerope_bands(128)
    assert b["splits"] == (12, 32, 42, 42) and sum(b["splits"]) == 128 and b["d_a"] == 32
    assert b["t"].shape[1] == 6 and b["h"].shape[1] == 21 and b["w"].shape[1] == 21
    assert b["t"].shape[1] + 16 + 21 + 21 == 64
    # Wan's 3D temporal band has 128 - 2 * 42 = 44 channels (22 frequencies);
    # the 4D table keeps its last (lowest) six: theta^(-2j/44), j = 16..21
    for c, j in enumerate(range(16, 22)):
        assert abs(torch.angle(b["t"][1, c]).item() - 10000.0 ** (-2.0 * j / 44)) < 1e-12
    assert abs(torch.angle(b["h"][1, 0]).item() - 1.0) < 1e-12
    assert abs(torch.angle(b["h"][1, 20]).item() - 10000.0 ** (-40.0 / 42)) < 1e-12
    p = PR.precompute_freqs_cis_4d_wan_rerope(128)
    for k in ("t", "h", "w"):
        assert torch.equal(p[k], b[k])


def _token_freqs(f, h, w, P, start=0):
    bands = A.rerope_bands(128)
    verts = A.simplex_vertices(10, 32)
    return bands, verts, [A.player_freqs(bands, f, h, w, verts, p, start_frame=start)
                          for p in range(P)]


def test_player_freqs_band_layout():
    f, h, w = 3, 4, 5
    bands, verts, fr = _token_freqs(f, h, w, P=2, start=2)
    p0, p1 = fr
    assert p0.shape == (f * h * w, 1, 64)
    # agent band (columns 6..21) constant over tokens and different per player
    assert torch.equal(p0[:, 0, 6:22], p0[:1, 0, 6:22].expand(f * h * w, 16))
    assert not torch.allclose(p0[0, 0, 6:22], p1[0, 0, 6:22])
    assert torch.allclose(torch.angle(p0[0, 0, 6:22]), verts[0].double(), atol=1e-12)
    rng = np.random.default_rng(0)
    for i in rng.choice(f * h * w, 12, replace=False):
        t, y, x = i // (h * w), (i // w) % h, i % w
        assert torch.equal(p0[i, 0, :6], bands["t"][2 + t])
        assert torch.equal(p0[i, 0, 22:43], bands["h"][y])
        assert torch.equal(p0[i, 0, 43:], bands["w"][x])


def test_hub_freqs_temporal_only():
    bands = A.rerope_bands(128)
    K = 4
    hb = A.hub_freqs(bands, 3, K, start_frame=5)
    assert hb.shape == (3 * K, 1, 64)
    for i in range(3 * K):
        assert torch.equal(hb[i, 0, :6], bands["t"][5 + i // K])
    assert torch.equal(hb[:, 0, 6:], torch.ones(3 * K, 58, dtype=torch.complex128))


def test_product_freqs_match_oracle():
    f, h, w, P, K = 3, 4, 5, 3, 7
    bands, verts, fr = _token_freqs(f, h, w, P, start=4)
    pb = PR.precompute_freqs_cis_4d_wan_rerope(128)
    pv = PR.build_simplex_vertices(10, 32)
    got = PR.build_self_attn_freqs_with_hub(pb, pv, f, h, w, "cpu", list(range(P)), K,
                                            start_frame=4)
    want = torch.cat(fr + [A.hub_freqs(bands, f, K, start_frame=4)], dim=0)
    assert got.shape == want.shape
    assert torch.allclose(got.to(torch.complex128), want, atol=1e-7)
    assert torch.equal(got[:P * f * h * w], want[:P * f * h * w])
    cs, sn = PR.freqs_to_cos_sin(got)
    assert torch.allclose(cs, want[:, 0].real.float(), atol=1e-7)
    assert torch.allclose(sn, want[:, 0].imag.float(), atol=1e-7)


def test_cos_sin_of_a_table_is_converted_once():
    """The conversion of the same table object is reused (every layer of a
    step receives the same table); an in-place change of the table, or
    another table object, converts again."""
    t = torch.polar(torch.ones(6, 1, 4, dtype=torch.float64),
                    torch.arange(24, dtype=torch.float64).reshape(6, 1, 4) / 7)
    cs, sn = PR.freqs_to_cos_sin(t)
    again = PR.freqs_to_cos_sin(t)
    assert again[0] is cs and again[1] is sn
    t.mul_(1j)                                    # rotate every entry by 90 degrees in place
    cs2, sn2 = PR.freqs_to_cos_sin(t)
    assert cs2 is not cs and torch.allclose(cs2, -sn) and torch.allclose(sn2, cs)
    other = t.clone()
    assert PR.freqs_to_cos_sin(other)[0] is not cs2
    assert torch.equal(PR.freqs_to_cos_sin(other)[0], cs2)


# ---- camera ------------------------------------------------------------------

def _poses(P, T, seed):
    rng = np.random.default_rng(seed)
    pose = np.zeros((P, T, 5))
    pose[..., :3] = rng.normal(0, 1.0, (P, T, 3))
    pose[..., 3] = rng.uniform(-180, 180, (P, T))
    pose[..., 4] = rng.uniform(-30, 30, (P, T))
    return pose


def test_camera_to_world_is_rigid():
    pose = _poses(3, 5, 1)
    c2w = A.camera_to_world(pose)
    R = c2w[..., :3, :3]
    assert np.allclose(np.swapaxes(R, -1, -2) @ R, np.eye(3), atol=1e-12)
    assert np.allclose(np.linalg.det(R), 1.0, atol=1e-12)
    assert np.allclose(c2w[..., :3, 3], pose[..., :3])
    assert np.allclose(c2w[..., 3, :], [0, 0, 0, 1])
    yaw, pitch = np.deg2rad(pose[..., 3]), np.deg2rad(pose[..., 4])
    fwd = np.stack([np.cos(pitch) * np.cos(yaw), np.cos(pitch) * np.sin(yaw), -np.sin(pitch)], -1)
    assert np.allclose(-c2w[..., :3, 2], fwd, atol=1e-12)          # camera looks along -z
    assert np.allclose(c2w[..., 2, 0], 0.0, atol=1e-12)            # right axis stays level
    # yaw 0, pitch 0: forward +x, right -y, up +z
    c = A.camera_to_world(np.array([1.0, 2.0, 3.0, 0.0, 0.0]))
    assert np.allclose(c[:3, :3], [[0, 0, -1], [-1, 0, 0], [0, 1, 0]], atol=1e-12)
    assert np.allclose(PC.camera_to_world(pose), c2w)


def test_camera12_identities():
    P, T = 3, 4
    c2w = A.camera_to_world(_poses(P, T, 2))
    c12 = A.camera12(c2w, 1.0).astype(np.float64)
    assert c12.shape == (P, T, 12)
    rel = c12.reshape(P, T, 3, 4)
    assert np.allclose(rel[0, 0], np.hstack([np.eye(3), np.zeros((3, 1))]), atol=1e-6)
    R = rel[..., :3]
    assert np.allclose(np.swapaxes(R, -1, -2) @ R, np.eye(3), atol=1e-5)
    # invariance under one rigid motion of the whole scene
    G = A.camera_to_world(np.array([0.3, -2.0, 5.0, 40.0, 10.0]))
    assert np.allclose(A.camera12(G[None, None] @ c2w, 1.0), c12, atol=1e-5)
    # translation / pos_scale, rotation unchanged
    c12s = A.camera12(c2w, 4.0).reshape(P, T, 3, 4).astype(np.float64)
    assert np.allclose(c12s[..., 3] * 4.0, rel[..., 3], atol=1e-5)
    assert np.allclose(c12s[..., :3], R, atol=1e-6)
    # relative transforms compose: inv(anchor) @ c2w
    full = np.concatenate([rel, np.broadcast_to([0, 0, 0, 1.0], (P, T, 1, 4))], axis=2)
    want = np.linalg.inv(c2w[0, 0])[None, None] @ c2w
    assert np.allclose(full, want, atol=1e-5)
    got = PC.camera12_from_absolute_c2w(torch.from_numpy(c2w), 1.0).numpy()
    assert np.allclose(got, c12, atol=1e-6)


def test_camera_tokens_order_and_hub_zeros():
    """tests/test_camera_pose_qk.py:6-33: per-(player, frame) rows broadcast
    to L tokens player-major, hub rows zero."""
    P, F, L, C, K = 2, 3, 4, 12, 2
    cam = torch.arange(P * F * C, dtype=torch.float32).reshape(P, F, C)
    ref = torch.zeros(1, P * F * L, 16)
    tok = PC.build_camera_tokens(cam, F, L, P, ref, include_hub=True, num_hub_tokens=K)
    assert tok.shape == (1, P * F * L + F * K, C)
    for p in range(P):
        for f in range(F):
            for l in range(L):
                assert torch.equal(tok[0, (p * F + f) * L + l], cam[p, f])
    assert (tok[0, P * F * L:] == 0).all()


# ---- masked attention ----------------------------------------------------------

@pytest.mark.parametrize("kind", ["labels", "membership"])
def test_masked_attention_equals_sdpa(kind):
    rng = np.random.default_rng(3)
    P, T, L, N, KL, KG, n, W, H, D = 4, 6, 5, 2, 2, 3, 3, 4, 2, 16
    if kind == "labels":
        labels = np.array([[0, 0, 1, 1]] * T)
        active = np.ones((T, N), bool)
        active[3:, 1] = False
        topo = FullTopology(P, T, L, N, KL, KG, n, W, True, labels=labels, active=active)
    else:
        mem = rng.random((T, N, P)) < 0.4
        go = ~mem.any(1)
        topo = FullTopology(P, T, L, N, KL, KG, n, W, True, membership=mem, global_only=go)
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(topo.S, H, D, generator=g) for _ in range(3))
    got = A.masked_attention(q, k, v, topo)
    m = torch.from_numpy(mask_rows(topo))
    sd = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(0, 1)[None], k.transpose(0, 1)[None], v.transpose(0, 1)[None],
        attn_mask=m[None, None])[0].transpose(0, 1)
    dead = torch.from_numpy(inactive_local_rows(topo))
    assert torch.allclose(got[~dead], sd[~dead], atol=1e-5)
    assert (got[dead] == 0).all()
    if kind == "labels":
        assert dead.any()
        # the dense mask gives an inactive hub row only its self edge: SDPA
        # returns the row's own value there
        assert torch.allclose(sd[dead], v[dead], atol=1e-6)
