"""fp32 CPU restatement of the hierarchical attention numerics.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* ``masked_attention``  -- ``flash_attention(mask=...)`` = SDPA with a boolean
  mask (multics/models/attention.py:39-54), fp32, with inactive local-hub query
  rows written as 0 (hier_segmented_attention.py:104-109,
  hier_tiled_attention.py:432-459).  Evaluated one row block at a time from
  ``oracle.masks.mask_rows`` so C2-sized rows never need an S x S matrix.
* ``attention_grads_at`` -- dQ at chosen query rows and dK / dV at chosen key
  rows of ``masked_attention`` (the SDPA backward: dS = P (dP - delta)),
  for bench-size sequences where autograd over every row is too large.
* ``rms_norm``, ``camera_qk``, ``rope_apply``, ``project_qk`` -- the Q/K
  prologue (attention.py:231-242, 307-320, 355-365; rope.py:248-254) with the
  reference's bf16 rounding points; RoPE in float64 as the reference does.
* ``precompute_freqs_cis``, ``rerope_bands``, ``simplex_vertices``,
  ``player_freqs``, ``hub_freqs`` -- rope.py:103-237 (float64).
* ``camera_to_world``, ``camera12`` -- data/raw_inputs.py:250-273,
  data/dataset.py:49-90.

Parity pins (tests/test_oracle_rope_camera.py, tests/test_oracle_grads.py):
* ``masked_attention`` -- against torch's ``scaled_dot_product_attention`` with
  the dense mask of ``oracle.masks`` (itself pinned against the reference's
  tests and golden layouts) on every live row; inactive local-hub rows 0.
* ``attention_grads_at`` -- against torch autograd through
  ``masked_attention`` on small shapes.
* ``precompute_freqs_cis`` / ``rerope_bands`` -- closed-form angles, unit
  modulus and the group law; the temporal band is the lowest six frequencies
  of the 44-channel Wan band.
* ``simplex_vertices`` -- the invariants of tests/test_simplex_rope.py:21-32
  (unit norm, squared distance 2m/(m-1)), centring and the m = 2 closed form.
* ``player_freqs`` / ``hub_freqs`` -- agent-band constancy and per-player
  difference (tests/test_simplex_rope.py:35-54) and per-band indexing.
* ``camera_to_world`` / ``camera12`` -- rigid-transform identities (proper
  rotations, anchor -> [I | 0], invariance under a global rigid motion,
  1/pos_scale translation, composition).
* ``rms_norm`` / ``camera_qk`` / ``rope_apply`` / ``project_qk``
  (tests/test_oracle_prologue.py) -- against implementations sharing no code
  with them: ``torch.nn.functional.rms_norm`` over the whole model dim then
  the bf16 gain product; the reference's bf16 ``nn.Linear`` camera adapter and
  bf16 add; an explicit real rotation of adjacent channel pairs, plus pair-norm
  preservation and the relative-position identity; their composition in the
  reference's order (camera add -> norm -> RoPE).  Per-head RMS, eps outside
  the square root, the gain before the bf16 cast, an unrounded camera term,
  half-split RoPE pairs and the camera added after the norm are each planted
  and rejected by the same checks.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from .masks import FullTopology, inactive_local_rows, mask_rows

ROPE_SPLITS = (12, 32, 42, 42)   # rope.py:5


def bf16(x: torch.Tensor) -> torch.Tensor:
    """Round to bfloat16 and back to float32."""
    return x.to(torch.bfloat16).to(torch.float32)


def masked_attention(q, k, v, topo: FullTopology, *, rows=None, row_block: int = 4096,
                     scale=None) -> torch.Tensor:
    """fp32 hierarchical attention over the full-sequence token order.

    ``q, k, v``: [S, H, D] tensors (any float dtype; computed in fp32).
    Returns [len(rows), H, D] fp32 (all rows when ``rows`` is None).
    """
    S, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    rows = np.arange(S) if rows is None else np.asarray(rows)
    qf, kf, vf = (t.float() for t in (q, k, v))
    dead = inactive_local_rows(topo)
    out = torch.zeros((len(rows), H, D), dtype=torch.float32)
    for r0 in range(0, len(rows), row_block):
        rr = rows[r0:r0 + row_block]
        m = torch.from_numpy(mask_rows(topo, q_idx=rr))
        live = ~torch.from_numpy(dead[rr])
        s = torch.einsum("qhd,khd->hqk", qf[torch.from_numpy(rr)], kf) * scale
        s = s.masked_fill(~m[None], float("-inf"))
        p = torch.softmax(s, dim=-1)
        p = torch.nan_to_num(p, nan=0.0)
        o = torch.einsum("hqk,khd->qhd", p, vf)
        out[r0:r0 + len(rr)] = o * live[:, None, None]
    return out


def attention_grads_at(q, k, v, dout, topo: FullTopology, *, q_rows, k_rows, scale=None,
                       row_block: int = 2048):
    """Gradients of ``sum(masked_attention(q, k, v) * dout)``: dQ at ``q_rows``
    and dK, dV at ``k_rows`` ([n, H, D] fp32 each).

    Per query row i with visible keys j: P_ij = softmax_j(scale q_i.k_j),
    O_i = sum_j P_ij v_j, delta_i = dO_i.O_i, dS_ij = P_ij (dO_i.v_j - delta_i);
    dQ_i = scale sum_j dS_ij k_j, dK_j = scale sum_i dS_ij q_i and
    dV_j = sum_i P_ij dO_i.  Inactive local-hub rows output 0, so their dO
    counts as 0.  dK / dV need every row that sees a chosen key, so all rows
    are visited, ``row_block`` at a time (memory O(row_block x S)).
    """
    S, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    qf, kf, vf, df = (t.float() for t in (q, k, v, dout))
    df = df * torch.from_numpy(~inactive_local_rows(topo))[:, None, None]
    q_rows = np.ascontiguousarray(q_rows, dtype=np.int64)
    k_rows = np.ascontiguousarray(k_rows, dtype=np.int64)
    q_pos = {int(r): i for i, r in enumerate(q_rows)}
    kr = torch.from_numpy(k_rows)
    dq = torch.zeros((len(q_rows), H, D))
    dk = torch.zeros((len(k_rows), H, D))
    dv = torch.zeros((len(k_rows), H, D))
    for r0 in range(0, S, row_block):
        rr = np.arange(r0, min(S, r0 + row_block))
        rt = torch.from_numpy(rr)
        m = torch.from_numpy(mask_rows(topo, q_idx=rr))                     # [b, S]
        s = torch.einsum("qhd,khd->hqk", qf[rt], kf) * scale
        s = s.masked_fill(~m[None], float("-inf"))
        p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)             # [H, b, S]
        o = torch.einsum("hqk,khd->qhd", p, vf)
        delta = (df[rt] * o).sum(-1)                                        # [b, H]
        # dK, dV at the chosen keys
        dp_k = torch.einsum("qhd,khd->hqk", df[rt], vf[kr])                 # [H, b, nk]
        p_k = p[:, :, kr]
        ds_k = p_k * (dp_k - delta.T[:, :, None])
        dk += torch.einsum("hqk,qhd->khd", ds_k, qf[rt]) * scale
        dv += torch.einsum("hqk,qhd->khd", p_k, df[rt])
        # dQ at the chosen rows of this block
        sel = [i for i, r in enumerate(rr) if int(r) in q_pos]
        if sel:
            si = torch.tensor(sel)
            dp = torch.einsum("qhd,khd->hqk", df[rt[si]], vf)
            ds = p[:, si] * (dp - delta[si].T[:, :, None])
            g = torch.einsum("hqk,khd->qhd", ds, kf) * scale
            dq[torch.tensor([q_pos[int(rr[i])] for i in sel])] = g
    return dq, dk, dv


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm in fp32, cast to bf16, times the bf16 gain (attention.py:231-242)."""
    xf = x.float()
    y = bf16(xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps))
    return bf16(y * weight.float())


def camera_qk(qx, kx, cam, w_q, w_k):
    """qx + cam_q(cam), kx + cam_k(cam) with bf16 rounding (attention.py:307-320)."""
    cq = bf16(cam.float() @ w_q.float().t())
    ck = bf16(cam.float() @ w_k.float().t())
    return bf16(qx.float() + cq), bf16(kx.float() + ck)


def rope_apply(x: torch.Tensor, freqs: torch.Tensor, num_heads: int) -> torch.Tensor:
    """Rotate channel pairs by complex128 freqs [S,1,D/2] in float64 (rope.py:248-254)."""
    S, dim = x.shape
    xc = torch.view_as_complex(x.double().reshape(S, num_heads, -1, 2).contiguous())
    out = torch.view_as_real(xc * freqs.reshape(S, 1, -1)).reshape(S, dim)
    return bf16(out.float())


def project_qk(qx, kx, *, norm_q_w, norm_k_w, freqs, num_heads, eps, cam=None, w_cam_q=None,
               w_cam_k=None):
    """The Q/K tail of _project_self_attn_qkv (attention.py:355-365) from projected qx/kx."""
    qx, kx = bf16(qx.float()), bf16(kx.float())
    if cam is not None:
        qx, kx = camera_qk(qx, kx, cam, w_cam_q, w_cam_k)
    q = rms_norm(qx, norm_q_w, eps)
    k = rms_norm(kx, norm_k_w, eps)
    return rope_apply(q, freqs, num_heads), rope_apply(k, freqs, num_heads)


# ---------------------------------------------------------------------------
# RoPE frequency tables (float64)
# ---------------------------------------------------------------------------

def precompute_freqs_cis(dim: int, end: int = 1024, theta: float = 10000.0) -> torch.Tensor:
    """rope.py:103-107: e^{i * t * theta^(-2j/dim)}, shape [end, dim//2]."""
    j = torch.arange(0, dim, 2)[: dim // 2].double()
    inv = 1.0 / theta ** (j / dim)
    ang = torch.outer(torch.arange(end).double(), inv)
    return torch.polar(torch.ones_like(ang), ang)


def rerope_bands(head_dim: int = 128, end: int = 1024, theta: float = 10000.0,
                 splits=ROPE_SPLITS) -> dict:
    """rope.py:129-144: temporal band = the lowest d_t/2 frequencies of Wan's 3D temporal band."""
    d_t, d_a, d_h, d_w = splits
    d_t_old = head_dim - 2 * (head_dim // 3)
    t_old = precompute_freqs_cis(d_t_old, end, theta)
    return {"t": t_old[:, -(d_t // 2):], "h": precompute_freqs_cis(d_h, end, theta),
            "w": precompute_freqs_cis(d_w, end, theta), "splits": splits, "d_a": d_a}


def simplex_vertices(pool_size: int, d_agent: int) -> torch.Tensor:
    """rope.py:110-126: unit vertices of a regular simplex, float32 [m, d_agent//2]."""
    m, half = int(pool_size), d_agent // 2
    if m < 2 or m > half + 1:
        raise ValueError("invalid simplex pool size")
    c = torch.eye(m, dtype=torch.float64) - 1.0 / m
    c = c / c.norm(dim=1, keepdim=True).clamp(min=1e-12)
    out = torch.zeros(m, half, dtype=torch.float32)
    out[:, :m] = c.float()
    return out


def player_freqs(bands, f, h, w, vertices, vertex_id, gamma=1.0, start_frame=0) -> torch.Tensor:
    """rope.py:155-188: [f*h*w, 1, 64] complex128 in (t | agent | h | w) band order."""
    d_t, d_a, d_h, d_w = bands["splits"]
    ft = bands["t"][start_frame:start_frame + f]
    fh, fw = bands["h"][:h], bands["w"][:w]
    tt = ft[:, None, None, :].expand(f, h, w, d_t // 2)
    hh = fh[None, :, None, :].expand(f, h, w, d_h // 2)
    ww = fw[None, None, :, :].expand(f, h, w, d_w // 2)
    ang = vertices[vertex_id].double() * float(gamma)
    aa = torch.polar(torch.ones_like(ang), ang)[None].expand(f * h * w, -1)
    return torch.cat([tt.reshape(-1, d_t // 2), aa, hh.reshape(-1, d_h // 2),
                      ww.reshape(-1, d_w // 2)], dim=-1)[:, None, :]


def hub_freqs(bands, f, num_hub_tokens, start_frame=0) -> torch.Tensor:
    """rope.py:223-237: temporal phase per hub-token frame slot, identity elsewhere."""
    d_t, d_a, d_h, d_w = bands["splits"]
    ft = bands["t"][start_frame:start_frame + f].repeat_interleave(num_hub_tokens, dim=0)
    ident = torch.ones(f * num_hub_tokens, (d_a + d_h + d_w) // 2, dtype=torch.complex128)
    return torch.cat([ft, ident], dim=-1)[:, None, :]


# ---------------------------------------------------------------------------
# camera12
# ---------------------------------------------------------------------------

def camera_to_world(pose: np.ndarray) -> np.ndarray:
    """data/raw_inputs.py:250-273: [...,5] (x,y,z,yaw,pitch deg) -> [...,4,4] c2w."""
    yaw, pitch = np.deg2rad(pose[..., 3]), np.deg2rad(pose[..., 4])
    fwd = np.stack([np.cos(pitch) * np.cos(yaw), np.cos(pitch) * np.sin(yaw), -np.sin(pitch)], -1)
    fwd /= np.linalg.norm(fwd, axis=-1, keepdims=True).clip(min=1e-12)
    up_w = np.zeros_like(fwd)
    up_w[..., 2] = 1.0
    right = np.cross(fwd, up_w)
    right /= np.linalg.norm(right, axis=-1, keepdims=True).clip(min=1e-12)
    up = np.cross(right, fwd)
    up /= np.linalg.norm(up, axis=-1, keepdims=True).clip(min=1e-12)
    out = np.broadcast_to(np.eye(4), (*pose.shape[:-1], 4, 4)).copy()
    out[..., :3, 0], out[..., :3, 1], out[..., :3, 2] = right, up, -fwd
    out[..., :3, 3] = pose[..., :3]
    return out


def camera12(c2w_abs: np.ndarray, pos_scale: float) -> np.ndarray:
    """data/dataset.py:49-90: anchor-relative top 3x4 rows, translation / pos_scale -> [P,T,12]."""
    c2w = np.asarray(c2w_abs, dtype=np.float64)
    anchor = c2w[0, 0]
    w2c = np.eye(4)
    w2c[:3, :3] = anchor[:3, :3].T
    w2c[:3, 3] = -(anchor[:3, :3].T @ anchor[:3, 3])
    rel = w2c[None, None] @ c2w
    rel[..., :3, 3] /= float(pos_scale)
    return rel[..., :3, :].reshape(c2w.shape[0], c2w.shape[1], 12).astype(np.float32)
