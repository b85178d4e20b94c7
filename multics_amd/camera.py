"""Camera12 pose features and their expansion to self-attention token order.

* ``camera_to_world``  -- eye poses ``[...,5]`` (x, y, z, yaw, pitch in degrees)
  to c2w matrices with right / up / back axes (multics/data/raw_inputs.py:250-273).
* ``camera12_from_absolute_c2w`` -- anchor-relative top 3x4 rows with the
  translation divided by ``pos_scale`` (multics/data/dataset.py:49-90).
* ``build_camera_tokens`` -- per (player, frame) 12-vectors broadcast to the
  frame's L tokens in player-major order, zero rows for hub tokens
  (DiTBlock._build_camera_tokens, multics/models/blocks.py:108-148).
"""

from __future__ import annotations

import numpy as np
import torch


def camera_to_world(pose: np.ndarray) -> np.ndarray:
    yaw = np.deg2rad(pose[..., 3])
    pitch = np.deg2rad(pose[..., 4])
    forward = np.stack([np.cos(pitch) * np.cos(yaw), np.cos(pitch) * np.sin(yaw), -np.sin(pitch)],
                       axis=-1)
    forward /= np.linalg.norm(forward, axis=-1, keepdims=True).clip(min=1e-12)
    world_up = np.zeros_like(forward)
    world_up[..., 2] = 1.0
    right = np.cross(forward, world_up)
    right /= np.linalg.norm(right, axis=-1, keepdims=True).clip(min=1e-12)
    up = np.cross(right, forward)
    up /= np.linalg.norm(up, axis=-1, keepdims=True).clip(min=1e-12)
    c2w = np.broadcast_to(np.eye(4, dtype=np.float64), (*pose.shape[:-1], 4, 4)).copy()
    c2w[..., :3, 0] = right
    c2w[..., :3, 1] = up
    c2w[..., :3, 2] = -forward
    c2w[..., :3, 3] = pose[..., :3]
    return c2w


def camera12_from_absolute_c2w(c2w_abs: torch.Tensor, pos_scale: float) -> torch.Tensor:
    """``[P,T,4,4]`` -> float32 ``[P,T,12]`` anchored at player 0, frame 0."""
    if c2w_abs.ndim != 4 or tuple(c2w_abs.shape[-2:]) != (4, 4):
        raise ValueError(f"absolute c2w must be [P,T,4,4], got {tuple(c2w_abs.shape)}")
    if not torch.isfinite(c2w_abs).all():
        raise ValueError("absolute c2w contains NaN/Inf")
    if not np.isfinite(pos_scale) or float(pos_scale) <= 0:
        raise ValueError(f"camera pos_scale must be positive, got {pos_scale}")
    c2w = c2w_abs.to(dtype=torch.float64)
    bottom = torch.tensor([0.0, 0.0, 0.0, 1.0], dtype=c2w.dtype, device=c2w.device)
    if not torch.allclose(c2w[..., 3, :], bottom, atol=1e-9, rtol=0.0):
        raise ValueError("absolute c2w homogeneous row is not [0,0,0,1]")
    rot = c2w[..., :3, :3]
    eye3 = torch.eye(3, dtype=c2w.dtype, device=c2w.device)
    if not torch.allclose(rot.transpose(-1, -2) @ rot, eye3, atol=2e-7, rtol=0.0):
        raise ValueError("absolute c2w rotation is not orthonormal")
    if not torch.allclose(torch.linalg.det(rot), torch.ones(rot.shape[:-2], dtype=c2w.dtype,
                                                            device=c2w.device), atol=2e-7, rtol=0.0):
        raise ValueError("absolute c2w rotation determinant is not +1")
    anchor = c2w[0, 0]
    w2c = torch.eye(4, dtype=c2w.dtype, device=c2w.device)
    w2c[:3, :3] = anchor[:3, :3].T
    w2c[:3, 3] = -(anchor[:3, :3].T @ anchor[:3, 3])
    rel = w2c.view(1, 1, 4, 4) @ c2w
    rel[..., :3, 3] /= float(pos_scale)
    return rel[..., :3, :].reshape(c2w.shape[0], c2w.shape[1], 12).float()


def build_camera_tokens(camera_pose: torch.Tensor, num_frames: int, num_patches: int,
                        num_players: int, ref_x: torch.Tensor, include_hub: bool,
                        num_hub_tokens: int = 0):
    """``[P,F,C]`` or ``[B,P,F,C]`` -> ``[B, P*F*L (+ F*K), C]`` in ``ref_x``'s dtype/device."""
    if camera_pose is None:
        return None
    cam = camera_pose
    if cam.dim() == 3:
        cam = cam.unsqueeze(0)
    elif cam.dim() != 4:
        raise ValueError(f"camera_pose must be [P,F,C] or [B,P,F,C], got shape {tuple(camera_pose.shape)}")
    if cam.shape[1] != num_players or cam.shape[2] != num_frames:
        raise ValueError(f"camera_pose expects P={num_players}, F={num_frames}, got {tuple(cam.shape[1:3])}")
    if cam.shape[0] != ref_x.shape[0]:
        raise ValueError(f"camera_pose batch {cam.shape[0]} must match self-attn batch {ref_x.shape[0]}")
    cam = cam.to(device=ref_x.device, dtype=ref_x.dtype)
    b, p, f, c = cam.shape
    tokens = cam[:, :, :, None, :].expand(b, p, f, num_patches, c).reshape(b, p * f * num_patches, c)
    if include_hub:
        tokens = torch.cat([tokens, tokens.new_zeros(b, f * num_hub_tokens, c)], dim=1)
    return tokens
