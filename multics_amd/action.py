"""Cached attention of the action branches (mouse temporal self-attention and
keyboard cross-attention) over rolling KV caches, on the HIP frame-window
attention (``hier_frame_attn``).

Reference: multics/models/blocks.py:230-375 (``_ensure_action_cache``,
``_action_temporal_cached_attn``, ``_action_keyboard_cached_attn``) and the
rolling cache append of multics/models/attention.py:90-163.  The functions
keep the reference's arguments, cache dict format (``k`` / ``v`` ``[B, size,
heads, head_dim]``, ``global_end_index`` / ``local_end_index``) and the
frame-window mask; the attention itself runs in one HIP launch per call.
"""

from __future__ import annotations

import ctypes as C
import math

import torch

from . import _capi
from .module import rope_apply
from .rolling import rolling_cache_append  # noqa: F401  (re-exported)


def _stream(dev) -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def ensure_action_cache(parent: dict, name: str, batch: int, n_heads: int, head_dim: int,
                        tokens_per_frame: int, frames: int, device, dtype) -> dict:
    """blocks.py:230-254: the rolling cache ``parent[name]``, (re)allocated
    when missing or of another shape."""
    size = frames * tokens_per_frame
    c = parent.get(name)
    if c is None or c["k"].shape[0] != batch or c["k"].shape[1] < size or \
            c["k"].shape[2] != n_heads or c["k"].shape[3] != head_dim:
        z = lambda: torch.zeros([batch, size, n_heads, head_dim], device=device, dtype=dtype)
        parent[name] = {"k": z(), "v": z(),
                        "global_end_index": torch.tensor([0], dtype=torch.long, device=device),
                        "local_end_index": torch.tensor([0], dtype=torch.long, device=device)}
    return parent[name]


def frame_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_frame: torch.Tensor,
                    k_frame: torch.Tensor, n_block: int, local_attn: int,
                    scale=None) -> torch.Tensor:
    """SDPA of ``q [B, Lq, H, D]`` over ``k, v [B, Lk, H, D]`` (bf16, GPU)
    with the frame-window mask of blocks.py:303-306 / 366-372:
    key j is visible to query i when ``k_frame[j] // n_block <= q_frame[i] //
    n_block`` and, for ``local_attn != -1``, ``q_frame[i] - k_frame[j] <
    local_attn``.  Returns ``[B, Lq, H, D]`` bf16 (0 for a query that sees
    no key)."""
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        raise RuntimeError("frame-window attention is inference-only (q/k/v require grad); run "
                           "the cached action branches under torch.no_grad() or "
                           "torch.inference_mode()")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != torch.bfloat16 or not t.is_cuda or t.dim() != 4 or t.stride(3) != 1:
            raise NotImplementedError(f"{name} must be a bf16 GPU tensor [B, L, H, D] with unit "
                                      "channel stride")
    B, Lq, H, D = q.shape
    if k.shape[0] != B or k.shape[2:] != (H, D) or v.shape != k.shape:
        raise ValueError(f"k/v {tuple(k.shape)} / {tuple(v.shape)} do not match q {tuple(q.shape)}")
    if D not in (64, 128):
        raise NotImplementedError(f"head_dim must be 64 or 128, got {D}")
    if local_attn == 0 or local_attn < -1 or n_block < 1:
        raise ValueError(f"invalid local_attn={local_attn} / n_block={n_block}")
    qf = torch.as_tensor(q_frame, dtype=torch.int32, device=q.device).contiguous()
    kf = torch.as_tensor(k_frame, dtype=torch.int32, device=q.device).contiguous()
    if qf.numel() != Lq or kf.numel() != k.shape[1]:
        raise ValueError("q_frame / k_frame lengths must match Lq / Lk")
    out = torch.empty((B, Lq, H, D), dtype=torch.bfloat16, device=q.device)
    a = _capi.HierFrameAttnArgs(
        B=B, Lq=Lq, Lk=k.shape[1], H=H, D=D, n_block=int(n_block), local_attn=int(local_attn),
        scale=float(scale if scale is not None else 1.0 / math.sqrt(D)),
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), o=out.data_ptr(),
        q_sb=q.stride(0), q_ss=q.stride(1), q_sh=q.stride(2), k_sb=k.stride(0),
        k_ss=k.stride(1), k_sh=k.stride(2), v_sb=v.stride(0), v_ss=v.stride(1),
        v_sh=v.stride(2), o_sb=out.stride(0), o_ss=out.stride(1), o_sh=out.stride(2),
        q_frame=qf.data_ptr(), k_frame=kf.data_ptr())
    _capi.call("hier_frame_attn", C.byref(a), _stream(q.device))
    return out


def _window(cache, attn_start, local_end):
    g_start = int(cache["global_end_index"].item()) - int(cache["local_end_index"].item())
    return (cache["k"][:, attn_start:local_end], cache["v"][:, attn_start:local_end],
            g_start + torch.arange(attn_start, local_end))


def action_temporal_cached_attention(attn, x, freqs_temporal, kv_cache, start_frame, n_block,
                                     local_attn):
    """blocks.py:256-308: mouse-branch temporal self-attention, one token per
    frame (``x [B, f, dim]``), over the rolling ``kv_cache["action_temporal"]``."""
    B, f, dim = x.shape
    nh = attn.num_heads
    hd = dim // nh
    q = rope_apply(attn.norm_q(attn.q(x)), freqs_temporal, nh)
    k = rope_apply(attn.norm_k(attn.k(x)), freqs_temporal, nh)
    v = attn.v(x)
    retention = local_attn + f if local_attn != -1 else None
    cache = ensure_action_cache(kv_cache, "action_temporal", B, nh, hd, tokens_per_frame=1,
                                frames=retention if retention is not None else start_frame + f,
                                device=x.device, dtype=x.dtype)
    attn_start, local_end = rolling_cache_append(
        cache, k.view(B, f, nh, hd), v.view(B, f, nh, hd), current_start=start_frame,
        current_end=start_frame + f,
        local_attn_size=retention if retention is not None else -1, sink_size=0,
        tokens_per_frame=1)
    wk, wv, gk = _window(cache, attn_start, local_end)
    out = frame_attention(q.view(B, f, nh, hd), wk, wv, start_frame + torch.arange(f), gk,
                          n_block, local_attn)
    return attn.o(out.view(B, f, dim))


def action_keyboard_cached_attention(attn, x, kbd_ctx, kv_cache, start_frame, n_block, local_attn,
                                     num_patches, tokens_per_kbd_frame):
    """blocks.py:310-375: keyboard cross-attention of the block's video
    tokens ``x [B, f*num_patches, dim]`` (frame-major) over the rolling
    ``kv_cache["action_keyboard"]`` of keyboard tokens."""
    B, _, dim = x.shape
    nh = attn.num_heads
    hd = dim // nh
    tpf = tokens_per_kbd_frame
    f = kbd_ctx.shape[1] // tpf
    ctx = kbd_ctx[:, 257:] if getattr(attn, "has_image_input", False) else kbd_ctx
    q = attn.norm_q(attn.q(x))
    k = attn.norm_k(attn.k(ctx))
    v = attn.v(ctx)
    retention = local_attn + f if local_attn != -1 else None
    cache = ensure_action_cache(kv_cache, "action_keyboard", B, nh, hd, tokens_per_frame=tpf,
                                frames=retention if retention is not None else start_frame + f,
                                device=x.device, dtype=x.dtype)
    attn_start, local_end = rolling_cache_append(
        cache, k.view(B, f * tpf, nh, hd), v.view(B, f * tpf, nh, hd),
        current_start=start_frame * tpf, current_end=(start_frame + f) * tpf,
        local_attn_size=retention if retention is not None else -1, sink_size=0,
        tokens_per_frame=tpf)
    wk, wv, gtok = _window(cache, attn_start, local_end)
    qf = (start_frame + torch.arange(f)).repeat_interleave(num_patches)
    out = frame_attention(q.view(B, -1, nh, hd), wk, wv, qf, gtok // tpf, n_block, local_attn)
    return attn.o(out.view(B, -1, dim))
