"""Launchers of the HIP attention kernels under the reference's plugin names.

``hierarchical_tiled_full_sequence_attention`` keeps the reference signature
(multics/models/kernels/hier_tiled_attention.py:734-796) and error behaviour;
the layouts it receives come from this package's
``build_hier_tiled_full_sequence_layouts`` and carry the tile list of the HIP
forward, so all temporal blocks run in one launch.
"""

from __future__ import annotations

import ctypes as C
import math
from typing import Optional, Sequence

import torch

from . import _capi
from . import metadata as M
from .metadata import HierTiledBlockLayout, TileList, backward_lists, folded_key_list


def _stream(dev) -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _rows_view(t: torch.Tensor):
    """(tensor, token stride, head stride) of a [S,H,D] / [1,S,H,D] bf16 tensor."""
    if t.dim() == 4:
        if t.shape[0] != 1:
            raise NotImplementedError("hierarchical attention supports B=1")
        t = t[0]
    if t.dim() != 3:
        raise ValueError(f"expected [S,H,D] or [1,S,H,D], got {tuple(t.shape)}")
    if t.stride(2) != 1:
        t = t.contiguous()
    return t, t.stride(0), t.stride(1)


def hier_attention_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tiles: TileList,
                           out: torch.Tensor, *, lse: Optional[torch.Tensor] = None,
                           item_range: Optional[tuple] = None,
                           scale: Optional[float] = None) -> torch.Tensor:
    """Run ``hier_attn_fwd`` over (a range of) the work items of ``tiles``.

    ``q`` / ``out`` rows are addressed by the tile list's query rows, ``k`` / ``v``
    rows by its key indices; all are bf16 with a unit-stride head dimension.
    ``lse`` (optional, fp32 [H, S_q]) receives the natural-log softmax normaliser.
    Without ``item_range``, a list that carries the forward's own items
    (``TileList.fwd_items``: the players' ragged last items folded into their
    hubs' groups) runs those.  The launch reads ``metadata.launch_list(tiles)``:
    the same items with each key list cut to the tiles their rows can see.
    """
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
        if t.dtype != torch.bfloat16:
            raise NotImplementedError(f"{name} must be bf16, got {t.dtype}")
        if not t.is_cuda:
            raise NotImplementedError("hierarchical attention requires a GPU tensor")
    q3, q_ss, q_sh = _rows_view(q)
    k3, k_ss, k_sh = _rows_view(k)
    v3, v_ss, v_sh = _rows_view(v)
    o3, o_ss, o_sh = _rows_view(out)
    if o3.data_ptr() != (out[0] if out.dim() == 4 else out).data_ptr():
        raise ValueError("out must have a unit-stride head dimension")
    H, D = q3.shape[1], q3.shape[2]
    if k3.shape[1:] != (H, D) or v3.shape[1:] != (H, D) or o3.shape[1:] != (H, D):
        raise ValueError("q/k/v/out head shapes differ")
    if tiles.rows_per_item != 128:
        raise ValueError("hier_attn_fwd processes work items of up to 128 query rows")
    if k3.shape[0] < tiles.key_extent or v3.shape[0] < tiles.key_extent:
        raise ValueError(f"K/V hold {k3.shape[0]} rows, the tile list addresses {tiles.key_extent}")
    if q3.shape[0] < tiles.row_extent or o3.shape[0] < tiles.row_extent:
        raise ValueError(f"Q/out hold {q3.shape[0]} rows, the tile list addresses {tiles.row_extent}")
    if lse is not None and (lse.dtype != torch.float32 or lse.dim() != 2 or lse.shape[0] != H
                            or lse.shape[1] < tiles.row_extent or lse.stride(1) != 1):
        raise ValueError("lse must be fp32 [H, >=rows] with unit row stride")
    first, last = item_range if item_range is not None else (0, tiles.n_items)
    if last <= first:
        return out
    run = M.launch_list(tiles)          # each key list cut to the tiles its rows see
    items, row_table = run.items, tiles.row_table
    if item_range is None and run.fwd_items is not None:
        items, last = run.fwd_items, tiles.fwd_n_items
    args = _capi.HierFwdArgs(
        H=H, D=D, n_items=last - first, scale=float(scale if scale is not None else 1.0 / math.sqrt(D)),
        kv_rows=min(k3.shape[0], v3.shape[0]), reserved=0,
        q=q3.data_ptr(), k=k3.data_ptr(), v=v3.data_ptr(), o=o3.data_ptr(),
        lse=None if lse is None else lse.data_ptr(),
        q_ss=q_ss, q_sh=q_sh, k_ss=k_ss, k_sh=k_sh, v_ss=v_ss, v_sh=v_sh, o_ss=o_ss, o_sh=o_sh,
        lse_stride_h=0 if lse is None else lse.stride(0),
        tile_items=items.data_ptr() + first * 8 * 4, tile_kv_idx=tiles.kv_idx.data_ptr(),
        tile_kv_mask=tiles.kv_mask.data_ptr(), tile_blk_and=tiles.blk_and.data_ptr(),
        row_table=None if row_table is None else row_table.data_ptr())
    _capi.call("hier_attn_fwd", C.byref(args), _stream(q.device))
    return out


STE_CLASSES = 16


# Value written into output buffers that the kernels are expected to overwrite
# entirely (see _covers_all_rows); None leaves them uninitialised.  Tests set
# NaN to show that every row is written.
_UNCLEARED_FILL: Optional[float] = None


def _uncleared(like: torch.Tensor = None, *, size=None, dtype=None, device=None) -> torch.Tensor:
    """A buffer every row of which a kernel writes (``torch.empty``, or filled
    with ``_UNCLEARED_FILL`` when a test sets it)."""
    t = torch.empty_like(like) if like is not None else \
        torch.empty(size, dtype=dtype, device=device)
    if _UNCLEARED_FILL is not None:
        t.fill_(_UNCLEARED_FILL)
    return t


def _covers_all_rows(tiles: TileList) -> bool:
    """Whether the items of a full-sequence list own every row of
    [0, row_extent) exactly once, with queries and keys the same rows.  The
    builder records the first fact from the groups' row descriptors when it
    builds the list (``rows_exact_cover``; derived key-major lists keep the
    forward items' descriptors, so they inherit it).  Then dq_kernel writes
    every row of dQ, the forward every row of O and LSE, and dkv_kernel every
    key row of dK / dV over the key-major list."""
    return bool(tiles.rows_exact_cover) and tiles.row_extent == tiles.key_extent


def hier_attention_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                            dout: torch.Tensor, lse: torch.Tensor, tiles: TileList, *,
                            scale: Optional[float] = None,
                            key_tiles: Optional[TileList] = None,
                            ste_geometry: Optional[tuple] = None,
                            ste_pass: str = "dq",
                            no_alloc_workspace: bool = False):
    """``hier_attn_bwd``: gradients ``(dq, dk, dv)`` (bf16, shaped like q/k/v) of
    ``hier_attention_forward(q, k, v, tiles)`` given its output, its ``lse``
    and the output gradient.  ``tiles`` must be a full-sequence tile list;
    its key-major counterpart is built (and cached) on first use.

    With ``ste_geometry=(P, T, L, N, KL)`` a fourth result is returned: the
    sum of dS = P (dP - delta) over the membership-gated edges of every bit,
    as an fp32 ``[T, N, P]`` tensor (see ``membership_grad``).  The sums are
    taken inside the dQ pass over the forward list's gated entries
    (``ste_pass="dq"``, the default) or by a separate pass over the STE list
    (``ste_pass="list"``); both give the same sums up to fp32 rounding.

    ``no_alloc_workspace=True`` calls ``hier_attn_bwd_noalloc``, whose
    per-row workspace lives in the library's device array instead of a
    tensor allocated here (same results; 2 x H x rows <= 4M floats).

    Both passes run ``metadata.launch_list`` of their lists (key lists cut
    to the tiles their rows can see).
    """
    # the derivations read the built list, not a launch list cut from it
    tiles = M.built_list(tiles)
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out), ("dout", dout)):
        if t.dtype != torch.bfloat16:
            raise NotImplementedError(f"{name} must be bf16, got {t.dtype}")
        if not t.is_cuda:
            raise NotImplementedError("hierarchical attention requires a GPU tensor")
    q3, q_ss, q_sh = _rows_view(q)
    k3, k_ss, k_sh = _rows_view(k)
    v3, v_ss, v_sh = _rows_view(v)
    o3, o_ss, o_sh = _rows_view(out)
    d3, do_ss, do_sh = _rows_view(dout)
    H, D = q3.shape[1], q3.shape[2]
    for t in (k3, v3, o3, d3):
        if t.shape[1:] != (H, D):
            raise ValueError("q/k/v/out/dout head shapes differ")
    if tiles.rows_per_item != 128:
        raise ValueError("hier_attn_bwd processes work items of up to 128 rows")
    if k3.shape[0] < tiles.key_extent or v3.shape[0] < tiles.key_extent:
        raise ValueError(f"K/V hold {k3.shape[0]} rows, the tile list addresses {tiles.key_extent}")
    if min(q3.shape[0], o3.shape[0], d3.shape[0]) < tiles.row_extent:
        raise ValueError(f"Q/out/dout hold fewer rows than the tile list addresses ({tiles.row_extent})")
    if lse.dtype != torch.float32 or lse.dim() != 2 or lse.shape[0] != H or \
            lse.shape[1] < tiles.row_extent or lse.stride(1) != 1:
        raise ValueError("lse must be fp32 [H, >=rows] with unit row stride")
    ste = cls = None
    if ste_pass not in ("dq", "list"):
        raise ValueError(f"ste_pass must be 'dq' or 'list', got {ste_pass!r}")
    if ste_geometry is not None:
        P_, T_, L_, N_, KL_ = (int(x) for x in ste_geometry)
        if max(P_, N_) > STE_CLASSES:
            raise NotImplementedError(f"membership STE supports up to {STE_CLASSES} players / groups")
    list_ste = ste_geometry is not None and ste_pass == "list"
    if key_tiles is not None and not list_ste:
        kt = key_tiles
    else:
        kt, ste = backward_lists(tiles, ste_geometry if list_ste else None)
        # the players' last key rows in their hubs' key items, as the forward
        # folds their query rows (when the list has that fold)
        kt = key_tiles if key_tiles is not None else folded_key_list(tiles, kt)
    if ste_geometry is not None and not list_ste:
        cls = M.launch_ste_first(tiles, ste_geometry)
    dev = q.device
    # every row the kernels own is written; a buffer needs clearing only when
    # some of its rows belongs to no work item: dQ over the forward list,
    # dK / dV over the key-major list (a caller's key_tiles included)
    full_q = _covers_all_rows(tiles) and q3.shape[0] == tiles.row_extent
    full_kv = _covers_all_rows(kt) and kt.row_extent == tiles.key_extent and \
        k3.shape[0] == kt.row_extent and v3.shape[0] == kt.row_extent
    dq = _uncleared(q3) if full_q else torch.zeros_like(q3)
    dk = _uncleared(k3) if full_kv else torch.zeros_like(k3)
    dv = _uncleared(v3) if full_kv else torch.zeros_like(v3)
    # delta / lse2 of every query row are written by the dQ pass before the
    # key-major pass reads them; rows of no item read as 0 from a cleared buffer
    ws = None
    if not no_alloc_workspace:
        wshape = dict(size=(2, H, lse.shape[1]), dtype=torch.float32, device=dev)
        ws = _uncleared(**wshape) if full_q else torch.zeros(**wshape)
    if ste_geometry is not None:
        n_cls = max(P_, N_)     # classes are groups (player rows) or players (hub rows)
        # the dQ pass writes every row of every item; the STE-list pass only
        # the rows of its items
        pshape = dict(size=(H, tiles.row_extent, n_cls), dtype=torch.float32, device=dev)
        partial = _uncleared(**pshape) if full_q and not list_ste else torch.zeros(**pshape)
    args = _capi.HierBwdArgs(
        H=H, D=D, n_items=tiles.n_items, n_key_items=kt.n_items,
        scale=float(scale if scale is not None else 1.0 / math.sqrt(D)),
        kv_rows=min(k3.shape[0], v3.shape[0]), q_rows=min(q3.shape[0], d3.shape[0]), reserved=0,
        q=q3.data_ptr(), k=k3.data_ptr(), v=v3.data_ptr(), o=o3.data_ptr(), dout=d3.data_ptr(),
        lse=lse.data_ptr(), delta=None if ws is None else ws[0].data_ptr(),
        lse2=None if ws is None else ws[1].data_ptr(),
        dq=dq.data_ptr(), dk=dk.data_ptr(), dv=dv.data_ptr(),
        q_ss=q_ss, q_sh=q_sh, k_ss=k_ss, k_sh=k_sh, v_ss=v_ss, v_sh=v_sh, o_ss=o_ss, o_sh=o_sh,
        do_ss=do_ss, do_sh=do_sh, dq_ss=dq.stride(0), dq_sh=dq.stride(1), dk_ss=dk.stride(0),
        dk_sh=dk.stride(1), dv_ss=dv.stride(0), dv_sh=dv.stride(1), lse_stride_h=lse.stride(0),
        tile_items=M.launch_list(tiles).items.data_ptr(), tile_kv_idx=tiles.kv_idx.data_ptr(),
        tile_kv_mask=tiles.kv_mask.data_ptr(), tile_blk_and=tiles.blk_and.data_ptr(),
        key_items=M.launch_list(kt).items.data_ptr(), key_q_idx=kt.kv_idx.data_ptr(),
        key_q_mask=kt.kv_mask.data_ptr(), key_blk_and=kt.blk_and.data_ptr(),
        key_row_table=None if kt.row_table is None else kt.row_table.data_ptr())
    if ste is not None:
        sl, scls = ste
        args.n_ste_items, args.ste_classes = sl.n_items, n_cls
        args.ste_items, args.ste_kv_idx = sl.items.data_ptr(), sl.kv_idx.data_ptr()
        args.ste_kv_mask, args.ste_kv_class = sl.kv_mask.data_ptr(), scls.data_ptr()
        args.ste_partial, args.ste_stride_h = partial.data_ptr(), partial.stride(0)
    if cls is not None:
        args.ste_classes, args.tile_kv_class = n_cls, cls[0].data_ptr()
        args.tile_ste_first = cls[1].data_ptr()
        args.ste_partial, args.ste_stride_h = partial.data_ptr(), partial.stride(0)
    _capi.call("hier_attn_bwd_noalloc" if no_alloc_workspace else "hier_attn_bwd", C.byref(args),
               _stream(dev))
    shape = lambda g, like: g.reshape(like.shape) if like.dim() == 4 else g
    res = (shape(dq, q), shape(dk, k), shape(dv, v))
    if ste_geometry is None:
        return res
    P_, T_, L_, N_, KL_ = (int(x) for x in ste_geometry)
    sums = torch.empty((T_, N_, P_), dtype=torch.float32, device=dev)
    red = _capi.HierSteReduceArgs(H=H, P=P_, T=T_, L=L_, N=N_, KL=KL_, classes=n_cls,
                                  partial=partial.data_ptr(), stride_h=partial.stride(0),
                                  out=sums.data_ptr())
    _capi.call("hier_ste_reduce", C.byref(red), _stream(dev))
    return res + (sums,)


def membership_grad(logits: torch.Tensor, gated_ds: torch.Tensor) -> torch.Tensor:
    """Straight-through gradient of soft membership logits ``[T, N, P]``.

    The forward uses the hard membership ``logits > 0``.  Each edge whose
    existence depends on one membership bit (t, g, p) -- player p's row at
    frame t to a local-hub key of group g, or group g's hub row at frame t to a
    key of player p -- carries the surrogate logit bias
    ``sigmoid(logit) - stopgrad(sigmoid(logit))`` (zero in value), so
    ``dL/dlogit = sigmoid'(logit) * sum of dS over those edges`` with
    dS = dL/d(scaled score) = P (dP - delta).  Edges that are off have P = 0
    and contribute nothing; same-group player-to-player edges depend on two
    players' bits jointly and carry no surrogate bias.
    """
    sig = torch.sigmoid(logits.float())
    return (sig * (1.0 - sig) * gated_ds.to(sig.device)).to(logits.dtype)


class HierAttentionFunction(torch.autograd.Function):
    """Differentiable hierarchical attention: forward ``hier_attn_fwd`` (keeps
    the LSE), backward ``hier_attn_bwd``.  Inputs ``[S, H, D]`` (or
    ``[1, S, H, D]``) bf16 over a full-sequence tile list; optional membership
    logits ``[T, N, P]`` receive the straight-through gradient of
    ``membership_grad`` (their hard value must be the membership the tile list
    was built from; ``ste_geometry = (P, T, L, N, KL)``)."""

    @staticmethod
    def forward(ctx, q, k, v, tiles: TileList, scale: Optional[float] = None,
                logits: Optional[torch.Tensor] = None, ste_geometry: Optional[tuple] = None):
        q3 = _rows_view(q)[0]
        H = q3.shape[1]
        # the output token-major whatever q's layout (the training prologue
        # hands q over head-major): the o-projection reads it as [S, H*D]
        # with no copy
        if _covers_all_rows(tiles) and q3.shape[0] == tiles.row_extent:
            # the kernel writes every row's output and LSE (0 and -inf for a
            # row that sees no key)
            out = _uncleared(size=tuple(q.shape), dtype=q.dtype, device=q.device)
            lse = _uncleared(size=(H, q3.shape[0]), dtype=torch.float32, device=q.device)
        else:
            out = torch.zeros(tuple(q.shape), dtype=q.dtype, device=q.device)
            lse = torch.full((H, q3.shape[0]), float("-inf"), dtype=torch.float32, device=q.device)
        hier_attention_forward(q, k, v, tiles, out, lse=lse, scale=scale)
        if logits is not None:
            ctx.save_for_backward(q, k, v, out, lse, logits)
        else:
            ctx.save_for_backward(q, k, v, out, lse)
        ctx.tiles, ctx.scale, ctx.ste_geometry = tiles, scale, ste_geometry
        return out

    @staticmethod
    def backward(ctx, dout):
        saved = ctx.saved_tensors
        q, k, v, out, lse = saved[:5]
        logits = saved[5] if len(saved) > 5 else None
        want_ste = logits is not None and ctx.needs_input_grad[5]
        res = hier_attention_backward(q, k, v, out, dout.contiguous().to(torch.bfloat16), lse,
                                      ctx.tiles, scale=ctx.scale,
                                      ste_geometry=ctx.ste_geometry if want_ste else None)
        dlogits = membership_grad(logits, res[3]) if want_ste else None
        return res[0], res[1], res[2], None, None, dlogits, None


def hier_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tiles: TileList,
                   scale: Optional[float] = None, *, membership_logits: Optional[torch.Tensor] = None,
                   ste_geometry: Optional[tuple] = None) -> torch.Tensor:
    """Autograd-enabled hierarchical attention over a full-sequence tile list."""
    if membership_logits is not None and ste_geometry is None:
        raise ValueError("membership_logits need ste_geometry=(P, T, L, N, KL)")
    return HierAttentionFunction.apply(q, k, v, tiles, scale, membership_logits, ste_geometry)


def hierarchical_tiled_full_sequence_attention(*, roped_q: torch.Tensor, roped_k: torch.Tensor,
                                               value: torch.Tensor,
                                               layouts: Sequence[HierTiledBlockLayout]) -> torch.Tensor:
    """Blockwise forward on projected full-sequence Q/K/V (reference signature,
    hier_tiled_attention.py:734-796); returns ``[B, S, H*D]``."""
    if roped_k.shape != value.shape or roped_q.ndim != 4 or roped_k.ndim != 4:
        raise ValueError(
            f"Tiled128 expects Q [B,Sq,H,D] and matching K/V [B,Sk,H,D], "
            f"got {roped_q.shape}, {roped_k.shape}, {value.shape}")
    batch, seq_len, heads, head_dim = roped_q.shape
    if roped_k.shape[0] != batch or roped_k.shape[2:] != (heads, head_dim):
        raise ValueError(
            f"Tiled128 Q/K batch/head shapes must match, got {roped_q.shape}, {roped_k.shape}")
    if batch != 1 or head_dim not in (64, 128) or roped_q.dtype != torch.bfloat16:
        raise NotImplementedError(
            "hierarchical attention supports B=1, BF16, head_dim 64/128; "
            f"got B={batch}, dtype={roped_q.dtype}, head_dim={head_dim}")
    if not roped_q.is_cuda:
        raise NotImplementedError("hierarchical attention requires a GPU tensor")
    if roped_k.dtype != roped_q.dtype or value.dtype != roped_q.dtype:
        raise ValueError("Tiled128 Q/K/V dtypes must match")
    out = torch.zeros_like(roped_q)
    if not layouts:
        return out.reshape(batch, seq_len, heads * head_dim)
    tiles = layouts[0].tiles
    if tiles is None or any(l.tiles is not tiles for l in layouts):
        raise ValueError("layouts must come from one build_hier_tiled_full_sequence_layouts call")
    blocks = sorted(l.block for l in layouts)
    if blocks == list(range(len(tiles.item_ranges))):
        hier_attention_forward(roped_q, roped_k, value, tiles, out)
    else:
        for b in blocks:
            for rng in tiles.item_ranges[b]:
                hier_attention_forward(roped_q, roped_k, value, tiles, out, item_range=rng)
    return out.reshape(batch, seq_len, heads * head_dim)


def _frame_list(frames: torch.Tensor, width: int) -> tuple:
    """Frame id of each cached frame from a per-token frame tensor."""
    if width <= 0:
        return ()
    return tuple(int(x) for x in frames.reshape(-1, width)[:, 0].tolist())


def _active_frames(active_tokens: torch.Tensor, width: int) -> tuple:
    if width <= 0:
        return ()
    return tuple(bool(x) for x in active_tokens.reshape(-1, width).any(dim=1).tolist())


def hierarchical_cached_attention(*, roped_q, agent_frames, agent_keys, agent_vals, local_frames,
                                  local_keys, local_vals, local_active_tokens, global_frames,
                                  global_keys, global_vals, labels, active, P, N, L, KL, KG,
                                  n_frames, n_block, local_attn, direct_player, membership=None,
                                  global_only=None, hier_no_local_hub=False):
    """The cached-backend plugin call (reference keyword set,
    hier_segmented_attention.py:398-501, hier_tiled_attention.py:658-731,
    hier_packed_attention.py:105-244, hier_paged_attention.py:79-268): per-stream
    cache windows in, ``[1, S, H*D]`` out.  The streams are concatenated into
    one K/V pool in the reference's pool order (as the reference backends do);
    callers that keep their cache in a ``paged_cache.HierPagedKVCache`` skip
    that copy (``SelfAttention.causal_forward``).  Labels and membership
    topologies are both accepted."""
    b, s, heads, head_dim = roped_q.shape
    if b != 1 or head_dim not in (64, 128) or roped_q.dtype != torch.bfloat16:
        raise NotImplementedError(
            "hierarchical attention supports B=1, BF16, head_dim 64/128; "
            f"got B={b}, dtype={roped_q.dtype}, head_dim={head_dim}")
    if not roped_q.is_cuda:
        raise NotImplementedError("hierarchical attention requires a GPU tensor")
    no_local = bool(hier_no_local_hub)
    agent_frame_lists = tuple(_frame_list(x, L) for x in agent_frames)
    local_frame_lists = () if no_local else tuple(_frame_list(x, KL) for x in local_frames)
    global_frame_list = _frame_list(global_frames, KG) if KG > 0 else ()
    local_active_frames = () if no_local else tuple(_active_frames(x, KL)
                                                    for x in local_active_tokens)
    labels_cpu = None if labels is None else tuple(tuple(int(x) for x in r) for r in labels.tolist())
    active_cpu = tuple(tuple(bool(x) for x in r) for r in active.tolist())
    mem = None if membership is None else membership.detach().to("cpu", torch.bool).numpy()
    go = None if global_only is None else global_only.detach().to("cpu", torch.bool).numpy()
    tiles = M._build_metadata(
        device=roped_q.device, P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n_frames, n_block=n_block,
        local_attn=local_attn, agent_frame_lists=agent_frame_lists,
        local_frame_lists=local_frame_lists, global_frame_list=global_frame_list,
        local_active_frames=local_active_frames, labels=labels_cpu, q_active=active_cpu,
        direct_player=bool(direct_player), block_m=16, membership=mem, global_only=go,
        hier_no_local_hub=no_local, return_tiles=True)[6]
    streams_k = list(agent_keys) + ([] if no_local else list(local_keys)) + [global_keys]
    streams_v = list(agent_vals) + ([] if no_local else list(local_vals)) + [global_vals]
    k = torch.cat(streams_k, dim=1).reshape(-1, heads, head_dim)
    v = torch.cat(streams_v, dim=1).reshape(-1, heads, head_dim)
    out = torch.zeros((s, heads, head_dim), dtype=torch.bfloat16, device=roped_q.device)
    hier_attention_forward(roped_q[0], k, v, tiles, out)
    return out.reshape(1, s, heads * head_dim)


def hierarchical_segmented_attention(**kw):
    """hier_segmented_attention.py:398-501 (labels topology)."""
    if kw.get("membership") is not None:
        raise ValueError("hierarchical_segmented_attention takes the labels topology; "
                         "use hierarchical_paged_kv_attention for membership")
    return hierarchical_cached_attention(**kw)


def hierarchical_tiled_cached_attention(**kw):
    """hier_tiled_attention.py:658-731 (labels topology)."""
    if kw.get("membership") is not None:
        raise ValueError("hierarchical_tiled_cached_attention takes the labels topology; "
                         "use hierarchical_paged_kv_attention for membership")
    return hierarchical_cached_attention(**kw)


def hierarchical_packed_varlen_attention(**kw):
    """hier_packed_attention.py:105-244."""
    return hierarchical_cached_attention(**kw)


def hierarchical_paged_kv_attention(**kw):
    """hier_paged_attention.py:79-268 (inference only: refuses autograd inputs)."""
    if any(torch.is_tensor(t) and t.requires_grad
           for t in [kw.get("roped_q")] + list(kw.get("agent_keys", [])) + [kw.get("global_keys")]):
        raise RuntimeError("hierarchical_paged_kv_attention is inference-only (inputs require grad)")
    return hierarchical_cached_attention(**kw)


def clear_hier_paged_state() -> None:
    """hier_paged_attention.py:74-76: drop cached metadata."""
    M.clear_metadata_cache()


def qkv_prologue(qx: torch.Tensor, kx: torch.Tensor, vx: Optional[torch.Tensor], *,
                 norm_q_w: torch.Tensor, norm_k_w: torch.Tensor, rope_cos: torch.Tensor,
                 rope_sin: torch.Tensor, num_heads: int, eps: float,
                 cam: Optional[torch.Tensor] = None, w_cam_q: Optional[torch.Tensor] = None,
                 w_cam_k: Optional[torch.Tensor] = None, out_layout: str = "shd"):
    """Fused camera adapter + RMSNorm + gain + RoPE (``hier_qkv_prologue``).

    Inputs are ``[S, H*D]`` bf16 projections; returns ``(q, k, v)`` bf16 as
    ``[S, H, D]`` (``out_layout="shd"``) or head-major ``[H, S, D]`` views
    presented as ``[S, H, D]`` (``"hsd"``).  ``v`` is None when ``vx`` is None.
    """
    S, dim = qx.shape
    H = int(num_heads)
    D = dim // H
    dev = qx.device
    for t in (qx, kx) + ((vx,) if vx is not None else ()):
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.shape != (S, dim):
            raise ValueError("projections must be contiguous bf16 [S, H*D]")
    if out_layout == "shd":
        mk = lambda: torch.empty((S, H, D), dtype=torch.bfloat16, device=dev)
        q, k = mk(), mk()
        v = mk() if vx is not None else None
        ss, sh = H * D, D
    elif out_layout == "hsd":
        mk = lambda: torch.empty((H, S, D), dtype=torch.bfloat16, device=dev)
        qh, kh = mk(), mk()
        vh = mk() if vx is not None else None
        q, k = qh.permute(1, 0, 2), kh.permute(1, 0, 2)
        v = vh.permute(1, 0, 2) if vh is not None else None
        ss, sh = D, S * D
    else:
        raise ValueError(f"unknown layout {out_layout!r}")
    nw = [x.contiguous() for x in (norm_q_w, norm_k_w)]
    cs = rope_cos.contiguous().float()
    sn = rope_sin.contiguous().float()
    if cs.shape != (S, D // 2) or sn.shape != (S, D // 2):
        raise ValueError(f"rope tables must be [S, D/2] = {(S, D // 2)}, got {tuple(cs.shape)}")
    camc = None if cam is None else cam.to(torch.bfloat16).contiguous()
    wq = None if w_cam_q is None else w_cam_q.to(torch.bfloat16).contiguous()
    wk = None if w_cam_k is None else w_cam_k.to(torch.bfloat16).contiguous()
    args = _capi.HierPrologueArgs(
        S=S, H=H, D=D, eps=float(eps), qx=qx.data_ptr(), kx=kx.data_ptr(),
        vx=None if vx is None else vx.data_ptr(), cam=None if camc is None else camc.data_ptr(),
        w_cam_q=None if wq is None else wq.data_ptr(), w_cam_k=None if wk is None else wk.data_ptr(),
        C=0 if camc is None else camc.shape[-1], norm_q_w=nw[0].data_ptr(), norm_k_w=nw[1].data_ptr(),
        rope_cos=cs.data_ptr(), rope_sin=sn.data_ptr(), q_out=q.data_ptr(), k_out=k.data_ptr(),
        v_out=None if v is None else v.data_ptr(), out_stride_s=ss, out_stride_h=sh)
    _capi.call("hier_qkv_prologue", C.byref(args), _stream(dev))
    return q, k, v


def gated_residual(x: torch.Tensor, gate: torch.Tensor, residual: torch.Tensor, *,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x + gate * residual`` in one HIP pass (``hier_gated_residual``):
    GateModule.forward of the DiT block (multics/models/blocks.py:31-35) as
    applied after self-attention (blocks.py:661, 668).

    ``x`` and ``residual`` are bf16 ``[..., S, dim]``.  ``gate`` is bf16 and
    either the same shape (the reference's materialised gate) or compact,
    ``[..., F, dim]`` with F dividing S: each of its rows serves S / F
    consecutive rows -- a frame's tokens share their player-frame's gate_msa
    (blocks.py:604-616) -- so the expanded gate is never built.  Bit-identical
    to torch's bf16 expression.  ``out`` may be ``x`` (in place)."""
    for name, t in (("x", x), ("gate", gate), ("residual", residual)):
        if t.dtype != torch.bfloat16:
            raise NotImplementedError(f"gated_residual supports bf16, got {name} {t.dtype}")
        if not t.is_cuda:
            raise NotImplementedError("gated_residual requires GPU tensors")
    if residual.shape != x.shape or x.dim() < 2:
        raise ValueError(f"x {tuple(x.shape)} and residual {tuple(residual.shape)} must match")
    dim, S = x.shape[-1], x.shape[-2]
    lead = x.shape[:-2]
    if gate.shape[:-2] != lead or gate.shape[-1] != dim or gate.shape[-2] < 1 or \
            S % gate.shape[-2] != 0:
        raise ValueError(f"gate {tuple(gate.shape)} must be [..., F, {dim}] with F dividing {S}")
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != x.dtype:
        raise ValueError("out must match x")
    rows = x.numel() // dim
    xs, ys, gs, os_ = (t.reshape(-1, dim) for t in (x, residual, gate, out))
    for t in (xs, ys, gs, os_):
        if t.stride(-1) != 1:
            raise ValueError("gated_residual needs a unit channel stride")
    if os_.data_ptr() != out.data_ptr():
        raise ValueError("out must be contiguous")
    args = _capi.HierGateArgs(rows=rows, dim=dim, rows_per_gate=S // gate.shape[-2],
                              x=xs.data_ptr(), y=ys.data_ptr(), gate=gs.data_ptr(),
                              out=os_.data_ptr(), x_ss=xs.stride(0), y_ss=ys.stride(0),
                              gate_ss=gs.stride(0), out_ss=os_.stride(0))
    _capi.call("hier_gated_residual", C.byref(args), _stream(x.device))
    return out


PROLOGUE_BWD_TOKENS_PER_WAVE = 16


class QKPrologueFunction(torch.autograd.Function):
    """Differentiable q / k projection tail on the HIP kernels: forward
    ``hier_qkv_prologue`` (camera adapter, RMSNorm, gain, RoPE fused), backward
    ``hier_qk_prologue_bwd`` (the same chain's gradient recomputed in fp32 from
    the forward's inputs), plus the camera-weight gradient as the GEMM
    ``d_proj^T . cam`` and the gains' column sums.  Replaces the autograd of
    attention.py:355-365 / 307-320 / 231-242 and rope.py:248-254 on the
    training path.  Inputs: ``qx, kx`` [S, H*D] bf16 (the q / k projections),
    the RMSNorm gains, fp32 cos / sin [S, D/2], optional camera rows [S, 12]
    and adapter weights [H*D, 12].  Returns q, k as [S, H, D] views of
    head-major storage."""

    @staticmethod
    def forward(ctx, qx, kx, norm_q_w, norm_k_w, cam, w_cam_q, w_cam_k, rope_cos, rope_sin,
                num_heads: int, eps: float):
        q, k, _ = qkv_prologue(qx, kx, None, norm_q_w=norm_q_w, norm_k_w=norm_k_w,
                               rope_cos=rope_cos, rope_sin=rope_sin, num_heads=num_heads, eps=eps,
                               cam=cam, w_cam_q=w_cam_q, w_cam_k=w_cam_k, out_layout="hsd")
        ctx.save_for_backward(qx, kx, norm_q_w, norm_k_w, cam, w_cam_q, w_cam_k, rope_cos,
                              rope_sin)
        ctx.num_heads, ctx.eps = num_heads, eps
        return q, k

    @staticmethod
    def backward(ctx, dq, dk):
        qx, kx, wq, wk, cam, wcq, wck, cs, sn = ctx.saved_tensors
        H = ctx.num_heads
        S, dim = qx.shape
        D = dim // H
        dev = qx.device
        dq = torch.zeros_like(qx).view(S, H, D) if dq is None else dq
        dk = torch.zeros_like(kx).view(S, H, D) if dk is None else dk
        grads = []
        for g_ in (dq, dk):
            g_ = g_.to(torch.bfloat16)
            if g_.stride(2) != 1 or g_.stride(0) % 8 or g_.stride(1) % 8:
                g_ = g_.contiguous()
            grads.append(g_)
        dq, dk = grads
        dqx = torch.empty_like(qx)
        dkx = torch.empty_like(kx)
        args = _capi.HierPrologueBwdArgs(
            S=S, H=H, D=D, eps=float(ctx.eps), C=0 if cam is None else cam.shape[-1],
            tokens_per_wave=PROLOGUE_BWD_TOKENS_PER_WAVE, qx=qx.data_ptr(), kx=kx.data_ptr(),
            cam=None if cam is None else cam.data_ptr(),
            w_cam_q=None if cam is None else wcq.data_ptr(),
            w_cam_k=None if cam is None else wck.data_ptr(),
            norm_q_w=wq.data_ptr(), norm_k_w=wk.data_ptr(), rope_cos=cs.data_ptr(),
            rope_sin=sn.data_ptr(), dq=dq.data_ptr(), dk=dk.data_ptr(), dq_ss=dq.stride(0),
            dq_sh=dq.stride(1), dk_ss=dk.stride(0), dk_sh=dk.stride(1), dqx=dqx.data_ptr(),
            dkx=dkx.data_ptr())
        waves = int(_capi.lib().hier_qk_prologue_bwd_waves(C.byref(args)))
        if waves < 0:
            raise NotImplementedError("prologue backward: too many tokens")
        part = torch.empty((2, max(waves, 1), dim), dtype=torch.float32, device=dev)
        args.dw_q_partial, args.dw_k_partial = part[0].data_ptr(), part[1].data_ptr()
        _capi.call("hier_qk_prologue_bwd", C.byref(args), _stream(dev))
        dw = part[:, :waves].sum(dim=1) if waves else torch.zeros((2, dim), device=dev)
        dwq, dwk = (x.to(wq.dtype) for x in dw)
        dwcq = dwck = dcam = None
        if cam is not None:
            if ctx.needs_input_grad[5]:
                dwcq = torch.mm(dqx.t(), cam.to(dqx.dtype)).to(wcq.dtype)
            if ctx.needs_input_grad[6]:
                dwck = torch.mm(dkx.t(), cam.to(dkx.dtype)).to(wck.dtype)
            if ctx.needs_input_grad[4]:
                dcam = (torch.mm(dqx, wcq.to(dqx.dtype)) + torch.mm(dkx, wck.to(dkx.dtype))).to(
                    cam.dtype)
        return dqx, dkx, dwq, dwk, dcam, dwcq, dwck, None, None, None, None


def qk_prologue_train(qx, kx, *, norm_q_w, norm_k_w, rope_cos, rope_sin, num_heads, eps,
                      cam=None, w_cam_q=None, w_cam_k=None):
    """``QKPrologueFunction.apply`` with the argument checks of
    ``qkv_prologue``: q, k as [S, H, D] (head-major storage), differentiable
    in the projections, the gains and the camera adapter."""
    cs = rope_cos.contiguous().float()
    sn = rope_sin.contiguous().float()
    camc = None if cam is None else cam.to(torch.bfloat16).contiguous()
    return QKPrologueFunction.apply(qx.contiguous(), kx.contiguous(), norm_q_w, norm_k_w, camc,
                                    w_cam_q, w_cam_k, cs, sn, int(num_heads), float(eps))
