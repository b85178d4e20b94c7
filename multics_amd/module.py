"""Drop-in ``SelfAttention`` for the Wan-DiT blocks, on the HIP kernels.

Same constructor, parameters (state-dict keys ``q, k, v, o, norm_q, norm_k,
cam_q, cam_k``), mutable attributes and call signatures as the reference module
(multics/models/attention.py:255-442):

* ``forward_hier_tiled_ste(x, freqs, mask, *, group_labels, active_group, ...)``
  -- the training / full-sequence hierarchical forward.  The reference takes the
  Tiled128 value and the FlexAttention Jacobian (attention.py:367-434); here
  value and Jacobian both come from the HIP kernels (``hier_attn_fwd`` /
  ``hier_attn_bwd``), so the straight-through combination is the identity.
  ``mask`` (a Flex BlockMask in the reference) is accepted and not needed: the
  tile list comes from the group arguments.
* ``forward_hier_membership(...)`` -- the same for membership / global_only
  topologies, optionally with soft membership logits that receive the
  straight-through gradient (``kernels.membership_grad``).
* ``forward(x, freqs, mask=None, cam_tokens=None)`` -- dense boolean masks go
  to ``scaled_dot_product_attention`` as in the reference (attention.py:39-54).
* ``causal_forward(...)`` / ``causal_forward_hier_hub(...)`` -- one block of a
  chunked causal rollout through a ``paged_cache.HierPagedKVCache``
  (attention.py:456-1043): the block's K/V go into their pool pages, the tile
  list addresses the pool, one HIP forward computes every stream.

Q/K/V projection: with autograd active, torch ops with the reference's
rounding points (camera adapter, RMSNorm in fp32, RoPE in float64); without
autograd, the fused HIP prologue (camera + RMSNorm + gain + RoPE in one pass).
"""

from __future__ import annotations


import torch
import torch.nn as nn
import torch.nn.functional as F

from . import metadata as M
from .kernels import (_covers_all_rows, _uncleared, gated_residual, hier_attention,
                      hier_attention_forward, qk_prologue_train, qkv_prologue)
from .hier_masks import HierBlockMask
from .kv_cache import stream_pool
from .paged_cache import HierPagedKVCache
from .rolling import rolling_bool_cache_append, rolling_cache_append
from .rope import freqs_to_cos_sin
from .topology import _prepare_hier_group_tensors, _prepare_hier_membership_tensors


class RMSNorm(nn.Module):
    """attention.py:231-242: normalise in fp32, cast back, times the gain."""

    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)).to(x.dtype) * \
            self.weight


class GateModule(nn.Module):
    """blocks.py:31-35: ``x + gate * residual``, on the HIP gated-residual pass
    (``kernels.gated_residual``; bf16 GPU tensors).  ``gate`` is the
    reference's materialised gate (same shape as ``x``) or the compact
    per-frame gate ``[..., F, dim]``."""

    def forward(self, x, gate, residual):
        return gated_residual(x, gate, residual)


class CompatibleLinear(nn.Linear):
    """nn.Linear with the reference's extra constructor arguments
    (compatible_linear.py:38-50).  The reference zero-pads the input dimension
    to ``input_alignment`` for one CUDA GEMM path; padding with zeros does not
    change the product, so this is a plain linear layer."""

    def __init__(self, in_features, out_features, bias=True, *, output_chunk_size=0,
                 input_alignment=1, device=None, dtype=None):
        if output_chunk_size < 0 or input_alignment < 1:
            raise ValueError("output_chunk_size must be >= 0 and input_alignment >= 1")
        super().__init__(in_features, out_features, bias=bias, device=device, dtype=dtype)
        self.output_chunk_size = output_chunk_size
        self.input_alignment = input_alignment


def rope_apply(x: torch.Tensor, freqs: torch.Tensor, num_heads: int) -> torch.Tensor:
    """rope.py:248-254: rotate channel pairs by complex ``freqs`` [S, 1, D/2] in
    float64 and cast back to the input dtype."""
    b, s, dim = x.shape
    xc = torch.view_as_complex(x.to(torch.float64).reshape(b, s, num_heads, -1, 2))
    return torch.view_as_real(xc * freqs.to(x.device)).flatten(2).to(x.dtype)


def _attn_out(tiles, s, H, D, device):
    """Output buffer of a full-sequence forward: uncleared when the list's
    items own every one of the s rows (the kernel then writes each, 0 for a
    row that sees no key), zero-filled otherwise."""
    if _covers_all_rows(tiles) and tiles.row_extent == s:
        return _uncleared(size=(s, H, D), dtype=torch.bfloat16, device=device)
    return torch.zeros((s, H, D), dtype=torch.bfloat16, device=device)


class SelfAttention(nn.Module):
    def __init__(self, dim: int, num_heads: int, eps: float = 1e-06):
        super().__init__()
        self.dim = dim
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.q = nn.Linear(dim, dim)
        self.k = nn.Linear(dim, dim)
        self.v = nn.Linear(dim, dim)
        self.o = nn.Linear(dim, dim)
        self.norm_q = RMSNorm(dim, eps=eps)
        self.norm_k = RMSNorm(dim, eps=eps)
        self.eps = eps
        self.sink_size = 0
        self.local_attn_size = 6
        self.num_frame_per_block = 7
        self.attn_impl = "sdpa"
        self.max_attention_size = self.local_attn_size * 3072
        self.hier_no_local_hub = False
        self.cam_dim = None
        self.cam_q = None
        self.cam_k = None
        self.cam_dropout_p = 0.0

    # ---- camera adapters (attention.py:278-320) ---------------------------------

    def enable_camera_pose_qk(self, cam_dim: int, dropout_p: float = 0.1):
        """Zero-initialised, bias-free camera adapters on Q and K."""
        cam_dim = int(cam_dim)
        dropout_p = float(dropout_p)
        if not 0.0 <= dropout_p < 1.0:
            raise ValueError(f"camera dropout_p must be in [0,1), got {dropout_p}")
        if self.cam_q is not None and self.cam_dim == cam_dim:
            self.cam_dropout_p = dropout_p
            return
        device, dtype = self.q.weight.device, self.q.weight.dtype
        self.cam_dim = cam_dim
        self.cam_dropout_p = dropout_p
        self.cam_q = CompatibleLinear(cam_dim, self.dim, bias=False, input_alignment=16).to(
            device=device, dtype=dtype)
        self.cam_k = CompatibleLinear(cam_dim, self.dim, bias=False, input_alignment=16).to(
            device=device, dtype=dtype)
        nn.init.zeros_(self.cam_q.weight)
        nn.init.zeros_(self.cam_k.weight)

    def _check_cam(self, qx, cam_tokens):
        if cam_tokens is None:
            return None
        if self.cam_q is None or self.cam_k is None:
            raise RuntimeError("camera_pose was provided but enable_camera_pose_qk() was not called")
        if cam_tokens.shape[:2] != qx.shape[:2]:
            raise ValueError(f"camera tokens shape {tuple(cam_tokens.shape[:2])} must match q/k "
                             f"tokens {tuple(qx.shape[:2])}")
        return cam_tokens.to(device=qx.device, dtype=qx.dtype)

    def _apply_camera_qk(self, qx, kx, cam_tokens=None):
        cam = self._check_cam(qx, cam_tokens)
        if cam is None:
            return qx, kx
        cam = F.dropout(cam, p=self.cam_dropout_p, training=self.training)
        return qx + self.cam_q(cam), kx + self.cam_k(cam)

    # ---- projections ------------------------------------------------------------

    def _project_self_attn_qkv(self, x, freqs, cam_tokens=None):
        """Differentiable Q/K/V (attention.py:355-365)."""
        qx, kx = self._apply_camera_qk(self.q(x), self.k(x), cam_tokens)
        q = rope_apply(self.norm_q(qx), freqs, self.num_heads)
        k = rope_apply(self.norm_k(kx), freqs, self.num_heads)
        return q, k, self.v(x)

    def _fused_ok(self, x, cam_tokens) -> bool:
        dropout = cam_tokens is not None and self.training and self.cam_dropout_p > 0
        return (x.is_cuda and x.dtype == torch.bfloat16 and x.shape[0] == 1 and not dropout and
                self.q.weight.dtype == torch.bfloat16 and self.norm_q.weight.dtype == torch.bfloat16
                and self.head_dim in (64, 128))

    def _project_fused(self, x, freqs, cam_tokens=None):
        """No-grad Q/K/V: GEMMs, then the fused HIP prologue on q and k.
        Returns [S, H, D] views: q and k of head-major storage (each head's
        keys one contiguous slab: the K gathers fetch fewer bytes from HBM,
        at the same speed), V the v projection itself, read in place (the
        attention kernels take any row / head strides)."""
        cam = self._check_cam(x, cam_tokens)
        qx, kx, vx = (lin(x)[0].contiguous() for lin in (self.q, self.k, self.v))
        cs, sn = freqs_to_cos_sin(freqs, device=x.device)
        q, k, _ = qkv_prologue(
            qx, kx, None, norm_q_w=self.norm_q.weight, norm_k_w=self.norm_k.weight, rope_cos=cs,
            rope_sin=sn, num_heads=self.num_heads, eps=self.norm_q.eps,
            cam=None if cam is None else cam[0],
            w_cam_q=None if cam is None else self.cam_q.weight,
            w_cam_k=None if cam is None else self.cam_k.weight, out_layout="hsd")
        return q, k, vx.view(vx.shape[0], self.num_heads, self.head_dim)

    def _project_train(self, x, freqs, cam_tokens):
        """Differentiable [S, H, D] bf16 Q/K/V.  On the GPU, for bf16 weights and
        model dims that are multiples of 512 (up to 4096), the q / k tail runs
        on the HIP prologue forward and backward (``qk_prologue_train``) after
        the three GEMMs; otherwise the reference's torch ops
        (``_project_self_attn_qkv``)."""
        s = x.shape[1]
        H, D = self.num_heads, self.head_dim
        dim = H * D
        if self._fused_ok(x, cam_tokens) and dim % 512 == 0 and dim <= 4096:
            cam = self._check_cam(x, cam_tokens)
            qx, kx, vx = (lin(x)[0] for lin in (self.q, self.k, self.v))
            cs, sn = freqs_to_cos_sin(freqs, device=x.device)
            q, k = qk_prologue_train(
                qx, kx, norm_q_w=self.norm_q.weight, norm_k_w=self.norm_k.weight, rope_cos=cs,
                rope_sin=sn, num_heads=H, eps=self.norm_q.eps,
                cam=None if cam is None else cam[0],
                w_cam_q=None if cam is None else self.cam_q.weight,
                w_cam_k=None if cam is None else self.cam_k.weight)
            return q, k, vx.view(s, H, D)
        return tuple(t.to(torch.bfloat16).view(s, H, D)
                     for t in self._project_self_attn_qkv(x, freqs, cam_tokens))

    def _qkv_blocks(self, x, freqs, cam_tokens):
        """[S, H, D] bf16 Q/K/V of a [1, S, dim] input (fused prologue when it applies)."""
        s = x.shape[1]
        H, D = self.num_heads, self.head_dim
        if self._fused_ok(x, cam_tokens):
            return self._project_fused(x, freqs, cam_tokens)
        return tuple(t.to(torch.bfloat16).view(s, H, D)
                     for t in self._project_self_attn_qkv(x, freqs, cam_tokens))

    def _hier(self, x, freqs, tiles, cam_tokens, logits=None, geometry=None):
        b, s, dim = x.shape
        if b != 1:
            raise NotImplementedError("hierarchical attention supports B=1")
        H, D = self.num_heads, self.head_dim
        if torch.is_grad_enabled():
            q, k, v = self._project_train(x, freqs, cam_tokens)
            y = hier_attention(q, k, v, tiles, membership_logits=logits, ste_geometry=geometry)
        else:
            q, k, v = self._qkv_blocks(x, freqs, cam_tokens)
            y = _attn_out(tiles, s, H, D, x.device)
            hier_attention_forward(q, k, v, tiles, y)
        return self.o(y.reshape(1, s, dim).to(self.o.weight.dtype))

    # ---- entry points -------------------------------------------------------------

    def forward_hier_tiled_ste(self, x, freqs, mask, *, group_labels, active_group, num_players,
                               num_frames, num_patches, num_groups, num_local_hub_tokens,
                               num_global_hub_tokens, direct_player, tiled_layouts=None,
                               cam_tokens=None):
        """Full-sequence hierarchical attention (labels topology), reference
        signature (attention.py:367-434)."""
        if tiled_layouts is None:
            # the module needs only the HIP tile list (merged hub groups):
            # no reference-format layouts are built
            labels, active = M.tiled_full_sequence_inputs(
                num_players=num_players, num_frames=num_frames, num_groups=num_groups,
                num_frame_per_block=self.num_frame_per_block,
                local_attn_size=self.local_attn_size, group_labels=group_labels,
                active_group=active_group)
            tiles = M.full_sequence_tiles(
                device=x.device, P=int(num_players), T=int(num_frames), L=int(num_patches),
                N=int(num_groups), KL=int(num_local_hub_tokens), KG=int(num_global_hub_tokens),
                n=self.num_frame_per_block, window=self.local_attn_size,
                direct=bool(direct_player), labels=labels, active=active)
            return self._hier(x, freqs, tiles, cam_tokens)
        tiles = tiled_layouts[0].tiles
        if tiles is None or any(l.tiles is not tiles for l in tiled_layouts):
            raise ValueError("tiled_layouts must come from one build_hier_tiled_full_sequence_layouts call")
        return self._hier(x, freqs, tiles, cam_tokens)

    def forward_hier_membership(self, x, freqs, *, num_players, num_frames, num_patches, num_groups,
                                num_local_hub_tokens, num_global_hub_tokens, direct_player,
                                membership=None, global_only=None, membership_logits=None,
                                active_group=None, cam_tokens=None):
        """Full-sequence hierarchical attention for a membership topology
        ``[T, N, P]`` (hier_masks.py:127-193, 510-641).  With
        ``membership_logits`` the hard membership is ``logits > 0`` and the
        logits receive the straight-through gradient."""
        P, T, L = int(num_players), int(num_frames), int(num_patches)
        N, KL, KG = int(num_groups), int(num_local_hub_tokens), int(num_global_hub_tokens)
        if membership_logits is not None:
            if tuple(membership_logits.shape) != (T, N, P):
                raise ValueError(f"membership_logits must be [T,N,P] = {(T, N, P)}")
            if global_only is None and active_group is None and membership_logits.is_cuda:
                # the lists of logits > 0, rebuilt on the device every call
                # with no host read-back
                tiles = M.membership_logits_tiles(
                    membership_logits, P=P, T=T, L=L, N=N, KL=KL, KG=KG,
                    n=self.num_frame_per_block, window=self.local_attn_size,
                    direct=direct_player, no_local=self.hier_no_local_hub)
                return self._hier(x, freqs, tiles, cam_tokens, logits=membership_logits,
                                  geometry=(P, T, L, N, KL))
            mem = (membership_logits.detach() > 0).cpu().numpy()
        elif membership is not None:
            mem = torch.as_tensor(membership).detach().to("cpu", torch.bool).numpy().reshape(T, N, P)
        else:
            raise ValueError("membership or membership_logits is required")
        go = (~mem.any(1) if global_only is None else
              torch.as_tensor(global_only).detach().to("cpu", torch.bool).numpy().reshape(T, P))
        act = None if active_group is None else \
            torch.as_tensor(active_group).detach().to("cpu", torch.bool).numpy().reshape(T, N)
        tiles = M.full_sequence_tiles(device=x.device, P=P, T=T, L=L, N=N, KL=KL, KG=KG,
                                      n=self.num_frame_per_block, window=self.local_attn_size,
                                      direct=direct_player, membership=mem, global_only=go,
                                      active=act, no_local=self.hier_no_local_hub)
        geometry = (P, T, L, N, KL) if membership_logits is not None else None
        return self._hier(x, freqs, tiles, cam_tokens, logits=membership_logits, geometry=geometry)

    def forward(self, x, freqs, mask=None, cam_tokens=None):
        """attention.py:436-442.  ``mask`` is a ``hier_masks.HierBlockMask``
        (the drop-in for the reference's FlexAttention BlockMask of the
        hierarchical topology: HIP forward, and HIP backward under autograd),
        a dense boolean mask or None (``scaled_dot_product_attention``)."""
        if isinstance(mask, HierBlockMask):
            return self._forward_block_mask(x, freqs, mask, cam_tokens)
        if mask is not None and not torch.is_tensor(mask):
            raise NotImplementedError(
                f"unsupported mask type {type(mask).__name__}: pass the HierBlockMask of "
                "multics_amd.hier_masks.build_stage2_hier_flex_block_mask, a dense bool mask or None")
        q, k, v = self._project_self_attn_qkv(x, freqs, cam_tokens)
        b, s, _ = q.shape
        H = self.num_heads
        split = lambda t: t.view(b, s, H, self.head_dim).transpose(1, 2)
        am = None if mask is None else mask.to(device=q.device, dtype=torch.bool)
        y = F.scaled_dot_product_attention(split(q), split(k), split(v), attn_mask=am)
        return self.o(y.transpose(1, 2).reshape(b, s, self.dim))

    def _forward_block_mask(self, x, freqs, mask, cam_tokens):
        """The FlexAttention path (attention.py:322-353, 436-442) on the HIP
        kernels.  Every edge of the mask except one class is in the tile list;
        the exception, an inactive local-hub row's self edge, is a softmax over
        one key, so that row's output is its own value (and its query and key
        get no gradient from it)."""
        b, s, dim = x.shape
        if b != 1:
            raise NotImplementedError("hierarchical attention supports B=1")
        if s != mask.S:
            raise ValueError(f"x has {s} tokens, the block mask covers S={mask.S}")
        H, D = self.num_heads, self.head_dim
        if torch.is_grad_enabled():
            q, k, v = self._project_train(x, freqs, cam_tokens)
            y = hier_attention(q, k, v, mask.tiles)
        else:
            q, k, v = self._qkv_blocks(x, freqs, cam_tokens)
            y = _attn_out(mask.tiles, s, H, D, x.device)
            hier_attention_forward(q, k, v, mask.tiles, y)
        if mask.self_rows.numel():
            rows = mask.self_rows.to(x.device)
            y = y.index_copy(0, rows, v.index_select(0, rows).to(y.dtype))
        return self.o(y.reshape(1, s, dim).to(self.o.weight.dtype))

    # ---- cached rollout (attention.py:456-1043) ------------------------------------

    def causal_forward_hier_hub(self, x, freqs, kv_cache, current_start=0, num_frames=None,
                                num_players=None, num_hub_tokens=None, cam_tokens=None,
                                group_labels=None, active_group=None, direct_player=False,
                                membership=None, global_only=None):
        """One block ``x [B, P*n*L + n*(N*KL+KG), dim]`` of a cached rollout.

        Same checks and errors as the reference; the block's K/V are written
        into ``kv_cache`` (refresh in place when the block is re-run) and the
        block attends to the cached window of every stream.  B is 1 as in the
        reference, or the batch of ``kv_cache`` (e.g. the positive and
        negative prompts of classifier-free guidance, which the reference runs
        as two calls on two caches): the members share the topology and run
        in one attention launch."""
        paged = isinstance(kv_cache, HierPagedKVCache)
        if not paged and not (isinstance(kv_cache, dict) and kv_cache.get("hier_hub", False)):
            raise ValueError("Hierarchical causal attention requires a hier KV cache "
                             "(a paged_cache.HierPagedKVCache or the reference's cache dict)")
        if torch.is_grad_enabled() and (x.requires_grad or
                                        any(p.requires_grad for p in self.parameters())):
            # the reference's cached backends refuse autograd the same way
            # (hier_paged_attention.py:123-124); its cached rollouts run under
            # torch.inference_mode (training.py:1112)
            raise RuntimeError("cached hierarchical attention is inference-only (autograd is "
                               "enabled and the input or the weights require grad); run it "
                               "under torch.no_grad() or torch.inference_mode()")
        b, s, dim = x.shape
        cache_b = kv_cache.B if paged else 1
        if b != cache_b:
            raise NotImplementedError("hierarchical attention supports B=1" if cache_b == 1 else
                                      f"the KV cache holds a batch of {cache_b}, got B={b}")
        H, D = self.num_heads, self.head_dim
        P = int(num_players if num_players is not None else kv_cache["num_players"])
        N, KL, KG = int(kv_cache["num_groups"]), int(kv_cache["num_local_hub_tokens"]), \
            int(kv_cache["num_global_hub_tokens"])
        no_local = bool(getattr(self, "hier_no_local_hub", False))
        if bool(kv_cache.get("hier_no_local_hub", False)) != no_local:
            raise ValueError("hier_no_local_hub mismatch between SelfAttention and KV cache")
        if paged and P != kv_cache.P:
            raise ValueError(f"num_players={P} does not match the KV cache ({kv_cache.P})")
        n = int(num_frames)
        k_total = int(num_hub_tokens if num_hub_tokens is not None else N * KL + KG)
        if k_total != N * KL + KG:
            raise ValueError(f"hier_hub K_total mismatch: {k_total} != {N}*{KL}+{KG}")
        if no_local and (KL != 0 or KG <= 0):
            raise ValueError("hier_no_local_hub cached attention requires K_L=0 and K_G>0; "
                             f"got K_L={KL}, K_G={KG}")
        use_mem = membership is not None
        if use_mem:
            mem, go, act = _prepare_hier_membership_tensors(membership, global_only, active_group,
                                                            P, n, N, "cpu", allow_full_t=True)
            labels = None
        else:
            labels, act = _prepare_hier_group_tensors(group_labels, active_group, P, n, N, "cpu")
            if n > 1 and labels.numel() and not torch.equal(labels, labels[:1].expand_as(labels)):
                raise ValueError("hier_hub cached inference requires group_labels constant inside "
                                 "each latent block")
        hub_len = n * k_total
        agent_len = s - hub_len
        if agent_len <= 0 or agent_len % (P * n) != 0:
            raise ValueError(f"hier_hub causal seq shape invalid: S={s}, hub_len={hub_len}, P={P}, "
                             f"n={n}")
        L = agent_len // (P * n)
        if paged and L != kv_cache.L:
            raise ValueError(f"tokens per player frame {L} do not match the KV cache ({kv_cache.L})")
        if freqs.shape[0] != s:
            raise ValueError("hier_hub causal_forward expects freqs.shape[0] == seq_len")
        start_frame = int(current_start) // max(P * L, 1)
        if use_mem:
            T_full = int(mem.shape[0])
            if start_frame < 0 or start_frame + n > T_full:
                raise ValueError(f"hier_hub membership T={T_full} does not cover cached block "
                                 f"[{start_frame},{start_frame + n})")
            mb = mem[start_frame:start_frame + n]
            gb = go[start_frame:start_frame + n]
            if n > 1 and (not torch.equal(mb, mb[:1].expand_as(mb)) or
                          not torch.equal(gb, gb[:1].expand_as(gb))):
                raise ValueError("hier_hub cached inference requires membership / global_only "
                                 "constant inside each latent block")
            act = act[start_frame:start_frame + n]
        if not paged:
            return self._causal_rolling(
                x, freqs, kv_cache, start_frame=start_frame, n=n, P=P, N=N, L=L, KL=KL, KG=KG,
                labels=labels, act=act, mem=mem if use_mem else None,
                go=go if use_mem else None, no_local=no_local, direct_player=direct_player,
                cam_tokens=cam_tokens)
        if b == 1:
            q, k, v = self._qkv_blocks(x, freqs, cam_tokens)
        else:   # batch-major heads: member i's head h is head i * H + h
            parts = [self._qkv_blocks(x[i:i + 1], freqs,
                                      None if cam_tokens is None else cam_tokens[i:i + 1])
                     for i in range(b)]
            q, k, v = (torch.stack([pt[j] for pt in parts], dim=1).view(s, b * H, D)
                       for j in range(3))
        kv_cache.append(k, v, start_frame, n, act.numpy())
        frames, bases, lact = kv_cache.window(start_frame + n - 1)
        tiles = M.cached_tiles(
            device=x.device, P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n,
            n_block=int(self.num_frame_per_block), local_attn=int(self.local_attn_size),
            frames=frames, tile_bases=bases, local_active_frames=lact,
            labels=None if labels is None else labels.tolist(), q_active=act.tolist(),
            direct_player=bool(direct_player),
            membership=mem.numpy() if use_mem else None,
            global_only=go.numpy() if use_mem else None, hier_no_local_hub=no_local)
        out = torch.zeros((s, b * H, D), dtype=torch.bfloat16, device=x.device)
        hier_attention_forward(q, kv_cache.k, kv_cache.v, tiles, out)
        out = out.view(s, b, dim).transpose(0, 1)
        return self.o(out.to(self.o.weight.dtype))

    def _causal_rolling(self, x, freqs, kv_cache, *, start_frame, n, P, N, L, KL, KG, labels,
                        act, mem, go, no_local, direct_player, cam_tokens):
        """One cached block over the reference's cache dict: the block's K/V are
        appended to every stream's rolling buffer (attention.py:605-666,
        rolling.py), the windows are read where they lie -- in place when the
        buffers are slices of one pool (``kv_cache.initialize_hier_kv_cache``),
        else concatenated as the reference's backends do -- and one HIP
        forward computes every stream."""
        s, dim = x.shape[1], x.shape[2]
        H, D = self.num_heads, self.head_dim
        dev = x.device
        W = int(self.local_attn_size)
        retention = W + n if W != -1 else -1
        q, k, v = self._qkv_blocks(x, freqs, cam_tokens)
        a_len = P * n * L
        l0, g0 = a_len, a_len + n * N * KL
        agents, hubs, glob = kv_cache["agent_caches"], kv_cache["local_hubs"], kv_cache["global_hub"]
        f0, f1 = start_frame, start_frame + n
        ka, va = k[:a_len].reshape(P, n * L, H, D), v[:a_len].reshape(P, n * L, H, D)
        for p in range(P):
            rolling_cache_append(agents[p], ka[p][None], va[p][None], f0 * L, f1 * L, retention, 0, L)
        if not no_local:
            kl, vl = k[l0:g0].reshape(n, N, KL, H, D), v[l0:g0].reshape(n, N, KL, H, D)
            act_dev = act.to(dev)
            for g in range(N):
                rolling_bool_cache_append(hubs[g], "active", act_dev[:, g].repeat_interleave(KL),
                                          f0 * KL, f1 * KL, retention, 0, KL)
                rolling_cache_append(hubs[g], kl[:, g].reshape(1, n * KL, H, D),
                                     vl[:, g].reshape(1, n * KL, H, D), f0 * KL, f1 * KL,
                                     retention, 0, KL)
        if KG > 0:
            rolling_cache_append(glob, k[g0:].reshape(1, n * KG, H, D),
                                 v[g0:].reshape(1, n * KG, H, D), f0 * KG, f1 * KG, retention, 0,
                                 KG)
        end_frame = f1 - 1

        def window(c, tpf):          # attention.py:667-674
            local_end = int(c["local_end_index"].item())
            n_cached = local_end // tpf if tpf > 0 else 0
            first = end_frame - n_cached + 1
            return list(range(first, first + n_cached)), local_end

        streams = [(c, L) for c in agents]
        if not no_local:
            streams += [(c, KL) for c in hubs]
        if KG > 0:
            streams += [(glob, KG)]
        wins = [window(c, tpf) for c, tpf in streams]
        pool = stream_pool(kv_cache)
        if pool is not None and (no_local or len(hubs) == N):
            pk, pv, offs = pool
            offs = list(offs[:P + (0 if no_local else N)]) + [offs[-1]]
            kpool, vpool = pk[0], pv[0]
        else:                        # buffers outside one pool: concatenate the windows
            kpool = torch.cat([c["k"][0, :e] for (c, _), (_, e) in zip(streams, wins)], dim=0)
            vpool = torch.cat([c["v"][0, :e] for (c, _), (_, e) in zip(streams, wins)], dim=0)
            offs, o = [], 0
            for _, e in wins:
                offs.append(o)
                o += e
            if KG == 0:
                offs.append(o)
        base = lambda i, tpf: [offs[i] + j * tpf for j in range(len(wins[i][0]))]
        agent_b = [base(p, L) for p in range(P)]
        local_b = [] if no_local else [base(P + g, KL) for g in range(N)]
        gi = P + (0 if no_local else N)
        glob_b = base(gi, KG) if KG > 0 else []
        lact = []
        if not no_local:
            for g in range(N):
                nf = len(wins[P + g][0])
                a = hubs[g]["active"][:nf * KL].reshape(nf, KL).any(dim=1).tolist() \
                    if KL > 0 else [True] * nf
                lact.append([bool(x_) for x_ in a])
        tiles = M.cached_stream_tiles(
            device=dev, P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n,
            n_block=int(self.num_frame_per_block), local_attn=W,
            agent_frame_lists=[wins[p][0] for p in range(P)],
            local_frame_lists=[] if no_local else [wins[P + g][0] for g in range(N)],
            global_frame_list=wins[gi][0] if KG > 0 else [], local_active_frames=lact,
            labels=None if labels is None else labels.tolist(), q_active=act.tolist(),
            direct_player=bool(direct_player), tile_bases=(agent_b, local_b, glob_b),
            membership=None if mem is None else mem.numpy(),
            global_only=None if go is None else go.numpy(), hier_no_local_hub=no_local)
        out = torch.zeros((s, H, D), dtype=torch.bfloat16, device=dev)
        hier_attention_forward(q, kpool, vpool, tiles, out)
        return self.o(out.view(1, s, dim).to(self.o.weight.dtype))

    def causal_forward(self, x, freqs, mask=None, grid_sizes=None, seq_lens=None, kv_cache=None,
                       current_start=0, cache_start=None, num_frames=None, num_players=None,
                       num_hub_tokens=None, cam_tokens=None, group_labels=None, active_group=None,
                       direct_player=False, membership=None, global_only=None):
        """attention.py:1007-1043."""
        if kv_cache is not None and kv_cache.get("hier_hub", False):
            return self.causal_forward_hier_hub(
                x, freqs, kv_cache, current_start=current_start, num_frames=num_frames,
                num_players=num_players, num_hub_tokens=num_hub_tokens, cam_tokens=cam_tokens,
                group_labels=group_labels, active_group=active_group, direct_player=direct_player,
                membership=membership, global_only=global_only)
        raise ValueError("Hierarchical causal attention requires a hier KV cache")
