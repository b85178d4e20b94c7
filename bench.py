"""Benchmark: hierarchical-attention forward on one MI355X.

Workload (configuration C2, a "Wan2.2-5B-shaped layer"): 4 players x 42 latent
frames x 220 tokens, groups {0,1},{2,3} fixed, K_L=5 local and K_G=6 global hub
tokens per frame, n=3 frames per causal block, window W=21, 24 heads x 128,
bf16, q/k/v ~ 0.5 N(0,1) (synthetic).  One "step" is one full-sequence forward
of the hierarchical attention of one layer: all 14 temporal blocks in one
launch, Q/K/V already resident in HBM.  Metadata (topology build) is built
once before timing, like the reference's cached layouts; its device latency is
reported separately, as is the fused Q/K prologue.

Prints one JSON line (the driver contract).  ``--config p6|c3|p10|...`` makes
another full-sequence configuration the headline line.  Unless ``--no-suite``,
the line's ``extra.suite`` also carries, from the same run: the forward at 6, 8
and 10 players; the training step of configuration C5 (forward + backward +
membership STE, P=4, T=21, W=7); and the per-chunk latency of the cached
rollout of config C4 (10 players, chunks of 6 frames through the paged KV
cache, steady state of the denoising passes).
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 (256 CU x 2.4 GHz x 4096 FLOP/clk)
SEED = 20260813

CONFIGS = {
    # name: (P, T, L, N, KL, KG, n, W, H, D, grouping)
    "c2": (4, 42, 220, 2, 5, 6, 3, 21, 24, 128, "fixed"),
    "c2_w7": (4, 42, 220, 2, 5, 6, 3, 7, 24, 128, "fixed"),
    "p6": (6, 42, 220, 3, 5, 6, 3, 21, 24, 128, "pairs"),
    "c3": (8, 42, 220, 3, 5, 6, 3, 21, 24, 128, "dynamic"),
    "p10": (10, 42, 220, 4, 5, 6, 3, 21, 24, 128, "random_block"),
    "c5": (4, 21, 220, 2, 5, 6, 3, 7, 24, 128, "logits"),
    "c4": (10, 42, 220, 4, 5, 6, 3, 21, 24, 128, "random_block"),
}


def grouping(name, P, T, N, rng):
    """Synthetic topologies; returns (labels or None, membership or None, global_only or None)."""
    if name == "fixed":
        labels = np.array([[p // 2 for p in range(P)]] * T)
        return labels, None, None
    if name == "pairs":
        labels = np.array([[min(p // 2, N - 1) for p in range(P)]] * T)
        return labels, None, None
    if name == "dynamic":
        # 2D random walk, distance threshold 0.3, components of size >= 2 take
        # slots by (-size, min id); the rest are global-only.  Recomputed per frame.
        pos = rng.random((P, 2))
        mem = np.zeros((T, N, P), dtype=bool)
        go = np.zeros((T, P), dtype=bool)
        for t in range(T):
            pos = np.clip(pos + rng.normal(0, 0.05, pos.shape), 0, 1)
            d = np.linalg.norm(pos[:, None] - pos[None], axis=-1) < 0.3
            comp = -np.ones(P, dtype=int)
            c = 0
            for p in range(P):
                if comp[p] >= 0:
                    continue
                stack = [p]
                comp[p] = c
                while stack:
                    x = stack.pop()
                    for y in np.nonzero(d[x])[0]:
                        if comp[y] < 0:
                            comp[y] = c
                            stack.append(y)
                c += 1
            groups = [np.nonzero(comp == i)[0] for i in range(c)]
            groups = sorted([g for g in groups if len(g) >= 2], key=lambda g: (-len(g), g.min()))
            for slot, g in enumerate(groups[:N]):
                mem[t, slot, g] = True
            go[t] = ~mem[t].any(0)
        return None, mem, go
    if name == "logits":
        # soft membership logits ~ N(0,1) per (frame, group, player), constant
        # inside each 3-frame block; the hard membership is logits > 0
        lg = np.repeat(rng.standard_normal((T // 3, N, P)), 3, axis=0)[:T]
        mem = lg > 0
        return lg, mem, ~mem.any(1)
    if name == "random_block":
        mem = np.zeros((T, N, P), dtype=bool)
        for b in range(0, T, 3):
            g = rng.integers(3, N + 1)
            assign = rng.integers(0, g, size=P)
            for t in range(b, min(b + 3, T)):
                mem[t, assign, np.arange(P)] = True
        go = ~mem.any(1)
        return None, mem, go
    raise ValueError(name)


def build_case(cfg, device):
    from multics_amd import metadata as M
    P, T, L, N, KL, KG, n, W, H, D, grp = CONFIGS[cfg]
    rng = np.random.default_rng(SEED)
    first, mem, go = grouping(grp, P, T, N, rng)
    labels = None if grp == "logits" else first      # "logits": first = the soft logits
    topo = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W, direct=True,
                                    labels=labels, membership=mem, global_only=go)
    t0 = time.perf_counter()
    res = M.build(topo, device)
    torch.cuda.synchronize()
    host_build_s = time.perf_counter() - t0
    return topo, res.tiles, host_build_s, (first, mem, go)


def camera_tokens(P, T, L, K, dev, pos_scale=1.0):
    """Camera12 tokens ``[S, 12]`` bf16 of seeded per-frame poses: yaw ~
    U(-180, 180) deg, pitch ~ U(-30, 30) deg, position a random walk with
    N(0, 0.05) m steps; anchored at player 0 frame 0 (dataset.py:49-90,
    raw_inputs.py:250-273), broadcast to each frame's L tokens, zero rows for
    the K hub tokens per frame (blocks.py:108-148)."""
    from multics_amd.camera import build_camera_tokens, camera12_from_absolute_c2w, camera_to_world
    rng = np.random.default_rng(SEED + 1)
    pose = np.zeros((P, T, 5))
    pose[..., :3] = np.cumsum(rng.normal(0.0, 0.05, (P, T, 3)), axis=1)
    pose[..., 3] = rng.uniform(-180.0, 180.0, (P, T))
    pose[..., 4] = rng.uniform(-30.0, 30.0, (P, T))
    c12 = camera12_from_absolute_c2w(torch.from_numpy(camera_to_world(pose)), pos_scale)
    ref = torch.empty(1, 0, dtype=torch.bfloat16, device=dev)
    return build_camera_tokens(c12, T, L, P, ref, include_hub=True, num_hub_tokens=K)[0].contiguous()


def rope_tables(P, T, L, K, D, dev):
    """fp32 cos / sin ``[S, D/2]`` of the simplex 4D RoPE table of a full
    sequence (pool of 10 vertices, vertex id = player index, 11 x 20 patch
    grid; WanModel.build_self_attn_freqs_with_hub, wan_video_dit.py:338-359)."""
    from multics_amd import rope
    h, w = (11, 20) if L == 220 else (1, L)
    bands = rope.precompute_freqs_cis_4d_wan_rerope(D)
    verts = rope.build_simplex_vertices(10, rope.WAN_REROPE_SPLITS[1])
    freqs = rope.build_self_attn_freqs_with_hub(bands, verts, T, h, w, "cpu", list(range(P)), K)
    return rope.freqs_to_cos_sin(freqs, device=dev)


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), else the machine type."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def profiled_traffic(cfg):
    """HBM bytes per launch of the forward kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of the same workload (counter values scaled
    by the copy-kernel calibration recorded with them), or None."""
    f = ROOT / "profiles" / f"attn_fwd_{cfg}.json"
    if not f.exists():
        return None
    d = json.loads(f.read_text())
    return int(d["traffic_bytes_per_launch"])


def time_events(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(steps):
        start.record()
        fn()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end))
    return times


def cpu_baseline(cfg, topo_args, budget_s=20.0):
    """The oracle's masked-SDPA restatement (dense bool mask + fp32 SDPA) on a
    bounded sample of (temporal block, head) pairs, extrapolated to the layer."""
    from oracle.masks import FullTopology, mask_rows
    P, T, L, N, KL, KG, n, W, H, D, _ = CONFIGS[cfg]
    labels, mem, go = topo_args
    ft = FullTopology(P, T, L, N, KL, KG, n, W, True, labels=labels, membership=mem, global_only=go)
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    S = ft.S
    g = torch.Generator().manual_seed(SEED)
    b = min(7, T // n - 1)                       # a steady-state block
    frames = range(b * n, b * n + n)
    local_start, global_start = P * T * L, P * T * L + T * N * KL
    rows = [(p * T + f) * L + i for p in range(P) for f in frames for i in range(L)]
    rows += [local_start + (f * N + gg) * KL + i for f in frames for gg in range(N) for i in range(KL)]
    rows += [global_start + f * KG + i for f in frames for i in range(KG)]
    rows = np.array(rows)
    mask = torch.zeros(len(rows), S, dtype=torch.bool)
    for r0 in range(0, len(rows), 256):
        mask[r0:r0 + 256] = torch.from_numpy(mask_rows(ft, q_idx=rows[r0:r0 + 256]))
    q = torch.randn(1, 1, len(rows), D, generator=g) * 0.5
    k = torch.randn(1, 1, S, D, generator=g) * 0.5
    v = torch.randn(1, 1, S, D, generator=g) * 0.5
    done, t_sum = 0, 0.0
    while done < H and (done == 0 or t_sum < budget_s):
        t0 = time.perf_counter()
        torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask[None, None])
        t_sum += time.perf_counter() - t0
        done += 1
    per_block_head = t_sum / done
    ms_layer = per_block_head * (T // n) * H * 1e3
    return dict(ms_layer=ms_layer, sample=f"{done} head(s) of temporal block {b} of {T // n} "
                f"({len(rows)} query rows x {S} keys, dense mask SDPA fp32), extrapolated x"
                f"{(T // n) * H / done:.0f}", cores=cores, threads=torch.get_num_threads(),
                cpu=cpu_model())


def bench_forward_cfg(cfg, dev, steps=10, warmup=3):
    """Full-sequence forward of another configuration: ms and useful TFLOP/s."""
    from multics_amd.kernels import hier_attention_forward
    P, T, L, N, KL, KG, n, W, H, D, grp = CONFIGS[cfg]
    topo, tiles, _, _ = build_case(cfg, dev)
    S = P * T * L + T * (N * KL + KG)
    g = torch.Generator(device=dev).manual_seed(SEED)
    q, k, v = ((torch.randn(H, S, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
               .permute(1, 0, 2) for _ in range(3))
    out = torch.empty(S, H, D, dtype=torch.bfloat16, device=dev)
    ms = float(np.median(time_events(lambda: hier_attention_forward(q, k, v, tiles, out),
                                     steps, warmup)))
    flop = 4.0 * H * D * tiles.logical_pairs
    del q, k, v, out
    return {"players": P, "tokens": S, "window": W, "ms_per_layer": round(ms, 4),
            "useful_tflops": round(flop / (ms * 1e-3) / 1e12, 2),
            "frac_peak": round(flop / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "grouping": grp}


def bench_training(dev, steps=10, warmup=3):
    """Config C5: forward + backward + membership STE of one attention layer."""
    from multics_amd.kernels import hier_attention
    P, T, L, N, KL, KG, n, W, H, D, grp = CONFIGS["c5"]
    topo, tiles, _, (logits, mem, go) = build_case("c5", dev)
    S = P * T * L + T * (N * KL + KG)
    g = torch.Generator(device=dev).manual_seed(SEED)
    mk = lambda: (torch.randn(H, S, D, generator=g, device=dev) * 0.5).to(torch.bfloat16) \
        .permute(1, 0, 2).contiguous().requires_grad_(True)
    q, k, v = mk(), mk(), mk()
    dout = torch.randn(S, H, D, generator=g, device=dev).to(torch.bfloat16)
    lg = torch.from_numpy(logits).float().to(dev).requires_grad_(True)
    geo = (P, T, L, N, KL)

    def fwd():
        return hier_attention(q, k, v, tiles, membership_logits=lg, ste_geometry=geo)

    def step():
        q.grad = k.grad = v.grad = lg.grad = None
        fwd().backward(dout)

    from multics_amd import metadata as M
    plan = M.MembershipLogitsPlan(device=dev, P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                  direct=True)

    def rebuild():
        """The lists of the current logits rebuilt on the device with no
        host read-back (``MembershipLogitsPlan``): membership from the
        logits, the tile-list pass, both key-major passes, the STE classes."""
        t_ = plan.build(lg)
        M.launch_ste_first(t_, geo)
        return t_

    def rebuild_host():
        """The same lists through the host topology: membership read back,
        both metadata passes (count read-back), both key-major passes (totals
        read-back), the STE classes."""
        m = (lg.detach() > 0).cpu().numpy()
        t_ = M.build(M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                              direct=True, membership=m, global_only=~m.any(1)),
                     dev).tiles
        M.backward_lists(t_, None)
        M.launch_ste_first(t_, geo)
        return t_

    def step_rebuild():
        t_ = rebuild()
        q.grad = k.grad = v.grad = lg.grad = None
        hier_attention(q, k, v, t_, membership_logits=lg, ste_geometry=geo).backward(dout)

    t_plan = rebuild()

    def step_plan():
        """A step over the plan's lists built once: the same lists as a
        rebuilding step (the plan folds no tails into the hubs' items),
        without the rebuild."""
        q.grad = k.grad = v.grad = lg.grad = None
        hier_attention(q, k, v, t_plan, membership_logits=lg, ste_geometry=geo).backward(dout)

    ms_fwd = float(np.median(time_events(lambda: fwd(), steps, warmup)))
    ms_step = float(np.median(time_events(step, steps, warmup)))
    ms_meta = float(np.median(time_events(rebuild, steps, warmup)))
    ms_meta_host = float(np.median(time_events(rebuild_host, steps, warmup)))
    ms_step_rebuild = float(np.median(time_events(step_rebuild, steps, warmup)))
    ms_step_plan = float(np.median(time_events(step_plan, steps, warmup)))
    E = tiles.logical_pairs
    flop_f, flop_b = 4.0 * H * D * E, 10.0 * H * D * E
    ms_bwd = ms_step - ms_fwd
    return {"players": P, "frames": T, "window": W, "tokens": S, "useful_pairs": E,
            "ms_fwd": round(ms_fwd, 4), "ms_fwd_bwd": round(ms_step, 4),
            "ms_bwd": round(ms_bwd, 4),
            "ms_metadata_rebuild": round(ms_meta, 4),
            "ms_metadata_rebuild_host": round(ms_meta_host, 4),
            "ms_fwd_bwd_with_rebuild": round(ms_step_rebuild, 4),
            "ms_fwd_bwd_plan_lists": round(ms_step_plan, 4),
            "useful_tflops_fwd_bwd": round((flop_f + flop_b) / (ms_step * 1e-3) / 1e12, 2),
            "useful_tflops_bwd": round(flop_b / (ms_bwd * 1e-3) / 1e12, 2),
            "note": "bwd = dQ (query-major, with the membership STE sums) + dK/dV (key-major); "
                    "useful FLOP 4*H*D*E fwd, 10*H*D*E bwd; *_rebuild: every step rebuilds "
                    "the forward and key-major lists and the STE classes from the logits on "
                    "the device with no host read-back (MembershipLogitsPlan), as a step "
                    "whose logits flipped membership must; ms_fwd_bwd_plan_lists: a step over "
                    "those lists built once (they fold no player tails into the hubs' items, "
                    "unlike the lists of ms_fwd_bwd), so with_rebuild - plan_lists is the "
                    "rebuild's own cost; ms_metadata_rebuild_host: the same lists through the "
                    "host topology (membership, count and totals read back)"}


def bench_module_training(dev, steps=10, warmup=3):
    """Config C5 through the drop-in module under autograd: one training step
    (forward + backward) of ``SelfAttention.forward_hier_membership`` with
    soft membership logits and the camera adapter -- the q / k / v GEMMs, the
    HIP projection tail (camera, RMSNorm, gain, RoPE) forward and backward,
    the lists of the current logits rebuilt on the device, the HIP attention
    forward and backward with the membership STE, the o-projection.  Beside
    it the same step with the reference's torch projection tail
    (attention.py:355-365: fp32 RMSNorm, float64 RoPE) in place of the HIP
    one.  Random bf16 weights, x ~ 0.5 N(0,1), dy ~ N(0,1)."""
    from multics_amd.kernels import hier_attention
    from multics_amd.module import SelfAttention
    from multics_amd import metadata as M
    from multics_amd import rope
    P, T, L, N, KL, KG, n, W, H, D, grp = CONFIGS["c5"]
    dim = H * D
    logits, _, _ = grouping(grp, P, T, N, np.random.default_rng(SEED))
    torch.manual_seed(SEED)
    m = SelfAttention(dim, H).to(device=dev, dtype=torch.bfloat16).train()
    m.num_frame_per_block, m.local_attn_size = n, W
    m.enable_camera_pose_qk(12, dropout_p=0.0)
    with torch.no_grad():
        for lin in (m.q, m.k, m.v, m.o):
            lin.weight.normal_(0.0, 0.02)
        m.cam_q.weight.normal_(0.0, 0.02)
        m.cam_k.weight.normal_(0.0, 0.02)
    S = P * T * L + T * (N * KL + KG)
    h, w = (11, 20) if L == 220 else (1, L)
    bands = rope.precompute_freqs_cis_4d_wan_rerope(D)
    verts = rope.build_simplex_vertices(10, rope.WAN_REROPE_SPLITS[1])
    freqs = rope.build_self_attn_freqs_with_hub(bands, verts, T, h, w, "cpu", list(range(P)),
                                                N * KL + KG).to(dev)
    cam = camera_tokens(P, T, L, N * KL + KG, dev)[None]
    g = torch.Generator(device=dev).manual_seed(SEED)
    x = (torch.randn(1, S, dim, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    dy = torch.randn(1, S, dim, generator=g, device=dev).to(torch.bfloat16)
    lg = torch.from_numpy(logits).float().to(dev).requires_grad_(True)
    kw = dict(num_players=P, num_frames=T, num_patches=L, num_groups=N, num_local_hub_tokens=KL,
              num_global_hub_tokens=KG, direct_player=True, membership_logits=lg, cam_tokens=cam)

    def step_hip():
        m.zero_grad(set_to_none=True)
        lg.grad = None
        m.forward_hier_membership(x, freqs, **kw).backward(dy)

    def step_torch_tail():
        m.zero_grad(set_to_none=True)
        lg.grad = None
        tiles = M.membership_logits_tiles(lg, P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                          direct=True)
        q, k, v = (t.view(S, H, D) for t in m._project_self_attn_qkv(x, freqs, cam))
        y = hier_attention(q, k, v, tiles, membership_logits=lg, ste_geometry=(P, T, L, N, KL))
        m.o(y.reshape(1, S, dim)).backward(dy)

    ms_hip = float(np.median(time_events(step_hip, steps, warmup)))
    ms_torch = float(np.median(time_events(step_torch_tail, steps, warmup)))
    return {"tokens": S, "dim": dim, "ms_step": round(ms_hip, 4),
            "ms_step_torch_tail": round(ms_torch, 4),
            "note": "module training step (fwd + bwd): GEMMs, projection tail (HIP fwd + bwd), "
                    "lists rebuilt from the logits on the device, attention with membership "
                    "STE, o-projection; ms_step_torch_tail: the same step with the reference's "
                    "torch projection tail"}


def bench_layer(dev, steps=10, warmup=3):
    """C2 through the drop-in module: ``SelfAttention.forward(x, freqs, mask,
    cam_tokens)`` (attention.py:436-442 signature) under no_grad, with the
    block mask of ``build_stage2_hier_flex_block_mask``: the q / k / v GEMMs,
    the fused camera + RMSNorm + RoPE prologue on q and k, the attention
    (V read in place from the v projection) and the o-projection.  Random
    bf16 weights, camera adapter on (random weights, no dropout), camera12 of
    seeded poses, the simplex RoPE table.  The GEMMs are also timed alone on
    the same shapes."""
    import torch.nn.functional as F
    from multics_amd import rope
    from multics_amd.hier_masks import build_stage2_hier_flex_block_mask
    from multics_amd.module import SelfAttention
    P, T, L, N, KL, KG, n, W, H, D, grp = CONFIGS["c2"]
    dim = H * D
    labels, _, _ = grouping(grp, P, T, N, np.random.default_rng(SEED))
    torch.manual_seed(SEED)
    layer = SelfAttention(dim, H).to(device=dev, dtype=torch.bfloat16).eval()
    layer.num_frame_per_block, layer.local_attn_size = n, W
    layer.enable_camera_pose_qk(12, dropout_p=0.0)
    with torch.no_grad():
        layer.cam_q.weight.normal_(0.0, 0.02)
        layer.cam_k.weight.normal_(0.0, 0.02)
    lab = torch.from_numpy(np.asarray(labels)).long()
    mask, S, _ = build_stage2_hier_flex_block_mask(P, T, L, N, KL, KG, n, W, lab, None, True, dev)
    h, w = (11, 20) if L == 220 else (1, L)
    bands = rope.precompute_freqs_cis_4d_wan_rerope(D)
    verts = rope.build_simplex_vertices(10, rope.WAN_REROPE_SPLITS[1])
    freqs = rope.build_self_attn_freqs_with_hub(bands, verts, T, h, w, "cpu", list(range(P)),
                                                N * KL + KG).to(dev)
    cam = camera_tokens(P, T, L, N * KL + KG, dev)[None]
    x = torch.randn(1, S, dim, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        ms_layer = float(np.median(time_events(lambda: layer(x, freqs, mask, cam_tokens=cam),
                                               steps, warmup)))

        def gemms():
            for lin in (layer.q, layer.k, layer.v, layer.o):
                F.linear(x, lin.weight, lin.bias)

        ms_gemm = float(np.median(time_events(gemms, steps, warmup)))
    E = mask.tiles.logical_pairs
    flop_gemm = 8.0 * S * dim * dim
    flop_attn = 4.0 * H * D * E
    return {"tokens": S, "dim": dim, "ms_layer": round(ms_layer, 4),
            "ms_gemms_qkvo": round(ms_gemm, 4),
            "ms_rest": round(ms_layer - ms_gemm, 4),
            "tflops_layer": round((flop_gemm + flop_attn) / (ms_layer * 1e-3) / 1e12, 1),
            "note": "module forward under no_grad (GEMMs + fused q/k prologue + attention + "
                    "o-projection); ms_rest = layer - the four GEMMs alone (prologue, "
                    "attention, the cos/sin table, the output buffer); GEMM FLOP 8*S*dim^2"}


def bench_block_tail(dev, steps=10, warmup=3):
    """C2 after the attention: the o-projection and the gated residual of the
    DiT block, x = x + gate_msa * o(attn) (blocks.py:604-616, 661-668), for
    the 4 x 9,240 player rows.  torch: the gate expanded per frame to every
    token (as the block builds it) and the bf16 expression (two passes);
    HIP: ``gated_residual`` reading the compact [P, T, dim] gate in one pass.
    Both after the same hipBLASLt GEMM; outputs compared bit for bit."""
    import torch.nn.functional as F
    from multics_amd.kernels import gated_residual
    P, T, L, N, KL, KG, n, W, H, D, grp = CONFIGS["c2"]
    dim = H * D
    g = torch.Generator(device=dev).manual_seed(SEED + 3)
    rnd = lambda *s: torch.randn(*s, generator=g, device=dev).to(torch.bfloat16)
    attn, x = rnd(P * T * L, dim), rnd(P, T * L, dim)
    w_o, b_o = rnd(dim, dim) * 0.02, rnd(dim)
    gate = rnd(P, T, dim)

    def oproj():
        return F.linear(attn, w_o, b_o).view(P, T * L, dim)

    def torch_tail(y):
        full = gate.unsqueeze(2).expand(-1, -1, L, -1).reshape(P, T * L, dim)
        return x + full * y

    y = oproj()
    same = bool(torch.equal(torch_tail(y), gated_residual(x, gate, y)))
    ms = {}
    for name, fn in (("gemm", oproj), ("torch_gate", lambda: torch_tail(y)),
                     ("hip_gate", lambda: gated_residual(x, gate, y)),
                     ("gemm_torch_gate", lambda: torch_tail(oproj())),
                     ("gemm_hip_gate", lambda: gated_residual(x, gate, oproj()))):
        ms[name] = float(np.median(time_events(fn, steps, warmup)))
    hbm = 3 * x.numel() * 2
    return {"rows": P * T * L, "dim": dim, "bit_identical": same,
            **{f"ms_{k}": round(v, 4) for k, v in ms.items()},
            "hip_gate_gbs": round(hbm / (ms["hip_gate"] * 1e-3) / 1e9, 1),
            "note": "o-projection (hipBLASLt) + gated residual x + gate_msa * y; the HIP pass "
                    "reads x, y and the compact per-frame gate once and writes once "
                    "(hip_gate_gbs over 3 x rows x dim x 2 B)"}


def bench_rollout(dev, passes=10):
    """Config C4: cached rollout, 10 players, chunk = 6 latent frames = 2 blocks
    of 3 through the paged KV cache; time one denoising pass over a chunk in
    the steady state (window full, metadata cached)."""
    from multics_amd import metadata as M
    from multics_amd.kernels import hier_attention_forward
    from multics_amd.paged_cache import HierPagedKVCache
    P, T, L, N, KL, KG, n, W, H, D, grp = CONFIGS["c4"]
    rng = np.random.default_rng(SEED)
    _, mem, go = grouping(grp, P, T, N, rng)
    act_full = mem.any(-1)
    cache = HierPagedKVCache(num_players=P, num_groups=N, num_patches=L, num_local_hub_tokens=KL,
                             num_global_hub_tokens=KG, num_heads=H, head_dim=D, local_attn_size=W,
                             num_frame_per_block=n, device=dev)
    S = P * n * L + n * (N * KL + KG)
    g = torch.Generator(device=dev).manual_seed(SEED)
    q, k, v = ((torch.randn(S, H, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
               for _ in range(3))
    out = torch.empty(S, H, D, dtype=torch.bfloat16, device=dev)

    def block_tiles(b):
        frames, bases, lact = cache.window(b * n + n - 1)
        return M.cached_tiles(device=dev, P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n, n_block=n,
                              local_attn=W, frames=frames, tile_bases=bases,
                              local_active_frames=lact, labels=None,
                              q_active=act_full[b * n:b * n + n].tolist(), direct_player=True,
                              membership=mem, global_only=go)

    first = (W + n) // n                     # blocks that fill the window
    for b in range(first):
        cache.append(k, v, b * n, n, act_full[b * n:b * n + n])
    chunk = [first, first + 1]
    t0 = time.perf_counter()
    tl = {}
    for b in chunk:
        cache.append(k, v, b * n, n, act_full[b * n:b * n + n])
        tl[b] = block_tiles(b)
    torch.cuda.synchronize()
    meta_ms = (time.perf_counter() - t0) * 1e3 / len(chunk)

    def one_pass():
        for b in chunk:
            cache.append(k, v, b * n, n, act_full[b * n:b * n + n])
            hier_attention_forward(q, cache.k, cache.v, tl[b], out)

    ms = float(np.median(time_events(one_pass, passes, 3)))
    pairs = sum(tl[b].logical_pairs for b in chunk)
    return {"players": P, "chunk_frames": 2 * n, "query_rows": 2 * S,
            "cached_frames_per_stream": cache.R, "ms_per_chunk": round(ms, 4),
            "useful_tflops": round(4.0 * H * D * pairs / (ms * 1e-3) / 1e12, 2),
            "first_pass_metadata_ms_per_block": round(meta_ms, 2),
            "note": "per denoising pass: paged append + HIP forward for 2 blocks; metadata "
                    "is built on a block's first pass and reused by its later passes"}


def bench_rollout_cfg(dev, passes=10):
    """Config C4 with classifier-free guidance: the positive and negative
    prompt caches (wan_video_Nplayers.py:645-648, two model calls per block
    at :739-776) as one batch-2 paged cache, so each block is one append and
    one attention launch over 2*H heads; against two caches of H heads and
    two launches per block.  Same steady state as ``bench_rollout``."""
    from multics_amd import metadata as M
    from multics_amd.kernels import hier_attention_forward
    from multics_amd.paged_cache import HierPagedKVCache
    P, T, L, N, KL, KG, n, W, H, D, grp = CONFIGS["c4"]
    rng = np.random.default_rng(SEED)
    _, mem, go = grouping(grp, P, T, N, rng)
    act_full = mem.any(-1)
    S = P * n * L + n * (N * KL + KG)
    g = torch.Generator(device=dev).manual_seed(SEED)
    q2, k2, v2 = ((torch.randn(S, 2 * H, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
                  for _ in range(3))
    halves = [tuple(t[:, i * H:(i + 1) * H].contiguous() for t in (q2, k2, v2)) for i in range(2)]
    kw = dict(num_players=P, num_groups=N, num_patches=L, num_local_hub_tokens=KL,
              num_global_hub_tokens=KG, num_heads=H, head_dim=D, local_attn_size=W,
              num_frame_per_block=n, device=dev)
    both = HierPagedKVCache(batch=2, **kw)
    pair = [HierPagedKVCache(**kw) for _ in range(2)]
    first = (W + n) // n
    chunk = [first, first + 1]
    tl = {}
    for b in range(first + 2):
        a = act_full[b * n:b * n + n]
        both.append(k2, v2, b * n, n, a)
        for c, (_, kh, vh) in zip(pair, halves):
            c.append(kh, vh, b * n, n, a)
        if b in chunk:
            frames, bases, lact = both.window(b * n + n - 1)
            tl[b] = M.cached_tiles(device=dev, P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n, n_block=n,
                                   local_attn=W, frames=frames, tile_bases=bases,
                                   local_active_frames=lact, labels=None,
                                   q_active=act_full[b * n:b * n + n].tolist(),
                                   direct_player=True, membership=mem, global_only=go)
    out2 = torch.empty(S, 2 * H, D, dtype=torch.bfloat16, device=dev)
    outs = [torch.empty(S, H, D, dtype=torch.bfloat16, device=dev) for _ in range(2)]

    def batched():
        for b in chunk:
            both.append(k2, v2, b * n, n, act_full[b * n:b * n + n])
            hier_attention_forward(q2, both.k, both.v, tl[b], out2)

    def two_calls():
        for b in chunk:
            for c, (qh, kh, vh), o in zip(pair, halves, outs):
                c.append(kh, vh, b * n, n, act_full[b * n:b * n + n])
                hier_attention_forward(qh, c.k, c.v, tl[b], o)

    ms_b = float(np.median(time_events(batched, passes, 3)))
    ms_2 = float(np.median(time_events(two_calls, passes, 3)))
    pairs = 2 * sum(tl[b].logical_pairs for b in chunk)
    return {"players": P, "chunk_frames": 2 * n, "prompts": 2,
            "ms_per_chunk_batched": round(ms_b, 4), "ms_per_chunk_two_calls": round(ms_2, 4),
            "useful_tflops_batched": round(4.0 * H * D * pairs / (ms_b * 1e-3) / 1e12, 2),
            "note": "CFG pair as one batch-2 paged cache (2*H heads per launch) vs two caches"}


def bench_action_temporal(dev, passes=20):
    """The mouse branch's cached temporal attention at C4 scale
    (blocks.py:256-308): one sequence per spatial token of every player
    (P*L = 2,200), the block's 3 frames attending to the cached window of
    W + n = 24 frames, 24 heads of 128.  HIP frame-window attention against
    the reference's ``F.scaled_dot_product_attention(attn_mask=...)`` on the
    same GPU; HBM-bound on reading the window once."""
    from multics_amd.action import frame_attention
    P, T, L, N, KL, KG, n, W, H, D, grp = CONFIGS["c4"]
    B, f, win = P * L, n, W + n
    g = torch.Generator(device=dev).manual_seed(SEED)
    q = (torch.randn(B, f, H, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    k = (torch.randn(B, win, H, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    v = torch.randn(B, win, H, D, generator=g, device=dev).to(torch.bfloat16)
    start = 2 * W                                     # a steady-state block: window full
    qf = torch.arange(start, start + f)
    kf = torch.arange(start + f - win, start + f)
    qf_d, kf_d = qf.to(torch.int32).to(dev), kf.to(torch.int32).to(dev)
    mask = ((kf[None, :] // n) <= (qf[:, None] // n)) & ((qf[:, None] - kf[None, :]) < W)
    mask = mask.to(dev)
    qt, kt, vt = (t.transpose(1, 2) for t in (q, k, v))
    ms_hip = float(np.median(time_events(lambda: frame_attention(q, k, v, qf_d, kf_d, n, W),
                                         passes, 3)))
    ms_sdpa = float(np.median(time_events(
        lambda: torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask),
        passes, 3)))
    got = frame_attention(q, k, v, qf_d, kf_d, n, W).float()
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask)
    diff = (got - ref.transpose(1, 2).float()).abs().max().item()
    bytes_ = 2 * (2 * B * win * H * D + 2 * B * f * H * D)
    return {"sequences": B, "queries_per_seq": f, "window_frames": win, "heads": H, "head_dim": D,
            "ms_hip": round(ms_hip, 4), "ms_torch_sdpa": round(ms_sdpa, 4),
            "hbm_gb_per_call": round(bytes_ / 1e9, 3),
            "achieved_gbs": round(bytes_ / (ms_hip * 1e-3) / 1e9, 1),
            "frac_hbm": round(bytes_ / (ms_hip * 1e-3) / 8e12, 4),
            "max_abs_vs_sdpa": round(diff, 5)}


# the suite of the default run, in its order: name -> fn(dev[, steps, warmup])
SUITES = {
    "fwd_c2_w7": lambda dev, *a: bench_forward_cfg("c2_w7", dev, *a),
    "fwd_p6": lambda dev, *a: bench_forward_cfg("p6", dev, *a),
    "fwd_c3": lambda dev, *a: bench_forward_cfg("c3", dev, *a),
    "fwd_p10": lambda dev, *a: bench_forward_cfg("p10", dev, *a),
    "layer_c2": bench_layer,
    "block_tail_c2": bench_block_tail,
    "training_c5": bench_training,
    "module_training_c5": bench_module_training,
    "rollout_c4": lambda dev, *a: bench_rollout(dev, *a[:1]),
    "rollout_c4_cfg": lambda dev, *a: bench_rollout_cfg(dev, *a[:1]),
    "action_temporal_c4": lambda dev, *a: bench_action_temporal(dev, *a[:1]),
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--no-suite", action="store_true",
                    help="skip the other configurations (6/8/10 players, training, rollout)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run one 256 MiB device copy (HBM counter calibration)")
    ap.add_argument("--only", choices=sorted(SUITES),
                    help="run one entry of the suite alone and print its line (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the hierarchical attention of one layer shards by "
              "head or temporal block with no exchange inside the kernel; "
              "multi-GPU runs are not part of this build.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from multics_amd.kernels import hier_attention_forward, qkv_prologue
    dev = torch.device("cuda", 0)
    if args.only:
        res = SUITES[args.only](dev, max(args.steps, 1), args.warmup)
        print(json.dumps({"suite": args.only, **res}), flush=True)
        return
    P, T, L, N, KL, KG, n, W, H, D, grp = CONFIGS[args.config]
    topo, tiles, host_build_s, topo_args = build_case(args.config, dev)
    S = P * T * L + T * (N * KL + KG)

    # metadata builder latency (device passes + the count readback)
    from multics_amd import metadata as M
    meta_ms = []
    for _ in range(5):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        M.build(topo, dev)
        torch.cuda.synchronize()
        meta_ms.append((time.perf_counter() - t0) * 1e3)

    g = torch.Generator(device=dev).manual_seed(SEED)
    mk = lambda: (torch.randn(H, S, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    # the layout the module's no-grad path feeds the kernel: q / k head-major
    # (the prologue's [H, S, D] storage as [S, H, D] views), v token-major
    # (the v projection, read in place)
    q, k = (mk().permute(1, 0, 2) for _ in range(2))
    v = mk().permute(1, 0, 2).contiguous()
    out = torch.empty(S, H, D, dtype=torch.bfloat16, device=dev)

    def step():
        hier_attention_forward(q, k, v, tiles, out)

    times = time_events(step, args.steps, args.warmup)
    ms = float(np.median(times))
    ms_mean = float(np.mean(times))
    useful_flop = 4.0 * H * D * tiles.logical_pairs
    tflops = useful_flop / (ms * 1e-3) / 1e12

    # fused Q/K prologue (camera + RMSNorm + RoPE) on the same sequence: camera12
    # tokens of seeded poses and the simplex 4D RoPE table of the layout
    dim = H * D
    qx = (torch.randn(S, dim, generator=g, device=dev)).to(torch.bfloat16)
    kx = (torch.randn(S, dim, generator=g, device=dev)).to(torch.bfloat16)
    cam = camera_tokens(P, T, L, N * KL + KG, dev)
    wcq = (0.02 * torch.randn(dim, 12, generator=g, device=dev)).to(torch.bfloat16)
    wck = (0.02 * torch.randn(dim, 12, generator=g, device=dev)).to(torch.bfloat16)
    nw = torch.ones(dim, dtype=torch.bfloat16, device=dev)
    cs, sn = rope_tables(P, T, L, N * KL + KG, D, dev)
    pro = time_events(lambda: qkv_prologue(qx, kx, None, norm_q_w=nw, norm_k_w=nw, rope_cos=cs,
                                           rope_sin=sn, num_heads=H, eps=1e-6, cam=cam,
                                           w_cam_q=wcq, w_cam_k=wck, out_layout="hsd"),
                      max(args.steps // 5, 3), 2)
    pro_ms = float(np.median(pro))

    if args.calib_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()

    cpu = None
    if not args.no_cpu_baseline:
        cb = cpu_baseline(args.config, topo_args, args.cpu_budget)
        cpu = {"value": round(useful_flop / (cb["ms_layer"] * 1e-3) / 1e12, 6),
               "unit": "TFLOP/s (useful)", "ms_per_layer": round(cb["ms_layer"], 1),
               "cores": cb["cores"], "threads": cb["threads"], "kind": "port",
               "cpu": cb["cpu"], "sample": cb["sample"]}

    line = {
        "metric": "hier-attn useful TFLOP/s + ms/layer fwd (bf16, 4 and 10 players, 1 GPU)",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "ms_per_step_mean": round(ms_mean, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (q/k/v ~ 0.5 N(0,1), seeded)",
        "config": {"workload": f"{args.config}: full-sequence hierarchical attention fwd, P={P} "
                   f"T={T} L={L} N={N} K_L={KL} K_G={KG} n={n} W={W} H={H} D={D} ({grp} groups)",
                   "players": P, "tokens": S, "useful_pairs": tiles.logical_pairs,
                   "useful_gflop": round(useful_flop / 1e9, 1), "seed": SEED},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": profiled_traffic(args.config)},
        "cpu_baseline": cpu,
        "extra": {"metadata_build_ms": round(float(np.median(meta_ms)), 3),
                  "prologue_ms": round(pro_ms, 4), "work_items": (tiles.fwd_n_items or tiles.n_items) * H},
    }
    if not args.no_suite:
        suite = {}
        for name, fn in SUITES.items():
            if name != f"fwd_{args.config}":
                suite[name] = fn(dev)
        line["extra"]["suite"] = suite
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
