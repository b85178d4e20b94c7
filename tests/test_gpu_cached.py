"""Cached rollout on the GPU: paged KV cache + HIP forward against the cached
oracle (oracle/cached.py, pinned to the full-sequence mask), through the
drop-in module and through the reference-named cached backend call."""

import numpy as np
import pytest
import torch

from multics_amd import metadata as M
from multics_amd.kernels import (
    hier_attention_forward,
    hierarchical_paged_kv_attention,
    hierarchical_segmented_attention,
)
from multics_amd.kv_cache import (HierKVCachePipelineMixin, initialize_hier_kv_cache,
                                  stream_pool)
from multics_amd.module import SelfAttention
from multics_amd.paged_cache import HierPagedKVCache
from oracle.cached import HierCacheState, cached_block_forward
from tests.gpu_util import err_stats, need_gpu, say

pytestmark = pytest.mark.gpu
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def test_kv_append_scatters_rows():
    need_gpu()
    c = HierPagedKVCache(num_players=2, num_groups=2, num_patches=6, num_local_hub_tokens=2,
                         num_global_hub_tokens=3, num_heads=3, head_dim=64, local_attn_size=2,
                         num_frame_per_block=2, device="cuda")
    S = 2 * 2 * 6 + 2 * (2 * 2 + 3)
    g = torch.Generator(device="cuda").manual_seed(0)
    k = torch.randn(S, 3, 64, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(S, 3, 64, generator=g, device="cuda").to(torch.bfloat16)
    say("kv append")
    c.append(k, v, 5, 2, np.ones((2, 2), bool))
    torch.cuda.synchronize()
    rows = torch.from_numpy(c.block_rows(5, 2)).long().cuda()
    assert torch.equal(c.k[rows], k) and torch.equal(c.v[rows], v)
    other = torch.ones(c.k.shape[0], dtype=torch.bool, device="cuda")
    other[rows] = False
    assert torch.count_nonzero(c.k[other]) == 0


def _module(dim, H, seed):
    torch.manual_seed(seed)
    m = SelfAttention(dim, H, eps=1e-6)
    for lin in (m.q, m.k, m.v, m.o):
        torch.nn.init.normal_(lin.weight, std=0.05)
        torch.nn.init.zeros_(lin.bias)
    return m.to("cuda", torch.bfloat16).eval()


CASES = [
    # name, P, T, L, N, KL, KG, n, W, H, D, direct, kind
    ("labels_w3", 4, 9, 20, 2, 5, 6, 3, 3, 2, 128, True, "labels"),
    ("labels_w6_nodirect", 3, 12, 16, 2, 2, 3, 3, 6, 2, 64, False, "labels"),
    ("membership_w3", 4, 9, 12, 3, 2, 3, 3, 3, 2, 128, True, "membership"),
]


def _cache(store, P, N, L, KL, KG, H, D, W, n):
    """A layer's KV cache: the paged pool, the reference's cache dict over one
    pool (``kv_cache.initialize_hier_kv_cache``), or that dict with every
    stream buffer replaced by its own tensor, as the reference allocates them
    (read by concatenation)."""
    if store == "paged":
        return HierPagedKVCache(num_players=P, num_groups=N, num_patches=L,
                                num_local_hub_tokens=KL, num_global_hub_tokens=KG, num_heads=H,
                                head_dim=D, local_attn_size=W, num_frame_per_block=n,
                                device="cuda")
    entry = initialize_hier_kv_cache(
        num_layers=1, batch_size=1, dtype=torch.bfloat16, device="cuda", num_players=P,
        num_groups=N, num_local_hub_tokens=KL, num_global_hub_tokens=KG, frame_seq_length=L,
        local_attn_size=W, num_frame_per_block=n, num_heads=H, head_dim=D)[0]
    if store == "separate_dict":
        for c in list(entry["agent_caches"]) + list(entry["local_hubs"]) + [entry["global_hub"]]:
            c["k"], c["v"] = torch.zeros_like(c["k"]), torch.zeros_like(c["v"])
        assert stream_pool(entry) is None
    else:
        assert stream_pool(entry) is not None
    return entry


STORES = ["paged", "pooled_dict", "separate_dict"]


@pytest.mark.parametrize("store", STORES)
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_module_rollout_matches_cached_oracle(case, store):
    need_gpu()
    name, P, T, L, N, KL, KG, n, W, H, D, direct, kind = case
    dim = H * D
    m = _module(dim, H, seed=1)
    m.num_frame_per_block, m.local_attn_size = n, W
    rng = np.random.default_rng(2)
    cache = _cache(store, P, N, L, KL, KG, H, D, W, n)
    st = HierCacheState(P, N, L, KL, KG, H, D, W, n)
    if kind == "membership":
        mem = np.zeros((T, N, P), bool)
        go = np.zeros((T, P), bool)
        for b in range(T // n):
            mb = rng.random((N, P)) < 0.45
            mem[b * n:(b + 1) * n] = mb
            go[b * n:(b + 1) * n] = ~mb.any(0) & (rng.random(P) < 0.7)
    S = P * n * L + n * (N * KL + KG)
    g = torch.Generator().manual_seed(3)
    for b in range(T // n):
        kw = dict(direct_player=direct)
        okw = dict(n_block=n, direct=direct)
        if kind == "membership":
            kw.update(membership=torch.from_numpy(mem), global_only=torch.from_numpy(go))
            okw.update(membership=mem, global_only=go)
        else:
            lab = np.repeat(rng.integers(0, N, size=(1, P)), n, axis=0)
            act = np.zeros((n, N), bool)
            act[np.arange(n)[:, None], lab] = True
            kw.update(group_labels=torch.from_numpy(lab), active_group=torch.from_numpy(act))
            okw.update(labels=lab, active=act)
        ang = torch.rand(S, 1, D // 2, generator=g, dtype=torch.float64) * 6.283
        freqs = torch.polar(torch.ones_like(ang), ang)
        for step in range(2):       # two denoising passes over the block, then the next block
            x = torch.randn(1, S, dim, generator=g).to("cuda", torch.bfloat16)
            say(f"rollout {name} ({store}) block {b} step {step}")
            with torch.no_grad():
                y = m.causal_forward(x, freqs, kv_cache=cache, current_start=b * n * P * L,
                                     num_frames=n, num_players=P, **kw)
                q, k, v = m._project_self_attn_qkv(x, freqs)
            torch.cuda.synchronize()
            as3 = lambda t: t[0].view(S, H, D).float().cpu()
            att = cached_block_forward(st, as3(q), as3(k), as3(v), b * n, **okw)
            ref = torch.nn.functional.linear(att.reshape(1, S, dim), m.o.weight.float().cpu(),
                                             m.o.bias.float().cpu())
            mx, mn = err_stats(y, ref)
            say(f"  max-abs {mx:.3e} mean-abs {mn:.3e}")
            assert mx <= MAX_ABS and mn <= MEAN_ABS


def test_reference_cached_backend_call():
    """The plugin keyword call on per-stream windows taken from the oracle's caches."""
    need_gpu()
    P, T, L, N, KL, KG, n, W, H, D = 3, 6, 16, 2, 2, 3, 3, 3, 2, 128
    st = HierCacheState(P, N, L, KL, KG, H, D, W, n)
    rng = np.random.default_rng(5)
    g = torch.Generator().manual_seed(6)
    S = P * n * L + n * (N * KL + KG)
    for b in range(T // n):
        lab = np.repeat(rng.integers(0, N, size=(1, P)), n, axis=0)
        act = np.zeros((n, N), bool)
        act[np.arange(n)[:, None], lab] = True
        q, k, v = [(torch.randn(S, H, D, generator=g) * 0.5).to(torch.bfloat16).float()
                   for _ in range(3)]
        ref = cached_block_forward(st, q, k, v, b * n, n_block=n, direct=True, labels=lab,
                                   active=act)
        end = b * n + n - 1
        frames = lambda c, w: (end - c.local_end // w + 1 + torch.arange(c.local_end) // w).cuda()
        flat = lambda t: t.reshape(1, t.shape[0], H * D).to("cuda", torch.bfloat16)
        kw = dict(
            roped_q=q.to("cuda", torch.bfloat16)[None],
            agent_frames=[frames(c, L) for c in st.agent],
            agent_keys=[flat(c.k[:c.local_end]) for c in st.agent],
            agent_vals=[flat(c.v[:c.local_end]) for c in st.agent],
            local_frames=[frames(c, KL) for c in st.local],
            local_keys=[flat(c.k[:c.local_end]) for c in st.local],
            local_vals=[flat(c.v[:c.local_end]) for c in st.local],
            local_active_tokens=[c.active[:c.local_end].cuda() for c in st.local],
            global_frames=frames(st.glob, KG),
            global_keys=flat(st.glob.k[:st.glob.local_end]),
            global_vals=flat(st.glob.v[:st.glob.local_end]),
            labels=torch.from_numpy(lab).cuda(), active=torch.from_numpy(act).cuda(),
            P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n, n_block=n, local_attn=W, direct_player=True)
        say(f"plugin call block {b}")
        for fn in (hierarchical_segmented_attention, hierarchical_paged_kv_attention):
            y = fn(**kw)
            torch.cuda.synchronize()
            mx, mn = err_stats(y.reshape(S, H, D), ref)
            say(f"  {fn.__name__}: max-abs {mx:.3e} mean-abs {mn:.3e}")
            assert mx <= MAX_ABS and mn <= MEAN_ABS
    with pytest.raises(RuntimeError):
        kw["roped_q"] = kw["roped_q"].clone().requires_grad_(True)
        hierarchical_paged_kv_attention(**kw)


def test_cfg_batch_cache_matches_two_caches():
    """A batch-2 paged cache (the classifier-free-guidance prompt pair) in one
    launch over 2*H heads equals two caches of H heads: the pools and the
    attention outputs bit for bit, the module's outputs up to the
    o-projection's GEMM."""
    need_gpu()
    P, T, L, N, KL, KG, n, W, H, D = 4, 9, 12, 2, 2, 3, 3, 3, 2, 128
    dim = H * D
    m = _module(dim, H, seed=4)
    m.num_frame_per_block, m.local_attn_size = n, W
    kw = dict(num_players=P, num_groups=N, num_patches=L, num_local_hub_tokens=KL,
              num_global_hub_tokens=KG, num_heads=H, head_dim=D, local_attn_size=W,
              num_frame_per_block=n, device="cuda")
    both = HierPagedKVCache(batch=2, **kw)
    pair = [HierPagedKVCache(**kw) for _ in range(2)]
    rng = np.random.default_rng(8)
    S = P * n * L + n * (N * KL + KG)
    g = torch.Generator().manual_seed(9)
    for b in range(T // n):
        lab = np.repeat(rng.integers(0, N, size=(1, P)), n, axis=0)
        act = np.zeros((n, N), bool)
        act[np.arange(n)[:, None], lab] = True
        kw_b = dict(group_labels=torch.from_numpy(lab), active_group=torch.from_numpy(act),
                    direct_player=True, current_start=b * n * P * L, num_frames=n, num_players=P)
        ang = torch.rand(S, 1, D // 2, generator=g, dtype=torch.float64) * 6.283
        freqs = torch.polar(torch.ones_like(ang), ang)
        for step in range(2):
            x = torch.randn(2, S, dim, generator=g).to("cuda", torch.bfloat16)
            say(f"cfg batch block {b} step {step}")
            with torch.no_grad():
                y2 = m.causal_forward(x, freqs, kv_cache=both, **kw_b)
                ys = [m.causal_forward(x[i:i + 1], freqs, kv_cache=c, **kw_b)
                      for i, c in enumerate(pair)]
            torch.cuda.synchronize()
            for i in range(2):
                mx, mn = err_stats(y2[i:i + 1], ys[i])
                say(f"  member {i}: max-abs {mx:.3e} mean-abs {mn:.3e}")
                assert mx <= 1e-2 and mn <= 1e-4
    pools = both.k.view(both.k.shape[0], 2, H, D), both.v.view(both.v.shape[0], 2, H, D)
    for i, c in enumerate(pair):
        assert torch.equal(pools[0][:, i], c.k) and torch.equal(pools[1][:, i], c.v)
    # the attention launch itself: 2*H heads in one call == H heads per call
    frames, bases, lact = both.window(T - 1)
    tiles = M.cached_tiles(device="cuda", P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n, n_block=n,
                           local_attn=W, frames=frames, tile_bases=bases, local_active_frames=lact,
                           labels=lab.tolist(), q_active=act.tolist(), direct_player=True)
    q2 = torch.randn(S, 2 * H, D, generator=g).to("cuda", torch.bfloat16)
    out2 = torch.zeros_like(q2)
    hier_attention_forward(q2, both.k, both.v, tiles, out2)
    for i, c in enumerate(pair):
        o = torch.zeros(S, H, D, dtype=torch.bfloat16, device="cuda")
        hier_attention_forward(q2[:, i * H:(i + 1) * H].contiguous(), c.k, c.v, tiles, o)
        assert torch.equal(out2[:, i * H:(i + 1) * H], o)


def _rollout(m, cache, P, T, L, N, KL, KG, n, H, D, seed, passes=2):
    """Outputs of every (block, pass) of a labels rollout through ``cache``."""
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    S = P * n * L + n * (N * KL + KG)
    outs = []
    for b in range(T // n):
        lab = np.repeat(rng.integers(0, N, size=(1, P)), n, axis=0)
        act = np.zeros((n, N), bool)
        act[np.arange(n)[:, None], lab] = True
        ang = torch.rand(S, 1, D // 2, generator=g, dtype=torch.float64) * 6.283
        freqs = torch.polar(torch.ones_like(ang), ang)
        for _ in range(passes):
            x = torch.randn(1, S, H * D, generator=g).to("cuda", torch.bfloat16)
            with torch.inference_mode():
                outs.append(m.causal_forward(
                    x, freqs, kv_cache=cache, current_start=b * n * P * L, num_frames=n,
                    num_players=P, num_hub_tokens=N * KL + KG, group_labels=torch.from_numpy(lab),
                    active_group=torch.from_numpy(act), direct_player=True))
    torch.cuda.synchronize()
    return outs


def test_pooled_and_separate_dicts_agree_bit_for_bit():
    """The same rolling-buffer contents read in place from the pool or
    concatenated from separate tensors give identical outputs."""
    need_gpu()
    P, T, L, N, KL, KG, n, W, H, D = 4, 12, 20, 2, 5, 6, 3, 3, 2, 128
    m = _module(H * D, H, seed=4)
    m.num_frame_per_block, m.local_attn_size = n, W
    say("pooled vs separate cache dicts")
    a = _rollout(m, _cache("pooled_dict", P, N, L, KL, KG, H, D, W, n), P, T, L, N, KL, KG, n,
                 H, D, seed=9)
    b = _rollout(m, _cache("separate_dict", P, N, L, KL, KG, H, D, W, n), P, T, L, N, KL, KG, n,
                 H, D, seed=9)
    for i, (x, y) in enumerate(zip(a, b)):
        assert torch.equal(x, y), i


class _Blocks:
    def __init__(self, attn):
        self.self_attn = attn


class _Dit:
    def __init__(self, attn, N, KL, KG):
        self.blocks = [_Blocks(attn)]
        self.num_groups, self.num_local_hub_tokens, self.num_global_hub_tokens = N, KL, KG
        self.hier_no_local_hub = False


class _Pipe(HierKVCachePipelineMixin):
    """The attributes of WanVideoNPlayersPipeline that its cache methods read."""

    def __init__(self, attn, P, N, L, KL, KG, W, n):
        self.dit = _Dit(attn, N, KL, KG)
        self.num_players, self.frame_seq_length = P, L
        self.local_attn_size, self.num_frame_per_block = W, n
        self.num_transformer_blocks = 2
        self.torch_dtype = torch.bfloat16
        self.kv_cache1 = None
        self.crossattn_cache = None

    def _initialize_crossattn_cache(self, batch_size, dtype, device):
        self.crossattn_cache = [{"is_init": True} for _ in range(self.num_transformer_blocks)]


def test_pipeline_cache_methods_reset_and_reuse():
    """The drop-in pipeline methods: allocate for training, roll out, reset
    through init_kv_cache_for_training (detach + _reset_kv_cache), roll out
    again -- the second rollout equals the first bit for bit."""
    need_gpu()
    P, T, L, N, KL, KG, n, W, H, D = 3, 9, 16, 2, 2, 3, 3, 3, 2, 64
    m = _module(H * D, H, seed=5)
    m.num_frame_per_block, m.local_attn_size = n, W
    pipe = _Pipe(m, P, N, L, KL, KG, W, n)
    pipe.init_kv_cache_for_training(batch_size=P, device=torch.device("cuda"))
    assert len(pipe.kv_cache1) == 2 and pipe.crossattn_cache is not None
    say("pipeline cache methods: first rollout")
    first = _rollout(m, pipe.kv_cache1[0], P, T, L, N, KL, KG, n, H, D, seed=12)
    pipe.init_kv_cache_for_training(batch_size=P, device=torch.device("cuda"))
    assert all(not c["is_init"] for c in pipe.crossattn_cache)
    assert int(pipe.kv_cache1[0]["agent_caches"][0]["local_end_index"].item()) == 0
    assert stream_pool(pipe.kv_cache1[0]) is not None
    say("pipeline cache methods: second rollout")
    second = _rollout(m, pipe.kv_cache1[0], P, T, L, N, KL, KG, n, H, D, seed=12)
    for i, (x, y) in enumerate(zip(first, second)):
        assert torch.equal(x, y), i
