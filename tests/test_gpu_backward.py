"""HIP backward (dQ, dK, dV) against fp32 autograd of the dense-mask oracle.

The reference differentiates its training forward through FlexAttention on the
dense hierarchical mask (attention.py:322-353, 367-434); the oracle here is the
same function -- softmax(QK^T / sqrt(D) + mask) V with inactive local-hub rows
multiplied by 0 -- in fp32 torch autograd on the CPU, from the same bf16
inputs.  Gradients are bf16 and meet both the north-star bound, max-abs <=
2e-2 and mean-abs <= 2e-3 against the fp32 reference, and a bound relative to
the gradient's size: max-abs <= 2e-2 * max|ref| and mean-abs <= 1e-2 *
mean|ref|.
"""

import math

import numpy as np
import pytest
import torch

from multics_amd import metadata as M
from multics_amd.kernels import hier_attention, hier_attention_backward, hier_attention_forward
from oracle.attention import masked_attention
from oracle.masks import FullTopology
from tests.gpu_util import need_gpu, say

pytestmark = pytest.mark.gpu
REL_MAX, REL_MEAN = 2e-2, 1e-2
ABS_MAX, ABS_MEAN = 2e-2, 2e-3


def _topology(case, rng):
    name, P, T, L, N, KL, KG, n, W, H, D, direct, kind = case
    if kind == "membership":
        mem = rng.random((T, N, P)) < 0.4
        go = ~mem.any(1) & (rng.random((T, P)) < 0.6)
        full = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                        direct=direct, membership=mem, global_only=go)
        return FullTopology(P, T, L, N, KL, KG, n, W, direct, membership=mem, global_only=go), full
    labels = np.array([[p % N for p in range(P)]] * T)
    if T >= 2 * n:
        labels[n:2 * n] = [(p + 1) % N for p in range(P)]
    active = np.zeros((T, N), dtype=bool)
    active[np.arange(T)[:, None], labels] = True
    if kind == "inactive":
        active[:, -1] = False
    full = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W,
                                    direct=direct, labels=labels, active=active)
    return FullTopology(P, T, L, N, KL, KG, n, W, direct, labels=labels, active=active), full


CASES = [
    # name, P, T, L, N, KL, KG, n, W, H, D, direct, kind
    ("d128_w4", 4, 6, 20, 2, 5, 6, 3, 4, 2, 128, True, "labels"),
    ("d128_nodirect", 4, 6, 20, 2, 5, 6, 3, -1, 2, 128, False, "labels"),
    ("d64_c1", 4, 3, 64, 2, 1, 1, 3, 21, 2, 64, True, "labels"),
    ("d128_inactive", 3, 6, 37, 3, 2, 3, 2, 4, 2, 128, True, "inactive"),
    ("d128_membership", 6, 6, 24, 3, 2, 3, 3, 4, 2, 128, True, "membership"),
]


def _check(name, got, ref):
    err = (got.float().cpu() - ref).abs()
    scale_max = ref.abs().max().item()
    scale_mean = ref.abs().mean().item()
    say(f"  {name}: max-abs {err.max().item():.3e} (ref max {scale_max:.3e}) "
        f"mean-abs {err.mean().item():.3e} (ref mean {scale_mean:.3e})")
    assert torch.isfinite(got.float()).all()
    assert err.max().item() <= ABS_MAX and err.mean().item() <= ABS_MEAN
    assert err.max().item() <= REL_MAX * scale_max + 1e-6
    assert err.mean().item() <= REL_MEAN * scale_mean + 1e-7


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_backward_matches_oracle_autograd(case):
    need_gpu()
    rng = np.random.default_rng(11)
    topo, full = _topology(case, rng)
    H, D = case[9], case[10]
    say("backward", case[0], "S", topo.S)
    g = torch.Generator().manual_seed(5)
    q, k, v = [(torch.randn(topo.S, H, D, generator=g) * 0.5).to(torch.bfloat16) for _ in range(3)]
    dout = torch.randn(topo.S, H, D, generator=g).to(torch.bfloat16)
    tiles = M.build(full, "cuda").tiles

    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    out = hier_attention(qd, kd, vd, tiles)
    out.backward(dout.cuda())
    torch.cuda.synchronize()

    qf, kf, vf = (t.float().requires_grad_(True) for t in (q, k, v))
    ref = masked_attention(qf, kf, vf, topo)
    ref.backward(dout.float())
    _check("out", out.detach(), ref.detach())
    _check("dq", qd.grad, qf.grad)
    _check("dk", kd.grad, kf.grad)
    _check("dv", vd.grad, vf.grad)


def test_backward_is_deterministic():
    need_gpu()
    rng = np.random.default_rng(2)
    topo, full = _topology(CASES[0], rng)
    H, D = 2, 128
    g = torch.Generator().manual_seed(9)
    q, k, v, dout = [torch.randn(topo.S, H, D, generator=g).to(torch.bfloat16).cuda() for _ in range(4)]
    tiles = M.build(full, "cuda").tiles
    say("backward determinism")
    res = []
    for _ in range(2):
        qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
        hier_attention(qd, kd, vd, tiles).backward(dout)
        res.append(torch.cat([qd.grad, kd.grad, vd.grad]))
    torch.cuda.synchronize()
    assert torch.equal(res[0], res[1])


def test_backward_argument_errors():
    need_gpu()
    rng = np.random.default_rng(2)
    topo, full = _topology(CASES[0], rng)
    tiles = M.build(full, "cuda").tiles
    H, D = 2, 128
    x = torch.zeros(topo.S, H, D, dtype=torch.bfloat16, device="cuda")
    lse = torch.zeros(H, topo.S, device="cuda")
    with pytest.raises(NotImplementedError):
        hier_attention_backward(x.float(), x, x, x, x, lse, tiles)
    with pytest.raises(ValueError):
        hier_attention_backward(x, x[:-1], x, x, x, lse, tiles)
    with pytest.raises(ValueError):
        hier_attention_backward(x, x, x, x, x, lse.double(), tiles)


def test_membership_ste_gradient_matches_oracle():
    """Soft membership logits ~ N(0, 1): hard forward on logits > 0, the
    straight-through logit gradient of oracle/ste.py (fp32 autograd)."""
    need_gpu()
    from oracle.ste import ste_attention
    rng = np.random.default_rng(21)
    P, T, L, N, KL, KG, n, W, H, D = 4, 6, 24, 2, 5, 6, 3, 4, 2, 128
    logits = torch.from_numpy(rng.standard_normal((T, N, P))).float()
    mem = (logits > 0).numpy()
    go = ~mem.any(1)
    topo = FullTopology(P, T, L, N, KL, KG, n, W, True, membership=mem, global_only=go)
    full = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W, direct=True,
                                    membership=mem, global_only=go)
    g = torch.Generator().manual_seed(4)
    q, k, v = [(torch.randn(topo.S, H, D, generator=g) * 0.5).to(torch.bfloat16) for _ in range(3)]
    dout = torch.randn(topo.S, H, D, generator=g).to(torch.bfloat16)
    tiles = M.build(full, "cuda").tiles
    say("membership STE", topo.S)
    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    lg = logits.cuda().requires_grad_(True)
    out = hier_attention(qd, kd, vd, tiles, membership_logits=lg, ste_geometry=(P, T, L, N, KL))
    out.backward(dout.cuda())
    torch.cuda.synchronize()
    qf, kf, vf = (t.float().requires_grad_(True) for t in (q, k, v))
    lf = logits.clone().requires_grad_(True)
    ref = ste_attention(qf, kf, vf, topo, lf)
    ref.backward(dout.float())
    _check("dq", qd.grad, qf.grad)
    _check("dk", kd.grad, kf.grad)
    _check("dv", vd.grad, vf.grad)
    _check("dlogits", lg.grad, lf.grad)
    assert (lf.grad != 0).any()


@pytest.mark.parametrize("cfg", ["small", "c5"])
def test_ste_in_dq_pass_equals_the_separate_pass(cfg):
    """The membership STE summed inside the dQ pass (forward-list classes)
    against the separate pass over the STE list: dQ / dK / dV bit-identical
    (also to the backward without STE), the per-bit sums equal up to fp32
    summation order."""
    need_gpu()
    import bench
    if cfg == "c5":
        P, T, L, N, KL, KG, n, W, _, D, grp = bench.CONFIGS["c5"]
        logits, mem, go = bench.grouping(grp, P, T, N, np.random.default_rng(bench.SEED))
        H = 4
    else:
        P, T, L, N, KL, KG, n, W, H, D = 4, 6, 24, 2, 5, 6, 3, 4, 2, 128
        logits = np.random.default_rng(22).standard_normal((T, N, P)).astype(np.float32)
        mem = logits > 0
        go = ~mem.any(1)
    topo = FullTopology(P, T, L, N, KL, KG, n, W, True, membership=mem, global_only=go)
    full = M.full_sequence_topology(P=P, T=T, L=L, N=N, KL=KL, KG=KG, n=n, window=W, direct=True,
                                    membership=mem, global_only=go)
    tiles = M.build(full, "cuda").tiles
    g = torch.Generator().manual_seed(5)
    q, k, v = [(torch.randn(topo.S, H, D, generator=g) * 0.5).to(torch.bfloat16).cuda()
               for _ in range(3)]
    dout = torch.randn(topo.S, H, D, generator=g).to(torch.bfloat16).cuda()
    say("STE in dQ vs separate pass", cfg, topo.S)
    out = torch.zeros_like(q)
    lse = torch.full((H, topo.S), float("-inf"), dtype=torch.float32, device="cuda")
    hier_attention_forward(q, k, v, tiles, out, lse=lse)
    geo = (P, T, L, N, KL)
    plain = hier_attention_backward(q, k, v, out, dout, lse, tiles)
    fold = hier_attention_backward(q, k, v, out, dout, lse, tiles, ste_geometry=geo)
    sep = hier_attention_backward(q, k, v, out, dout, lse, tiles, ste_geometry=geo,
                                  ste_pass="list")
    torch.cuda.synchronize()
    for i, name in enumerate(("dq", "dk", "dv")):
        assert torch.equal(fold[i], plain[i]), name
        assert torch.equal(sep[i], plain[i]), name
    a, b = fold[3].double().cpu(), sep[3].double().cpu()
    scale = b.abs().max().item()
    say(f"  gated sums: max |fold - separate| {(a - b).abs().max().item():.3e} (max {scale:.3e})")
    assert scale > 0 and (a != 0).any()
    assert ((a - b).abs() <= 1e-5 * scale + 1e-6 * b.abs()).all()


@pytest.mark.parametrize("case", [CASES[3], CASES[4]], ids=[CASES[3][0], CASES[4][0]])
def test_uncleared_buffers_are_fully_written(case, monkeypatch):
    """When a list's items own every row, the forward output / LSE and dQ / dK
    / dV are left uncleared.  Pre-filled with NaN instead (the test hook
    ``_UNCLEARED_FILL``), the results equal the zero-filled path bit for bit,
    on topologies with inactive local-hub rows (queries and keys with empty
    lists) and membership orphans: every row is written by a kernel."""
    need_gpu()
    from multics_amd import kernels as K
    rng = np.random.default_rng(11)
    topo, full = _topology(case, rng)
    H, D = case[9], case[10]
    say("uncleared buffers", case[0], "S", topo.S)
    g = torch.Generator().manual_seed(5)
    q, k, v, dout = [(torch.randn(topo.S, H, D, generator=g) * 0.5).to(torch.bfloat16).cuda()
                     for _ in range(4)]
    tiles = M.build(full, "cuda").tiles
    assert K._covers_all_rows(tiles)
    ste = None
    if case[-1] == "membership":
        # logits whose hard value is the topology's membership: the STE sums
        # (partial buffer) and the delta / lse2 workspace are uncleared too
        P, T, N = case[1], case[2], case[4]
        lg = torch.from_numpy(np.where(topo.membership, 1.0, -1.0) *
                              (0.5 + rng.random((T, N, P)))).float().cuda()
        ste = (lg, (P, T, case[3], N, case[5]))

    def run():
        qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
        if ste is None:
            out = hier_attention(qd, kd, vd, tiles)
        else:
            ld = ste[0].clone().requires_grad_(True)
            out = hier_attention(qd, kd, vd, tiles, membership_logits=ld, ste_geometry=ste[1])
        out.backward(dout)
        torch.cuda.synchronize()
        return out.detach(), qd.grad, kd.grad, vd.grad, (ld.grad if ste else qd.grad)

    monkeypatch.setattr(K, "_UNCLEARED_FILL", float("nan"))
    nan_run = run()
    monkeypatch.setattr(K, "_covers_all_rows", lambda t: False)
    zero_run = run()
    for name, a, b in zip(("out", "dq", "dk", "dv", "dlogits"), nan_run, zero_run):
        assert torch.isfinite(a.float()).all(), name
        assert torch.equal(a, b), name
