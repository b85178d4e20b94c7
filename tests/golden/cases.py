"""Topology cases shared by the golden-vector script and the tests.

Each case is a plain JSON-serialisable dict of builder inputs.  The shapes
follow the reference's own metadata tests
(tests/test_hier_segmented_metadata.py:111-174, tests/test_hier_tiled_layout.py:30-206,
tests/test_hier_tiled_ste_kernel.py:24-60), the benchmark configurations C1 and
C2, and the reference grouping fixtures (tests/fixtures/grouping/*.labels.npz,
whose membership rows are copied into ``fixture_membership.npz`` as data).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def _cached(P, N, L, KL, KG, n_frames, n_block, local_attn, agent_frames, local_frames,
            global_frames, local_active, labels, q_active, direct, membership=None,
            global_only=None, no_local=False, block_m=16):
    return dict(P=P, N=N, L=L, KL=KL, KG=KG, n_frames=n_frames, n_block=n_block,
                local_attn=local_attn, agent_frames=agent_frames, local_frames=local_frames,
                global_frames=global_frames, local_active=local_active, labels=labels,
                q_active=q_active, direct=direct, membership=membership,
                global_only=global_only, no_local=no_local, block_m=block_m)


def _steady(P, N, L, KL, KG, n, W, block, labels_row, direct, *, T=None, mem=None, go=None,
            block_m=16, active_rows=None):
    """Cached call for temporal block ``block`` after a rolling cache of W+n frames."""
    b1 = (block + 1) * n
    retention = b1 if W == -1 else W + n
    frames = list(range(max(0, b1 - retention), b1))
    qf = frames[-n:]
    if mem is not None:
        act = [[bool(any(mem[t][g])) for g in range(N)] for t in range(len(mem))]
        q_active = [act[t] for t in qf]
        local_active = [[act[f][g] for f in frames] for g in range(N)]
        labels = None
    else:
        labels = [list(labels_row)] * n
        if active_rows is None:
            active_rows = [[g in labels_row for g in range(N)]] * (b1)
        q_active = [list(active_rows[t]) for t in qf]
        local_active = [[bool(active_rows[f][g]) for f in frames] for g in range(N)]
    return _cached(P, N, L, KL, KG, n, n, W, [frames] * P, [frames] * N, frames,
                   local_active, labels, q_active, direct, membership=mem,
                   global_only=go, block_m=block_m)


def _fixture_rows(name):
    data = np.load(HERE / "fixture_membership.npz")
    return data[f"{name}/membership"].astype(bool), data[f"{name}/global_only"].astype(bool)


def segmented_cases():
    out = []
    # the reference metadata test's own parameterisation
    for P in (2, 4, 6, 8):
        for direct in (False, True):
            N = max(2, P // 2 + 1)
            frames = list(range(1, 7))
            row = [p % (N - 1) for p in range(P)]
            act = [g in row for g in range(N)]
            la = [[(f + g) % 3 != 0 and act[g] for f in frames] for g in range(N)]
            out.append((f"reftest_P{P}_d{int(direct)}", _cached(
                P, N, 3, 2, 2, 2, 2, 4, [frames] * P, [frames] * N, frames, la,
                [row] * 2, [act] * 2, direct)))
    # C1 shapes (P4, N2, KL=KG=1, L=64)
    out.append(("c1_n1_first", _steady(4, 2, 64, 1, 1, 1, -1, 0, [0, 0, 1, 1], True)))
    out.append(("c1_n1_last", _steady(4, 2, 64, 1, 1, 1, -1, 2, [0, 0, 1, 1], True)))
    out.append(("c1_n3_w21", _steady(4, 2, 64, 1, 1, 3, 21, 0, [0, 0, 1, 1], True)))
    # membership: anchor in two slots, a global-only orphan, an empty slot that
    # becomes active, global_only varying over key frames
    T = 6
    mem = np.zeros((T, 3, 4), dtype=bool)
    go = np.zeros((T, 4), dtype=bool)
    for t in range(T):
        mem[t, 0, [0, 1]] = True
        mem[t, 1, [0, 2]] = True
        if t >= 4:
            mem[t, 2, 3] = True
        else:
            go[t, 3] = True
    go[1, 1] = True
    for direct in (False, True):
        for bm in (16, 5):
            out.append((f"mem_anchor_d{int(direct)}_bm{bm}", _steady(
                4, 3, 5, 2, 3, 2, 4, 2, None, direct, mem=mem.tolist(), go=go.tolist(),
                block_m=bm)))
    # no-local topology (K_L=0)
    frames = list(range(0, 4))
    out.append(("nolocal_labels", _cached(
        3, 2, 6, 0, 4, 2, 2, -1, [frames] * 3, [], frames, [], [[0, 0, 1]] * 2,
        [[True, True]] * 2, True, no_local=True, block_m=6)))
    # reference grouping fixtures: membership changing mid clip
    for name, P, N, L in (("p6_moving_pairs", 6, 3, 4), ("p10_moving_pairs", 10, 4, 3),
                          ("p4_round_start", 4, 2, 4)):
        m, g = _fixture_rows(name)
        change = [t for t in range(1, m.shape[0]) if not np.array_equal(m[t], m[t - 1])]
        blk = (change[0] // 3) if change else 7
        out.append((f"fx_{name}", _steady(P, N, L, 2, 3, 3, 21, blk, None, True,
                                          mem=m.tolist(), go=g.tolist(), block_m=max(L, 3))))
    # C2 steady-state and final block, labels {0,1},{2,3}
    out.append(("c2_block7", _steady(4, 2, 220, 5, 6, 3, 21, 7, [0, 0, 1, 1], True)))
    out.append(("c2_block13_paged", _steady(4, 2, 220, 5, 6, 3, 21, 13, [0, 0, 1, 1], True,
                                            block_m=220)))
    return out


def tiled_cached_cases():
    out = []
    labels = [[0, 0, 1, 1]] * 3 + [[0, 1, 0, 1]] * 3 + [[1, 1, 0, 0]] * 3
    for b in range(3):
        c = _steady(4, 2, 5, 2, 3, 3, 4, b, labels[3 * b], True,
                    active_rows=[[True, True]] * 9)
        c.pop("block_m")
        out.append((f"reftest_block{b}", c))
    frames = list(range(1, 7))
    la = [[(f + g) % 3 != 0 and g < 2 for f in frames] for g in range(3)]
    for direct in (False, True):
        c = _cached(3, 3, 4, 2, 2, 2, 2, 4, [frames] * 3, [frames] * 3, frames, la,
                    [[0, 0, 1]] * 2, [[True, True, False]] * 2, direct)
        c.pop("block_m")
        out.append((f"inactive_d{int(direct)}", c))
    c = _steady(4, 2, 64, 1, 1, 3, 21, 0, [0, 0, 1, 1], True)
    c.pop("block_m")
    out.append(("c1_n3", c))
    c = _steady(4, 2, 220, 5, 6, 3, 21, 7, [0, 0, 1, 1], True)
    c.pop("block_m")
    out.append(("c2_block7", c))
    return out


def full_sequence_cases():
    out = []
    lab1 = [[0, 0, 1, 1]] * 3 + [[0, 2, 2, 0]] * 3 + [[1, 1, 2, 2]] * 3
    act1 = [[g in row for g in range(3)] for row in lab1]
    for direct in (False, True):
        out.append((f"reftest1_d{int(direct)}", dict(P=4, T=9, L=7, N=3, KL=2, KG=3, n=3, window=4,
                                                   labels=lab1, active=act1, direct=direct)))
    lab2 = [[0, 0, 1, 1]] * 3 + [[0, 1, 0, 1]] * 3 + [[1, 1, 0, 0]] * 3
    out.append(("reftest3", dict(P=4, T=9, L=5, N=2, KL=2, KG=3, n=3, window=4, labels=lab2,
                                 active=[[True, True]] * 9, direct=True)))
    out.append(("ste_shape", dict(P=2, T=3, L=17, N=3, KL=2, KG=2, n=3, window=7,
                                  labels=[[0, 1]] * 3, active=[[True, True, False]] * 3,
                                  direct=True)))
    for n, w in ((1, -1), (3, 21)):
        out.append((f"c1_n{n}", dict(P=4, T=3, L=64, N=2, KL=1, KG=1, n=n, window=w,
                                     labels=[[0, 0, 1, 1]] * 3, active=[[True, True]] * 3,
                                     direct=True)))
    for w in (21, 7):
        out.append((f"c2_w{w}", dict(P=4, T=42, L=220, N=2, KL=5, KG=6, n=3, window=w,
                                     labels=[[0, 0, 1, 1]] * 42, active=[[True, True]] * 42,
                                     direct=True)))
    return out
