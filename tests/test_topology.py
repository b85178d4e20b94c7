"""The topology normalisers (multics_amd/topology.py, reference
hier_masks.py:22-214) on the CPU: normal forms against the oracle's, and the
refusal cases the reference tests assert
(tests/test_hier_flexible_membership_mask.py:262-293 and the shape checks of
hier_masks.py:22-193)."""

import numpy as np
import pytest
import torch

from multics_amd import topology as TP
from oracle.masks import FullTopology


def test_labels_normal_form_matches_oracle():
    T, P, N = 4, 4, 3
    labels = torch.tensor([[0, 0, 1, 1], [0, 2, 2, 1], [1, 1, 1, 1], [2, 0, 0, 2]])
    lab, act = TP._prepare_hier_group_tensors(labels, None, P, T, N, "cpu")
    assert lab.dtype == torch.long and torch.equal(lab, labels)
    _, oact, go, labels_form = FullTopology(P, T, 2, N, 1, 1, 2, -1, True,
                                            labels=labels.numpy()).normalized()
    assert labels_form and not go.any()
    assert np.array_equal(act.numpy(), oact)         # active = scatter of the labels
    lab3, act3 = TP._prepare_hier_group_tensors(labels[None], act[None], P, T, N, "cpu")
    assert torch.equal(lab3, lab) and torch.equal(act3, act)


def test_labels_refusals():
    T, P, N = 3, 4, 2
    with pytest.raises(ValueError, match=r"must be in \[0,2\)"):
        TP._prepare_hier_group_tensors(torch.tensor([[-1, 0, 0, 1]] * T), None, P, T, N, "cpu")
    with pytest.raises(ValueError, match=r"must be in \[0,2\)"):
        TP._prepare_hier_group_tensors(torch.tensor([[0, 2, 0, 1]] * T), None, P, T, N, "cpu")
    with pytest.raises(ValueError, match="requires group_labels"):
        TP._prepare_hier_group_tensors(None, None, P, T, N, "cpu")
    with pytest.raises(ValueError, match="batch B=1"):
        TP._prepare_hier_group_tensors(torch.zeros(2, T, P, dtype=torch.long), None, P, T, N,
                                       "cpu")
    with pytest.raises(ValueError, match=r"\[T=3,P=4\]"):
        TP._prepare_hier_group_tensors(torch.zeros(T, P + 1, dtype=torch.long), None, P, T, N,
                                       "cpu")
    with pytest.raises(ValueError, match=r"active_group must be \[T=3,N=2\]"):
        TP._prepare_hier_group_tensors(torch.zeros(T, P, dtype=torch.long),
                                       torch.ones(T, N + 1, dtype=torch.bool), P, T, N, "cpu")


def test_membership_normal_form_matches_oracle():
    rng = np.random.default_rng(0)
    T, N, P = 5, 3, 4
    mem = rng.random((T, N, P)) < 0.4
    go = ~mem.any(1)
    m, g, act = TP._prepare_hier_membership_tensors(torch.from_numpy(mem)[None],
                                                    torch.from_numpy(go)[None], None, P, T, N,
                                                    "cpu")
    assert m.dtype == torch.bool and np.array_equal(m.numpy(), mem)
    assert np.array_equal(g.numpy(), go)
    _, oact, ogo, labels_form = FullTopology(P, T, 2, N, 1, 1, 2, -1, True, membership=mem,
                                             global_only=go).normalized()
    assert not labels_form
    assert np.array_equal(act.numpy(), oact) and np.array_equal(g.numpy(), ogo)
    # full-clip tensors for a cached block: T may exceed the block's frames
    m2, _, act2 = TP._prepare_hier_membership_tensors(torch.from_numpy(mem),
                                                      torch.from_numpy(go),
                                                      torch.ones(2, N, dtype=torch.bool), P, 2,
                                                      N, "cpu", allow_full_t=True)
    assert m2.shape == (T, N, P) and np.array_equal(act2.numpy(), mem.any(-1))


def test_membership_refusals():
    T, N, P = 4, 2, 3
    mem = torch.zeros(T, N, P, dtype=torch.bool)
    go = torch.zeros(T, P, dtype=torch.bool)
    with pytest.raises(ValueError, match="requires membership"):
        TP._prepare_hier_membership_tensors(None, go, None, P, T, N, "cpu")
    with pytest.raises(ValueError, match="requires global_only"):
        TP._prepare_hier_membership_tensors(mem, None, None, P, T, N, "cpu")
    with pytest.raises(ValueError, match="num_players"):
        TP._prepare_hier_membership_tensors(mem, go, None, P + 1, T, N, "cpu")
    with pytest.raises(ValueError, match="num_groups"):
        TP._prepare_hier_membership_tensors(mem, go, None, P, T, N + 1, "cpu")
    with pytest.raises(ValueError, match="must be"):
        TP._prepare_hier_membership_tensors(mem, go, None, P, T + 1, N, "cpu")
    with pytest.raises(ValueError, match="shorter than current block"):
        TP._prepare_hier_membership_tensors(mem, go, None, P, T + 1, N, "cpu", allow_full_t=True)
    with pytest.raises(ValueError, match="global_only must be"):
        TP._prepare_hier_membership_tensors(mem, go[:, :-1], None, P, T, N, "cpu")
    with pytest.raises(ValueError, match="batch B must be 1"):
        TP._prepare_hier_membership_tensors(mem[None].expand(2, T, N, P), go, None, P, T, N, "cpu")
    with pytest.raises(ValueError, match="rank 3 or 4"):
        TP._prepare_hier_membership_tensors(mem[0], go, None, P, T, N, "cpu")
    with pytest.raises(ValueError, match="active_group must be"):
        TP._prepare_hier_membership_tensors(mem, go, torch.ones(T, N + 1, dtype=torch.bool), P, T,
                                            N, "cpu")


def test_refuse_membership_on_scalar_kernel():
    """tests/test_hier_flexible_membership_mask.py:279-293."""
    with pytest.raises(ValueError, match="hier_tiled_ste"):
        TP._refuse_membership_on_scalar_kernel(attn_impl="hier_tiled_ste")
    with pytest.raises(ValueError, match="tiled128"):
        TP._refuse_membership_on_scalar_kernel(infer_kernel="tiled128")
    with pytest.raises(ValueError, match="segmented"):
        TP._refuse_membership_on_scalar_kernel(infer_kernel="segmented")
    TP._refuse_membership_on_scalar_kernel(attn_impl="flex", infer_kernel="paged_kv")


def test_debug_labels_and_slices():
    mem = torch.zeros(2, 3, 4, dtype=torch.bool)
    mem[0, 1, 0] = mem[0, 2, 1] = mem[1, 0, 2] = True
    lab = TP._debug_labels_from_membership(mem)
    assert lab.tolist() == [[1, 2, -1, -1], [-1, -1, 0, -1]]
    act = torch.arange(12).reshape(6, 2) % 3 == 0
    assert torch.equal(TP._slice_hier_active_group_for_cached_mask(act, 2, 3), act[2:5])
    assert torch.equal(TP._slice_hier_active_group_for_cached_mask(act[:3], 4, 3), act[:3])
    assert TP._slice_hier_active_group_for_cached_mask(None, 0, 3) is None
    with pytest.raises(ValueError, match="does not cover"):
        TP._slice_hier_active_group_for_cached_mask(act, 5, 2)
    with pytest.raises(ValueError, match="invalid cached"):
        TP._slice_hier_active_group_for_cached_mask(act, -1, 2)
    with pytest.raises(ValueError, match="K_L=0 and K_G>0"):
        TP._validate_hier_no_local_topology(True, 1, 2)
    with pytest.raises(ValueError, match="K_L=0 and K_G>0"):
        TP._validate_hier_no_local_topology(True, 0, 0)
    TP._validate_hier_no_local_topology(True, 0, 3)
    TP._validate_hier_no_local_topology(False, 5, 6)


def test_query_active_mask_rows():
    P, T, L, N, KL, KG = 2, 3, 4, 2, 2, 3
    active = torch.tensor([[True, False], [False, True], [True, True]])
    m = TP.build_hier_query_active_mask(active_group=active, num_players=P, num_frames=T,
                                        num_patches=L, num_groups=N, num_local_hub_tokens=KL,
                                        num_global_hub_tokens=KG, device="cpu",
                                        dtype=torch.float32)
    topo = FullTopology(P, T, L, N, KL, KG, 3, -1, True, labels=np.zeros((T, P), int),
                        active=active.numpy())
    from oracle.masks import inactive_local_rows
    assert m.shape == (1, topo.S, 1)
    assert np.array_equal(m[0, :, 0].numpy() == 0, inactive_local_rows(topo))
    with pytest.raises(ValueError):
        TP.build_hier_query_active_mask(active_group=active[:2], num_players=P, num_frames=T,
                                        num_patches=L, num_groups=N, num_local_hub_tokens=KL,
                                        num_global_hub_tokens=KG, device="cpu",
                                        dtype=torch.float32)
