"""The packed-varlen plan (hier_packed_attention.py:32-102) on the CPU.

Inputs are the reference's own ``_build_metadata`` arrays (golden vectors
written by the reference builder) of every golden case built with one program
per segment.  The oracle's ``varlen_plan`` and the product's
``metadata._get_varlen_plan`` must agree exactly, and the plan must expand to
exactly the (query, key) pairs of the segment lists (brute force over the
golden arrays), whose count is the reference's own ``logical_pairs``.  The
refusal cases (programs that split a segment, segments that do not partition
the query rows) raise ``AssertionError`` in both, as in the reference.
"""

import numpy as np
import pytest
import torch

from multics_amd.metadata import _get_varlen_plan, clear_varlen_plan_cache
from oracle.metadata import CachedTopology, segmented_metadata, varlen_plan
from tests import golden_io as G
from tests.test_oracle_metadata import topo_from


def _packed_cases():
    out = []
    for name in G.cases("seg"):
        g = G.golden()
        ps = g[f"seg/{name}/prog_seg"]
        if len(ps) == len(g[f"seg/{name}/kv_count"]) and (ps == np.arange(len(ps))).all():
            out.append(name)
    return out


def _arrays(name):
    """The golden arrays (the oracle's restatement where the golden file keeps
    only a digest; the two are byte-equal by test_oracle_metadata)."""
    inp = G.inputs("seg", name)
    ref = segmented_metadata(topo_from(inp), inp["block_m"])
    for f in ("prog_qbase", "prog_nq", "prog_seg", "kv_index", "kv_count"):
        G.assert_same(f"seg/{name}/{f}", ref[f])
    return ref


@pytest.mark.parametrize("name", _packed_cases())
def test_plan_matches_segments(name):
    a = _arrays(name)
    qt = int(np.asarray(a["prog_nq"]).sum())
    want = varlen_plan(a["kv_index"], a["kv_count"], a["prog_qbase"], a["prog_nq"],
                       a["prog_seg"], qt)
    t = {k: torch.from_numpy(np.ascontiguousarray(a[k])) for k in
         ("kv_index", "kv_count", "prog_qbase", "prog_nq", "prog_seg")}
    clear_varlen_plan_cache()
    got = _get_varlen_plan(kv_index=t["kv_index"], kv_count=t["kv_count"], qbase=t["prog_qbase"],
                           qlen=t["prog_nq"], seg_ids=t["prog_seg"], query_tokens=qt)
    for k in ("q_index", "k_index", "cu_q", "cu_k"):
        assert got[k].dtype == (torch.int64 if k.endswith("index") else torch.int32), k
        assert np.array_equal(got[k].numpy(), want[k]), k
    for k in ("max_q", "max_k", "min_k_index", "max_k_index"):
        assert got[k] == want[k], k
    # cache hit returns the same plan object
    assert _get_varlen_plan(kv_index=t["kv_index"], kv_count=t["kv_count"], qbase=t["prog_qbase"],
                            qlen=t["prog_nq"], seg_ids=t["prog_seg"], query_tokens=qt) is got
    # brute force: the plan's pairs are exactly the segment lists' pairs
    kv = np.asarray(a["kv_index"]).astype(np.int64)
    width = int(kv.max()) + 1 if kv.size else 1
    seg_codes = []
    for s, (b, n) in enumerate(zip(a["prog_qbase"], a["prog_nq"])):
        keys = kv[s][:int(a["kv_count"][s])]
        rows = np.arange(int(b), int(b) + int(n), dtype=np.int64)
        seg_codes.append((rows[:, None] * width + keys[None, :]).ravel())
    plan_codes = []
    cq, ck = want["cu_q"], want["cu_k"]
    for i in range(len(cq) - 1):
        rows = want["q_index"][cq[i]:cq[i + 1]]
        keys = want["k_index"][ck[i]:ck[i + 1]]
        plan_codes.append((rows[:, None] * width + keys[None, :]).ravel())
    cat = lambda xs: np.sort(np.concatenate(xs)) if xs else np.zeros(0, np.int64)
    seg_all, plan_all = cat(seg_codes), cat(plan_codes)
    assert np.array_equal(plan_all, seg_all)
    assert len(np.unique(plan_all)) == len(plan_all)
    assert len(plan_all) == G.scalar(f"seg/{name}/logical_pairs")


def test_plan_refusals():
    name = _packed_cases()[0]
    a = _arrays(name)
    qt = int(np.asarray(a["prog_nq"]).sum())
    t = {k: torch.from_numpy(np.ascontiguousarray(a[k])) for k in
         ("kv_index", "kv_count", "prog_qbase", "prog_nq", "prog_seg")}
    bad_seg = t["prog_seg"].clone()
    bad_seg[-1] = 0
    bad_q = t["prog_qbase"].clone()
    bad_q[1] += 1
    for kw in (dict(seg_ids=bad_seg), dict(qbase=bad_q), dict(query_tokens=qt + 1)):
        args = dict(kv_index=t["kv_index"], kv_count=t["kv_count"], qbase=t["prog_qbase"],
                    qlen=t["prog_nq"], seg_ids=t["prog_seg"], query_tokens=qt)
        args.update(kw)
        clear_varlen_plan_cache()
        with pytest.raises(AssertionError):
            _get_varlen_plan(**args)
        with pytest.raises(AssertionError):
            varlen_plan(args["kv_index"].numpy(), args["kv_count"].numpy(), args["qbase"].numpy(),
                        args["qlen"].numpy(), args["seg_ids"].numpy(), args["query_tokens"])
