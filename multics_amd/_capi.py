"""ctypes binding of the C ABI in ``include/hierattn.h``.

The library is loaded from ``multics_amd/_lib/libhierattn.so`` (built in tree
by ``multics_amd.build``), or from the file named by ``HIERATTN_LIB``.  There is no fallback: when the library is missing
the import of a compute entry point raises.  Error codes map back to the
exception types the reference raises for the same conditions
(multics/models/kernels/hier_segmented_attention.py:425-431 NotImplementedError,
multics/models/attention.py:500-506 ValueError,
multics/models/kernels/hier_paged_attention.py:37-47 RuntimeError,
multics/models/kernels/hier_packed_attention.py:54-64 AssertionError).
"""

from __future__ import annotations

import ctypes as C
import os
import threading
from pathlib import Path

LIB_PATH = Path(os.environ.get("HIERATTN_LIB") or
                Path(__file__).resolve().parent / "_lib" / "libhierattn.so")

HIER_OK, HIER_EINVAL, HIER_EUNSUPPORTED, HIER_ELAUNCH, HIER_EINTERNAL = 0, -1, -2, -3, -4

i32, i64, f32, vp = C.c_int32, C.c_int64, C.c_float, C.c_void_p


class HierTopo(C.Structure):
    _fields_ = [(n, i32) for n in ("P", "N", "L", "KL", "KG", "n_frames", "n_block",
                                   "local_attn", "direct", "no_local", "use_membership", "B",
                                   "fa_max", "fl_max", "fg_max", "T_mem")] + \
               [(n, vp) for n in ("fa", "fl", "fg", "agent_frames", "local_frames",
                                  "global_frames", "local_active", "q_frames", "labels",
                                  "q_active", "membership", "global_only", "ref_agent_base",
                                  "ref_local_base", "ref_global_base", "tile_agent_base",
                                  "tile_local_base", "tile_global_base", "ref_qbase",
                                  "tile_qbase")] + \
               [("ref_qstride", i32 * 3), ("tile_qstride", i32 * 3)]


class HierMetaCounts(C.Structure):
    _fields_ = [(n, vp) for n in ("seg_count", "tiled_count", "dense_count", "logical_count",
                                  "tile_count")]


class HierMetaOut(C.Structure):
    _fields_ = [("block_m", i32)] + \
               [(n, vp) for n in ("seg_prog_off", "seg_kv_off", "seg_max_k", "seg_prog_qbase",
                                  "seg_prog_nq", "seg_prog_seg", "seg_kv_index", "seg_kv_count",
                                  "tiled_prog_off", "tiled_kv_off", "tiled_max_k",
                                  "tiled_prog_qbase", "tiled_prog_nq", "tiled_prog_seg",
                                  "tiled_kv_index", "tiled_kv_valid", "tiled_kv_count",
                                  "tile_kv_off", "tile_item_off")] + \
               [("rows_per_item", i32)] + \
               [(n, vp) for n in ("tile_kv_idx", "tile_kv_mask", "tile_blk_and", "tile_items")]


class HierPrologueArgs(C.Structure):
    _fields_ = [("S", i32), ("H", i32), ("D", i32), ("eps", f32)] + \
               [(n, vp) for n in ("qx", "kx", "vx", "cam", "w_cam_q", "w_cam_k")] + \
               [("C", i32)] + \
               [(n, vp) for n in ("norm_q_w", "norm_k_w", "rope_cos", "rope_sin", "q_out",
                                  "k_out", "v_out")] + \
               [("out_stride_s", i64), ("out_stride_h", i64)]


class HierFwdArgs(C.Structure):
    _fields_ = [("H", i32), ("D", i32), ("n_items", i32), ("scale", f32), ("kv_rows", i32),
                ("reserved", i32)] + \
               [(n, vp) for n in ("q", "k", "v", "o", "lse")] + \
               [(n, i64) for n in ("q_ss", "q_sh", "k_ss", "k_sh", "v_ss", "v_sh", "o_ss", "o_sh",
                                   "lse_stride_h")] + \
               [(n, vp) for n in ("tile_items", "tile_kv_idx", "tile_kv_mask", "tile_blk_and",
                                  "row_table")]


class HierBwdArgs(C.Structure):
    _fields_ = [("H", i32), ("D", i32), ("n_items", i32), ("n_key_items", i32), ("scale", f32),
                ("kv_rows", i32), ("q_rows", i32), ("reserved", i32)] + \
               [(n, vp) for n in ("q", "k", "v", "o", "dout", "lse", "delta", "lse2", "dq", "dk",
                                  "dv")] + \
               [(n, i64) for n in ("q_ss", "q_sh", "k_ss", "k_sh", "v_ss", "v_sh", "o_ss", "o_sh",
                                   "do_ss", "do_sh", "dq_ss", "dq_sh", "dk_ss", "dk_sh", "dv_ss",
                                   "dv_sh", "lse_stride_h")] + \
               [(n, vp) for n in ("tile_items", "tile_kv_idx", "tile_kv_mask", "tile_blk_and",
                                  "key_items", "key_q_idx", "key_q_mask", "key_blk_and")] + \
               [("n_ste_items", i32), ("ste_classes", i32)] + \
               [(n, vp) for n in ("ste_items", "ste_kv_idx", "ste_kv_mask", "ste_kv_class",
                                  "ste_partial")] + \
               [("ste_stride_h", i64), ("tile_kv_class", vp), ("tile_ste_first", vp),
                ("key_row_table", vp)]


class HierPageArgs(C.Structure):
    _fields_ = [("H", i32), ("D", i32), ("n_rows", i32), ("pool_rows", i32),
                ("k_src", vp), ("v_src", vp)] + \
               [(n, i64) for n in ("k_src_ss", "k_src_sh", "v_src_ss", "v_src_sh")] + \
               [("dst_rows", vp), ("k_pool", vp), ("v_pool", vp), ("pool_ss", i64),
                ("pool_sh", i64)]


class HierFrameAttnArgs(C.Structure):
    _fields_ = [(n, i32) for n in ("B", "Lq", "Lk", "H", "D", "n_block", "local_attn")] + \
               [("scale", f32)] + [(n, vp) for n in ("q", "k", "v", "o")] + \
               [(n, i64) for n in ("q_sb", "q_ss", "q_sh", "k_sb", "k_ss", "k_sh", "v_sb", "v_ss",
                                   "v_sh", "o_sb", "o_ss", "o_sh")] + \
               [("q_frame", vp), ("k_frame", vp)]


class HierDeriveArgs(C.Structure):
    _fields_ = [(n, i32) for n in ("n_items", "n_groups", "rows", "nq_max", "kv_len", "P", "T",
                                   "L", "N", "KL")] + \
               [(n, vp) for n in ("items", "kv_idx", "kv_mask", "ws")] + \
               [("ws_bytes", i64), ("totals", vp), ("key_entries", i64), ("ste_entries", i64)] + \
               [(n, vp) for n in ("key_items", "key_q_idx", "key_q_mask", "key_blk_and",
                                  "ste_items", "ste_kv_idx", "ste_kv_mask", "ste_blk_and",
                                  "ste_kv_class")]


class HierGateArgs(C.Structure):
    _fields_ = [("rows", i64), ("dim", i32), ("rows_per_gate", i32)] + \
               [(n, vp) for n in ("x", "y", "gate", "out")] + \
               [(n, i64) for n in ("x_ss", "y_ss", "gate_ss", "out_ss")]


class HierSteReduceArgs(C.Structure):
    _fields_ = [(n, i32) for n in ("H", "P", "T", "L", "N", "KL", "classes")] + \
               [("partial", vp), ("stride_h", i64), ("out", vp)]


class HierMembershipArgs(C.Structure):
    _fields_ = [(n, i32) for n in ("T", "N", "P", "B", "n", "fl_max")] + \
               [(n, vp) for n in ("logits", "la_frame", "membership", "global_only", "q_active",
                                  "local_active")]


class HierPrologueBwdArgs(C.Structure):
    _fields_ = [("S", i32), ("H", i32), ("D", i32), ("eps", f32), ("C", i32),
                ("tokens_per_wave", i32)] + \
               [(n, vp) for n in ("qx", "kx", "cam", "w_cam_q", "w_cam_k", "norm_q_w", "norm_k_w",
                                  "rope_cos", "rope_sin", "dq", "dk")] + \
               [(n, i64) for n in ("dq_ss", "dq_sh", "dk_ss", "dk_sh")] + \
               [(n, vp) for n in ("dqx", "dkx", "dw_q_partial", "dw_k_partial")]


class HierMergeArgs(C.Structure):
    _fields_ = [(n, i32) for n in ("n_groups", "n_src", "rows", "rows_per_item")] + \
               [(n, vp) for n in ("items", "kv_idx", "kv_mask", "blk_and", "acc", "src_item",
                                  "src_group", "src_shift", "out_off", "out_cap", "group_desc",
                                  "group_item_off", "out_items", "src_from", "src_nbits")]


class HierTrimArgs(C.Structure):
    _fields_ = [("n_items", i32), ("reserved", i32)] + \
               [(n, vp) for n in ("items", "kv_mask", "row_table", "out_items")]


EXPORTS = {
    "hier_meta_count": [C.POINTER(HierTopo), C.POINTER(HierMetaCounts), vp],
    "hier_meta_build": [C.POINTER(HierTopo), C.POINTER(HierMetaOut), vp],
    "hier_derive_workspace": [C.POINTER(HierDeriveArgs)],
    "hier_derive_count": [C.POINTER(HierDeriveArgs), vp],
    "hier_derive_build": [C.POINTER(HierDeriveArgs), vp],
    "hier_derive_ste_classes": [C.POINTER(HierDeriveArgs), vp, vp, vp],
    "hier_membership_from_logits": [C.POINTER(HierMembershipArgs), vp],
    "hier_merge_hub_lists": [C.POINTER(HierMergeArgs), vp],
    "hier_trim_key_lists": [C.POINTER(HierTrimArgs), vp],
    "hier_qkv_prologue": [C.POINTER(HierPrologueArgs), vp],
    "hier_qk_prologue_bwd_waves": [C.POINTER(HierPrologueBwdArgs)],
    "hier_qk_prologue_bwd": [C.POINTER(HierPrologueBwdArgs), vp],
    "hier_attn_fwd": [C.POINTER(HierFwdArgs), vp],
    "hier_attn_bwd": [C.POINTER(HierBwdArgs), vp],
    "hier_attn_bwd_noalloc": [C.POINTER(HierBwdArgs), vp],
    "hier_ste_reduce": [C.POINTER(HierSteReduceArgs), vp],
    "hier_kv_append": [C.POINTER(HierPageArgs), vp],
    "hier_frame_attn": [C.POINTER(HierFrameAttnArgs), vp],
    "hier_gated_residual": [C.POINTER(HierGateArgs), vp],
    "hier_last_error": [],
    "hier_version": [],
}

_lock = threading.Lock()
_lib = None


def lib() -> C.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"hierattn HIP library not built: {LIB_PATH} is missing "
                    "(run `python -m multics_amd.build` or __graft_entry__.build())")
            handle = C.CDLL(str(LIB_PATH))
            for name, argtypes in EXPORTS.items():
                fn = getattr(handle, name)
                fn.argtypes = argtypes
                fn.restype = C.c_char_p if name in ("hier_last_error", "hier_version") else \
                    (C.c_int64 if name == "hier_derive_workspace" else C.c_int)
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc == HIER_OK:
        return
    msg = f"{what}: {lib().hier_last_error().decode(errors='replace')}"
    if rc == HIER_EINVAL:
        raise ValueError(msg)
    if rc == HIER_EUNSUPPORTED:
        raise NotImplementedError(msg)
    if rc == HIER_EINTERNAL:
        raise AssertionError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
