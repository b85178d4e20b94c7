"""The C-ABI library: it loads, exports every symbol the header declares, and
the ctypes structures have the C compiler's layout (no compute calls)."""

import ctypes as C
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from multics_amd import _capi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "hierattn.h"
STRUCTS = {
    "HierTopo": _capi.HierTopo,
    "HierMetaCounts": _capi.HierMetaCounts,
    "HierMetaOut": _capi.HierMetaOut,
    "HierPrologueArgs": _capi.HierPrologueArgs,
    "HierFwdArgs": _capi.HierFwdArgs,
    "HierBwdArgs": _capi.HierBwdArgs,
    "HierPageArgs": _capi.HierPageArgs,
    "HierFrameAttnArgs": _capi.HierFrameAttnArgs,
    "HierDeriveArgs": _capi.HierDeriveArgs,
    "HierGateArgs": _capi.HierGateArgs,
    "HierSteReduceArgs": _capi.HierSteReduceArgs,
    "HierMembershipArgs": _capi.HierMembershipArgs,
    "HierPrologueBwdArgs": _capi.HierPrologueBwdArgs,
    "HierMergeArgs": _capi.HierMergeArgs,
    "HierTrimArgs": _capi.HierTrimArgs,
}


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(hier_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _capi.lib()
    names = declared_functions()
    assert names, "no declarations parsed"
    assert set(names) == set(_capi.EXPORTS), names
    for name in names:
        assert hasattr(lib, name), name
    assert lib.hier_version().startswith(b"hierattn")
    assert lib.hier_last_error() == b""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_ctypes_struct_layout_matches_c(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "hierattn.h"', 'int main(void){']
    for sname, cls in STRUCTS.items():
        lines.append(f'printf("{sname} size %zu\\n", sizeof({sname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{sname} {fname} %zu\\n", offsetof({sname}, {fname}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        sname, field, val = line.split()
        got[(sname, field)] = int(val)
    for sname, cls in STRUCTS.items():
        assert got[(sname, "size")] == C.sizeof(cls), sname
        for fname, _ in cls._fields_:
            assert got[(sname, fname)] == getattr(cls, fname).offset, (sname, fname)


def test_error_codes_map_to_reference_exception_types():
    with pytest.raises(ValueError):
        _capi.check(_capi.HIER_EINVAL, "x")
    with pytest.raises(NotImplementedError):
        _capi.check(_capi.HIER_EUNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _capi.check(_capi.HIER_ELAUNCH, "x")
    with pytest.raises(AssertionError):
        _capi.check(_capi.HIER_EINTERNAL, "x")
    _capi.check(_capi.HIER_OK, "x")


def test_null_arguments_are_rejected_without_a_gpu():
    lib = _capi.lib()
    assert lib.hier_attn_fwd(None, None) == _capi.HIER_EINVAL
    assert b"NULL" in lib.hier_last_error()
    assert lib.hier_qkv_prologue(None, None) == _capi.HIER_EINVAL
    assert lib.hier_meta_count(None, None, None) == _capi.HIER_EINVAL
    assert lib.hier_meta_build(None, None, None) == _capi.HIER_EINVAL
    assert lib.hier_kv_append(None, None) == _capi.HIER_EINVAL
    assert lib.hier_frame_attn(None, None) == _capi.HIER_EINVAL


def test_frame_attention_argument_checks_without_a_gpu():
    """Invalid shapes are refused and an empty batch returns before any
    launch (nothing here is dereferenced)."""
    lib = _capi.lib()
    fake = 1 << 20
    a = _capi.HierFrameAttnArgs(B=0, Lq=3, Lk=24, H=2, D=128, n_block=3, local_attn=21,
                                scale=0.088, q=fake, k=fake, v=fake, o=fake, q_frame=fake,
                                k_frame=fake)
    assert lib.hier_frame_attn(C.byref(a), None) == _capi.HIER_OK
    a.D = 96
    assert lib.hier_frame_attn(C.byref(a), None) == _capi.HIER_EUNSUPPORTED
    a.D, a.local_attn = 128, 0
    assert lib.hier_frame_attn(C.byref(a), None) == _capi.HIER_EINVAL
    a.local_attn, a.n_block = 21, 0
    assert lib.hier_frame_attn(C.byref(a), None) == _capi.HIER_EINVAL


def test_forward_rejects_views_past_the_24_bit_row_limit_without_a_gpu():
    """The tile copies address rows with a 24 x 24-bit multiply: more than 2^24
    K/V rows is refused before anything is launched (n_items = 0 here, so no
    kernel could run even if the check were missing)."""
    lib = _capi.lib()
    fake = 1 << 20   # 16-byte aligned, never dereferenced
    a = _capi.HierFwdArgs(H=1, D=64, n_items=0, scale=0.125, kv_rows=(1 << 24) + 1,
                          q=fake, k=fake, v=fake, o=fake, q_ss=64, q_sh=64, k_ss=64, k_sh=64,
                          v_ss=64, v_sh=64, o_ss=64, o_sh=64, tile_items=fake, tile_kv_idx=fake,
                          tile_kv_mask=fake, tile_blk_and=fake)
    assert lib.hier_attn_fwd(C.byref(a), None) == _capi.HIER_EUNSUPPORTED
    assert b"2^24" in lib.hier_last_error()
    a.kv_rows = 1 << 24
    assert lib.hier_attn_fwd(C.byref(a), None) == _capi.HIER_OK
