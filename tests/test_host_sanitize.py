"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU only, no kernel launch).

Every ``multics_amd/csrc/*.hip`` file is compiled with the sanitizers on its
host pass only (the device code is built as usual and never runs), linked
with ``tests/sanitize/host_checks.cpp``, and run.  The driver calls every
entry point of ``include/hierattn.h`` with hostile arguments -- NULL and
misaligned pointers, negative, huge and overflowing sizes and strides -- and
with valid arguments describing empty work, and sizes the derive workspace
over a grid of shapes.  Each call must return its documented code without a
sanitizer report (a signed overflow, an out-of-bounds host access, a host
read of a device pointer).  The driver refuses to run when a GPU is visible:
its device pointers are stand-ins.
"""

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "multics_amd" / "csrc"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = ROCM / "bin" / "hipcc"
CLANG = ROCM / "llvm" / "bin" / "clang++"

pytestmark = pytest.mark.skipif(
    not (HIPCC.exists() and CLANG.exists()) or Path("/dev/kfd").exists(),
    reason="needs hipcc and clang++, and no visible GPU (the checks use stand-in device pointers)")


def _compile(src: Path, out: Path):
    cmd = [str(HIPCC), "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fno-gpu-sanitize",
           "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=undefined",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           f"-I{ROOT / 'include'}", f"-I{CSRC}", "-c", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-4000:]
    return out


def test_host_entry_points_under_sanitizers(tmp_path):
    sources = sorted(CSRC.glob("*.hip"))
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda s: _compile(s, tmp_path / (s.stem + ".o")), sources))
    drv = tmp_path / "host_checks.o"
    subprocess.run([str(CLANG), "-O1", "-g", "-std=c++17", f"-I{ROOT / 'include'}",
                    "-Xarch_host", "-fsanitize=address", "-c",
                    str(ROOT / "tests" / "sanitize" / "host_checks.cpp"), "-o", str(drv)],
                   check=True, capture_output=True)
    exe = tmp_path / "host_checks"
    link = [str(CLANG), "-fsanitize=address,undefined", *map(str, objs), str(drv),
            f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}", "-o", str(exe)]
    res = subprocess.run(link, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    run = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    report = run.stdout + run.stderr
    assert "runtime error" not in report and "AddressSanitizer" not in report, report[-6000:]
    assert run.returncode == 0 and "host checks done: 0 failed" in run.stdout, report[-6000:]
