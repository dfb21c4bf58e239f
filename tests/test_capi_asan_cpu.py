"""Host sanitizer build of the C ABI's validation and dispatch (CPU only).

csrc/capi.cpp is compiled for the host alone with AddressSanitizer and
UndefinedBehaviorSanitizer (each -fsanitize= behind -Xarch_host, so no device
code is built with them) and linked with tests/asan/capi_driver.cpp, whose
recorders stand in for the kernel launchers.  The driver runs the bad-argument
cases of test_capi_cpu.py through every entry point and checks which
launchers valid problems reach; any out-of-bounds access, leak, overflow or
other undefined behaviour aborts it."""

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "triton-sigmoid_amd" / "csrc"
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=all"]


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_capi_under_address_and_ub_sanitizers(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    common = ["-x", "hip", "--cuda-host-only", "-std=c++17", "-O1", "-g", *SAN,
              f"-I{CSRC}", f"-I{ROOT / 'include'}"]
    objs = []
    for src in (CSRC / "capi.cpp", ROOT / "tests" / "asan" / "capi_driver.cpp"):
        obj = tmp_path / (src.stem + ".o")
        subprocess.run([hipcc, *common, "-c", str(src), "-o", str(obj)], check=True, capture_output=True)
        objs.append(str(obj))
    exe = tmp_path / "capi_driver"
    subprocess.run([hipcc, *SAN, *objs, "-o", str(exe)], check=True, capture_output=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    res = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "all checks passed" in res.stdout
    assert "Sanitizer" not in res.stderr, res.stderr
