"""AddressSanitizer over the C ABI's host code (CPU only): the library's argument checks, size
queries and error reporting (gdn_api.hip, gdn_norm.hip, gdn_decode.hip) built with ASan on the
host side (-Xarch_host -fsanitize=address; the GPU code is not instrumented) into a driver that
calls every entry point with bad, null, misaligned, unsupported and edge-case arguments
(tests/asan/abi_driver.hip). Nothing reaches a launch, so no GPU is needed. The kernel tables
are stand-ins without kernels (tests/asan/tables_stub.hip)."""

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_c_abi_host_code_under_asan(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    csrc = ROOT / "tjev_amd" / "csrc"
    exe = tmp_path / "abi_asan"
    cmd = [hipcc, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fno-omit-frame-pointer",
           "-Xarch_host", "-fsanitize=address", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           str(csrc / "gdn_api.hip"), str(csrc / "gdn_norm.hip"), str(csrc / "gdn_decode.hip"),
           str(ROOT / "tests" / "asan" / "tables_stub.hip"), str(ROOT / "tests" / "asan" / "abi_driver.hip"),
           "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    if build.returncode:
        err = "\n".join(l for l in build.stderr.splitlines() if "not a recognized feature" not in l)
        pytest.fail(f"ASan build failed:\n{err[-4000:]}")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:halt_on_error=1:exitcode=86")
    run = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    out = run.stdout + run.stderr
    assert "ERROR: AddressSanitizer" not in out, out[-4000:]
    assert run.returncode == 0, out[-4000:]
    assert "0 mismatches" in run.stdout
