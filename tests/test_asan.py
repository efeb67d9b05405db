"""Sanitizer runs on the CPU (AddressSanitizer + UndefinedBehaviorSanitizer, leaks included for the
oracle):

* the oracle: `make -C oracle asan` builds oracle/moe_oracle.c + oracle/decoder_oracle.c with the
  driver oracle/asan_oracle_main.c, which calls every entry point on small and ragged shapes;
* the library's host code: `build.build_asan()` builds the HIP sources with the sanitizers on their
  host half and links tests/native/asan_host.cpp, which drives the public C ABI.  Without a HIP
  device it covers every create's host preparation (MXFP4 repack, bias permutation, gamma folding,
  dense tiling, RoPE table) and the argument checks; with one, every entry point.
"""
import os
import pathlib
import shutil
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent


def _env(leaks: bool):
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = f"detect_leaks={1 if leaks else 0}:abort_on_error=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1"
    return env


def test_oracle_under_asan():
    if shutil.which("gcc") is None or shutil.which("make") is None:
        pytest.skip("gcc / make not available")
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "asan"], check=True, capture_output=True)
    r = subprocess.run([str(ROOT / "oracle" / "_build" / "oracle_asan")], capture_output=True, text=True,
                       env=_env(True), timeout=600)
    assert r.returncode == 0 and "asan oracle ok" in r.stdout, r.stderr[-4000:]
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]


def test_host_library_under_asan():
    sys.path.insert(0, str(ROOT / "burn-extended_amd"))
    import build
    if not pathlib.Path(build.HIPCC).exists():
        pytest.skip("hipcc not available")
    exe = build.build_asan()
    # the HIP runtime keeps allocations until exit: leaks are not checked here
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=_env(False), timeout=900)
    assert r.returncode == 0 and "asan host ok" in r.stdout, (r.stdout[-2000:], r.stderr[-4000:])
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
