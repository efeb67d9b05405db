"""Builds the HIP library libburnext_moe.so (gfx950) in-tree: burn-extended_amd/lib/ (the MoE layer
and the GPT-OSS decoder step around it)."""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libburnext_moe.so"
SOURCES = ["kernels.hip", "gemm.hip", "fused.hip", "layer.hip", "decoder.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -packed-fp32-ops off: hipcc forms packed fp32 ops from plain float code on its own; they are
# kept out of every kernel here.  The host pass warns that it does not know the feature.
# atomic optimizer off: it turns the expert GEMV's single-lane ticket atomic into a wave-reduced
# one whose result is consumed at once, i.e. a full vmcnt(0) drain of the weight prefetch.
FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-mllvm", "-amdgpu-atomic-optimizer-strategy=None", "-Wall", "-Wno-unused-result"]


def build(verbose: bool = False) -> pathlib.Path:
    LIB_DIR.mkdir(exist_ok=True)
    objs = [str(LIB_DIR / (src.rsplit(".", 1)[0] + ".o")) for src in SOURCES]
    cmds = [[HIPCC, *FLAGS, "-c", str(CSRC / src), "-o", obj] for src, obj in zip(SOURCES, objs)]
    # the translation units compile independently: one hipcc process each
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(cmds)) as pool:
        for f in [pool.submit(_run, c, verbose) for c in cmds]:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "--offload-arch=gfx950", "-o", str(tmp), *objs, "-lpthread"], verbose)
    shutil.move(str(tmp), str(LIB))
    for o in objs:
        os.remove(o)
    build_checks(verbose)
    return LIB


# Test-only GPU programs (tests/native/*_check.hip, one executable each in lib/checks/): exhaustive
# checks of device helpers the library compiles in, run by the GPU tests.
CHECK_DIR = LIB_DIR / "checks"
CHECKS = ["bf16_convert_check"]


def build_checks(verbose: bool = False) -> list[pathlib.Path]:
    CHECK_DIR.mkdir(parents=True, exist_ok=True)
    out = []
    for name in CHECKS:
        exe = CHECK_DIR / name
        _run([HIPCC, *FLAGS, "-o", str(exe), str(PKG.parent / "tests" / "native" / f"{name}.hip")], verbose)
        out.append(exe)
    return out


# Host-side sanitizers for build_asan: every -fsanitize option is given to the host half of the
# compile only (device code is built as for the library).
ASAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-Xarch_host",
             "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer", "-g"]
ASAN_DIR = LIB_DIR / "asan"
ASAN_EXE = ASAN_DIR / "asan_host"
ASAN_DRIVER = PKG.parent / "tests" / "native" / "asan_host.cpp"


def build_asan(verbose: bool = False, force: bool = False) -> pathlib.Path:
    """The library sources with AddressSanitizer + UndefinedBehaviorSanitizer on the host code, linked
    into the driver tests/native/asan_host.cpp (lib/asan/asan_host).  Skipped when the executable is
    newer than every source unless `force`."""
    srcs = [CSRC / f for f in SOURCES] + [ASAN_DRIVER]
    deps = srcs + list(CSRC.glob("*.hpp")) + list((PKG.parent / "include").glob("*.h"))
    if not force and ASAN_EXE.exists() and ASAN_EXE.stat().st_mtime > max(d.stat().st_mtime for d in deps):
        return ASAN_EXE
    ASAN_DIR.mkdir(parents=True, exist_ok=True)
    objs = [str(ASAN_DIR / (pathlib.Path(f).stem + ".o")) for f in srcs]
    inc = ["-I", str(PKG.parent / "include")]
    cmds = [[HIPCC, *FLAGS, *ASAN_HOST, *inc, "-c", str(src), "-o", obj] for src, obj in zip(srcs, objs)]
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(cmds)) as pool:
        for f in [pool.submit(_run, c, verbose) for c in cmds]:
            f.result()
    tmp = ASAN_EXE.with_suffix(".tmp")
    _run([HIPCC, "--offload-arch=gfx950", *ASAN_HOST, "-o", str(tmp), *objs, "-lpthread"], verbose)
    shutil.move(str(tmp), str(ASAN_EXE))
    for o in objs:
        os.remove(o)
    return ASAN_EXE


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


if __name__ == "__main__":
    print(build(verbose=True))
