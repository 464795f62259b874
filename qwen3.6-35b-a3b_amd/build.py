"""Build libmoe_gfx950.so from csrc/*.hip with hipcc for gfx950 (in-tree; no cmake, no JIT cache).

`build()` always recompiles. Objects go to csrc/_build/ (git-ignored); the shared library lands
next to this file so the package loads it from its own directory.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libmoe_gfx950.so"
ARCH = os.environ.get("MOE_GPU_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# Packed-FP32 instructions are disabled for all device code; the host pass only warns about it.
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _compile(src: Path, obj: Path) -> tuple[Path, int, str]:
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    return src, p.returncode, (p.stdout + p.stderr)


def build(verbose: bool = False) -> Path:
    srcs = sorted(CSRC.glob("*.hip"))
    bdir = CSRC / "_build"
    bdir.mkdir(exist_ok=True)
    objs = [bdir / (s.stem + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = list(ex.map(lambda so: _compile(*so), zip(srcs, objs)))
    failed = [(s, log) for s, rc, log in results if rc != 0]
    for s, rc, log in results:
        if verbose or rc != 0:
            noisy = [l for l in log.splitlines() if "packed-fp32-ops" not in l and l.strip()]
            if noisy:
                print(f"--- {s.name}\n" + "\n".join(noisy), file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed for: " + ", ".join(s.name for s, _ in failed))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("link failed:\n" + p.stdout + p.stderr)
    os.replace(tmp, OUT)
    build_hostcheck()
    build_probe()
    return OUT


PROBE = PKG / "libmoe_peak_probe.so"


def build_probe() -> Path:
    """libmoe_peak_probe.so: the HBM read and f16 MFMA peak probes bench.py reports beside the
    published peaks (csrc/probe/). Measurement infrastructure; the MoE library does not link it."""
    src = CSRC / "probe" / "peak_probe.hip"
    tmp = PROBE.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, "-shared", "-o", str(tmp), str(src)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("peak probe build failed:\n" + p.stdout + p.stderr)
    os.replace(tmp, PROBE)
    return PROBE


HOSTCHECK = PKG / "libmoe_hostcheck.so"


def build_hostcheck() -> Path:
    """libmoe_hostcheck.so: host-callable builds of device helpers (csrc/hostcheck/) that the CPU
    tests check without a GPU. Test infrastructure; the product library does not link it."""
    src = CSRC / "hostcheck" / "hostcheck.hip"
    tmp = HOSTCHECK.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, "-shared", "-o", str(tmp), str(src)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("hostcheck build failed:\n" + p.stdout + p.stderr)
    os.replace(tmp, HOSTCHECK)
    return HOSTCHECK


ASAN_LIB = PKG / "libmoe_gfx950_asan.so"


def asan_runtime() -> Path:
    """The ROCm clang's AddressSanitizer runtime (to preload into a process that loads ASAN_LIB)."""
    clang = Path(HIPCC).resolve().parent.parent / "llvm" / "bin" / "clang"
    p = subprocess.run([str(clang) if clang.exists() else "clang",
                        "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    return Path(p.stdout.strip())


def build_asan() -> Path:
    """libmoe_gfx950_asan.so: the library with abi.hip (every entry point's argument checks and
    workspace carving) compiled for the host with AddressSanitizer, linked with the other objects
    of build(). Test infrastructure for the CPU tier; the device code is the same as the product's."""
    bdir = CSRC / "_build"
    others = [bdir / (s.stem + ".o") for s in sorted(CSRC.glob("*.hip")) if s.stem != "abi"]
    if not all(o.exists() for o in others):
        build()
    obj = bdir / "abi_asan.o"
    cmd = [HIPCC, *FLAGS, "-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host",
           "-fno-omit-frame-pointer", "-c", str(CSRC / "abi.hip"), "-o", str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("asan compile failed:\n" + p.stdout + p.stderr)
    tmp = ASAN_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address",
           "-shared-libasan", "-o", str(tmp), *map(str, others), str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("asan link failed:\n" + p.stdout + p.stderr)
    os.replace(tmp, ASAN_LIB)
    return ASAN_LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
