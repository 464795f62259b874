"""The host-side refusals under AddressSanitizer (no GPU): abi.hip, where every entry point checks
its arguments and carves the workspace, is built for the host with -fsanitize=address
(build.build_asan); a child Python with the ASan runtime preloaded binds that library and makes
the refusal calls of test_abi_cpu through ctypes. It must finish cleanly with no ASan report."""
import importlib.util
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]

CHILD = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[2]); sys.path.insert(0, sys.argv[2] + "/tests")
import __graft_entry__ as ge
pkg = ge.load_package()
L = pkg._lib
lib = ctypes.CDLL(sys.argv[1])
for name, (res, args) in L.SIGNATURES.items():
    fn = getattr(lib, name); fn.restype = res; fn.argtypes = args
L.lib = lib
import test_abi_cpu as T
T.test_refusals_happen_on_the_host(pkg)
T.test_abi_version_and_enums_match_header(pkg)
T.test_workspace_bytes_is_monotone(pkg)
print("asan child ok", flush=True)
"""


def _build_module():
    spec = importlib.util.spec_from_file_location("_moe_build", ROOT / "qwen3.6-35b-a3b_amd" / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    return b


def test_refusals_under_asan():
    b = _build_module()
    lib = b.build_asan()
    nm = subprocess.run(["nm", "-D", str(lib)], capture_output=True, text=True).stdout
    assert "__asan_report" in nm, "abi.hip's host code is not instrumented"
    rt = b.asan_runtime()
    assert rt.is_file(), f"no ASan runtime at {rt}"
    env = dict(os.environ, LD_PRELOAD=str(rt), ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    p = subprocess.run([sys.executable, "-c", CHILD, str(lib), str(ROOT)], capture_output=True,
                       text=True, env=env, timeout=300)
    report = p.stdout[-2000:] + p.stderr[-4000:]
    assert "AddressSanitizer" not in p.stderr, report
    assert p.returncode == 0 and "asan child ok" in p.stdout, report
