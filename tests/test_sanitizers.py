"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

* The oracle (oracle/gdn2_oracle.c) rebuilt by gcc with
  -fsanitize=address,undefined -fno-sanitize-recover=all: its own tests
  (closed forms, golden vectors, finite differences) run against that build in
  a child process with libasan preloaded, and must pass with no report.
* The library's host code (the C ABI's argument checks, Gdn2Config, shape
  algebra, the seeded parameter initialisers, the workspace sizing) rebuilt
  by hipcc with the same sanitizers on the host side only (-Xarch_host; the
  GPU code is compiled as usual and not run here): the host-only tests run
  against it in a child process with clang's ASan runtime preloaded.

Python itself is not instrumented, so leak checking is off (the interpreter's
own allocations would be reported)."""
import glob
import importlib.util
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "burn-gdn2_amd")
SAN = ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]
ENV = {"ASAN_OPTIONS": "detect_leaks=0:verify_asan_link_order=0:abort_on_error=0",
       "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}

# The child: point the loader at the sanitized build, then run the given test files.
CHILD = """
import sys
sys.path[:0] = [{root!r}, {pkg!r}, {tests!r}]
which, path = sys.argv[1], sys.argv[2]
if which == "oracle":
    from oracle import oracle
    oracle._LIB_PATH = path
else:
    from gdn2_amd import _capi
    _capi.LIB_PATH = path
import pytest
sys.exit(pytest.main(["-q", "-p", "no:cacheprovider", "-m", "not gpu"] + sys.argv[3:]))
"""


def _run_child(which, lib, preload, tests):
    code = CHILD.format(root=ROOT, pkg=PKG, tests=os.path.join(ROOT, "tests"))
    env = dict(os.environ, LD_PRELOAD=preload, **ENV)
    r = subprocess.run([sys.executable, "-c", code, which, lib] + [os.path.join(ROOT, "tests", t) for t in tests],
                       env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    return out


def test_oracle_under_asan_ubsan(tmp_path):
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("no gcc")
    asan = subprocess.run([cc, "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(asan) or not os.path.exists(asan):
        pytest.skip("gcc has no libasan")
    lib = str(tmp_path / "libgdn2_oracle_san.so")
    subprocess.run([cc, "-O1", "-g", "-fopenmp", "-fPIC", "-shared"] + SAN +
                   [os.path.join(ROOT, "oracle", "gdn2_oracle.c"), "-o", lib, "-lm"], check=True)
    out = _run_child("oracle", lib, asan, ["test_oracle.py", "test_oracle_bwd.py", "test_oracle_layer_bwd.py"])
    assert " passed" in out and " failed" not in out


def test_library_host_code_under_asan_ubsan(tmp_path):
    rts = glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")
    spec = importlib.util.spec_from_file_location("gdn2_amd_build", os.path.join(PKG, "build.py"))
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    if not rts or not os.path.exists(b.HIPCC):
        pytest.skip("no hipcc / clang ASan runtime")
    flags = [("-O1" if f == "-O3" else f) for f in b.FLAGS] + ["-g"]
    for f in SAN:
        flags += ["-Xarch_host", f]
    lib = str(tmp_path / "libgdn2_amd_san.so")
    r = subprocess.run([b.HIPCC] + flags + b.sources() + ["-o", lib] + b.LIBS, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    out = _run_child("library", lib, rts[0], ["test_layer_host.py", "test_capi_exports.py"])
    assert " passed" in out and " failed" not in out
