#!/usr/bin/env python3
"""Build libgdn2_amd.so for gfx950 in-tree (burn-gdn2_amd/libgdn2_amd.so).

Each source in csrc/ is compiled by its own hipcc (in parallel), then the
objects are linked.  Flags:
  --offload-arch=gfx950       MI355X only
  -packed-fp32-ops (disabled) no v_pk_*_f32 generation: some packed-FP32 forms
                              have given wrong results without an error on this
                              hardware, so hipcc must not emit them
"""
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
OUT = os.path.join(HERE, "libgdn2_amd.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden",
    "-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc"),
]
LIBS = ["-L/opt/rocm/lib", "-lhipblaslt", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib"]


def sources():
    return sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")) + glob.glob(os.path.join(HERE, "csrc", "*.cpp")))


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd))
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l]
    return r.returncode, msgs


def build(verbose=False, jobs=None):
    """Compiles every source to an object in _build/ (in parallel, one hipcc
    per source), then links the shared library."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    compile_flags = [f for f in FLAGS if f != "-shared"]
    srcs = sources()
    objs = [os.path.join(objdir, os.path.basename(src) + ".o") for src in srcs]
    jobs = jobs or max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(lambda so: _run([HIPCC] + compile_flags + ["-c", so[0], "-o", so[1]], verbose),
                              zip(srcs, objs)))
    failed = [(src, msgs) for src, (rc, msgs) in zip(srcs, results) if rc != 0]
    for src, msgs in failed:
        sys.stderr.write(f"{src}:\n" + "\n".join(msgs) + "\n")
    if failed:
        raise RuntimeError("hipcc failed building libgdn2_amd.so")
    tmp = OUT + ".tmp"
    rc, msgs = _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + objs + ["-o", tmp] + LIBS, verbose)
    if rc != 0:
        sys.stderr.write("\n".join(msgs) + "\n")
        raise RuntimeError("linking libgdn2_amd.so failed")
    if verbose:
        for _, (_, msgs) in zip(srcs, results):
            if msgs:
                print("\n".join(msgs))
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
