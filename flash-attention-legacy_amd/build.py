"""Build libfal_hip.so (the gfx950 attention library) in-tree with hipcc.

Usage:  python flash-attention-legacy_amd/build.py [--jobs N] [--verbose]

Replaces the reference's nvcc ``CUDAExtension`` build (setup.py:48-82): every
``csrc/*.hip`` file is compiled for ``--offload-arch=gfx950`` and linked into
``flash_attn_legacy/libfal_hip.so`` next to the Python package that loads it.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "flash_attn_legacy", "libfal_hip.so")
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-result",
    # No packed-fp32 VALU ops: keep fp32 arithmetic on the scalar-per-lane forms.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found (ROCm is required to build libfal_hip.so)")
    return exe


def _compile(src: str, verbose: bool, objdir: str = OBJ, defines=()) -> str:
    obj = os.path.join(objdir, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *[f"-D{d}" for d in defines], "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature name; that warning is harmless.
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{msgs}")
    if msgs.strip() and verbose:
        print(msgs)
    return obj


def build(jobs: int | None = None, verbose: bool = False, out: str = OUT, defines=()) -> str:
    """Compile and link; returns the path of the shared library.  `defines` are extra
    NAME=VALUE macros (kernel tunables); `out` is the library path to write."""
    # the pipelined forward and dK/dV loops are generated text (csrc/gen_*_pipe.py)
    sys.path.insert(0, CSRC)
    try:
        import gen_bwd_pipe
        import gen_dq_pipe
        import gen_fwd_pipe
        gen_fwd_pipe.main()
        gen_bwd_pipe.main()
        gen_dq_pipe.main()
    finally:
        sys.path.remove(CSRC)
    objdir = OBJ if not defines else os.path.join(OBJ, "_".join(defines).replace("=", "-"))
    os.makedirs(objdir, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, objdir, defines), srcs))
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    _check_stubs(tmp)
    os.replace(tmp, out)
    return out


def _check_stubs(lib: str) -> None:
    """Fail if a kernel's host launch stub is referenced but not defined: hipcc's host
    pass can drop a kernel instantiation without a diagnostic, which would only show
    up as a dlopen error on the GPU host."""
    nm = shutil.which("nm")
    if not nm:
        return
    r = subprocess.run([nm, "-D", "--undefined-only", lib], capture_output=True, text=True)
    missing = [l.split()[-1] for l in r.stdout.splitlines() if "__device_stub__" in l]
    if missing:
        raise RuntimeError(f"{lib}: undefined kernel stubs (host pass dropped them): {missing}")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--out", default=OUT, help="library path to write")
    ap.add_argument("-D", dest="defines", action="append", default=[], help="NAME=VALUE tunable macro")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose, a.out, tuple(a.defines)))
    return 0


if __name__ == "__main__":
    sys.exit(main())
