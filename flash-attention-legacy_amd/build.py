"""Build libfal_hip.so (the gfx950 attention library) in-tree with hipcc.

Usage:  python flash-attention-legacy_amd/build.py [--jobs N] [--verbose] [--regen]
        python flash-attention-legacy_amd/build.py --out X.so [-D NAME=VALUE] [--knob fwd.KDIST=3] [--measure]

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


def _compile(src: str, verbose: bool, objdir: str = OBJ, flags=()) -> str:
    obj = os.path.join(objdir, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *flags, "-c", src, "-o", obj]
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


GENERATORS = (("gen_fwd_pipe", "fal_fwd_pipe.inc"), ("gen_bwd_pipe", "fal_bwd_pipe.inc"),
              ("gen_dq_pipe", "fal_dq_pipe.inc"))
GEN_DIR = os.path.join(CSRC, "gen")     # the tracked generated asm loops


def _generators():
    sys.path.insert(0, CSRC)
    try:
        import importlib
        return {name: importlib.import_module(name) for name, _ in GENERATORS}
    finally:
        sys.path.remove(CSRC)


def check_generated(regen: bool = False) -> None:
    """The tracked csrc/gen/*.inc must equal what the generators render with their
    default knobs.  A mismatch is an error (nothing is rewritten) unless `regen`."""
    mods = _generators()
    for name, inc in GENERATORS:
        path = os.path.join(GEN_DIR, inc)
        text = mods[name].render()
        old = open(path).read() if os.path.exists(path) else None
        if old == text:
            continue
        if not regen:
            raise RuntimeError(f"{path} differs from {name}.py's output; run build.py --regen "
                               "after changing a generator")
        with open(path, "w") as f:
            f.write(text)


def _parse_knobs(knobs) -> dict:
    """['fwd.KDIST=3', 'bwd.ABL=nob'] -> {'gen_fwd_pipe': {'KDIST': '3'}, ...}"""
    out: dict = {}
    short = {"fwd": "gen_fwd_pipe", "bwd": "gen_bwd_pipe", "dq": "gen_dq_pipe"}
    for kv in knobs:
        key, _, val = kv.partition("=")
        gen, _, name = key.partition(".")
        if gen not in short or not name or not _:
            raise ValueError(f"knob {kv!r}: expected fwd.NAME=VALUE, bwd.NAME=VALUE or dq.NAME=VALUE")
        out.setdefault(short[gen], {})[name] = val
    return out


def build(jobs: int | None = None, verbose: bool = False, out: str = OUT, defines=(), knobs=(),
          measure: bool = False, regen: bool = False) -> str:
    """Compile and link; returns the path of the shared library.

    The default build reads nothing from the environment: it compiles csrc/*.hip with the
    tracked generated loops (csrc/gen/) and fails if those differ from their generators.
    `defines` (NAME=VALUE C++ tunables) and `knobs` (generator knobs, fwd.NAME=VALUE ...)
    make a variant build; `measure` also admits the ablation knobs, whose results are
    wrong.  A variant build must name its own `out`, so it never replaces the product
    library, and its generated loops go to its own folder under _build/."""
    variant = bool(defines or knobs or measure)
    if variant and os.path.abspath(out) == os.path.abspath(OUT):
        raise ValueError("a build with -D/--knob/--measure must write its own library (--out)")
    check_generated(regen)
    tag = "_".join([*defines, *knobs] + (["measure"] if measure else [])).replace("=", "-").replace(",", "+")
    objdir = OBJ if not variant else os.path.join(OBJ, tag or "variant")
    os.makedirs(objdir, exist_ok=True)
    gen_dir = GEN_DIR
    if knobs or measure:
        gen_dir = os.path.join(objdir, "gen")
        os.makedirs(gen_dir, exist_ok=True)
        mods, kn = _generators(), _parse_knobs(knobs)
        for name, inc in GENERATORS:
            with open(os.path.join(gen_dir, inc), "w") as f:
                f.write(mods[name].render(kn.get(name), measure=measure))
    flags = [f"-I{gen_dir}", *[f"-D{d}" for d in defines]]
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, objdir, flags), srcs))
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
    ap.add_argument("--knob", dest="knobs", action="append", default=[],
                    help="generator knob: fwd.NAME=VALUE, bwd.NAME=VALUE or dq.NAME=VALUE")
    ap.add_argument("--measure", action="store_true",
                    help="admit ablation knobs (timing-only builds whose results are wrong)")
    ap.add_argument("--regen", action="store_true",
                    help="rewrite the tracked csrc/gen/*.inc from the generators")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose, a.out, tuple(a.defines), tuple(a.knobs), a.measure, a.regen))
    return 0


if __name__ == "__main__":
    sys.exit(main())
