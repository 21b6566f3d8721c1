"""The build is deterministic and has no side effects on tracked sources.

* The generated asm loops (csrc/gen/*.inc) are rendered from their generators with
  fixed default knobs; no environment variable changes that text, and the default
  build only checks the tracked files, it never rewrites them.
* Generator knobs and ablations reach a build only as explicit build.py arguments,
  ablations only with --measure, and such a variant build must write a library of
  its own, never the product library.
"""

import json
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "flash-attention-legacy_amd")
CSRC = os.path.join(PKG, "csrc")

# every FAL_* variable an earlier build or a generator ever consulted, set to values
# that would change the kernel (or break it) if they were read
HOSTILE_ENV = {
    "FAL_PIPE_MEASURE": "1", "FAL_PIPE_ABL": "nodma,nobar,novalu", "FAL_PIPE_DEBUG": "CYC",
    "FAL_PIPE_KDIST": "3", "FAL_PIPE_VRING": "5", "FAL_PIPE_VDIST": "2", "FAL_PIPE_DMA_AUX": " nt",
    "FAL_PIPE_GSTRIDE": "2", "FAL_BWDP_MEASURE": "1", "FAL_BWDP_ABL": "noa,nob",
    "FAL_BWDP_ADIST": "3", "FAL_BWDP_BDIST": "8", "FAL_DQP_ADIST": "2", "FAL_DQP_QDIST": "8",
}

_RENDER = r"""
import hashlib, json, sys
sys.path.insert(0, sys.argv[1])
import gen_fwd_pipe, gen_bwd_pipe, gen_dq_pipe
print(json.dumps({m.__name__: hashlib.sha256(m.render().encode()).hexdigest()
                  for m in (gen_fwd_pipe, gen_bwd_pipe, gen_dq_pipe)}))
"""


def _digests(env):
    r = subprocess.run([sys.executable, "-c", _RENDER, CSRC], env=env, capture_output=True,
                       text=True, check=True)
    return json.loads(r.stdout)


def _tracked_digests():
    import hashlib
    return {f"gen_{n}_pipe": hashlib.sha256(open(os.path.join(CSRC, "gen", f"fal_{n}_pipe.inc"), "rb")
                                            .read()).hexdigest() for n in ("fwd", "bwd", "dq")}


def test_generated_loops_match_their_generators():
    assert _digests(dict(os.environ)) == _tracked_digests()


def test_environment_does_not_reach_the_generated_loops():
    env = {k: v for k, v in os.environ.items() if not k.startswith("FAL_")}
    env.update(HOSTILE_ENV)
    assert _digests(env) == _tracked_digests()


def test_no_source_reads_the_environment():
    # the C++ sources see macros only through build.py's explicit -D arguments
    for name in os.listdir(CSRC):
        path = os.path.join(CSRC, name)
        if os.path.isfile(path) and name.endswith((".py", ".hip", ".h")):
            text = open(path).read()
            text = re.sub(r'""".*?"""', "", text, flags=re.S)   # docstrings may mention it
            assert "os.environ" not in text and "getenv" not in text, name


def _build_mod():
    sys.path.insert(0, PKG)
    try:
        import build
        return build
    finally:
        sys.path.remove(PKG)


def test_default_check_never_rewrites_tracked_files(tmp_path, monkeypatch):
    b = _build_mod()
    gen = tmp_path / "gen"
    gen.mkdir()
    for _, inc in b.GENERATORS:
        (gen / inc).write_text(open(os.path.join(b.GEN_DIR, inc)).read())
    monkeypatch.setattr(b, "GEN_DIR", str(gen))
    b.check_generated()                       # identical: passes
    stale = gen / "fal_fwd_pipe.inc"
    stale.write_text(stale.read_text() + "// stale\n")
    with pytest.raises(RuntimeError, match="--regen"):
        b.check_generated()
    assert stale.read_text().endswith("// stale\n")   # not rewritten
    b.check_generated(regen=True)
    assert stale.read_text() == open(os.path.join(PKG, "csrc", "gen", "fal_fwd_pipe.inc")).read()


def test_variant_builds_need_their_own_library_and_measure_for_ablations():
    b = _build_mod()
    for kw in ({"defines": ("FAL_FWD_GQA4=0",)}, {"knobs": ("fwd.KDIST=3",)}, {"measure": True}):
        with pytest.raises(ValueError, match="--out"):
            b.build(**kw)
    sys.path.insert(0, CSRC)
    try:
        import gen_bwd_pipe
        import gen_fwd_pipe
    finally:
        sys.path.remove(CSRC)
    with pytest.raises(ValueError, match="measurement"):
        gen_fwd_pipe.render({"ABL": "nodma"})
    with pytest.raises(ValueError, match="unknown"):
        gen_bwd_pipe.render({"DEBUG": "CYC"})
    assert gen_fwd_pipe.render({"ABL": "nodma"}, measure=True) != gen_fwd_pipe.render()
    # rendering a variant leaves the module on its defaults
    assert gen_fwd_pipe.KDIST == gen_fwd_pipe.DEFAULTS["KDIST"] and not gen_fwd_pipe.ABL
    with pytest.raises(ValueError, match="fwd.NAME"):
        b._parse_knobs(["KDIST=3"])
