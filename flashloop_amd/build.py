"""Build ``libflashloop_amd.so`` (gfx950) from ``flashloop_amd/csrc`` with hipcc.

Usage: ``python -m flashloop_amd.build`` (or ``build()`` from Python).  The shared
library is written next to this file so it travels with the source tree.  Each
``.hip`` file is compiled to an object in ``flashloop_amd/_build`` (in parallel) and
linked once.  Every build recompiles.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libflashloop_amd.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    # Packed FP32 (v_pk_*_f32) forms are disabled: only scalar FP32 VALU ops are emitted.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{PKG.parent / 'include'}",
]
# the codec must never contract a*b+c into an FMA: its reference rounds each op; the
# top-k's softmax weight image is reproduced bit for bit on the CPU
PER_FILE_FLAGS = {"pack.hip": ["-ffp-contract=off"], "topk.hip": ["-ffp-contract=off"]}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build flashloop_amd)")


def _compile(src: Path, hipcc: str, extra: list[str]) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc, *COMMON_FLAGS, *PER_FILE_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    warn = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if warn.strip():
        print(f"[flashloop_amd.build] {src.name}:\n{warn}", file=sys.stderr)
    return obj


# Extra hipcc flags a caller may add: diagnostics only, none changes the generated code.
ALLOWED_EXTRA_FLAGS = frozenset({"-Rpass-analysis=kernel-resource-usage", "-save-temps"})


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    hipcc = _hipcc()
    extra = list(extra_flags or [])
    bad = [f for f in extra if f not in ALLOWED_EXTRA_FLAGS]
    if bad:
        raise ValueError(f"flags not allowed in the library build: {bad} (allowed: {sorted(ALLOWED_EXTRA_FLAGS)})")
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc, extra), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[flashloop_amd.build] wrote {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True, extra_flags=sys.argv[1:])
