"""Build libtgx_hip.so (hand-written HIP for gfx950) in-tree.

The library is compiled with hipcc straight from the sources under csrc/ into
tiga/_lib/libtgx_hip.so, so it travels with the source tree to a GPU host.
Run ``python tiga-lang_amd/build_native.py`` or call :func:`build`.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
LIB_DIR = HERE / "tiga" / "_lib"
LIB = LIB_DIR / "libtgx_hip.so"
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=fast",
    # Keep the compiler from forming packed fp32 VALU ops (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build")
    return path


def _included_sources(src: Path) -> list[Path]:
    """The source files `src` includes (a .hip built again with other
    settings), for the incremental check."""
    names = re.findall(r'^#include "([^"]+\.hip)"', src.read_text(), re.M)
    return [CSRC / n for n in names]


# The edge-MLP translation units take minutes each (most of the build):
# they start first.
_SLOW_FIRST = ("tgx_nn_math.hip", "tgx_nn_math_i64.hip", "tgx_nn.hip", "tgx_nn_i64.hip",
               "tgx_nn_wide_math.hip", "tgx_nn_wide.hip")


def sources() -> list[Path]:
    """Every source: the slow edge-MLP units first, then the largest (with
    what it includes) first."""
    def key(src: Path):
        size = sum(f.stat().st_size for f in [src, *_included_sources(src)])
        slow = _SLOW_FIRST.index(src.name) if src.name in _SLOW_FIRST else len(_SLOW_FIRST)
        return (slow, -size, src.name)
    return sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.cpp")], key=key)


def build(verbose: bool = False, jobs: int = 8, incremental: bool = False) -> Path:
    """Compile every source to an object in parallel, then link the .so.

    incremental=True reuses an object that is newer than its source and
    every header (for development; the default compiles everything)."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    obj_dir = HERE / "_build"
    obj_dir.mkdir(exist_ok=True)
    hipcc = _hipcc()
    procs = []
    objects = []
    headers = [*CSRC.glob("*.h"), *INCLUDE.glob("*.h")]
    newest_header = max((h.stat().st_mtime for h in headers), default=0.0)
    for src in sources():
        obj = obj_dir / (src.name + ".o")
        objects.append(obj)
        newest_source = max(f.stat().st_mtime for f in [src, *_included_sources(src)])
        if incremental and obj.exists() and \
                obj.stat().st_mtime > max(newest_source, newest_header):
            continue
        cmd = [hipcc, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
        if src.suffix == ".cpp":
            cmd = [hipcc, f"--offload-arch={ARCH}", "-O2", "-fPIC", "-std=c++17", "-pthread",
                   "-Wno-unused-result", f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o",
                   str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        while sum(p.poll() is None for _, p in procs) >= jobs:
            procs[[p.poll() is None for _, p in procs].index(True)][1].wait()
    failed = []
    for src, p in procs:
        out = p.communicate()[0].decode(errors="replace")
        out = "\n".join(l for l in out.splitlines()
                        if "packed-fp32-ops" not in l and l.strip())
        if p.returncode != 0:
            failed.append(f"{src.name}:\n{out}")
        elif out and verbose:
            print(out)
    if failed:
        raise RuntimeError("HIP build failed:\n" + "\n".join(failed))
    tmp = LIB.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", "-o", str(tmp),
            *map(str, objects)]
    if verbose:
        print(" ".join(link), flush=True)
    subprocess.run(link, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv, incremental="--incremental" in sys.argv)
    print(path)
