"""Build ``lib/libmi355.so`` from ``csrc/`` with hipcc for gfx950 (in-tree, so the library travels with the tree).

Usage: ``python lithos-metal_amd/build.py`` (or ``__graft_entry__.build()``). Always recompiles.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT = ROOT / "lib" / "libmi355.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
         # no packed-FP32 instructions anywhere (they have given silent wrong results on this pool)
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def sources():
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    objs = []
    obj_dir = ROOT / "lib" / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    procs = []
    for src in sources():
        obj = obj_dir / (src.name + ".o")
        cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objs.append(obj)
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        msgs = "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l and l.strip())
        if p.returncode != 0:
            failed.append((src, msgs))
        elif verbose and msgs:
            print(msgs)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n\n".join(f"{s}:\n{m}" for s, m in failed))
    tmp = OUT.with_suffix(".so.tmp")
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-lhiprtc", "-o", str(tmp)], check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
