"""Build of the gfx950 MoE-layer library ``libftmoe.so`` (in-tree).

hipcc compiles every ``csrc/*.hip`` for gfx950 only and links one shared
library next to this file; Python loads it with ctypes (``_lib.py``).
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libftmoe.so"
INCLUDE = PKG.parent / "include"

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU ops (v_pk_* f32) are kept out of the code objects: some of their forms
    # have given wrong results now and then on these boxes
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the MI355X build needs ROCm's hipcc")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source and link ``libftmoe.so``; returns its path."""
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    cc = hipcc()
    procs = []
    objs = []
    for src in sources():
        obj = objdir / (src.stem + ".o")
        objs.append(obj)
        cmd = [cc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    errors = []
    for src, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        lines = [ln for ln in text.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
        if p.returncode != 0:
            errors.append(f"{src.name}:\n" + "\n".join(lines))
        elif verbose and lines:
            print("\n".join(lines))
    if errors:
        raise RuntimeError("hipcc failed:\n" + "\n\n".join(errors))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout.decode(errors="replace"))
    # a kernel whose host-side instantiation the compiler dropped shows up as an
    # undefined symbol of the library's own namespace: fail the build on it
    nm = shutil.which("nm")
    if nm:
        und = subprocess.run([nm, "-D", "--undefined-only", "-C", str(tmp)], stdout=subprocess.PIPE,
                             stderr=subprocess.STDOUT).stdout.decode(errors="replace")
        missing = [ln.strip() for ln in und.splitlines() if "ftmoe::" in ln]
        if missing:
            os.unlink(tmp)
            raise RuntimeError("libftmoe.so has undefined library symbols:\n" + "\n".join(missing))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
