"""Builds the GPU test helpers of tests/gpu_helpers/ (hipcc, gfx950, the
library's compile flags) into shared libraries beside their sources."""

from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
HELPERS = {"libbf16check.so": "bf16_rounding.hip", "libquantcheck.so": "quant_division.hip"}


def build() -> list[Path]:
    import sys

    if str(ROOT) not in sys.path:
        sys.path.insert(0, str(ROOT))
    from freetoken_amd import build as hipbuild

    out = []
    for lib, src in HELPERS.items():
        dst = HERE / lib
        cmd = [hipbuild.hipcc(), *hipbuild.HIPCC_FLAGS, f"-I{ROOT / 'freetoken_amd' / 'csrc'}", "-shared",
               str(HERE / src), "-o", str(dst)]
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n" + r.stdout.decode(errors="replace"))
        out.append(dst)
    return out


if __name__ == "__main__":
    print(build())
