"""AddressSanitizer builds of the host-side code on the path (CPU only): the
hybrid decode's CPU expert executor (freetoken_amd/csrc/cpu_experts.hip, its
host code; no GPU code is instrumented) and the CPU baseline's restatement of
the reference executor (oracle/cpu_moe/cpu_moe.cpp), each driven by a harness
in tests/asan/ over exact-size heap banks.  A heap overflow, use-after-free
or leak fails the run."""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CLANG = Path("/opt/rocm/llvm/bin/clang++")
# host-only instrumentation: the sanitizer flag goes to the host compilation of the .hip file
HOST_ASAN = "-Xarch_host -fsanitize=address -Xarch_host -fno-omit-frame-pointer".split()


def _run(cmd, cwd, env=None):
    r = subprocess.run(cmd, cwd=cwd, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=600)
    out = r.stdout.decode(errors="replace")
    assert r.returncode == 0, f"{' '.join(map(str, cmd))}\n{out[-4000:]}"
    return out


def _asan_env():
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=1:abort_on_error=0:halt_on_error=1"
    return env


@pytest.mark.skipif(not CLANG.exists() or shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="needs ROCm's clang and hipcc")
def test_cpu_executor_under_asan(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    inc = [f"-I{ROOT / 'include'}", f"-I{ROOT / 'freetoken_amd' / 'csrc'}"]
    _run([hipcc, "--offload-arch=gfx950", "-O1", "-g", "-std=c++20", *HOST_ASAN, *inc, "-c",
          str(ROOT / "freetoken_amd" / "csrc" / "cpu_experts.hip"), "-o", "cpu_experts.o"], tmp_path)
    _run([str(CLANG), "-O1", "-g", "-std=c++20", "-fsanitize=address", "-fno-omit-frame-pointer", *inc,
          "-D__HIP_PLATFORM_AMD__", "-c", str(ROOT / "tests" / "asan" / "executor_asan.cpp"), "-o", "harness.o"],
         tmp_path)
    _run([str(CLANG), "-fsanitize=address", "harness.o", "cpu_experts.o", "-L/opt/rocm/lib", "-lamdhip64",
          "-Wl,-rpath,/opt/rocm/lib", "-pthread", "-o", "executor_asan"], tmp_path)
    out = _run([str(tmp_path / "executor_asan")], tmp_path, _asan_env())
    assert "asan executor ok" in out and "AddressSanitizer" not in out, out[-2000:]


@pytest.mark.skipif(not CLANG.exists(), reason="needs ROCm's clang")
def test_cpu_baseline_restatement_under_asan(tmp_path):
    _run([str(CLANG), "-O1", "-g", "-std=c++17", "-fsanitize=address", "-fno-omit-frame-pointer", "-pthread",
          str(ROOT / "oracle" / "cpu_moe" / "cpu_moe.cpp"), str(ROOT / "tests" / "asan" / "cpu_moe_asan.cpp"),
          "-o", "cpu_moe_asan"], tmp_path)
    out = _run([str(tmp_path / "cpu_moe_asan")], tmp_path, _asan_env())
    assert "asan cpu_moe ok" in out and "AddressSanitizer" not in out, out[-2000:]
