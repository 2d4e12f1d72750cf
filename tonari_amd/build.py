"""Compile libtonari_hip.so for gfx950 with hipcc and the host provider
libtonari_cpu.so with g++ (in-tree, no JIT cache).

Flags that matter for parity and safety:
  -ffp-contract=off                      no implicit FMA contraction; the
                                         broad phase asks for fma explicitly
  -fno-gpu-flush-denormals-to-zero       IEEE denormals, like the CPU path
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                         no packed FP32 instructions
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = [os.path.join(HERE, "csrc", "tonari_hip.hip")]
HEADERS = [os.path.join(HERE, "csrc", "nl_device.h"), os.path.join(ROOT, "include", "tonari_hip.h")]
OUTPUT = os.path.join(HERE, "_lib", "libtonari_hip.so")
CPU_SOURCES = [os.path.join(HERE, "csrc", "cpu", "nl_cpu.cpp")]
CPU_OUTPUT = os.path.join(HERE, "_lib", "libtonari_cpu.so")
ARCH = "gfx950"


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build tonari_amd")
    return path


def command(output: str = OUTPUT, extra: list[str] | None = None) -> list[str]:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-ffp-contract=off",
        "-fno-gpu-flush-denormals-to-zero",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(ROOT, "include"),
        f'-DTNR_OFFLOAD_ARCH="{ARCH}"',
        *(extra or []),
        *SOURCES,
        "-o", output,
    ]


def cpu_command(output: str = CPU_OUTPUT) -> list[str]:
    """The host provider: plain C++17 with threads; -ffp-contract=off keeps
    every operation of the predicate rounded on its own (x86-64 arithmetic
    is SSE, no extended precision)."""
    cxx = shutil.which("g++") or "g++"
    return [
        cxx, "-O3", "-std=c++17", "-fPIC", "-shared", "-pthread", "-ffp-contract=off",
        "-fno-fast-math", "-Wall", "-Wextra",
        "-I", os.path.join(ROOT, "include"),
        *CPU_SOURCES,
        "-o", output,
    ]


def _run(cmd: list[str], output: str, verbose: bool, what: str) -> None:
    tmp = output + ".tmp"
    cmd = [tmp if c == output else c for c in cmd]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        sys.stderr.write(result.stdout + result.stderr)
        raise RuntimeError(f"failed to build {what}")
    os.replace(tmp, output)


def build_cpu(verbose: bool = False) -> str:
    os.makedirs(os.path.dirname(CPU_OUTPUT), exist_ok=True)
    _run(cpu_command(), CPU_OUTPUT, verbose, "libtonari_cpu.so")
    return CPU_OUTPUT


def build(verbose: bool = False) -> str:
    os.makedirs(os.path.dirname(OUTPUT), exist_ok=True)
    _run(command(OUTPUT), OUTPUT, verbose, "libtonari_hip.so")
    build_cpu(verbose)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))
    print(CPU_OUTPUT)
