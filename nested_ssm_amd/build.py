"""Build the gfx950 shared library `libnssm_hip.so` in-tree with hipcc.

Usage: python -m nested_ssm_amd.build [--debug]

The library holds the HIP kernels and the C ABI declared in include/nssm.h.
It is built next to this file so it travels with the source tree.
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libnssm_hip.so")
SOURCES = [os.path.join(CSRC, "nssm_step.hip")]
HEADERS = [os.path.join(CSRC, "nssm_formats.h"), os.path.join(ROOT, "include", "nssm.h")]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libnssm_hip.so)")


def compile_flags(debug: bool = False) -> list:
    return [
        f"--offload-arch={ARCH}",
        "-O1" if debug else "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        "-Wno-unused-result",
        # packed fp32 VALU forms are kept out of generated code on purpose
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(ROOT, "include"),
    ]


def build(debug: bool = False, verbose: bool = True) -> str:
    """Compile every HIP source into LIB (always recompiles)."""
    tmp = LIB + ".tmp"
    cmd = [hipcc()] + compile_flags(debug) + SOURCES + ["-o", tmp]
    if verbose:
        print("[nssm build]", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")
    noisy = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if noisy and verbose:
        sys.stderr.write("\n".join(noisy) + "\n")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(debug="--debug" in sys.argv)
