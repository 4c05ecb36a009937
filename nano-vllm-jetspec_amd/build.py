"""Builds libtreeverify.so (gfx950) in-tree with hipcc.

    python nano-vllm-jetspec_amd/build.py [--verbose]

The library lands next to the Python package (jetspec_amd/libtreeverify.so), which
is where jetspec_amd._lib loads it from.  Every call recompiles.
"""
from __future__ import annotations

import argparse
import os
from pathlib import Path
import shutil
import subprocess
import sys

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
OUTPUT = HERE / "jetspec_amd" / "libtreeverify.so"
ARCH = "gfx950"

SOURCES = ("tv_common.cpp", "tv_plan.cpp", "tv_kvcache.hip", "tv_attention.hip", "tv_rope.hip", "tv_accept.hip", "tv_metadata.hip", "tv_plan_device.hip")

# Packed-FP32 VALU instructions are kept out of the device code (they are not
# needed: the hot loops are MFMA and single-precision VALU work).
HIP_FLAGS = (
    "-O3", "-std=c++17", "-fPIC", "-shared",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
)


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; install ROCm or put hipcc on PATH")
    return path


def check_m0_discipline(verbose: bool = False) -> None:
    """The attention kernel issues its global->LDS DMA from inline asm that sets M0.

    That is only sound while no compiler-generated instruction of the kernel uses M0,
    so compile the device code to assembly and require every M0 reference to be one
    of those `s_mov_b32 m0, sN` writes.
    """
    import re
    import tempfile

    with tempfile.TemporaryDirectory() as tmp:
        asm = Path(tmp) / "tv_attention.s"
        cmd = [hipcc(), "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-S", "--cuda-device-only",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{REPO / 'include'}",
               f"-I{CSRC}", str(CSRC / "tv_attention.hip"), "-o", str(asm)]
        result = subprocess.run(cmd, capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError("hipcc -S failed:\n" + result.stderr)
        # Explicit M0 operands other than the DMA's own writes, and the instructions that
        # read M0 implicitly (indexed register moves).
        implicit = re.compile(r"^\s*(s_set_gpr_idx_on|s_movrel|v_movrel)")
        bad = [line.strip() for line in asm.read_text().splitlines()
               if not line.lstrip().startswith(";")
               and ((re.search(r"\bm0\b", line) and not re.match(r"\s*s_mov_b32 m0, s\d+\s*$", line))
                    or implicit.match(line))]
        if bad:
            raise RuntimeError("compiler-generated M0 use would be clobbered by the DMA asm: " + "; ".join(bad[:5]))
        if verbose:
            print("M0 discipline ok", flush=True)


def build(verbose: bool = False, extra_flags: tuple[str, ...] = ()) -> Path:
    tmp = OUTPUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIP_FLAGS, *extra_flags, f"-I{REPO / 'include'}", f"-I{CSRC}",
           *[str(CSRC / name) for name in SOURCES], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    env = dict(os.environ)
    result = subprocess.run(cmd, capture_output=True, text=True, env=env)
    # hipcc's host pass does not know the packed-fp32 feature flag and says so; that
    # warning is expected and filtered out of the report.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    messages = [line for line in (result.stdout + result.stderr).splitlines() if noise not in line]
    if result.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(messages))
    if verbose and messages:
        print("\n".join(messages), flush=True)
    check_m0_discipline(verbose)
    os.replace(tmp, OUTPUT)
    return OUTPUT


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--verbose", action="store_true")
    args = parser.parse_args()
    path = build(verbose=args.verbose)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
