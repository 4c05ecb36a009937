"""Builds libtreeverify.so (gfx950) in-tree with hipcc.

    python nano-vllm-jetspec_amd/build.py [--verbose]

The library lands next to the Python package (jetspec_amd/libtreeverify.so), which
is where jetspec_amd._lib loads it from.  Every call recompiles: each source is
compiled to an object in parallel (the attention kernel is instantiated per query
group in its own translation unit), then the objects are linked.
"""
from __future__ import annotations

import argparse
from concurrent.futures import ThreadPoolExecutor
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

# Query heads per KV head the attention kernel is instantiated for.
GROUPS = (1, 2, 3, 4, 5, 6, 7, 8, 16)
# ... and at head sizes 64 and 256 for the power-of-two groups.
GROUPS_D64 = (1, 2, 4, 8, 16)
GROUPS_D256 = (1, 2, 4, 8, 16)
ATTENTION_GROUP_SOURCES = (tuple(f"tv_attention_g{g}.hip" for g in GROUPS) +
                           tuple(f"tv_attention_d64_g{g}.hip" for g in GROUPS_D64) +
                           tuple(f"tv_attention_d256_g{g}.hip" for g in GROUPS_D256))
SOURCES = ("tv_common.cpp", "tv_plan.cpp", "tv_kvcache.hip", "tv_attention.hip", *ATTENTION_GROUP_SOURCES,
           "tv_attention_fp32.hip",
           "tv_rope.hip", "tv_accept.hip", "tv_metadata.hip", "tv_plan_device.hip")

# Packed-FP32 VALU instructions are kept out of the device code (they are not
# needed: the hot loops are MFMA and single-precision VALU work).
HIP_FLAGS = (
    "-O3", "-std=c++17", "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
)
# hipcc's host pass does not know the packed-fp32 feature flag and says so; that
# warning is expected and filtered out of the report.
NOISE = "'-packed-fp32-ops' is not a recognized feature"


def _jobs() -> int:
    try:
        requested = int(os.environ.get("MAX_JOBS", "0"))
    except ValueError:
        requested = 0
    return max(1, min(requested or (os.cpu_count() or 1), 16, len(SOURCES)))


def _run(cmd: list[str], what: str) -> list[str]:
    result = subprocess.run(cmd, capture_output=True, text=True)
    messages = [line for line in (result.stdout + result.stderr).splitlines() if NOISE not in line]
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {what}:\n" + "\n".join(messages))
    return messages


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; install ROCm or put hipcc on PATH")
    return path


def _check_m0(source: str, tmp: Path) -> None:
    import re

    asm = tmp / (Path(source).stem + ".s")
    cmd = [hipcc(), "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-S", "--cuda-device-only",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{REPO / 'include'}",
           f"-I{CSRC}", str(CSRC / source), "-o", str(asm)]
    _run(cmd, source + " (-S)")
    # Explicit M0 operands other than the DMA's own writes, and the instructions that
    # read M0 implicitly (indexed register moves).
    implicit = re.compile(r"^\s*(s_set_gpr_idx_on|s_movrel|v_movrel)")
    bad = [line.strip() for line in asm.read_text().splitlines()
           if not line.lstrip().startswith(";")
           and ((re.search(r"\bm0\b", line) and not re.match(r"\s*s_mov_b32 m0, s\d+\s*$", line))
                or implicit.match(line))]
    if bad:
        raise RuntimeError(f"{source}: compiler-generated M0 use would be clobbered by the DMA asm: "
                           + "; ".join(bad[:5]))


def check_m0_discipline(verbose: bool = False, jobs: int | None = None) -> None:
    """The attention kernel issues its global->LDS DMA from inline asm that sets M0.

    That is only sound while no compiler-generated instruction of the kernel uses M0,
    so compile each translation unit holding an instance of the kernel to assembly and
    require every M0 reference to be one of those `s_mov_b32 m0, sN` writes.
    """
    import tempfile

    with tempfile.TemporaryDirectory() as tmp, ThreadPoolExecutor(jobs or _jobs()) as pool:
        list(pool.map(lambda src: _check_m0(src, Path(tmp)), ATTENTION_GROUP_SOURCES))
    if verbose:
        print("M0 discipline ok", flush=True)


def build(verbose: bool = False, extra_flags: tuple[str, ...] = ()) -> Path:
    import tempfile

    tmp_so = OUTPUT.with_suffix(".so.tmp")
    jobs = _jobs()
    with tempfile.TemporaryDirectory() as tmp:
        objects = [Path(tmp) / (name.replace(".", "_") + ".o") for name in SOURCES]

        def compile_one(index: int) -> list[str]:
            cmd = [hipcc(), *HIP_FLAGS, *extra_flags, f"-I{REPO / 'include'}", f"-I{CSRC}", "-c",
                   str(CSRC / SOURCES[index]), "-o", str(objects[index])]
            if verbose:
                print(" ".join(cmd), flush=True)
            return _run(cmd, SOURCES[index])

        with ThreadPoolExecutor(jobs) as pool:
            messages = [line for lines in pool.map(compile_one, range(len(SOURCES))) for line in lines]
        link = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objects), "-o", str(tmp_so)]
        messages += _run(link, "link")
    if verbose and messages:
        print("\n".join(messages), flush=True)
    check_m0_discipline(verbose, jobs)
    os.replace(tmp_so, OUTPUT)
    build_examples(verbose)
    return OUTPUT


EXAMPLES = HERE / "examples"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def build_examples(verbose: bool = False) -> list[Path]:
    """The C callers of the library (examples/*.c): plain gcc against the C ABI and the
    HIP runtime, linked to the in-tree libtreeverify.so through an $ORIGIN rpath."""
    built = []
    for source in sorted(EXAMPLES.glob("*.c")):
        binary = source.with_suffix("")
        cmd = ["gcc", "-O2", "-std=c11", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}",
               f"-I{REPO / 'include'}", str(source), f"-L{OUTPUT.parent}", "-ltreeverify", f"-L{ROCM / 'lib'}",
               "-lamdhip64", "-lm", "-Wl,-rpath,$ORIGIN/../jetspec_amd", f"-Wl,-rpath,{ROCM / 'lib'}",
               "-o", str(binary)]
        if verbose:
            print(" ".join(cmd), flush=True)
        messages = _run(cmd, source.name)
        if messages:
            raise RuntimeError(f"{source.name}: compiler warnings:\n" + "\n".join(messages))
        built.append(binary)
    return built


_RESOURCE_FIELDS = (("TotalSGPRs", "SGPR"), ("VGPRs", "VGPR"), ("AGPRs", "AGPR"), ("SGPRs Spill", "SGPR spill"),
                    ("VGPRs Spill", "VGPR spill"), ("ScratchSize [bytes/lane]", "scratch B/lane"),
                    ("LDS Size [bytes/block]", "LDS B/block"), ("Occupancy [waves/SIMD]", "waves/SIMD"))


def _demangle(names: list[str]) -> list[str]:
    """Readable kernel names: the attention instances as <operand type, probability mode, G>,
    the others through c++filt when it is installed."""
    import re

    tool = shutil.which("c++filt")
    plain = names
    if tool:
        # Older demanglers do not know the mangling of __bf16 and _Float16: spell them as
        # vendor-extended types.
        spelled = [n.replace("DF16b", "u6__bf16").replace("DF16_", "u8_Float16") for n in names]
        out = subprocess.run([tool], input="\n".join(spelled), capture_output=True, text=True).stdout.splitlines()
        plain = out if len(out) == len(names) else names
    readable = []
    for name, fallback in zip(names, plain):
        m = re.search(r"tree_attention_kernelI(DF16b|DF16_)Lb([01])ELi(\d+)E", name)
        if m:
            operand = "bf16" if m.group(1) == "DF16b" else "f16"
            mode = "exact P" if m.group(2) == "1" else f"{operand} P"
            readable.append(f"tree_attention_kernel<{operand}, {mode}, G={m.group(3)}>")
        else:
            readable.append(fallback.replace("(anonymous namespace)::", ""))
    return readable


def resource_usage(jobs: int | None = None) -> list[dict]:
    """The compiler's own resource report (-Rpass-analysis=kernel-resource-usage) for every
    kernel of every device translation unit: registers, spills, LDS and waves per SIMD."""
    import re
    import tempfile

    sources = [s for s in SOURCES if s.endswith(".hip")]

    def report(source: str) -> list[dict]:
        with tempfile.TemporaryDirectory() as tmp:
            cmd = [hipcc(), *HIP_FLAGS, f"-I{REPO / 'include'}", f"-I{CSRC}", "-c", "--cuda-device-only",
                   "-Rpass-analysis=kernel-resource-usage", str(CSRC / source), "-o", str(Path(tmp) / "k.o")]
            lines = _run(cmd, source + " (resource usage)")
        kernels, current = [], None
        for line in lines:
            m = re.search(r"remark: Function Name: (\S+)", line)
            if m:
                current = {"source": source, "kernel": m.group(1)}
                kernels.append(current)
                continue
            m = re.search(r"remark:\s+([^:]+): (\S+) \[-Rpass", line)
            if m and current is not None:
                current[m.group(1).strip()] = m.group(2)
        return kernels

    with ThreadPoolExecutor(jobs or _jobs()) as pool:
        kernels = [k for ks in pool.map(report, sources) for k in ks]
    for k, name in zip(kernels, _demangle([k["kernel"] for k in kernels])):
        k["name"] = name
    return kernels


def resource_table(kernels: list[dict]) -> str:
    head = "| source | kernel | " + " | ".join(label for _, label in _RESOURCE_FIELDS) + " |"
    rule = "|---|---|" + "---:|" * len(_RESOURCE_FIELDS)
    rows = [f"| {k['source']} | `{k['name']}` | " + " | ".join(k.get(field, "") for field, _ in _RESOURCE_FIELDS) + " |"
            for k in kernels]
    return "\n".join([head, rule, *rows])


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--verbose", action="store_true")
    parser.add_argument("--resources", action="store_true",
                        help="print the compiler's per-kernel resource report (registers, spills, LDS, occupancy) "
                             "as a markdown table instead of building")
    args = parser.parse_args()
    if args.resources:
        print(resource_table(resource_usage()))
        return 0
    path = build(verbose=args.verbose)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
