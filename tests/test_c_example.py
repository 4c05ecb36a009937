"""The C-ABI example (nano-vllm-jetspec_amd/examples/verify_round.c): a plain C caller that
runs one verify round (append, visibility bits, plan, attention, accepted-path commit)
through libtreeverify.so and the HIP runtime, with no Python or torch in the process.

CPU: the built example resolves its libraries and starts (it reports that no GPU is
present).  GPU: it runs the round and its own host checks pass: the pool byte for byte
after the append and the commit, the attention within the bf16 gate of a
double-precision softmax over each row's visible keys.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

EXAMPLE = Path(__file__).resolve().parents[1] / "nano-vllm-jetspec_amd" / "examples" / "verify_round"


def run_example(timeout: float) -> subprocess.CompletedProcess:
    if not EXAMPLE.exists():
        pytest.fail(f"{EXAMPLE} is not built; run nano-vllm-jetspec_amd/build.py")
    return subprocess.run([str(EXAMPLE)], capture_output=True, text=True, timeout=timeout)


def test_example_links_against_the_library():
    libraries = subprocess.run(["ldd", str(EXAMPLE)], capture_output=True, text=True, timeout=30).stdout
    assert "libtreeverify.so" in libraries and "not found" not in libraries, libraries


def test_example_reports_a_missing_gpu():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present (the GPU test runs the round)")
    result = run_example(60)
    assert result.returncode == 2 and "no GPU" in result.stderr


@pytest.mark.gpu
def test_example_runs_one_verify_round():
    print(f"[c example] {EXAMPLE}", flush=True)
    result = run_example(120)
    print(result.stdout, result.stderr, flush=True)
    assert result.returncode == 0, result.stderr
    assert "byte-exact: yes" in result.stdout and result.stdout.startswith("verify_round:")
