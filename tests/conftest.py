"""Test configuration: import paths and the `gpu` marker.

CPU tests (`-m "not gpu"`) cover the oracle against the reference's known answers,
the host logic (metadata, planner, acceptance) and the C-ABI library's exports.
GPU tests (`-m gpu`) run the HIP kernels through the C ABI and compare them with
the oracle; they require an MI355X and fail (not skip) without one.
"""
from __future__ import annotations

from pathlib import Path
import sys

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "nano-vllm-jetspec_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")
