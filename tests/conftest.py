"""Shared pytest setup: the `gpu` marker, import paths, and per-config shapes."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("llm.c_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


# The layer shapes of the benchmark configurations: (T, d, F, E, k) and the
# weight scales (router std, expert std).  C3's MoE layer is one block of
# the 8-layer decoder at batch 8 x seq 512; C4 is the 64-sequence decode step.
CONFIGS = {
    "c1": dict(T=256, d=128, F=512, E=4, k=2, std_router=0.02, std_expert=0.02),
    "c2": dict(T=4096, d=256, F=1024, E=8, k=2, std_router=0.1, std_expert=0.02),
    "c3": dict(T=4096, d=512, F=2048, E=8, k=2, std_router=0.02, std_expert=0.02),
    "c4": dict(T=64, d=512, F=2048, E=16, k=2, std_router=0.02, std_expert=0.02),
    "c5": dict(T=16384, d=2048, F=8192, E=64, k=4, std_router=0.02, std_expert=0.02),
}
