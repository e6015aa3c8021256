"""pytest configuration: the `gpu` marker and import paths.

The product package `dilution` lives under `dilution-attention_amd/`; the CPU
oracle under `oracle/` (importable only from tests, smoke() and the bench's
CPU-baseline leg).
"""

from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (os.path.join(ROOT, "dilution-attention_amd"), ROOT):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
