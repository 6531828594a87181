"""Shared pytest setup.

* ``gpu`` marks tests that need a HIP device (gfx950); they are skipped
  when torch sees no GPU and must pass on the MI355X.
* The repository root is put on sys.path so that ``oracle`` (the CPU
  checker) and ``pocketlm_amd`` import from the tree.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
GOLDEN = REPO / "tests" / "golden"
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X, gfx950)")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def golden():
    cache: dict[str, np.lib.npyio.NpzFile] = {}

    def load(name: str):
        if name not in cache:
            cache[name] = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
        return cache[name]

    return load


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle

    oracle.lib()
    return oracle


def rel_l2(actual, expected) -> float:
    a = np.asarray(actual, dtype=np.float64).reshape(-1)
    e = np.asarray(expected, dtype=np.float64).reshape(-1)
    denom = float(np.linalg.norm(e))
    num = float(np.linalg.norm(a - e))
    if denom == 0.0:
        return num
    return num / denom


def items_from(g, prefix: str):
    n = int(g[f"{prefix}_count"])
    return [tuple(g[f"{prefix}_{k}{e}"] for k in ("g", "gs", "u", "us", "d", "ds")) for e in range(n)]
