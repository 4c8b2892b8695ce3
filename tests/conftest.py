"""Shared pytest configuration: the `gpu` marker, repo-root imports and the
golden-vector loader."""

from __future__ import annotations

import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN_NAMES = sorted(p.stem for p in GOLDEN.glob("*.npz"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built library")


def load_golden(name: str) -> dict:
    """One golden vector: input bits, shape, every stream and the decoded bits
    written by the reference encoder (tests/golden/make_golden.py)."""
    with np.load(GOLDEN / f"{name}.npz") as g:
        d = {k: g[k] for k in g.files}
    d["rows"], d["cols"] = (int(v) for v in d["shape"])
    return d


def golden_as_encoding(g: dict) -> dict:
    """The golden streams in the oracle's dict layout."""
    return {
        "sm": g["sm"], "ec": g["ec"], "esc": g["esc"], "fallback_bitmap": g["fallback_bitmap"],
        "fallback_raw": g["fallback_raw"], "codebook": g["codebook"], "shape": (g["rows"], g["cols"]),
    }


@pytest.fixture(scope="session")
def gpu():
    """cuda:0 with the built library loaded; skips only where no GPU exists.
    On a GPU machine a missing library is an error, not a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP GPU in this environment")
    from se12_amd import _native

    _native.lib()
    return torch.device("cuda", 0)
