"""Shared pytest setup: import paths, the `gpu` marker, the device context fixture."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "pipeline-parallelism-deep-learning-library_amd"
for p in (str(REPO), str(PKG), str(Path(__file__).resolve().parent)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def ctx():
    import linalg_hip as L
    c = L.Context.new(0)
    yield c
    c.close()


@pytest.fixture()
def pool(ctx):
    from helpers import Pool
    p = Pool(ctx)
    yield p
    p.free_all()
