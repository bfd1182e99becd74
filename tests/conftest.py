"""Shared fixtures. Tests marked `gpu` need an MI355X and the built
libvx_hip_dispatch.so; everything else runs on the CPU."""

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def hiplib():
    """The HIP dispatch library on a machine with a GPU. A GPU test that
    cannot get one fails: it never falls back to something else."""
    from vx_amd.runtime import DispatchLibrary

    lib = DispatchLibrary()
    n = lib.device_count()
    assert n >= 1, "no GPU visible to libvx_hip_dispatch.so"
    return lib


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


def announce(what: str) -> None:
    """Name the case on stderr before a GPU step, so a run that dies in it
    says which one."""
    print(f"[case] {what}", file=sys.stderr, flush=True)
