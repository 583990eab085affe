"""Shared pytest setup.

Markers: ``gpu`` for tests that need an MI355X (run on the GPU box with
``-m gpu``); everything else runs on the CPU container.  The repository root
and the package directory ``simd-ml-kernels_amd`` are put on sys.path so that
``import oracle.oracle`` and ``import simd_ml_kernels`` work from a checkout.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "simd-ml-kernels_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950); run with -m gpu")


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle as o
    return o


@pytest.fixture(scope="session")
def ref_lib():
    """The reference's own kernels built from /root/reference (oracle/_ref); skip if absent."""
    from oracle import oracle as o
    r = o.ref()
    if r is None:
        pytest.skip("oracle/_ref/libsmk_ref.so not built (needs /root/reference at build time)")
    return r
