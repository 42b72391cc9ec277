"""pytest configuration: the `gpu` marker, import paths and shared fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "stablediffusion-cpp_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def orc():
    from oracle import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle import Reference, have_reference

    if not have_reference():
        pytest.skip("oracle/_ref/libsdref.so not built (reference tree absent when build() ran)")
    return Reference()


@pytest.fixture(scope="session")
def be():
    import sdhip

    # No skip: on the GPU box a missing library or device must fail loudly.
    return sdhip.Backend()
