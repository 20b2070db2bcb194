"""Test configuration.

Markers: `gpu` tests need an MI355X (they run through the C ABI of the
built library and compare with the CPU oracle); everything else runs on the
CPU. The library and the oracle must be built beforehand
(`__graft_entry__.build()`); a missing library fails loudly rather than
skipping, so a GPU run can never pass on something other than the HIP path.
"""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def mc():
    import minicompiler_amd

    minicompiler_amd.library()  # raises LibraryMissing if not built
    return minicompiler_amd


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as orc

    orc.lib()
    return orc


@pytest.fixture(scope="session")
def device(mc):
    """Device 0's description; GPU tests fail (not skip) without a device."""
    if mc.device_count() < 1:
        pytest.fail("no HIP device visible to a test marked gpu")
    return mc.device_json()
