"""Shared test set-up.

Markers: `gpu` tests need an MI355X (gfx950) and run the HIP path through
the C ABI; everything else runs on the CPU.
"""
import pathlib
import sys

import numpy as np
import pytest

REPO = pathlib.Path(__file__).resolve().parent.parent
PKG = REPO / "vpipe-sensenova-u1.5_amd"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")


@pytest.fixture(scope="session")
def golden():
    def load(name):
        with np.load(GOLDEN / name, allow_pickle=False) as z:
            return {k: z[k] for k in z.files}
    return load


@pytest.fixture(scope="session")
def ops():
    """One u15h context for all GPU tests.  Fails (does not skip) when the
    library is missing on a GPU box: a GPU test must never pass without the
    native code."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("SKIPPED: no GPU in this process -- NOTHING was run")
    import u15h
    o = u15h.Ops(0)
    yield o
    torch.cuda.synchronize()
    o.close()
