import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402
import oracle  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run on the GPU box)")


@pytest.fixture(scope="session")
def pkg():
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def L(pkg):
    return pkg.lib()


@pytest.fixture(scope="session")
def synth(pkg):
    import importlib
    return importlib.import_module("bare_metal_gpt2_amd.synth")


def tol_check(got, ref, max_abs=2e-2, rel_l2=1e-3):
    """The fp16 parity bar: max |got-ref| <= 2e-2 and ||got-ref||/||ref|| <= 1e-3."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = float(np.abs(got - ref).max()) if got.size else 0.0
    nrm = float(np.linalg.norm(ref))
    rel = float(np.linalg.norm(got - ref) / nrm) if nrm > 0 else float(np.linalg.norm(got - ref))
    assert err <= max_abs and rel <= rel_l2, f"max abs {err:.3e} (<= {max_abs}), rel-L2 {rel:.3e} (<= {rel_l2})"
    return err, rel
