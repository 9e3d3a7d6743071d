"""Shared pytest setup: the ``gpu`` marker, package import by path, common fixtures."""

from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def load_package():
    """Import ``faster-cosyvoice_amd/`` as the package ``faster_cosyvoice_amd``."""
    name = "faster_cosyvoice_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = REPO / "faster-cosyvoice_amd"
    spec = importlib.util.spec_from_file_location(name, pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libfcvdit.so")


@pytest.fixture(scope="session")
def fcv():
    return load_package()


@pytest.fixture(scope="session")
def full22(fcv):
    """The 22-block DiT with seed-0 N(0, 0.02) weights on cuda:0 (GPU tests only)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from tests.gpu_helpers import make_estimator, say
    say("[full22] drawing 22-layer weights")
    sd = fcv.synthetic.random_state_dict(fcv.synthetic.DiTDims(), seed=0)
    return sd, make_estimator(fcv, sd, depth=22)


@pytest.fixture(scope="session")
def sharp22(fcv):
    """The 22-block DiT on the peaked-attention recipe of ``tests/recipes.py`` (GPU tests only)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from tests import recipes
    from tests.gpu_helpers import make_estimator, say
    say("[sharp22] drawing 22-layer weights, peaked-attention recipe")
    sd = recipes.state_dict(fcv, recipes.SHARP22)
    return sd, make_estimator(fcv, sd, depth=22)
