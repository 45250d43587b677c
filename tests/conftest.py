import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO / "kohaku-tt_amd", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def _built():
    pkg = REPO / "kohaku-tt_amd" / "kohakutt_amd"
    return (pkg / "libkohakutt_amd.so").exists() and (pkg / "_torch_ops.so").exists()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")
    # Test modules import the package at collection; build it here when it is missing
    # (on the GPU box the libraries come prebuilt with the tree).
    if not _built():
        # Loaded by path: the package's __init__ refuses to import before the libraries exist.
        import importlib.util

        spec = importlib.util.spec_from_file_location(
            "_kohakutt_amd_build", REPO / "kohaku-tt_amd" / "kohakutt_amd" / "_build.py"
        )
        build = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(build)
        build.build_all()


@pytest.fixture(scope="session")
def native():
    """The package with its native libraries (built here first when they are missing;
    on the GPU box they come prebuilt with the tree)."""
    import kohakutt_amd

    return kohakutt_amd


@pytest.fixture(scope="session")
def dev(native):
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
