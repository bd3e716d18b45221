"""Shared fixtures. GPU tests are marked ``gpu`` and skip cleanly without a GPU."""
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _cuda_ok():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


def pytest_collection_modifyitems(config, items):
    if _cuda_ok():
        return
    skip = pytest.mark.skip(reason="no GPU visible (torch.cuda.is_available() is False)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def fa():
    """The package flashattn-cuda_amd (fails loudly if its extension is not built)."""
    import __graft_entry__ as ge
    return ge.import_package()


@pytest.fixture(scope="session")
def capi():
    import __graft_entry__ as ge
    return ge.import_capi()


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda:0")


def pytest_terminal_summary(terminalreporter):
    """Print the forward error envelope the GPU tests measured (tests/errlog.py)."""
    try:
        import errlog
    except ImportError:   # pragma: no cover
        return
    lines = errlog.summary_lines()
    if lines:
        terminalreporter.section("forward error envelope")
        for line in lines:
            terminalreporter.write_line(line)
