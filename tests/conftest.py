"""Test configuration: the ``gpu`` marker, repo-root imports, the package loader."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def pkg():
    import __graft_entry__
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _no_registered_gemm_configs():
    """Every test starts and ends with the cost model's plans: a per-shape entry that one
    test registers (tactics.prepare, mxl_set_gemm_config) is process-wide state."""
    yield
    mod = sys.modules.get("vllm_mach_amd._lib")
    if mod is not None and getattr(mod, "_lib", None) is not None:
        mod.call("mxl_clear_gemm_configs")
