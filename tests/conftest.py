"""pytest configuration: the ``gpu`` marker and import paths.

Tests marked ``gpu`` need an MI355X and call the HIP library through its C
ABI; everything else runs on the CPU (oracle pins, host logic, ABI
exports).  The oracle under oracle/ is the checker only.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


@pytest.fixture(autouse=True)
def _fixed_launch_config(tmp_path_factory: pytest.TempPathFactory,
                         monkeypatch: pytest.MonkeyPatch) -> None:
    """Tests run the fallback launch configuration (one key split), the one
    the tile-exact oracle comparisons assume, and never touch the user's
    autotune cache; tests of the cache and of key splits opt out."""
    monkeypatch.setenv("REPERCEP_FP8_DISABLE_AUTOTUNE", "1")
    monkeypatch.setenv("REPERCEP_FP8_AUTOTUNE_CACHE",
                       str(tmp_path_factory.mktemp("autotune") / "fp8_autotune.json"))


@pytest.fixture(scope="session")
def gpu() -> "object":
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a GPU (run with -m 'not gpu')")
    from repercep_runtime_amd import _capi

    _capi.lib()  # raises if the library is missing: no silent fallback
    return torch.device("cuda", 0)
